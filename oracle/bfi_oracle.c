/*
 * bfi_oracle.c — TEST INFRASTRUCTURE ONLY (see bfi_oracle.h).
 *
 * CPU restatement of crates/bfi-runtime/src/sample.rs and engine/spec.rs of
 * SeanHogg/builderforce-inference. Each function cites the reference lines it follows.
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off, glibc libm).
 */
#include "bfi_oracle.h"

#include <float.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ORC_MUTATE (test-only): each value plants one plausible mistake so the pinning tests can
 * show they catch it (tests/test_oracle_pins.py::test_pins_catch_planted_mistakes).
 * The shipped oracle is built with ORC_MUTATE undefined (= 0). */
#ifndef ORC_MUTATE
#define ORC_MUTATE 0
#endif

/* ---- Rng: sample.rs:441-460 (xorshift64, shifts 13/7/17; no multiply) ---------------- */

uint64_t orc_rng_next(uint64_t *state) {
    uint64_t x = *state;
    if (x == 0) x = 0x9E3779B97F4A7C15ull; /* sample.rs:447-449 */
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    *state = x;
    return x;
}

float orc_rng_f32(uint64_t *state) {
    /* sample.rs:457-459: (next_u64() >> 40) as f32 / (1u32 << 24) as f32 */
    return (float)(orc_rng_next(state) >> 40) / (float)(1u << 24);
}

uint64_t orc_slot_rng_seed(uint64_t seed, uint64_t prompt_len) {
    /* spec.rs:185-187 */
    return seed ^ 0xa0761d6478bd642full ^ (prompt_len * 0x9e3779b97f4a7c15ull);
}

/* ---- argmax: sample.rs:429-439 ------------------------------------------------------- */

uint32_t orc_argmax(const uint32_t *ids, const float *v, size_t n) {
    uint32_t best_i = 0;
    float best_v = -INFINITY;
    for (size_t j = 0; j < n; j++) {
        if (ORC_MUTATE == 9 ? v[j] >= best_v : v[j] > best_v) {
            best_v = v[j];
            best_i = ids ? ids[j] : (uint32_t)j;
        }
    }
    return best_i;
}

/* ---- draw: sample.rs:311-323 --------------------------------------------------------- */

static float rust_f32_max(float a, float b) {
    /* f32::max: NaN-ignoring (IEEE maxNum) */
    return fmaxf(a, b);
}

uint32_t orc_draw(const uint32_t *ids, const float *w, size_t n, float u) {
    float sum = 0.0f;
    for (size_t j = 0; j < n; j++) sum += w[j]; /* :313 iter().sum() sequential */
    float r = u * rust_f32_max(sum, 0.0f);      /* :314 */
    float cum = 0.0f;
    for (size_t j = 0; j < n; j++) { /* :316-321 */
        cum += w[j];
        if (ORC_MUTATE == 5 ? r < cum : r <= cum) return ids[j];
    }
    return n ? ids[n - 1] : 0; /* :322 */
}

/* ---- stable sort, descending by weight (sample.rs:393, 398) ------------------------- */

/* comparator of sample.rs:393: b.1.partial_cmp(&a.1).unwrap_or(Equal); element a goes
 * strictly before b only when a.w > b.w. A stable merge takes the right run's head first
 * only when it is strictly greater. */
static void merge_desc(uint32_t *ids, float *w, uint32_t *tid, float *tw, size_t n) {
    for (size_t width = 1; width < n; width *= 2) {
        for (size_t lo = 0; lo < n; lo += 2 * width) {
            size_t mid = lo + width < n ? lo + width : n;
            size_t hi = lo + 2 * width < n ? lo + 2 * width : n;
            size_t i = lo, j = mid, k = lo;
            while (i < mid && j < hi) {
                if (ORC_MUTATE == 8 ? w[j] >= w[i] : w[j] > w[i]) { /* right strictly greater -> goes first */
                    tid[k] = ids[j];
                    tw[k++] = w[j++];
                } else {
                    tid[k] = ids[i];
                    tw[k++] = w[i++];
                }
            }
            while (i < mid) {
                tid[k] = ids[i];
                tw[k++] = w[i++];
            }
            while (j < hi) {
                tid[k] = ids[j];
                tw[k++] = w[j++];
            }
        }
        memcpy(ids, tid, n * sizeof(uint32_t));
        memcpy(w, tw, n * sizeof(float));
    }
}

static int stable_sort_desc(uint32_t *ids, float *w, size_t n) {
    if (n < 2) return 0;
    uint32_t *tid = (uint32_t *)malloc(n * sizeof(uint32_t));
    float *tw = (float *)malloc(n * sizeof(float));
    if (!tid || !tw) {
        free(tid);
        free(tw);
        return -1;
    }
    merge_desc(ids, w, tid, tw, n);
    free(tid);
    free(tw);
    return 0;
}

/* ---- history helpers ----------------------------------------------------------------- */

/* `HashSet<u32>` of prev (sample.rs:347, 361) restricted to ids < n_vocab (only those can
 * match an element of vals), plus the multiset counts the frequency extension needs. */
static uint32_t *history_counts(const uint32_t *prev, size_t n_prev, size_t n_vocab) {
    uint32_t *cnt = (uint32_t *)calloc(n_vocab ? n_vocab : 1, sizeof(uint32_t));
    if (!cnt) return NULL;
    for (size_t j = 0; j < n_prev; j++)
        if (prev[j] < n_vocab) cnt[prev[j]]++;
    return cnt;
}

static int mask_allows(const uint32_t *mask, size_t i) {
    return (mask[i >> 5] >> (i & 31)) & 1u;
}

/* ---- target: sample.rs:325-427 ------------------------------------------------------- */

int orc_target(const float *logits, size_t n_vocab, const uint32_t *prev, size_t n_prev,
               const bfi_smp_row_params *p, const uint32_t *mask, uint32_t *out_ids,
               float *out_w, float *out_s, orc_target_info *info) {
    orc_target_info local;
    if (!info) info = &local;
    memset(info, 0, sizeof(*info));
    info->len_k = info->len_p = info->len_m = -1;
    if (n_vocab == 0) { /* :327-329 */
        info->kind = 0;
        info->token = 0;
        return 0;
    }

    /* :331-337 — the id-union grammar sets every id outside the set to -inf; the packed
     * mask carries the same set (bit = allowed). */
    float *masked = (float *)malloc(n_vocab * sizeof(float));
    if (!masked) return -1;
    for (size_t i = 0; i < n_vocab; i++)
        masked[i] = (mask && !mask_allows(mask, i)) ? -INFINITY : logits[i];

    /* :339-343 vals in index order */
    uint32_t *ids = out_ids;
    float *w = out_w;
    for (size_t i = 0; i < n_vocab; i++) {
        ids[i] = (uint32_t)i;
        w[i] = masked[i];
    }

    uint32_t *cnt = NULL;
    if (n_prev > 0) {
        cnt = history_counts(prev, n_prev, n_vocab);
        if (!cnt) {
            free(masked);
            return -1;
        }
    }
    if (ORC_MUTATE == 1 && p->presence_penalty != 0.0f && n_prev > 0)
        for (size_t i = 0; i < n_vocab; i++)
            if (cnt[i]) w[i] -= p->presence_penalty;
    /* :345-357 repeat penalty (f32 arithmetic: (rp - 1.0).abs() > f32::EPSILON) */
    if (fabsf(p->repeat_penalty - 1.0f) > FLT_EPSILON && n_prev > 0) {
        for (size_t i = 0; i < n_vocab; i++) {
            if (cnt[i]) {
                if (ORC_MUTATE == 6 || w[i] > 0.0f)
                    w[i] /= p->repeat_penalty;
                else
                    w[i] *= p->repeat_penalty;
            }
        }
    }
    /* :359-367 presence penalty */
    if (ORC_MUTATE != 1 && p->presence_penalty != 0.0f && n_prev > 0) {
        for (size_t i = 0; i < n_vocab; i++)
            if (cnt[i]) w[i] -= p->presence_penalty;
    }
    /* extension (not in the reference): frequency penalty, OpenAI semantics
     * l -= f * count, applied after presence; two f32 roundings, no FMA. */
    if (p->frequency_penalty != 0.0f && n_prev > 0) {
        for (size_t i = 0; i < n_vocab; i++) {
            if (cnt[i]) {
                float fc = p->frequency_penalty * (float)cnt[i];
                w[i] -= fc;
            }
        }
    }
    free(cnt);

    /* :369-371 greedy exit */
    if (!(p->temperature > 0.0f)) {
        if (out_s) memcpy(out_s, w, n_vocab * sizeof(float));
        info->kind = 0;
        info->token = orc_argmax(ids, w, n_vocab);
        free(masked);
        return 0;
    }

    /* :373-375 true division by T */
    for (size_t i = 0; i < n_vocab; i++)
        w[i] = ORC_MUTATE == 2 ? w[i] * (1.0f / p->temperature) : w[i] / p->temperature;
    if (out_s) memcpy(out_s, w, n_vocab * sizeof(float));

    /* :377-390 max fold, exp, sequential sum, normalize */
    float mx = -INFINITY;
    for (size_t i = 0; i < n_vocab; i++) mx = rust_f32_max(mx, w[i]);
    float sum = 0.0f;
    for (size_t i = 0; i < n_vocab; i++) {
        w[i] = expf(w[i] - mx);
        sum += w[i];
    }
    if (sum > 0.0f)
        for (size_t i = 0; i < n_vocab; i++) w[i] /= sum;
    info->max = mx;
    info->sum = sum;

    size_t len = n_vocab;
    /* :392-395 top-k */
    if (p->top_k > 0 && (size_t)p->top_k < len) {
        if (stable_sort_desc(ids, w, len)) {
            free(masked);
            return -1;
        }
        info->sorted = 1;
        len = (size_t)p->top_k + (ORC_MUTATE == 7 ? 1 : 0);
        info->len_k = (int64_t)len;
    }
    /* :397-409 top-p */
    if (p->top_p < 1.0f) {
        if (stable_sort_desc(ids, w, len)) {
            free(masked);
            return -1;
        }
        info->sorted = 1;
        float cum = 0.0f;
        size_t cut = len;
        for (size_t i = 0; i < len; i++) {
            cum += w[i];
            if (ORC_MUTATE == 3 ? cum > p->top_p : cum >= p->top_p) {
                cut = i + 1;
                break;
            }
        }
        len = cut > 1 ? cut : 1;
        info->len_p = (int64_t)len;
    }
    /* :411-424 min-p (retain keeps order) */
    if (p->min_p > 0.0f) {
        float max_p = 0.0f;
        for (size_t i = 0; i < len; i++) max_p = rust_f32_max(max_p, w[i]);
        float thresh = ORC_MUTATE == 4 ? p->min_p : p->min_p * max_p;
        size_t k = 0;
        for (size_t i = 0; i < len; i++) {
            if (w[i] >= thresh) {
                ids[k] = ids[i];
                w[k++] = w[i];
            }
        }
        len = k;
        info->len_m = (int64_t)len;
        if (len == 0) { /* :415-422 argmax over the masked, un-penalized logits */
            info->kind = 0;
            info->minp_fallback = 1;
            info->token = ORC_MUTATE == 13 ? orc_argmax(NULL, out_s ? out_s : masked, n_vocab)
                                           : orc_argmax(NULL, masked, n_vocab);
            free(masked);
            return 0;
        }
    }
    free(masked);
    info->kind = 1;
    info->len = (int64_t)len;
    return 0;
}

/* sample(): sample.rs:304-309 with the uniform passed in (the reference uses
 * Rng(p.seed).f32()). */
uint32_t orc_sample(const float *logits, size_t n_vocab, const uint32_t *prev, size_t n_prev,
                    const bfi_smp_row_params *p, const uint32_t *mask, float u) {
    if (n_vocab == 0) return 0;
    uint32_t *ids = (uint32_t *)malloc(n_vocab * sizeof(uint32_t));
    float *w = (float *)malloc(n_vocab * sizeof(float));
    orc_target_info info;
    uint32_t tok = 0;
    if (ids && w && orc_target(logits, n_vocab, prev, n_prev, p, mask, ids, w, NULL, &info) == 0)
        tok = info.kind == 0 ? info.token : orc_draw(ids, w, (size_t)info.len, u);
    free(ids);
    free(w);
    return tok;
}

/* ---- judge: spec.rs:79-97 ------------------------------------------------------------ */

int orc_judge(int32_t kind, uint32_t token, const uint32_t *ids, const float *w, size_t n,
              uint32_t d, float u, float u2, uint32_t *reject_token) {
    if (kind == 0) { /* :81-82 */
        if (token == d) return 1;
        *reject_token = token;
        return 0;
    }
    float sum = 0.0f; /* :84 */
    for (size_t j = 0; j < n; j++) sum += w[j];
    float p_d = 0.0f; /* :85 find() = first match */
    for (size_t j = 0; j < n; j++)
        if (ids[j] == d) {
            p_d = w[j];
            break;
        }
    if (sum > 0.0f && (ORC_MUTATE == 10 ? u <= p_d / sum : u < p_d / sum)) return 1; /* :86-88 */
    /* :89 residual = vals without d, order kept */
    uint32_t *rid = (uint32_t *)malloc((n ? n : 1) * sizeof(uint32_t));
    float *rw = (float *)malloc((n ? n : 1) * sizeof(float));
    size_t m = 0;
    int all_nonpos = 1;
    for (size_t j = 0; j < n; j++) {
        if (ORC_MUTATE == 11 || ids[j] != d) {
            rid[m] = ids[j];
            rw[m] = w[j];
            if (!(w[j] <= 0.0f)) all_nonpos = 0; /* :90 all(w <= 0): a NaN weight is not <= 0 */
            m++;
        }
    }
    int verdict;
    if (m == 0 || all_nonpos) { /* :90-93 */
        verdict = 1;
    } else {
        *reject_token = orc_draw(rid, rw, m, u2); /* :94 */
        verdict = 0;
    }
    free(rid);
    free(rw);
    return verdict;
}

/* ---- draft: spec.rs:44-68 ------------------------------------------------------------ */

size_t orc_draft(const uint32_t *ctx, size_t len, size_t k, size_t ngram_max, size_t ngram_min,
                 uint32_t *out) {
    if (k == 0) return 0;
    size_t lo = ngram_min > 1 ? ngram_min : 1;
    for (size_t n = ngram_max; n >= lo && n > 0; n--) {
        if (len < n + 1) continue;
        const uint32_t *tail = ctx + (len - n);
        for (size_t it = 0; it < len - n; it++) {
            size_t start = ORC_MUTATE == 12 ? it : len - n - 1 - it;
            if (memcmp(ctx + start, tail, n * sizeof(uint32_t)) == 0) {
                size_t from = start + n;
                size_t to = from + k < len ? from + k : len;
                if (from < to) {
                    memcpy(out, ctx + from, (to - from) * sizeof(uint32_t));
                    return to - from;
                }
            }
        }
    }
    return 0;
}

/* ---- parse_id_union: sample.rs:207-221, strip_root 231-235 --------------------------- */

/* char::is_whitespace: the Unicode White_Space property (Rust core's table). */
static int is_white_space(uint32_t cp) {
    switch (cp) {
    case 0x09: case 0x0A: case 0x0B: case 0x0C: case 0x0D: case 0x20: case 0x85: case 0xA0:
    case 0x1680: case 0x2028: case 0x2029: case 0x202F: case 0x205F: case 0x3000:
        return 1;
    default:
        return cp >= 0x2000 && cp <= 0x200A;
    }
}

/* The code point encoded at s (UTF-8; s < e) and its byte length. */
static uint32_t utf8_at(const char *s, const char *e, int *len) {
    const unsigned char c = (unsigned char)s[0];
    int n = 1;
    uint32_t cp = c;
    if (c >= 0xF0) { n = 4; cp = c & 0x07; }
    else if (c >= 0xE0) { n = 3; cp = c & 0x0F; }
    else if (c >= 0xC0) { n = 2; cp = c & 0x1F; }
    if (e - s < n) { *len = 1; return c; }
    for (int i = 1; i < n; i++) cp = (cp << 6) | ((unsigned char)s[i] & 0x3F);
    *len = n;
    return cp;
}

/* str::trim: White_Space code points off both ends. */
static void trim(const char **s, const char **e) {
    int n;
    while (*s < *e && is_white_space(utf8_at(*s, *e, &n))) *s += n;
    while (*e > *s) {
        const char *p = *e - 1;
        while (p > *s && (((unsigned char)*p) & 0xC0) == 0x80) p--; /* the last code point's start */
        if (!is_white_space(utf8_at(p, *e, &n)) || p + n != *e) break;
        *e = p;
    }
}

static int starts(const char *s, const char *e, const char *pre) {
    size_t n = strlen(pre);
    return (size_t)(e - s) >= n && memcmp(s, pre, n) == 0;
}

/* `str::parse::<u32>()`: optional '+', decimal digits, no overflow. */
static int parse_u32(const char *s, const char *e, uint32_t *v) {
    if (s < e && *s == '+') s++;
    if (s >= e) return 0;
    uint64_t x = 0;
    for (; s < e; s++) {
        if (*s < '0' || *s > '9') return 0;
        x = x * 10 + (uint64_t)(*s - '0');
        if (x > 0xFFFFFFFFull) return 0;
    }
    *v = (uint32_t)x;
    return 1;
}

int orc_parse_id_union(const char *g, int64_t n_vocab, uint32_t *mask_out) {
    const char *s = g, *e = g + strlen(g);
    trim(&s, &e); /* strip_root: trim, "root", trim, "::=", trim */
    if (!starts(s, e, "root")) return 0;
    s += 4;
    trim(&s, &e);
    if (!starts(s, e, "::=")) return 0;
    s += 3;
    trim(&s, &e);
    size_t words = (size_t)((n_vocab + 31) / 32);
    uint32_t *tmp = (uint32_t *)calloc(words ? words : 1, sizeof(uint32_t));
    if (!tmp) return 0;
    int any = 0;
    const char *part = s;
    for (;;) {
        const char *bar = part;
        while (bar < e && *bar != '|') bar++;
        const char *ps = part, *pe = bar;
        trim(&ps, &pe);
        if (!starts(ps, pe, "id(") || pe == ps || pe[-1] != ')') {
            free(tmp);
            return 0;
        }
        ps += 3;
        pe -= 1;
        trim(&ps, &pe);
        uint32_t id;
        if (!parse_u32(ps, pe, &id)) {
            free(tmp);
            return 0;
        }
        any = 1;
        if ((int64_t)id < n_vocab) tmp[id >> 5] |= 1u << (id & 31);
        if (bar >= e) break;
        part = bar + 1;
    }
    if (!any) {
        free(tmp);
        return 0;
    }
    memcpy(mask_out, tmp, words * sizeof(uint32_t));
    free(tmp);
    return 1;
}

/* ---- batched helpers ------------------------------------------------------------------ */

static void row_to_f32(const void *logits, int dtype, int64_t row_stride, int64_t b,
                       int64_t n_vocab, float *dst) {
    if (dtype == 0) {
        memcpy(dst, (const float *)logits + b * row_stride, (size_t)n_vocab * sizeof(float));
    } else {
        const uint16_t *src = (const uint16_t *)logits + b * row_stride;
        for (int64_t i = 0; i < n_vocab; i++) {
            uint32_t bits = (uint32_t)src[i] << 16; /* bf16 -> f32 is exact */
            memcpy(&dst[i], &bits, 4);
        }
    }
}

typedef struct {
    int64_t r0, r1, n_vocab, row_stride, mask_stride, cap;
    const void *logits;
    int dtype;
    const bfi_smp_row_params *params;
    const uint32_t *hist, *mask;
    const int64_t *hist_off;
    const float *u;
    uint32_t *out, *ids_out, *token;
    int32_t *kind, *kept_len;
    float *probs, *s_out, *stats;
    int target_mode;
} rows_job;

static void *rows_worker(void *arg) {
    rows_job *j = (rows_job *)arg;
    size_t V = (size_t)j->n_vocab;
    float *row = (float *)malloc((V ? V : 1) * sizeof(float));
    uint32_t *ids = (uint32_t *)malloc((V ? V : 1) * sizeof(uint32_t));
    float *w = (float *)malloc((V ? V : 1) * sizeof(float));
    if (!row || !ids || !w) goto done;
    for (int64_t b = j->r0; b < j->r1; b++) {
        row_to_f32(j->logits, j->dtype, j->row_stride, b, j->n_vocab, row);
        const uint32_t *prev = NULL;
        size_t n_prev = 0;
        if (j->hist_off) {
            prev = j->hist + j->hist_off[b];
            n_prev = (size_t)(j->hist_off[b + 1] - j->hist_off[b]);
        }
        const uint32_t *m = j->mask ? j->mask + b * j->mask_stride : NULL;
        orc_target_info info;
        float *s_row = j->s_out ? j->s_out + b * j->n_vocab : NULL;
        if (orc_target(row, V, prev, n_prev, &j->params[b], m, ids, w, s_row, &info) != 0)
            continue;
        uint32_t tok = info.kind == 0 ? info.token : orc_draw(ids, w, (size_t)info.len, j->u[b]);
        if (!j->target_mode) {
            j->out[b] = tok;
            continue;
        }
        j->token[b] = tok;
        j->kind[b] = info.kind;
        j->kept_len[b] = info.kind == 0 ? 0 : (int32_t)info.len;
        if (info.kind == 1) {
            int64_t n = info.len < j->cap ? info.len : j->cap;
            memcpy(j->ids_out + b * j->cap, ids, (size_t)n * sizeof(uint32_t));
            memcpy(j->probs + b * j->cap, w, (size_t)n * sizeof(float));
        }
        if (j->stats) {
            j->stats[b * 8 + 0] = info.max;
            j->stats[b * 8 + 1] = info.sum;
            j->stats[b * 8 + 2] = (float)info.len_k;
            j->stats[b * 8 + 3] = (float)info.len_p;
            j->stats[b * 8 + 4] = (float)info.len_m;
            j->stats[b * 8 + 5] = (float)info.sorted;
            j->stats[b * 8 + 6] = (float)info.minp_fallback;
            j->stats[b * 8 + 7] = 0.0f;
        }
    }
done:
    free(row);
    free(ids);
    free(w);
    return NULL;
}

static void run_rows(rows_job *tmpl, int64_t n_rows, int threads) {
    if (threads < 1) threads = 1;
    if (threads > n_rows) threads = (int)(n_rows > 0 ? n_rows : 1);
    pthread_t th[256];
    rows_job jobs[256];
    if (threads > 256) threads = 256;
    for (int t = 0; t < threads; t++) {
        jobs[t] = *tmpl;
        jobs[t].r0 = n_rows * t / threads;
        jobs[t].r1 = n_rows * (t + 1) / threads;
    }
    if (threads == 1) {
        rows_worker(&jobs[0]);
        return;
    }
    for (int t = 0; t < threads; t++) pthread_create(&th[t], NULL, rows_worker, &jobs[t]);
    for (int t = 0; t < threads; t++) pthread_join(th[t], NULL);
}

void orc_sample_rows(int64_t n_rows, int64_t n_vocab, const void *logits, int dtype,
                     int64_t row_stride, const bfi_smp_row_params *params, const uint32_t *hist,
                     const int64_t *hist_off, const uint32_t *mask, int64_t mask_stride,
                     const float *u, uint32_t *out, int threads) {
    rows_job j;
    memset(&j, 0, sizeof(j));
    j.n_vocab = n_vocab;
    j.logits = logits;
    j.dtype = dtype;
    j.row_stride = row_stride;
    j.params = params;
    j.hist = hist;
    j.hist_off = hist_off;
    j.mask = mask;
    j.mask_stride = mask_stride;
    j.u = u;
    j.out = out;
    run_rows(&j, n_rows, threads);
}

void orc_target_rows(int64_t n_rows, int64_t n_vocab, const void *logits, int dtype,
                     int64_t row_stride, const bfi_smp_row_params *params, const uint32_t *hist,
                     const int64_t *hist_off, const uint32_t *mask, int64_t mask_stride,
                     const float *u, uint32_t *token, int32_t *kind, int32_t *kept_len,
                     uint32_t *ids, float *probs, int64_t cap, float *s_out, float *stats,
                     int threads) {
    rows_job j;
    memset(&j, 0, sizeof(j));
    j.n_vocab = n_vocab;
    j.logits = logits;
    j.dtype = dtype;
    j.row_stride = row_stride;
    j.params = params;
    j.hist = hist;
    j.hist_off = hist_off;
    j.mask = mask;
    j.mask_stride = mask_stride;
    j.u = u;
    j.token = token;
    j.kind = kind;
    j.kept_len = kept_len;
    j.ids_out = ids;
    j.probs = probs;
    j.cap = cap;
    j.s_out = s_out;
    j.stats = stats;
    j.target_mode = 1;
    run_rows(&j, n_rows, threads);
}

/* ---- verify of one sequence: spec.rs:137-162 (judge loop) ---------------------------- */

void orc_verify_seq(const void *rows, int dtype, int64_t n_vocab, int64_t row_stride,
                    const bfi_smp_row_params *p, const uint32_t *hist, size_t n_hist,
                    const uint32_t *drafts, size_t draft_len, const uint32_t *masks,
                    int64_t mask_stride, const float *u_pairs, float u_bonus,
                    int32_t *accepted, uint32_t *next) {
    size_t V = (size_t)n_vocab;
    float *row = (float *)malloc((V ? V : 1) * sizeof(float));
    uint32_t *ids = (uint32_t *)malloc((V ? V : 1) * sizeof(uint32_t));
    float *w = (float *)malloc((V ? V : 1) * sizeof(float));
    uint32_t *h = (uint32_t *)malloc((n_hist + draft_len + 1) * sizeof(uint32_t));
    *accepted = 0;
    *next = 0;
    if (!row || !ids || !w || !h) goto done;
    if (n_hist) memcpy(h, hist, n_hist * sizeof(uint32_t));
    for (size_t i = 0; i <= draft_len; i++) {
        row_to_f32(rows, dtype, row_stride, (int64_t)i, n_vocab, row);
        const uint32_t *m = masks ? masks + (int64_t)i * mask_stride : NULL;
        size_t hn = n_hist + i; /* all_ids grows with every accepted draft (spec.rs:141-142) */
        orc_target_info info;
        if (orc_target(row, V, h, hn, p, m, ids, w, NULL, &info) != 0) goto done;
        if (i == draft_len) { /* all accepted: what the next step's pick() samples */
            *next = info.kind == 0 ? info.token : orc_draw(ids, w, (size_t)info.len, u_bonus);
            break;
        }
        uint32_t rej = 0;
        int acc = orc_judge(info.kind, info.token, ids, w, (size_t)info.len, drafts[i],
                            u_pairs[2 * i], u_pairs[2 * i + 1], &rej);
        if (!acc) {
            *next = rej;
            break;
        }
        *accepted = (int32_t)(i + 1);
        h[n_hist + i] = drafts[i];
    }
done:
    free(row);
    free(ids);
    free(w);
    free(h);
}

/* ---- the output head (crates/bfi-core/src/cpu.rs) ---------------------------------------- */

/* cpu.rs:92-120: mean_sq = sum(v * v) / d; scale = (mean_sq + eps).sqrt().recip();
 * out = x * scale * w. */
void orc_rms_norm(const float *x, const float *w, int w_per_row, float eps, int64_t n_rows, int64_t d,
                  float *out) {
    for (int64_t r = 0; r < n_rows; r++) {
        const float *xs = x + r * d;
        const float *ws = w_per_row ? w + r * d : w;
        float s = -0.0f;
        for (int64_t i = 0; i < d; i++) s = s + xs[i] * xs[i];
        const float mean_sq = s / (float)d;
        const float scale = 1.0f / sqrtf(mean_sq + eps);
        for (int64_t i = 0; i < d; i++) out[r * d + i] = xs[i] * scale * ws[i];
    }
}

/* cpu.rs:498-514: out[t][o] = dot(w[o], x[t]), the dot a sequential f32 sum of products. */
void orc_matmul_f32(const float *w, const float *x, int64_t n_tokens, int64_t n_out, int64_t n_in,
                    float *out) {
    for (int64_t t = 0; t < n_tokens; t++)
        for (int64_t o = 0; o < n_out; o++) {
            const float *wr = w + o * n_in, *xr = x + t * n_in;
            float s = -0.0f;
            for (int64_t i = 0; i < n_in; i++) s = s + wr[i] * xr[i];
            out[t * n_out + o] = s;
        }
}

/* ---- lm_head weight formats (crates/bfi-gguf/src/types/, one file a format) ---------------- */

/* IEEE binary16 widened to binary32 (f16.rs:4-6, the `half` crate's exact conversion). */
static float orc_f16(const uint8_t *p) {
    const uint16_t h = (uint16_t)(p[0] | (p[1] << 8));
    const uint32_t sign = (uint32_t)(h >> 15) << 31, ex = (h >> 10) & 0x1Fu, man = h & 0x3FFu;
    float v;
    if (ex == 0) {
        v = ldexpf((float)man, -24); /* subnormal (or zero): man * 2^-24, exact */
        uint32_t b;
        memcpy(&b, &v, 4);
        b |= sign;
        memcpy(&v, &b, 4);
        return v;
    }
    uint32_t b = ex == 31 ? (sign | 0x7F800000u | (man << 13)) : (sign | ((ex - 15u + 127u) << 23) | (man << 13));
    memcpy(&v, &b, 4);
    return v;
}

/* dequant_row of each type, for n weights (whole blocks): f16.rs, bf16.rs, q8_0.rs:4-9,
 * q4_0.rs:4-12, q4_k.rs:6-29, q5_k.rs:6-36, q6_k.rs:4-29, q1_0.rs, pq2_0.rs, ptq1_0.rs. Returns 0, or -1 for a type not
 * restated. */
int orc_dequant(int type, const uint8_t *src, int64_t n, float *dst) {
    for (int64_t i = 0; i < n; i++) {
        float v;
        if (type == 1) {
            v = orc_f16(src + 2 * i);
        } else if (type == 30) {
            const uint32_t b = ((uint32_t)src[2 * i] | ((uint32_t)src[2 * i + 1] << 8)) << 16;
            memcpy(&v, &b, 4);
        } else if (type == 8) {
            const uint8_t *blk = src + (i / 32) * 34;
            const float d = orc_f16(blk);
            v = (float)(int8_t)blk[2 + i % 32] * d;
        } else if (type == 2) {
            const uint8_t *blk = src + (i / 32) * 18;
            const float d = orc_f16(blk);
            const int64_t j = i % 32;
            const uint8_t byte = blk[2 + (j % 16)];
            v = ((float)(j < 16 ? (byte & 0x0F) : (byte >> 4)) - 8.0f) * d;
        } else if (type == 12 || type == 13) {
            /* q4_k.rs:6-29, q5_k.rs:6-36, k_scale.rs:3-11 */
            const int bb = type == 12 ? 144 : 176;
            const uint8_t *blk = src + (i / 256) * bb, *scl = blk + 4;
            const int64_t k = i % 256, group = k / 64, hi = (k % 64) / 32, l = k % 32;
            const int j = (int)(2 * group + hi);
            unsigned sc, mn;
            if (j < 4) {
                sc = scl[j] & 63;
                mn = scl[j + 4] & 63;
            } else {
                sc = (scl[j + 4] & 0x0F) | ((scl[j - 4] >> 6) << 4);
                mn = (scl[j + 4] >> 4) | ((scl[j] >> 6) << 4);
            }
            const float d = orc_f16(blk), dmin = orc_f16(blk + 2);
            const float d1 = d * (float)sc, m1 = dmin * (float)mn;
            const uint8_t byte = blk[(type == 12 ? 16 : 48) + group * 32 + l];
            float qv = (float)(hi ? (byte >> 4) : (byte & 0x0F));
            if (type == 13) qv = qv + (((blk[16 + l] >> j) & 1) ? 16.0f : 0.0f);
            const float p = d1 * qv;
            v = p - m1;
        } else if (type == 14) {
            const uint8_t *blk = src + (i / 256) * 210;
            const int64_t k = i % 256, half = k / 128, r = k % 128, l = r % 32;
            const uint8_t *ql = blk + half * 64, *qh = blk + 128 + half * 32, *sc = blk + 192 + half * 8;
            const float d = orc_f16(blk + 208);
            int q;
            float s;
            if (r < 32) {
                q = ((ql[l] & 0x0F) | ((qh[l] & 3) << 4)) - 32;
                s = (float)(int8_t)sc[l / 16];
            } else if (r < 64) {
                q = ((ql[l + 32] & 0x0F) | (((qh[l] >> 2) & 3) << 4)) - 32;
                s = (float)(int8_t)sc[l / 16 + 2];
            } else if (r < 96) {
                q = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                s = (float)(int8_t)sc[l / 16 + 4];
            } else {
                q = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                s = (float)(int8_t)sc[l / 16 + 6];
            }
            v = d * s * (float)q;
        } else if (type == 41) {
            /* q1_0.rs:34-45: 18-byte blocks of 128, sign bits LSB first, set +d, clear -d */
            const uint8_t *blk = src + (i / 128) * 18;
            const int64_t j = i % 128;
            const float d = orc_f16(blk);
            v = ((blk[2 + j / 8] >> (j % 8)) & 1) ? d : -d;
        } else if (type == 142) {
            /* pq2_0.rs:26-36: 34-byte blocks of 128, 2-bit codes LSB first, (code - 1) * d */
            const uint8_t *blk = src + (i / 128) * 34;
            const int64_t j = i % 128;
            v = ((float)((blk[2 + j / 4] >> (2 * (j % 4))) & 3) - 1.0f) * orc_f16(blk);
        } else if (type == 143) {
            /* ptq1_0.rs:30-75: 28-byte blocks (qs[24], qh[2], d), base-3 digits read by
             * multiplying; weights 0..79 are digit j/16 of qs[j%16], 80..119 digit (j-80)/8 of
             * qs[16 + (j-80)%8], 120..127 digit (j-120)/2 of qh[(j-120)%2] */
            static const unsigned pow3[5] = {1, 3, 9, 27, 81};
            const uint8_t *blk = src + (i / 128) * 28;
            const int64_t j = i % 128;
            uint8_t byte;
            unsigned dig;
            if (j < 80) {
                byte = blk[j % 16];
                dig = (unsigned)(j / 16);
            } else if (j < 120) {
                byte = blk[16 + (j - 80) % 8];
                dig = (unsigned)((j - 80) / 8);
            } else {
                byte = blk[24 + (j - 120) % 2];
                dig = (unsigned)((j - 120) / 2);
            }
            const unsigned trit = ((unsigned)(uint8_t)(byte * pow3[dig]) * 3u) >> 8;
            v = ((float)trit - 1.0f) * orc_f16(blk + 26);
        } else {
            return -1;
        }
        dst[i] = v;
    }
    return 0;
}

/* matmul_quant's dot order for a type with a fused block dot (cpu.rs:550-563 with
 * q8_0.rs:11-15 / q4_0.rs:14-18): per block of `block` weights the products summed from -0.0,
 * the block sums added from +0.0; w holds the dequantized weights. block 0: one dot over the
 * row (orc_matmul_f32's order). */
void orc_matmul_blocked(const float *w, const float *x, int64_t n_tokens, int64_t n_out, int64_t n_in,
                        int64_t block, float *out) {
    if (block <= 0) {
        orc_matmul_f32(w, x, n_tokens, n_out, n_in, out);
        return;
    }
    for (int64_t t = 0; t < n_tokens; t++)
        for (int64_t o = 0; o < n_out; o++) {
            const float *wr = w + o * n_in, *xr = x + t * n_in;
            float s = 0.0f;
            for (int64_t b = 0; b < n_in; b += block) {
                float p = -0.0f;
                for (int64_t i = b; i < b + block && i < n_in; i++) p = p + wr[i] * xr[i];
                s = s + p;
            }
            out[t * n_out + o] = s;
        }
}

/* The Q1_0 row dot (cpu.rs:550-553, simd.rs:74-80, q1_0.rs:48-64) over dequantized weights
 * (+-d): per block of `block` the activations added from +0.0 with the sign of their weight,
 * that sum times the block's scale |w|, the blocks added from +0.0. */
void orc_matmul_signs(const float *w, const float *x, int64_t n_tokens, int64_t n_out, int64_t n_in,
                      int64_t block, float *out) {
    for (int64_t t = 0; t < n_tokens; t++)
        for (int64_t o = 0; o < n_out; o++) {
            const float *wr = w + o * n_in, *xr = x + t * n_in;
            float s = 0.0f;
            for (int64_t b = 0; b < n_in; b += block) {
                float p = 0.0f;
                for (int64_t i = b; i < b + block && i < n_in; i++) p = signbit(wr[i]) ? p - xr[i] : p + xr[i];
                s = s + p * fabsf(wr[b]);
            }
            out[t * n_out + o] = s;
        }
}
