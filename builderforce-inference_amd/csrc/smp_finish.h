// smp_finish.h — the end of a row: the row aggregates from the chunk results, the candidate
// list, the top-k / top-p / min-p cut and the draw or judge (sample.rs:369-423, 312-323;
// spec.rs:81-95), and the emission of the result, as the select kernel's fast finish and
// its general path use them. Templated on the kernel's LDS layout `SM`, which must provide
// u.cb.keys, misc, cpre, fx and tr; BLOCK is the including kernel's.
#pragma once
#include "smp_common.h"

namespace bfi {

// Phase timestamp into the workgroup's LDS trace (diagnostics; no-op without a trace buffer).
#define BFI_FTRACE(a, sm, i)                                                     \
    do {                                                                         \
        if ((a).trace && threadIdx.x == 0) (sm).tr[(i)] = wall_clock64();        \
    } while (0)

// (value, index) as a 64-bit key whose unsigned max is the reference's argmax (largest
// value, then lowest index; sample.rs:429-439).
__device__ __forceinline__ uint64_t argmax_key(float v, uint32_t i) { return ((uint64_t)ord32(v) << 32) | ~i; }
__device__ __forceinline__ ArgMax argmax_of_key(uint64_t k) {
    return k ? ArgMax{unord32((uint32_t)(k >> 32)), ~(uint32_t)k} : ArgMax{-__builtin_inff(), 0xFFFFFFFFu};
}
__device__ __forceinline__ float unord_or_ninf(uint32_t o) { return o ? unord32(o) : -__builtin_inff(); }

// Slot for each lane with `pred` in an LDS list whose length is *ctr: one atomic per wave.
__device__ __forceinline__ uint32_t wave_append(uint32_t* ctr, bool pred) {
    const uint64_t m = __ballot(pred);
    if (!m) return 0u;
    const int leader = __ffsll((unsigned long long)m) - 1;
    uint32_t base = 0;
    if (lane_id() == leader) base = lds_add(ctr, (uint32_t)__popcll(m));
    base = (uint32_t)__builtin_amdgcn_readlane((int)base, leader);
    return base + (uint32_t)__popcll(m & lanes_below());
}

// ---- result emission (sample / target / verify) ----------------------------------------

// Stores the row's outcome. For spec verify, `verdict` is 1 = Accept, 0 = Reject(token),
// and the last row of a sequence to finish resolves the accepted prefix (spec.rs:140-162).
template <typename SM>
__device__ __forceinline__ void emit(const KArgs& a, SM& sm, const RowCtx& C, uint32_t token, uint32_t verdict) {
    const int tid = threadIdx.x;
    if (!C.verify) {
        if (tid == 0) {
            if (a.out_tok) a.out_tok[C.row] = token;
        }
        return;
    }
    if (tid == 0) {
        a.row_res[2 * C.row] = C.judged ? verdict : 2u;
        a.row_res[2 * C.row + 1] = token;
    }
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        uint32_t prev = glb_add(&a.seq_ctr[C.seq], 1u);
        sm.misc[MISC_LAST] = prev == (uint32_t)C.dl;
    }
    __syncthreads();
    if (!sm.misc[MISC_LAST]) return;
    __threadfence();
    if (tid == 0) {
        a.seq_ctr[C.seq] = 0;
        const int base = C.seq * a.rows_per_seq;
        int acc = C.dl;
        for (int i = 0; i < C.dl; i++) {
            if (__hip_atomic_load(&a.row_res[2 * (base + i)], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0u) {
                acc = i;
                break;
            }
        }
        a.out_accepted[C.seq] = acc;
        a.out_next[C.seq] =
            __hip_atomic_load(&a.row_res[2 * (base + acc) + 1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

__device__ __forceinline__ void emit_target_token(const KArgs& a, const RowCtx& C, uint32_t tok) {
    if (threadIdx.x == 0 && a.t_kind) {
        a.t_kind[C.row] = BFI_SMP_TARGET_TOKEN;
        a.t_kept[C.row] = 0;
        a.t_listed[C.row] = 0;
        if (a.out_tok) a.out_tok[C.row] = tok;
    }
}

// Token target (greedy, min-p fallback): judge is exact equality (spec.rs:81-82).
template <typename SM>
__device__ __forceinline__ void finish_token(const KArgs& a, SM& sm, const RowCtx& C, uint32_t tok) {
    emit_target_token(a, C, tok);
    if (C.judged)
        emit(a, sm, C, tok, tok == C.draft ? 1u : 0u);
    else
        emit(a, sm, C, tok, 1u);
}

// ---- combine: bounded candidates -------------------------------------------------------
//
// The list in sm.u.cb.keys holds every element whose (penalized) value is >= th: the
// non-history elements from the chunks' candidates (complete above each chunk's bound) and
// the history ids at their penalized values. The kept set is a prefix of its sorted order
// when the cut falls inside it; `exhaustive` = every finite element is listed, and
// `minp_complete` = every element passing min-p is listed.

constexpr int64_t L_UNKNOWN = INT64_MAX;  // lies beyond the listed prefix

// Resolves L = min(L_k, L_p, L_m) (sample.rs:392-414) from the per-position flags; returns
// false when the cut lies beyond the listed prefix.
__device__ __forceinline__ bool resolve_L(int64_t Lk, int64_t Lp, int64_t Lm, int N, bool exhaustive, int64_t& L) {
    L = min(Lk, min(Lp, Lm));
    return L != L_UNKNOWN && (L <= N || exhaustive);
}

// List positions held by wave 0 in registers: position j = E * lane + e (e < E).
struct WPos {
    int64_t pos;  // -1 when absent
    int lane, e;
};
// First position (in list order) whose pred is set.
template <int E>
__device__ __forceinline__ WPos wave_first(const bool (&pred)[E]) {
    int fe = E;
#pragma clang loop unroll(full)
    for (int e = E - 1; e >= 0; e--)
        if (pred[e]) fe = e;
    const uint64_t hit = __ballot(fe < E);
    if (!hit) return WPos{-1, 0, 0};
    const int l0 = __ffsll((unsigned long long)hit) - 1;
    const int e0 = __builtin_amdgcn_readlane(fe, l0);
    return WPos{(int64_t)E * l0 + e0, l0, e0};
}
// Value of a per-position register array at position f (f.pos >= 0).
template <int E, typename T>
__device__ __forceinline__ T wave_at(const T (&v)[E], WPos f) {
    static_assert(sizeof(T) == 4, "32-bit values");
    // read every candidate from lane f.lane (wave-uniform values), then pick f.e: no
    // dynamically indexed register array
    uint32_t x = 0;
#pragma clang loop unroll(full)
    for (int e = 0; e < E; e++) {
        const uint32_t r = (uint32_t)__builtin_amdgcn_readlane(__builtin_bit_cast(int, v[e]), f.lane);
        x = e == f.e ? r : x;
    }
    return __builtin_bit_cast(T, x);
}
// Inclusive prefix sums over positions (f64).
template <int E>
__device__ __forceinline__ void wave_cum(const double (&w)[E], double (&c)[E]) {
    double run = 0.0;
#pragma clang loop unroll(full)
    for (int e = 0; e < E; e++) {
        run += w[e];
        c[e] = run;
    }
    const double pre = wave_incl_scan_d(run) - run;
#pragma clang loop unroll(full)
    for (int e = 0; e < E; e++) c[e] += pre;
}

// Lists of at most 64 * E entries: wave 0 does top-k / top-p / min-p, the listing and the
// draw or judge in registers with DPP scans and ballots, no block barrier; the other waves
// wait for the result. E = 1: the (unsorted) keys are sorted in registers here; E > 1: the
// keys in sm.u.cb.keys are already sorted. Returns false when the list does not decide the
// cut (nothing has been written then).
template <int E, typename SM>
__device__ __forceinline__ bool combine_wave(const KArgs& a, SM& sm, const RowCtx& C, int N, bool sorted, float M,
                                             float S, ArgMax rawmax, bool exhaustive, bool minp_complete) {
    enum { R_TOK = 0, R_VERDICT = 1, R_KIND = 2 };  // R_KIND: 0 weights, 1 token target, 2 undecided
    BFI_FTRACE(a, sm, 13);
    if (wave_id() == 0) {
        const int lane = lane_id();
        bool valid[E];
        float s[E], p[E];
        uint32_t idx[E];
        int64_t jj[E];
#pragma clang loop unroll(full)
        for (int e = 0; e < E; e++) {
            jj[e] = (int64_t)E * lane + e;
            valid[e] = jj[e] < N;
            uint64_t key = valid[e] ? sm.u.cb.keys[jj[e]] : 0ull;
            if (E == 1) key = wave_sort_desc(key);
            s[e] = sorted ? key_s(key) : unord32((uint32_t)key);
            idx[e] = sorted ? key_idx(key) : ~(uint32_t)(key >> 32);
            p[e] = valid[e] ? expf(s[e] - M) / S : 0.0f;  // sample.rs:383, 388
        }
        const int64_t Lk = C.kmode ? C.k : a.V;
        const int64_t lim = Lk < N ? Lk : N;
        int64_t Lp = Lk, Lm = L_UNKNOWN;
        double w[E], cum[E];
        bool pred[E];
        if (sorted && C.pmode) {  // sample.rs:397-409
#pragma clang loop unroll(full)
            for (int e = 0; e < E; e++) w[e] = (double)p[e];
            wave_cum<E>(w, cum);
#pragma clang loop unroll(full)
            for (int e = 0; e < E; e++) pred[e] = jj[e] < lim && cum[e] >= (double)C.top_p;
            const WPos f = wave_first<E>(pred);
            if (f.pos >= 0) Lp = f.pos + 1;
            else if (!(Lk <= N || exhaustive)) Lp = L_UNKNOWN;
        }
        float thresh = 0.0f;
        uint32_t kind = 0, tok = 0, verdict = 1;
        if (C.mmode) {  // sample.rs:411-414
            thresh = C.min_p * (1.0f / S);
            if (sorted) {
                const int64_t trunc = min(Lk, Lp);
                const int64_t n_in = trunc < N ? trunc : N;
#pragma clang loop unroll(full)
                for (int e = 0; e < E; e++) pred[e] = jj[e] < n_in && p[e] < thresh;
                const WPos f = wave_first<E>(pred);
                if (f.pos >= 0) Lm = f.pos;
                else if (trunc <= N) Lm = trunc;
                else if (minp_complete || exhaustive) Lm = N;
            } else {
                uint32_t c = 0;
#pragma clang loop unroll(full)
                for (int e = 0; e < E; e++) c += (valid[e] && p[e] >= thresh) ? 1u : 0u;
                c = wave_sum_u(c);
                if (minp_complete || exhaustive) Lm = c;
            }
            if (Lm == 0) {  // sample.rs:415-422
                kind = 1;
                tok = rawmax.v > -__builtin_inff() ? rawmax.i : 0u;
                verdict = C.judged ? (tok == C.draft) : 1u;
            }
        }
        int64_t L = 0;
        if (kind == 0) {
            bool ok;
            if (sorted) {
                ok = resolve_L(Lk, Lp, C.mmode ? Lm : L_UNKNOWN, N, exhaustive, L);
            } else {
                ok = Lm != L_UNKNOWN;
                L = Lm;
            }
            if (!ok) kind = 2;
        }
        if (kind == 0) {
            const int64_t nl = sorted ? (L < N ? L : N) : N;
            bool kept[E];
#pragma clang loop unroll(full)
            for (int e = 0; e < E; e++) kept[e] = sorted ? jj[e] < nl : (valid[e] && p[e] >= thresh);
            if (a.t_kind) {  // kept entries with p > 0, in draw order
                uint32_t nlst = 0;
#pragma clang loop unroll(full)
                for (int e = 0; e < E; e++) nlst += (kept[e] && p[e] > 0.0f) ? 1u : 0u;
                const uint32_t incl = wave_scan_incl(nlst, 0u, [](uint32_t x, uint32_t y) { return x + y; });
                uint32_t o = incl - nlst;
#pragma clang loop unroll(full)
                for (int e = 0; e < E; e++) {
                    if (kept[e] && p[e] > 0.0f) {
                        if ((int64_t)o < a.t_cap) {
                            a.t_ids[(int64_t)C.row * a.t_cap + o] = idx[e];
                            a.t_probs[(int64_t)C.row * a.t_cap + o] = p[e];
                        }
                        o++;
                    }
                }
                const uint32_t total = lane63(incl);
                if (lane == 0) {
                    a.t_kind[C.row] = BFI_SMP_TARGET_WEIGHTS;
                    a.t_kept[C.row] = (int32_t)L;
                    a.t_listed[C.row] = (int32_t)min((int64_t)total, a.t_cap);
                }
            }
#pragma clang loop unroll(full)
            for (int e = 0; e < E; e++) w[e] = kept[e] ? (double)p[e] : 0.0;
            wave_cum<E>(w, cum);
            const double sum = lane63(cum[E - 1]);
            if (!C.judged) {  // draw, sample.rs:312-323
                const double r = (double)C.u * sum;
#pragma clang loop unroll(full)
                for (int e = 0; e < E; e++) pred[e] = kept[e] && cum[e] >= r;
                WPos f = wave_first<E>(pred);
                if (f.pos < 0) f = WPos{0, 0, 0};
                tok = wave_at<E>(idx, f);
            } else {  // judge, spec.rs:83-95
#pragma clang loop unroll(full)
                for (int e = 0; e < E; e++) pred[e] = kept[e] && idx[e] == C.draft;
                const WPos fd = wave_first<E>(pred);
                const double p_d = fd.pos >= 0 ? (double)wave_at<E>(p, fd) : 0.0;
                if (sum > 0.0 && (double)C.u < p_d / sum) {
                    tok = C.draft;
                    verdict = 1;
                } else {
                    bool res[E];
                    bool anypos = false;
#pragma clang loop unroll(full)
                    for (int e = 0; e < E; e++) {
                        res[e] = kept[e] && jj[e] != fd.pos;
                        anypos = anypos || (res[e] && p[e] > 0.0f);
                    }
                    if (__ballot(anypos) == 0) {  // residual empty or all <= 0
                        tok = C.draft;
                        verdict = 1;
                    } else {
#pragma clang loop unroll(full)
                        for (int e = 0; e < E; e++) w[e] = res[e] ? (double)p[e] : 0.0;
                        wave_cum<E>(w, cum);
                        const double r2 = (double)C.u2 * (sum - p_d);
#pragma clang loop unroll(full)
                        for (int e = 0; e < E; e++) pred[e] = res[e] && cum[e] >= r2;
                        WPos f = wave_first<E>(pred);
                        if (f.pos < 0) f = WPos{0, 0, 0};
                        tok = wave_at<E>(idx, f);
                        verdict = 0;
                    }
                }
            }
        }
        if (lane == 0) {
            sm.misc[4 + R_TOK] = tok;
            sm.misc[4 + R_VERDICT] = verdict;
            sm.misc[4 + R_KIND] = kind;
        }
    }
    BFI_FTRACE(a, sm, 14);
    __syncthreads();
    const uint32_t tok = sm.misc[4 + R_TOK], verdict = sm.misc[4 + R_VERDICT], kind = sm.misc[4 + R_KIND];
    __syncthreads();
    BFI_FTRACE(a, sm, 15);
    if (kind == 2) return false;
    if (kind == 1) {
        finish_token(a, sm, C, tok);
        return true;
    }
    if (a.t_kind && threadIdx.x == 0 && a.out_tok) a.out_tok[C.row] = tok;
    emit(a, sm, C, tok, verdict);
    return true;
}


// Rows bounded by top-k <= CAND_CAP or min-p > 0, every chunk within CAND_CAP.
// The min-p bound on values: p >= min_p * max p needs s >= M + ln(min_p) (with a margin).
__device__ __forceinline__ float minp_bound(const RowCtx& C, float M) {
    if (!C.mmode) return -__builtin_inff();
    const float lm = logf(C.min_p);
    return M + lm - (1e-4f + 1e-5f * (fabsf(M) + fabsf(lm)));
}

// Candidate loads in flight per thread when gathering a list.
constexpr int GU = 8;

// The first GU * BLOCK candidates of the flattened chunk lists (prefix sm.cpre): thread t
// holds f = g * BLOCK + t (g < GU); absent entries read as (0, -inf).
struct CandBatch {
    Cand cd[GU];
};
template <typename SM>
__device__ __forceinline__ CandBatch load_cands(const KArgs& a, const SM& sm, int row, int nc, uint32_t b0) {
    const uint32_t tot = sm.cpre[nc];
    const Cand* cands = a.cands + (int64_t)row * nc * CAND_CAP;
    const uint32_t f0 = b0 + threadIdx.x;
    // the chunk of each f: the largest c < nc with cpre[c] <= f, by GU binary searches
    // whose LDS reads are independent (their latencies overlap)
    int lo[GU];
#pragma unroll
    for (int g = 0; g < GU; g++) lo[g] = 0;
    int top = 1;
    while (top * 2 < nc) top *= 2;
    for (int st = top; st > 0; st >>= 1) {
#pragma unroll
        for (int g = 0; g < GU; g++) {
            // c >= nc reads cpre[nc] = the total, which no f < total passes (an f beyond
            // the total loads nothing); no branch, so the GU reads go out together
            const int c = min(lo[g] + st, nc);
            lo[g] = sm.cpre[c] <= f0 + g * BLOCK ? c : lo[g];
        }
    }
    uint32_t start[GU];
#pragma unroll
    for (int g = 0; g < GU; g++) start[g] = sm.cpre[lo[g]];
    CandBatch B;
#pragma unroll
    for (int g = 0; g < GU; g++) {
        const uint32_t f = f0 + g * BLOCK;
        B.cd[g].idx = 0;
        B.cd[g].x = -__builtin_inff();
        if (f < tot) B.cd[g] = cands[(int64_t)lo[g] * CAND_CAP + (f - start[g])];
    }
    return B;
}

// Appends the candidates of B whose exact value is >= th and that `excluded` does not
// reject (history ids listed apart) to the list. Every thread of the block calls it.
template <typename SM, typename X>
__device__ __forceinline__ void append_cands(SM& sm, const RowCtx& C, const CandBatch& B, float th, bool sorted,
                                             X excluded) {
    float v[GU];
    uint32_t take = 0;  // bit g: entry g is appended
#pragma unroll
    for (int g = 0; g < GU; g++) {
        v[g] = raw_value(C, B.cd[g].x, true);  // masked logit / T, exact
        if (v[g] >= th && v[g] > -__builtin_inff() && !excluded(B.cd[g].idx))
            take |= 1u << g;
    }
    // one reservation per wave for all its entries
    const uint32_t n = (uint32_t)__popc(take);
    const uint32_t incl = wave_scan_incl(n, 0u, [](uint32_t x, uint32_t y) { return x + y; });
    const uint32_t tot = lane63(incl);
    uint32_t base = 0;
    if (tot) {
        if (lane_id() == 0) base = lds_add(&sm.misc[MISC_N], tot);
        base = (uint32_t)__builtin_amdgcn_readfirstlane((int)base);
    }
    uint32_t slot = base + incl - n;
#pragma unroll
    for (int g = 0; g < GU; g++) {
        if ((take >> g) & 1u) {
            if (slot < NMAX)
                sm.u.cb.keys[slot] = sorted ? key64(v[g], B.cd[g].idx)
                                            : (((uint64_t)(~B.cd[g].idx) << 32) | ord32(v[g]));
            slot++;
        }
    }
}


// append_cands' exclusion for lists without a separate history
struct NoExclusion {
    __device__ __forceinline__ bool operator()(uint32_t) const { return false; }
};
constexpr NoExclusion no_exclusion{};

// Candidates chunk c contributes to a list complete above th (the repair pass re-reads the
// chunks whose own bound lies above th).
__device__ __forceinline__ uint32_t chunk_take(const ChunkPart& mine, float th) {
    return (mine.theta <= th && mine.m >= th) ? mine.ncand : 0u;
}

// ---- fast finish ------------------------------------------------------------------------
//
// The common row, on short code (three barriers): every chunk handed over a candidate list,
// penalties (if any) were applied by the stream pass, and the list above the row's bound
// holds at most 8 * WAVE entries (WIDE; else WAVE). One wave forms the row aggregates from
// the chunk results with DPP (no LDS round trips), the block gathers the list, one wave
// sorts and draws (combine_wave). `row_ctx()` returns the row's context; it is called after
// the chunk results' loads are issued. Returns false, having emitted nothing, for any other
// row. sort_list_regs (WIDE) must be visible where this is instantiated.
template <bool WIDE, typename SM, typename F>
__device__ __forceinline__ bool select_fast(const KArgs& a, SM& sm, int row, F row_ctx) {
    const int tid = threadIdx.x, lane = lane_id();
    const int nc = a.n_chunks;
    if (nc > WAVE) return false;
    // the chunk results go out before the row's parameters: the two latencies overlap
    ChunkPart mine;
    mine.m = -__builtin_inff();
    mine.sum = 0.0;
    mine.arg = 0xFFFFFFFFu;
    mine.ncand = 0;
    mine.theta = -__builtin_inff();
    mine.raw_m = -__builtin_inff();
    mine.raw_arg = 0xFFFFFFFFu;
    if (tid < nc) mine = a.parts[(int64_t)row * nc + tid];
    // The first BLOCK / nc candidates of every chunk go out with the chunk results (thread t:
    // chunk t / per, slot t % per); when no chunk hands over more, they are the whole list and
    // the gather needs no second round trip. Slots past a chunk's count are ignored.
    const uint32_t per = (uint32_t)BLOCK / (uint32_t)nc;
    const uint32_t sc = (uint32_t)tid / per, sj = (uint32_t)tid % per;
    Cand spec{0u, -__builtin_inff()};
    if (sc < (uint32_t)nc) spec = a.cands[((int64_t)row * nc + sc) * CAND_CAP + sj];
    const RowCtx C = row_ctx();
    if (!C.active) return true;  // a verify row past its draft: nothing to emit
    BFI_FTRACE(a, sm, 8);
    const bool cand_row = C.kmode || C.pmode || C.mmode;
    if (C.pen_hash || !(C.greedy || (cand_row && C.stream_ok))) return false;
    const bool sorted = C.kmode || C.pmode;  // else min-p only: index order (sample.rs:411-414)
    enum { F_STATUS = 0, F_TOK = 1, F_M = 2, F_S = 3, F_TH = 4, F_THM = 5, F_RAWV = 6, F_RAWI = 7 };
    uint32_t* fx = sm.fx;
    if (wave_id() == 0) {
        const bool in = lane < nc;
        uint32_t status = 0;  // 0: list, 1: token (greedy), 2: leave to k_select, 3: list, prefetched
        if (C.greedy) {  // sample.rs:369-371, 429-439: argmax of the penalized logits
            const ArgMax am = argmax_of_key(wave_max_u64(in ? argmax_key(mine.m, mine.arg) : 0ull));
            status = 1;
            if (lane == 0) fx[F_TOK] = am.v > -__builtin_inff() ? am.i : 0u;
        } else {
            const bool open = in && (mine.ncand == NCAND_UNBOUNDED || mine.ncand == NCAND_OVERFLOW);
            const float M = wave_max(in ? mine.m : -__builtin_inff());
            if (__ballot(open) || !(M > -__builtin_inff())) {
                status = 2;
            } else {
                // S: the chunks' sums moved to the row max (sample.rs:376-386)
                const double wc = in && mine.m > -__builtin_inff() ? mine.sum * (double)expf(mine.m - M) : 0.0;
                const float S = (float)wave_sum_d(wc);
                const float th_m = minp_bound(C, M);
                const float th = fmaxf(wave_max(in ? mine.theta : -__builtin_inff()), th_m);
                const uint32_t take = in ? chunk_take(mine, th) : 0u;
                if (__ballot(take > per) == 0ull) status = 3;
                const uint32_t incl = wave_scan_incl(take, 0u, [](uint32_t x, uint32_t y) { return x + y; });
                if (in) sm.cpre[lane] = incl - take;
                const ArgMax rawmax = C.min_p > 1.0f
                    ? argmax_of_key(wave_max_u64(in ? argmax_key(mine.raw_m, mine.raw_arg) : 0ull))
                    : ArgMax{-__builtin_inff(), 0xFFFFFFFFu};
                if (lane == 0) {
                    sm.cpre[nc] = lane63(incl);
                    fx[F_M] = __float_as_uint(M);
                    fx[F_S] = __float_as_uint(S);
                    fx[F_TH] = __float_as_uint(th);
                    fx[F_THM] = __float_as_uint(th_m);
                    fx[F_RAWV] = __float_as_uint(rawmax.v);
                    fx[F_RAWI] = rawmax.i;
                    sm.misc[MISC_N] = 0;
                }
            }
        }
        if (lane == 0) fx[F_STATUS] = status;
    }
    __syncthreads();
    BFI_FTRACE(a, sm, 1);
    const uint32_t status = fx[F_STATUS];
    if (status == 1) {
        finish_token(a, sm, C, fx[F_TOK]);
        return true;
    }
    if (status == 2) return false;
    const float M = __uint_as_float(fx[F_M]), S = __uint_as_float(fx[F_S]);
    const float th = __uint_as_float(fx[F_TH]), th_m = __uint_as_float(fx[F_THM]);
    const ArgMax rawmax{__uint_as_float(fx[F_RAWV]), fx[F_RAWI]};
    if (status == 3) {
        CandBatch B;
#pragma unroll
        for (int g = 0; g < GU; g++) B.cd[g] = Cand{0u, -__builtin_inff()};
        if (sc < (uint32_t)nc && sj < sm.cpre[sc + 1] - sm.cpre[sc]) B.cd[0] = spec;
        append_cands(sm, C, B, th, sorted, no_exclusion);
    } else {
        for (uint32_t b0 = 0; b0 < sm.cpre[nc]; b0 += GU * BLOCK)  // uniform trip count
            append_cands(sm, C, load_cands(a, sm, row, nc, b0), th, sorted, no_exclusion);
    }
    __syncthreads();
    BFI_FTRACE(a, sm, 3);
    if (a.t_stats && tid == 0) {
        a.t_stats[row * 4 + 0] = M;
        a.t_stats[row * 4 + 1] = S;
        a.t_stats[row * 4 + 3] = 1.0f;
    }
    const int N = (int)sm.misc[MISC_N];
    if (a.trace && tid == 0) sm.tr[6] = ((uint64_t)sm.cpre[nc] << 32) | (uint32_t)N;
    const bool exhaustive = !(th > -__builtin_inff());
    const bool minp_complete = th <= th_m;
    if (N <= WAVE) return combine_wave<1>(a, sm, C, N, sorted, M, S, rawmax, exhaustive, minp_complete);
    if constexpr (WIDE) {
        if (N > 8 * WAVE || N > BLOCK) return false;
        sort_list_regs(sm, N);
        BFI_FTRACE(a, sm, 5);
        return combine_wave<8>(a, sm, C, N, sorted, M, S, rawmax, exhaustive, minp_complete);
    }
    return false;
}


}  // namespace bfi
