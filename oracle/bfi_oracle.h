/*
 * bfi_oracle.h — TEST INFRASTRUCTURE ONLY.
 *
 * A CPU restatement, in plain C, of the reference token sampler
 * (crates/bfi-runtime/src/sample.rs, crates/bfi-runtime/src/engine/spec.rs of
 * SeanHogg/builderforce-inference). It is the parity checker for the HIP library and the
 * CPU baseline of bench.py. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product library never links or calls it.
 *
 * Arithmetic follows the reference line by line in IEEE f32 (built with
 * -ffp-contract=off, no fast-math, glibc expf — the libm call Rust's f32::exp lowers to on
 * x86_64-unknown-linux-gnu). Sorting is a stable merge sort with the reference comparator
 * (descending probability, NaN compares Equal).
 *
 * Pinning status (what checks each function; see tests/test_oracle*.py):
 *   orc_rng_*, orc_slot_rng_seed   golden vectors (tests/golden/rng_vectors.json)
 *   orc_argmax, orc_draw           reference KATs + brute force on tiny inputs
 *   orc_target, orc_sample         13 reference KATs (sample.rs:466-689) + numpy/f64
 *                                  closed forms (softmax, top-k via argsort, top-p cumsum,
 *                                  min-p) + brute force over all params at V <= 8
 *   orc_judge, orc_draft           6 reference KATs (spec.rs:193-256) incl. the Monte-Carlo
 *                                  distribution check
 *   orc_parse_id_union             reference KAT grammar_id_mask_rejects_forbidden_token;
 *                                  the Unicode White_Space trim (str::trim) against
 *                                  oracle/constraint.py's independent statement
 *   frequency penalty              parity unpinned: absent in the reference (sample.rs:18-21);
 *                                  this file defines the extension, pinned only by the
 *                                  closed form l - f*count in the tests
 *   packed allow-mask              equivalent to the id-union HashSet mask (sample.rs:331-337);
 *                                  pinned by comparing against orc_parse_id_union
 *   orc_rms_norm, orc_matmul_f32   reference KATs rms_norm_ones / matmul_f32_identity
 *                                  (cpu.rs:835-855) + numpy's sequential float32 accumulate
 *                                  and correctly rounded sqrt on random rows
 *   orc_dequant                    F16: all 65,536 codes against numpy's float16; BF16: against
 *                                  torch's bfloat16; Q8_0 / Q4_0 / Q4_K / Q5_K / Q6_K: the
 *                                  reference's KATs (q8_0.rs, q4_0.rs, q6_k.rs,
 *                                  types/mod.rs:300-328) and encoder-built layouts with known
 *                                  values at every nibble, high bit and (packed) scale;
 *                                  Q1_0 / PQ2_0 / PTQ1_0: the reference's KATs (q1_0.rs,
 *                                  pq2_0.rs, ptq1_0.rs tests) and a base-3 encoder's blocks
 *                                  decoded back at every weight
 *   orc_matmul_blocked             a closed form where block sums keep what one row sum loses
 *                                  (2^24 then 63 ones: 2^24 + 32 against 2^24)
 *   orc_matmul_signs               the same closed form through the scale (a block of ones
 *                                  summed before its scale of 2^-7) and a product-first sum
 *                                  that differs from it
 */
#ifndef BFI_ORACLE_H
#define BFI_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#include "../include/bfi_sampler.h" /* bfi_smp_row_params layout only */

#ifdef __cplusplus
extern "C" {
#endif

typedef struct orc_target_info {
    int32_t kind;     /* 0 = Token, 1 = Weights */
    uint32_t token;   /* Token id (kind 0) */
    int64_t len;      /* kept length (kind 1) */
    float max;        /* softmax max (T > 0) */
    float sum;        /* softmax sequential f32 sum (T > 0) */
    int64_t len_k;    /* vals.len() after top-k (-1 if inactive) */
    int64_t len_p;    /* vals.len() after top-p (-1 if inactive) */
    int64_t len_m;    /* vals.len() after min-p (-1 if inactive) */
    int32_t sorted;   /* 1 when vals were sorted (top-k or top-p active) */
    int32_t minp_fallback; /* 1 when min-p emptied vals and argmax(masked) was returned */
} orc_target_info;

uint64_t orc_rng_next(uint64_t *state);
float orc_rng_f32(uint64_t *state);
uint64_t orc_slot_rng_seed(uint64_t seed, uint64_t prompt_len);

uint32_t orc_argmax(const uint32_t *ids, const float *v, size_t n);
uint32_t orc_draw(const uint32_t *ids, const float *w, size_t n, float u);

/* target(): out_ids/out_w need room for n_vocab entries. out_s (nullable, n_vocab floats)
 * receives the transformed logits: penalized (greedy) or penalized / T (T > 0). */
int orc_target(const float *logits, size_t n_vocab, const uint32_t *prev, size_t n_prev,
               const bfi_smp_row_params *p, const uint32_t *mask, uint32_t *out_ids,
               float *out_w, float *out_s, orc_target_info *info);
uint32_t orc_sample(const float *logits, size_t n_vocab, const uint32_t *prev, size_t n_prev,
                    const bfi_smp_row_params *p, const uint32_t *mask, float u);

/* judge(): returns 1 = Accept, 0 = Reject (then *reject_token is set). */
int orc_judge(int32_t kind, uint32_t token, const uint32_t *ids, const float *w, size_t n,
              uint32_t d, float u, float u2, uint32_t *reject_token);
size_t orc_draft(const uint32_t *ctx, size_t len, size_t k, size_t ngram_max, size_t ngram_min,
                 uint32_t *out);
int orc_parse_id_union(const char *grammar, int64_t n_vocab, uint32_t *mask_out);

/* Batched helpers (threads = 0 -> 1). dtype 0 = f32, 1 = bf16 (upcast exactly to f32). */
void orc_sample_rows(int64_t n_rows, int64_t n_vocab, const void *logits, int dtype,
                     int64_t row_stride, const bfi_smp_row_params *params, const uint32_t *hist,
                     const int64_t *hist_off, const uint32_t *mask, int64_t mask_stride,
                     const float *u, uint32_t *out, int threads);

/* target() per row into [n_rows][cap] outputs (mirrors bfi_smp_target_rows). */
void orc_target_rows(int64_t n_rows, int64_t n_vocab, const void *logits, int dtype,
                     int64_t row_stride, const bfi_smp_row_params *params, const uint32_t *hist,
                     const int64_t *hist_off, const uint32_t *mask, int64_t mask_stride,
                     const float *u, uint32_t *token, int32_t *kind, int32_t *kept_len,
                     uint32_t *ids, float *probs, int64_t cap, float *s_out, float *stats,
                     int threads);

/* Spec verify of one sequence (spec.rs:137-162 without the host stop rules): rows are
 * draft_len + 1 logits rows `row_stride` apart; masks one per row or NULL. */
void orc_verify_seq(const void *rows, int dtype, int64_t n_vocab, int64_t row_stride,
                    const bfi_smp_row_params *p, const uint32_t *hist, size_t n_hist,
                    const uint32_t *drafts, size_t draft_len, const uint32_t *masks,
                    int64_t mask_stride, const float *u_pairs, float u_bonus,
                    int32_t *accepted, uint32_t *next);

/* The CPU backend's output head (crates/bfi-core/src/cpu.rs), which produces the logits the
 * sampler reads (qwen3.rs:258-265 `head`): rms_norm (cpu.rs:92-120) and matmul_f32
 * (cpu.rs:498-514 over scalar_dot_f32, simd.rs:61-63). Sums run one f32 addition at a time
 * in index order from -0.0 (Rust's f32 `Sum`). w of rms_norm: [d] or [n_rows, d]. */
void orc_rms_norm(const float *x, const float *w, int w_per_row, float eps, int64_t n_rows, int64_t d,
                  float *out);
void orc_matmul_f32(const float *w, const float *x, int64_t n_tokens, int64_t n_out, int64_t n_in,
                    float *out);
int orc_dequant(int type, const uint8_t *src, int64_t n, float *dst);
void orc_matmul_blocked(const float *w, const float *x, int64_t n_tokens, int64_t n_out, int64_t n_in,
                        int64_t block, float *out);
void orc_matmul_signs(const float *w, const float *x, int64_t n_tokens, int64_t n_out, int64_t n_in,
                      int64_t block, float *out);

#ifdef __cplusplus
}
#endif

#endif
