/*
 * bfi_sampler.h — C ABI of the MI355X (gfx950) token sampler.
 *
 * This library replaces the host-side token-sampling path of bfi-runtime:
 *   - `sample()` / `target()` / `draw()`      crates/bfi-runtime/src/sample.rs:304-427
 *   - the per-step sampling of `generate_batch` crates/bfi-runtime/src/engine/mod.rs:297-337
 *   - the verify loop of `take_token_spec`      crates/bfi-runtime/src/engine/spec.rs:101-181
 *     with `judge()`                            crates/bfi-runtime/src/engine/spec.rs:79-97
 *
 * Conventions
 *   - Every entry point returns an `int` status (BFI_SMP_OK on success); no C++
 *     exception or abort crosses this boundary. On failure the message is kept
 *     per context (bfi_smp_last_error(ctx)), or per thread when ctx is NULL.
 *   - Buffers named `d_*` are device pointers (HIP device memory on the context's
 *     device); `stream` is a hipStream_t (NULL = legacy default stream). Calls on a
 *     device pointer API are asynchronous with respect to the host.
 *   - A context owns a device workspace and per-row counters. One context must not be
 *     used by two host threads at the same time, and two calls on the same context
 *     must not overlap on different streams.
 *   - Semantics follow the reference's `target()` step order exactly:
 *     mask -> repeat -> presence -> (frequency) -> greedy exit -> /T -> softmax
 *     -> top-k -> top-p -> min-p -> draw.  Token ids must equal the reference
 *     sampler's except where u lies within 1e-6 of a CDF boundary or logits tie.
 */
#ifndef BFI_SAMPLER_H
#define BFI_SAMPLER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BFI_SMP_ABI_VERSION 1

/* Status codes. */
#define BFI_SMP_OK 0
#define BFI_SMP_EINVAL 1 /* bad argument (null pointer, size out of range, bad dtype) */
#define BFI_SMP_EHIP 2   /* a HIP runtime call failed (no device, launch failure, ...) */
#define BFI_SMP_ENOMEM 3 /* device workspace allocation failed */

/* Logit element types. */
#define BFI_SMP_F32 0
#define BFI_SMP_BF16 1

/* Target kinds written by bfi_smp_target_rows (sample.rs:297-301 `Target`). */
#define BFI_SMP_TARGET_TOKEN 0
#define BFI_SMP_TARGET_WEIGHTS 1

/*
 * Per-row numeric sampling parameters: the numeric fields of `SampleParams`
 * (crates/bfi-runtime/src/sample.rs:9-31). String constraints (grammar, json_object,
 * tool_choice) cross this boundary already resolved into a packed allow-mask.
 * The reference broadcasts one SampleParams over a batch (engine/mod.rs:297-301);
 * an array of these with identical entries reproduces that.
 */
typedef struct bfi_smp_row_params {
    float temperature;       /* sample.rs:13   <= 0 -> greedy argmax of penalized logits */
    int32_t top_k;           /* sample.rs:15   active iff 0 < top_k < n_vocab */
    float top_p;             /* sample.rs:16   active iff top_p < 1 */
    float min_p;             /* sample.rs:17   active iff min_p > 0 */
    float repeat_penalty;    /* sample.rs:18-19 active iff |rp - 1| > FLT_EPSILON and history non-empty */
    float presence_penalty;  /* sample.rs:20-21 active iff != 0 and history non-empty */
    float frequency_penalty; /* extension (absent in the reference): l -= f * count(id in history),
                                applied after presence; 0 = off, bit-identical to the reference */
    uint32_t reserved;       /* must be 0 */
} bfi_smp_row_params;

typedef struct bfi_smp_ctx bfi_smp_ctx;

/* ---- context ------------------------------------------------------------ */

/* Creates a context on HIP device `device`. No counterpart in the reference (its
 * sampler is a free function); it holds what the reference re-creates per call. */
int bfi_smp_create(int device, bfi_smp_ctx **out);
void bfi_smp_destroy(bfi_smp_ctx *ctx);
/* Last error message of `ctx` (or of the calling thread when ctx is NULL). Never NULL. */
const char *bfi_smp_last_error(const bfi_smp_ctx *ctx);
int bfi_smp_abi_version(void);

/* Profiling (no counterpart in the reference; for benchmarks): while enabled, every launch
 * times its three kernels (the streaming pass over the logits, the quantizing pass, the
 * per-row pass) with start/stop HIP events recorded in the kernels' own dispatch packets on
 * the caller's stream. Profiling may be switched on for some launches only; the record
 * keeps them until bfi_smp_profile waits for them, writes the summed times in ms to
 * kernel_ms[0..3] (k_stream, k_quant, k_row, and the whole call from k_stream's start to
 * k_row's end, gaps included) and clears it (at most 65536 launches). */
int bfi_smp_set_profiling(bfi_smp_ctx *ctx, int enabled);
int bfi_smp_profile(bfi_smp_ctx *ctx, double *kernel_ms, int64_t *launches);

/* Phase trace (diagnostics, no counterpart in the reference): while enabled, each launch
 * records wall-clock (100 MHz) timestamps at phase boundaries of every workgroup into a
 * context buffer: 8 words per streaming workgroup (row-major by row, chunk), then 16 per
 * row for its row-pass workgroup.
 * bfi_smp_trace copies the last launch's record (synchronous) and returns the word count. */
int bfi_smp_set_tracing(bfi_smp_ctx *ctx, int enabled);
int64_t bfi_smp_trace(bfi_smp_ctx *ctx, uint64_t *out, int64_t max_words);

/* ---- batched sampling: generate_batch's per-step call ------------------- */

/*
 * Samples one token per row: out[b] = sample(masked(row b), hist[b], params[b]) with the
 * draw's uniform supplied per row (the reference uses Rng(seed).f32(), sample.rs:307).
 *   d_logits     n_rows rows of n_vocab logits, `row_stride` elements apart (dtype F32/BF16)
 *   d_params     n_rows bfi_smp_row_params
 *   d_hist       penalty histories, concatenated (u32 token ids; ids >= n_vocab are ignored)
 *   d_hist_off   n_rows + 1 offsets into d_hist (int64); row b uses [off[b], off[b+1])
 *                (may be NULL when no row uses a penalty)
 *   d_mask       NULL, or n_rows packed allow-masks of ceil(n_vocab/32) u32 words,
 *                `mask_stride` words apart; bit (id & 31) of word (id >> 5) set = allowed.
 *                Disallowed logits become -inf before the penalties (sample.rs:331-337).
 *   d_u          n_rows uniforms in [0, 1)
 *   d_out        n_rows token ids
 * Replaces: sample.rs:304-309 called once per live slot in engine/mod.rs:316-322.
 */
int bfi_smp_sample_rows(bfi_smp_ctx *ctx, const void *d_logits, int dtype, int64_t n_rows,
                        int64_t n_vocab, int64_t row_stride, const bfi_smp_row_params *d_params,
                        const uint32_t *d_hist, const int64_t *d_hist_off, const uint32_t *d_mask,
                        int64_t mask_stride, const float *d_u, uint32_t *d_out, void *stream);

/*
 * bfi_smp_sample_rows without any allocation: no counterpart in the reference; for callers
 * that cannot allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). Same arguments and results as bfi_smp_sample_rows, but
 * the kernels' workspace is a fixed array of BFI_SMP_NOALLOC_BYTES per device, which the
 * library holds from its load until the process ends (its address is resolved once per
 * device by bfi_smp_create). A call whose rows need more workspace than that fails with
 * BFI_SMP_EINVAL and a message naming both sizes (8 rows at n_vocab = 151936, or 64
 * rows at n_vocab = 16384). Every call on a device shares the one array: calls that overlap
 * on one GPU (other streams, other contexts, other threads) race, so the caller orders them.
 * Profiling and tracing records are not kept for these calls.
 */
#define BFI_SMP_NOALLOC_BYTES (64u << 20)
int bfi_smp_sample_rows_noalloc(bfi_smp_ctx *ctx, const void *d_logits, int dtype, int64_t n_rows,
                                int64_t n_vocab, int64_t row_stride, const bfi_smp_row_params *d_params,
                                const uint32_t *d_hist, const int64_t *d_hist_off, const uint32_t *d_mask,
                                int64_t mask_stride, const float *d_u, uint32_t *d_out, void *stream);

/*
 * The distribution `sample` draws from, per row (sample.rs:326-427 `target()`), plus the
 * drawn token. For each row b:
 *   d_kind[b]      BFI_SMP_TARGET_TOKEN (greedy / min-p fallback) or _WEIGHTS
 *   d_token[b]     the token sample() returns with uniform d_u[b]
 *   d_kept_len[b]  length of the reference's `vals` after top-k/top-p/min-p (0 for TOKEN)
 *   d_listed[b]    entries written to d_ids/d_probs (<= min(kept_len, cap)); entries whose
 *                  probability is exactly 0 are counted in kept_len but never listed
 *   d_ids/d_probs  row-major [n_rows][cap]: the kept (id, probability) pairs in draw order
 *   d_stats        optional [n_rows][4] floats: {max, sum, kept mass, mode}
 * Replaces: sample.rs:326-427 (used by judge() in spec verify).
 */
int bfi_smp_target_rows(bfi_smp_ctx *ctx, const void *d_logits, int dtype, int64_t n_rows,
                        int64_t n_vocab, int64_t row_stride, const bfi_smp_row_params *d_params,
                        const uint32_t *d_hist, const int64_t *d_hist_off, const uint32_t *d_mask,
                        int64_t mask_stride, const float *d_u, uint32_t *d_token, int32_t *d_kind,
                        int32_t *d_kept_len, int32_t *d_listed, uint32_t *d_ids, float *d_probs,
                        int64_t cap, float *d_stats, void *stream);

/* ---- spec-lookup verify ------------------------------------------------- */

/*
 * Judges n_seq drafts at once (engine/spec.rs:137-162). Sequence s owns rows
 * [s*rows_per_seq, s*rows_per_seq + draft_len[s]] of d_logits (row i = logits after
 * tokens[..=i], arch.rs:35-60). Row i (< draft_len[s]) is judged against drafts[s][i] with
 * the target built from history hist[s] + drafts[s][0..i) (spec.rs:141-142), using
 * u = d_u_pairs[(s*(rows_per_seq-1)+i)*2], u2 = ...+1 (two slot_rng draws per judged row).
 *   d_out_accepted[s]  number of leading drafts accepted by judge() (the host still applies
 *                      EOS / tool-stop / budget rules, spec.rs:148-160)
 *   d_out_next[s]      the Reject(t) correction of the first rejected draft, or, when all
 *                      draft_len[s] drafts are accepted, sample(row draft_len[s]) with
 *                      uniform d_u_bonus[s] (what the next step's pick() returns).
 *   d_mask             NULL, or one mask per logits row (n_seq*rows_per_seq rows).
 * Replaces: spec.rs:137-162 and 79-97.
 */
int bfi_smp_verify(bfi_smp_ctx *ctx, const void *d_logits, int dtype, int64_t n_seq,
                   int64_t rows_per_seq, int64_t n_vocab, int64_t row_stride,
                   const bfi_smp_row_params *d_params, const uint32_t *d_hist,
                   const int64_t *d_hist_off, const uint32_t *d_drafts, const int32_t *d_draft_len,
                   const uint32_t *d_mask, int64_t mask_stride, const float *d_u_pairs,
                   const float *d_u_bonus, int32_t *d_out_accepted, uint32_t *d_out_next,
                   void *stream);

/* ---- host-pointer drop-in for `sample()` ------------------------------- */

/*
 * `pub fn sample(logits: &[f32], prev: &[u32], p: &SampleParams) -> u32` (sample.rs:304)
 * for one host row: copies to the device, samples, copies back (synchronous).
 * `u` is the draw uniform (the reference uses Rng(p.seed).f32()). `allow_mask` (host, may
 * be NULL) is the id-union grammar as a packed mask. n_vocab == 0 returns token 0 like the
 * reference. The PCIe copy of n_vocab floats dominates; batched device-resident callers
 * should use bfi_smp_sample_rows.
 */
int bfi_smp_sample_host(bfi_smp_ctx *ctx, const float *logits, int64_t n_vocab,
                        const uint32_t *prev, int64_t n_prev, const bfi_smp_row_params *params,
                        const uint32_t *allow_mask, float u, uint32_t *out_token);

/* ---- device-resident logits: the output head ---------------------------- */

/*
 * The reference's `head` (crates/bfi-models/src/qwen3.rs:258-265: `rms_norm` then
 * `matmul_q` with f32 weights, then `tutil::logit_rows`, tutil.rs:196-207) on the device, so
 * a decode step's logits never leave HBM: d_x is [n_tokens, n_embd] f32 hidden rows, d_norm_w
 * the output norm's weights ([n_embd], or [n_tokens, n_embd] when norm_per_row != 0,
 * cpu.rs:98-115), d_w the lm_head weights [n_vocab, n_embd] f32, d_logits [n_tokens,
 * n_vocab] f32. Rounding as the CPU backend's (cpu.rs:92-120, 498-514): the mean of squares
 * and every dot product summed one f32 addition at a time in index order (from -0.0, Rust's
 * f32 `Sum`), sqrt and 1/x correctly rounded, x * scale * w left to right; the logits are
 * bit-identical to the reference's. Quantized lm_head weights: bfi_smp_dequant, then
 * bfi_smp_head_typed. Asynchronous on `stream`; n_tokens <= 2^20.
 */
int bfi_smp_head(bfi_smp_ctx *ctx, const float *d_x, const float *d_norm_w, int norm_per_row,
                 float eps, const float *d_w, int64_t n_tokens, int64_t n_embd, int64_t n_vocab,
                 float *d_logits, void *stream);

/*
 * bfi_smp_head into the context's workspace, then bfi_smp_sample_rows over those logits
 * (row_stride n_vocab, f32): the fused step of a device-resident decode loop — hidden rows in,
 * one u32 token a row out (4 bytes a row to read back instead of 4 n_vocab).
 */
int bfi_smp_head_sample_rows(bfi_smp_ctx *ctx, const float *d_x, const float *d_norm_w,
                             int norm_per_row, float eps, const float *d_w, int64_t n_tokens,
                             int64_t n_embd, int64_t n_vocab, const bfi_smp_row_params *d_params,
                             const uint32_t *d_hist, const int64_t *d_hist_off,
                             const uint32_t *d_mask, int64_t mask_stride, const float *d_u,
                             uint32_t *d_out, void *stream);

/*
 * Dequantizes n_weights weights of a GGML tensor (d_src: its bytes on the device, rows of
 * whole blocks) to f32 in d_dst, every value exactly as the reference's dequant_row computes
 * it (crates/bfi-gguf/src/types/, one file a format; replaces `dequant_tensor`, types/mod.rs, as
 * `matmul_quant` uses it, crates/bfi-core/src/cpu.rs:515-563): ggml_type 1 (F16), 30 (BF16),
 * 8 (Q8_0: q * d), 2 (Q4_0: (nibble - 8) * d), 14 (Q6_K: (d * scale) * q), 12 and 13 (Q4_K,
 * Q5_K: (d * scale) * q - dmin * min), 41 (Q1_0: +-d), 142 (PQ2_0: (code - 1) * d), 143 (PTQ1_0:
 * (trit - 1) * d). A model's lm_head is dequantized once, at load.
 * BFI_SMP_EINVAL for another type or a partial block.
 */
int bfi_smp_dequant(bfi_smp_ctx *ctx, int32_t ggml_type, const void *d_src, int64_t n_weights,
                    float *d_dst, void *stream);

/*
 * bfi_smp_head over lm_head weights dequantized from GGML type ggml_type (d_w: bfi_smp_dequant's
 * output; 0 for f32 weights), in the dot order `matmul_quant` uses for that type
 * (cpu.rs:515-563): Q8_0 and Q4_0 have a fused block dot (q8_0.rs:11-15, q4_0.rs:14-18) — each
 * 32-weight block's products summed from -0.0, the block sums added from +0.0 — when n_embd is
 * a multiple of 32; PQ2_0 and PTQ1_0 the same over 128-weight blocks (pq2_0.rs:38-42,
 * ptq1_0.rs:72-76); Q1_0 (q1_0.rs:48-64, simd.rs:74-80) adds each block's inputs with their
 * weight's sign from +0.0 and multiplies that sum by the block's scale (n_embd a multiple of
 * 128); F16, BF16, Q4_K, Q5_K, Q6_K (no block dot) and rows of partial blocks take one dot over
 * the row, as f32 weights do. Logits bit-identical to the reference's for that
 * tensor.
 */
int bfi_smp_head_typed(bfi_smp_ctx *ctx, const float *d_x, const float *d_norm_w, int norm_per_row,
                       float eps, const float *d_w, int32_t ggml_type, int64_t n_tokens,
                       int64_t n_embd, int64_t n_vocab, float *d_logits, void *stream);

/* bfi_smp_head_sample_rows over weights dequantized from ggml_type (bfi_smp_head_typed's
 * order): the fused decode step of a GGUF model with a quantized lm_head. */
int bfi_smp_head_typed_sample_rows(bfi_smp_ctx *ctx, const float *d_x, const float *d_norm_w,
                                   int norm_per_row, float eps, const float *d_w, int32_t ggml_type,
                                   int64_t n_tokens, int64_t n_embd, int64_t n_vocab,
                                   const bfi_smp_row_params *d_params, const uint32_t *d_hist,
                                   const int64_t *d_hist_off, const uint32_t *d_mask,
                                   int64_t mask_stride, const float *d_u, uint32_t *d_out,
                                   void *stream);

/* ---- host-side helpers (no GPU work) ------------------------------------ */

/* xorshift64 step of `Rng::next_u64` (sample.rs:445-455); updates *state. */
uint64_t bfi_rng_next_u64(uint64_t *state);
/* `Rng::f32` (sample.rs:457-459): (next_u64 >> 40) / 2^24. */
float bfi_rng_f32(uint64_t *state);
/* Seed of `slot_rng(params, prompt_len)` (spec.rs:185-187). */
uint64_t bfi_slot_rng_seed(uint64_t seed, uint64_t prompt_len);
/* `draft(ctx, k, ngram_max, ngram_min)` (spec.rs:46-68): writes up to k ids to out,
 * returns how many. */
size_t bfi_draft(const uint32_t *ctx_ids, size_t len, size_t k, size_t ngram_max,
                 size_t ngram_min, uint32_t *out);
/* `parse_id_union` (sample.rs:208-221) into a packed allow-mask of ceil(n_vocab/32) words.
 * Returns 1 when `grammar` is an id union (mask written; ids >= n_vocab ignored), 0 when
 * it is not (mask untouched). */
int bfi_parse_id_union(const char *grammar, int64_t n_vocab, uint32_t *mask_out);

/* Host half of take_token_spec after a GPU verify (spec.rs:140-179): replays the stop
 * rules of push_token (engine/mod.rs:451-462) over the kernel's verdicts for one sequence
 * and advances the slot RNG by two draws per judged row. Rules: an EOS draft is never
 * appended and ends the slot (Pushed::Eos); a draft with closes_tool[i] != 0 is appended,
 * counted and ends the slot (Pushed::Stopped, spec.rs:150-153) — the caller evaluates
 * should_stop_tool (engine/mod.rs:548) on the generated ids through drafted[i];
 * closes_tool may be NULL (no draft closes a tool call); the budget `max_tokens` counts
 * `generated` tokens so far. eos < 0 means no EOS id. Outputs: pushed ids, accepted count
 * (SpecStats::accepted), done flag, pending correction (-1 = none). */
int bfi_spec_replay(const uint32_t *drafted, const uint8_t *closes_tool, size_t n_drafted,
                    int32_t kernel_accepted, uint32_t kernel_next, int64_t eos, size_t generated,
                    size_t max_tokens, uint64_t *rng_state, uint32_t *pushed_out, size_t *n_pushed,
                    size_t *accepted, int *done, int64_t *pending);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* BFI_SAMPLER_H */
