/* bfi_mask.h — C ABI of the MI355X allow-mask producer for constrained decode.
 *
 * Replaces the per-step, per-vocabulary-id scan of the reference's decode-based constraint:
 * `apply_constraint` (crates/bfi-runtime/src/sample.rs:63-90) with `token_allowed`
 * (sample.rs:92-107), `tool_call_prefix_ok` (sample.rs:110-136), `json_name_so_far`
 * (sample.rs:144-206), `parse_id_union` / `parse_literal_root` (sample.rs:208-234) and
 * `json_object_prefix_ok` (sample.rs:236-286). The reference masks logits to -inf in place;
 * this library writes the equivalent packed allow-mask (bit id&31 of word id>>5, 1 = allowed)
 * that `bfi_smp_sample_rows` / `bfi_smp_target_rows` take as `d_mask` (include/bfi_sampler.h).
 *
 * The vocabulary's decoded pieces (`decode(id)` of the reference, as UTF-8 bytes) are
 * uploaded once per context. Per step, the host scans the generated text once (the pieces of
 * the generated ids, concatenated, as the reference's `so_far`) into an automaton state; one
 * GPU thread per vocabulary id continues that state over its piece.
 *
 * Conventions as in bfi_sampler.h: `int` status (BFI_SMP_OK = 0, BFI_SMP_EINVAL,
 * BFI_SMP_EHIP, BFI_SMP_ENOMEM), per-context error text, `stream` a hipStream_t.
 */
#ifndef BFI_MASK_H
#define BFI_MASK_H

#include <stddef.h>
#include <stdint.h>

#include "bfi_sampler.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ToolChoice (crates/bfi-runtime/src/tools.rs:21-31); REQUIRED and NAMED constrain. */
#define BFI_TOOL_NONE 0
#define BFI_TOOL_AUTO 1
#define BFI_TOOL_REQUIRED 2
#define BFI_TOOL_NAMED 3

/* Limits of one call (the per-call tables travel in the kernel's arguments). */
#define BFI_MASK_MAX_TOOL_NAMES 64
#define BFI_MASK_MAX_TABLE_BYTES 3072 /* tool names + the named tool + the literal tail */

/* The constraint fields of SampleParams (sample.rs:14-31): json_object, tool_choice,
 * tool_names, grammar. Strings are UTF-8 bytes with explicit lengths. */
typedef struct bfi_constraint {
    int32_t json_object;              /* SampleParams::json_object (0/1) */
    int32_t tool_choice;              /* BFI_TOOL_* */
    const uint8_t *tool_name;         /* ToolChoice::Named(..) value */
    int64_t tool_name_len;
    const uint8_t *const *tool_names; /* SampleParams::tool_names */
    const int64_t *tool_name_lens;
    int32_t n_tool_names;
    const uint8_t *grammar;           /* SampleParams::grammar, or NULL for None */
    int64_t grammar_len;
} bfi_constraint;

typedef struct bfi_mask_ctx bfi_mask_ctx;

/* A context on `device`. No reference counterpart (the reference holds the tokenizer in the
 * Engine, engine/mod.rs). */
int bfi_mask_create(int device, bfi_mask_ctx **out);
void bfi_mask_destroy(bfi_mask_ctx *ctx);
const char *bfi_mask_error(const bfi_mask_ctx *ctx);

/* The vocabulary: piece i = bytes[offsets[i] .. offsets[i+1]) (host memory, offsets
 * non-decreasing, offsets[0] = 0), the reference's `decode(i)`. Copied to the device;
 * replaces any earlier vocabulary of the context. */
int bfi_mask_set_vocab(bfi_mask_ctx *ctx, const uint8_t *bytes, const int64_t *offsets, int64_t n_vocab);

/* `apply_constraint(logits, generated, p, decode)` (sample.rs:63-90) as an allow-mask over
 * the context's vocabulary: d_mask (device, ceil(n_vocab/32) words) gets bit i set when the
 * reference leaves logit i finite. `so_far` (host) is the concatenated pieces of the
 * generated ids (sample.rs:82). *constrained receives 0 when the constraint does not
 * restrict anything (sample.rs:69-71; the mask is all ones then), else 1. */
int bfi_mask_build(bfi_mask_ctx *ctx, const uint8_t *so_far, int64_t so_far_len, const bfi_constraint *c,
                   uint32_t *d_mask, int32_t *constrained, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* BFI_MASK_H */
