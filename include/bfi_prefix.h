/* bfi_prefix.h — C ABI of the prefix cache: longest-prefix reuse of a sequence's model state
 * across generate calls, with the cached state held in device memory (HBM).
 *
 * Replaces `PrefixCache` (crates/bfi-runtime/src/engine/prefix.rs:114-347): a cache bounded by
 * BYTES, not entries; each entry is a token sequence plus the model state after it (the used
 * rows of every K/V tensor, the recurrent tensors, the logits at its end). The engine looks
 * the prompt up before prefill (engine/mod.rs:359-381), inserts the prompt state after it
 * (mod.rs:386-388, `insert_copy`) and the finished sequence in `finish` (mod.rs:466-475,
 * `insert_owned`). The entry points keep the reference's names, results and error cases:
 *
 *   lookup   prefix.rs:168-214  the best resume point (deepest hash-marked match confirmed
 *                               token by token; a rewindable entry serves any prefix of itself;
 *                               a share under one BLOCK found by comparing entries directly)
 *   restore  prefix.rs:217-230  the entry's state into the caller's full-capacity tensors (used
 *                               rows copied, the rest zero) and its logits when the hit resumes at
 *                               the entry's end; marks the entry used (LRU)
 *   insert   prefix.rs:233-246, 248-260, 262-307  caches a state: drops entries it supersedes,
 *                               evicts least recently used entries to fit, skips a state larger
 *                               than the whole budget
 *
 * `insert` always copies the used rows (device to device, on `stream`); the reference's
 * `insert_owned` moves its host buffers instead, which leaves the cache in the same state.
 *
 * Memory: device >= 0 keeps entries in that device's memory (hipMalloc per entry; copies and
 * zero fills are queued on `stream`, a hipStream_t, NULL = the null stream); device == -1 keeps
 * them in host memory (memcpy), which the CPU tests use. Not thread-safe: one cache per engine,
 * like the reference's field of `Engine`. Status codes as in bfi_sampler.h (BFI_SMP_OK,
 * BFI_SMP_EINVAL, BFI_SMP_EHIP, BFI_SMP_ENOMEM); error text per cache (bfi_pc_last_error).
 */
#ifndef BFI_PREFIX_H
#define BFI_PREFIX_H

#include <stddef.h>
#include <stdint.h>

#include "bfi_sampler.h"

#ifdef __cplusplus
extern "C" {
#endif

/* prefix.rs:29 `BLOCK`: the hash-probe granularity of rewindable entries. */
#define BFI_PC_BLOCK 64

typedef struct bfi_pc bfi_pc;

/* One tensor of a state (`SeqState::k[i]`, `v[i]`, `recurrent[i]`, prefix.rs:42-92).
 * row_bytes > 0: `rows` rows of row_bytes bytes each (a K/V layer: one row per position);
 * the cache keeps the first `n` rows (the state's used rows, `Kept::Rows`).
 * row_bytes == 0: a whole tensor of `rows` bytes, kept whole (`Kept::Whole`).
 * A recurrent slot with data == NULL is a layer without recurrent state (`None`). */
typedef struct {
    void* data;
    uint64_t row_bytes;
    uint64_t rows;
} bfi_pc_tensor;

/* A sequence state (`bfi_models::SeqState` + `Logits`): n used positions, the K/V tensors (any
 * fixed order the caller keeps, e.g. K layers then V layers), the recurrent slots and the
 * logits after the last position. */
typedef struct {
    uint64_t n;
    const bfi_pc_tensor* kv;
    uint64_t n_kv;
    const bfi_pc_tensor* rec;
    uint64_t n_rec;
    float* logits;
    uint64_t n_logits;
} bfi_pc_state;

/* prefix.rs:31-40 `Hit`. */
typedef struct {
    uint64_t id;
    uint64_t matched; /* prompt tokens the entry agrees with */
    uint64_t restore; /* tokens to restore (matched, or one less to leave a token to forward) */
} bfi_pc_hit;

/* prefix.rs:132-142 `PrefixCache::new(budget_bytes)` (the engine's default budget is 1 GiB,
 * options.rs:4). */
int bfi_pc_create(int device, uint64_t budget_bytes, bfi_pc** out);
void bfi_pc_destroy(bfi_pc* pc);
const char* bfi_pc_last_error(const bfi_pc* pc);

/* prefix.rs:168-214 `lookup`: *found = 1 and *hit filled, or *found = 0 (`None`). */
int bfi_pc_lookup(const bfi_pc* pc, const uint32_t* ids, uint64_t n_ids, bfi_pc_hit* hit, int* found);

/* prefix.rs:217-230 `restore`: copies the entry of `hit` into dst (whose layout must match the
 * inserted state's: the same tensor counts and row sizes, capacities at least the kept rows)
 * and sets *n = hit->restore; the logits are copied, and *logits_restored = 1, only when the
 * hit resumes at the entry's end. *found = 0 when the entry is gone (`None`). */
int bfi_pc_restore(bfi_pc* pc, const bfi_pc_hit* hit, const bfi_pc_state* dst, uint64_t* n, int* logits_restored,
                   int* found, void* stream);

/* prefix.rs:233-246 `insert_copy` (and `insert_owned`, 248-260): caches tokens[0, n_tokens)
 * with the state st (st->n must equal n_tokens, else nothing is cached, as in the reference). */
int bfi_pc_insert(bfi_pc* pc, const uint32_t* tokens, uint64_t n_tokens, const bfi_pc_state* st, void* stream);

/* prefix.rs:144-164: bytes held, entries, forwarded-token counter, clear. */
uint64_t bfi_pc_used_bytes(const bfi_pc* pc);
uint64_t bfi_pc_len(const bfi_pc* pc);
void bfi_pc_note_forward(bfi_pc* pc, uint64_t n);
uint64_t bfi_pc_forwarded(const bfi_pc* pc);
void bfi_pc_clear(bfi_pc* pc);

#ifdef __cplusplus
}
#endif

#endif /* BFI_PREFIX_H */
