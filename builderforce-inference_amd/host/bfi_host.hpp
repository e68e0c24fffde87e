// bfi_host.hpp — C++ host mirror of bfi-runtime's sampling interface over the C ABI.
//
// The reference exposes a free function `sample(logits, prev, &SampleParams) -> u32`
// (crates/bfi-runtime/src/sample.rs:304), the Engine's batched step (engine/mod.rs:297-337)
// and the spec-lookup step (engine/spec.rs:101-181). This header keeps those names and
// argument meanings; the numeric work runs on the GPU through include/bfi_sampler.h.
#pragma once

#include <cstdint>
#include <optional>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/bfi_sampler.h"

namespace bfi {

// sample.rs:9-50 (numeric fields + the id-union grammar; json/tool constraints arrive
// already resolved into `allow_mask`).
struct SampleParams {
    uint32_t max_tokens = 256;
    float temperature = 0.0f;
    int32_t top_k = 0;
    float top_p = 1.0f;
    float min_p = 0.0f;
    float repeat_penalty = 1.0f;
    float presence_penalty = 0.0f;
    float frequency_penalty = 0.0f;  // extension; 0 = reference behaviour
    uint64_t seed = 0;
    std::optional<std::string> grammar;

    bfi_smp_row_params row() const {
        bfi_smp_row_params p{};
        p.temperature = temperature;
        p.top_k = top_k;
        p.top_p = top_p;
        p.min_p = min_p;
        p.repeat_penalty = repeat_penalty;
        p.presence_penalty = presence_penalty;
        p.frequency_penalty = frequency_penalty;
        return p;
    }
};

// xorshift64 `Rng` (sample.rs:441-460).
struct Rng {
    uint64_t state;
    explicit Rng(uint64_t s) : state(s) {}
    uint64_t next_u64() { return bfi_rng_next_u64(&state); }
    float f32() { return bfi_rng_f32(&state); }
};

inline Rng slot_rng(const SampleParams& p, size_t prompt_len) {  // spec.rs:185-187
    return Rng(bfi_slot_rng_seed(p.seed, prompt_len));
}

// spec.rs:24-42
struct SpecStats {
    uint64_t verify_passes = 0, drafted = 0, accepted = 0;
    double acceptance() const { return drafted == 0 ? 0.0 : (double)accepted / (double)drafted; }
};

// spec.rs:10-22
struct SpecLookup {
    size_t draft_len = 4, ngram_max = 3, ngram_min = 2;
};

std::vector<uint32_t> draft(const std::vector<uint32_t>& ctx, size_t k, size_t ngram_max, size_t ngram_min);
// `parse_id_union` (sample.rs:208-221) as a packed allow-mask; nullopt when not an id union.
std::optional<std::vector<uint32_t>> id_union_mask(const std::string& grammar, int64_t n_vocab);

struct Error : std::runtime_error {
    int code;
    Error(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

// The host half of take_token_spec (spec.rs:137-179) after the GPU verify: applies the stop
// rules to the kernel's verdicts and advances the slot RNG by two draws per judged row.
struct SpecReplay {
    std::vector<uint32_t> pushed;  // tokens appended to all_ids (EOS never appended)
    size_t accepted = 0;           // counted into SpecStats::accepted
    bool done = false;             // EOS / tool stop / budget reached
    std::optional<uint32_t> pending;
    uint32_t kernel_next = 0;      // verify_step: the kernel's correction or bonus sample
};

// One sequence of a batched verify step (the GenSlot fields take_token_spec uses).
struct SpecSeq {
    std::vector<uint32_t> drafted;  // draft() after t0 (empty: nothing judged)
    std::vector<bool> closes_tool;  // per draft: appending it completes a tool call
    Rng rng{0};                     // slot_rng (spec.rs:185-187), advanced by the replay
    size_t generated = 0;           // tokens generated so far, t0 included
    size_t max_tokens = 0;
    float u_bonus = 0.0f;           // Rng(params.seed).f32(): the next pick's uniform
};
// kernel_accepted / kernel_next: bfi_smp_verify outputs of this sequence. `generated` is
// how many tokens the slot has generated so far (incl. t0), max_tokens its budget.
// closes_tool[i] (empty: none): appending drafted[i] completes a tool call, i.e. the
// caller's should_stop_tool (engine/mod.rs:548) holds for the generated ids through it.
SpecReplay replay_spec(const std::vector<uint32_t>& drafted, int32_t kernel_accepted, uint32_t kernel_next,
                       std::optional<uint32_t> eos, size_t generated, size_t max_tokens, Rng& slot_rng,
                       const std::vector<bool>& closes_tool = {});

// Owns a bfi_smp_ctx. Not for concurrent use (one per engine thread, like the reference's
// Mutex<Option<Loaded>>).
class Sampler {
  public:
    explicit Sampler(int device = 0);
    ~Sampler();
    Sampler(const Sampler&) = delete;
    Sampler& operator=(const Sampler&) = delete;

    // sample.rs:304: host row, uniform Rng(p.seed).f32(), id-union grammar honoured.
    uint32_t sample(const float* logits, size_t n_vocab, const uint32_t* prev, size_t n_prev,
                    const SampleParams& p);

    // generate_batch's per-step call (engine/mod.rs:316-322) over device rows.
    void sample_rows(const void* d_logits, int dtype, int64_t n_rows, int64_t n_vocab, int64_t row_stride,
                     const bfi_smp_row_params* d_params, const uint32_t* d_hist, const int64_t* d_hist_off,
                     const uint32_t* d_mask, int64_t mask_stride, const float* d_u, uint32_t* d_out,
                     void* stream);

    // spec-lookup verify over device rows (engine/spec.rs:137-162, one call for all
    // sequences; include/bfi_sampler.h bfi_smp_verify).
    void verify(const void* d_logits, int dtype, int64_t n_seq, int64_t rows_per_seq, int64_t n_vocab,
                int64_t row_stride, const bfi_smp_row_params* d_params, const uint32_t* d_hist,
                const int64_t* d_hist_off, const uint32_t* d_drafts, const int32_t* d_draft_len,
                const uint32_t* d_mask, int64_t mask_stride, const float* d_u_pairs, const float* d_u_bonus,
                int32_t* d_out_accepted, uint32_t* d_out_next, void* stream);

    // The verify half of take_token_spec for every live sequence at once: after the
    // caller's forward_each produced rows_per_seq rows per sequence (sequence s: rows
    // [s * rows_per_seq, s * rows_per_seq + drafted.size()], rows_per_seq > every draft's
    // length), judges all drafts in one verify call with uniforms from each slot RNG and
    // replays the stop rules per sequence (advancing the slot RNGs). d_hist / d_hist_off:
    // each sequence's all_ids before its drafts (t0 included). Synchronizes `stream`.
    std::vector<SpecReplay> verify_step(const void* d_logits, int dtype, int64_t rows_per_seq,
                                               int64_t n_vocab, int64_t row_stride,
                                               const bfi_smp_row_params* d_params, const uint32_t* d_hist,
                                               const int64_t* d_hist_off, const uint32_t* d_mask,
                                               int64_t mask_stride, std::vector<SpecSeq>& seqs,
                                               std::optional<uint32_t> eos, void* stream);

    bfi_smp_ctx* ctx() { return ctx_; }

  private:
    void check(int rc);
    void* staging(size_t bytes);  // device staging of verify_step's small arrays
    bfi_smp_ctx* ctx_ = nullptr;
    void* dbuf_ = nullptr;
    size_t dcap_ = 0;
};

// mix_decode (engine/mod.rs:560-580): every live sequence takes one step per round;
// returns the number of shared rounds.
template <typename T, typename Live, typename Step>
uint64_t mix_decode(std::vector<T>& seqs, Live live, Step step) {
    uint64_t steps = 0;
    for (;;) {
        bool any = false;
        for (auto& s : seqs) any = any || live(s);
        if (!any) return steps;
        steps++;
        for (auto& s : seqs)
            if (live(s)) step(s);
        if (steps >= 1000000) return steps;
    }
}

}  // namespace bfi
