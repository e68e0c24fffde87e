// bfi_host.cpp — host-side helpers of the C ABI and the C++ mirror (bfi_host.hpp): Rng,
// slot_rng, draft, the id-union grammar and the spec replay. No GPU calls (bfi_sampler.cpp
// holds the Sampler class).
#include "bfi_host.hpp"

#include "bfi_grammar.hpp"

#include <cstring>

extern "C" {

uint64_t bfi_rng_next_u64(uint64_t* state) {  // sample.rs:445-455
    uint64_t x = *state;
    if (x == 0) x = 0x9E3779B97F4A7C15ull;
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    *state = x;
    return x;
}

float bfi_rng_f32(uint64_t* state) {  // sample.rs:457-459
    return (float)(bfi_rng_next_u64(state) >> 40) / (float)(1u << 24);
}

uint64_t bfi_slot_rng_seed(uint64_t seed, uint64_t prompt_len) {  // spec.rs:185-187
    return seed ^ 0xa0761d6478bd642full ^ (prompt_len * 0x9e3779b97f4a7c15ull);
}

size_t bfi_draft(const uint32_t* ctx, size_t len, size_t k, size_t ngram_max, size_t ngram_min, uint32_t* out) {
    // spec.rs:46-68: most recent earlier occurrence of the last n-gram, n = max..min
    if (k == 0 || (len && !ctx) || !out) return 0;
    const size_t lo = ngram_min > 1 ? ngram_min : 1;
    for (size_t n = ngram_max; n >= lo && n > 0; n--) {
        if (len < n + 1) continue;
        const uint32_t* tail = ctx + (len - n);
        for (size_t start = len - n; start-- > 0;) {
            if (std::memcmp(ctx + start, tail, n * sizeof(uint32_t)) == 0) {
                const size_t from = start + n;
                const size_t to = from + k < len ? from + k : len;
                if (from < to) {
                    std::memcpy(out, ctx + from, (to - from) * sizeof(uint32_t));
                    return to - from;
                }
            }
        }
    }
    return 0;
}

}  // extern "C"

extern "C" int bfi_parse_id_union(const char* grammar, int64_t n_vocab, uint32_t* mask_out) {
    // sample.rs:207-221 parse_id_union, 231-235 strip_root (Unicode str::trim)
    if (!grammar || n_vocab < 0 || (n_vocab > 0 && !mask_out)) return 0;
    std::vector<uint32_t> ids;
    if (!bfig::parse_id_union(grammar, &ids)) return 0;
    const size_t words = (size_t)((n_vocab + 31) / 32);
    std::memset(mask_out, 0, words * sizeof(uint32_t));
    for (uint32_t id : ids)
        if ((int64_t)id < n_vocab) mask_out[id >> 5] |= 1u << (id & 31);
    return 1;
}

namespace bfi {

std::vector<uint32_t> draft(const std::vector<uint32_t>& ctx, size_t k, size_t ngram_max, size_t ngram_min) {
    std::vector<uint32_t> out(k);
    out.resize(bfi_draft(ctx.data(), ctx.size(), k, ngram_max, ngram_min, out.data()));
    return out;
}

std::optional<std::vector<uint32_t>> id_union_mask(const std::string& grammar, int64_t n_vocab) {
    std::vector<uint32_t> m((size_t)((n_vocab + 31) / 32));
    if (!bfi_parse_id_union(grammar.c_str(), n_vocab, m.data())) return std::nullopt;
    return m;
}

SpecReplay replay_spec(const std::vector<uint32_t>& drafted, int32_t kernel_accepted, uint32_t kernel_next,
                       std::optional<uint32_t> eos, size_t generated, size_t max_tokens, Rng& rng,
                       const std::vector<bool>& closes_tool) {
    // spec.rs:140-162 with the verdicts already computed on the GPU
    SpecReplay r;
    std::optional<uint32_t> correction;
    for (size_t i = 0; i < drafted.size(); i++) {
        (void)rng.f32();  // u  (spec.rs:142)
        (void)rng.f32();  // u2
        if ((int32_t)i >= kernel_accepted) {  // Verdict::Reject(t)
            correction = kernel_next;
            break;
        }
        const uint32_t d = drafted[i];
        if (eos && d == *eos) {  // Pushed::Eos: not appended, not counted
            r.done = true;
            break;
        }
        r.pushed.push_back(d);
        r.accepted++;
        if (i < closes_tool.size() && closes_tool[i]) {  // Pushed::Stopped (spec.rs:150-153)
            r.done = true;
            break;
        }
        if (generated + r.pushed.size() >= max_tokens) {  // budget_spent
            r.done = true;
            break;
        }
    }
    if (!r.done) r.pending = correction;  // spec.rs:177-179
    return r;
}

}  // namespace bfi

// C entry point of replay_spec for callers without C++ (and the CPU tests).
extern "C" int bfi_spec_replay(const uint32_t* drafted, const uint8_t* closes_tool, size_t n_drafted,
                               int32_t kernel_accepted, uint32_t kernel_next, int64_t eos, size_t generated,
                               size_t max_tokens, uint64_t* rng_state, uint32_t* pushed_out, size_t* n_pushed,
                               size_t* accepted, int* done, int64_t* pending) {
    if ((n_drafted && !drafted) || !rng_state || !pushed_out || !n_pushed || !accepted || !done || !pending)
        return BFI_SMP_EINVAL;
    std::vector<uint32_t> d(drafted, drafted + n_drafted);
    std::vector<bool> stops;
    if (closes_tool) stops.assign(closes_tool, closes_tool + n_drafted);
    bfi::Rng rng(*rng_state);
    std::optional<uint32_t> e;
    if (eos >= 0) e = (uint32_t)eos;
    bfi::SpecReplay r = bfi::replay_spec(d, kernel_accepted, kernel_next, e, generated, max_tokens, rng, stops);
    *rng_state = rng.state;
    if (!r.pushed.empty()) std::memcpy(pushed_out, r.pushed.data(), r.pushed.size() * sizeof(uint32_t));
    *n_pushed = r.pushed.size();
    *accepted = r.accepted;
    *done = r.done ? 1 : 0;
    *pending = r.pending ? (int64_t)*r.pending : -1;
    return BFI_SMP_OK;
}
