// bfi_sampler.cpp — the Sampler class of the C++ mirror (bfi_host.hpp) over the GPU entry
// points of include/bfi_sampler.h, and the batched speculative verify step.
#include <hip/hip_runtime.h>

#include <cstring>

#include "bfi_host.hpp"

namespace bfi {

Sampler::Sampler(int device) { check(bfi_smp_create(device, &ctx_)); }

Sampler::~Sampler() {
    if (dbuf_) (void)hipFree(dbuf_);
    bfi_smp_destroy(ctx_);
}

void Sampler::check(int rc) {
    if (rc != BFI_SMP_OK) throw Error(rc, bfi_smp_last_error(ctx_));
}

uint32_t Sampler::sample(const float* logits, size_t n_vocab, const uint32_t* prev, size_t n_prev,
                         const SampleParams& p) {
    std::optional<std::vector<uint32_t>> mask;
    if (p.grammar) mask = id_union_mask(*p.grammar, (int64_t)n_vocab);
    const bfi_smp_row_params row = p.row();
    const float u = Rng(p.seed).f32();  // sample.rs:307 re-seeds every call
    uint32_t tok = 0;
    check(bfi_smp_sample_host(ctx_, logits, (int64_t)n_vocab, prev, (int64_t)n_prev, &row,
                              mask ? mask->data() : nullptr, u, &tok));
    return tok;
}

void Sampler::sample_rows(const void* d_logits, int dtype, int64_t n_rows, int64_t n_vocab, int64_t row_stride,
                          const bfi_smp_row_params* d_params, const uint32_t* d_hist, const int64_t* d_hist_off,
                          const uint32_t* d_mask, int64_t mask_stride, const float* d_u, uint32_t* d_out,
                          void* stream) {
    check(bfi_smp_sample_rows(ctx_, d_logits, dtype, n_rows, n_vocab, row_stride, d_params, d_hist, d_hist_off,
                              d_mask, mask_stride, d_u, d_out, stream));
}

void Sampler::verify(const void* d_logits, int dtype, int64_t n_seq, int64_t rows_per_seq, int64_t n_vocab,
                     int64_t row_stride, const bfi_smp_row_params* d_params, const uint32_t* d_hist,
                     const int64_t* d_hist_off, const uint32_t* d_drafts, const int32_t* d_draft_len,
                     const uint32_t* d_mask, int64_t mask_stride, const float* d_u_pairs, const float* d_u_bonus,
                     int32_t* d_out_accepted, uint32_t* d_out_next, void* stream) {
    check(bfi_smp_verify(ctx_, d_logits, dtype, n_seq, rows_per_seq, n_vocab, row_stride, d_params, d_hist,
                         d_hist_off, d_drafts, d_draft_len, d_mask, mask_stride, d_u_pairs, d_u_bonus,
                         d_out_accepted, d_out_next, stream));
}

void* Sampler::staging(size_t bytes) {
    if (bytes > dcap_) {
        if (dbuf_) (void)hipFree(dbuf_);
        dbuf_ = nullptr;
        dcap_ = 0;
        if (hipMalloc(&dbuf_, bytes) != hipSuccess) throw Error(BFI_SMP_EHIP, "hipMalloc of the verify staging");
        dcap_ = bytes;
    }
    return dbuf_;
}

std::vector<SpecReplay> Sampler::verify_step(const void* d_logits, int dtype, int64_t rows_per_seq, int64_t n_vocab,
                                             int64_t row_stride, const bfi_smp_row_params* d_params,
                                             const uint32_t* d_hist, const int64_t* d_hist_off,
                                             const uint32_t* d_mask, int64_t mask_stride, std::vector<SpecSeq>& seqs,
                                             std::optional<uint32_t> eos, void* stream) {
    const int64_t n_seq = (int64_t)seqs.size();
    if (rows_per_seq < 1) throw Error(BFI_SMP_EINVAL, "rows_per_seq < 1");
    const size_t K = (size_t)rows_per_seq - 1;
    // the kernel's inputs: drafts, their counts, and the uniforms of each judged row from a
    // copy of the slot RNG (two draws per draft, spec.rs:142); the replay below advances the
    // RNG itself by the draws the reference makes
    std::vector<uint32_t> drafts((size_t)n_seq * (K ? K : 1), 0u);
    std::vector<int32_t> dlen((size_t)n_seq);
    std::vector<float> upairs((size_t)n_seq * (K ? K : 1) * 2, 0.0f), ubonus((size_t)n_seq);
    for (int64_t s = 0; s < n_seq; s++) {
        const SpecSeq& q = seqs[(size_t)s];
        if (q.drafted.size() > K) throw Error(BFI_SMP_EINVAL, "a draft longer than rows_per_seq - 1");
        dlen[(size_t)s] = (int32_t)q.drafted.size();
        Rng r = q.rng;
        for (size_t i = 0; i < q.drafted.size(); i++) {
            drafts[(size_t)s * K + i] = q.drafted[i];
            upairs[((size_t)s * K + i) * 2] = r.f32();
            upairs[((size_t)s * K + i) * 2 + 1] = r.f32();
        }
        ubonus[(size_t)s] = q.u_bonus;
    }
    auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
    const size_t o_dr = 0, o_dl = al(drafts.size() * 4), o_up = o_dl + al(dlen.size() * 4),
                 o_ub = o_up + al(upairs.size() * 4), o_acc = o_ub + al(ubonus.size() * 4),
                 o_nx = o_acc + al((size_t)n_seq * 4), total = o_nx + al((size_t)n_seq * 4);
    char* d = (char*)staging(total);
    hipStream_t st = (hipStream_t)stream;
    auto up = [&](size_t off, const void* src, size_t n) {
        if (n && hipMemcpyAsync(d + off, src, n, hipMemcpyHostToDevice, st) != hipSuccess)
            throw Error(BFI_SMP_EHIP, "hipMemcpyAsync to the verify staging");
    };
    up(o_dr, drafts.data(), drafts.size() * 4);
    up(o_dl, dlen.data(), dlen.size() * 4);
    up(o_up, upairs.data(), upairs.size() * 4);
    up(o_ub, ubonus.data(), ubonus.size() * 4);
    verify(d_logits, dtype, n_seq, rows_per_seq, n_vocab, row_stride, d_params, d_hist, d_hist_off,
           (const uint32_t*)(d + o_dr), (const int32_t*)(d + o_dl), d_mask, mask_stride, (const float*)(d + o_up),
           (const float*)(d + o_ub), (int32_t*)(d + o_acc), (uint32_t*)(d + o_nx), stream);
    std::vector<int32_t> acc((size_t)n_seq);
    std::vector<uint32_t> nxt((size_t)n_seq);
    if (hipMemcpyAsync(acc.data(), d + o_acc, acc.size() * 4, hipMemcpyDeviceToHost, st) != hipSuccess ||
        hipMemcpyAsync(nxt.data(), d + o_nx, nxt.size() * 4, hipMemcpyDeviceToHost, st) != hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess)
        throw Error(BFI_SMP_EHIP, "reading the verdicts back");
    std::vector<SpecReplay> out;
    out.reserve(seqs.size());
    for (int64_t s = 0; s < n_seq; s++) {
        SpecSeq& q = seqs[(size_t)s];
        out.push_back(replay_spec(q.drafted, acc[(size_t)s], nxt[(size_t)s], eos, q.generated, q.max_tokens, q.rng,
                                  q.closes_tool));
        out.back().kernel_next = nxt[(size_t)s];
    }
    return out;
}

}  // namespace bfi
