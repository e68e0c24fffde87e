// smp_stream.hip — the streaming pass of the gfx950 token sampler.
//
// One launch covers every row of a batch (generate_batch's per-step call, engine/mod.rs:
// 316-322) or every draft row of a spec-verify step (engine/spec.rs:137-162). Workgroup
// (row, chunk) reads `chunk` logits of one row once from HBM with 16-byte loads, keeps them
// in VGPRs, applies the allow-mask and the temperature division (sample.rs:331-337,
// 373-375), and writes per chunk: the max, the f64 sum of exp(s - max), and the elements
// that can still be kept under the row's top-k or min-p bound. Penalties are left to the
// select kernel, which corrects the few history ids.
#include <hip/hip_ext.h>

#include "smp_common.h"

namespace bfi {

// The stream kernel needs only reduction scratch (no history: penalties are applied as
// sparse corrections by the select kernel).
struct __align__(16) StreamSmem {
    float rf[NWAVE];
    uint32_t ru[NWAVE];
    double rd[NWAVE];
    uint32_t misc[8];
};

// ---- the kernel --------------------------------------------------------------------------

template <bool BF16, int VEC>
__global__ __launch_bounds__(BLOCK, 5) void k_stream(KArgs a) {
    constexpr int EPV = Elem<BF16>::EPV;
    __shared__ StreamSmem sm;
    const int tid = threadIdx.x;

    // workgroups are dispatched round-robin over the 8 XCDs: give each XCD a contiguous
    // range of (row, chunk) so a row's chunks share one L2
    const uint32_t G = gridDim.x, bid = blockIdx.x;
    const uint32_t q8 = G / 8, r8 = G % 8, xcd = bid % 8, slot = bid / 8;
    const uint32_t logical = xcd < r8 ? xcd * (q8 + 1) + slot : r8 * (q8 + 1) + (xcd - r8) * q8 + slot;
    const int row = (int)(logical / (uint32_t)a.n_chunks);
    const int chunk = (int)(logical % (uint32_t)a.n_chunks);
    const int64_t tb = (int64_t)logical * 8;
    BFI_TRACE(a, tb, 0);
    if (row >= a.n_rows) return;
    const RowCtx C = make_ctx(a, row);
    if (!C.active) return;

    const uint32_t V = (uint32_t)a.V;
    const uint32_t c0 = (uint32_t)chunk * (uint32_t)a.chunk;
    const uint32_t c1 = min(c0 + (uint32_t)a.chunk, V);
    const uint32_t em = (1u << EPV) - 1u;

    float x[VEC][EPV];
    load_tile<BF16, VEC>(a, row, c0, c1, x);
    BFI_TRACE(a, tb, 1);

    ChunkPart part;
    part.pad = 0;
    part.pad2 = 0;
    part.raw_m = -__builtin_inff();
    part.raw_arg = 0xFFFFFFFFu;
    part.arg = 0;
    // pass 1, vector by vector as the loads land: the mask (sample.rs:331-337) in place and
    // the running max of the masked logits (with its first index for greedy rows and the
    // min-p fallback, sample.rs:415-422). max(x / T) = max(x) / T for T > 0, so the chunk's
    // exact maximum takes one division.
    const bool track_arg = C.greedy || (C.min_p > 1.0f);
    ArgMax best{-__builtin_inff(), 0xFFFFFFFFu};
    float lm = -__builtin_inff();
#pragma unroll
    for (int q = 0; q < VEC; q++) {
        const uint32_t id0 = c0 + (uint32_t)(q * BLOCK + tid) * EPV;
        if (C.mrow) {
            const uint32_t mb = id0 < c1 ? (C.mrow[id0 >> 5] >> (id0 & 31)) & em : 0u;
#pragma unroll
            for (int e = 0; e < EPV; e++) x[q][e] = ((mb >> e) & 1u) ? x[q][e] : -__builtin_inff();
        }
        if (track_arg) {
#pragma unroll
            for (int e = 0; e < EPV; e++) best = argmax_merge(best, ArgMax{x[q][e], id0 + e});
        } else {
#pragma unroll
            for (int e = 0; e < EPV; e++) lm = fmaxf(lm, x[q][e]);
        }
    }
    BFI_TRACE(a, tb, 2);
    if (track_arg) {
        best = block_argmax(best, sm.rf, sm.ru);
        lm = best.v;
        part.raw_arg = best.i;
    } else {
        lm = block_max(lm, sm.rf);
    }
    part.raw_m = lm;  // the chunk's largest masked logit
    if (C.greedy) {
        part.m = best.v;
        part.arg = best.i;
        part.sum = 0.0;
        part.ncand = 0;
        part.theta = -__builtin_inff();
    } else {
        const float mc = div_T(lm, C);  // exact (sample.rs:373-375)
        BFI_TRACE(a, tb, 3);
        part.m = mc;
        const bool kb = C.kmode && C.k <= CAND_CAP;
        const float margin = 1e-4f + 1e-5f * fabsf(mc);
        // min-p bound of this chunk: p >= min_p * max p needs s >= max_s + ln(min_p)
        float th = __builtin_inff();
        if (C.mmode && mc > -__builtin_inff()) {
            const float lmp = logf(C.min_p);
            th = mc + lmp - (margin + 1e-5f * fabsf(lmp));
        }
        // pass 2: the f64 sum of the terms stream_term (each vector's EPV terms added in
        // f32 first) and the count of masked logits at or above the bound th
        double ls = 0.0;
        uint32_t lc = 0;
        const float xth = x_bound(C, th);
        if (lm > -__builtin_inff()) {
#pragma unroll
            for (int q = 0; q < VEC; q++) {
                float g = 0.0f;
#pragma unroll
                for (int e = 0; e < EPV; e++) {
                    g += stream_term(C, x[q][e], lm);
                    lc += (x[q][e] >= xth) ? 1u : 0u;
                }
                ls += (double)g;
            }
        }
        uint32_t cnt;
        part.sum = block_sum_du(ls, lc, cnt, sm.rd, sm.ru);
        BFI_TRACE(a, tb, 4);
        if (!(mc > -__builtin_inff())) {
            part.ncand = 0;
            part.theta = -__builtin_inff();
        } else if (!(C.mmode || kb)) {
            part.ncand = NCAND_UNBOUNDED;
            part.theta = __builtin_inff();
        } else {
            uint32_t my = lc;  // this thread's candidates at th
            if (kb && (!C.mmode || cnt > (uint32_t)CAND_CAP)) {
                // top-k bound: the smallest power-of-two distance below the chunk max
                // holding k elements, then bisection toward a tight count
                float d = 0.25f, lo = 0.0f;
                uint32_t c = 0;
                int it = 0;
                for (; it < 18; it++) {
                    c = block_sum_u(tile_count_ge<BF16, VEC>(x, x_bound(C, mc - d)), sm.ru);
                    if (c >= (uint32_t)C.k) break;
                    lo = d;
                    d *= 2.0f;
                }
                float tk;
                if (c < (uint32_t)C.k) {
                    tk = -__builtin_inff();
                } else {
                    float hi = d;
                    const uint32_t want = max(2u * (uint32_t)C.k, 64u);
                    for (int j = 0; j < 12 && c > want; j++) {
                        const float mid = 0.5f * (lo + hi);
                        const uint32_t cm = block_sum_u(tile_count_ge<BF16, VEC>(x, x_bound(C, mc - mid)), sm.ru);
                        if (cm >= (uint32_t)C.k) {
                            hi = mid;
                            c = cm;
                        } else {
                            lo = mid;
                        }
                    }
                    tk = mc - hi - margin;
                }
                th = C.mmode ? fmaxf(th, tk) : tk;
                my = tile_count_ge<BF16, VEC>(x, x_bound(C, th));
                cnt = block_sum_u(my, sm.ru);
            }
            part.theta = th;
            if (cnt > (uint32_t)CAND_CAP) {
                part.ncand = NCAND_OVERFLOW;
            } else {
                // every element whose exact value is >= th (a few just below may come along)
                part.ncand = cnt;
                const float xw = x_bound(C, th);
                uint32_t tot;
                uint32_t o = block_excl_scan<uint32_t>(my, sm.ru, tot);
                if (my) {
                    Cand* dst = a.cands + ((int64_t)row * a.n_chunks + chunk) * CAND_CAP;
#pragma unroll
                    for (int q = 0; q < VEC; q++)
#pragma unroll
                        for (int e = 0; e < EPV; e++) {
                            if (x[q][e] >= xw && x[q][e] > -__builtin_inff()) {
                                dst[o].idx = c0 + (uint32_t)(q * BLOCK + tid) * EPV + e;
                                dst[o].x = x[q][e];
                                o++;
                            }
                        }
                }
            }
        }
    }
    if (tid == 0) a.parts[(int64_t)row * a.n_chunks + chunk] = part;
    BFI_TRACE(a, tb, 5);
}

// ---- launch ----------------------------------------------------------------------------

// `start` / `stop` (optional) time the kernel itself (hipExtLaunchKernelGGL records them in
// the dispatch).
hipError_t launch_stream(const KArgs& a, int bf16, int vec, hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
    const dim3 grid((unsigned)((int64_t)a.n_rows * a.n_chunks)), block(BLOCK);
#define BFI_LAUNCH(B, VV) hipExtLaunchKernelGGL((k_stream<B, VV>), grid, block, 0, stream, start, stop, 0, a)
    if (!bf16) {
        if (vec == 8) BFI_LAUNCH(false, 8);
        else if (vec == 4) BFI_LAUNCH(false, 4);
        else BFI_LAUNCH(false, 2);
    } else {
        if (vec == 4) BFI_LAUNCH(true, 4);
        else if (vec == 2) BFI_LAUNCH(true, 2);
        else BFI_LAUNCH(true, 1);
    }
#undef BFI_LAUNCH
    return hipGetLastError();
}

}  // namespace bfi
