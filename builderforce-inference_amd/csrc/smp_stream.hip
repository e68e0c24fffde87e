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
// sparse corrections by the select kernel). Each exchange has slots of its own, so one
// barrier per exchange suffices.
constexpr int SEG = 512;  // candidates one wave stages in LDS
struct __align__(16) StreamSmem {
    double ws[NWAVE];   // per-wave sums (relative to the wave max)
    float wm[NWAVE];    // per-wave maxima of the masked logits
    float wbv[NWAVE];   // per-wave argmax value (greedy rows: penalized; min_p > 1: raw)
    uint32_t wa[NWAVE]; // per-wave first index of that value
    uint32_t wc[NWAVE]; // per-wave candidate counts
    uint32_t wc2[NWAVE];
    float rf[NWAVE];
    uint32_t ru[NWAVE];
    double rd[NWAVE];
    union {
        uint32_t hc[CHUNK_MAX / 2];  // history counts of the chunk's ids, two 16-bit halves a word
        Cand stage[NWAVE][SEG];      // each wave's candidates before the coalesced copy out
    } u;
};
static_assert(NWAVE * SEG * sizeof(Cand) == CHUNK_MAX * 2, "the count array and the stage share LDS");

// Stages this wave's elements at or above xw in LDS (the first SEG of them), in element
// slot order then lane order; returns how many there are (wave-uniform).
template <bool BF16, int VEC>
__device__ __forceinline__ uint32_t stage_cands(const float (&x)[VEC][Elem<BF16>::EPV], float xw, Cand* seg,
                                                uint32_t c0) {
    constexpr int EPV = Elem<BF16>::EPV;
    uint32_t n = 0;
#pragma unroll
    for (int q = 0; q < VEC; q++)
#pragma unroll
        for (int e = 0; e < EPV; e++) {
            const bool take = x[q][e] >= xw;
            const uint64_t bal = __ballot(take);
            if (bal) {
                const uint32_t pos =
                    n + __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
                if (take && pos < (uint32_t)SEG) {
                    seg[pos].idx = c0 + (uint32_t)(q * BLOCK + threadIdx.x) * EPV + e;
                    seg[pos].x = x[q][e];
                }
                n += (uint32_t)__popcll(bal);
            }
        }
    return n;
}

// The same elements straight to global memory from offset o (a wave with more than SEG).
template <bool BF16, int VEC>
__device__ __forceinline__ void emit_cands(const float (&x)[VEC][Elem<BF16>::EPV], float xw, Cand* dst, uint32_t o,
                                           uint32_t c0) {
    constexpr int EPV = Elem<BF16>::EPV;
#pragma unroll
    for (int q = 0; q < VEC; q++)
#pragma unroll
        for (int e = 0; e < EPV; e++) {
            const bool take = x[q][e] >= xw;
            const uint64_t bal = __ballot(take);
            if (bal) {
                if (take) {
                    const uint32_t r =
                        __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
                    dst[o + r].idx = c0 + (uint32_t)(q * BLOCK + threadIdx.x) * EPV + e;
                    dst[o + r].x = x[q][e];
                }
                o += (uint32_t)__popcll(bal);
            }
        }
}

// ---- the kernel --------------------------------------------------------------------------

template <bool BF16, int VEC, bool FULL>
__device__ __forceinline__ void stream_chunk(const KArgs& a, StreamSmem& sm, int row, int chunk, uint32_t c0,
                                             uint32_t c1, uint32_t logical, bool tron, uint64_t t0);

template <bool BF16, int VEC>
__global__ __launch_bounds__(BLOCK, 5) void k_stream(KArgs a) {
    __shared__ StreamSmem sm;

    // workgroups are dispatched round-robin over the 8 XCDs: give each XCD a contiguous
    // range of (row, chunk) so a row's chunks share one L2
    const uint32_t G = gridDim.x, bid = blockIdx.x;
    const uint32_t q8 = G / 8, r8 = G % 8, xcd = bid % 8, slot = bid / 8;
    const uint32_t logical = xcd < r8 ? xcd * (q8 + 1) + slot : r8 * (q8 + 1) + (xcd - r8) * q8 + slot;
    const int row = (int)(logical / (uint32_t)a.n_chunks);
    const int chunk = (int)(logical % (uint32_t)a.n_chunks);
    // phase timestamps (diagnostics) are kept in scalar registers and stored at the end
    const bool tron = a.trace != nullptr;
    const uint64_t t0 = tron ? wall_clock64() : 0;
    if (row >= a.n_rows) return;

    const uint32_t V = (uint32_t)a.V;
    const uint32_t c0 = (uint32_t)chunk * (uint32_t)a.chunk;
    const uint32_t c1 = min(c0 + (uint32_t)a.chunk, V);
    // a full, aligned chunk (all but a row's last) takes the unconditional path, compiled
    // apart so its vector-by-vector waits are not merged with the guarded loads
    if (a.vec_ok && c1 - c0 == (uint32_t)(BLOCK * VEC * Elem<BF16>::EPV))
        stream_chunk<BF16, VEC, true>(a, sm, row, chunk, c0, c1, logical, tron, t0);
    else
        stream_chunk<BF16, VEC, false>(a, sm, row, chunk, c0, c1, logical, tron, t0);
}

template <bool BF16, int VEC, bool FULL>
__device__ __forceinline__ void stream_chunk(const KArgs& a, StreamSmem& sm, int row, int chunk, uint32_t c0,
                                             uint32_t c1, uint32_t logical, bool tron, uint64_t t0) {
    constexpr int EPV = Elem<BF16>::EPV;
    const int tid = threadIdx.x, lane = lane_id(), w = wave_id();
    uint64_t ts[8] = {t0, 0, 0, 0, 0, 0, 0, 0};
#define BFI_STAMP(i)                          \
    do {                                     \
        if (tron) ts[(i)] = wall_clock64(); \
    } while (0)
    const uint32_t em = (1u << EPV) - 1u;

    // The loads depend on kernel arguments only and go out first: the row's parameters
    // (scalar loads that queue behind other workgroups' traffic) arrive meanwhile. The
    // allow-mask words go before the logits, so pass 1 can start on the first vector while
    // the rest are in flight. A history of at most PREPEN_H ids is applied here
    // (sample.rs:345-367): its ids go out after the first half of a full chunk's logits, so
    // that the two scalar loads of the row's offsets they need do not hold up the logits,
    // and before the second half, so they land while pass 1 is still waiting for data.
    const HistView hv = row_history(a, row);
    const uint32_t* mrow = a.mask ? a.mask + (int64_t)row * a.mask_stride : nullptr;
    uint32_t mwd[VEC];
    if (mrow) {
#pragma unroll
        for (int q = 0; q < VEC; q++) {
            const uint32_t id0 = c0 + (uint32_t)(q * BLOCK + tid) * EPV;
            mwd[q] = id0 < c1 ? mrow[id0 >> 5] : 0u;
        }
    }
    float x[VEC][EPV];
    if (FULL) load_full_range<BF16, VEC, 0, (VEC + 1) / 2>(a, row, c0, x);
    constexpr int HPT = PREPEN_H / BLOCK;
    uint32_t hid[HPT];
    {
        const int64_t hn = hv.size();
        if (hn > 0 && hn <= (int64_t)PREPEN_H) {
#pragma unroll
            for (int g = 0; g < HPT; g++) {
                const int64_t j = (int64_t)g * BLOCK + tid;
                hid[g] = j < hn ? hv.at(j) : 0xFFFFFFFFu;
            }
        }
    }
    if (FULL) load_full_range<BF16, VEC, (VEC + 1) / 2, VEC>(a, row, c0, x);
    else load_tile<BF16, VEC>(a, row, c0, c1, x);
    BFI_STAMP(1);
    const RowCtx C = make_ctx(a, row);
    if (!C.active) return;  // a verify row past its draft: the loads are dropped

    // penalties: the ids inside this chunk are counted in LDS (the barriers pass while the
    // second half of the logits is in flight), then each thread reads the counts of its
    // elements and pass 1 penalizes them as they arrive
    uint32_t cw[VEC][EPV / 2];
    if (C.prepen) {
        uint4* hc4 = reinterpret_cast<uint4*>(sm.u.hc);
        for (int i = tid; i < CHUNK_MAX / 8; i += BLOCK) hc4[i] = make_uint4(0u, 0u, 0u, 0u);
        __syncthreads();  // cleared before any count lands
#pragma unroll
        for (int g = 0; g < HPT; g++) {  // 16-bit counts: at most PREPEN_H each
            const uint32_t d = hid[g] - c0;
            if (hid[g] < c1 && hid[g] >= c0) lds_add(&sm.u.hc[d >> 1], 1u << (16 * (d & 1u)));
        }
        __syncthreads();
#pragma unroll
        for (int q = 0; q < VEC; q++) {
            const uint32_t d0 = (uint32_t)(q * BLOCK + tid) * EPV;
            if constexpr (EPV == 4) {
                const uint2 v = *reinterpret_cast<const uint2*>(&sm.u.hc[d0 >> 1]);
                cw[q][0] = v.x;
                cw[q][1] = v.y;
            } else {
                const uint4 v = *reinterpret_cast<const uint4*>(&sm.u.hc[d0 >> 1]);
                cw[q][0] = v.x;
                cw[q][1] = v.y;
                cw[q][2] = v.z;
                cw[q][3] = v.w;
            }
        }
    }

    ChunkPart part;
    part.pad = 0;
    part.pad2 = 0;
    part.raw_m = -__builtin_inff();
    part.raw_arg = 0xFFFFFFFFu;
    part.arg = 0;
    // pass 1, vector by vector as the loads land: the mask (sample.rs:331-337) and the
    // penalties in place, the running max (with its first index: greedy rows over the
    // penalized values, sample.rs:429-439; rows with min_p > 1 over the masked, un-penalized
    // ones for the min-p fallback, sample.rs:415-422) and the running sum of
    // exp((x - max) / T) rescaled when the max grows (sample.rs:376-386 sums exp(s - max)).
    // max(x / T) = max(x) / T for T > 0, so the chunk's exact maximum takes one division.
    const bool track_raw = !C.greedy && (C.min_p > 1.0f);
    const bool track_arg = C.greedy || track_raw;
    const bool sums = !C.greedy;
    ArgMax best{-__builtin_inff(), 0xFFFFFFFFu};
    float m = -__builtin_inff(), s = 0.0f;
#pragma unroll
    for (int q = 0; q < VEC; q++) {
        const uint32_t id0 = c0 + (uint32_t)(q * BLOCK + tid) * EPV;
        if (mrow) {
            const uint32_t mb = (mwd[q] >> (id0 & 31)) & em;
#pragma unroll
            for (int e = 0; e < EPV; e++) x[q][e] = ((mb >> e) & 1u) ? x[q][e] : -__builtin_inff();
        }
        if (track_raw) {
#pragma unroll
            for (int e = 0; e < EPV; e++) best = argmax_merge(best, ArgMax{x[q][e], id0 + e});
        }
        if (C.prepen) {
            uint32_t any = 0;
#pragma unroll
            for (int i = 0; i < EPV / 2; i++) any |= cw[q][i];
            if (any) {  // rare: a history id among these elements
#pragma unroll
                for (int e = 0; e < EPV; e++) {
                    const uint32_t cnt = (cw[q][e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
                    if (cnt) x[q][e] = penalize(x[q][e], cnt, C.pen);
                }
            }
        }
        if (C.greedy) {
#pragma unroll
            for (int e = 0; e < EPV; e++) best = argmax_merge(best, ArgMax{x[q][e], id0 + e});
        }
        float vm = x[q][0];
#pragma unroll
        for (int e = 1; e < EPV; e++) vm = fmaxf(vm, x[q][e]);
        const float mn = fmaxf(m, vm);
        if (sums) {
            const float mz = mn > -__builtin_inff() ? mn : 0.0f;  // all masked so far: terms are 0
            float g = 0.0f;
#pragma unroll
            for (int e = 0; e < EPV; e++) g += stream_term(C, x[q][e], mz);
            s = s * stream_term(C, m, mz) + g;
        }
        m = mn;
    }
    BFI_STAMP(2);
    // the wave's (max, sum), then the chunk's from the NWAVE wave results (one barrier)
    {
        const float mw = wave_max(m);
        double sw = 0.0;
        if (sums) {
            const float mwz = mw > -__builtin_inff() ? mw : 0.0f;
            sw = wave_sum_d((double)(s * stream_term(C, m, mwz)));
        }
        ArgMax bw{mw, 0xFFFFFFFFu};
        if (track_arg) bw = wave_argmax(best);
        if (lane == 0) {
            sm.wm[w] = mw;
            sm.ws[w] = sw;
            sm.wbv[w] = bw.v;
            sm.wa[w] = bw.i;
        }
    }
    __syncthreads();
    float lm = sm.wm[0];
#pragma unroll
    for (int i = 1; i < NWAVE; i++) lm = fmaxf(lm, sm.wm[i]);
    part.raw_m = lm;  // the reference point of the sums: the chunk's largest (penalized) logit
    if (track_arg) {
        best = ArgMax{sm.wbv[0], sm.wa[0]};
#pragma unroll
        for (int i = 1; i < NWAVE; i++) best = argmax_merge(best, ArgMax{sm.wbv[i], sm.wa[i]});
        part.raw_arg = best.i;
        if (!C.greedy) part.raw_m = best.v;  // min_p > 1: the masked, un-penalized maximum
    }
    BFI_STAMP(3);
    if (C.greedy) {
        part.m = best.v;
        part.arg = best.i;
        part.sum = 0.0;
        part.ncand = 0;
        part.theta = -__builtin_inff();
    } else {
        double ls = 0.0;
        if (lm > -__builtin_inff()) {
#pragma unroll
            for (int i = 0; i < NWAVE; i++) ls += sm.ws[i] * (double)stream_term(C, sm.wm[i], lm);
        }
        part.sum = ls;
        const float mc = div_T(lm, C);  // exact (sample.rs:373-375)
        part.m = mc;
        const bool kb = C.kmode && C.k <= CAND_CAP;
        const float margin = 1e-4f + 1e-5f * fabsf(mc);
        if (!(mc > -__builtin_inff())) {
            part.ncand = 0;
            part.theta = -__builtin_inff();
        } else if (!(C.mmode || kb)) {
            part.ncand = NCAND_UNBOUNDED;
            part.theta = __builtin_inff();
        } else {
            // min-p bound of this chunk: p >= min_p * max p needs s >= max_s + ln(min_p)
            float th = __builtin_inff();
            if (C.mmode) {
                const float lmp = logf(C.min_p);
                th = mc + lmp - (margin + 1e-5f * fabsf(lmp));
            }
            // candidates are finite elements at or above x_bound(th)
            float xw = fmaxf(x_bound(C, th), -__FLT_MAX__);
            Cand* seg = sm.u.stage[w];
            uint32_t wc = C.mmode ? stage_cands<BF16, VEC>(x, xw, seg, c0) : 0u;
            BFI_STAMP(4);
            if (lane == 0) sm.wc[w] = wc;
            __syncthreads();
            BFI_STAMP(5);
            uint32_t cnt = 0, pre = 0;
#pragma unroll
            for (int i = 0; i < NWAVE; i++) {
                const uint32_t c = sm.wc[i];
                pre += i < w ? c : 0u;
                cnt += c;
            }
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
                xw = fmaxf(x_bound(C, th), -__FLT_MAX__);
                wc = stage_cands<BF16, VEC>(x, xw, seg, c0);
                if (lane == 0) sm.wc2[w] = wc;
                __syncthreads();
                cnt = 0;
                pre = 0;
#pragma unroll
                for (int i = 0; i < NWAVE; i++) {
                    const uint32_t ci = sm.wc2[i];
                    pre += i < w ? ci : 0u;
                    cnt += ci;
                }
            }
            part.theta = th;
            if (cnt > (uint32_t)CAND_CAP) {
                part.ncand = NCAND_OVERFLOW;
            } else {
                // every element whose exact value is >= th (a few just below may come along):
                // each wave's staged run, copied out at the wave's offset
                part.ncand = cnt;
                Cand* dst = a.cands + ((int64_t)row * a.n_chunks + chunk) * CAND_CAP + pre;
                if (wc <= (uint32_t)SEG) {
                    for (uint32_t j = (uint32_t)lane; j < wc; j += WAVE) dst[j] = seg[j];
                } else {
                    emit_cands<BF16, VEC>(x, xw, dst, 0u, c0);
                }
            }
        }
    }
    BFI_STAMP(6);
    if (tid == 0) a.parts[(int64_t)row * a.n_chunks + chunk] = part;
    BFI_STAMP(7);
    if (tron && tid == 0) {
        const int64_t tb = (int64_t)logical * 8;
#pragma unroll
        for (int i = 0; i < 8; i++) a.trace[tb + i] = ts[i];
    }
#undef BFI_STAMP
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
