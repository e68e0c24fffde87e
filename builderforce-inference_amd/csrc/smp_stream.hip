// smp_stream.hip — the streaming pass of the gfx950 token sampler.
//
// One launch covers every row of a batch (generate_batch's per-step call, engine/mod.rs:
// 316-322) or every draft row of a spec-verify step (engine/spec.rs:137-162). Workgroup
// (row, chunk) reads `chunk` logits of one row once from HBM with 16-byte loads, keeps them
// in VGPRs and applies the allow-mask (sample.rs:331-337) and, for histories of at most
// PREPEN_H ids, the penalties (sample.rs:345-367). Per chunk it writes the exact maximum of
// x / T (sample.rs:373-379), the first index of the maximum for greedy rows (sample.rs:
// 429-439) and of the un-penalized maximum for the min-p fallback (sample.rs:415-422), an
// approximate f64 mass, and for top-k / top-p rows a 128-bucket histogram of how far below
// the chunk maximum its elements lie. The last workgroup of a row to finish (an arrival
// counter) combines the chunks: the row maximum, the approximate normalizer mass before
// each chunk (the quantizing pass's prediction of the running sum, smp_quant.hip) and the
// bound the kept set lies above (the candidates the passes after it gather).
#include <hip/hip_ext.h>

#include "smp_common.h"

namespace bfi {

struct __align__(16) StreamSmem {
    double ws[NWAVE];   // per-wave sums (relative to the wave max)
    float wm[NWAVE];    // per-wave maxima of the masked logits
    float wbv[NWAVE];   // per-wave argmax value (greedy rows: penalized; min_p > 1: raw)
    uint32_t wa[NWAVE]; // per-wave first index of that value
    uint32_t last;      // this workgroup finishes the row
    uint32_t pad[3];
    float xm[NCMAX];    // the row finisher: each chunk's maximum
    uint32_t hc[CHUNK_MAX / 2];  // history counts of the chunk's ids, two 16-bit halves a word;
                                 // then the histogram (HBINS words); the row finisher's grids
};
static_assert(2 * HBINS <= CHUNK_MAX / 2, "the histogram reuses the count array");

constexpr int HB_CBITS = 20;              // histogram bins: count bits (a chunk holds at most 8192)
static_assert(CHUNK_MAX < (1 << HB_CBITS), "bin counts");
constexpr int NGRID = 512;                // gather-bound grid: bounds -g/8 log2-units, g < NGRID
constexpr double MFIX = 1099511627776.0;  // 2^40: fixed point of the grid masses
static_assert(NGRID * 3 + NCMAX * 3 <= CHUNK_MAX / 2, "the grids and the chunk factors reuse the count array");

// The candidate bound from the chunks' histograms: bin j of chunk c holds the count and the
// mass (terms relative to the chunk maximum) of the elements j/4 .. (j+1)/4 log2-units below
// the chunk maximum xm_c, which lies o_c = (xmax - xm_c) log2(e) / T below the row's. On a
// grid of bounds theta_g = -g/8 (log2-units of exp(s - M)) the bins entirely above theta_g
// give lower bounds on the count and on the mass of the elements above it (the masses
// lowered for the estimates' and the f32 accumulation's errors); the bound is the highest
// theta_g whose lower bounds reach k (top-k) or the top-p share of an upper bound on the
// normalizer with margins for the reference's rounding (sample.rs:392-409). Every kept
// element lies above it.
constexpr int HPER = 16;  // histogram words a thread loads at a time

// The first HPER * BLOCK words of a row's chunk histograms (the last bin of each is not used):
// loaded at the start of the row finisher, beside its other loads.
__device__ __forceinline__ void hist_prefetch(const KArgs& a, int row, uint64_t (&hv)[HPER]) {
    const int tid = threadIdx.x;
    const int nc = a.n_chunks;
    const uint64_t* vh = reinterpret_cast<const uint64_t*>(a.vhist + (int64_t)row * nc * 2 * HBINS);
#pragma unroll
    for (int r = 0; r < HPER; r++) {
        const int idx = r * BLOCK + tid;
        hv[r] = (idx < nc * HBINS && (idx % HBINS) != HBINS - 1) ? ld_dev64(vh + idx) : 0ull;
    }
}

__device__ __forceinline__ float gather_bound(const KArgs& a, StreamSmem& sm, const RowCtx& C, float xmax,
                                              double S_hi, const uint64_t (&hv0)[HPER]) {
    const int tid = threadIdx.x;
    const int nc = a.n_chunks;
    uint32_t* CL = sm.hc;
    uint64_t* ML = reinterpret_cast<uint64_t*>(sm.hc + NGRID);
    for (int g = tid; g < NGRID; g += BLOCK) {
        CL[g] = 0u;
        ML[g] = 0ull;
    }
    __syncthreads();
    const float eps = 0x1p-8f;
    // per chunk: its maximum's offset below the row's in grid units, and the factor that
    // takes its bins' masses (relative to its maximum) to the row's scale, lowered for the
    // estimates' errors (one exp2 per chunk, not per bin)
    double* CS = reinterpret_cast<double*>(sm.hc + NGRID * 3);
    float* CO = reinterpret_cast<float*>(CS + NCMAX);
    if (tid < nc) {
        const float o = (xmax - sm.xm[tid]) * C.rTl;
        CO[tid] = 8.0f * o + 8.0f * eps;
        CS[tid] = C.pmode ? exp2(-(double)o - (double)eps) * (1.0 - 0x1p-9) * MFIX : 0.0;
    }
    __syncthreads();
    // the chunks' histograms, HPER bins per thread in flight together (the first batch
    // prefetched)
    constexpr int PER = HPER;
    const uint32_t* vh = a.vhist + (int64_t)C.row * nc * 2 * HBINS;
    for (int b0 = 0; b0 < nc * HBINS; b0 += PER * BLOCK) {
        uint64_t hv[PER];
#pragma unroll
        for (int r = 0; r < PER; r++) {
            const int idx = b0 + r * BLOCK + tid;
            hv[r] = b0 == 0 ? hv0[r]
                            : (idx < nc * HBINS && (idx % HBINS) != HBINS - 1)
                                  ? ld_dev64(reinterpret_cast<const uint64_t*>(vh) + idx)
                                  : 0ull;
        }
#pragma unroll
        for (int r = 0; r < PER; r++) {
            const uint32_t cnt = C.kmode ? (uint32_t)(hv[r] & ((1u << HB_CBITS) - 1u)) : 0u;
            const float ms = C.pmode ? (float)(hv[r] >> HB_CBITS) * 0x1p-24f : 0.0f;
            if (!cnt && !(ms > 0.0f)) continue;
            const int idx = b0 + r * BLOCK + tid;
            const int c = idx / HBINS, j = idx % HBINS;
            const float glo = ceilf(CO[c] + (float)(8 * (j + 1) / HBIN_PER_LOG2));
            if (glo < (float)NGRID) {
                const int g = (int)glo;
                if (cnt) lds_add(&CL[g], cnt);
                if (ms > 0.0f) lds_add64(&ML[g], (uint64_t)((double)ms * CS[c]));
            }
        }
    }
    __syncthreads();
    // inclusive prefixes over the grid: thread t holds points PG*t .. PG*t + PG - 1
    constexpr int PG = NGRID / BLOCK;
    uint32_t cs = 0;
    uint64_t ms = 0;
#pragma unroll
    for (int i = 0; i < PG; i++) {
        cs += CL[tid * PG + i];
        ms += ML[tid * PG + i];
    }
    uint32_t ct;
    uint64_t mt;
    uint32_t cpre = block_excl_scan<uint32_t>(cs, sm.wa, ct);
    uint64_t mpre = block_excl_scan<uint64_t>(ms, reinterpret_cast<uint64_t*>(sm.ws), mt);
    uint32_t gk = 0xFFFFFFFFu, gp = 0xFFFFFFFFu;
    const double tgt = (double)fminf(C.top_p * 1.01f + 3e-4f, 2.0f) * S_hi * MFIX;
#pragma unroll
    for (int i = 0; i < PG; i++) {
        cpre += CL[tid * PG + i];
        mpre += ML[tid * PG + i];
        const uint32_t g = (uint32_t)(tid * PG + i);
        if (C.kmode && cpre >= (uint32_t)C.k) gk = min(gk, g);
        if (C.pmode && (double)mpre >= tgt) gp = min(gp, g);
    }
    gk = block_min_u(gk, sm.wa);
    gp = block_min_u(gp, sm.wa);
    float th = -__builtin_inff();
    if (C.kmode && gk != 0xFFFFFFFFu) th = fmaxf(th, -(float)gk / 8.0f);
    if (C.pmode && gp != 0xFFFFFFFFu) th = fmaxf(th, -(float)gp / 8.0f);
    return th;
}

// The row results from all chunks (the last workgroup of the row; every thread calls it).
__device__ __forceinline__ void finish_row(const KArgs& a, StreamSmem& sm, const RowCtx& C) {
    const int row = C.row;
    const int tid = threadIdx.x;
    const int nc = a.n_chunks;
    static_assert(NCMAX <= BLOCK, "one chunk per thread");
    // the histograms the candidate bound reads, in flight with the chunk results
    const bool bound = !C.greedy && (C.kmode || C.pmode) && !(C.min_p >= 0x1p-10f) && !C.pen_hash;
    uint64_t hv[HPER];
    if (bound) hist_prefetch(a, row, hv);
    ChunkPart P;
    P.m = -__builtin_inff();
    P.xm = -__builtin_inff();
    P.raw_m = -__builtin_inff();
    P.arg = P.raw_arg = 0xFFFFFFFFu;
    P.sum = 0.0;
    if (tid < nc) {
        uint64_t* pp = reinterpret_cast<uint64_t*>(a.parts + (int64_t)row * nc + tid);
        uint64_t w[4];
#pragma unroll
        for (int i = 0; i < 4; i++) w[i] = ld_dev64(pp + i);
        P = __builtin_bit_cast(ChunkPart, w);
        sm.xm[tid] = P.xm;
    }
    RowInfo R;
    R.M = block_max(P.m, sm.wm);
    R.xmax = block_max(P.xm, sm.wm);
    R.gk = C.greedy ? block_max_u64(tid < nc ? argmax_key(P.m, P.arg) : 0ull, reinterpret_cast<uint64_t*>(sm.ws)) : 0ull;
    R.rk = C.min_p > 1.0f ? block_max_u64(tid < nc ? argmax_key(P.raw_m, P.raw_arg) : 0ull,
                                          reinterpret_cast<uint64_t*>(sm.ws))
                          : 0ull;
    R.th = __builtin_inff();
    R.S_apx = 0.0f;
    if (!C.greedy) {
        const double mass = P.xm > -__builtin_inff() ? P.sum * exp2((double)((P.xm - R.xmax) * C.rTl)) : 0.0;
        double tot;
        const double pre = block_excl_scan<double>(mass, sm.ws, tot);
        // the chunk maximum's term, from below: exactly 1 for the row maximum, else its
        // estimate less the estimate's error (the roundings of x / T and of M)
        float lb = 0.0f;
        if (P.m == R.M) lb = 1.0f;
        else if (P.xm > -__builtin_inff())
            lb = exp2f((P.xm - R.xmax) * C.rTl) * (1.0f - 0x1p-12f - fabsf(R.M) * 0x1p-22f);
        const float lbw = wave_scan_incl(lb, 0.0f, [](float u, float v) { return fmaxf(u, v); });
        if (lane_id() == WAVE - 1) sm.wm[wave_id()] = lbw;
        __syncthreads();
        float lbx = __int_as_float(__shfl_up(__float_as_int(lbw), 1));  // the exclusive prefix maximum
        lbx = lane_id() == 0 ? 0.0f : lbx;
#pragma unroll
        for (int w = 0; w < NWAVE; w++) lbx = w < wave_id() ? fmaxf(lbx, sm.wm[w]) : lbx;
        __syncthreads();
        if (tid < nc) a.qpre[(int64_t)row * nc + tid] = QPre{(float)pre, fmaxf(lbx, 0.0f)};
        R.S_apx = (float)tot;
        const bool list_mode = C.kmode || C.pmode || C.mmode;
        float th = -__builtin_inff();
        if (bound && R.xmax > -__builtin_inff()) th = gather_bound(a, sm, C, R.xmax, tot * (1.0 + 1e-4), hv);
        if (C.mmode) th = fmaxf(th, log2f(C.min_p) - 0x1p-6f);
        if (list_mode) R.th = th;
    }
    if (tid == 0) {
        a.rinfo[row] = R;
        a.rowcnt[row] = 0u;
        a.arrive[row] = 0u;
    }
}

template <bool BF16, int VEC, bool FULL>
__device__ __forceinline__ void stream_chunk(const KArgs& a, StreamSmem& sm, int row, int chunk, uint32_t c0,
                                             uint32_t c1);

// Phase timestamp of a workgroup (diagnostics): words after the quantizing pass's and the rows'.
#define BFI_STRACE(a, row, chunk, i)                                                                  \
    BFI_TRACE(a, (int64_t)(a).n_rows * (a).n_chunks * 8 + (int64_t)(a).n_rows * 16 +                 \
                     ((int64_t)(row) * (a).n_chunks + (chunk)) * 8,                                  \
              i)

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
    if (row >= a.n_rows) return;
    const uint32_t V = (uint32_t)a.V;
    const uint32_t c0 = (uint32_t)chunk * (uint32_t)a.chunk;
    const uint32_t c1 = min(c0 + (uint32_t)a.chunk, V);
    // a full, aligned chunk (all but a row's last) takes the unconditional path, compiled
    // apart so its vector-by-vector waits are not merged with the guarded loads
    if (a.vec_ok && c1 - c0 == (uint32_t)(BLOCK * VEC * Elem<BF16>::EPV))
        stream_chunk<BF16, VEC, true>(a, sm, row, chunk, c0, c1);
    else
        stream_chunk<BF16, VEC, false>(a, sm, row, chunk, c0, c1);
}

template <bool BF16, int VEC, bool FULL>
__device__ __forceinline__ void stream_chunk(const KArgs& a, StreamSmem& sm, int row, int chunk, uint32_t c0,
                                             uint32_t c1) {
    constexpr int EPV = Elem<BF16>::EPV;
    const int tid = threadIdx.x, lane = lane_id(), w = wave_id();
    const uint32_t em = (1u << EPV) - 1u;

    // The loads depend on kernel arguments only and go out first: the row's parameters
    // (scalar loads that queue behind other workgroups' traffic) arrive meanwhile. The
    // allow-mask words go before the logits, so the pass can start on the first vector while
    // the rest are in flight; the history ids go between the two halves of the logits.
    BFI_STRACE(a, row, chunk, 0);
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
    const RowCtx C = make_ctx(a, row);
    if (!C.active) return;  // a verify row past its draft: the loads are dropped

    // penalties: the ids inside this chunk are counted in LDS (the barriers pass while the
    // second half of the logits is in flight), then each thread reads the counts of its
    // elements and the pass penalizes them as they arrive
    uint32_t cw[VEC][EPV / 2];
    if (C.prepen) {
        uint4* hc4 = reinterpret_cast<uint4*>(sm.hc);
        for (int i = tid; i < CHUNK_MAX / 8; i += BLOCK) hc4[i] = make_uint4(0u, 0u, 0u, 0u);
        __syncthreads();  // cleared before any count lands
#pragma unroll
        for (int g = 0; g < HPT; g++) {  // 16-bit counts: at most PREPEN_H each
            const uint32_t d = hid[g] - c0;
            if (hid[g] < c1 && hid[g] >= c0) lds_add(&sm.hc[d >> 1], 1u << (16 * (d & 1u)));
        }
        __syncthreads();
#pragma unroll
        for (int q = 0; q < VEC; q++) {
            const uint32_t d0 = (uint32_t)(q * BLOCK + tid) * EPV;
            if constexpr (EPV == 4) {
                const uint2 v = *reinterpret_cast<const uint2*>(&sm.hc[d0 >> 1]);
                cw[q][0] = v.x;
                cw[q][1] = v.y;
            } else {
                const uint4 v = *reinterpret_cast<const uint4*>(&sm.hc[d0 >> 1]);
                cw[q][0] = v.x;
                cw[q][1] = v.y;
                cw[q][2] = v.z;
                cw[q][3] = v.w;
            }
        }
    }

    ChunkPart part;
    part.pad = 0;
    part.raw_arg = 0xFFFFFFFFu;
    part.arg = 0;
    // the pass, vector by vector as the loads land: the mask and the penalties in place,
    // the running max (with its first index: greedy rows over the penalized values; rows
    // with min_p > 1 over the masked, un-penalized ones) and the running sum of
    // exp((x - max) / T) rescaled when the max grows (an estimate of the row's normalizer
    // that the row kernel uses only to size its candidate gathering).
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
    BFI_STRACE(a, row, chunk, 1);
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
    // the histogram's bins, cleared while the exchange above settles (the history counts
    // in the same words are all read by now)
    // (rows with min_p >= 2^-10 skip it: every kept element has p >= min_p * max p,
    // sample.rs:411-414, so the min-p bound alone keeps the candidates within 10 log2-units
    // of the maximum)
    const bool want_hist = !C.greedy && (C.kmode || C.pmode) && !(C.min_p >= 0x1p-10f) && a.vhist != nullptr;
    if (want_hist) {
        if (C.prepen) __syncthreads();
        for (int i = tid; i < 2 * HBINS; i += BLOCK) sm.hc[i] = 0u;
    }
    __syncthreads();
    BFI_STRACE(a, row, chunk, 2);
    float lm = sm.wm[0];
#pragma unroll
    for (int i = 1; i < NWAVE; i++) lm = fmaxf(lm, sm.wm[i]);
    part.raw_m = lm;  // the chunk's largest (penalized) masked logit: the sums' reference point
    if (track_arg) {
        best = ArgMax{sm.wbv[0], sm.wa[0]};
#pragma unroll
        for (int i = 1; i < NWAVE; i++) best = argmax_merge(best, ArgMax{sm.wbv[i], sm.wa[i]});
        part.raw_arg = best.i;
        if (!C.greedy) part.raw_m = best.v;  // min_p > 1: the masked, un-penalized maximum
    }
    if (C.greedy) {
        part.m = best.v;
        part.arg = best.i;
        part.sum = 0.0;
        part.xm = best.v;
    } else {
        double ls = 0.0;
        if (lm > -__builtin_inff()) {
#pragma unroll
            for (int i = 0; i < NWAVE; i++) ls += sm.ws[i] * (double)stream_term(C, sm.wm[i], lm);
        }
        part.sum = ls;
        part.m = div_T(lm, C);  // exact (sample.rs:373-375): max(x / T) = max(x) / T
        part.xm = lm;
    }
    if (want_hist) {
        // bin j: the element lies j/4 .. (j+1)/4 log2-units below the chunk maximum; its
        // count and (top-p rows) its term 2^((x - xm) log2(e) / T) go there; the elements
        // further down and the masked ones are not counted.
        // one 64-bit add per element: the count in the low HB_CBITS bits, the term in fixed
        // point (2^-24 units of the chunk maximum's, truncated: a lower bound) above them
        if (lm > -__builtin_inff()) {
            uint64_t* hb = reinterpret_cast<uint64_t*>(sm.hc);
            const bool pm = C.pmode;
#pragma unroll
            for (int q = 0; q < VEC; q++)
#pragma unroll
                for (int e = 0; e < EPV; e++) {
                    const float d = (x[q][e] - lm) * C.rTl;
                    const float f = -d * (float)HBIN_PER_LOG2;
                    if (f < (float)(HBINS - 1)) {
                        const uint32_t fx = pm ? (uint32_t)(__builtin_amdgcn_exp2f(d) * 16777216.0f) : 0u;
                        lds_add64(&hb[(uint32_t)f], ((uint64_t)fx << HB_CBITS) | 1u);
                    }
                }
        }
        __syncthreads();
        uint32_t* dst = a.vhist + ((int64_t)row * a.n_chunks + chunk) * 2 * HBINS;
        for (int i = tid; i < 2 * HBINS; i += BLOCK) st_dev(dst + i, sm.hc[i]);
    }
    BFI_STRACE(a, row, chunk, 3);
    if (tid < 4) {
        const uint64_t* pw = reinterpret_cast<const uint64_t*>(&part);
        uint64_t v = pw[0];
#pragma unroll
        for (int i = 1; i < 4; i++) v = tid == i ? pw[i] : v;
        st_dev64(reinterpret_cast<uint64_t*>(a.parts + (int64_t)row * a.n_chunks + chunk) + tid, v);
    }
    // the last chunk of the row to arrive finishes it: the chunk results go out with
    // device-coherent stores, each wave waits for its own before the count, and the finisher
    // reads them from the coherence point (no cache writeback or invalidation, which would
    // cost every workgroup and evict the logits the others stream)
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __syncthreads();
    if (tid == 0) sm.last = glb_add(&a.arrive[row], 1u) == (uint32_t)(a.n_chunks - 1) ? 1u : 0u;
    __syncthreads();
    BFI_STRACE(a, row, chunk, 4);
    if (!sm.last) return;
    finish_row(a, sm, C);
    BFI_STRACE(a, row, chunk, 5);
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
