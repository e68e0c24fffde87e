// smp_quant.hip — the quantizing pass of the gfx950 token sampler (between the streaming pass
// and the row kernel), one 512-thread workgroup per (row, chunk) over the whole GPU.
//
// The reference's normalizer is a sequential f32 sum over the row (sample.rs:381-386). While
// the running sum stays inside one binade [2^k, 2^(k+1)), each addition moves it by a whole
// number of units u = 2^(k-23): RN(e / u) (smp_exact.h). From the row maximum M and the
// approximate normalizer mass before this chunk (both from the streaming pass's row
// finisher), a workgroup predicts the running sum before each of its elements, and so the
// binade each addition lands in. The prediction is an interval: the estimated prefix
// widened by QEPS relative both ways (several times the f32 sum's largest drift from the
// exact one on the benchmark rows), raised to the largest term added so far (the f32 sum
// never falls below any of its terms). An element is "certain" when the interval before its
// addition and the one after lie in one binade; its units are then RN(e / u) at that
// binade, exactly (a precise estimate, or glibc's expf where the estimate lies near a
// rounding boundary). The others ("windows": near a binade boundary, the row's first
// terms, ties) are listed with their exact exp(s - M). In index order, the certain elements
// between two windows all lie in one binade (the intervals never decrease, so a change of
// binade needs an interval that straddles the boundary: a window), and the pass sums them
// per gap as a run. The row kernel chains the chunks: it adds a run in one step after
// checking that the actual running sum lies in the run's binade and stays there, and walks
// the windows exactly; a failed check re-streams the rest of the chunk exactly, so a wrong
// prediction costs time, never the result. On the way the pass gathers the candidates of
// the kept set into the row's list.
#include <hip/hip_ext.h>

#define BFI_BLOCK 512
#include "smp_chain.h"
#include "smp_common.h"
#include "smp_exact.h"

namespace bfi {

constexpr float QEPS = 0x1p-9f;   // relative width of the running-sum prediction
constexpr float RHO0 = 0x1p-19f;  // relative error bound of the precise exp estimate
constexpr float L2E_HI = 1.44269502162933349609375f;  // fl(log2(e))
constexpr float L2E_LO = 1.925963033500011079e-8f;    // log2(e) - L2E_HI
constexpr float LN2_F = 0.693147180559945309f;
constexpr uint32_t UE_BIAS = 1024u;
constexpr int QVMAX = 4;             // 16-byte vectors per thread

struct __align__(16) QuantSmem {
    uint32_t hc[CHUNK_MAX / 2];  // history counts of the chunk's ids (two 16-bit halves a word)
    uint32_t rq[QWIN + 1];   // per run: units
    uint32_t rhi[QWIN + 1];  // per run: its unit exponent + 150 (0: no element)
    float vs[QVMAX][NWAVE];  // per vector, per wave: sums of the estimates
    float vm[QVMAX][NWAVE];  // per vector, per wave: largest term (lower bound)
    uint32_t vc[QVMAX][NWAVE];  // per vector, per wave: window counts
    uint32_t wg[NWAVE];
    uint32_t wb[NWAVE];
    uint32_t gbase;
};

__device__ __forceinline__ uint32_t lds_min(uint32_t* p, uint32_t v) {
    return __hip_atomic_fetch_min((BFI_LDS uint32_t*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// exp(fl(x / T) - M) exactly as the reference rounds it (sample.rs:374, 383); out of line:
// glibc's expf should exist once in the kernel's code.
__device__ __noinline__ float quant_exact(float x, float T, float rT, int32_t fast_div, float M) {
    float s;
    const uint32_t ax = __float_as_uint(x) & 0x7FFFFFFFu;
    if (fast_div && !((ax - 1u < 0x0D7FFFFFu) || (ax - 0x71800000u < 0x0E000000u))) {
        const float q = x * rT;
        const float er = __builtin_fmaf(-q, T, x);
        s = er != er ? q : __builtin_fmaf(er, rT, q);
    } else {
        s = x / T;
    }
    return expf_ref(s - M);
}

template <bool BF16, int QV, bool FULL>
__device__ __forceinline__ void quant_chunk(const KArgs& a, QuantSmem& sm, int row, int chunk, uint32_t c0,
                                            uint32_t c1);

template <bool BF16, int QV>
__global__ __launch_bounds__(BLOCK) __attribute__((amdgpu_waves_per_eu(4))) void k_quant(KArgs a) {  // 2 workgroups per CU
    __shared__ QuantSmem sm;
    const uint32_t G = gridDim.x, bid = blockIdx.x;
    const uint32_t q8 = G / 8, r8 = G % 8, xcd = bid % 8, slot = bid / 8;
    const uint32_t logical = xcd < r8 ? xcd * (q8 + 1) + slot : r8 * (q8 + 1) + (xcd - r8) * q8 + slot;
    const int row = (int)(logical / (uint32_t)a.n_chunks);
    const int chunk = (int)(logical % (uint32_t)a.n_chunks);
    if (row >= a.n_rows) return;
    const uint32_t V = (uint32_t)a.V;
    const uint32_t c0 = (uint32_t)chunk * (uint32_t)a.chunk;
    const uint32_t c1 = min(c0 + (uint32_t)a.chunk, V);
    if (a.vec_ok && c1 - c0 == (uint32_t)(BLOCK * QV * Elem<BF16>::EPV))
        quant_chunk<BF16, QV, true>(a, sm, row, chunk, c0, c1);
    else
        quant_chunk<BF16, QV, false>(a, sm, row, chunk, c0, c1);
}

// The units RN(e / 2^ue) of one element (ue = elo - 150) from the precise estimate: s =
// fl(x / T) exactly (Markstein's corrected quotient, for |x| in [2^-100, 2^100) and T in
// [2^-20, 2^20]), d = fl(s - M) as the reference rounds it, exp(d) = 2^(h + l) with
// h = fl(d log2(e)) and l its rounding error plus log2(e)'s own, as exp2(h) (1 + l ln 2),
// within RHO0 of glibc's expf(d); below 2^-120, 2^(h - ue) directly with its exponent's
// rounding added to the bound. `sure`: the estimate lies far enough from a rounding
// boundary (else the element is a window and its exact value decides). Straight-line.
__device__ __forceinline__ uint32_t elem_units(float xv, uint32_t elo, bool fdiv, float T, float rT, float M,
                                               bool& sure) {
    const int32_t ue = (int32_t)elo - 150;
    const uint32_t ax = __float_as_uint(xv) & 0x7FFFFFFFu;
    const bool dok = fdiv & (((ax - 0x0D800000u) < 0x64000000u) | (ax == 0u));
    const float q0 = xv * rT;
    const float r0 = __builtin_fmaf(-q0, T, xv);
    const float d = __builtin_fmaf(r0, rT, q0) - M;
    const float h = d * L2E_HI;
    const float l = __builtin_fmaf(d, L2E_LO, __builtin_fmaf(d, L2E_HI, -h));
    const bool tiny = h < -120.0f;
    const float z = __builtin_amdgcn_exp2f(tiny ? h - (float)ue : h);
    const float tz = __builtin_fmaf(z, l * LN2_F, z);
    const float t = tiny ? tz : __builtin_ldexpf(tz, -ue);
    const float rho = tiny ? __builtin_fmaf(fabsf(h) + 160.0f, 0x1p-24f, RHO0) : RHO0;
    const float qf = __builtin_rintf(t);
    sure = dok & (__builtin_fmaf(t, rho, fabsf(t - qf)) < 0.5f) & (t < 8388608.0f);
    return (uint32_t)qf;
}

// The term's lower bound for the running-sum prediction: exactly 1 for the row maximum's
// value (exp(0)), else the cheap estimate less its error.
__device__ __forceinline__ float term_lb(float x, float ev, float xmax, float M) {
    return x == xmax ? 1.0f : ev * (1.0f - 0x1p-12f - fabsf(M) * 0x1p-22f);
}

template <bool BF16, int QV, bool FULL>
__device__ __forceinline__ void quant_chunk(const KArgs& a, QuantSmem& sm, int row, int chunk, uint32_t c0,
                                            uint32_t c1) {
    constexpr int EPV = Elem<BF16>::EPV;
    static_assert(QV <= QVMAX, "per-vector tables");
    const int tid = threadIdx.x, lane = lane_id(), w = wave_id();
    const uint32_t em = (1u << EPV) - 1u;
    const int nc = a.n_chunks;
    const int64_t rc = (int64_t)row * nc + chunk;
    const int64_t tb = rc * 8;  // diagnostics: this workgroup's phase stamps
    BFI_TRACE(a, tb, 0);
    // the logits first (they depend on nothing), then the row's context and results
    const uint32_t* mrow = a.mask ? a.mask + (int64_t)row * a.mask_stride : nullptr;
    uint32_t mwd[QV];
    if (mrow) {
#pragma unroll
        for (int q = 0; q < QV; q++) {
            const uint32_t id0 = c0 + (uint32_t)(q * BLOCK + tid) * EPV;
            mwd[q] = id0 < c1 ? mrow[id0 >> 5] : 0u;
        }
    }
    float x[QV][EPV];
    if (FULL) load_full_tile<BF16, QV>(a, row, c0, x);
    else load_tile<BF16, QV>(a, row, c0, c1, x);
    const RowCtx C = make_ctx(a, row);
    if (!C.active) return;
    const float M = ld_uniform(&a.rinfo[row].M);
    if (!quant_row(C, M)) return;
    const float th = ld_uniform(&a.rinfo[row].th);
    const float xmax = ld_uniform(&a.rinfo[row].xmax);
    const float xm = ld_uniform(&a.parts[rc].xm);
    const float Pc = ld_uniform(&a.qpre[rc].P);
    const float Lc = ld_uniform(&a.qpre[rc].lb);
    QHead* const head = a.qhead + rc;
    QItem* const items = a.qitem + rc * (a.qcap + 1);
    const float Kc = -(M * 1.44269504088896341f);
    // candidates: (x / T - M) log2(e) estimated as x * rTl + Kc, above the bound less the
    // estimate's error (the roundings of x / T, of M and of the products, in log2-units)
    const float gth = th - (0x1p-8f + (fabsf(M) * 12.0f + 200.0f) * 0x1p-24f);
    const float amax = xm > -__builtin_inff() ? __builtin_fmaf(xm, C.rTl, Kc) : -__builtin_inff();
    const bool gather = amax >= gth;
    // a chunk whose largest term is below half a unit of the predicted running sum's lowest
    // binade adds nothing: one zero run, valid from that binade up
    const float lo0 = fmaxf(Pc * (1.0f - QEPS), Lc);
    const uint32_t elo0 = max(__float_as_uint(lo0) >> 23, 1u);
    const int32_t ue0 = (int32_t)elo0 - 150;
    const bool trivial = amax < -120.0f ? ue0 > -100 : __builtin_ldexpf(__builtin_amdgcn_exp2f(amax), -ue0) < 0.49f;
    BFI_TRACE(a, tb, 1);
    if (trivial) {
        if (tid == 0) {
            head->nwin = 0u;
            head->flags = 0u;
            items[0] = QItem{QI_NONE, 0.0f, 0u, ue0};
        }
        if (!gather) return;
    }
    // the mask and the penalties (histories of at most PREPEN_H ids, counted in LDS)
    constexpr int HPT = PREPEN_H / BLOCK;
    if (C.prepen) {
        const int64_t hn = C.h.size();
        uint32_t hid[HPT];
#pragma unroll
        for (int g = 0; g < HPT; g++) {
            const int64_t j = (int64_t)g * BLOCK + tid;
            hid[g] = j < hn ? C.h.at(j) : 0xFFFFFFFFu;
        }
        uint4* hc4 = reinterpret_cast<uint4*>(sm.hc);
        for (int i = tid; i < CHUNK_MAX / 8; i += BLOCK) hc4[i] = make_uint4(0u, 0u, 0u, 0u);
        __syncthreads();
#pragma unroll
        for (int g = 0; g < HPT; g++) {
            const uint32_t d = hid[g] - c0;
            if (hid[g] < c1 && hid[g] >= c0) lds_add(&sm.hc[d >> 1], 1u << (16 * (d & 1u)));
        }
        __syncthreads();
    }
#pragma unroll
    for (int q = 0; q < QV; q++) {
        const uint32_t id0 = c0 + (uint32_t)(q * BLOCK + tid) * EPV;
        if (mrow) {
            const uint32_t mb = (mwd[q] >> (id0 & 31)) & em;
#pragma unroll
            for (int e = 0; e < EPV; e++) x[q][e] = ((mb >> e) & 1u) ? x[q][e] : -__builtin_inff();
        }
        if (C.prepen) {
            const uint32_t d0 = (uint32_t)(q * BLOCK + tid) * EPV;
            uint32_t cw[EPV / 2];
            if constexpr (EPV == 4) {
                const uint2 v = *reinterpret_cast<const uint2*>(&sm.hc[d0 >> 1]);
                cw[0] = v.x;
                cw[1] = v.y;
            } else {
                const uint4 v = *reinterpret_cast<const uint4*>(&sm.hc[d0 >> 1]);
                cw[0] = v.x;
                cw[1] = v.y;
                cw[2] = v.z;
                cw[3] = v.w;
            }
            uint32_t any = 0;
#pragma unroll
            for (int i = 0; i < EPV / 2; i++) any |= cw[i];
            if (any) {  // rare: a history id among these elements
#pragma unroll
                for (int e = 0; e < EPV; e++) {
                    const uint32_t cnt = (cw[e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
                    if (cnt) x[q][e] = penalize(x[q][e], cnt, C.pen);
                }
            }
        }
    }
    BFI_TRACE(a, tb, 2);

    uint32_t qflags = QF_EXACT, qn = 0;  // this chunk's summary (for the first chunk's walk below)
    if (!trivial) {
        // the prediction: cheap estimates e ~ 2^(x rTl + Kc) (shifted below 2^-120), their
        // prefix sums and the largest term's lower bound so far (index order: vector,
        // thread, element), from the row's values at the chunk's start
        float ev[QV][EPV];
        float vpre[QV], vmx[QV], vsum[QV], vtop[QV];
#pragma unroll
        for (int q = 0; q < QV; q++) {
            float g = 0.0f, gm = 0.0f, gt = 0.0f;
#pragma unroll
            for (int e = 0; e < EPV; e++) {
                const float a_ = __builtin_fmaf(x[q][e], C.rTl, Kc);
                const float z = __builtin_amdgcn_exp2f(a_ < -120.0f ? a_ + 64.0f : a_);
                ev[q][e] = x[q][e] > -__builtin_inff() ? (a_ < -120.0f ? __builtin_ldexpf(z, -64) : z) : 0.0f;
                g += ev[q][e];
                gt = fmaxf(gt, ev[q][e]);
                gm = fmaxf(gm, term_lb(x[q][e], ev[q][e], xmax, M));
            }
            vsum[q] = g;
            vtop[q] = gt;
            const float incl = wave_scan_incl(g, 0.0f, [](float u, float v) { return u + v; });
            const float inclm = wave_scan_incl(gm, 0.0f, [](float u, float v) { return fmaxf(u, v); });
            if (lane == WAVE - 1) {
                sm.vs[q][w] = incl;
                sm.vm[q][w] = inclm;
            }
            vpre[q] = wave_excl_of_incl(incl, 0.0f);
            vmx[q] = wave_excl_of_incl(inclm, 0.0f);
        }
        __syncthreads();
        {
            float run = Pc, runm = Lc;
#pragma unroll
            for (int q = 0; q < QV; q++) {
                float tot = 0.0f, mine = 0.0f, totm = 0.0f, minem = 0.0f;
#pragma unroll
                for (int ww = 0; ww < NWAVE; ww++) {
                    const float v = sm.vs[q][ww], vm = sm.vm[q][ww];
                    mine += ww < w ? v : 0.0f;
                    minem = ww < w ? fmaxf(minem, vm) : minem;
                    tot += v;
                    totm = fmaxf(totm, vm);
                }
                vpre[q] += run + mine;
                vmx[q] = fmaxf(vmx[q], fmaxf(runm, minem));
                run += tot;
                runm = fmaxf(runm, totm);
            }
        }
        BFI_TRACE(a, tb, 3);
        // classify and quantize: window bits (the interval straddles a binade boundary, or
        // the estimate lies near a rounding boundary: the chain adds these exactly) and zero
        // bits (masked: they add nothing at any binade). The running sums below 2^-125 (the
        // subnormals and the lowest normal binade) share one spacing, 2^-149: one binade.
        // The units come from the precise estimate: s = fl(x / T) exactly (Markstein's
        // corrected quotient), d = fl(s - M) as the reference rounds it, exp(d) = 2^(h + l)
        // with h = fl(d log2(e)) and l its rounding error plus log2(e)'s own, as
        // exp2(h) (1 + l ln 2), within RHO0 of glibc's expf(d). A certain element keeps
        // (units << 8 | ue + 150) (its units are below 2^23).
        uint32_t pk[QV][EPV];
        uint32_t wm[QV], zm[QV], vs1[QV];  // vs1: the vector lies in one binade (its elo), else 0
        const bool fdiv = __builtin_amdgcn_readfirstlane(C.fast_div ? 1 : 0) != 0;
#pragma unroll
        for (int q = 0; q < QV; q++) {
            // the vector as a whole: the interval from before its first element to after its
            // last one; in one binade, no element of it can straddle a boundary
            const float vlo = fmaxf(vpre[q] * (1.0f - QEPS), vmx[q]);
            const float vhi = (vpre[q] + vsum[q]) * (1.0f + QEPS);
            const uint32_t velo = max(__float_as_uint(vlo) >> 23, 1u), vehi = max(__float_as_uint(vhi) >> 23, 1u);
            const bool same = velo == vehi;
            vs1[q] = same ? velo : 0u;
            uint32_t elo_e[EPV], wq = 0, zq = 0;
            if (same) {
#pragma unroll
                for (int e = 0; e < EPV; e++) elo_e[e] = velo;
            } else {
                float A = vpre[q], L = vmx[q];
#pragma unroll
                for (int e = 0; e < EPV; e++) {
                    const float v = ev[q][e];
                    const float lo = fmaxf(A * (1.0f - QEPS), L);
                    const float An = A + v;
                    const float hi = An * (1.0f + QEPS);
                    const uint32_t elo = max(__float_as_uint(lo) >> 23, 1u), ehi = max(__float_as_uint(hi) >> 23, 1u);
                    elo_e[e] = elo;
                    wq |= elo != ehi ? 1u << e : 0u;
                    A = An;
                    L = fmaxf(L, term_lb(x[q][e], v, xmax, M));
                }
            }
            // the units; a vector whose largest term is below a quarter unit adds nothing
            const bool negl = same & (__builtin_ldexpf(vtop[q], -((int32_t)velo - 150)) < 0.25f) &
                              (vtop[q] >= 0x1p-120f);
#pragma unroll
            for (int e = 0; e < EPV; e++) {
                const bool zero = !(x[q][e] > -__builtin_inff());
                zq |= zero ? 1u << e : 0u;
                pk[q][e] = zero ? 0u : (elo_e[e] & 0xFFu);  // (no units: checked at this binade)
            }
            if (!negl) {
#pragma unroll
                for (int e = 0; e < EPV; e++) {
                    bool sure;
                    const uint32_t u = elem_units(x[q][e], elo_e[e], fdiv, C.T, C.rT, M, sure);
                    const bool zero = (zq >> e) & 1u;
                    const bool win = !zero & (((wq >> e) & 1u) | !sure);
                    wq = win ? wq | (1u << e) : wq & ~(1u << e);
                    pk[q][e] = (zero | win) ? 0u : (u << 8) | (elo_e[e] & 0xFFu);
                }
            }
            wm[q] = wq & ~zq;
            zm[q] = zq;
        }
        BFI_TRACE(a, tb, 4);
        // window positions in index order
        uint32_t wpre[QV];
#pragma unroll
        for (int q = 0; q < QV; q++) {
            const uint32_t c = (uint32_t)__popc(wm[q]);
            const uint32_t incl = wave_scan_incl(c, 0u, [](uint32_t u, uint32_t v) { return u + v; });
            if (lane == WAVE - 1) sm.vc[q][w] = incl;
            wpre[q] = incl - c;
        }
        __syncthreads();
        uint32_t nwin;
        {
            uint32_t run = 0;
#pragma unroll
            for (int q = 0; q < QV; q++) {
                uint32_t tot = 0, mine = 0;
#pragma unroll
                for (int ww = 0; ww < NWAVE; ww++) {
                    const uint32_t v = sm.vc[q][ww];
                    mine += ww < w ? v : 0u;
                    tot += v;
                }
                wpre[q] += run + mine;
                run += tot;
            }
            nwin = run;
        }
        uint32_t flags = nwin > (uint32_t)a.qcap ? QF_EXACT : 0u;
        uint32_t bad = 0;
        if (!flags) {
            // the windows' (index, x) into their items (the exact values come below), the run
            // tables cleared
#pragma unroll
            for (int q = 0; q < QV; q++) {
                const uint32_t id0 = c0 + (uint32_t)(q * BLOCK + tid) * EPV;
                uint32_t m = wm[q];
                uint32_t pos = wpre[q];
                while (m) {
                    const int i = __builtin_ctz(m);
                    m &= m - 1u;
                    float xe = x[q][0];
#pragma unroll
                    for (int e = 1; e < EPV; e++) xe = e == i ? x[q][e] : xe;
                    *reinterpret_cast<uint2*>(&items[pos]) = make_uint2(id0 + (uint32_t)i, __float_as_uint(xe));
                    pos++;
                }
            }
            for (uint32_t k = (uint32_t)tid; k <= nwin; k += BLOCK) {
                sm.rq[k] = 0u;
                sm.rhi[k] = 0u;
            }
            __syncthreads();
            BFI_TRACE(a, tb, 5);
            // the runs: run k holds the certain elements with k windows before them; a thread
            // sums its consecutive elements of one run and adds them to the run once (a vector
            // without windows joins the thread's current run whole)
            uint32_t key = 0, acc = 0, klo = 0xFFFFFFFFu, khi = 0u, nflush = 0;
            bool have = false;
#pragma unroll
            for (int q = 0; q < QV; q++) {
                if (wm[q] == 0u) {
                    if (zm[q] == (1u << EPV) - 1u) continue;
                    uint32_t vq = 0, vh = 0, vl = 0xFFu;
#pragma unroll
                    for (int e = 0; e < EPV; e++) {
                        vq += pk[q][e] >> 8;
                        const uint32_t b = pk[q][e] & 0xFFu;
                        vh = max(vh, b);
                        vl = ((zm[q] >> e) & 1u) ? vl : min(vl, b);
                    }
                    const uint32_t k = wpre[q];
                    if (have && k != key) {
                        lds_add(&sm.rq[key], acc);
                        lds_max(&sm.rhi[key], khi);
                        bad |= (acc != 0u && klo != khi) ? 1u : 0u;
                        nflush++;
                        acc = 0;
                        klo = 0xFFFFFFFFu;
                        khi = 0u;
                    }
                    have = true;
                    key = k;
                    acc += vq;
                    klo = min(klo, vl);
                    khi = max(khi, vh);
                    continue;
                }
#pragma unroll
                for (int e = 0; e < EPV; e++) {
                    if (((wm[q] | zm[q]) >> e) & 1u) continue;
                    const uint32_t k = wpre[q] + (uint32_t)__popc(wm[q] & ((1u << e) - 1u));
                    if (have && k != key) {
                        lds_add(&sm.rq[key], acc);
                        lds_max(&sm.rhi[key], khi);
                        bad |= (acc != 0u && klo != khi) ? 1u : 0u;
                        nflush++;
                        acc = 0;
                        klo = 0xFFFFFFFFu;
                        khi = 0u;
                    }
                    have = true;
                    key = k;
                    acc += pk[q][e] >> 8;
                    const uint32_t b = pk[q][e] & 0xFFu;
                    klo = min(klo, b);
                    khi = max(khi, b);
                }
            }
            // (the elements of a run all lie in one binade; a thread checks its own part)
            bad |= (have && acc != 0u && klo != khi) ? 1u : 0u;
            // most waves hold one run: one atomic per wave
            const uint64_t hb = __ballot(have);
            const int ld = hb ? __ffsll((unsigned long long)hb) - 1 : 0;
            const uint32_t k0 = (uint32_t)__builtin_amdgcn_readlane((int)key, ld);
            const bool one = __ballot(have && (nflush != 0 || key != k0)) == 0ull;
            if (one) {
                if (hb) {
                    const uint32_t s = wave_sum_u(have ? acc : 0u);
                    const uint32_t l = wave_min_u(have ? klo : 0xFFFFFFFFu);
                    const uint32_t h = lane63(
                        wave_scan_incl(have ? khi : 0u, 0u, [](uint32_t u, uint32_t v) { return max(u, v); }));
                    bad |= (s != 0u && l != h) ? 1u : 0u;
                    if (lane == 0) {
                        lds_add(&sm.rq[k0], s);
                        lds_max(&sm.rhi[k0], h);
                    }
                }
            } else if (have) {
                lds_add(&sm.rq[key], acc);
                lds_max(&sm.rhi[key], khi);
            }
            __threadfence_block();
            __syncthreads();
            // the items: the windows' exact values (the whole block, in window order) and the
            // runs before them; then the tail run
            for (uint32_t k = (uint32_t)tid; k <= nwin; k += BLOCK) {
                const uint32_t q = sm.rq[k];
                const uint32_t hi = sm.rhi[k];
                const int32_t ue = hi ? (int32_t)hi - 150 : -(int32_t)UE_BIAS;  // empty: any binade
                QItem it;
                it.id = QI_NONE;
                it.e = 0.0f;
                if (k < nwin) {
                    const uint2 wv = *reinterpret_cast<const uint2*>(&items[k]);
                    it.id = wv.x;
                    it.e = quant_exact(__uint_as_float(wv.y), C.T, C.rT, C.fast_div ? 1 : 0, M);
                }
                it.q = q;
                it.ue = ue;
                items[k] = it;
            }
            const uint32_t wb = __ballot(bad != 0u) ? 1u : 0u;
            if (lane == 0) sm.wb[w] = wb;
            __syncthreads();
#pragma unroll
            for (int ww = 0; ww < NWAVE; ww++) flags |= sm.wb[ww] ? QF_EXACT : 0u;
        }
        if (tid == 0) {
            head->nwin = flags ? 0u : nwin;
            head->flags = flags;
        }
        qflags = flags;
        qn = nwin;
        if (a.trace && tid == 0) a.trace[tb + 6] = nwin;  // diagnostics: windows
    }

    // the candidates of the kept set into the row's list: positions from a block scan, one
    // global count per workgroup
    if (gather) {
        uint32_t tk[QV];
        uint32_t nt = 0;
#pragma unroll
        for (int q = 0; q < QV; q++) {
            tk[q] = 0;
#pragma unroll
            for (int e = 0; e < EPV; e++)
                tk[q] |= (x[q][e] > -__builtin_inff() && __builtin_fmaf(x[q][e], C.rTl, Kc) >= gth) ? 1u << e : 0u;
            nt += (uint32_t)__popc(tk[q]);
        }
        uint32_t tot;
        uint32_t pos = block_excl_scan<uint32_t>(nt, sm.wg, tot);
        if (tot) {
            if (tid == 0) sm.gbase = glb_add(a.rowcnt + row, tot);
            __syncthreads();
            pos += sm.gbase;
            uint64_t* list = a.spill + (int64_t)row * 4 * a.V;
#pragma unroll
            for (int q = 0; q < QV; q++) {
                const uint32_t id0 = c0 + (uint32_t)(q * BLOCK + tid) * EPV;
                uint32_t m = tk[q];
                while (m) {
                    const int i = __builtin_ctz(m);
                    m &= m - 1u;
                    float xe = x[q][0];
#pragma unroll
                    for (int e = 1; e < EPV; e++) xe = e == i ? x[q][e] : xe;
                    if (pos < (uint32_t)a.V) list[pos] = ((uint64_t)(id0 + (uint32_t)i) << 32) | __float_as_uint(xe);
                    pos++;
                }
            }
        }
        BFI_TRACE(a, tb, 7);
    }
    // a row's first chunk starts from 0: its items are walked here, off the row kernel's
    // path, and become one, the exact sum after the chunk (if the walk needs no re-stream)
    if (chunk == 0 && !trivial && qflags == 0u) {
        __threadfence_block();
        __syncthreads();
        if (w == 0) {
            typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
            uint32_t m = 0u;
            int32_t ue = -149;
            const uint32_t n = qn + 1u;
            const uint32_t hit = chain_run(
                [&](uint32_t j) {
                    const u32x4 v = *(const BFI_GLB u32x4*)(items + j);
                    return QItem{v.x, __uint_as_float(v.y), v.z, (int32_t)v.w};
                },
                0u, n, (uint32_t)a.V, m, ue);
            if (hit == n && lane == 0) {
                items[0] = QItem{QI_SET, state_value(m, ue), 0u, -(int32_t)UE_BIAS};
                head->nwin = 0u;
            }
        }
    }
}

// `vec` is the streaming pass's 16-byte vectors per thread at 256 threads (its chunk); this
// pass covers the same chunk with 512 threads.
hipError_t launch_quant(const KArgs& a, int bf16, int vec, hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
    const dim3 grid((unsigned)((int64_t)a.n_rows * a.n_chunks)), block(BLOCK);
#define BFI_LAUNCH(B, QQ) hipExtLaunchKernelGGL((k_quant<B, QQ>), grid, block, 0, stream, start, stop, 0, a)
    if (!bf16) {
        if (vec == 8) BFI_LAUNCH(false, 4);
        else if (vec == 4) BFI_LAUNCH(false, 2);
        else BFI_LAUNCH(false, 1);
    } else {
        if (vec == 4) BFI_LAUNCH(true, 2);
        else BFI_LAUNCH(true, 1);  // vec 2: full; vec 1: half the threads past the chunk's end
    }
#undef BFI_LAUNCH
    return hipGetLastError();
}

}  // namespace bfi
