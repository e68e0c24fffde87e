// smp_quant.hip — the quantizing pass of the gfx950 token sampler (between the streaming pass
// and the row kernel), one 512-thread workgroup per (row, chunk) over the whole GPU.
//
// The reference's normalizer is a sequential f32 sum over the row (sample.rs:381-386). While
// the running sum stays inside one binade [2^k, 2^(k+1)), each addition moves it by a whole
// number of units u = 2^(k-23): RN(e / u) (smp_exact.h). The pass computes every term
// e = expf(fl(x / T) - M) exactly as the reference does (glibc's expf in double precision,
// full rate on CDNA's VALU). From the row maximum M and the approximate normalizer mass
// before this chunk (both from the streaming pass's row finisher), a workgroup predicts the
// running sum before each of its elements, and so the binade each addition lands in. The
// prediction is an interval: the prefix of the exact terms widened by QEPS relative both
// ways (about twice the f32 sum's largest drift from the exact one on the benchmark rows),
// raised to the largest term added so far (the f32 sum never falls below any of its terms).
// An element is "certain" when the interval before its addition and the one after lie in
// one binade; its units are then RN(e / u) at that binade, exactly. The others ("windows":
// near a binade boundary, ties, terms of 2^23 units or more) are listed with their exact e.
// In index order, the certain elements between two windows all lie in one binade (the
// intervals never decrease, so a change of binade needs an interval that straddles the
// boundary: a window), and the pass sums them per gap as a run. The row kernel chains the
// chunks: it adds a run in one step after checking that the actual running sum lies in the
// run's binade and stays there, and walks the windows exactly; a failed check re-streams
// the rest of the chunk exactly, so a wrong prediction costs time, never the result. On the
// way the pass gathers the candidates of the kept set into the row's list.
#include <hip/hip_ext.h>

#define BFI_BLOCK 512
#include "smp_chain.h"
#include "smp_common.h"
#include "smp_exact.h"

namespace bfi {

// Relative width of the running-sum prediction: about twice the largest drift of the f32
// sum from the exact one on the benchmark rows (2^-10.9). A wider margin lists more windows
// (bands near a binade boundary grow with it); a narrower one lets more rows outrun their
// prediction, whose chunks are then streamed exactly (time, never the result).
constexpr float QEPS = 0x1p-10f;
constexpr uint32_t UE_BIAS = 1024u;
constexpr int QVMAX = 4;             // 16-byte vectors per thread
constexpr int NSLOT = QVMAX * NWAVE;  // (vector, wave) slots of a chunk, in index order

// SHARED (the 16-byte, four-vector f32 chunks): the run table takes the history counts' space
// (the counts are read before the first run is), so the workgroup fits 33 KB of LDS and four
// workgroups share a CU; a first chunk's walk then reads its windows' terms from its items.
template <bool SHARED>
struct __align__(16) QuantSmemT {
    uint64_t etab[32];       // glibc's expf table (EXP2_32), per-lane reads from LDS
    union {
        uint32_t hc[CHUNK_MAX / 2];  // history counts of the chunk's ids (two 16-bit halves a word);
                                     // in a row's first chunk, later: the windows' terms (not SHARED)
        uint32_t rq_s[SHARED ? QWIN + 1 : 1];  // SHARED: per run, units
    };
    uint32_t rq_o[SHARED ? 1 : QWIN + 1];      // not SHARED: per run, units
    uint32_t rhi[QWIN + 1];  // per run: its unit exponent + 150 (0: no element)
    float vs[NSLOT];         // per (vector, wave): sum of the terms
    float vm[NSLOT];         // per (vector, wave): largest term (the running sum's lower bound)
    uint32_t vc[NSLOT];      // per (vector, wave): window count
    uint32_t wg[NWAVE];
    uint32_t wb[NWAVE];
    uint32_t gbase;
    __device__ __forceinline__ uint32_t* rq() { return SHARED ? rq_s : rq_o; }
};
static_assert(NSLOT <= WAVE, "one lane per (vector, wave) slot");
static_assert(QWIN <= CHUNK_MAX / 2, "a first chunk's window terms fit the history counts' space");

template <class S> constexpr bool kSharedRq = false;
template <> constexpr bool kSharedRq<QuantSmemT<true>> = true;

__device__ __forceinline__ uint32_t lds_min(uint32_t* p, uint32_t v) {
    return __hip_atomic_fetch_min((BFI_LDS uint32_t*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// The exclusive prefixes (sum and maximum), over the chunk's (vector, wave) slots in index
// order, of the per-slot values vs and vm, at this wave's slot of each vector (wave-uniform).
template <int QV>
__device__ __forceinline__ void slot_prefix(const float* vs, const float* vm, int w, float (&pre)[QV],
                                            float (&pmax)[QV]) {
    const int lane = lane_id();
    const float tv = lane < QV * NWAVE ? vs[lane] : 0.0f;
    const float tm = lane < QV * NWAVE ? vm[lane] : 0.0f;
    const float ts = wave_excl_of_incl(wave_scan_incl(tv, 0.0f, [](float u, float v) { return u + v; }), 0.0f);
    const float tx =
        wave_excl_of_incl(wave_scan_incl(tm, 0.0f, [](float u, float v) { return fmaxf(u, v); }), 0.0f);
#pragma unroll
    for (int q = 0; q < QV; q++) {
        pre[q] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ts), q * NWAVE + w));
        pmax[q] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(tx), q * NWAVE + w));
    }
}

template <bool BF16, int QV, bool FULL, class Smem>
__device__ __forceinline__ void quant_chunk(const KArgs& a, Smem& sm, int row, int chunk, uint32_t c0,
                                            uint32_t c1);

template <bool BF16, int QV>
__global__ __launch_bounds__(BLOCK) __attribute__((amdgpu_waves_per_eu(!BF16 && QV == 4 ? 8 : 6))) void k_quant(
    KArgs a) {  // four workgroups per CU for the four-vector f32 chunks, else three
    using Smem = QuantSmemT<!BF16 && QV == 4>;
    __shared__ Smem sm;
    const uint32_t G = gridDim.x, bid = blockIdx.x;
    const uint32_t nc = (uint32_t)a.n_chunks;
    // each XCD takes a contiguous block [L0, L0 + size) of the (row, chunk) order (its rows'
    // chunks share its L2), and within it the rows' first chunks go first: their workgroups
    // end with the walk of their items, the longest tail of the pass
    const uint32_t q8 = G / 8, r8 = G % 8, xcd = bid % 8, slot = bid / 8;
    const uint32_t L0 = xcd < r8 ? xcd * (q8 + 1) : r8 * (q8 + 1) + (xcd - r8) * q8;
    const uint32_t size = q8 + (xcd < r8 ? 1u : 0u);
    const uint32_t m0 = (L0 + nc - 1) / nc * nc;  // the block's first row start
    const uint32_t n0 = m0 < L0 + size ? (L0 + size - m0 + nc - 1) / nc : 0u;  // row starts in it
    uint32_t logical;
    if (slot < n0) {
        logical = m0 + slot * nc;
    } else {
        const uint32_t t = slot - n0;
        if (t < m0 - L0 || nc == 1u) {
            logical = L0 + t;
        } else {
            const uint32_t t2 = t - (m0 - L0);
            logical = m0 + t2 / (nc - 1u) * nc + 1u + t2 % (nc - 1u);
        }
    }
    const int row = (int)(logical / nc);
    const int chunk = (int)(logical % nc);
    if (row >= a.n_rows) return;
    const uint32_t V = (uint32_t)a.V;
    const uint32_t c0 = (uint32_t)chunk * (uint32_t)a.chunk;
    const uint32_t c1 = min(c0 + (uint32_t)a.chunk, V);
    if (a.vec_ok && c1 - c0 == (uint32_t)(BLOCK * QV * Elem<BF16>::EPV))
        quant_chunk<BF16, QV, true, Smem>(a, sm, row, chunk, c0, c1);
    else
        quant_chunk<BF16, QV, false, Smem>(a, sm, row, chunk, c0, c1);
}

// The terms e = expf(fl(x / T) - M) of a thread's elements, exactly as the reference
// computes them (sample.rs:373-385). MODE 0: T = 1 (x / T = x); 1: Markstein's corrected
// quotient (exact for |x| in [2^-100, 2^100) and T in [2^-20, 2^20]; outside that range of
// x, |x / T| lies below 2^-80, where fl(s - M) = -M for the |M| >= 2^-50 the mode requires,
// or above 2^80 > |M|, where it is negative enough that e is 0, or -inf / NaN for a masked
// element, whose e is 0); 2: IEEE division.
template <int MODE, int QV, int EPV>
__device__ __forceinline__ void exact_terms(const float (&x)[QV][EPV], float (&ev)[QV][EPV], float T, float rT,
                                            float M, const uint64_t* tab) {
#pragma unroll
    for (int q = 0; q < QV; q++)
#pragma unroll
        for (int e = 0; e < EPV; e++) {
            float s;
            if (MODE == 0) {
                s = x[q][e];
            } else if (MODE == 1) {
                const float q0 = x[q][e] * rT;
                const float r0 = __builtin_fmaf(-q0, T, x[q][e]);
                s = __builtin_fmaf(r0, rT, q0);
            } else {
                s = x[q][e] / T;
            }
            ev[q][e] = expf_nonpos(s - M, tab);
            if (e == EPV - 1) __builtin_amdgcn_sched_barrier(0);  // a vector at a time: bounded registers
        }
}

template <bool BF16, int QV, bool FULL, class Smem>
__device__ __forceinline__ void quant_chunk(const KArgs& a, Smem& sm, int row, int chunk, uint32_t c0,
                                            uint32_t c1) {
    constexpr int EPV = Elem<BF16>::EPV;
    static_assert(QV <= QVMAX, "per-vector tables");
    const int tid = threadIdx.x, lane = lane_id();
    const int w = __builtin_amdgcn_readfirstlane(wave_id());
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
    if (tid < 32) sm.etab[tid] = EXP2_32[tid];
    const RowCtx C = make_ctx(a, row);
    if (!C.active) return;
    const float M = ld_uniform(&a.rinfo[row].M);
    if (!quant_row(C, M)) return;
    const float th = ld_uniform(&a.rinfo[row].th);
    const float xm = ld_uniform(&a.parts[rc].xm);
    const float Pc = ld_uniform(&a.qpre[rc].P);
    const float Lc = ld_uniform(&a.qpre[rc].lb);
    QHead* const head = a.qhead + rc;
    QItem* const items = a.qitem + rc * (a.qcap + 1);
    const float Kc = -(M * 1.44269504088896341f);
    // candidates: the row's bound th on (x / T - M) log2(e), less the margin its estimates
    // carry (the roundings of x / T, of M and of the products, in log2-units); an element is
    // a candidate when its exact term reaches 2^gth, lowered once more for exp2's rounding
    const float gth = th - (0x1p-8f + (fabsf(M) * 12.0f + 200.0f) * 0x1p-24f);
    const float egth = gth > -__builtin_inff() ? __builtin_amdgcn_exp2f(gth) * (1.0f - 0x1p-10f) : 0.0f;
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
    }
    __syncthreads();  // (the history counts and the expf table)
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

    // the exact terms, and the candidates among them
    float ev[QV][EPV];
    {
        const float aM = fabsf(M);
        if (C.T == 1.0f) exact_terms<0, QV, EPV>(x, ev, C.T, C.rT, M, sm.etab);
        else if (C.fast_div && aM >= 0x1p-50f && aM < 0x1p80f) exact_terms<1, QV, EPV>(x, ev, C.T, C.rT, M, sm.etab);
        else exact_terms<2, QV, EPV>(x, ev, C.T, C.rT, M, sm.etab);
    }
    uint32_t tk[QV];
    if (egth > 0.0f) {  // (a masked element's term is 0: below the bound)
#pragma unroll
        for (int q = 0; q < QV; q++) {
            tk[q] = 0;
#pragma unroll
            for (int e = 0; e < EPV; e++) tk[q] |= ev[q][e] >= egth ? 1u << e : 0u;
        }
    } else {
#pragma unroll
        for (int q = 0; q < QV; q++) {
            tk[q] = 0;
#pragma unroll
            for (int e = 0; e < EPV; e++) tk[q] |= x[q][e] > -__builtin_inff() ? 1u << e : 0u;
        }
    }

    // the candidates' positions in the row's list: a block scan and one global count per
    // workgroup, issued now (its value is first needed at the end)
    uint32_t gpos = 0, gtot = 0, gbase = 0;
    if (gather) {
        uint32_t nt = 0;
#pragma unroll
        for (int q = 0; q < QV; q++) nt += (uint32_t)__popc(tk[q]);
        gpos = block_excl_scan<uint32_t>(nt, sm.wg, gtot);
        if (gtot && tid == 0) gbase = glb_add(a.rowcnt + row, gtot);
    }

    uint32_t qflags = QF_EXACT, qn = 0;  // this chunk's summary (for the first chunk's walk below)
    if (!trivial) {
        // the prediction: prefix sums of the terms (index order: vector, thread, element) from
        // the row's values at the chunk's start, and a lower bound: 1 once a term equal to 1
        // (the row maximum's, exp(0)) has been added (the element walk below also raises it
        // to each term it passes)
        float vpre[QV], vmx[QV], vsum[QV];
#pragma unroll
        for (int q = 0; q < QV; q++) {
            float g = 0.0f;
            bool one = false;
#pragma unroll
            for (int e = 0; e < EPV; e++) {
                g += ev[q][e];
                one = one || ev[q][e] == 1.0f;
            }
            vsum[q] = g;
            const float incl = wave_scan_incl(g, 0.0f, [](float u, float v) { return u + v; });
            const uint64_t ob = __ballot(one);
            if (lane == WAVE - 1) {
                sm.vs[q * NWAVE + w] = incl;
                sm.vm[q * NWAVE + w] = ob ? 1.0f : 0.0f;
            }
            vpre[q] = wave_excl_of_incl(incl, 0.0f);
            vmx[q] = (ob & lanes_below()) ? 1.0f : 0.0f;
        }
        __syncthreads();
        {
            float spre[QV], smax[QV];
            slot_prefix<QV>(sm.vs, sm.vm, w, spre, smax);
#pragma unroll
            for (int q = 0; q < QV; q++) {
                vpre[q] += Pc + spre[q];
                vmx[q] = fmaxf(vmx[q], fmaxf(Lc, smax[q]));
            }
        }
        BFI_TRACE(a, tb, 3);
        // classify and quantize: window bits (the interval straddles a binade boundary, a tie
        // of RN, or 2^23 units or more: the chain adds these exactly) and zero bits (e = 0:
        // nothing at any binade). The running sums below 2^-125 (the subnormals and the
        // lowest normal binade) share one spacing, 2^-149: one binade. A certain element's
        // units are recomputed from e where the runs are summed; each keeps its binade
        // (ue + 150) in a byte of eb.
        static_assert(QV * EPV <= 32, "one bit per element of a thread");
        constexpr int EBW = (EPV + 3) / 4;  // words of packed binades per vector
        uint32_t wmask = 0, zmask = 0;      // window and zero bits: bit q * EPV + e
        uint32_t eb[QV][EBW];
        uint32_t vqs[QV];                   // per vector: its units, 2^23 + RN(t) each
        uint32_t fbits = 0;                 // bit q: vector q lies in one binade
#pragma unroll
        for (int q = 0; q < QV; q++) {
            // the vector as a whole: the interval from before its first element to after its
            // last one; in one binade, no element of it can straddle a boundary
            const float vlo = fmaxf(vpre[q] * (1.0f - QEPS), vmx[q]);
            const float vhi = (vpre[q] + vsum[q]) * (1.0f + QEPS);
            const uint32_t velo = max(__float_as_uint(vlo) >> 23, 1u), vehi = max(__float_as_uint(vhi) >> 23, 1u);
            uint32_t wq = 0, zq = 0, vq = 0;
            // t + 2^23 rounds t to an integer (ties to even) in the low mantissa bits, for t
            // below 2^23 (larger t is a window, whose units are not used)
            if (velo == vehi) {  // one binade for the whole vector: only ties and large terms
                const int32_t k = 150 - (int32_t)velo;
#pragma unroll
                for (int e = 0; e < EPV; e++) {
                    const float t = __builtin_ldexpf(ev[q][e], k);
                    const float y = t + 8388608.0f;
                    const float qf = y - 8388608.0f;
                    // (a zero term gives t = 0: neither)
                    wq |= ((fabsf(t - qf) == 0.5f) | !(t < 8388608.0f)) ? 1u << e : 0u;
                    zq |= !(ev[q][e] > 0.0f) ? 1u << e : 0u;
                    vq += __float_as_uint(y);
                }
                fbits |= 1u << q;
#pragma unroll
                for (int i = 0; i < EBW; i++) eb[q][i] = (velo & 0xFFu) * 0x01010101u;
            } else {
                uint32_t elo_e[EPV];
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
                    L = fmaxf(L, v);
                }
#pragma unroll
                for (int e = 0; e < EPV; e++) {
                    const bool zero = !(ev[q][e] > 0.0f);
                    const float t = __builtin_ldexpf(ev[q][e], 150 - (int32_t)elo_e[e]);
                    const float y = t + 8388608.0f;
                    const float qf = y - 8388608.0f;
                    const bool win = !zero & (((wq >> e) & 1u) | (fabsf(t - qf) == 0.5f) | !(t < 8388608.0f));
                    zq |= zero ? 1u << e : 0u;
                    wq = win ? wq | (1u << e) : wq & ~(1u << e);
                    vq += __float_as_uint(y);
                }
#pragma unroll
                for (int i = 0; i < EBW; i++) {
                    uint32_t wd = 0;
#pragma unroll
                    for (int e = 4 * i; e < EPV && e < 4 * i + 4; e++) wd |= (elo_e[e] & 0xFFu) << (8 * (e - 4 * i));
                    eb[q][i] = wd;
                }
            }
            vqs[q] = vq - (uint32_t)EPV * 0x4B000000u;
            wmask |= wq << (q * EPV);
            zmask |= zq << (q * EPV);
        }
        // an element's binade and units (certain elements)
        auto elo_of = [&](int q, int e) { return (eb[q][e >> 2] >> (8 * (e & 3))) & 0xFFu; };
        auto units_at = [&](int q, int e, uint32_t elo) {
            return (uint32_t)__builtin_rintf(__builtin_ldexpf(ev[q][e], 150 - (int32_t)elo));
        };
        BFI_TRACE(a, tb, 4);
        // window positions in index order
        uint32_t wpre[QV];
        if (__ballot(wmask != 0u)) {
#pragma unroll
            for (int q = 0; q < QV; q++) {
                const uint32_t c = (uint32_t)__popc((wmask >> (q * EPV)) & em);
                const uint32_t incl = wave_scan_incl(c, 0u, [](uint32_t u, uint32_t v) { return u + v; });
                if (lane == WAVE - 1) sm.vc[q * NWAVE + w] = incl;
                wpre[q] = incl - c;
            }
        } else {  // (most waves: no window)
#pragma unroll
            for (int q = 0; q < QV; q++) wpre[q] = 0u;
            if (lane < QV) sm.vc[lane * NWAVE + w] = 0u;
        }
        __syncthreads();
        uint32_t nwin;
        {
            const uint32_t tv = lane < QV * NWAVE ? sm.vc[lane] : 0u;
            const uint32_t ti = wave_scan_incl(tv, 0u, [](uint32_t u, uint32_t v) { return u + v; });
            const uint32_t te = ti - tv;
            nwin = (uint32_t)__builtin_amdgcn_readlane((int)ti, QV * NWAVE - 1);
#pragma unroll
            for (int q = 0; q < QV; q++) wpre[q] += (uint32_t)__builtin_amdgcn_readlane((int)te, q * NWAVE + w);
        }
        uint32_t flags = nwin > (uint32_t)a.qcap ? QF_EXACT : 0u;
        uint32_t bad = 0;
        if (!flags) {
            // the windows' (index, e) into their items, the run tables cleared
#pragma unroll
            for (int q = 0; q < QV; q++) {
                const uint32_t id0 = c0 + (uint32_t)(q * BLOCK + tid) * EPV;
                uint32_t m = (wmask >> (q * EPV)) & em;
                uint32_t pos = wpre[q];
                while (m) {
                    const int i = __builtin_ctz(m);
                    m &= m - 1u;
                    float ee = ev[q][0];
#pragma unroll
                    for (int e = 1; e < EPV; e++) ee = e == i ? ev[q][e] : ee;
                    *reinterpret_cast<uint2*>(&items[pos]) = make_uint2(id0 + (uint32_t)i, __float_as_uint(ee));
                    if (!kSharedRq<Smem> && chunk == 0) sm.hc[pos] = __float_as_uint(ee);  // (for the walk below)
                    pos++;
                }
            }
            for (uint32_t k = (uint32_t)tid; k <= nwin; k += BLOCK) {
                sm.rq()[k] = 0u;
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
                const uint32_t wmq = (wmask >> (q * EPV)) & em, zmq = (zmask >> (q * EPV)) & em;
                if (wmq == 0u) {
                    if (zmq == em) continue;
                    // (a vector without windows: its units were summed where it was classified;
                    // in one binade, that binade, else its nonzero elements' lowest and highest)
                    const uint32_t vq = vqs[q];
                    uint32_t vh = eb[q][0] & 0xFFu, vl = vh;
                    if (!((fbits >> q) & 1u)) {
                        vh = 0;
                        vl = 0xFFu;
#pragma unroll
                        for (int e = 0; e < EPV; e++) {
                            const bool z = (zmq >> e) & 1u;
                            const uint32_t b = elo_of(q, e);
                            vh = z ? vh : max(vh, b);
                            vl = z ? vl : min(vl, b);
                        }
                    }
                    const uint32_t k = wpre[q];
                    if (have && k != key) {
                        lds_add(&sm.rq()[key], acc);
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
                    if (((wmq | zmq) >> e) & 1u) continue;
                    const uint32_t k = wpre[q] + (uint32_t)__popc(wmq & ((1u << e) - 1u));
                    if (have && k != key) {
                        lds_add(&sm.rq()[key], acc);
                        lds_max(&sm.rhi[key], khi);
                        bad |= (acc != 0u && klo != khi) ? 1u : 0u;
                        nflush++;
                        acc = 0;
                        klo = 0xFFFFFFFFu;
                        khi = 0u;
                    }
                    have = true;
                    key = k;
                    const uint32_t b = elo_of(q, e);
                    acc += units_at(q, e, b);
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
                        lds_add(&sm.rq()[k0], s);
                        lds_max(&sm.rhi[k0], h);
                    }
                }
            } else if (have) {
                lds_add(&sm.rq()[key], acc);
                lds_max(&sm.rhi[key], khi);
            }
            __threadfence_block();
            __syncthreads();
            // the items' runs (the window halves are written): the run before each window
            // element, then the tail run
            for (uint32_t k = (uint32_t)tid; k <= nwin; k += BLOCK) {
                const uint32_t q = sm.rq()[k];
                const uint32_t hi = sm.rhi[k];
                const int32_t ue = hi ? (int32_t)hi - 150 : -(int32_t)UE_BIAS;  // empty: any binade
                if (k < nwin) *reinterpret_cast<uint2*>(&items[k].q) = make_uint2(q, (uint32_t)ue);
                else items[k] = QItem{QI_NONE, 0.0f, q, ue};
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
    }

    // the candidates of the kept set into the row's list, as (id, e)
    if (gather) {
        if (gtot) {
            if (tid == 0) sm.gbase = gbase;
            __syncthreads();
            uint32_t pos = gpos + sm.gbase;
            uint64_t* list = a.spill + (int64_t)row * 4 * a.V;
#pragma unroll
            for (int q = 0; q < QV; q++) {
                const uint32_t id0 = c0 + (uint32_t)(q * BLOCK + tid) * EPV;
                uint32_t m = tk[q];
                while (m) {
                    const int i = __builtin_ctz(m);
                    m &= m - 1u;
                    float ee = ev[q][0];
#pragma unroll
                    for (int e = 1; e < EPV; e++) ee = e == i ? ev[q][e] : ee;
                    if (pos < (uint32_t)a.V) list[pos] = ((uint64_t)(id0 + (uint32_t)i) << 32) | __float_as_uint(ee);
                    pos++;
                }
            }
        }
        BFI_TRACE(a, tb, 7);
    }
    // a row's first chunk starts from 0: its items are walked here, off the row kernel's
    // path, and become one, the exact sum after the chunk (if the walk needs no re-stream)
    uint64_t tsync = 0;  // diagnostics
    if (chunk == 0 && !trivial && qflags == 0u) {
        __threadfence_block();
        __syncthreads();
        if (a.trace && tid == 0) tsync = wall_clock64() - a.trace[tb];
        if (w == 0) {
            uint32_t m = 0u;
            int32_t ue = -149;
            const uint32_t n = qn + 1u;
            // the items from LDS: the runs' tables and the windows' terms (the history
            // counts' space); an element's index only has to be below V here
            const uint32_t hit = chain_run(
                [&](uint32_t j) {
                    const uint32_t hi = sm.rhi[j];
                    const bool el = j < qn;
                    const float ej = kSharedRq<Smem> ? *(const BFI_GLB float*)&items[j].e : __uint_as_float(sm.hc[j]);
                return QItem{el ? 0u : QI_NONE, el ? ej : 0.0f, sm.rq()[j],
                                 hi ? (int32_t)hi - 150 : -(int32_t)UE_BIAS};
                },
                0u, n, (uint32_t)a.V, m, ue);
            if (hit == n && lane == 0) {
                items[0] = QItem{QI_SET, state_value(m, ue), 0u, -(int32_t)UE_BIAS};
                head->nwin = 0u;
            }
        }
    }
    // diagnostics: the windows (bits 0-19), and the times from the start stamp to the first
    // chunk's walk (bits 20-41) and to here (bits 42-63)
    if (a.trace && tid == 0)
        a.trace[tb + 6] = (uint64_t)qn | ((tsync & 0x3FFFFFull) << 20) | (((wall_clock64() - a.trace[tb]) & 0x3FFFFFull) << 42);
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
