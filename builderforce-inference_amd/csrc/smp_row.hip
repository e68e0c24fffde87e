// smp_row.hip — the row pass of the gfx950 token sampler: one workgroup of 512 threads
// per row finishes `target()` and `draw()` (sample.rs:326-427, 312-323) or `judge()`
// (spec.rs:79-97) with the reference's own f32 results.
//
// After the streaming pass (smp_stream.hip) has found each chunk's maximum, this kernel
//   1. forms the row maximum M (sample.rs:377-379) and, for greedy rows, the argmax
//      (sample.rs:369-371, 429-439);
//   2. streams the row once more (from the caches, where the streaming pass left it) and
//      computes the normalizer S = sum of exp(s - M) exactly as the reference's sequential
//      f32 loop rounds it (sample.rs:381-386), by binade-quantized prefix sums with the
//      rare events done as real f32 additions (smp_exact.h); on the way it gathers the
//      candidates of the kept set (elements above a bound that top-k, top-p or min-p
//      guarantees the kept set lies above) into LDS;
//   3. gives each candidate its exact probability fl(expf(s - M) / S) and its reference
//      order key (descending p, then ascending index: the stable sort of sample.rs:393,398);
//   4. walks the candidates in that order by value buckets (a counting sort, no full sort):
//      whole buckets are added as quantized sums, and only a bucket in which an event lies
//      (a binade crossing, a tie, the top-p cut, the drawn position) is sorted and walked
//      element by element. The walks give the top-p cut (sample.rs:397-409), the kept sum
//      and the drawn token (sample.rs:312-323), or the judge's verdict and residual draw.
// Rows without top-k / top-p draw in index order; without any filter they stream the row
// twice more for the draw (sum, then the position).
#include <hip/hip_ext.h>

#define BFI_BLOCK 512
#include "smp_chain.h"
#include "smp_common.h"
#include "smp_exact.h"

namespace bfi {

constexpr int LCAP = 8192;   // candidates held in LDS (beyond: the row's global spill area)
constexpr int NB = 1024;     // value buckets of a walk
constexpr int SORTCAP = 1024;  // candidate lists up to this size are sorted outright
constexpr int RNV_F32 = 4;   // 16-byte vectors per thread per step of a row stream (f32)
constexpr int RNV_BF16 = 2;  // (bf16)

struct __align__(16) RowSmem {
    uint64_t list[LCAP];   // gathered candidates (id << 32 | bits(x)), then keys, then scratch
    uint64_t grp[LCAP];    // the keys grouped by bucket
    uint32_t bcnt[NB];     // per bucket: element count
    uint32_t boff[NB];     // per bucket: first position in grp
    uint32_t bfill[NB];    // per bucket: fill counter, then scratch
    uint32_t bsm[NB];      // per bucket: a walk's running sum before it, in units (recorded walks)
    uint32_t bsx[NB];      //   and (rank << 10 | unit exponent + 512); 0: not recorded
    uint32_t bq[NB];       // per bucket: units its keys add at the predicted binade (bucket_units)
    uint32_t bk[NB];       //   and that binade's unit exponent + 512 (0: none; bit 31: a tie of RN)
    uint64_t pq_excl;      // the key bq leaves out
    uint32_t pq_ok;        // bq/bk hold the current list's prediction
    uint32_t coff[NCMAX + 1];  // the chain: first item of each chunk
    uint32_t cflag[NCMAX];     //   and its flags
    uint32_t wu[NWAVE];
    uint32_t wu2[NWAVE];
    float wf[NWAVE];
    double wd[NWAVE];
    uint64_t w64[NWAVE];
    uint32_t misc[16];
    float mf[16];
};

__shared__ RowSmem g_sm;  // the row kernel's LDS

enum {
    MS_N = 0, MS_STOP = 1, MS_STOPLO = 2, MS_FLAG = 3, MS_TOK = 4, MS_VERDICT = 5, MS_KIND = 6, MS_LAST = 7,
    MS_NV = 8, MS_CLO = 9, MS_CHI = 10, MS_CNEXT = 11, MS_NFB = 12
};
enum { MF_S = 0, MF_CUM = 1 };

// ---- row-wide history tables (global workspace) ---------------------------------------
//
// The reference's `HashSet(prev)` (sample.rs:347, 361) as a bitmap over the vocabulary,
// plus the multiset counts of the frequency extension as dense counts over the set ids
// (rank of an id = popcount prefix of the bitmap). Built once per row per launch.

struct HistTabs {
    const uint32_t* bm;
    const uint32_t* pre;
    const uint32_t* cnt;
    bool dense;  // counts are in cnt (else, more than GDCAP distinct ids: scanned)
};

__device__ __noinline__ HistTabs hist_tabs(uint32_t* bm, int32_t nw, uint32_t V, HistView h, int32_t freq_on) {
    RowSmem& sm = g_sm;
    const int tid = threadIdx.x;
    uint32_t* pre = bm + nw;
    uint32_t* cnt = pre + nw;
    for (int w = tid; w < nw; w += BLOCK) bm[w] = 0u;
    if (freq_on)
        for (int w = tid; w < GDCAP; w += BLOCK) cnt[w] = 0u;
    __threadfence();
    __syncthreads();
    const int64_t H = h.size();
    for (int64_t j = tid; j < H; j += BLOCK) {
        const uint32_t id = h.at(j);
        if (id < V) glb_or(&bm[id >> 5], 1u << (id & 31));
    }
    __threadfence();
    __syncthreads();
    bool dense = false;
    if (freq_on) {
        const int per = (nw + BLOCK - 1) / BLOCK;
        const int w0 = tid * per;
        uint32_t s = 0;
        for (int w = w0; w < w0 + per && w < nw; w++) s += __popc(bm[w]);
        uint32_t tot;
        uint32_t run = block_excl_scan<uint32_t>(s, sm.wu, tot);
        for (int w = w0; w < w0 + per && w < nw; w++) {
            pre[w] = run;
            run += __popc(bm[w]);
        }
        dense = tot <= (uint32_t)GDCAP;
        __threadfence();
        __syncthreads();
        if (dense) {
            for (int64_t j = tid; j < H; j += BLOCK) {
                const uint32_t id = h.at(j);
                if (id < V) glb_add(&cnt[dense_rank(pre[id >> 5], bm[id >> 5], id & 31)], 1u);
            }
        }
        __threadfence();
        __syncthreads();
    }
    HistTabs T;
    T.bm = bm;
    T.pre = pre;
    T.cnt = cnt;
    T.dense = dense;
    return T;
}
__device__ __forceinline__ HistTabs build_hist_tabs(const KArgs& a, RowSmem& sm, const RowCtx& C) {
    (void)sm;
    if (!C.pen_on) return HistTabs{nullptr, nullptr, nullptr, false};
    return hist_tabs(a.row_pen + (int64_t)C.row * (2 * (int64_t)a.bm_words + GDCAP), a.bm_words, (uint32_t)a.V, C.h,
                     C.pen.freq_on ? 1 : 0);
}

// Occurrences of history id `id` (the frequency extension's count).
__device__ __forceinline__ uint32_t hist_count(const HistTabs& T, const RowCtx& C, uint32_t id) {
    if (!C.pen.freq_on) return 1u;
    if (T.dense) return T.cnt[dense_rank(T.pre[id >> 5], T.bm[id >> 5], id & 31)];
    return C.h.count_scan(id);
}

// The masked, penalized logit of element id (sample.rs:331-367) from its raw logit.
__device__ __forceinline__ float pen_logit(const HistTabs& T, const RowCtx& C, uint32_t id, float l, bool allowed,
                                           bool in_hist) {
    float x = allowed ? l : -__builtin_inff();
    if (in_hist) x = penalize(x, hist_count(T, C, id), C.pen);
    return x;
}

// Raw logit of element id (one scalar or vector load).
template <bool BF16>
__device__ __forceinline__ float load_logit(const KArgs& a, int row, uint32_t id) {
    if (BF16)
        return __uint_as_float((uint32_t)((const uint16_t*)a.logits)[(int64_t)row * a.row_stride + id] << 16);
    return ((const float*)a.logits)[(int64_t)row * a.row_stride + id];
}
template <bool BF16>
__device__ __forceinline__ float elem_x(const KArgs& a, const HistTabs& T, const RowCtx& C, uint32_t id) {
    const float l = load_logit<BF16>(a, C.row, id);
    const bool allowed = !C.mrow || ((C.mrow[id >> 5] >> (id & 31)) & 1u);
    const bool inh = C.pen_on && ((T.bm[id >> 5] >> (id & 31)) & 1u);
    return pen_logit(T, C, id, l, allowed, inh);
}

// fl(e / S), correctly rounded (a double quotient of two floats rounds to the float
// quotient: 53 >= 2 * 24 + 2).
__device__ __forceinline__ float exact_p(float e, float S) { return (float)((double)e / (double)S); }

// ---- block helpers for 1024 threads ----------------------------------------------------

__device__ __forceinline__ uint32_t wave_sum_sat(uint32_t v) {
    return lane63(wave_scan_incl(v, 0u, [](uint32_t x, uint32_t y) { return sat_add(x, y); }));
}
__device__ __forceinline__ uint32_t wave_scan_sat(uint32_t v) {
    return wave_scan_incl(v, 0u, [](uint32_t x, uint32_t y) { return sat_add(x, y); });
}
// Saturating block sum and an OR of flags in one barrier pair.
__device__ __forceinline__ uint32_t block_sum_sat_or(uint32_t v, uint32_t f, uint32_t& fo, RowSmem& sm) {
    v = wave_sum_sat(v);
    const uint32_t fw = __ballot(f != 0u) ? 1u : 0u;
    if (lane_id() == 0) {
        sm.wu[wave_id()] = v;
        sm.wu2[wave_id()] = fw;
    }
    __syncthreads();
    uint32_t r = 0, ro = 0;
#pragma unroll
    for (int w = 0; w < NWAVE; w++) {
        r = sat_add(r, sm.wu[w]);
        ro |= sm.wu2[w];
    }
    __syncthreads();
    fo = ro;
    return r;
}
// Exclusive saturating block scan (thread order); `total` receives the block sum.
__device__ __forceinline__ uint32_t block_excl_scan_sat(uint32_t v, uint32_t& total, RowSmem& sm) {
    const uint32_t x = wave_scan_sat(v);
    if (lane_id() == WAVE - 1) sm.wu[wave_id()] = x;
    __syncthreads();
    uint32_t pre = 0, tot = 0;
#pragma unroll
    for (int w = 0; w < NWAVE; w++) {
        const uint32_t s = sm.wu[w];
        if (w < wave_id()) pre = sat_add(pre, s);
        tot = sat_add(tot, s);
    }
    __syncthreads();
    total = tot;
    // the in-wave exclusive prefix is the previous lane's inclusive one (a subtraction
    // would be wrong once the sum saturates)
    const uint32_t up = (uint32_t)__shfl_up((int)x, 1);
    const uint32_t ex = lane_id() == 0 ? 0u : up;
    return sat_add(pre, ex);
}

}  // namespace bfi

namespace bfi {

// ---- row streams: sequential f32 sums over the row in index order ------------------------
//
// A stream walks the row in index order and sums v_i from 0 exactly as the reference's
// sequential f32 loop does: v_i = e_i = expf(s_i - M) (the normalizer, sample.rs:381-386) or
// v_i = p_i = fl(e_i / S) (the draw over an unfiltered row, sample.rs:313-321). Per element
// a hardware exp2 estimate of t = v / u (u = the spacing of the running sum's binade)
// rounds to the exact unit count unless the estimate lies too close to a rounding
// boundary; those few elements get the exact value (glibc expf, exact division). Options:
// a threshold th (stop at the first i whose running sum reaches th: sample.rs:318), an
// excluded index (spec.rs:89: the residual without the draft), and gathering of elements
// whose d * log2(e) (d = s - M, estimated) is at least gth into the candidate list.
//
// A stream is one out-of-line function (its arguments by value, in its own registers), so
// the kernel's code holds one copy of the loop whatever the number of streams a row needs.


struct StreamArgs {
    const void* logits;     // the row's first logit
    const uint32_t* mrow;   // allow-mask row, or null
    const uint32_t* hbm;    // history bitmap, or null (no penalties)
    const uint32_t* hpre;   // its popcount prefix and dense counts (frequency extension)
    const uint32_t* hcnt;
    const uint32_t* hbase;  // the history itself (counts beyond the dense table)
    const uint32_t* hext;
    int64_t hnb, hnx;
    uint64_t* spill;        // the row's spill area (its candidate list)
    uint64_t* trace;        // the row's 16 diagnostic words, or null
    uint32_t V;
    uint32_t lo, hi;        // the element range streamed
    float s0;               // the running sum before element lo
    int32_t vec_ok, hdense, fast_div;
    float T, rT, rTl;
    float rp, pp, fp;
    int32_t rep_on, pres_on, freq_on;
    float M, S, th;
    int64_t excl;           // excluded index (-1: none)
    int32_t kind;           // 0: e, 1: p
    int32_t gather;
    float gth;              // gather bound on d * log2(e)
};
struct StreamOut {
    float cum;     // the sum at the stop (or over the whole row)
    int64_t stop;  // the index where the running sum first reached th, or -1
};

// Global-memory views of the stream's pointers (they arrive in a by-value struct, where the
// compiler no longer sees that they point to global memory: generic loads would also count
// against the LDS counter, so every LDS wait would wait for the logits in flight).
template <typename T>
__device__ __forceinline__ const BFI_GLB T* gl(const T* p) {
    return (const BFI_GLB T*)p;
}
template <typename T>
__device__ __forceinline__ BFI_GLB T* gl(T* p) {
    return (BFI_GLB T*)p;
}

// The exact value of a finite masked, penalized logit x: e = expf(fl(fl(x / T) - M))
// (sample.rs:374, 383), or p = fl(e / S) (sample.rs:388). Out of line: rare, and its code
// (an f64 division, glibc's expf) should exist once.
__device__ __forceinline__ float exact_value(float x, float T, float rT, int32_t fast_div, float M, float S,
                                          int32_t kind) {
    float s;
    if (fast_div) {
        const uint32_t ax = __float_as_uint(x) & 0x7FFFFFFFu;
        const bool ok = !((ax - 1u < 0x0D7FFFFFu) || (ax - 0x71800000u < 0x0E000000u));
        if (ok) {
            const float q = x * rT;
            const float er = __builtin_fmaf(-q, T, x);
            s = er != er ? q : __builtin_fmaf(er, rT, q);
        } else {
            s = x / T;
        }
    } else {
        s = x / T;
    }
    const float e = expf_ref(s - M);
    return kind ? exact_p(e, S) : e;
}

__device__ __forceinline__ uint32_t sa_count(const StreamArgs& A, uint32_t id) {
    if (!A.freq_on) return 1u;
    if (A.hdense) return gl(A.hcnt)[dense_rank(gl(A.hpre)[id >> 5], gl(A.hbm)[id >> 5], id & 31)];
    uint32_t c = 0;
    for (int64_t j = 0; j < A.hnb; j++) c += gl(A.hbase)[j] == id;
    for (int64_t j = 0; j < A.hnx; j++) c += gl(A.hext)[j] == id;
    return c;
}
__device__ __forceinline__ float sa_penalize(const StreamArgs& A, float x, uint32_t id) {
    Pen P;
    P.rp = A.rp;
    P.pp = A.pp;
    P.fp = A.fp;
    P.rep_on = A.rep_on;
    P.pres_on = A.pres_on;
    P.freq_on = A.freq_on;
    return penalize(x, sa_count(A, id), P);
}

// The estimate of t = v / u for an element: the exact s = fl(x / T) (Markstein's corrected
// quotient, exact for |x| in [2^-100, 2^100) and T in [2^-20, 2^20]) and the exact
// d = fl(s - M) the reference computes, then exp(d) = 2^(h + l) with h = fl(d log2(e)) and
// l its rounding error plus log2(e)'s own (both exact by FMA), as exp2(h) (1 + l ln 2).
// Its relative error against glibc's expf(d) is the hardware exp2's (about an ulp) plus
// expf's half ulp and the correction's rounding; RHO (2^-19, 16 ulps) bounds it with a wide
// margin (kind 1 adds fl(1/S) and the product's roundings, and the reference's division's).
// Elements whose estimate lies within RHO of a rounding boundary, and the few the estimate
// does not cover (|x| outside the quotient's range, exp2 below the normal range while the
// running sum is still subnormal), take the exact value.
constexpr float RHO0 = 0x1p-19f;
constexpr float RHO1 = 0x1p-19f + 0x1p-21f;
constexpr float L2E_HI = 1.44269502162933349609375f;      // fl(log2(e))
constexpr float L2E_LO = 1.925963033500011079e-8f;        // log2(e) - L2E_HI
constexpr float LN2_F = 0.693147180559945309f;

struct StreamState {
    uint32_t m;
    int32_t ue;
    uint32_t tu;  // threshold in units (0xFFFFFFFF: none)
};
__device__ __forceinline__ StreamState stream_state(float s, const StreamArgs& A) {
    const SumState ss = sum_state(s);
    StreamState st;
    st.m = ss.m;
    st.ue = ss.ue;
    st.tu = A.th < __builtin_inff() ? thresh_units(fmaxf(A.th, 0.0f), ss.ue) : 0xFFFFFFFFu;
    return st;
}

// Unit estimate of element x at the state: returns RN(t) when certain (amb false), else
// amb = true (the caller takes the exact value). h receives d log2(e) (the gather test).
__device__ __forceinline__ uint32_t stream_est(const StreamArgs& A, const StreamState& st, float rS, float x,
                                               float& h_out, bool& amb) {
    if (!(x > -__builtin_inff())) {  // masked: exp(-inf) = 0 exactly
        h_out = -__builtin_inff();
        amb = false;
        return 0u;
    }
    const uint32_t ax = __float_as_uint(x) & 0x7FFFFFFFu;
    const bool ok = A.fast_div && !((ax - 1u < 0x0D7FFFFFu) || (ax - 0x71800000u < 0x0E000000u));
    const float q0 = x * A.rT;
    const float r0 = __builtin_fmaf(-q0, A.T, x);
    const float sx = __builtin_fmaf(r0, A.rT, q0);
    const float d = sx - A.M;
    const float h = d * L2E_HI;
    const float l = __builtin_fmaf(d, L2E_LO, __builtin_fmaf(d, L2E_HI, -h));
    h_out = h;
    const float e0 = __builtin_amdgcn_exp2f(h);
    float ev = __builtin_fmaf(e0, l * LN2_F, e0);
    if (A.kind) ev *= rS;
    const float t = __builtin_ldexpf(ev, -st.ue);
    const float qf = __builtin_rintf(t);
    const float f = fabsf(t - qf);
    amb = !ok || (h < -125.0f && st.ue < -125) || !(__builtin_fmaf(t, A.kind ? RHO1 : RHO0, f) < 0.5f) ||
          !(t < 8388608.0f);
    return amb ? 0u : (uint32_t)qf;
}

// The exact unit count of element x at the state (tie: its rounding depends on the running
// sum's parity, an event).
__device__ __forceinline__ uint32_t stream_exact_units(const StreamArgs& A, const StreamState& st, float x,
                                                       bool& tie) {
    const float t = units_of(exact_value(x, A.T, A.rT, A.fast_div, A.M, A.S, A.kind), st.ue);
    tie = quant_tie(t);
    return quant_units(t);
}

// Unit counts of one vector's EPV elements: estimates, then the uncertain ones exactly (a
// short loop, rarely entered).
template <int EPV>
__device__ __forceinline__ void vector_units(const StreamArgs& A, const StreamState& st, float rS,
                                             const float (&x)[EPV], uint32_t (&u)[EPV], uint32_t& tiem,
                                             float (&h)[EPV], uint32_t& nex) {
    uint32_t am = 0;
#pragma unroll
    for (int e = 0; e < EPV; e++) {
        bool amb;
        u[e] = stream_est(A, st, rS, x[e], h[e], amb);
        am |= amb ? (1u << e) : 0u;
    }
    tiem = 0;
    while (am) {
        const int i = __builtin_ctz(am);
        am &= am - 1u;
        float xe = x[0];
#pragma unroll
        for (int e = 1; e < EPV; e++) xe = e == i ? x[e] : xe;
        bool tie;
        const uint32_t ue = stream_exact_units(A, st, xe, tie);
        nex++;
#pragma unroll
        for (int e = 0; e < EPV; e++) u[e] = e == i ? ue : u[e];
        tiem |= tie ? (1u << i) : 0u;
    }
}

template <bool BF16, int NV>
struct RawT {
    uint4 w[NV];
    uint32_t mw[NV];
    uint32_t pw[NV];
};

// The stream's arguments made wave-uniform (scalar registers, uniform branches).
__device__ __forceinline__ uint64_t rfl64(uint64_t v) {
    return ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(v >> 32)) << 32) |
           (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
}
template <typename T>
__device__ __forceinline__ T* rflp(T* p) {
    return (T*)rfl64((uint64_t)p);
}
__device__ __forceinline__ int32_t rfli(int32_t v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ float rflf(float v) { return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v))); }
__device__ __forceinline__ StreamArgs uniform_args(const StreamArgs& A) {
    StreamArgs U;
    U.logits = rflp(A.logits);
    U.mrow = rflp(A.mrow);
    U.hbm = rflp(A.hbm);
    U.hpre = rflp(A.hpre);
    U.hcnt = rflp(A.hcnt);
    U.hbase = rflp(A.hbase);
    U.hext = rflp(A.hext);
    U.hnb = (int64_t)rfl64((uint64_t)A.hnb);
    U.hnx = (int64_t)rfl64((uint64_t)A.hnx);
    U.spill = rflp(A.spill);
    U.trace = rflp(A.trace);
    U.V = (uint32_t)rfli((int32_t)A.V);
    U.lo = (uint32_t)rfli((int32_t)A.lo);
    U.hi = (uint32_t)rfli((int32_t)A.hi);
    U.s0 = rflf(A.s0);
    U.vec_ok = rfli(A.vec_ok);
    U.hdense = rfli(A.hdense);
    U.fast_div = rfli(A.fast_div);
    U.T = rflf(A.T);
    U.rT = rflf(A.rT);
    U.rTl = rflf(A.rTl);
    U.rp = rflf(A.rp);
    U.pp = rflf(A.pp);
    U.fp = rflf(A.fp);
    U.rep_on = rfli(A.rep_on);
    U.pres_on = rfli(A.pres_on);
    U.freq_on = rfli(A.freq_on);
    U.M = rflf(A.M);
    U.S = rflf(A.S);
    U.th = rflf(A.th);
    U.excl = (int64_t)rfl64((uint64_t)A.excl);
    U.kind = rfli(A.kind);
    U.gather = rfli(A.gather);
    U.gth = rflf(A.gth);
    return U;
}

// One step's raw words: the logits (16 bytes per vector), and the allow-mask and history
// bitmap words of every vector. FULL steps lie inside the range: every load is
// unconditional (absent tables read the row's own first words, discarded later), so no
// load is merged with another path and nothing waits for them before they are used. The
// range's first and last steps load element by element; elements outside it read as -inf.
template <bool BF16, int NV, bool FULL>
__device__ __forceinline__ void row_load(const StreamArgs& A, uint32_t base, RawT<BF16, NV>& r) {
    constexpr int EPV = Elem<BF16>::EPV;
    typedef typename Elem<BF16>::T ET;
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    const BFI_GLB ET* rp = gl((const ET*)A.logits);
    const uint32_t V = A.V;
    const BFI_GLB uint32_t* mp = gl(A.mrow ? A.mrow : (const uint32_t*)A.logits);
    const BFI_GLB uint32_t* pp = gl(A.hbm ? A.hbm : (const uint32_t*)A.logits);
#pragma unroll
    for (int q = 0; q < NV; q++) {
        const uint32_t id0 = base + (uint32_t)(q * BLOCK + threadIdx.x) * EPV;
        if (FULL) {
            const u32x4 v = *(const BFI_GLB u32x4*)(rp + id0);
            r.w[q] = make_uint4(v.x, v.y, v.z, v.w);
        } else {
            const uint32_t ninf = BF16 ? 0xFF80FF80u : 0xFF800000u;
            uint32_t ww[4] = {ninf, ninf, ninf, ninf};
#pragma unroll
            for (int e = 0; e < EPV; e++) {
                if (id0 + e >= A.hi || id0 + e < A.lo) continue;
                if (BF16) {
                    const uint32_t b = (uint32_t)rp[id0 + e];
                    ww[e >> 1] = (e & 1) ? (ww[e >> 1] & 0xFFFFu) | (b << 16) : (ww[e >> 1] & 0xFFFF0000u) | b;
                } else {
                    ww[e] = __float_as_uint((float)rp[id0 + e]);
                }
            }
            r.w[q] = make_uint4(ww[0], ww[1], ww[2], ww[3]);
        }
        const uint32_t wi = FULL ? id0 >> 5 : (id0 < V ? id0 >> 5 : 0u);
        r.mw[q] = mp[wi];
        r.pw[q] = pp[wi];
    }
}

// Masked, penalized logits of one vector.
template <bool BF16, int NV>
__device__ __forceinline__ void row_decode(const StreamArgs& A, const RawT<BF16, NV>& r, int q, uint32_t id0,
                                           float (&x)[Elem<BF16>::EPV]) {
    constexpr int EPV = Elem<BF16>::EPV;
    unpack16<BF16, NV>(r.w[q], x);
    const uint32_t em = (1u << EPV) - 1u;
    const uint32_t mb = A.mrow ? (r.mw[q] >> (id0 & 31)) & em : em;
    const uint32_t pb = A.hbm ? (r.pw[q] >> (id0 & 31)) & em : 0u;
#pragma unroll
    for (int e = 0; e < EPV; e++) x[e] = ((mb >> e) & 1u) ? x[e] : -__builtin_inff();
    if (pb) {
#pragma unroll
        for (int e = 0; e < EPV; e++)
            if ((pb >> e) & 1u) x[e] = sa_penalize(A, x[e], id0 + e);
    }
}

// Appends (id, e) to the row's candidate list (the first V entries of its spill area): e is
// the element's exact term expf(fl(x / T) - M) (sample.rs:374, 383), computed here for the
// few elements taken.
__device__ __forceinline__ void list_append(const StreamArgs& A, bool take, uint32_t id, float x) {
    const uint64_t bal = __ballot(take);
    if (!bal) return;
    const int leader = __ffsll((unsigned long long)bal) - 1;
    uint32_t base = 0;
    if (lane_id() == leader) base = lds_add(&g_sm.misc[MS_N], (uint32_t)__popcll(bal));
    base = (uint32_t)__builtin_amdgcn_readlane((int)base, leader);
    if (take) {
        const uint32_t pos = base + (uint32_t)__popcll(bal & lanes_below());
        const float e = exact_value(x, A.T, A.rT, A.fast_div, A.M, 1.0f, 0);
        if (pos < A.V) gl(A.spill)[pos] = ((uint64_t)id << 32) | __float_as_uint(e);
    }
}

// The running state of a stream (every thread holds the same).
struct StreamRun {
    StreamState st;
    uint32_t nex, nslow, nevt;
    uint64_t tslow, tfast, tmark;
};

// One step of a stream over the words in r (ids base ..): returns true when it stopped
// (out filled).
template <bool BF16, int NV>
__device__ __forceinline__ bool stream_step(const StreamArgs& A, float rS, const RawT<BF16, NV>& ra, uint32_t base,
                                            StreamRun& R, StreamOut& out) {
    RowSmem& sm = g_sm;
    constexpr int EPV = Elem<BF16>::EPV;
    const int tid = threadIdx.x;
    uint32_t qs = 0, tf = 0;
#pragma unroll
    for (int q = 0; q < NV; q++) {
        const uint32_t id0 = base + (uint32_t)(q * BLOCK + tid) * EPV;
        float xq[EPV];
        row_decode<BF16, NV>(A, ra, q, id0, xq);
        uint32_t uq[EPV], tiem;
        float hq[EPV];
        vector_units<EPV>(A, R.st, rS, xq, uq, tiem, hq, R.nex);
#pragma unroll
        for (int e = 0; e < EPV; e++) {
            const uint32_t id = id0 + e;
            const bool ex = (int64_t)id == A.excl;
            qs = sat_add(qs, ex ? 0u : uq[e]);
            tf |= (!ex && ((tiem >> e) & 1u)) ? 1u : 0u;
            if (A.gather) list_append(A, hq[e] >= A.gth && xq[e] > -__builtin_inff(), id, xq[e]);
        }
    }
    uint32_t anytie;
    const uint32_t tot = block_sum_sat_or(qs, tf, anytie, sm);
    const uint32_t run = sat_add(R.st.m, tot);
    if (!anytie && run < M_TOP && run < R.st.tu) {
        R.st.m = run;
        if (A.trace) {
            const uint64_t now = wall_clock64();
            R.tfast += now - R.tmark;
            R.tmark = now;
        }
        return false;
    }
    R.nslow++;
    // an event in this step: vector by vector, element by element in index order
#pragma unroll
    for (int q = 0; q < NV; q++) {
        const uint32_t id0 = base + (uint32_t)(q * BLOCK + tid) * EPV;
        float xq[EPV];
        row_decode<BF16, NV>(A, ra, q, id0, xq);
        int done = -1;  // positions (thread * EPV + e) of this vector up to here are summed
#pragma unroll 1
        for (;;) {
            uint32_t lp[EPV];
            bool ev[EPV];
            uint32_t tt = 0;
            uint32_t uq[EPV], tiem;
            float hq[EPV];
            vector_units<EPV>(A, R.st, rS, xq, uq, tiem, hq, R.nex);
#pragma unroll
            for (int e = 0; e < EPV; e++) {
                const int pos = tid * EPV + e;
                const bool skip = pos <= done || (int64_t)(id0 + e) == A.excl;
                ev[e] = !skip && ((tiem >> e) & 1u);
                tt = sat_add(tt, skip ? 0u : uq[e]);
                lp[e] = tt;
            }
            uint32_t vt;
            const uint32_t pre = block_excl_scan_sat(tt, vt, sm);
            uint32_t first = 0xFFFFFFFFu;
#pragma unroll
            for (int e = EPV - 1; e >= 0; e--) {
                const uint32_t r = sat_add(R.st.m, sat_add(pre, lp[e]));
                if (ev[e] || r >= M_TOP || r >= R.st.tu) first = (uint32_t)(tid * EPV + e);
            }
            const uint32_t fw = wave_min_u(first);
            if (lane_id() == 0) sm.wu2[wave_id()] = fw;
            __syncthreads();
            uint32_t f = 0xFFFFFFFFu;
#pragma unroll
            for (int w = 0; w < NWAVE; w++) f = min(f, sm.wu2[w]);
            if (f == 0xFFFFFFFFu) {
                __syncthreads();
                R.st.m = sat_add(R.st.m, vt);
                break;
            }
            if ((uint32_t)tid == f / EPV) {
                const int e = (int)(f % EPV);
                // the event element's values, selected without indexing registers
                uint32_t ex = 0u, lpe = 0u;
                bool eve = false;
                float xe = 0.0f;
#pragma unroll
                for (int k = 0; k < EPV; k++) {
                    if (k + 1 == e) ex = lp[k];
                    if (k == e) {
                        lpe = lp[k];
                        eve = ev[k];
                        xe = xq[k];
                    }
                }
                const uint32_t rb4 = R.st.m + pre + ex;  // below 2^24: no event before
                const uint32_t ra4 = sat_add(R.st.m, sat_add(pre, lpe));
                float res;
                uint32_t stop = 0;
                if (!eve && ra4 < M_TOP) {
                    res = state_value(ra4, R.st.ue);  // the threshold, inside the binade
                    stop = 1;
                } else {
                    const float sb = state_value(rb4, R.st.ue);
                    const float v = exact_value(xe, A.T, A.rT, A.fast_div, A.M, A.S, A.kind);
                    res = sb + v;  // the reference's own rounding of this step
                    stop = res >= A.th ? 1u : 0u;
                }
                sm.mf[MF_S] = res;
                sm.misc[MS_STOP] = stop;
            }
            __syncthreads();
            const float sn = sm.mf[MF_S];
            const uint32_t stp = sm.misc[MS_STOP];
            __syncthreads();
            if (stp) {
                out.cum = sn;
                out.stop = (int64_t)(base + (uint32_t)q * BLOCK * EPV + f);
                return true;
            }
            R.st = stream_state(sn, A);
            R.nevt++;
            done = (int)f;
        }
    }
    if (A.trace) {
        const uint64_t now = wall_clock64();
        R.tslow += now - R.tmark;
        R.tmark = now;
    }
    return false;
}

template <bool BF16>
__device__ __noinline__ StreamOut row_stream(const StreamArgs Ain) {
    const StreamArgs A = uniform_args(Ain);
    constexpr int EPV = Elem<BF16>::EPV;
    constexpr int NV = BF16 ? RNV_BF16 : RNV_F32;
    constexpr uint32_t SPAN = (uint32_t)BLOCK * NV * EPV;
    const uint32_t hi = A.hi;
    const float rS = A.kind ? 1.0f / A.S : 0.0f;
    StreamRun R;
    R.st = stream_state(A.s0, A);
    R.nex = R.nslow = R.nevt = 0;
    R.tslow = R.tfast = 0;
    R.tmark = A.trace ? wall_clock64() : 0;
    StreamOut out{0.0f, -1};
    uint32_t base = A.lo & ~(uint32_t)(EPV - 1);
    if (base != A.lo && base < hi) {  // a range starting inside a vector: a guarded first step
        RawT<BF16, NV> rt;
        row_load<BF16, NV, false>(A, base, rt);
        if (stream_step<BF16, NV>(A, rS, rt, base, R, out)) return out;
        base += SPAN;
    }
    // full steps, each loading the next one's words before it works on its own
    const uint32_t nfull = A.vec_ok && base < hi ? (hi - base) / SPAN : 0u;
    if (nfull) {
        // unrolled by two so no words are copied between buffers; every iteration issues
        // the same loads (past the last full step they re-read it, from the cache), so the
        // waits before a step count only the loads issued after its own
        RawT<BF16, NV> ra, rb;
        row_load<BF16, NV, true>(A, base, ra);
        for (uint32_t i = 0; i < nfull; i += 2) {
            const uint32_t b0 = base + i * SPAN;
            const uint32_t b1 = base + min(i + 1, nfull - 1) * SPAN, b2 = base + min(i + 2, nfull - 1) * SPAN;
            row_load<BF16, NV, true>(A, b1, rb);
            if (stream_step<BF16, NV>(A, rS, ra, b0, R, out)) return out;
            if (i + 1 >= nfull) break;
            row_load<BF16, NV, true>(A, b2, ra);
            if (stream_step<BF16, NV>(A, rS, rb, b1, R, out)) return out;
        }
        base += nfull * SPAN;
    }
    for (; base < hi; base += SPAN) {  // the tail (or every step of an unaligned row)
        RawT<BF16, NV> rt;
        row_load<BF16, NV, false>(A, base, rt);
        if (stream_step<BF16, NV>(A, rS, rt, base, R, out)) return out;
    }
    out.cum = state_value(R.st.m, R.st.ue);
    return out;
}

}  // namespace bfi

namespace bfi {

// ---- the candidate list: exact keys, buckets, ordered walks ----------------------------
//
// Each gathered candidate gets its probability p = fl(expf(s - M) / S) and a key whose
// descending order is the reference's: (ord(p) << 32 | ~id) for the sorted modes (stable
// sort by descending p of an index-ordered list, sample.rs:393, 398), (~id << 32 | bits(p))
// for the index-ordered min-p mode (retain keeps order, sample.rs:413). A counting sort puts
// the keys into NB buckets by the key's high bits; within a bucket they stay unsorted.

struct ListInfo {
    const uint64_t* G;  // keys grouped by bucket (LDS or the row's spill area); small: sorted
    uint32_t n;         // keys in G (candidates with p >= p_lo > 0)
    uint32_t nb;        // buckets in use
    uint64_t kmax;      // the largest key
    int row;
    int small;          // n <= SORTCAP: the keys sorted in LDS, no buckets
    float* cum;         // small lists: LDS room for a walk's running sum after each element
    uint32_t top, sh;   // bucketed lists: bucket of a key = top - (key >> 32 >> sh)
};

__device__ __forceinline__ float key_p(uint64_t key, bool idxmode) {
    return idxmode ? __uint_as_float((uint32_t)key) : __uint_as_float((uint32_t)(key >> 32) & 0x7FFFFFFFu);
}
__device__ __forceinline__ uint32_t key_id(uint64_t key, bool idxmode) {
    return idxmode ? ~(uint32_t)(key >> 32) : ~(uint32_t)key;
}
__device__ __forceinline__ uint64_t make_key(float p, uint32_t id, bool idxmode) {
    return idxmode ? (((uint64_t)(~id) << 32) | __float_as_uint(p))
                   : (((uint64_t)(0x80000000u | __float_as_uint(p)) << 32) | (uint64_t)(~id));
}

// Turns the N gathered (id, e) entries of the row's list (e: the exact term) into keys, keeps
// those with p >= p_lo (> 0), compacted (LDS, then the row's spill area from 2V), and groups
// them by bucket; at most WAVE keys are sorted by one wave instead. Every thread calls it.
// pf: the N (<= BLOCK) entries are already in sm.list[0, N) (fetched at the row's start).
__device__ __forceinline__ ListInfo build_list(const KArgs& a, RowSmem& sm, const RowCtx& C, uint32_t N, float M,
                                               float S, float p_lo, bool idxmode, bool pf = false) {
    const int tid = threadIdx.x;
    const uint64_t* src = a.spill + (int64_t)C.row * 4 * a.V;
    uint64_t* ovf = a.spill + (int64_t)C.row * 4 * a.V + 2 * (int64_t)a.V;
    N = min(N, (uint32_t)a.V);
    uint64_t ent0 = 0;
    if (pf) ent0 = (uint32_t)tid < N ? sm.list[tid] : 0ull;  // (read before any key lands)
    if (tid == 0) sm.misc[MS_NV] = 0u;
    __syncthreads();
    uint32_t hmax = 0u, hmin = 0xFFFFFFFFu;
    uint64_t kmax = 0;
    constexpr int BB = 8;  // entries loaded at once (global memory latency)
    // entry j (in range or not: every lane of a wave takes part) into the list as a key
    auto take = [&](uint64_t ent, bool in) {
        const uint32_t id = (uint32_t)(ent >> 32);
        const float p = exact_p(__uint_as_float((uint32_t)ent), S);
        const bool valid = in && p > 0.0f && p >= p_lo;
        const uint64_t key = make_key(p, id, idxmode);
        const uint64_t bal = __ballot(valid);
        if (!bal) return;
        const int leader = __ffsll((unsigned long long)bal) - 1;
        uint32_t base = 0;
        if (lane_id() == leader) base = lds_add(&sm.misc[MS_NV], (uint32_t)__popcll(bal));
        base = (uint32_t)__builtin_amdgcn_readlane((int)base, leader);
        if (valid) {
            const uint32_t pos = base + (uint32_t)__popcll(bal & lanes_below());
            if (pos < (uint32_t)LCAP) sm.list[pos] = key;
            else ovf[pos] = key;
            const uint32_t hi = (uint32_t)(key >> 32);
            hmax = max(hmax, hi);
            hmin = min(hmin, hi);
            kmax = key > kmax ? key : kmax;
        }
    };
    if (pf) {
        take(ent0, (uint32_t)tid < N);
    } else {
        for (uint32_t j0 = tid; j0 < N; j0 += BB * BLOCK) {
            uint64_t ent[BB];
#pragma unroll
            for (int i = 0; i < BB; i++) {
                const uint32_t j = j0 + (uint32_t)(i * BLOCK);
                ent[i] = j < N ? src[j] : 0ull;
            }
#pragma unroll
            for (int i = 0; i < BB; i++) take(ent[i], j0 + (uint32_t)(i * BLOCK) < N);
        }
    }
    __threadfence_block();
    __syncthreads();
    const uint32_t nv = sm.misc[MS_NV];
    ListInfo L;
    L.n = nv;
    L.row = C.row;
    L.nb = 0;
    if (nv <= (uint32_t)WAVE) {
        // small: one wave sorts the keys into LDS
        L.small = 1;
        L.G = sm.list;
        L.cum = reinterpret_cast<float*>(sm.grp);
        if (wave_id() == 0) {
            const int lane = lane_id();
            uint64_t key = (uint32_t)lane < nv ? sm.list[lane] : 0ull;
            key = wave_sort_desc(key);
            sm.list[lane] = key;
            if (lane == 0) sm.w64[0] = key;
        }
        __syncthreads();
        L.kmax = sm.w64[0];
        __syncthreads();
        return L;
    }
    if (nv <= (uint32_t)SORTCAP) {
        // medium: runs of 64 keys sorted by one wave each in registers, then each key goes to
        // its rank (keys are distinct: their ids differ): its place in its own run plus, in
        // every other run, the keys above it (a branch-free binary search of the descending
        // run; the last run's padding zeros rank below every key)
        static_assert(SORTCAP <= 2 * BLOCK && SORTCAP <= LCAP, "two keys per thread, runs in the list");
        L.small = 1;
        const uint32_t nr = (nv + WAVE - 1) / WAVE;
        for (uint32_t r = (uint32_t)wave_id(); r < nr; r += NWAVE) {
            const uint32_t j = r * WAVE + (uint32_t)lane_id();
            const uint64_t key = wave_sort_desc(j < nv ? sm.list[j] : 0ull);
            sm.list[j] = key;
        }
        __syncthreads();
        uint64_t* out = sm.grp;
        for (uint32_t i = (uint32_t)tid; i < nv; i += BLOCK) {
            const uint64_t k = sm.list[i];
            const uint32_t own = i / WAVE;
            uint32_t rank = i % WAVE;
#pragma unroll 4
            for (uint32_t r = 0; r < nr; r++) {
                if (r == own) continue;
                const uint64_t* run = sm.list + r * WAVE;
                uint32_t c = 0;
#pragma unroll
                for (uint32_t st = WAVE / 2; st > 0; st >>= 1) c += run[c + st - 1] > k ? st : 0u;
                rank += c + (run[c] > k ? 1u : 0u);
            }
            out[rank] = k;
        }
        __syncthreads();
        L.G = out;
        L.cum = reinterpret_cast<float*>(sm.list);
        L.kmax = out[0];
        return L;
    }
    L.small = 0;
    L.cum = nullptr;
    // reductions: max/min of the high words, the largest key
    {
        const uint32_t wmx = lane63(wave_scan_incl(hmax, 0u, [](uint32_t x, uint32_t y) { return max(x, y); }));
        const uint32_t wmn = wave_min_u(hmin);
        const uint64_t wk = wave_max_u64(kmax);
        if (lane_id() == 0) {
            sm.wu[wave_id()] = wmx;
            sm.wu2[wave_id()] = wmn;
            sm.w64[wave_id()] = wk;
        }
        __syncthreads();
        hmax = 0u;
        hmin = 0xFFFFFFFFu;
        kmax = 0;
#pragma unroll
        for (int w = 0; w < NWAVE; w++) {
            hmax = max(hmax, sm.wu[w]);
            hmin = min(hmin, sm.wu2[w]);
            kmax = sm.w64[w] > kmax ? sm.w64[w] : kmax;
        }
        __syncthreads();
    }
    int sh = idxmode ? 0 : 18;
    while ((hmax >> sh) - (hmin >> sh) >= (uint32_t)NB) sh++;
    const uint32_t top = hmax >> sh;
    L.nb = top - (hmin >> sh) + 1;
    L.top = top;
    L.sh = (uint32_t)sh;
    L.kmax = kmax;
    uint64_t* G = nv <= (uint32_t)LCAP ? sm.grp : a.spill + (int64_t)C.row * 4 * a.V + a.V;
    L.G = G;
    for (int b = tid; b < NB; b += BLOCK) {
        sm.bcnt[b] = 0u;
        sm.bfill[b] = 0u;
        sm.bsx[b] = 0u;
    }
    if (tid == 0) sm.pq_ok = 0u;
    __syncthreads();
    for (uint32_t j0 = tid; j0 < nv; j0 += BB * BLOCK) {
        uint64_t k[BB];
#pragma unroll
        for (int i = 0; i < BB; i++) {
            const uint32_t j = j0 + (uint32_t)(i * BLOCK);
            k[i] = j < nv ? (j < (uint32_t)LCAP ? sm.list[j] : ovf[j]) : 0ull;
        }
#pragma unroll
        for (int i = 0; i < BB; i++)
            if (k[i]) lds_add(&sm.bcnt[top - ((uint32_t)(k[i] >> 32) >> sh)], 1u);
    }
    __syncthreads();
    {
        // each thread a run of NB / BLOCK consecutive buckets
        constexpr int PB = (NB + BLOCK - 1) / BLOCK;
        uint32_t c = 0;
#pragma unroll
        for (int i = 0; i < PB; i++) c += (tid * PB + i < NB) ? sm.bcnt[tid * PB + i] : 0u;
        uint32_t tot;
        uint32_t o = block_excl_scan<uint32_t>(c, sm.wu, tot);
#pragma unroll
        for (int i = 0; i < PB; i++)
            if (tid * PB + i < NB) {
                sm.boff[tid * PB + i] = o;
                o += sm.bcnt[tid * PB + i];
            }
    }
    __syncthreads();
    for (uint32_t j0 = tid; j0 < nv; j0 += BB * BLOCK) {
        uint64_t k[BB];
#pragma unroll
        for (int i = 0; i < BB; i++) {
            const uint32_t j = j0 + (uint32_t)(i * BLOCK);
            k[i] = j < nv ? (j < (uint32_t)LCAP ? sm.list[j] : ovf[j]) : 0ull;
        }
        uint32_t at[BB];
#pragma unroll
        for (int i = 0; i < BB; i++) {
            const uint32_t b = top - ((uint32_t)(k[i] >> 32) >> sh);
            at[i] = k[i] ? sm.boff[b] + lds_add(&sm.bfill[b], 1u) : 0u;
        }
#pragma unroll
        for (int i = 0; i < BB; i++)
            if (k[i]) G[at[i]] = k[i];
    }
    __threadfence_block();
    __syncthreads();
    return L;
}

// Orders LDS writes of this wave before its later LDS reads (lanes of one wave only).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Bitonic sort (descending) of n keys at buf by one wave; n a power of two.
__device__ __forceinline__ void wave_sort_lds(uint64_t* buf, int n) {
    const int lane = lane_id();
    for (int size = 2; size <= n; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = lane; i < n / 2; i += WAVE) {
                const int lo = 2 * i - (i & (stride - 1));
                const int hi = lo + stride;
                const bool desc = (lo & size) == 0;
                const uint64_t x = buf[lo], y = buf[hi];
                if ((x < y) == desc) {
                    buf[lo] = y;
                    buf[hi] = x;
                }
            }
            wave_lds_sync();
        }
    }
}

// The same in global memory (a bucket larger than LDS holds; the row's spill area), with a
// device-scope fence between stages so the lanes see each other's stores.
__device__ __forceinline__ void wave_sort_glb(uint64_t* buf, int n) {
    const int lane = lane_id();
    for (int size = 2; size <= n; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = lane; i < n / 2; i += WAVE) {
                const int lo = 2 * i - (i & (stride - 1));
                const int hi = lo + stride;
                const bool desc = (lo & size) == 0;
                const uint64_t x = __hip_atomic_load(&buf[lo], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                const uint64_t y = __hip_atomic_load(&buf[hi], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if ((x < y) == desc) {
                    __hip_atomic_store(&buf[lo], y, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    __hip_atomic_store(&buf[hi], x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
            __threadfence();
            __builtin_amdgcn_wave_barrier();
            __threadfence();
        }
    }
}

// The n keys of a bucket (at src), sorted descending into a scratch buffer of n2 (a power of
// two >= n) keys: LDS when they fit, else the row's spill area (its sort scratch).
// Wave 0; returns the buffer.
__device__ __forceinline__ uint64_t* sort_bucket(uint64_t* gscratch, const uint64_t* src, uint32_t n, int n2) {
    const int lane = lane_id();
    uint64_t* buf = n2 <= LCAP ? g_sm.list : gscratch;
    for (int j = lane; j < n2; j += WAVE) buf[j] = (uint32_t)j < n ? src[j] : 0ull;
    if (n2 <= LCAP) {
        wave_lds_sync();
        wave_sort_lds(buf, n2);
    } else {
        __threadfence();
        __builtin_amdgcn_wave_barrier();
        wave_sort_glb(buf, n2);
    }
    return buf;
}

// A walk in key order from cum = 0: for each element (the excluded key adds nothing and has
// no rank), cum = fl(cum + p). It stops at the first element where cum >= th (how 1) or at
// the R-th element (how 2), else runs out (how 0) with the list's total.
struct WalkOut {
    float cum;
    uint32_t rank;  // the stop element's rank (how 1, 2) or the element count (how 0)
    uint64_t key;
    int how;
};

struct WalkState {
    uint32_t m;
    int32_t ue;
    uint32_t tu;
    uint32_t r;
};
__device__ __forceinline__ void walk_set(WalkState& w, float s, float th) {
    const SumState ss = sum_state(s);
    w.m = ss.m;
    w.ue = ss.ue;
    w.tu = thresh_units(fmaxf(th, 0.0f), ss.ue);
    if (!(th < __builtin_inff())) w.tu = 0xFFFFFFFFu;
}

// Element-level walk over one wave-load of sorted keys (one per lane, 0 = none). Returns
// true when it stopped (o filled). Wave-uniform.
__device__ __forceinline__ bool walk_elems(WalkState& w, uint64_t key, float th, uint32_t R, uint64_t excl,
                                           bool idxmode, WalkOut& o, float* cum) {
    const int lane = lane_id();
    int done = -1;
    for (;;) {
        const bool valid = key != 0 && key != excl && lane > done;
        const float p = key_p(key, idxmode);
        const float t = units_of(p, w.ue);
        const uint32_t q = valid ? quant_units(t) : 0u;
        const bool tie = valid && quant_tie(t);
        const uint32_t c = valid ? 1u : 0u;
        const uint32_t Qi = wave_scan_sat(q);
        const uint32_t Ci = wave_scan_incl(c, 0u, [](uint32_t x, uint32_t y) { return x + y; });
        const uint32_t run = sat_add(w.m, Qi);
        const bool ev = valid && (tie || run >= M_TOP || run >= w.tu || (uint64_t)w.r + Ci >= (uint64_t)R);
        const uint64_t bal = __ballot(ev);
        const int j = bal ? __ffsll((unsigned long long)bal) - 1 : WAVE;
        // the elements before the first event are settled: their running sums
        if (cum && valid && lane < j) cum[w.r + Ci - 1] = state_value(run, w.ue);
        if (!bal) {
            w.m = lane63(run);
            w.r += lane63(Ci);
            return false;
        }
        const uint32_t run_j = (uint32_t)__builtin_amdgcn_readlane((int)run, j);
        const uint32_t runb = j ? (uint32_t)__builtin_amdgcn_readlane((int)run, j - 1) : w.m;
        const uint32_t ci_j = (uint32_t)__builtin_amdgcn_readlane((int)Ci, j);
        const bool tie_j = __builtin_amdgcn_readlane((int)tie, j) != 0;
        const uint64_t key_j = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(key >> 32), j) << 32) |
                               (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)key, j);
        const uint32_t rank_j = w.r + ci_j - 1;
        if (!tie_j && run_j < M_TOP) {
            o.cum = state_value(run_j, w.ue);
            o.rank = rank_j;
            o.key = key_j;
            o.how = run_j >= w.tu ? 1 : 2;
            if (cum && lane == 0) cum[rank_j] = o.cum;
            return true;
        }
        const float sn = state_value(runb, w.ue) + key_p(key_j, idxmode);
        if (cum && lane == 0) cum[rank_j] = sn;
        if (sn >= th || (uint64_t)w.r + ci_j >= (uint64_t)R) {
            o.cum = sn;
            o.rank = rank_j;
            o.key = key_j;
            o.how = sn >= th ? 1 : 2;
            return true;
        }
        walk_set(w, sn, th);
        w.r = rank_j + 1;
        done = j;
    }
}

// ---- walks over a bucketed (large) list ----------------------------------------------
//
// Rounds over the keys in bucket order, the whole block at once: from the walk's state,
// each thread takes WPT consecutive keys of a tile of whole buckets, their unit counts at
// the state's binade and their ranks come from a block scan, and the first key at which
// an event occurs (the sum leaving its binade, reaching the threshold, a tie of RN, the
// R-th element) names the bucket to walk element by element: the buckets before it are
// added whole (inside a bucket the order does not change a sum that stays in one binade
// without ties), that bucket is sorted and walked by one wave, and the next round starts
// after it.

constexpr int WPT = 16;                           // keys per thread per round
constexpr uint32_t WTILE = (uint32_t)BLOCK * WPT;  // keys per round

// The first key of bucket b (b == nb: the list's end).
__device__ __forceinline__ uint32_t bucket_start(const RowSmem& sm, const ListInfo& L, uint32_t b) {
    return b < L.nb ? sm.boff[b] : L.n;
}
// Largest bucket b in [lo, hi) with bucket_start(b) <= g.
__device__ __forceinline__ uint32_t bucket_of(const RowSmem& sm, const ListInfo& L, uint32_t lo, uint32_t hi,
                                              uint32_t g) {
    while (hi - lo > 1) {
        const uint32_t mid = (lo + hi) >> 1;
        if (bucket_start(sm, L, mid) <= g) lo = mid;
        else hi = mid;
    }
    return lo;
}

// The n keys of bucket b sorted descending into LDS (sm.list) or, above LCAP / 2 keys, the
// row's sort scratch; every thread calls it and gets the buffer.
__device__ __forceinline__ const uint64_t* sort_event_bucket(const ListInfo& L, uint32_t b, uint64_t* gscratch,
                                                             RowSmem& sm) {
    const int tid = threadIdx.x;
    const uint32_t n = sm.bcnt[b], o0 = sm.boff[b];
    if (n <= (uint32_t)(2 * BLOCK)) {
        // ranks by counting (keys are distinct), from a copy in the list's upper half
        uint64_t* src = sm.list + LCAP / 2;
        for (uint32_t j = (uint32_t)tid; j < n; j += BLOCK) src[j] = L.G[o0 + j];
        __syncthreads();
        const uint32_t i0 = (uint32_t)tid, i1 = (uint32_t)tid + BLOCK;
        const uint64_t k0 = i0 < n ? src[i0] : ~0ull;
        const uint64_t k1 = i1 < n ? src[i1] : ~0ull;
        uint32_t r0 = 0, r1 = 0;
#pragma unroll 4
        for (uint32_t j = 0; j < n; j++) {
            const uint64_t kj = src[j];
            r0 += kj > k0 ? 1u : 0u;
            r1 += kj > k1 ? 1u : 0u;
        }
        if (i0 < n) sm.list[r0] = k0;
        if (i1 < n) sm.list[r1] = k1;
        __syncthreads();
        return sm.list;
    }
    int n2 = WAVE;
    while ((uint32_t)n2 < n) n2 <<= 1;
    if (wave_id() == 0) (void)sort_bucket(gscratch, L.G + o0, n, n2);
    __syncthreads();
    return n2 <= LCAP ? sm.list : gscratch;  // (sort_bucket's buffer)
}

constexpr float PQ_EPS = 0x1p-13f;  // relative width of a bucket walk's predicted running sum

// Per bucket of a bucketed list: the units its keys add at the binade a walk's running sum
// lies in while it passes the bucket, as predicted from the real prefix of the bucket masses
// widened by PQ_EPS both ways (bq; bk: that unit exponent + 512, 0 where the prediction
// straddles a binade boundary, bit 31 where a key is a tie of RN there). The excluded key
// adds nothing. A walk takes a bucket's bq in one step when its state lies in that binade;
// a wrong prediction costs the bucket's serial sum, never the result. Every thread; each
// sums a contiguous run of keys and adds to a bucket once per bucket it touches.
__device__ __forceinline__ void bucket_units(const ListInfo& L, RowSmem& sm, uint64_t excl) {
    constexpr int KB = 8;  // keys loaded at once (the list may sit in global memory)
    const int tid = threadIdx.x;
    float* const bm = reinterpret_cast<float*>(sm.bfill);  // per bucket: real mass
    for (int b = tid; b < NB; b += BLOCK) {
        bm[b] = 0.0f;
        sm.bq[b] = 0u;
    }
    __syncthreads();
    const uint32_t per = (L.n + BLOCK - 1u) / BLOCK;
    const uint32_t j0 = min((uint32_t)tid * per, L.n), j1 = min(j0 + per, L.n);
    {
        uint32_t cb = 0xFFFFFFFFu;
        float acc = 0.0f;
        for (uint32_t jb = j0; jb < j1; jb += KB) {
            uint64_t k[KB];
#pragma unroll
            for (int i = 0; i < KB; i++) k[i] = jb + (uint32_t)i < j1 ? L.G[jb + i] : 0ull;
#pragma unroll
            for (int i = 0; i < KB; i++) {
                if (!k[i]) continue;
                const uint32_t b = L.top - ((uint32_t)(k[i] >> 32) >> L.sh);
                if (b != cb) {
                    if (cb != 0xFFFFFFFFu) atomicAdd(&bm[cb], acc);
                    cb = b;
                    acc = 0.0f;
                }
                acc += k[i] == excl ? 0.0f : key_p(k[i], false);
            }
        }
        if (cb != 0xFFFFFFFFu) atomicAdd(&bm[cb], acc);
    }
    __syncthreads();
    {
        static_assert(NB == 2 * BLOCK, "two buckets a thread");
        const uint32_t b0 = 2u * (uint32_t)tid;
        const float m0 = bm[b0], m1 = bm[b0 + 1u];
        float tot;
        const float P0 = block_excl_scan<float>(m0 + m1, sm.wf, tot);
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const uint32_t b = b0 + (uint32_t)i;
            const float P = i ? P0 + m0 : P0, m = i ? m1 : m0;
            uint32_t k = 0u;
            if (b < L.nb && m > 0.0f && P > 0.0f) {
                const float lo = P * (1.0f - PQ_EPS), hi = (P + m) * (1.0f + PQ_EPS);
                const uint32_t elo = max(__float_as_uint(lo) >> 23, 1u), ehi = max(__float_as_uint(hi) >> 23, 1u);
                if (elo == ehi) k = elo - 150u + 512u;
            }
            sm.bk[b] = k;
        }
    }
    __syncthreads();
    {
        uint32_t cb = 0xFFFFFFFFu, q = 0u, kb = 0u;
        bool tie = false;
        for (uint32_t jb = j0; jb < j1; jb += KB) {
            uint64_t k[KB];
#pragma unroll
            for (int i = 0; i < KB; i++) k[i] = jb + (uint32_t)i < j1 ? L.G[jb + i] : 0ull;
#pragma unroll
            for (int i = 0; i < KB; i++) {
                if (!k[i]) continue;
                const uint32_t b = L.top - ((uint32_t)(k[i] >> 32) >> L.sh);
                if (b != cb) {
                    if (kb) {
                        atomicAdd(&sm.bq[cb], min(q, M_TOP));
                        if (tie) atomicOr(&sm.bk[cb], 0x80000000u);
                    }
                    cb = b;
                    q = 0u;
                    tie = false;
                    kb = sm.bk[b] & 0x3FFu;
                }
                if (kb && k[i] != excl) {
                    const float t = units_of(key_p(k[i], false), (int32_t)kb - 512);
                    q = sat_add(q, quant_units(t));
                    tie = tie || quant_tie(t);
                }
            }
        }
        if (kb) {
            atomicAdd(&sm.bq[cb], min(q, M_TOP));
            if (tie) atomicOr(&sm.bk[cb], 0x80000000u);
        }
    }
    if (tid == 0) {
        sm.pq_excl = excl;
        sm.pq_ok = 1u;
    }
    __syncthreads();
}

__device__ __noinline__ WalkOut walk_big(const ListInfo L, float th, uint32_t R, uint64_t excl, int32_t idxmode,
                                            uint64_t* gscratch, bool rec, uint32_t from) {
    RowSmem& sm = g_sm;
    const int tid = threadIdx.x;
    uint32_t* const tq = sm.bfill;           // per thread: exclusive unit prefix of its keys
    uint32_t* const tc = sm.bfill + BLOCK;   // per thread: exclusive rank prefix
    static_assert(2 * BLOCK <= NB, "per-thread prefixes in the fill counters");
    WalkState w;
    walk_set(w, 0.0f, th);
    w.r = 0;
    WalkOut o{0.0f, 0u, 0ull, 0};
    bool stopped = false;
    uint32_t b0 = 0;
    if (from > 0u) {  // resume at a recorded bucket start
        const uint32_t x = sm.bsx[from];
        walk_set(w, state_value(sm.bsm[from], (int32_t)(x & 1023u) - 512), th);
        w.r = x >> 10;
        b0 = from;
    }
    while (b0 < L.nb && !stopped) {
        // the round's buckets [b0, b1): whole buckets within one tile, at least one
        const uint32_t e0 = sm.boff[b0];
        if (rec && tid == 0) {
            sm.bsm[b0] = w.m;
            sm.bsx[b0] = (w.r << 10) | (uint32_t)(w.ue + 512);
        }
        uint32_t b1 = bucket_of(sm, L, b0, L.nb + 1, e0 + WTILE);
        if (b1 <= b0) b1 = b0 + 1;
        const uint32_t e1 = bucket_start(sm, L, b1);
        // sub-tiles (more than one only for a single bucket larger than a tile)
        uint32_t qacc = 0, cacc = 0, first = 0xFFFFFFFFu;
        for (uint32_t s0 = e0; s0 < e1 && first == 0xFFFFFFFFu; s0 += WTILE) {
            const uint32_t j0 = s0 + (uint32_t)tid * WPT;
            uint32_t q[WPT], Q = 0, Cn = 0, tb = 0;
#pragma unroll
            for (int i = 0; i < WPT; i++) {
                const uint32_t j = j0 + (uint32_t)i;
                const uint64_t key = j < e1 ? L.G[j] : 0ull;
                const bool valid = key != 0ull && key != excl;
                const float t = units_of(key_p(key, idxmode), w.ue);
                q[i] = valid ? quant_units(t) : 0u;
                tb |= (valid && quant_tie(t)) ? 1u << i : 0u;
                tb |= valid ? 1u << (16 + i) : 0u;
                Q = sat_add(Q, q[i]);
                Cn += valid ? 1u : 0u;
            }
            uint32_t Qt, Ct;
            const uint32_t Qx = sat_add(qacc, block_excl_scan_sat(Q, Qt, sm));
            const uint32_t Cx = cacc + block_excl_scan<uint32_t>(Cn, sm.wu2, Ct);
            if (tid < BLOCK) {
                tq[tid] = Qx;
                tc[tid] = Cx;
            }
            // this thread's first event
            uint32_t run = sat_add(w.m, Qx), rk = w.r + Cx, mine = 0xFFFFFFFFu;
#pragma unroll
            for (int i = 0; i < WPT; i++) {
                const bool valid = (tb >> (16 + i)) & 1u;
                run = sat_add(run, q[i]);
                rk += valid ? 1u : 0u;
                const bool ev = valid && (((tb >> i) & 1u) || run >= M_TOP || run >= w.tu || rk >= R);
                if (ev && mine == 0xFFFFFFFFu) mine = j0 + (uint32_t)i;
            }
            first = block_min_u(mine, sm.wu);
            qacc = sat_add(qacc, Qt);
            cacc += Ct;
        }
        if (first == 0xFFFFFFFFu) {  // no event: every bucket of the round added whole
            w.m = sat_add(w.m, qacc);
            w.r += cacc;
            b0 = b1;
            continue;
        }
        // the event's bucket and the state at its start
        const uint32_t bs = bucket_of(sm, L, b0, b1, first);
        const uint32_t es = sm.boff[bs];
        if (bs > b0) {
            // (one sub-tile: the owner of key es adds its keys before es to its prefix)
            const uint32_t own = (es - e0) / WPT, skip = (es - e0) % WPT;
            if ((uint32_t)tid == own) {
                uint32_t qq = tq[own], cc = tc[own];
                for (uint32_t i = 0; i < skip; i++) {
                    const uint64_t key = L.G[e0 + own * WPT + i];
                    const bool valid = key != 0ull && key != excl;
                    qq = sat_add(qq, valid ? quant_units(units_of(key_p(key, idxmode), w.ue)) : 0u);
                    cc += valid ? 1u : 0u;
                }
                sm.misc[MS_NFB] = qq;
                sm.misc[MS_NV] = cc;
            }
            __syncthreads();
            w.m = sat_add(w.m, sm.misc[MS_NFB]);
            w.r += sm.misc[MS_NV];
            __syncthreads();
        }
        if (rec && tid == 0) {
            sm.bsm[bs] = w.m;
            sm.bsx[bs] = (w.r << 10) | (uint32_t)(w.ue + 512);
        }
        // the bucket sorted, then walked element by element from that state (wave 0)
        const uint64_t* buf = sort_event_bucket(L, bs, gscratch, sm);
        const uint32_t n = sm.bcnt[bs];
        if (wave_id() == 0) {
            const int lane = lane_id();
            for (uint32_t j = 0; j < n && !stopped; j += WAVE)
                stopped = walk_elems(w, j + (uint32_t)lane < n ? buf[j + lane] : 0ull, th, R, excl, idxmode, o, nullptr);
            if (lane == 0) {
                sm.misc[MS_FLAG] = stopped ? 1u : 0u;
                sm.misc[MS_STOP] = o.rank;
                sm.misc[MS_STOPLO] = (uint32_t)o.key;
                sm.misc[MS_TOK] = (uint32_t)(o.key >> 32);
                sm.misc[MS_KIND] = (uint32_t)o.how;
                sm.mf[MF_CUM] = o.cum;
                sm.misc[MS_CLO] = w.m;
                sm.misc[MS_CHI] = (uint32_t)w.ue;
                sm.misc[MS_CNEXT] = w.tu;
                sm.misc[MS_VERDICT] = w.r;
            }
        }
        __syncthreads();
        stopped = sm.misc[MS_FLAG] != 0u;
        o.rank = sm.misc[MS_STOP];
        o.key = ((uint64_t)sm.misc[MS_TOK] << 32) | sm.misc[MS_STOPLO];
        o.how = (int)sm.misc[MS_KIND];
        o.cum = sm.mf[MF_CUM];
        w.m = sm.misc[MS_CLO];
        w.ue = (int32_t)sm.misc[MS_CHI];
        w.tu = sm.misc[MS_CNEXT];
        w.r = sm.misc[MS_VERDICT];
        __syncthreads();
        b0 = bs + 1;
    }
    if (!stopped) {
        o.cum = state_value(w.m, w.ue);
        o.rank = w.r;
        o.key = 0;
        o.how = 0;
    }
    return o;
}

// The walk: over a small (sorted) list or a bucketed list in LDS by wave 0, the result
// broadcast through LDS to every thread; over a bucketed list in the spill area (more keys
// than LDS holds) by the block (walk_big). In LDS, wave 0 sums 64 buckets a step and walks
// the event buckets of up to 64 keys itself; a larger event bucket is sorted by the block.
// rec: a bucketed walk records the running state before the buckets it passes (bsm/bsx);
// from: a bucketed walk starts at bucket `from` with the state recorded there (an earlier walk
// over the same keys that excluded none, and an excluded key, if any, not before it).
__device__ __forceinline__ WalkOut walk(const ListInfo L, float th, uint32_t R, uint64_t excl, int32_t idxmode,
                                     uint64_t* gscratch, float* cum = nullptr, bool rec = false, uint32_t from = 0) {
    RowSmem& sm = g_sm;
    // buckets whose predicted units hold at the walk's binade take them whole; the others are
    // walked element by element (without a prediction: summed one key at a time, by the block
    // for a list in the spill area)
    const bool pq = !idxmode && !L.small && sm.pq_ok && sm.pq_excl == excl;
    if (!L.small && L.n > (uint32_t)LCAP && !pq) return walk_big(L, th, R, excl, idxmode, gscratch, rec, from);
    WalkOut o{0.0f, 0u, 0ull, 0};
    const int lane = lane_id();
    // (the walk's state lives in wave 0; the other waves only help sort large event buckets)
    WalkState w;
    walk_set(w, 0.0f, th);
    w.r = 0;
    bool stopped = false;
    if (L.small) {
        if (wave_id() == 0) {
            // the first WAVE keys as real f32 additions, one after another in straight-line code
            // (lane j's key read by every lane, the sum after it kept by lane j): at the head of
            // a descending list the running sum is small against its terms and leaves its
            // binade or meets a tie every few keys, each a round of the wave-wide walk below
            const uint32_t n0 = min(L.n, (uint32_t)WAVE);
            const uint64_t kl = (uint32_t)lane < n0 ? L.G[lane] : 0ull;
            const bool valid = (uint32_t)lane < n0 && kl != excl;
            const float pl = valid ? key_p(kl, idxmode) : 0.0f;
            float sl = 0.0f, sh = 0.0f;  // (adding 0 for the other lanes leaves the sum as it is)
#pragma unroll
            for (int j = 0; j < WAVE; j++) {
                sh = sh + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pl), j));
                sl = lane == j ? sh : sl;
            }
            const uint64_t vb = __ballot(valid);
            const uint32_t ci = (uint32_t)__popcll(vb & lanes_below()) + (valid ? 1u : 0u);  // rank + 1
            const float thr = fmaxf(th, 0.0f);  // (the wave-wide walk's threshold units)
            const uint64_t eb = __ballot(valid && (sl >= thr || ci >= R));
            const int js = eb ? __ffsll((unsigned long long)eb) - 1 : WAVE;
            if (cum && valid && lane <= js) cum[ci - 1u] = sl;
            if (eb) {
                const float s_j = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sl), js));
                const uint64_t k_j = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(kl >> 32), js) << 32) |
                                     (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)kl, js);
                o = WalkOut{s_j, (uint32_t)__builtin_amdgcn_readlane((int)ci, js) - 1u, k_j, s_j >= thr ? 1 : 2};
                stopped = true;
            } else {
                walk_set(w, sh, th);
                w.r = (uint32_t)__popcll(vb);
            }
            for (uint32_t j0 = n0; j0 < L.n && !stopped; j0 += WAVE)
                stopped = walk_elems(w, j0 + (uint32_t)lane < L.n ? L.G[j0 + lane] : 0ull, th, R, excl, idxmode, o, cum);
        }
    } else {
        uint32_t b0 = 0;
        if (from > 0u) {
            const uint32_t x = sm.bsx[from];
            walk_set(w, state_value(sm.bsm[from], (int32_t)(x & 1023u) - 512), th);
            w.r = x >> 10;
            b0 = from;
        }
        const uint32_t bex = excl ? L.top - ((uint32_t)(excl >> 32) >> L.sh) : 0xFFFFFFFFu;
        for (;;) {
            uint32_t big = L.nb;  // an event bucket of more than 64 keys (nb: the walk is over)
            if (wave_id() == 0) {
                while (b0 < L.nb && !stopped) {
                    const uint32_t b = b0 + (uint32_t)lane;
                    const uint32_t cnt = b < L.nb ? sm.bcnt[b] : 0u;
                    const uint32_t off = b < L.nb ? sm.boff[b] : 0u;
                    const uint32_t kb = pq && b < L.nb ? sm.bk[b] : 0u;
                    uint32_t Q = 0, c = 0;
                    bool tie = false, force = false;
                    if (pq) {
                        if (kb == (uint32_t)(w.ue + 512) && b != bex) {
                            Q = sm.bq[b];
                            c = cnt;
                        } else {
                            force = cnt > 0u;
                        }
                    } else {
                        for (uint32_t j = 0; j < cnt; j++) {
                            const uint64_t key = L.G[off + j];
                            if (key == excl) continue;
                            const float t = units_of(key_p(key, idxmode), w.ue);
                            Q = sat_add(Q, quant_units(t));
                            tie = tie || quant_tie(t);
                            c++;
                        }
                    }
                    const uint32_t Qi = wave_scan_sat(Q);
                    const uint32_t Ci = wave_scan_incl(c, 0u, [](uint32_t x, uint32_t y) { return x + y; });
                    const uint32_t run = sat_add(w.m, Qi);
                    const bool ev =
                        force || (c > 0 && (tie || run >= M_TOP || run >= w.tu || (uint64_t)w.r + Ci >= (uint64_t)R));
                    const uint64_t bal = __ballot(ev);
                    if (rec) {  // the state before each bucket up to the first event's
                        const int s1 = bal ? __ffsll((unsigned long long)bal) - 1 : WAVE;
                        // (the shuffles run on every lane: a lane outside exec reads back as 0)
                        const uint32_t Qu = (uint32_t)__shfl_up((int)Qi, 1), Cu = (uint32_t)__shfl_up((int)Ci, 1);
                        const uint32_t Qx = lane ? Qu : 0u, Cx = lane ? Cu : 0u;
                        if (b < L.nb && lane <= s1) {
                            sm.bsm[b] = sat_add(w.m, Qx);
                            sm.bsx[b] = ((w.r + Cx) << 10) | (uint32_t)(w.ue + 512);
                        }
                    }
                    if (!bal) {
                        w.m = lane63(run);
                        w.r += lane63(Ci);
                        b0 += WAVE;
                        continue;
                    }
                    const int s = __ffsll((unsigned long long)bal) - 1;
                    if (s > 0) {
                        w.m = (uint32_t)__builtin_amdgcn_readlane((int)run, s - 1);
                        w.r += (uint32_t)__builtin_amdgcn_readlane((int)Ci, s - 1);
                    }
                    // the bucket of the event, sorted and walked element by element
                    const uint32_t bs = b0 + (uint32_t)s;
                    const uint32_t n = sm.bcnt[bs], o0 = sm.boff[bs];
                    if (n > (uint32_t)WAVE) {
                        big = bs;
                        break;
                    }
                    uint64_t key = (uint32_t)lane < n ? L.G[o0 + lane] : 0ull;
                    key = wave_sort_desc(key);
                    stopped = walk_elems(w, key, th, R, excl, idxmode, o, nullptr);
                    b0 = bs + 1;
                }
                if (lane == 0) sm.misc[MS_CNEXT] = big;
            }
            __syncthreads();
            big = sm.misc[MS_CNEXT];
            __syncthreads();
            if (big >= L.nb) break;
            const uint64_t* buf = sort_event_bucket(L, big, gscratch, sm);
            if (wave_id() == 0) {
                const uint32_t n = sm.bcnt[big];
                for (uint32_t j0 = 0; j0 < n && !stopped; j0 += WAVE)
                    stopped = walk_elems(w, j0 + (uint32_t)lane < n ? buf[j0 + lane] : 0ull, th, R, excl, idxmode, o,
                                         nullptr);
                b0 = big + 1;
            }
            __syncthreads();  // (the sorted copy is read before the next sort overwrites it)
        }
    }
    if (wave_id() == 0) {
        if (!stopped) {
            o.cum = state_value(w.m, w.ue);
            o.rank = w.r;
            o.key = 0;
            o.how = 0;
        }
        if (lane == 0) {
            sm.mf[MF_CUM] = o.cum;
            sm.misc[MS_STOP] = o.rank;
            sm.misc[MS_STOPLO] = (uint32_t)o.key;
            sm.misc[MS_FLAG] = (uint32_t)(o.key >> 32);
            sm.misc[MS_KIND] = (uint32_t)o.how;
        }
    }
    __syncthreads();
    o.cum = sm.mf[MF_CUM];
    o.rank = sm.misc[MS_STOP];
    o.key = ((uint64_t)sm.misc[MS_FLAG] << 32) | sm.misc[MS_STOPLO];
    o.how = (int)sm.misc[MS_KIND];
    __syncthreads();
    return o;
}

// Lists the first `lim` keys in order (ids and probabilities) into the row's target
// arrays (target_rows' kept list). Wave 0.
__device__ __forceinline__ void list_kept(const ListInfo L, uint32_t* ids, float* probs, uint32_t lim, int32_t idxmode,
                                      uint64_t* gscratch) {
    RowSmem& sm = g_sm;
    if (L.small) {
        for (uint32_t j = (uint32_t)threadIdx.x; j < lim; j += BLOCK) {
            const uint64_t key = L.G[j];
            ids[j] = key_id(key, idxmode);
            probs[j] = key_p(key, idxmode);
        }
    } else if (wave_id() == 0) {
        const int lane = lane_id();
        uint32_t w = 0;
        for (uint32_t b = 0; b < L.nb && w < lim; b++) {
            const uint32_t n = sm.bcnt[b], o0 = sm.boff[b];
            if (!n) continue;
            int n2 = WAVE;
            while ((uint32_t)n2 < n) n2 <<= 1;
            const uint64_t* buf = sort_bucket(gscratch, L.G + o0, n, n2);
            for (uint32_t j = lane; j < n; j += WAVE) {
                const uint32_t pos = w + j;
                if (pos < lim) {
                    const uint64_t key = buf[j];
                    ids[pos] = key_id(key, idxmode);
                    probs[pos] = key_p(key, idxmode);
                }
            }
            w += n;
            wave_lds_sync();
        }
    }
    __syncthreads();
}

}  // namespace bfi

namespace bfi {

// ---- results -----------------------------------------------------------------------------

// Stores the row's outcome. For spec verify, `verdict` is 1 = Accept, 0 = Reject(token);
// the last row of a sequence to finish resolves the accepted prefix (spec.rs:140-162).
__device__ __forceinline__ void row_emit(const KArgs& a, RowSmem& sm, const RowCtx& C, uint32_t token, uint32_t verdict) {
    const int tid = threadIdx.x;
    if (!C.verify) {
        if (tid == 0 && a.out_tok) a.out_tok[C.row] = token;
        return;
    }
    if (tid == 0) {
        a.row_res[2 * C.row] = C.judged ? verdict : 2u;
        a.row_res[2 * C.row + 1] = token;
    }
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        const uint32_t prev = glb_add(&a.seq_ctr[C.seq], 1u);
        sm.misc[MS_LAST] = prev == (uint32_t)C.dl;
    }
    __syncthreads();
    if (!sm.misc[MS_LAST]) return;
    __threadfence();
    if (tid == 0) {
        a.seq_ctr[C.seq] = 0;
        const int base = C.seq * a.rows_per_seq;
        int acc = C.dl;
        for (int i = 0; i < C.dl; i++) {
            if (__hip_atomic_load(&a.row_res[2 * (base + i)], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0u) {
                acc = i;
                break;
            }
        }
        a.out_accepted[C.seq] = acc;
        a.out_next[C.seq] =
            __hip_atomic_load(&a.row_res[2 * (base + acc) + 1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// A token target (greedy, min-p fallback): judge is equality (spec.rs:81-82).
__device__ __forceinline__ void finish_token(const KArgs& a, RowSmem& sm, const RowCtx& C, uint32_t tok) {
    if (threadIdx.x == 0 && a.t_kind) {
        a.t_kind[C.row] = BFI_SMP_TARGET_TOKEN;
        a.t_kept[C.row] = 0;
        a.t_listed[C.row] = 0;
    }
    row_emit(a, sm, C, tok, C.judged ? (tok == C.draft ? 1u : 0u) : 1u);
}

__device__ __forceinline__ void target_weights(const KArgs& a, const RowCtx& C, int64_t L, int64_t listed) {
    if (threadIdx.x == 0 && a.t_kind) {
        a.t_kind[C.row] = BFI_SMP_TARGET_WEIGHTS;
        a.t_kept[C.row] = (int32_t)min(L, (int64_t)INT32_MAX);
        a.t_listed[C.row] = (int32_t)listed;
    }
}

__device__ __forceinline__ void put_stats(const KArgs& a, const RowCtx& C, float M, float S, float kept, float mode) {
    if (threadIdx.x == 0 && a.t_stats) {
        a.t_stats[C.row * 4 + 0] = M;
        a.t_stats[C.row * 4 + 1] = S;
        a.t_stats[C.row * 4 + 2] = kept;
        a.t_stats[C.row * 4 + 3] = mode;
    }
}

// ---- row maximum over the penalized values (histories the streaming pass left out) -------

template <bool BF16>
__device__ __noinline__ ArgMax row_max(const StreamArgs Ain) {
    const StreamArgs A = uniform_args(Ain);
    constexpr int EPV = Elem<BF16>::EPV;
    constexpr int NV = BF16 ? RNV_BF16 : RNV_F32;
    constexpr uint32_t SPAN = (uint32_t)BLOCK * NV * EPV;
    const uint32_t V = A.V;
    ArgMax best{-__builtin_inff(), 0xFFFFFFFFu};
    for (uint32_t base = 0; base < V; base += SPAN) {
        RawT<BF16, NV> r;
        row_load<BF16, NV, false>(A, base, r);
#pragma unroll
        for (int q = 0; q < NV; q++) {
            const uint32_t id0 = base + (uint32_t)(q * BLOCK + threadIdx.x) * EPV;
            float x[EPV];
            row_decode<BF16, NV>(A, r, q, id0, x);
#pragma unroll
            for (int e = 0; e < EPV; e++)
                if (id0 + e < V) best = argmax_merge(best, ArgMax{x[e], id0 + e});
        }
    }
    return block_argmax(best, g_sm.wf, g_sm.wu);
}

// ---- the normalizer from the quantizing pass's chunk summaries ---------------------------
//
// The chunks' items (smp_quant.hip) in index order: the run before each window element, the
// element, and each chunk's tail run. Wave 0 walks them 64 at a time from the running sum's
// exact state (m, ue): a run adds its units in one step when the state lies in the run's
// binade (a zero run: in its binade or above) and stays below the binade's top; a window
// element adds RN(e / u) units unless it is a tie or leaves the binade, in which case it is
// one real f32 addition (the reference's rounding of that step). A run that fails its check
// (a prediction the f32 sum's drift outran) and a chunk the pass left exact are re-streamed
// exactly (row_stream) from the state before them to the chunk's end; the walk continues at
// the next chunk. The items are staged in LDS (the grouped-key array, free at this point).

constexpr int QSTAGE = (int)(sizeof(RowSmem::grp) / (sizeof(QItem)));  // items the grouped-key array holds


// The chunk heads (thread c holds chunk c's): item offsets and flags into LDS; returns the
// item count. Every thread.
__device__ __forceinline__ uint32_t chain_heads(const QHead& h, int nc, RowSmem& sm) {
    const int tid = threadIdx.x;
    uint32_t n = 0;
    if (tid < nc) {
        sm.cflag[tid] = h.flags;
        n = (h.flags & QF_EXACT) ? 1u : h.nwin + 1u;
    }
    uint32_t tot;
    const uint32_t pre = block_excl_scan<uint32_t>(n, sm.wu, tot);
    if (tid < nc) sm.coff[tid] = pre;
    if (tid == 0) sm.coff[nc] = tot;
    __syncthreads();
    return tot;
}

// Largest chunk c in [lo, hi) with coff[c] <= g.
__device__ __forceinline__ int chunk_of(const RowSmem& sm, int lo, int hi, uint32_t g) {
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (sm.coff[mid] <= g) lo = mid;
        else hi = mid;
    }
    return lo;
}

struct ChainIO {
    float s;        // the running sum at item `next`
    uint32_t next;  // the item to continue at
    uint32_t lo, hi;  // out: elements to re-stream exactly from s (lo == hi: none)
};

// Walks the items from io.next until all are done (lo == hi) or a range must be re-streamed.
// Every thread calls it.
__device__ __forceinline__ ChainIO chain_walk(const QItem* items, uint32_t qstride, int32_t nc, uint32_t chunk, uint32_t V,
                                           uint32_t total, ChainIO io, uint64_t* tr) {
    RowSmem& sm = g_sm;
    const int tid = threadIdx.x;
    QItem* const stage = reinterpret_cast<QItem*>(sm.grp);
    items = rflp(items);
    qstride = (uint32_t)rfli((int32_t)qstride);
    tr = rflp(tr);
    nc = rfli(nc);
    chunk = (uint32_t)rfli((int32_t)chunk);
    V = (uint32_t)rfli((int32_t)V);
    total = (uint32_t)rfli((int32_t)total);
    float s = rflf(io.s);
    uint32_t next = (uint32_t)rfli((int32_t)io.next);
    while (next < total) {
        // stage the chunks from the one holding `next` while their items fit
        const int sc0 = chunk_of(sm, 0, nc, next);
        const uint32_t base = sm.coff[sc0];
        int sc1 = chunk_of(sm, sc0, nc + 1, base + (uint32_t)QSTAGE);
        if (sc1 <= sc0) sc1 = sc0 + 1;
        const uint32_t n = sm.coff[sc1] - base;
        constexpr int PER = QSTAGE / BLOCK;
        QItem v[PER];
#pragma unroll
        for (int r = 0; r < PER; r++) {
            const uint32_t g = (uint32_t)(r * BLOCK + tid);
            if (g < n) {
                const int c = chunk_of(sm, sc0, sc1, base + g);
                if (sm.cflag[c] & QF_EXACT) {
                    v[r] = QItem{QI_EXACT, 0.0f, 0u, (int32_t)(((uint32_t)c << 16))};
                } else {
                    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
                    const u32x4 it = *(const BFI_GLB u32x4*)(items + (int64_t)c * qstride + (base + g - sm.coff[c]));
                    v[r] = QItem{it.x, __uint_as_float(it.y), it.z, (int32_t)(((uint32_t)c << 16) | (it.w & 0xFFFFu))};
                }
            }
        }
#pragma unroll
        for (int r = 0; r < PER; r++) {
            const uint32_t g = (uint32_t)(r * BLOCK + tid);
            if (g < n) stage[g] = v[r];
        }
        __syncthreads();
        if (tr && tid == 0 && !gl(tr)[12]) gl(tr)[12] = wall_clock64();  // diagnostics: staged
        if (wave_id() == 0) {
            const int lane = lane_id();
            const SumState st0 = sum_state(s);
            uint32_t m = st0.m;
            int32_t ue = st0.ue;
            const uint32_t hit = chain_run([&](uint32_t j) { return stage[j]; }, next - base, n, V, m, ue);
            uint32_t flo = 0, fhi = 0, fnext = 0, fb = 0;
            if (hit < n) {
                // re-stream from the start of this item's run (after the previous window of
                // its chunk, else the chunk's start) to the chunk's end
                const QItem hi = stage[hit];
                const uint32_t c = item_chunk((uint32_t)hi.ue);
                if (tr && lane == 0) {  // diagnostics: why the walk left the summaries
                    const int sh = hi.id == QI_EXACT ? 0 : (item_ue((uint32_t)hi.ue) != ue ? 16 : 32);
                    gl(tr)[14] = gl(tr)[14] + (1ull << sh);
                    gl(tr)[13] = ((uint64_t)c << 48) | ((uint64_t)(hit - sm.coff[c] + base) << 32) |
                                ((uint64_t)(item_ue((uint32_t)hi.ue) & 0xFFFF) << 16) | (uint64_t)(ue & 0xFFFF);
                    gl(tr)[12] = ((uint64_t)hi.q << 32) | m;
                }
                uint32_t lo = c * chunk;
                if (hi.id != QI_EXACT && hit > 0) {
                    const QItem pv = stage[hit - 1];
                    if (item_chunk((uint32_t)pv.ue) == c && pv.id < V) lo = pv.id + 1u;
                }
                flo = lo;
                fhi = min((c + 1u) * chunk, V);
                fnext = sm.coff[c + 1];
                fb = 1;
            }
            if (tr && lane == 0 && !gl(tr)[13]) gl(tr)[13] = wall_clock64();  // diagnostics: walked
            if (lane == 0) {
                sm.mf[MF_S] = state_value(m, ue);
                sm.misc[MS_CLO] = flo;
                sm.misc[MS_CHI] = fhi;
                sm.misc[MS_CNEXT] = fb ? fnext : base + n;
            }
        }
        __syncthreads();
        s = sm.mf[MF_S];
        const uint32_t flo = sm.misc[MS_CLO], fhi = sm.misc[MS_CHI];
        next = sm.misc[MS_CNEXT];
        __syncthreads();
        if (fhi > flo) return ChainIO{s, next, flo, fhi};  // (an empty range needs no stream)
    }
    return ChainIO{s, next, 0u, 0u};
}

// ---- the row kernel ----------------------------------------------------------------------

constexpr uint32_t LINF = 0xFFFFFFFFu;

// Phase timestamps of a row (diagnostics): words [n_rows * n_chunks * 8 + row * 16 + i].
#define BFI_RTRACE(a, C, i)                                                                             \
    do {                                                                                                \
        if ((a).trace && threadIdx.x == 0)                                                              \
            (a).trace[(int64_t)(a).n_rows * (a).n_chunks * 8 + (int64_t)(C).row * 16 + (i)] = wall_clock64(); \
    } while (0)

// The exact probability of element id (its logit loaded, masked and penalized).
template <bool BF16>
__device__ __forceinline__ float exact_x_p(const KArgs& a, const HistTabs& T, const RowCtx& C, uint32_t id, float M,
                                           float S) {
    const float x = elem_x<BF16>(a, T, C, id);
    return x > -__builtin_inff() ? exact_value(x, C.T, C.rT, C.fast_div, M, S, 1) : 0.0f;
}

// The same without the history tables: the block counts id's occurrences in the history
// (sample.rs:345-367 penalize a history id once per occurrence count). Every thread.
template <bool BF16>
__device__ __forceinline__ float scan_x_p(const KArgs& a, RowSmem& sm, const RowCtx& C, uint32_t id, float M,
                                          float S) {
    uint32_t c = 0;
    if (C.pen_on) {
        const int64_t H = C.h.size();
        for (int64_t j = threadIdx.x; j < H; j += BLOCK) c += C.h.at(j) == id ? 1u : 0u;
        c = block_sum_u(c, sm.wu);
    }
    const float l = load_logit<BF16>(a, C.row, id);
    const bool allowed = !C.mrow || ((C.mrow[id >> 5] >> (id & 31)) & 1u);
    float x = allowed ? l : -__builtin_inff();
    if (c) x = penalize(x, c, C.pen);
    return x > -__builtin_inff() ? exact_value(x, C.T, C.rT, C.fast_div, M, S, 1) : 0.0f;
}

template <bool BF16>
__device__ __forceinline__ StreamArgs stream_args(const KArgs& a, const RowCtx& C, const HistTabs& T, float M) {
    StreamArgs A;
    A.logits = (const char*)a.logits + (int64_t)C.row * a.row_stride * (BF16 ? 2 : 4);
    A.mrow = C.mrow;
    A.hbm = C.pen_on ? T.bm : nullptr;
    A.hpre = T.pre;
    A.hcnt = T.cnt;
    A.hbase = C.h.base;
    A.hext = C.h.extra;
    A.hnb = C.h.nbase;
    A.hnx = C.h.nextra;
    A.spill = a.spill + (int64_t)C.row * 4 * a.V;
    A.trace = a.trace ? a.trace + (int64_t)a.n_rows * a.n_chunks * 8 + (int64_t)C.row * 16 : nullptr;
    A.V = (uint32_t)a.V;
    A.lo = 0u;
    A.hi = (uint32_t)a.V;
    A.s0 = 0.0f;
    A.vec_ok = a.vec_ok;
    A.hdense = T.dense ? 1 : 0;
    A.fast_div = C.fast_div ? 1 : 0;
    A.T = C.T;
    A.rT = C.rT;
    A.rTl = C.rTl;
    A.rp = C.pen.rp;
    A.pp = C.pen.pp;
    A.fp = C.pen.fp;
    A.rep_on = C.pen.rep_on;
    A.pres_on = C.pen.pres_on;
    A.freq_on = C.pen.freq_on;
    A.M = M;
    A.S = 0.0f;
    A.th = __builtin_inff();
    A.excl = -1;
    A.kind = 0;
    A.gather = 0;
    A.gth = 0.0f;
    return A;
}

// The bucket a bucketed walk toward threshold r can start at: the last bucket b <= bmax whose
// recorded running state lies below r (0 when none, or for a small list). Every thread.
__device__ __forceinline__ uint32_t walk_from(const ListInfo& L, float r, uint32_t bmax, RowSmem& sm) {
    if (L.small) return 0u;
    uint32_t best = 0u;
    for (uint32_t b = (uint32_t)threadIdx.x; b <= bmax && b < L.nb; b += BLOCK) {
        const uint32_t x = sm.bsx[b];
        if (x && state_value(sm.bsm[b], (int32_t)(x & 1023u) - 512) < r) best = max(best, b);
    }
    return 0xFFFFFFFFu - block_min_u(0xFFFFFFFFu - best, sm.wu);
}

// The first index i < n with cum[i] >= r (n when none); cum is non-decreasing (a running sum
// of non-negative terms). Wave 0 searches in two rounds of 64 probes; every thread gets it.
__device__ __forceinline__ uint32_t first_ge(const float* cum, uint32_t n, float r, RowSmem& sm) {
    if (wave_id() == 0) {
        const uint32_t lane = (uint32_t)lane_id();
        const uint32_t seg = (n + WAVE - 1) / WAVE;  // segment length (n <= 64 * 64)
        const uint32_t e = min((lane + 1) * seg, n);  // this lane's segment end
        const uint64_t hit = __ballot(e > lane * seg && cum[e - 1] >= r);
        uint32_t res = n;
        if (hit) {
            const uint32_t s0 = (uint32_t)(__ffsll((unsigned long long)hit) - 1) * seg;
            const uint32_t j = s0 + lane;
            const uint64_t h2 = __ballot(lane < seg && j < n && cum[j] >= r);
            res = s0 + (uint32_t)(__ffsll((unsigned long long)h2) - 1);
        }
        if (lane == 0) sm.misc[MS_STOP] = res;
    }
    __syncthreads();
    const uint32_t res = sm.misc[MS_STOP];
    __syncthreads();
    return res;
}

template <bool BF16>
__device__ __forceinline__ void row_main(const KArgs& a, RowSmem& sm, const int row) {
    const int tid = threadIdx.x;
    const RowCtx C = make_ctx(a, row);
    const int nc = a.n_chunks;
    // issued first, beside the row's other loads: the quantizing pass's chunk heads and, for a
    // short list (one entry a thread), its gathered candidates (both only read on its path)
    const uint32_t ncand = ld_uniform(a.rowcnt + row);
    const bool pf = ncand <= (uint32_t)BLOCK;
    uint64_t pfe = 0;
    if (pf && (uint32_t)tid < ncand) pfe = a.spill[(int64_t)row * 4 * a.V + tid];
    QHead hd{0u, 0u};
    if (tid < nc) hd = a.qhead[(int64_t)row * nc + tid];
    if (!C.active) return;  // a verify row past its draft
    const uint32_t V = (uint32_t)a.V;
    BFI_RTRACE(a, C, 0);
    // 1. the row results of the streaming pass: maximum, argmax keys, candidate bound
    const RowInfo& RI = a.rinfo[row];
    float M = ld_uniform(&RI.M);
    const float th = ld_uniform(&RI.th);
    uint64_t gk = ld_uniform(&RI.gk);
    const uint64_t rk = ld_uniform(&RI.rk);
    const uint32_t raw_tok = rk ? argmax_of_key(rk).i : 0u;  // min-p fallback (sample.rs:415-422)
    // the history tables, built when a stream or a lookup needs them
    HistTabs T{nullptr, nullptr, nullptr, false};
    bool tabs = false;
    BFI_RTRACE(a, C, 1);
    if (C.pen_hash) {  // the streaming pass left the penalties out: the maximum again
        T = build_hist_tabs(a, sm, C);
        tabs = true;
        const ArgMax am = row_max<BF16>(stream_args<BF16>(a, C, T, 0.0f));
        M = C.greedy ? am.v : div_T(am.v, C);
        gk = argmax_key(am.v, am.i);
    }
    BFI_RTRACE(a, C, 2);
    if (C.greedy) {  // sample.rs:369-371
        const ArgMax am = argmax_of_key(gk);
        finish_token(a, sm, C, am.v > -__builtin_inff() ? am.i : 0u);
        return;
    }
    const uint32_t Lk = C.kmode ? (uint32_t)C.k : V;
    if (!(M > -__builtin_inff())) {
        // every logit masked: exp(-inf - -inf) is NaN for all, so no cut applies, min-p keeps
        // nothing (argmax of -infs = 0), and the draw's `r <= cum` never holds: last id.
        put_stats(a, C, M, __builtin_nanf(""), __builtin_nanf(""), 0.0f);
        if (C.mmode) {
            finish_token(a, sm, C, 0u);
            return;
        }
        target_weights(a, C, Lk, 0);
        if (!C.judged) {
            row_emit(a, sm, C, Lk - 1, 1u);
        } else {
            const bool dk = C.draft < Lk;
            const uint32_t nres = Lk - (dk ? 1u : 0u);
            if (nres == 0) row_emit(a, sm, C, C.draft, 1u);
            else row_emit(a, sm, C, (dk && C.draft == Lk - 1) ? Lk - 2 : Lk - 1, 0u);
        }
        return;
    }
    const bool sorted = C.kmode || C.pmode;
    const bool list_mode = sorted || C.mmode;
    const float gth = th - (0x1p-8f + (fabsf(M) * 12.0f + 200.0f) * 0x1p-24f);
    BFI_RTRACE(a, C, 3);
    // 2. the normalizer (sample.rs:381-386) and the candidate list
    float S;
    uint32_t N = 0;
    bool listpf = false;  // the list's entries are in sm.list (the quantizing pass's, prefetched)
    if (quant_row(C, M)) {
        // the quantizing pass's chunk summaries, chained; it gathered the candidates
        const uint32_t total = chain_heads(hd, nc, sm);
        // (the list array is free until the list is built)
        listpf = pf && list_mode;
        if (listpf && (uint32_t)tid < ncand) sm.list[tid] = pfe;
        BFI_RTRACE(a, C, 10);
        ChainIO io{0.0f, 0u, 0u, 0u};
        uint32_t nfb = 0;
        for (;;) {
            io = chain_walk(a.qitem + (int64_t)row * nc * (a.qcap + 1), (uint32_t)(a.qcap + 1), nc,
                            (uint32_t)a.chunk, V, total, io,
                            a.trace ? a.trace + (int64_t)a.n_rows * nc * 8 + (int64_t)row * 16 : nullptr);
            if (io.hi <= io.lo) {
                if (io.next >= total) break;
                continue;
            }
            if (!tabs) {
                T = build_hist_tabs(a, sm, C);
                tabs = true;
            }
            StreamArgs fb = stream_args<BF16>(a, C, T, M);
            fb.lo = io.lo;
            fb.hi = io.hi;
            fb.s0 = io.s;
            io.s = row_stream<BF16>(fb).cum;
            nfb++;
            __syncthreads();
        }
        S = io.s;
        BFI_RTRACE(a, C, 11);
        if (a.trace && tid == 0) a.trace[(int64_t)a.n_rows * nc * 8 + (int64_t)row * 16 + 9] = nfb;
        N = list_mode ? ncand : 0u;
    } else {
        // the whole row streamed exactly, gathering the candidates on the way
        if (!tabs) {
            T = build_hist_tabs(a, sm, C);
            tabs = true;
        }
        if (tid == 0) sm.misc[MS_N] = 0u;
        __syncthreads();
        StreamArgs cfg = stream_args<BF16>(a, C, T, M);
        cfg.gather = list_mode ? 1 : 0;
        cfg.gth = gth;
        S = row_stream<BF16>(cfg).cum;
        __syncthreads();
        N = sm.misc[MS_N];
    }
    BFI_RTRACE(a, C, 4);
    if (a.trace && tid == 0) a.trace[(int64_t)a.n_rows * nc * 8 + (int64_t)row * 16 + 15] = N;
    uint64_t* const gscr = a.spill + (int64_t)row * 4 * a.V + 2 * (int64_t)a.V;  // the row's sort scratch
    bool exhaustive = !(th > -__builtin_inff());
    const float p1 = exact_p(1.0f, S);  // the largest probability (the maximum's e is 1)
    if (sorted) {
        for (int attempt = 0; attempt < 2; attempt++) {
            const float p_lo = exhaustive ? 0.0f : (float)(exp2((double)th) / (double)S * (1.0 + 0x1p-20));
            const ListInfo L = build_list(a, sm, C, N, M, S, p_lo, false, listpf && attempt == 0);
            if (!L.small) bucket_units(L, sm, 0ull);
            BFI_RTRACE(a, C, 5);
            // top-p (sample.rs:397-409); a sampled row's walks over a small list keep the
            // running sum after each element, from which the kept sum and the draw are read
            float* const cum = C.judged ? nullptr : L.cum;
            uint32_t ncum = 0;  // elements with a kept running sum
            uint32_t Lp = Lk;
            WalkOut o1{0.0f, 0u, 0ull, 0};
            if (C.pmode) {
                o1 = walk(L, C.top_p, Lk, 0ull, 0, gscr, cum, true);
                if (cum) ncum = o1.how ? o1.rank + 1 : o1.rank;
                if (o1.how == 1) Lp = o1.rank + 1;
                else if (o1.how == 0 && !exhaustive) Lp = LINF;
            }
            // min-p (sample.rs:411-424): thresh = min_p * max p, kept: p >= thresh
            uint32_t Lm = Lp;
            if (C.mmode) {
                const float thresh = C.min_p * key_p(L.kmax, false);
                if (thresh > 0.0f) {
                    uint32_t cnt = 0;
                    for (uint32_t j = tid; j < L.n; j += BLOCK) cnt += key_p(L.G[j], false) >= thresh ? 1u : 0u;
                    cnt = block_sum_u(cnt, sm.wu);
                    Lm = min(Lp, cnt);
                }
            }
            const uint32_t Lfin = min(Lp, Lm);
            BFI_RTRACE(a, C, 6);
            if (C.mmode && Lfin == 0) {
                put_stats(a, C, M, S, 0.0f, 2.0f);
                finish_token(a, sm, C, raw_tok);
                return;
            }
            if (Lfin == LINF || (Lfin > L.n && !exhaustive)) {  // the list does not reach the cut
                exhaustive = true;
                if (!tabs) {
                    T = build_hist_tabs(a, sm, C);
                    tabs = true;
                }
                if (tid == 0) sm.misc[MS_N] = 0u;
                __syncthreads();
                StreamArgs all = stream_args<BF16>(a, C, T, M);
                all.gather = 1;
                all.gth = -__builtin_inff();
                (void)row_stream<BF16>(all);
                __syncthreads();
                N = sm.misc[MS_N];
                continue;
            }
            const uint32_t npos = min(Lfin, L.n);  // kept elements with p > 0
            // the kept sum (sample.rs:313)
            float sum;
            uint64_t klast;
            if (C.pmode && o1.how == 1 && Lfin == Lp) {
                sum = o1.cum;
                klast = o1.key;
            } else if (cum && npos == Lfin && Lfin <= ncum) {
                sum = cum[Lfin - 1];  // (not a judged row: klast unused)
                klast = 0ull;
            } else {
                const WalkOut o2 = walk(L, __builtin_inff(), Lfin, 0ull, 0, gscr, cum, !C.pmode);
                sum = o2.cum;
                klast = o2.how == 2 ? o2.key : 0ull;
                if (cum) ncum = o2.how ? o2.rank + 1 : o2.rank;
            }
            put_stats(a, C, M, S, sum, 1.0f);
            BFI_RTRACE(a, C, 7);
            if (!C.judged) {  // draw (sample.rs:312-323)
                const float r = C.u * fmaxf(sum, 0.0f);
                uint32_t tok;
                if (cum && min(Lfin, L.n) <= ncum) {
                    // the first kept element whose running sum reaches r, else the Lfin-th
                    // (the walk's stop at R), else none
                    const uint32_t nk = min(Lfin, L.n);
                    const uint32_t i = first_ge(cum, nk, r, sm);
                    tok = i < nk ? key_id(L.G[i], false) : (Lfin <= L.n ? key_id(L.G[Lfin - 1], false) : 0u);
                } else {
                    const WalkOut o3 = walk(L, r, Lfin, 0ull, 0, gscr, nullptr, false, walk_from(L, r, L.nb, sm));
                    tok = o3.how ? key_id(o3.key, false) : 0u;
                }
                BFI_RTRACE(a, C, 8);
                if (a.t_kind) {
                    const uint32_t lim = (uint32_t)min((int64_t)npos, a.t_cap);
                    target_weights(a, C, Lfin, lim);
                    if (lim) list_kept(L, a.t_ids + (int64_t)row * a.t_cap, a.t_probs + (int64_t)row * a.t_cap, lim, 0, gscr);
                }
                row_emit(a, sm, C, tok, 1u);
                return;
            }
            // judge (spec.rs:83-95)
            const uint32_t d = C.draft;
            float pd = 0.0f;
            if (d < V) pd = scan_x_p<BF16>(a, sm, C, d, M, S);
            const uint64_t kd = make_key(pd, d, false);
            const bool dk = pd > 0.0f && (klast == 0ull || kd >= klast);
            const float pdk = dk ? pd : 0.0f;
            if (sum > 0.0f && C.u < exact_p(pdk, sum)) {
                row_emit(a, sm, C, d, 1u);
                return;
            }
            if (npos - (dk ? 1u : 0u) == 0u) {  // the residual has no positive weight
                row_emit(a, sm, C, d, 1u);
                return;
            }
            const uint64_t ex = dk ? kd : 0ull;
            const uint32_t Lr = Lfin - (dk ? 1u : 0u);
            // the residual's walks: the recorded states before the draft's bucket hold for the
            // residual too; the residual sum's walk records its own from there on, which the
            // residual draw then starts from
            const uint32_t bmax = dk && !L.small ? L.top - ((uint32_t)(kd >> 32) >> L.sh) : L.nb;
            const uint32_t from4 = walk_from(L, __builtin_inff(), bmax, sm);
            if (!L.small) {  // the full walk's records past the residual's start no longer hold
                for (uint32_t b = from4 + 1u + (uint32_t)tid; b < L.nb; b += BLOCK) sm.bsx[b] = 0u;
                __syncthreads();
            }
            if (ex && !L.small) bucket_units(L, sm, ex);
            const WalkOut o4 = walk(L, __builtin_inff(), Lr, ex, 0, gscr, nullptr, true, from4);
            const float r2 = C.u2 * fmaxf(o4.cum, 0.0f);
            const WalkOut o5 = walk(L, r2, Lr, ex, 0, gscr, nullptr, false, walk_from(L, r2, L.nb, sm));
            row_emit(a, sm, C, o5.how ? key_id(o5.key, false) : 0u, 0u);
            return;
        }
        return;  // not reached: the second attempt gathers every element
    }
    const float thresh = C.mmode ? C.min_p * p1 : 0.0f;
    if (C.mmode && thresh > 0.0f) {
        // min-p alone: the kept elements in index order (sample.rs:411-414)
        const ListInfo L = build_list(a, sm, C, N, M, S, thresh, true, listpf);
        if (L.n == 0) {
            put_stats(a, C, M, S, 0.0f, 2.0f);
            finish_token(a, sm, C, raw_tok);
            return;
        }
        const WalkOut o2 = walk(L, __builtin_inff(), L.n, 0ull, 1, gscr);
        const float sum = o2.cum;
        put_stats(a, C, M, S, sum, 3.0f);
        if (!C.judged) {
            const float r = C.u * fmaxf(sum, 0.0f);
            const WalkOut o3 = walk(L, r, L.n, 0ull, 1, gscr);
            if (a.t_kind) {
                const uint32_t lim = (uint32_t)min((int64_t)L.n, a.t_cap);
                target_weights(a, C, L.n, lim);
                if (lim) list_kept(L, a.t_ids + (int64_t)row * a.t_cap, a.t_probs + (int64_t)row * a.t_cap, lim, 1, gscr);
            }
            row_emit(a, sm, C, o3.how ? key_id(o3.key, true) : 0u, 1u);
            return;
        }
        const uint32_t d = C.draft;
        float pd = 0.0f;
        if (d < V) pd = scan_x_p<BF16>(a, sm, C, d, M, S);
        const bool dk = pd >= thresh && pd > 0.0f;
        const float pdk = dk ? pd : 0.0f;
        if (sum > 0.0f && C.u < exact_p(pdk, sum)) {
            row_emit(a, sm, C, d, 1u);
            return;
        }
        if (L.n - (dk ? 1u : 0u) == 0u) {
            row_emit(a, sm, C, d, 1u);
            return;
        }
        const uint64_t ex = dk ? make_key(pd, d, true) : 0ull;
        const uint32_t Lr = L.n - (dk ? 1u : 0u);
        const WalkOut o4 = walk(L, __builtin_inff(), Lr, ex, 1, gscr);
        const float r2 = C.u2 * fmaxf(o4.cum, 0.0f);
        const WalkOut o5 = walk(L, r2, Lr, ex, 1, gscr);
        row_emit(a, sm, C, o5.how ? key_id(o5.key, true) : 0u, 0u);
        return;
    }
    // no filter: the whole row in index order (sample.rs:312-323 over every element)
    if (!tabs) {
        T = build_hist_tabs(a, sm, C);
        tabs = true;
    }
    StreamArgs pc = stream_args<BF16>(a, C, T, M);
    pc.kind = 1;
    pc.S = S;
    const float sum = row_stream<BF16>(pc).cum;
    put_stats(a, C, M, S, sum, 4.0f);
    if (!C.judged) {
        StreamArgs dc = pc;
        dc.th = C.u * fmaxf(sum, 0.0f);
        const StreamOut so = row_stream<BF16>(dc);
        const uint32_t tok = so.stop >= 0 ? (uint32_t)so.stop : V - 1u;
        if (a.t_kind) {
            // the positive entries in index order, up to the cap
            uint32_t listed = 0;
            for (uint32_t b0 = 0; b0 < V; b0 += BLOCK) {
                const uint32_t id = b0 + (uint32_t)tid;
                float p = 0.0f;
                if (id < V) p = exact_x_p<BF16>(a, T, C, id, M, S);
                const bool pos = p > 0.0f;
                uint32_t tot;
                const uint32_t o = block_excl_scan<uint32_t>(pos ? 1u : 0u, sm.wu, tot);
                if (pos && (int64_t)(listed + o) < a.t_cap) {
                    a.t_ids[(int64_t)row * a.t_cap + listed + o] = id;
                    a.t_probs[(int64_t)row * a.t_cap + listed + o] = p;
                }
                listed += tot;
            }
            target_weights(a, C, V, min((int64_t)listed, a.t_cap));
        }
        row_emit(a, sm, C, tok, 1u);
        return;
    }
    const uint32_t d = C.draft;
    float pd = 0.0f;
    if (d < V) pd = exact_x_p<BF16>(a, T, C, d, M, S);
    if (sum > 0.0f && C.u < exact_p(pd, sum)) {
        row_emit(a, sm, C, d, 1u);
        return;
    }
    StreamArgs rc = pc;
    rc.excl = d < V ? (int64_t)d : -1;
    const float sres = row_stream<BF16>(rc).cum;
    if (!(sres > 0.0f)) {  // empty residual, or all of its weights 0
        row_emit(a, sm, C, d, 1u);
        return;
    }
    rc.th = C.u2 * sres;
    const StreamOut so = row_stream<BF16>(rc);
    const uint32_t last = (d == V - 1u) ? V - 2u : V - 1u;
    row_emit(a, sm, C, so.stop >= 0 ? (uint32_t)so.stop : last, 0u);
}

template <bool BF16>
__global__ __launch_bounds__(BLOCK) void k_row(KArgs a) {
    row_main<BF16>(a, g_sm, (int)blockIdx.x);
}

hipError_t launch_row(const KArgs& a, int bf16, hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
    const dim3 grid((unsigned)a.n_rows), block(BLOCK);
    if (bf16) hipExtLaunchKernelGGL((k_row<true>), grid, block, 0, stream, start, stop, 0, a);
    else hipExtLaunchKernelGGL((k_row<false>), grid, block, 0, stream, start, stop, 0, a);
    return hipGetLastError();
}

}  // namespace bfi
