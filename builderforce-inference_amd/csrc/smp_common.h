// smp_common.h — what both sampling kernels share: the per-row context (parameters,
// history view, mask), the 16-byte tile loader and an element's value (mask, penalties,
// / T) as sample.rs:331-375 computes it.
#pragma once
#include "smp_device.h"

namespace bfi {

enum { MISC_LAST = 0, MISC_N = 1, MISC_NDIST = 2, MISC_OVF = 3, MISC_HN = 7 };

// ---- per-row context -------------------------------------------------------------------

struct RowCtx {
    int row, seq, ri, dl;
    bool active, verify, judged;
    uint32_t draft;
    float u, u2;
    float T, rT, top_p, min_p;
    float rTl;  // log2(e) / T (the streaming pass's exp scale)
    bool fast_div;   // T in [2^-20, 2^20]: FMA-corrected reciprocal division is exact
    bool stream_ok;  // T in [2^-125, 2^125]: the streaming pass's bounds and terms are usable
    int32_t k;
    bool greedy, kmode, pmode, mmode;
    Pen pen;
    bool pen_on;
    // prepen: the stream pass applies the penalties (history of at most PREPEN_H ids), so
    // its chunk results and candidates are penalized; pen_hash: the select kernel keeps the
    // history in its LDS hash and corrects the chunk results itself
    bool prepen, pen_hash;
    HistView h;
    const uint32_t* mrow;
    const char* lrow;
};

// A row-uniform read of memory the kernels never write (parameters, offsets, uniforms,
// drafts): through the constant address space it becomes a scalar load, so nothing waits
// for it behind the logits' vector loads.
template <typename T>
__device__ __forceinline__ T ld_uniform(const T* p) {
    return *(const __attribute__((address_space(4))) T*)p;
}

// The history of a row (sample.rs:345-367 `prev`): its base ids, plus for spec verify the
// drafts before this row (spec.rs:137-162 appends each accepted draft). Reads only the
// row's two history offsets.
__device__ __forceinline__ HistView row_history(const KArgs& a, int row) {
    HistView h;
    const int rps = a.rows_per_seq;
    const int seq = rps > 0 ? row / rps : row;
    if (rps > 0) {
        h.extra = a.drafts + (int64_t)seq * (rps - 1);
        h.nextra = row % rps;
    } else {
        h.extra = nullptr;
        h.nextra = 0;
    }
    if (a.hist_off) {
        const int64_t o0 = ld_uniform(a.hist_off + seq), o1 = ld_uniform(a.hist_off + seq + 1);
        h.base = a.hist + o0;
        h.nbase = o1 > o0 ? o1 - o0 : 0;
    } else {
        h.base = nullptr;
        h.nbase = 0;
    }
    return h;
}

__device__ __forceinline__ RowCtx make_ctx(const KArgs& a, int row) {
    RowCtx C;
    C.row = row;
    C.verify = a.rows_per_seq > 0;
    if (C.verify) {
        int rps = a.rows_per_seq;
        C.seq = row / rps;
        C.ri = row % rps;
        int dl = ld_uniform(a.draft_len + C.seq);
        dl = dl < 0 ? 0 : (dl > rps - 1 ? rps - 1 : dl);
        C.dl = dl;
        C.active = C.ri <= dl;
        C.judged = C.ri < dl;
        const int64_t dbase = (int64_t)C.seq * (rps - 1);
        C.draft = C.judged ? ld_uniform(a.drafts + dbase + C.ri) : 0u;
        if (C.judged) {
            C.u = ld_uniform(a.u_pairs + (dbase + C.ri) * 2);
            C.u2 = ld_uniform(a.u_pairs + (dbase + C.ri) * 2 + 1);
        } else {
            C.u = ld_uniform(a.u_bonus + C.seq);
            C.u2 = 0.0f;
        }
    } else {
        C.seq = row;
        C.ri = 0;
        C.dl = 0;
        C.active = true;
        C.judged = false;
        C.draft = 0;
        C.u = a.u ? ld_uniform(a.u + row) : 0.0f;
        C.u2 = 0.0f;
    }
    C.h = row_history(a, row);
    // field by field: an aggregate copy would lose the address space
    const __attribute__((address_space(4))) uint32_t* pw =
        (const __attribute__((address_space(4))) uint32_t*)(a.params + C.seq);
    bfi_smp_row_params P;
    P.temperature = __uint_as_float(pw[0]);
    P.top_k = (int32_t)pw[1];
    P.top_p = __uint_as_float(pw[2]);
    P.min_p = __uint_as_float(pw[3]);
    P.repeat_penalty = __uint_as_float(pw[4]);
    P.presence_penalty = __uint_as_float(pw[5]);
    P.frequency_penalty = __uint_as_float(pw[6]);
    P.reserved = pw[7];
    const int64_t H = C.h.size();
    C.T = P.temperature;
    C.rT = 1.0f / P.temperature;  // IEEE, once per row
    C.rTl = C.rT * 1.44269504088896341f;
    C.fast_div = P.temperature >= 0x1p-20f && P.temperature <= 0x1p20f;
    C.stream_ok = P.temperature >= 0x1p-125f && P.temperature <= 0x1p125f;
    C.top_p = P.top_p;
    C.min_p = P.min_p;
    C.k = P.top_k;
    C.greedy = !(P.temperature > 0.0f);                    // sample.rs:369
    C.kmode = P.top_k > 0 && P.top_k < a.V;                // sample.rs:392
    C.pmode = P.top_p < 1.0f;                              // sample.rs:397
    C.mmode = P.min_p > 0.0f;                              // sample.rs:411
    C.pen.rp = P.repeat_penalty;
    C.pen.pp = P.presence_penalty;
    C.pen.fp = P.frequency_penalty;
    C.pen.rrp = 1.0f / P.repeat_penalty;  // IEEE, once per row
    C.pen.rdiv = P.repeat_penalty >= 0x1p-20f && P.repeat_penalty <= 0x1p20f;
    C.pen.rep_on = fabsf(P.repeat_penalty - 1.0f) > F32_EPS && H > 0;  // sample.rs:346
    C.pen.pres_on = P.presence_penalty != 0.0f && H > 0;               // sample.rs:360
    C.pen.freq_on = P.frequency_penalty != 0.0f && H > 0;
    C.pen_on = C.pen.rep_on || C.pen.pres_on || C.pen.freq_on;
    C.prepen = C.pen_on && H <= (int64_t)PREPEN_H && (C.greedy || C.stream_ok) && a.chunk <= CHUNK_MAX;
    C.pen_hash = C.pen_on && !C.prepen;
    C.mrow = a.mask ? a.mask + (int64_t)row * a.mask_stride : nullptr;
    const int esz = 4;  // overridden by the loader for bf16
    (void)esz;
    C.lrow = (const char*)a.logits;
    return C;
}

// Rows whose normalizer the quantizing pass summarizes (smp_quant.hip) and the row kernel
// chains: sampled rows whose penalties the streaming pass applied, whose temperature the
// estimates cover and whose maximum M (the streaming pass's) is finite. The others (and
// all-masked rows) take the row kernel's exact stream.
__device__ __forceinline__ bool quant_row(const RowCtx& C, float M) {
    return C.active && !C.greedy && !C.pen_hash && C.stream_ok && __builtin_fabsf(M) < __builtin_inff();
}

// ---- chunk loader ----------------------------------------------------------------------

template <bool BF16>
struct Elem;
template <>
struct Elem<false> {
    static constexpr int EPV = 4;
    typedef float T;
    __device__ __forceinline__ static float cvt(T v) { return v; }
};
template <>
struct Elem<true> {
    static constexpr int EPV = 8;
    typedef uint16_t T;
    __device__ __forceinline__ static float cvt(T v) { return __uint_as_float((uint32_t)v << 16); }
};

// Loads the elements thread `tid` owns in [c0, c1): vector q covers ids
// c0 + (q*BLOCK + tid)*EPV + [0, EPV). Out-of-range elements read as -inf. A full, aligned
// tile takes only unconditional 16-byte loads, so all VEC loads are in flight together.
template <bool BF16, int VEC>
__device__ __forceinline__ void unpack16(const uint4 w, float (&v)[Elem<BF16>::EPV]) {
    if (!BF16) {
        v[0] = __uint_as_float(w.x);
        v[1] = __uint_as_float(w.y);
        v[2] = __uint_as_float(w.z);
        v[3] = __uint_as_float(w.w);
    } else {
        const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
            v[2 * e] = __uint_as_float(ww[e] << 16);
            v[2 * e + 1] = __uint_as_float(ww[e] & 0xFFFF0000u);
        }
    }
}

// Vectors [Q0, Q1) of a full, aligned tile: the 16-byte loads are issued in order (q = Q0
// first), so a consumer that walks q upward waits only for the vectors it needs.
template <bool BF16, int VEC, int Q0, int Q1>
__device__ __forceinline__ void load_full_range(const KArgs& a, int row, uint32_t c0,
                                                float (&x)[VEC][Elem<BF16>::EPV]) {
    typedef typename Elem<BF16>::T T;
    const T* base = (const T*)a.logits + (int64_t)row * a.row_stride + c0 + (uint32_t)threadIdx.x * Elem<BF16>::EPV;
    uint4 w[VEC];
#pragma unroll
    for (int q = Q0; q < Q1; q++) {
        w[q] = *(const uint4*)(base + (uint32_t)(q * BLOCK) * Elem<BF16>::EPV);
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int q = Q0; q < Q1; q++) unpack16<BF16, VEC>(w[q], x[q]);
}
template <bool BF16, int VEC>
__device__ __forceinline__ void load_full_tile(const KArgs& a, int row, uint32_t c0,
                                               float (&x)[VEC][Elem<BF16>::EPV]) {
    load_full_range<BF16, VEC, 0, VEC>(a, row, c0, x);
}

template <bool BF16, int VEC>
__device__ __forceinline__ void load_tile(const KArgs& a, int row, uint32_t c0, uint32_t c1,
                                          float (&x)[VEC][Elem<BF16>::EPV]) {
    constexpr int EPV = Elem<BF16>::EPV;
    typedef typename Elem<BF16>::T T;
    const T* base = (const T*)a.logits + (int64_t)row * a.row_stride;
    const int tid = threadIdx.x;
    if (a.vec_ok && c1 - c0 == (uint32_t)(BLOCK * VEC * EPV)) {
        uint4 w[VEC];
#pragma unroll
        for (int q = 0; q < VEC; q++) w[q] = *(const uint4*)(base + c0 + (uint32_t)(q * BLOCK + tid) * EPV);
#pragma unroll
        for (int q = 0; q < VEC; q++) unpack16<BF16, VEC>(w[q], x[q]);
        return;
    }
#pragma unroll
    for (int q = 0; q < VEC; q++) {
        const uint32_t id0 = c0 + (uint32_t)(q * BLOCK + tid) * EPV;
        if (a.vec_ok && id0 + EPV <= c1) {
            unpack16<BF16, VEC>(*(const uint4*)(base + id0), x[q]);
        } else {
#pragma unroll
            for (int e = 0; e < EPV; e++)
                x[q][e] = (id0 + e < c1) ? Elem<BF16>::cvt(base[id0 + e]) : -__builtin_inff();
        }
    }
}

// x / T rounded like IEEE division (sample.rs:373-375). With r = RN(1/T), q = RN(x*r) is
// within one ulp of x/T, e = x - q*T is exact under FMA, and RN(q + e*r) is the correctly
// rounded quotient while no step underflows or overflows (Markstein's correction). This was
// checked bit-exhaustively against IEEE division over all f32 x with |x| in [2^-100, 2^100]
// for temperatures across [2^-20, 2^20]. Zeros give +-0 and infinities/NaN pass through (e
// is NaN there, and q is already the quotient). `div_ok` says whether x is in the checked
// range; other values take IEEE division.
__device__ __forceinline__ float div_T_fast(float x, const RowCtx& C) {
    const float q = x * C.rT;
    const float e = __builtin_fmaf(-q, C.T, x);
    const float s = __builtin_fmaf(e, C.rT, q);
    return e != e ? q : s;
}
__device__ __forceinline__ bool div_ok(float x) {
    const uint32_t a = __float_as_uint(x) & 0x7FFFFFFFu;
    // bad: nonzero below 2^-100, or finite at/above 2^100
    return !((a - 1u < 0x0D7FFFFFu) || (a - 0x71800000u < 0x0E000000u));
}
__device__ __forceinline__ float div_T(float x, const RowCtx& C) {
    return (C.fast_div && div_ok(x)) ? div_T_fast(x, C) : x / C.T;
}

// Value of one logit as the streaming pass sees it: masked (sample.rs:331-337), then / T
// unless greedy. Penalties are not applied here; the select kernel corrects the few
// history ids afterwards. Exact for |x| in [2^-100, 2^100] (see div_T_fast).
__device__ __forceinline__ float raw_value(const RowCtx& C, float x, bool allowed) {
    if (!allowed) return -__builtin_inff();
    return C.greedy ? x : div_T(x, C);
}
// Value with the penalties (sample.rs:345-375): mask, repeat, presence, frequency, / T.
__device__ __forceinline__ float pen_value(const RowCtx& C, float x, bool allowed, uint32_t count) {
    float v = allowed ? x : -__builtin_inff();
    v = penalize(v, count, C.pen);
    return C.greedy ? v : div_T(v, C);
}

// ---- small helpers ---------------------------------------------------------------------

// The streaming pass works on masked logits x. Its exp-sum term of x in a chunk whose
// largest masked logit is xm is 2^((x - xm) * (log2(e) / T)): x - xm is exact near the
// maximum (Sterbenz), so the large terms carry only the rounding of the scale and of
// v_exp_f32; the select kernel recomputes the terms of history ids with the same
// expression. Exact values x / T (div_T) are computed only where they are kept.
__device__ __forceinline__ float stream_term(const RowCtx& C, float x, float xm) {
    return __builtin_amdgcn_exp2f((x - xm) * C.rTl);
}
// A bound t on exact values x / T as a bound on masked logits: every x whose exact value
// is >= t is >= x_bound(t) (the product t * T, lowered by 2^-20 relative).
__device__ __forceinline__ float x_bound(const RowCtx& C, float t) {
    const float b = t * C.T;
    const float w = b - (fabsf(b) * 0x1p-20f + 0x1p-126f);
    return w == w ? w : b;  // +-inf stays
}

// Finite masked logits of a tile that are >= xth.
template <bool BF16, int VEC>
__device__ __forceinline__ uint32_t tile_count_ge(const float (&x)[VEC][Elem<BF16>::EPV], float xth) {
    constexpr int EPV = Elem<BF16>::EPV;
    uint32_t c = 0;
#pragma unroll
    for (int q = 0; q < VEC; q++)
#pragma unroll
        for (int e = 0; e < EPV; e++) c += (x[q][e] >= xth && x[q][e] > -__builtin_inff()) ? 1u : 0u;
    return c;
}

// The fixed-point mass of value s in a row with maximum M (the radix select's unit: its cuts
// and draws compare sums of these integers, so only their consistency matters, not the
// last ulp of the exponential; the hardware exp2 keeps the row passes short).
// It equals floor(e * scale) for scale = 2^b, 32 <= b <= 62, in f32 arithmetic: t = e * 2^(b-32)
// is exact (a power-of-two scaling of e <= 1), floor(t) < 2^31 is the high word, and the
// fraction t - floor(t) (exact for t >= 0) times 2^32, truncated, is the low word.
__device__ __forceinline__ uint64_t efix_of(float s, float M, double scale) {
    const float e = __builtin_amdgcn_exp2f((s - M) * 1.44269504088896341f);
    const float t = e * (float)(scale * 0x1p-32);
    const uint32_t hi = (uint32_t)t;
    const uint32_t lo = (uint32_t)(__builtin_amdgcn_fractf(t) * 0x1p32f);
    return ((uint64_t)hi << 32) | lo;
}

}  // namespace bfi
