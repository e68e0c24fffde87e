// smp_exact.h — the reference's float arithmetic, reproduced bit for bit on the device.
//
// The reference normalizes with `(l - max).exp()` and a sequential f32 sum over the whole
// vocabulary (sample.rs:377-390), cuts top-p on a sequential f32 cumsum (sample.rs:397-409)
// and draws on sequential f32 sums (sample.rs:312-323, spec.rs:84-94). Over 10^5 terms
// those sums drift from the exact sum by up to 5e-4 relative (small terms fall below half
// an ulp of the running sum and vanish), which moves a top-p cut by tens of ids. This header
// gives the pieces that let a parallel kernel return exactly the reference's f32 results:
//
//   expf_ref  — f32::exp on x86_64 Linux is glibc's expf. glibc computes it (e_expf.c) as
//               2^(k/32) * p(r) in double precision with FMA: z = x * 32/ln2, k = round(z),
//               r = z - k, table 2^(i/32), cubic polynomial. The restatement below uses the
//               same steps and constants (the table is 2^(i/32) rounded to double; the
//               polynomial coefficients are glibc's published ones) and matches the host's
//               expf on every float in [-103.97, 88.72] (exhaustive check, both signs).
//
//   Sequential sums by binades. While a running f32 sum s stays in one binade
//   [2^k, 2^(k+1)), every addition rounds to a multiple of u = 2^(k-23): adding v moves
//   s by RN(v/u) units exactly, unless v/u is a tie (then the parity of s decides) or the
//   sum leaves the binade. So a sum is an integer prefix sum of q = RN(v/u) in units of u
//   between "events" (a tie, or the step that leaves the binade, which is then done as one
//   real f32 addition). The state of a sum is (m, ue): s = m * 2^ue with m < 2^24.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bfi {

// ---- glibc expf ---------------------------------------------------------------------------

// 2^(i/32) rounded to double, minus i << 47 (so adding k << 47 scales by 2^(k/32) for the
// integer part of k/32).
__constant__ const uint64_t EXP2_32[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

// glibc's main path for x in [-103.97, 88.72]: 2^(k/32) from the table `tab` (EXP2_32, or a
// copy of it in LDS) times the cubic in r, in double precision with FMA, rounded to float.
__device__ __forceinline__ float expf_core(float x, const uint64_t* tab) {
    const double InvLn2N = 0x1.71547652b82fep+0 * 32.0;
    const double SHIFT = 0x1.8p+52;
    const double C0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    const double C1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    const double C2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const double xd = (double)x;
    double kd = __builtin_fma(InvLn2N, xd, SHIFT);
    const uint64_t ki = (uint64_t)__double_as_longlong(kd);
    kd -= SHIFT;
    const double r = __builtin_fma(InvLn2N, xd, -kd);
    const uint64_t t = tab[ki & 31u] + (ki << 47);
    const double s = __longlong_as_double((long long)t);
    const double z = __builtin_fma(C0, r, C1);
    const double r2 = r * r;
    double y = __builtin_fma(C2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    y = y * s;
    return (float)y;
}

// expf(x) exactly as glibc returns it. Table entry by a per-lane index: read from the
// constant table through a generic load (it stays in the scalar/vector caches).
__device__ __forceinline__ float expf_ref(float x) {
    const uint32_t ax = __float_as_uint(x) & 0x7FFFFFFFu;
    if (ax >= 0x42B00000u) {                 // |x| >= 88 or not finite
        if (x != x) return x + x;            // NaN
        if (x == -__builtin_inff()) return 0.0f;
        if (x == __builtin_inff()) return x;
        if (x > 0x1.62e42ep6f) return __builtin_inff();
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    return expf_core(x, EXP2_32);
}

// expf(x) for x <= 0 as glibc returns it, without branches: below its underflow bound
// (-0x1.9fe368p6, where glibc returns 0), at -inf and at NaN (a masked element's x) the
// result is 0; every other x takes glibc's main path. The main path runs for every x (its
// table index is masked to 0..31, so any input is safe) and the selection discards its
// value outside the range. `tab`: EXP2_32 or a copy in LDS.
__device__ __forceinline__ float expf_nonpos(float x, const uint64_t* tab) {
    const float y = expf_core(x, tab);
    return x >= -0x1.9fe368p6f ? y : 0.0f;
}

// ---- sequential f32 sums by binades -------------------------------------------------------

constexpr uint32_t M_TOP = 1u << 24;  // a binade holds mantissas m < 2^24 (in units of u)

// The state (m, ue) of a non-negative finite f32 s: s = m * 2^ue exactly; for normal s,
// m in [2^23, 2^24) and u = 2^ue is the spacing of floats in s's binade; subnormal s (and
// 0) share the spacing 2^-149 of the lowest binade.
struct SumState {
    uint32_t m;
    int32_t ue;
};
__device__ __forceinline__ SumState sum_state(float s) {
    const uint32_t b = __float_as_uint(s);
    const uint32_t E = b >> 23;
    SumState st;
    st.m = (b & 0x7FFFFFu) | (E ? 0x800000u : 0u);
    st.ue = (int32_t)(E ? E : 1u) - 150;
    return st;
}
// The float m * 2^ue (exact for m < 2^24 and the ue of a state).
__device__ __forceinline__ float state_value(uint32_t m, int32_t ue) { return __builtin_ldexpf((float)m, ue); }

// v * 2^-ue, exact (a power-of-two scaling; saturates to +inf, which counts as an event).
__device__ __forceinline__ float units_of(float v, int32_t ue) { return __builtin_ldexpf(v, -ue); }

// RN(t) as a saturating integer count; t >= 0.
__device__ __forceinline__ uint32_t quant_units(float t) {
    const float q = __builtin_rintf(t);
    return q < 4294967040.0f ? (uint32_t)q : 0xFFFFFFFFu;
}
// t is a tie of RN (fraction exactly 1/2): the parity of the running sum decides.
__device__ __forceinline__ bool quant_tie(float t) { return t - __builtin_floorf(t) == 0.5f && t < 16777216.0f; }

__device__ __forceinline__ uint32_t sat_add(uint32_t a, uint32_t b) { return __builtin_elementwise_add_sat(a, b); }

// Smallest unit count N with N * 2^ue >= th (th > 0), saturating.
__device__ __forceinline__ uint32_t thresh_units(float th, int32_t ue) {
    const float c = __builtin_ceilf(__builtin_ldexpf(th, -ue));
    return c < 4294967040.0f ? (uint32_t)c : 0xFFFFFFFFu;
}

}  // namespace bfi
