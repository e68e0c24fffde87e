// smp_chain.h — the normalizer's chain over the quantizing pass's chunk summaries, one wave.
//
// The items of a row (smp_quant.hip) in index order: the run of certain elements before each
// window element, the element, and each chunk's tail run. From the running sum's exact state
// (m, ue) (smp_exact.h), 256 items a step: a run adds its units in one step when the state
// lies in the run's binade (a zero run: in its binade or above) and stays below the binade's
// top; a window element adds RN(e / u) units unless it is a tie or leaves the binade, in
// which case it is one real f32 addition (the reference's own rounding of that step,
// sample.rs:381-386). Both kernels use it: the quantizing pass for a row's first chunk (its
// start, 0, is known there) and the row kernel for the rest.
#pragma once
#include "smp_device.h"
#include "smp_exact.h"

namespace bfi {

constexpr uint32_t QI_EXACT = 0xFFFFFFFEu;  // a chunk the quantizing pass left exact
constexpr uint32_t QI_SET = 0xFFFFFFFDu;    // the running sum becomes e (a row's first item)

// An item's run binade: the low 16 bits of its ue word, sign-extended (the row kernel keeps
// the chunk index in the high 16 bits of the staged copy).
__device__ __forceinline__ int32_t item_ue(uint32_t w) { return (int32_t)(int16_t)(w & 0xFFFFu); }
__device__ __forceinline__ uint32_t item_chunk(uint32_t w) { return w >> 16; }

// Walks items [i, n) (ld(j) loads item j, j < n; every lane calls it with its own j) from the
// exact state (m, ue). Returns n when all are added, else the index of the first item the
// walk cannot take (a chunk left exact, or a run whose check fails), with (m, ue) the state
// before that item's run. Each lane takes K consecutive items a step. Wave-uniform; every
// lane of the wave calls it.
template <int K = 1, class LD>
__device__ __forceinline__ uint32_t chain_run(LD ld, uint32_t i, uint32_t n, uint32_t V, uint32_t& m, int32_t& ue) {
    static_assert(K >= 1 && K <= 4, "a step's units stay below 2^32");
    const int lane = lane_id();
    while (i < n) {
        const uint32_t j0 = i + (uint32_t)lane * K;
        QItem it[K];
        uint32_t pre[K + 1];  // the lane's units before item k (each item's capped below 2^24)
        uint32_t evk = 0;     // bit k: item k stops the step whatever the sum before it
        pre[0] = 0u;
#pragma unroll
        for (int k = 0; k < K; k++) {
            const uint32_t j = j0 + (uint32_t)k;
            QItem x = ld(j < n ? j : n - 1u);
            if (j >= n) x = QItem{QI_NONE, 0.0f, 0u, (int32_t)0x0000FC00u};  // past the end: adds nothing
            it[k] = x;
            const int32_t rue = item_ue((uint32_t)x.ue);
            const bool rok = x.q == 0u ? ue >= rue : rue == ue;
            const bool el = x.id < V;
            const float t = units_of(x.e, ue);
            const float r = __builtin_rintf(t);
            const uint32_t qe = el ? quant_units(t) : 0u;
            const bool tie = el && __builtin_fabsf(t - r) == 0.5f && t < 16777216.0f;
            const uint32_t v = sat_add(rok ? x.q : 0u, qe);
            pre[k + 1] = pre[k] + min(v, M_TOP - 1u);
            evk |= (x.id == QI_EXACT || x.id == QI_SET || !rok || tie || v >= M_TOP) ? 1u << k : 0u;
        }
        const uint32_t qi = wave_scan_incl(pre[K], 0u, [](uint32_t x, uint32_t y) { return x + y; });
        const uint32_t base = sat_add(m, qi - pre[K]);  // the state before the lane's items
        // the lane's first item that stops the step: flagged, or the sum after it reaches the top
        int kf = K;
#pragma unroll
        for (int k = K - 1; k >= 0; k--)
            if (((evk >> k) & 1u) || sat_add(base, pre[k + 1]) >= M_TOP) kf = k;
        const uint64_t bal = __ballot(kf < K);
        if (!bal) {
            m = lane63(sat_add(m, qi));
            i += (uint32_t)(WAVE * K);
            continue;
        }
        // the item that stops the step, and the state before its run
        uint32_t b_l = base, id_l = QI_NONE, q_l = 0u, ue_l = 0u;
        float e_l = 0.0f;
#pragma unroll
        for (int k = 0; k < K; k++)
            if (k == kf) {
                b_l = sat_add(base, pre[k]);
                id_l = it[k].id;
                q_l = it[k].q;
                ue_l = (uint32_t)it[k].ue;
                e_l = it[k].e;
            }
        const int js = __ffsll((unsigned long long)bal) - 1;
        const uint32_t at = i + (uint32_t)js * K + (uint32_t)__builtin_amdgcn_readlane(kf, js);
        const uint32_t before = (uint32_t)__builtin_amdgcn_readlane((int)b_l, js);
        const uint32_t id_s = (uint32_t)__builtin_amdgcn_readlane((int)id_l, js);
        const uint32_t q_s = (uint32_t)__builtin_amdgcn_readlane((int)q_l, js);
        const int32_t rue_s = item_ue((uint32_t)__builtin_amdgcn_readlane((int)ue_l, js));
        const float e_s = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e_l), js));
        m = before;
        if (id_s == QI_SET) {  // (the row's first item: nothing before it)
            const SumState st = sum_state(e_s);
            m = st.m;
            ue = st.ue;
            i = at + 1u;
            continue;
        }
        const bool rok_s = q_s == 0u ? ue >= rue_s : rue_s == ue;
        if (id_s == QI_EXACT || !rok_s || (uint64_t)before + q_s >= (uint64_t)M_TOP) return at;
        // the element, added as the reference does
        const float sn = state_value(before + q_s, ue) + e_s;
        const SumState st = sum_state(sn);
        m = st.m;
        ue = st.ue;
        i = at + 1u;
    }
    return n;
}

}  // namespace bfi
