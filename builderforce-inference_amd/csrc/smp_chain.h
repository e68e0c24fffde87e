// smp_chain.h — the normalizer's chain over the quantizing pass's chunk summaries, one wave.
//
// The items of a row (smp_quant.hip) in index order: the run of certain elements before each
// window element, the element, and each chunk's tail run. From the running sum's exact state
// (m, ue) (smp_exact.h), 64 items at a time: a run adds its units in one step when the state
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

// Walks items [i, n) (ld(j) loads item j; every lane calls it with its own j) from the exact
// state (m, ue). Returns n when all are added, else the index of the first item the walk
// cannot take (a chunk left exact, or a run whose check fails), with (m, ue) the state
// before that item's run. Wave-uniform; every lane of the wave calls it.
template <class LD>
__device__ __forceinline__ uint32_t chain_run(LD ld, uint32_t i, uint32_t n, uint32_t V, uint32_t& m, int32_t& ue) {
    const int lane = lane_id();
    while (i < n) {
        const uint32_t j = i + (uint32_t)lane;
        QItem it = QItem{QI_NONE, 0.0f, 0u, (int32_t)0x0000FC00u};  // past the end: adds nothing
        if (j < n) it = ld(j);
        const int32_t rue = item_ue((uint32_t)it.ue);
        const bool rok = it.q == 0u ? ue >= rue : rue == ue;
        const bool el = it.id < V;
        const float t = units_of(it.e, ue);
        const uint32_t qe = el ? quant_units(t) : 0u;
        const bool tie = el && quant_tie(t);
        const uint32_t qi = wave_scan_incl(sat_add(rok ? it.q : 0u, qe), 0u,
                                           [](uint32_t x, uint32_t y) { return sat_add(x, y); });
        const uint32_t run = sat_add(m, qi);
        const bool ev = it.id == QI_EXACT || it.id == QI_SET || !rok || tie || run >= M_TOP;
        const uint64_t bal = __ballot(ev);
        if (!bal) {
            m = lane63(run);
            i += WAVE;
            continue;
        }
        const int js = __ffsll((unsigned long long)bal) - 1;
        const uint32_t before = js ? (uint32_t)__builtin_amdgcn_readlane((int)run, js - 1) : m;
        const uint32_t id_s = (uint32_t)__builtin_amdgcn_readlane((int)it.id, js);
        const uint32_t q_s = (uint32_t)__builtin_amdgcn_readlane((int)it.q, js);
        const int32_t rue_s = item_ue((uint32_t)__builtin_amdgcn_readlane(it.ue, js));
        const float e_s = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(it.e), js));
        m = before;
        if (id_s == QI_SET) {  // (the row's first item: nothing before it)
            const SumState st = sum_state(e_s);
            m = st.m;
            ue = st.ue;
            i += (uint32_t)js + 1u;
            continue;
        }
        const bool rok_s = q_s == 0u ? ue >= rue_s : rue_s == ue;
        if (id_s == QI_EXACT || !rok_s || (uint64_t)before + q_s >= (uint64_t)M_TOP) return i + (uint32_t)js;
        // the element, added as the reference does
        const float sn = state_value(before + q_s, ue) + e_s;
        const SumState st = sum_state(sn);
        m = st.m;
        ue = st.ue;
        i += (uint32_t)js + 1u;
    }
    return n;
}

}  // namespace bfi
