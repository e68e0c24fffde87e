// smp_device.h — device building blocks of the gfx950 sampler kernel.
//
// Wave64 reductions/scans (DPP-lowered shuffles), block (256-thread, 4-wave) reductions
// through LDS, the order-preserving float key, and the penalty/mask transform that restates
// crates/bfi-runtime/src/sample.rs:331-375 element by element.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/bfi_sampler.h"

namespace bfi {

// Threads per workgroup: each kernel's translation unit may set BFI_BLOCK before including
// this header (the streaming kernel uses 256 = 4 wave64s).
#ifndef BFI_BLOCK
#define BFI_BLOCK 256
#endif
constexpr int BLOCK = BFI_BLOCK;
constexpr int WAVE = 64;
constexpr int NWAVE = BLOCK / WAVE;
constexpr int CHUNK_MAX = 8192;        // logits elements per workgroup (stream phase)
constexpr int NCMAX = 256;             // chunks per row
constexpr int PREPEN_H = 1024;         // histories up to this length are applied by the stream pass
constexpr int GDCAP = 4096;            // distinct history ids counted per row (global tables)
constexpr int HBINS = 128;             // bins of the stream pass's per-chunk value histogram
constexpr int HBIN_PER_LOG2 = 4;       // bins per log2-unit below the chunk maximum (32 units)
constexpr float F32_EPS = 1.1920928955078125e-07f;  // f32::EPSILON

// Per (row, chunk) result of the streaming pass over the values s = x / T of the masked
// logits x (greedy: x itself), penalized when the row's context says prepen (else the
// row kernel applies the history itself).
struct ChunkPart {
    float m;          // max of s (exact)
    uint32_t arg;     // greedy: first index attaining m
    double sum;       // approximate sum of 2^((x - xm) log2(e) / T) over the chunk
    float xm;         // max of x (the sums' and the histogram's reference point)
    float raw_m;      // rows with min_p > 1: max of the masked, un-penalized logits
    uint32_t raw_arg; // first index of that maximum (greedy rows and rows with min_p > 1)
    uint32_t pad;
};

// Per row: what the streaming pass's last workgroup of the row derives from all chunks.
struct RowInfo {
    float M;        // row maximum of s = x / T (exact; greedy rows: of x)
    float xmax;     // row maximum of the masked (penalized) logits
    float th;       // every kept element has (x / T - M) log2(e) above th, before the passes'
                    // rounding margins (-inf: any; +inf: the row keeps no list)
    float S_apx;    // approximate normalizer (sum of exp(s - M), the chunk masses)
    uint64_t gk;    // greedy rows: argmax key of the penalized values
    uint64_t rk;    // rows with min_p > 1: argmax key of the masked, un-penalized values
};

// The normalizer's running sum where a chunk starts, as the row finisher predicts it: the
// approximate mass of the chunks before it, and a lower bound the f32 sum cannot go below
// (the largest term before the chunk: a sum of non-negative terms, each step rounded to
// nearest, never falls below any of its terms).
struct QPre {
    float P;
    float lb;
};

// The quantizing pass's summary of one chunk for the normalizer's chain (smp_quant.hip).
// In index order the chunk's elements are runs of "certain" elements, all added while the
// running f32 sum stays in one binade (their sum taken in units of that binade), separated
// by "window" elements, whose binade or rounding the pass could not settle: those near a
// binade boundary of the predicted running sum, and ties. Item k holds window element k
// with its exact exp(s - M) and the run before it; the last item holds the tail run.
constexpr int QWIN = 4096;          // window elements per chunk at most (beyond: the chunk is exact)
constexpr uint32_t QF_EXACT = 1u;   // the row kernel streams this chunk exactly
constexpr uint32_t QI_NONE = 0xFFFFFFFFu;  // item id of the tail run (no element)
struct QItem {
    uint32_t id;   // the window element (QI_NONE: none)
    float e;       // its exact exp(s - M)
    uint32_t q;    // units the run before it adds (unit 2^ue)
    int32_t ue;    // the run's unit exponent (with q == 0: the largest it was checked at)
};
struct QHead {
    uint32_t nwin;   // window elements (items: nwin + 1)
    uint32_t flags;  // QF_EXACT
};

// Everything a launch needs; passed by value.
struct KArgs {
    const void* logits;
    int64_t row_stride;
    int32_t V;
    int32_t n_rows;
    int32_t n_chunks;
    int32_t chunk;  // elements per chunk
    int32_t vec_ok; // rows are 16-byte aligned: vector loads allowed
    int32_t pad0;
    const bfi_smp_row_params* params;
    const uint32_t* hist;   // penalty histories (token ids)
    const int64_t* hist_off;
    const uint32_t* mask;
    int64_t mask_stride;
    const float* u;
    uint32_t* out_tok;
    // target introspection (all optional)
    int32_t* t_kind;
    int32_t* t_kept;
    int32_t* t_listed;
    uint32_t* t_ids;
    float* t_probs;
    int64_t t_cap;
    float* t_stats;
    // spec verify (rows_per_seq > 0)
    int32_t rows_per_seq;
    const uint32_t* drafts;
    const int32_t* draft_len;
    const float* u_pairs;
    const float* u_bonus;
    int32_t* out_accepted;
    uint32_t* out_next;
    // workspace
    ChunkPart* parts;
    uint32_t* vhist;     // per (row, chunk): HBINS 64-bit bins, count | fixed-point mass (top-k / top-p rows)
    uint32_t* seq_ctr;
    uint32_t* row_res;   // verify: 2 words per row {verdict, token}
    uint32_t* row_pen;   // per row: history bitmap[bm_words] + popcount prefix[bm_words] + counts[GDCAP]
    uint64_t* spill;     // per row: 4 * V keys (the candidate list, its grouped copy, sort scratch)
    RowInfo* rinfo;      // per row: the streaming pass's row results
    QPre* qpre;          // per (row, chunk): the running sum's prediction at the chunk's start
    QHead* qhead;        // per (row, chunk): the quantizing pass's summary
    QItem* qitem;        // per (row, chunk): qcap + 1 items
    uint32_t* arrive;    // per row: chunks done (the last one finishes the row; kept zero)
    uint32_t* rowcnt;    // per row: candidates gathered by the quantizing pass
    int32_t bm_words;
    int32_t qcap;        // window elements a chunk lists: min(QWIN, chunk)
    uint64_t* trace;     // optional phase timestamps (wall clock) per workgroup
};

// Phase timestamp of a workgroup (diagnostics; no-op without a trace buffer).
#define BFI_TRACE(a, base, i)                                                            \
    do {                                                                                 \
        if ((a).trace && threadIdx.x == 0) (a).trace[(base) + (i)] = wall_clock64();     \
    } while (0)

// ---- atomics with an explicit address space ------------------------------------------
// (generic-pointer atomics make the backend emit a runtime LDS/global test, which also
// trips an instruction-selection bug; LDS atomics are workgroup-scoped, global ones agent)
#define BFI_LDS __attribute__((address_space(3)))
#define BFI_GLB __attribute__((address_space(1)))
__device__ __forceinline__ uint32_t lds_add(uint32_t* p, uint32_t v) {
    return __hip_atomic_fetch_add((BFI_LDS uint32_t*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ uint32_t lds_or(uint32_t* p, uint32_t v) {
    return __hip_atomic_fetch_or((BFI_LDS uint32_t*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ uint32_t lds_max(uint32_t* p, uint32_t v) {
    return __hip_atomic_fetch_max((BFI_LDS uint32_t*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ uint64_t lds_max64(uint64_t* p, uint64_t v) {
    return __hip_atomic_fetch_max((BFI_LDS uint64_t*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ uint64_t lds_add64(uint64_t* p, uint64_t v) {
    return __hip_atomic_fetch_add((BFI_LDS uint64_t*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ uint32_t glb_add(uint32_t* p, uint32_t v) {
    return __hip_atomic_fetch_add((BFI_GLB uint32_t*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Device-coherent plain stores and loads (write-through past the non-coherent L2s, read
// from the coherence point): data one workgroup publishes for another of the same launch.
// The writer waits for its stores (s_waitcnt) before it counts itself done.
__device__ __forceinline__ void st_dev(uint32_t* p, uint32_t v) {
    __hip_atomic_store((BFI_GLB uint32_t*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev64(uint64_t* p, uint64_t v) {
    __hip_atomic_store((BFI_GLB uint64_t*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_dev(const uint32_t* p) {
    return __hip_atomic_load((const BFI_GLB uint32_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_dev64(const uint64_t* p) {
    return __hip_atomic_load((const BFI_GLB uint64_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t glb_or(uint32_t* p, uint32_t v) {
    return __hip_atomic_fetch_or((BFI_GLB uint32_t*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---- float order key ------------------------------------------------------------------

// Monotone map f32 -> u32 (larger float -> larger key). -0 folds onto +0 and NaN onto -inf,
// so equal probabilities always have equal keys.
__device__ __forceinline__ uint32_t ord32(float f) {
    if (f != f) f = -__builtin_inff();
    f = f + 0.0f;
    uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float unord32(uint32_t o) {
    uint32_t u = (o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o;
    return __uint_as_float(u);
}
// Sort key of the reference order (sample.rs:393,398): descending value, ties by ascending
// index (stable sort of an index-ordered list).
__device__ __forceinline__ uint64_t key64(float s, uint32_t idx) {
    return ((uint64_t)ord32(s) << 32) | (uint64_t)(~idx);
}
__device__ __forceinline__ uint32_t key_idx(uint64_t k) { return ~(uint32_t)k; }
__device__ __forceinline__ float key_s(uint64_t k) { return unord32((uint32_t)(k >> 32)); }

// ---- wave / block collectives ---------------------------------------------------------

__device__ __forceinline__ int lane_id() { return threadIdx.x & (WAVE - 1); }
__device__ __forceinline__ int wave_id() { return threadIdx.x / WAVE; }

// Wave-wide inclusive scans by DPP (no LDS crossbar): Hillis-Steele within each row of 16
// lanes (row_shr 1, 2, 4, 8), then row_bcast:15 into rows 1 and 3 and row_bcast:31 into
// rows 2 and 3. Lanes whose DPP source does not exist take the identity. Reductions read
// the total from lane 63 (a wave-uniform value).
template <int CTRL, int ROWMASK>
__device__ __forceinline__ uint32_t dpp32(uint32_t identity, uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp((int)identity, (int)v, CTRL, ROWMASK, 0xF, false);
}
template <int CTRL, int ROWMASK>
__device__ __forceinline__ uint64_t dpp64(uint64_t identity, uint64_t v) {
    const uint32_t lo = dpp32<CTRL, ROWMASK>((uint32_t)identity, (uint32_t)v);
    const uint32_t hi = dpp32<CTRL, ROWMASK>((uint32_t)(identity >> 32), (uint32_t)(v >> 32));
    return ((uint64_t)hi << 32) | lo;
}
template <int CTRL, int ROWMASK, typename T>
__device__ __forceinline__ T dpp_t(T identity, T v) {
    static_assert(sizeof(T) == 4 || sizeof(T) == 8, "32/64-bit only");
    if constexpr (sizeof(T) == 4) {
        return __builtin_bit_cast(T, dpp32<CTRL, ROWMASK>(__builtin_bit_cast(uint32_t, identity),
                                                           __builtin_bit_cast(uint32_t, v)));
    } else {
        return __builtin_bit_cast(T, dpp64<CTRL, ROWMASK>(__builtin_bit_cast(uint64_t, identity),
                                                           __builtin_bit_cast(uint64_t, v)));
    }
}
template <typename T, typename Op>
__device__ __forceinline__ T wave_scan_incl(T v, T identity, Op op) {
    v = op(v, dpp_t<0x111, 0xF>(identity, v));  // row_shr:1
    v = op(v, dpp_t<0x112, 0xF>(identity, v));  // row_shr:2
    v = op(v, dpp_t<0x114, 0xF>(identity, v));  // row_shr:4
    v = op(v, dpp_t<0x118, 0xF>(identity, v));  // row_shr:8
    v = op(v, dpp_t<0x142, 0xA>(identity, v));  // row_bcast:15 -> rows 1, 3
    v = op(v, dpp_t<0x143, 0xC>(identity, v));  // row_bcast:31 -> rows 2, 3
    return v;
}
template <typename T>
__device__ __forceinline__ T lane63(T v) {
    if constexpr (sizeof(T) == 4) {
        return __builtin_bit_cast(T, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
    } else {
        const uint64_t u = __builtin_bit_cast(uint64_t, v);
        const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, 63);
        const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), 63);
        return __builtin_bit_cast(T, ((uint64_t)hi << 32) | lo);
    }
}

__device__ __forceinline__ float wave_max(float v) {
    return lane63(wave_scan_incl(v, -__builtin_inff(), [](float x, float y) { return fmaxf(x, y); }));
}
__device__ __forceinline__ float wave_sum(float v) {
    return lane63(wave_scan_incl(v, 0.0f, [](float x, float y) { return x + y; }));
}
__device__ __forceinline__ double wave_sum_d(double v) {
    return lane63(wave_scan_incl(v, 0.0, [](double x, double y) { return x + y; }));
}
__device__ __forceinline__ uint32_t wave_sum_u(uint32_t v) {
    return lane63(wave_scan_incl(v, 0u, [](uint32_t x, uint32_t y) { return x + y; }));
}
__device__ __forceinline__ uint32_t wave_min_u(uint32_t v) {
    return lane63(wave_scan_incl(v, 0xFFFFFFFFu, [](uint32_t x, uint32_t y) { return x < y ? x : y; }));
}
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
    return lane63(wave_scan_incl(v, (uint64_t)0, [](uint64_t x, uint64_t y) { return x > y ? x : y; }));
}

// v of lane (lane ^ S), without the LDS crossbar: DPP quad_perm for 1 and 2, row_shl/shr:4
// for 4, row_ror:8 for 8, and gfx950's v_permlane16/32_swap for 16 and 32. All lanes must
// be active.
template <int S>
__device__ __forceinline__ uint32_t wave_xor32(uint32_t v) {
    const int lane = lane_id();
    if constexpr (S == 1) {
        return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
    } else if constexpr (S == 2) {
        return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
    } else if constexpr (S == 4) {
        const uint32_t up = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x104, 0xF, 0xF, false);  // row_shl:4
        const uint32_t dn = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xF, 0xF, false);  // row_shr:4
        return (lane & 4) ? dn : up;
    } else if constexpr (S == 8) {
        return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x128, 0xF, 0xF, false);  // row_ror:8
    } else if constexpr (S == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        return (lane & 16) ? r[0] : r[1];
    } else {
        static_assert(S == 32, "xor distance 1..32");
        const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        return (lane & 32) ? r[0] : r[1];
    }
}
template <int S>
__device__ __forceinline__ uint64_t wave_xor64(uint64_t v) {
    return ((uint64_t)wave_xor32<S>((uint32_t)(v >> 32)) << 32) | wave_xor32<S>((uint32_t)v);
}

// One compare-exchange stage of a bitonic network over keys held one per lane (position
// j): the partner is j ^ S; `desc` = this position's block sorts descending.
template <int S>
__device__ __forceinline__ uint64_t bitonic_step(uint64_t key, int j, bool desc) {
    const uint64_t other = wave_xor64<S>(key);
    const bool take_max = ((j & S) == 0) == desc;
    const uint64_t mx = other > key ? other : key, mn = other > key ? key : other;
    return take_max ? mx : mn;
}
// The stages of a bitonic merge of blocks of `size` with strides 32 .. 1 (in-wave part).
template <int TOP>
__device__ __forceinline__ uint64_t bitonic_wave_strides(uint64_t key, int j, bool desc) {
    if constexpr (TOP >= 32) key = bitonic_step<32>(key, j, desc);
    if constexpr (TOP >= 16) key = bitonic_step<16>(key, j, desc);
    if constexpr (TOP >= 8) key = bitonic_step<8>(key, j, desc);
    if constexpr (TOP >= 4) key = bitonic_step<4>(key, j, desc);
    if constexpr (TOP >= 2) key = bitonic_step<2>(key, j, desc);
    key = bitonic_step<1>(key, j, desc);
    return key;
}

// Bitonic sort of one key per lane across the wave, descending (lane 0 = largest).
__device__ __forceinline__ uint64_t wave_sort_desc(uint64_t key) {
    const int lane = lane_id();
    key = bitonic_wave_strides<1>(key, lane, (lane & 2) == 0);
    key = bitonic_wave_strides<2>(key, lane, (lane & 4) == 0);
    key = bitonic_wave_strides<4>(key, lane, (lane & 8) == 0);
    key = bitonic_wave_strides<8>(key, lane, (lane & 16) == 0);
    key = bitonic_wave_strides<16>(key, lane, (lane & 32) == 0);
    key = bitonic_wave_strides<32>(key, lane, true);
    return key;
}
__device__ __forceinline__ double wave_incl_scan_d(double v) {
    return wave_scan_incl(v, 0.0, [](double x, double y) { return x + y; });
}
__device__ __forceinline__ uint64_t lanes_below() { return (1ull << lane_id()) - 1ull; }

// Block reductions: `scr` is NWAVE words of LDS owned by the caller; both barriers are
// inside, so calls may follow each other.
__device__ __forceinline__ float block_max(float v, float* scr) {
    v = wave_max(v);
    if (lane_id() == 0) scr[wave_id()] = v;
    __syncthreads();
    float r = scr[0];
#pragma unroll
    for (int w = 1; w < NWAVE; w++) r = fmaxf(r, scr[w]);
    __syncthreads();
    return r;
}
__device__ __forceinline__ float block_sum(float v, float* scr) {
    v = wave_sum(v);
    if (lane_id() == 0) scr[wave_id()] = v;
    __syncthreads();
    float r = scr[0];
#pragma unroll
    for (int w = 1; w < NWAVE; w++) r += scr[w];
    __syncthreads();
    return r;
}
__device__ __forceinline__ double block_sum_d(double v, double* scr) {
    v = wave_sum_d(v);
    if (lane_id() == 0) scr[wave_id()] = v;
    __syncthreads();
    double r = scr[0];
#pragma unroll
    for (int w = 1; w < NWAVE; w++) r += scr[w];
    __syncthreads();
    return r;
}
__device__ __forceinline__ uint32_t block_sum_u(uint32_t v, uint32_t* scr) {
    v = wave_sum_u(v);
    if (lane_id() == 0) scr[wave_id()] = v;
    __syncthreads();
    uint32_t r = 0;
#pragma unroll
    for (int w = 0; w < NWAVE; w++) r += scr[w];
    __syncthreads();
    return r;
}
// Sum of a double and of a count in one pair of barriers.
__device__ __forceinline__ double block_sum_du(double v, uint32_t c, uint32_t& csum, double* scrd, uint32_t* scru) {
    v = wave_sum_d(v);
    c = wave_sum_u(c);
    if (lane_id() == 0) {
        scrd[wave_id()] = v;
        scru[wave_id()] = c;
    }
    __syncthreads();
    double r = scrd[0];
    uint32_t rc = scru[0];
#pragma unroll
    for (int w = 1; w < NWAVE; w++) {
        r += scrd[w];
        rc += scru[w];
    }
    __syncthreads();
    csum = rc;
    return r;
}
// Sum of a float and of a count in one pair of barriers.
__device__ __forceinline__ float block_sum_fu(float v, uint32_t c, uint32_t& csum, float* scrf, uint32_t* scru) {
    v = wave_sum(v);
    c = wave_sum_u(c);
    if (lane_id() == 0) {
        scrf[wave_id()] = v;
        scru[wave_id()] = c;
    }
    __syncthreads();
    float r = scrf[0];
    uint32_t rc = scru[0];
#pragma unroll
    for (int w = 1; w < NWAVE; w++) {
        r += scrf[w];
        rc += scru[w];
    }
    __syncthreads();
    csum = rc;
    return r;
}
__device__ __forceinline__ uint32_t block_min_u(uint32_t v, uint32_t* scr) {
    v = wave_min_u(v);
    if (lane_id() == 0) scr[wave_id()] = v;
    __syncthreads();
    uint32_t r = scr[0];
#pragma unroll
    for (int w = 1; w < NWAVE; w++) r = min(r, scr[w]);
    __syncthreads();
    return r;
}
__device__ __forceinline__ uint64_t block_max_u64(uint64_t v, uint64_t* scr) {
    v = wave_max_u64(v);
    if (lane_id() == 0) scr[wave_id()] = v;
    __syncthreads();
    uint64_t r = scr[0];
#pragma unroll
    for (int w = 1; w < NWAVE; w++) r = scr[w] > r ? scr[w] : r;
    __syncthreads();
    return r;
}

// The previous lane's value of an inclusive scan (lane 0: identity): the exclusive scan
// without subtracting the lane's own value (which, for floating point, cancels the smaller
// prefix away when the own value dominates it).
template <typename T>
__device__ __forceinline__ T wave_excl_of_incl(T x, T identity) {
    if constexpr (sizeof(T) == 4) {
        const T up = __builtin_bit_cast(T, __shfl_up(__builtin_bit_cast(int, x), 1));
        return lane_id() == 0 ? identity : up;
    } else {
        const uint64_t u = __builtin_bit_cast(uint64_t, x);
        const uint32_t lo = (uint32_t)__shfl_up((int)(uint32_t)u, 1);
        const uint32_t hi = (uint32_t)__shfl_up((int)(uint32_t)(u >> 32), 1);
        return lane_id() == 0 ? identity : __builtin_bit_cast(T, ((uint64_t)hi << 32) | lo);
    }
}

// Exclusive block scan; `total` receives the block sum. Fixed combination order, so the
// result is deterministic for floating-point T.
template <typename T>
__device__ __forceinline__ T block_excl_scan(T v, T* scr, T& total) {
    const T x = wave_scan_incl(v, (T)0, [](T a, T b) { return a + b; });
    if (lane_id() == WAVE - 1) scr[wave_id()] = x;
    __syncthreads();
    T pre = 0, tot = 0;
#pragma unroll
    for (int w = 0; w < NWAVE; w++) {
        T s = scr[w];
        if (w < wave_id()) pre += s;
        tot += s;
    }
    __syncthreads();
    total = tot;
    return pre + wave_excl_of_incl(x, (T)0);
}

// (value, index) argmax with the reference's tie rule (sample.rs:429-439): the first
// (lowest) index of the maximum; NaN never wins.
struct ArgMax {
    float v;
    uint32_t i;
};
__device__ __forceinline__ ArgMax argmax_merge(ArgMax a, ArgMax b) {
    if (b.v > a.v || (b.v == a.v && b.i < a.i)) return b;
    return a;
}
// (value, index) as a 64-bit key whose unsigned max is the reference's argmax (largest
// value, then lowest index; sample.rs:429-439); 0 = none.
__device__ __forceinline__ uint64_t argmax_key(float v, uint32_t i) { return ((uint64_t)ord32(v) << 32) | ~i; }
__device__ __forceinline__ ArgMax argmax_of_key(uint64_t k) {
    return k ? ArgMax{unord32((uint32_t)(k >> 32)), ~(uint32_t)k} : ArgMax{-__builtin_inff(), 0xFFFFFFFFu};
}
__device__ __forceinline__ ArgMax wave_argmax(ArgMax a) {
    // (value, index) packed in 64 bits for the DPP scan; merged with argmax_merge
    const uint64_t packed = ((uint64_t)__float_as_uint(a.v) << 32) | a.i;
    const uint64_t ident = ((uint64_t)__float_as_uint(-__builtin_inff()) << 32) | 0xFFFFFFFFu;
    const uint64_t r64 = lane63(wave_scan_incl(packed, ident, [](uint64_t x, uint64_t y) {
        const ArgMax m = argmax_merge(ArgMax{__uint_as_float((uint32_t)(x >> 32)), (uint32_t)x},
                                      ArgMax{__uint_as_float((uint32_t)(y >> 32)), (uint32_t)y});
        return ((uint64_t)__float_as_uint(m.v) << 32) | m.i;
    }));
    return ArgMax{__uint_as_float((uint32_t)(r64 >> 32)), (uint32_t)r64};
}
__device__ __forceinline__ ArgMax block_argmax(ArgMax a, float* scrv, uint32_t* scri) {
    a = wave_argmax(a);
    if (lane_id() == 0) {
        scrv[wave_id()] = a.v;
        scri[wave_id()] = a.i;
    }
    __syncthreads();
    ArgMax r{scrv[0], scri[0]};
#pragma unroll
    for (int w = 1; w < NWAVE; w++) r = argmax_merge(r, ArgMax{scrv[w], scri[w]});
    __syncthreads();
    return r;
}

// ---- penalties: sample.rs:345-367 (+ frequency extension) ------------------------------

struct Pen {
    float rp, pp, fp;
    float rrp;   // 1 / rp (IEEE): the corrected reciprocal quotient's reciprocal
    bool rep_on, pres_on, freq_on;
    bool rdiv;   // rp in [2^-20, 2^20]: x / rp as the corrected reciprocal quotient
};

// x / d rounded like IEEE division: q = RN(x * r) with r = RN(1/d), e = x - q*d exact under
// FMA, RN(q + e*r) (Markstein's correction) is the correctly rounded quotient for |x| in
// [2^-100, 2^100) (or x = 0) and d in [2^-20, 2^20] (checked bit-exhaustively on a strided
// sample of every float against IEEE division); other operands take IEEE division.
__device__ __forceinline__ float div_rn(float x, float d, float r, bool d_ok) {
    const uint32_t ax = __float_as_uint(x) & 0x7FFFFFFFu;
    const bool x_ok = ((ax - 0x0D800000u) < 0x64000000u) | (ax == 0u);
    if (d_ok & x_ok) {
        const float q = x * r;
        const float e = __builtin_fmaf(-q, d, x);
        const float s = __builtin_fmaf(e, r, q);
        return e != e ? q : s;
    }
    return x / d;
}

__device__ __forceinline__ float penalize(float x, uint32_t count, const Pen& P) {
    if (P.rep_on) x = (x > 0.0f) ? div_rn(x, P.rp, P.rrp, P.rdiv) : x * P.rp;  // sample.rs:350-354
    if (P.pres_on) x = x - P.pp;                          // sample.rs:364
    if (P.freq_on) {                                      // extension: two roundings, no FMA
        float fc = P.fp * (float)count;
        x = x - fc;
    }
    return x;
}

// History of one row: the base ids plus (spec verify) the drafts accepted before this row.
struct HistView {
    const uint32_t* base;
    int64_t nbase;
    const uint32_t* extra;
    int64_t nextra;
    __device__ __forceinline__ int64_t size() const { return nbase + nextra; }
    __device__ __forceinline__ uint32_t at(int64_t j) const {
        return j < nbase ? base[j] : extra[j - nbase];
    }
    // Occurrences of id: slow path for rows whose distinct-id table overflowed.
    __device__ __forceinline__ uint32_t count_scan(uint32_t id) const {
        uint32_t c = 0;
        for (int64_t j = 0; j < nbase; j++) c += base[j] == id;
        for (int64_t j = 0; j < nextra; j++) c += extra[j] == id;
        return c;
    }
};

// Dense rank of bit b of word w among all set bits (word prefix + in-word popcount).
__device__ __forceinline__ uint32_t dense_rank(uint32_t pre_w, uint32_t word, uint32_t b) {
    return pre_w + __popc(word & ((1u << b) - 1u));
}

}  // namespace bfi
