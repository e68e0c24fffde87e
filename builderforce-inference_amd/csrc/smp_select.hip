// smp_select.hip — the select pass of the gfx950 token sampler: one workgroup per row.
//
// It reads the streaming pass's per-chunk results, applies the repetition / presence /
// frequency penalties (sample.rs:345-368) to the row's history ids as corrections, and
// finishes the row:
//   - greedy: argmax (sample.rs:369-371, 429-439);
//   - bounded candidates (top-k <= 2048 or min-p > 0): gather, one sort in LDS, then
//     top-k / top-p / min-p and the draw by f64 scans (sample.rs:392-426, 312-323);
//   - rows without top-k/top-p: the draw in index order from per-chunk masses plus one
//     chunk re-read;
//   - unbounded rows (top-p without top-k/min-p, or candidate overflow): radix select over
//     the row (10-bit digits of a 64-bit (value, index) key, with counts and fixed-point
//     masses), re-reading the row.
// Spec verify applies judge() (spec.rs:79-97) to each row's target; the last row of a
// sequence to finish computes the accepted prefix.
#include <hip/hip_ext.h>

// One row per workgroup of 512 threads (8 wave64s, 2 per SIMD): the select pass is a
// chain of short dependent steps, and more waves per SIMD hide their latencies.
#define BFI_BLOCK 512
#include "smp_finish.h"

// Phase timestamps go to LDS and are written out when the workgroup ends, so that tracing
// adds no global store (and no wait for one) between phases.
#undef BFI_TRACE
#define BFI_TRACE(a, base, i)                                                   \
    do {                                                                        \
        if ((a).trace && threadIdx.x == 0) sm.tr[(i)] = wall_clock64();         \
    } while (0)

namespace bfi {

// ---- shared memory ---------------------------------------------------------------------

constexpr int NSPEC = 512;  // elements of the buckets gathered ahead for a following query

struct __align__(16) Smem {
    union {
        struct {
            uint64_t keys[NMAX];
            float p[NMAX];
        } cb;
        struct {
            uint64_t mass[NVB];
            uint32_t cnt[NVB];
        } hs;
    } u;
    // history set of the row (ids < V): open addressing, linear probing
    uint32_t hkey[HSLOTS];
    uint32_t hcnt[HSLOTS];
    float hraw[HSLOTS];        // value the streaming pass used (masked, /T)
    float hpen[HSLOTS];        // penalized value (sample.rs:345-375)
    uint16_t hlist[HSLOTS];    // the occupied slots, densely (order of insertion)
    // per-chunk tables (index = chunk)
    float cm[NCMAX];           // max over the chunk's non-history elements
    float cxm[NCMAX];          // the chunk's largest masked logit (streaming pass)
    uint32_t carg[NCMAX];      // its first index (greedy)
    double csum[NCMAX];        // sum of exp(s - cm) over them, or a chunk mass
    uint32_t cflag[NCMAX];     // ord32 of the largest history value, then the dirty flag
    uint64_t craw[NCMAX];      // fixed-point streaming-pass terms of the chunk's history ids
    uint64_t cpen[NCMAX];      // fixed-point penalized terms exp(s - M) of its history ids
    uint32_t cpre[NCMAX + 1];  // per-chunk candidate prefix (combine)
    float rf[NWAVE];
    float rf2[NWAVE];
    uint32_t ru[NWAVE];
    uint32_t ru2[NWAVE];
    double rd[NWAVE];
    uint64_t r64[NWAVE];
    uint64_t r64b[NWAVE];
    uint32_t misc[8];
    uint32_t fx[8];   // the fast finish's row values
    uint64_t tr[16];  // phase timestamps of this workgroup (diagnostics)
    // row aggregates built with LDS atomics (integer, so independent of the order)
    struct {
        uint64_t gkey;    // greedy: max over (value, index) keys (argmax_key)
        uint64_t rawkey;  // max (masked logit, index) key: the min-p fallback argmax
        uint64_t sfix;    // S in 2^-44 fixed point
        uint32_t mmax;    // ord32 of the largest chunk maximum
        uint32_t hmax;    // ord32 of the largest penalized history value
        uint32_t thr;     // ord32 of the largest chunk candidate bound
        uint32_t flags;   // 1: some chunk has no candidate list
        uint32_t nd;      // history ids that hold their chunk's maximum
        uint32_t kth;     // ord32 of the k-th largest chunk maximum (top-k rows, k <= chunks)
    } ag;
    // value buckets spec_lo..spec_hi of the row, complete (every element), gathered with an
    // earlier query for a query expected to follow; spec_lo > spec_hi when empty. Last, so
    // that the fields the fast finish uses keep their offsets and alignment.
    uint32_t spec_n, spec_lo, spec_hi, spec_pad;
    uint64_t spec[NSPEC];
};

constexpr double FIX52 = 4503599627370496.0;  // 2^52: fixed-point scale of the history corrections

// ---- history structures ----------------------------------------------------------------

// Row-wide history bitmap + dense counts in global scratch (fallback passes over the row).
__device__ __forceinline__ void build_row_pen(const KArgs& a, Smem& sm, const RowCtx& C) {
    if (!C.pen_on) return;
    const int tid = threadIdx.x;
    const int nw = a.bm_words;
    uint32_t* bm = a.row_pen + (int64_t)C.row * (2 * nw + GDCAP);
    uint32_t* pre = bm + nw;
    uint32_t* cnt = pre + nw;
    for (int w = tid; w < nw; w += BLOCK) bm[w] = 0;
    if (C.pen.freq_on)
        for (int w = tid; w < GDCAP; w += BLOCK) cnt[w] = 0;
    __threadfence();
    __syncthreads();
    const int64_t H = C.h.size();
    for (int64_t j = tid; j < H; j += BLOCK) {
        uint32_t id = C.h.at(j);
        if (id < (uint32_t)a.V) glb_or(&bm[id >> 5], 1u << (id & 31));
    }
    __threadfence();
    __syncthreads();
    if (C.pen.freq_on) {
        // popcount prefix over nw words: each thread a contiguous run
        const int per = (nw + BLOCK - 1) / BLOCK;
        const int w0 = tid * per;
        uint32_t s = 0;
        for (int w = w0; w < w0 + per && w < nw; w++) s += __popc(bm[w]);
        uint32_t tot;
        uint32_t run = block_excl_scan<uint32_t>(s, sm.ru, tot);
        for (int w = w0; w < w0 + per && w < nw; w++) {
            pre[w] = run;
            run += __popc(bm[w]);
        }
        if (tid == 0) sm.misc[MISC_NDIST] = tot;
        __threadfence();
        __syncthreads();
        if (tot <= GDCAP) {
            for (int64_t j = tid; j < H; j += BLOCK) {
                uint32_t id = C.h.at(j);
                if (id < (uint32_t)a.V) glb_add(&cnt[dense_rank(pre[id >> 5], bm[id >> 5], id & 31)], 1u);
            }
        }
        __threadfence();
        __syncthreads();
    }
}

// ---- history set (select kernel): ids < V with occurrence counts ------------------------

__device__ __forceinline__ uint32_t hslot0(uint32_t id) { return (id * 2654435761u) >> (32 - HSLOTS_LOG2); }

__device__ __forceinline__ uint32_t lds_cas(uint32_t* p, uint32_t expected, uint32_t desired) {
    __hip_atomic_compare_exchange_strong((BFI_LDS uint32_t*)p, &expected, desired, __ATOMIC_RELAXED,
                                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    return expected;  // the previous value
}

// Slot of `id`, or -1 when absent.
__device__ __forceinline__ int hist_find(const Smem& sm, uint32_t id) {
    uint32_t s = hslot0(id);
    for (int probe = 0; probe < HSLOTS; probe++) {
        const uint32_t k = sm.hkey[s];
        if (k == id) return (int)s;
        if (k == HEMPTY) return -1;
        s = (s + 1) & (HSLOTS - 1);
    }
    return -1;
}

// append_cands' exclusion of the ids the history hash lists apart (append_hist).
struct HistExcl {
    const Smem& sm;
    const RowCtx& C;
    __device__ __forceinline__ bool operator()(uint32_t id) const { return C.pen_hash && hist_find(sm, id) >= 0; }
};

// The reference's `HashSet(prev)` (sample.rs:347, 361) plus multiset counts (frequency
// extension). The thread that inserts an id first stores its masked logit in hraw. The id
// loads and the logit loads of HB entries per thread are each issued together.
// `after_clear()` runs between the two barriers (LDS written there is visible on return).
// Returns false when the row has more than HMAX distinct ids (inserts stop there, so the
// table never fills and every probe sequence ends).
constexpr int HB = 4;  // history entries per thread per round

// The ids this thread inserted first (single-round histories): their slots and masked
// logits stay in registers, so the logit loads can land while the table is finished.
struct HistOwn {
    bool regs;         // the owner lists below are complete (else hraw holds the logits)
    uint32_t own;      // bit g: entry g was inserted by this thread
    uint32_t id[HB];
    uint32_t slot[HB];
    uint32_t mw[HB];   // allow-mask word of the id
    float x[HB];       // logit
};

template <bool BF16, typename F>
__device__ __forceinline__ bool hist_build(const KArgs& a, Smem& sm, const RowCtx& C, HistOwn& ho, F after_clear) {
    const int tid = threadIdx.x;
    for (int k = tid; k < HSLOTS; k += BLOCK) {
        sm.hkey[k] = HEMPTY;
        sm.hcnt[k] = 0;
    }
    if (tid == 0) sm.misc[MISC_HN] = 0;
    const int64_t H = C.pen_hash ? C.h.size() : 0;
    const uint32_t V = (uint32_t)a.V;
    ho.regs = H <= (int64_t)HB * BLOCK;
    ho.own = 0;
    bool cleared = false;
    for (int64_t j0 = 0; j0 < H; j0 += (int64_t)HB * BLOCK) {
#pragma unroll
        for (int g = 0; g < HB; g++) {
            const int64_t j = j0 + g * BLOCK + tid;
            ho.id[g] = j < H ? C.h.at(j) : HEMPTY;
        }
#pragma unroll
        for (int g = 0; g < HB; g++) {
            const uint32_t ld = ho.id[g] < V ? ho.id[g] : 0u;
            if (BF16)
                ho.x[g] = __uint_as_float((uint32_t)((const uint16_t*)a.logits)[(int64_t)C.row * a.row_stride + ld] << 16);
            else
                ho.x[g] = ((const float*)a.logits)[(int64_t)C.row * a.row_stride + ld];
            ho.mw[g] = C.mrow ? C.mrow[ld >> 5] : 0xFFFFFFFFu;
        }
        if (!cleared) {
            __syncthreads();
            after_clear();
            cleared = true;
        }
#pragma unroll
        for (int g = 0; g < HB; g++) {
            const uint32_t id = ho.id[g];
            if (id >= V) continue;
            if (__hip_atomic_load((BFI_LDS uint32_t*)&sm.misc[MISC_HN], __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_WORKGROUP) > (uint32_t)HMAX)
                continue;
            uint32_t k = hslot0(id);
            for (int probe = 0; probe < HSLOTS; probe++) {
                const uint32_t prev = lds_cas(&sm.hkey[k], HEMPTY, id);
                if (prev == HEMPTY || prev == id) {
                    if (prev == HEMPTY) {
                        const uint32_t pos = lds_add(&sm.misc[MISC_HN], 1u);  // < HSLOTS: one per key
                        sm.hlist[pos] = (uint16_t)k;
                        ho.own |= 1u << g;
                        ho.slot[g] = k;
                        if (!ho.regs) sm.hraw[k] = ((ho.mw[g] >> (id & 31)) & 1u) ? ho.x[g] : -__builtin_inff();
                    }
                    lds_add(&sm.hcnt[k], 1u);
                    break;
                }
                k = (k + 1) & (HSLOTS - 1);
            }
        }
    }
    if (!cleared) {
        __syncthreads();
        after_clear();
    }
    __syncthreads();
    return sm.misc[MISC_HN] <= (uint32_t)HMAX;
}

// Wave-aggregated LDS atomics: the wave reduces first (DPP), then one lane updates LDS.
// Every lane of the wave must call them.
__device__ __forceinline__ void wave_lds_max(uint32_t* p, uint32_t v) {
    v = lane63(wave_scan_incl(v, 0u, [](uint32_t x, uint32_t y) { return x > y ? x : y; }));
    if (lane_id() == 0) lds_max(p, v);
}
__device__ __forceinline__ void wave_lds_max64(uint64_t* p, uint64_t v) {
    v = lane63(wave_scan_incl(v, (uint64_t)0, [](uint64_t x, uint64_t y) { return x > y ? x : y; }));
    if (lane_id() == 0) lds_max64(p, v);
}
__device__ __forceinline__ void wave_lds_add64(uint64_t* p, uint64_t v) {
    v = lane63(wave_scan_incl(v, (uint64_t)0, [](uint64_t x, uint64_t y) { return x + y; }));
    if (lane_id() == 0 && v) lds_add64(p, v);
}
__device__ __forceinline__ void wave_lds_add(uint32_t* p, uint32_t v) {
    v = lane63(wave_scan_incl(v, 0u, [](uint32_t x, uint32_t y) { return x + y; }));
    if (lane_id() == 0 && v) lds_add(p, v);
}


// Values of the history ids (dense slot list): hraw = the un-penalized value x / T, hpen =
// the penalized one (sample.rs:331-375). Per chunk, into craw, the terms stream_term the
// streaming pass added to the chunk's sum for these ids (recomputed with the same
// expression), in 2^52 fixed point. A history id equal to its chunk's maximum marks the
// chunk dirty (cflag, ag.nd). Row aggregates: the largest hpen (ag.hmax), or for greedy
// rows the argmax key (ag.gkey). sm.cm / sm.cxm must hold the chunk results.
__device__ __forceinline__ void hist_values(const KArgs& a, Smem& sm, const RowCtx& C, const HistOwn& ho) {
    uint64_t gk = 0;
    uint32_t hm = 0, nd = 0;
    auto one = [&](uint32_t k, uint32_t id, float x) __attribute__((always_inline)) {  // x: masked logit
        const float vr = raw_value(C, x, true), vp = pen_value(C, x, true, sm.hcnt[k]);
        sm.hraw[k] = vr;
        sm.hpen[k] = vp;
        const uint64_t key = argmax_key(vp, id);
        gk = key > gk ? key : gk;
        hm = max(hm, ord32(vp));
        if (vr > -__builtin_inff()) {
            const uint32_t c = id / (uint32_t)a.chunk;
            const float xm = sm.cxm[c];
            if (!C.greedy && xm > -__builtin_inff()) {
                const double t = (double)stream_term(C, x, xm);
                lds_add64(&sm.craw[c], (uint64_t)(t * FIX52));
            }
            if (vr == sm.cm[c]) {
                sm.cflag[c] = 1u;
                nd++;
            }
        }
    };
    if (ho.regs) {
#pragma unroll
        for (int g = 0; g < HB; g++)
            if ((ho.own >> g) & 1u)
                one(ho.slot[g], ho.id[g], ((ho.mw[g] >> (ho.id[g] & 31)) & 1u) ? ho.x[g] : -__builtin_inff());
    } else {
        const int nh = (int)sm.misc[MISC_HN];
        for (int j = threadIdx.x; j < nh; j += BLOCK) {
            const int k = sm.hlist[j];
            one((uint32_t)k, sm.hkey[k], sm.hraw[k]);
        }
    }
    if (C.greedy)
        wave_lds_max64(&sm.ag.gkey, gk);
    else
        wave_lds_max(&sm.ag.hmax, hm);
    wave_lds_add(&sm.ag.nd, nd);
    __syncthreads();
}


// Where the penalty membership/counts of an element come from in passes over the row.
struct PenSrc {
    bool hash;                  // LDS history hash (else the global row tables)
    const uint32_t* gbm;        // row tables (global)
    const uint32_t* gpre;
    const uint32_t* gcnt;
};

__device__ __forceinline__ uint32_t pen_bits(const Smem& sm, const PenSrc& S, uint32_t id0, int epv) {
    const uint32_t em = (1u << epv) - 1u;
    if (S.hash) {
        uint32_t b = 0;
        for (int e = 0; e < epv; e++) b |= (hist_find(sm, id0 + e) >= 0 ? 1u : 0u) << e;
        return b;
    }
    return (S.gbm[id0 >> 5] >> (id0 & 31)) & em;
}
__device__ __forceinline__ uint32_t pen_count(const Smem& sm, const PenSrc& S, const RowCtx& C, uint32_t id) {
    if (!C.pen.freq_on) return 0;
    if (S.hash) {
        const int k = hist_find(sm, id);
        return k >= 0 ? sm.hcnt[k] : 0u;
    }
    if (sm.misc[MISC_NDIST] > GDCAP) return C.h.count_scan(id);
    return S.gcnt[dense_rank(S.gpre[id >> 5], S.gbm[id >> 5], id & 31)];
}

// Raw words of one tile of a pass over the row: 16 bytes of logits, the allow-mask word and
// the history-membership word of every vector the thread owns. A tile's words are loaded as
// one batch before the previous tile is processed, and nothing reads them until then, so the
// loads of the next tile stay in flight while this one is worked on.
template <bool BF16, int VEC>
struct RawTile {
    uint4 w[VEC];
    uint32_t mw[VEC];
    uint32_t pw[VEC];
};

template <bool BF16, int VEC>
__device__ __forceinline__ void load_raw(const KArgs& a, const RowCtx& C, const PenSrc& P, uint32_t c0,
                                         uint32_t c1, RawTile<BF16, VEC>& r) {
    constexpr int EPV = Elem<BF16>::EPV;
    typedef typename Elem<BF16>::T T;
    const T* base = (const T*)a.logits + (int64_t)C.row * a.row_stride;
    const int tid = threadIdx.x;
    const uint32_t ninf = BF16 ? 0xFF80FF80u : 0xFF800000u;  // -inf in every element
    if (a.vec_ok && c1 - c0 == (uint32_t)(BLOCK * VEC * EPV)) {
#pragma unroll
        for (int q = 0; q < VEC; q++) r.w[q] = *(const uint4*)(base + c0 + (uint32_t)(q * BLOCK + tid) * EPV);
    } else {
#pragma unroll
        for (int q = 0; q < VEC; q++) {
            const uint32_t id0 = c0 + (uint32_t)(q * BLOCK + tid) * EPV;
            if (a.vec_ok && id0 + EPV <= c1) {
                r.w[q] = *(const uint4*)(base + id0);
            } else {
                uint32_t ww[4] = {ninf, ninf, ninf, ninf};
#pragma unroll
                for (int e = 0; e < EPV; e++) {
                    if (id0 + e >= c1) continue;
                    if (BF16) {
                        const uint32_t b = (uint32_t)base[id0 + e];
                        ww[e >> 1] = (e & 1) ? (ww[e >> 1] & 0xFFFFu) | (b << 16) : (ww[e >> 1] & 0xFFFF0000u) | b;
                    } else {
                        ww[e] = __float_as_uint((float)base[id0 + e]);
                    }
                }
                r.w[q] = make_uint4(ww[0], ww[1], ww[2], ww[3]);
            }
        }
    }
    // Every path issues the same loads: word indices clamped into the row, and a table the
    // row does not have read from the row's own logits (wi < V/32 words lie inside them) and
    // replaced afterwards. The compiler's waits before this tile's first use then count the
    // loads issued after it on every path alike.
    const bool pen_tab = C.pen_on && !P.hash;
    const uint32_t* mp = C.mrow ? C.mrow : (const uint32_t*)base;
    const uint32_t* pp = pen_tab ? P.gbm : (const uint32_t*)base;
#pragma unroll
    for (int q = 0; q < VEC; q++) {
        const uint32_t id0 = c0 + (uint32_t)(q * BLOCK + tid) * EPV;
        const uint32_t wi = id0 < c1 ? id0 >> 5 : 0u;
        r.mw[q] = mp[wi];
        r.pw[q] = pp[wi];
    }
}

// Streaming values (raw_value) of one vector without penalties: one range check for the
// vector, then the division of div_T_fast without its per-element branches (no element is
// infinite or NaN there); other vectors take raw_value per element.
template <int EPV>
__device__ __forceinline__ void raw_vector(const RowCtx& C, float (&x)[EPV], uint32_t mb) {
    if (C.greedy) {
#pragma unroll
        for (int e = 0; e < EPV; e++) x[e] = ((mb >> e) & 1u) ? x[e] : -__builtin_inff();
        return;
    }
    if (C.fast_div) {
        uint32_t hi = 0u, lo = 0xFFFFFFFFu;
#pragma unroll
        for (int e = 0; e < EPV; e++) {
            const uint32_t ab = __float_as_uint(x[e]) & 0x7FFFFFFFu;
            hi = max(hi, ab);
            lo = min(lo, ab - 1u);
        }
        // every element zero or with |x| in [2^-100, 2^100): div_ok holds for all of them
        if (hi < 0x71800000u && lo >= 0x0D7FFFFFu) {
#pragma unroll
            for (int e = 0; e < EPV; e++) {
                const float q = x[e] * C.rT;
                const float er = __builtin_fmaf(-q, C.T, x[e]);
                x[e] = __builtin_fmaf(er, C.rT, q);
            }
            if (C.mrow) {
#pragma unroll
                for (int e = 0; e < EPV; e++) x[e] = ((mb >> e) & 1u) ? x[e] : -__builtin_inff();
            }
            return;
        }
    }
#pragma unroll
    for (int e = 0; e < EPV; e++) x[e] = raw_value(C, x[e], (mb >> e) & 1u);
}

// In place over one tile of a pass over the row (words in r): the streaming value
// (raw_value) for every element, the penalized value (pen_value) for the history ids.
template <bool BF16, int VEC>
__device__ __forceinline__ void transform_raw(const Smem& sm, const RowCtx& C, const PenSrc& S, uint32_t c0,
                                              uint32_t c1, const RawTile<BF16, VEC>& r,
                                              float (&x)[VEC][Elem<BF16>::EPV]) {
    constexpr int EPV = Elem<BF16>::EPV;
    const int tid = threadIdx.x;
    const uint32_t em = (1u << EPV) - 1u;
#pragma unroll
    for (int q = 0; q < VEC; q++) {
        const uint32_t id0 = c0 + (uint32_t)(q * BLOCK + tid) * EPV;
        if (id0 >= c1) continue;  // all -inf already
        const uint32_t mb = C.mrow ? (r.mw[q] >> (id0 & 31)) & em : em;
        const uint32_t pb = !C.pen_on ? 0u : S.hash ? pen_bits(sm, S, id0, EPV) : (r.pw[q] >> (id0 & 31)) & em;
        // Every vector takes the vector path; the few history ids (per lane, so a wave runs
        // an element's fix-up only when one of its lanes has that element in the history) are
        // then recomputed from their raw logits.
        float xr[EPV];
#pragma unroll
        for (int e = 0; e < EPV; e++) xr[e] = x[q][e];
        raw_vector<EPV>(C, x[q], mb);
        if (pb) {
#pragma unroll
            for (int e = 0; e < EPV; e++)
                if ((pb >> e) & 1u) x[q][e] = pen_value(C, xr[e], (mb >> e) & 1u, pen_count(sm, S, C, id0 + e));
        }
    }
}

// One pass over [c0, c1) of the row: f(id, s) for every element, s = its value with the
// penalties from P; with SKIP_HIST, only for the ids outside the history hash, at their
// streaming-pass values.
template <bool BF16, int VEC, bool SKIP_HIST, typename F>
__device__ __forceinline__ void span_pass(const KArgs& a, const Smem& sm, const RowCtx& C, const PenSrc& P,
                                          uint32_t c0, uint32_t c1, F f) {
    constexpr int EPV = Elem<BF16>::EPV;
    constexpr uint32_t TILE = (uint32_t)BLOCK * VEC * EPV;
    const uint32_t em = (1u << EPV) - 1u;
    // two buffers, the loop unrolled by two: a tile's words are consumed from the registers
    // they were loaded into (a copy between buffers would wait for the loads in flight)
    RawTile<BF16, VEC> ra, rb;
    auto tile = [&](const RawTile<BF16, VEC>& r, uint32_t t0, uint32_t t1) __attribute__((always_inline)) {
        float x[VEC][EPV];
#pragma unroll
        for (int q = 0; q < VEC; q++) unpack16<BF16, VEC>(r.w[q], x[q]);
        if (!SKIP_HIST) transform_raw<BF16, VEC>(sm, C, P, t0, t1, r, x);
#pragma unroll
        for (int q = 0; q < VEC; q++) {
            const uint32_t id0 = t0 + (uint32_t)(q * BLOCK + threadIdx.x) * EPV;
            if (id0 >= t1) continue;
            const uint32_t mb = (SKIP_HIST && C.mrow) ? (r.mw[q] >> (id0 & 31)) & em : em;
#pragma unroll
            for (int e = 0; e < EPV; e++) {
                const uint32_t id = id0 + e;
                if (id >= t1) continue;
                if (SKIP_HIST) {
                    if (C.pen_hash && hist_find(sm, id) >= 0) continue;
                    f(id, raw_value(C, x[q][e], (mb >> e) & 1u));
                } else {
                    f(id, x[q][e]);
                }
            }
        }
    };
    // past the span's last tile, the "next" loads re-read the tile just loaded (cached), so
    // that every iteration issues the same loads
    if (c0 >= c1) return;
    load_raw<BF16, VEC>(a, C, P, c0, min(c0 + TILE, c1), ra);
    for (uint32_t t0 = c0;; t0 += 2 * TILE) {
        const uint32_t t1 = min(t0 + TILE, c1);
        const bool more1 = t1 < c1;
        load_raw<BF16, VEC>(a, C, P, more1 ? t1 : t0, more1 ? min(t1 + TILE, c1) : t1, rb);
        tile(ra, t0, t1);
        if (!more1) break;
        const uint32_t t2 = min(t1 + TILE, c1);
        const bool more2 = t2 < c1;
        load_raw<BF16, VEC>(a, C, P, more2 ? t2 : t1, more2 ? min(t2 + TILE, c1) : t2, ra);
        tile(rb, t1, t2);
        if (!more2) break;
    }
}

__device__ __forceinline__ uint32_t chunk_lo(const KArgs& a, uint32_t c) { return c * (uint32_t)a.chunk; }
__device__ __forceinline__ uint32_t chunk_hi(const KArgs& a, uint32_t c) {
    return min(c * (uint32_t)a.chunk + (uint32_t)a.chunk, (uint32_t)a.V);
}


// ---- f64 scans over a sorted list in LDS (bounded-candidate path) ----------------------

constexpr int PT = NMAX / BLOCK;  // positions per thread

// First position j < n (in list order) with pred(j) and inclusive cum(w) >= target, where
// w(j) is the weight of position j; UINT32_MAX if none.
template <typename W, typename P>
__device__ __forceinline__ uint32_t first_cum_ge(Smem& sm, int n, W w, P pred, double target) {
    const int tid = threadIdx.x;
    double loc[PT];
    double run = 0.0;
#pragma unroll
    for (int i = 0; i < PT; i++) {
        int j = tid * PT + i;
        run += (j < n) ? w(j) : 0.0;
        loc[i] = run;
    }
    double tot;
    double pre = block_excl_scan<double>(run, sm.rd, tot);
    uint32_t best = 0xFFFFFFFFu;
#pragma unroll
    for (int i = 0; i < PT; i++) {
        int j = tid * PT + i;
        if (best == 0xFFFFFFFFu && j < n && pred(j) && pre + loc[i] >= target) best = (uint32_t)j;
    }
    return block_min_u(best, sm.ru);
}

template <typename W>
__device__ __forceinline__ double list_sum(Smem& sm, int n, W w) {
    const int tid = threadIdx.x;
    double run = 0.0;
#pragma unroll
    for (int i = 0; i < PT; i++) {
        int j = tid * PT + i;
        run += (j < n) ? w(j) : 0.0;
    }
    return block_sum_d(run, sm.rd);
}

// Orders LDS writes of this wave before its later LDS reads (lanes of one wave only).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Bitonic sort of n (a power of two, <= 2 * NMAX) 64-bit keys in LDS, descending. A stage
// with stride <= 64 touches only its wave's own 128-key segments, so between two such stages
// a wave-level sync suffices; block barriers separate the others.
__device__ __forceinline__ void bitonic_sort_desc(uint64_t* k, int n) {
    for (int size = 2; size <= n; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = threadIdx.x; i < n / 2; i += BLOCK) {
                const int lo = 2 * i - (i & (stride - 1));
                const int hi = lo + stride;
                const bool desc = (lo & size) == 0;
                const uint64_t x = k[lo], y = k[hi];
                if ((x < y) == desc) {
                    k[lo] = y;
                    k[hi] = x;
                }
            }
            const int next = stride > 1 ? stride >> 1 : size;  // the next stage's stride
            const bool last = stride == 1 && size == n;
            if (!last && stride <= WAVE && next <= WAVE)
                wave_lds_sync();
            else
                __syncthreads();
        }
    }
}

// Sorts the N keys of the list (padding to a power of two with 0, which sorts last).
__device__ __forceinline__ void sort_list(Smem& sm, int N) {
    int n2 = 64;
    while (n2 < N) n2 <<= 1;
    for (int j = N + threadIdx.x; j < n2; j += BLOCK) sm.u.cb.keys[j] = 0ull;
    __syncthreads();
    bitonic_sort_desc(sm.u.cb.keys, n2);
}

// Sorts the list's N keys (64 < N <= BLOCK) descending into sm.u.cb.keys[0, N): one key per
// thread in registers; strides below 64 exchange within the wave (DPP / permlane), larger
// ones through two alternating LDS buffers (one barrier each).
__device__ __forceinline__ void sort_list_regs(Smem& sm, int N) {
    static_assert(3 * BLOCK <= NMAX, "exchange buffers");
    const int j = threadIdx.x;
    int n = 128;
    while (n < N) n <<= 1;
    uint64_t key = j < N ? sm.u.cb.keys[j] : 0ull;  // padding (0) sorts last
    key = bitonic_wave_strides<1>(key, j, (j & 2) == 0);
    key = bitonic_wave_strides<2>(key, j, (j & 4) == 0);
    key = bitonic_wave_strides<4>(key, j, (j & 8) == 0);
    key = bitonic_wave_strides<8>(key, j, (j & 16) == 0);
    key = bitonic_wave_strides<16>(key, j, (j & 32) == 0);
    key = bitonic_wave_strides<32>(key, j, (j & 64) == 0);
    int buf = 0;
    for (int size = 128; size <= n; size <<= 1) {
        const bool desc = (j & size) == 0;
        for (int stride = size >> 1; stride >= WAVE; stride >>= 1) {
            uint64_t* b = sm.u.cb.keys + BLOCK * (1 + buf);
            b[j] = key;
            __syncthreads();
            const uint64_t other = b[j ^ stride];
            buf ^= 1;
            const bool take_max = ((j & stride) == 0) == desc;
            const uint64_t mx = other > key ? other : key, mn = other > key ? key : other;
            key = take_max ? mx : mn;
        }
        key = bitonic_wave_strides<32>(key, j, desc);
    }
    if (j < N) sm.u.cb.keys[j] = key;
    __syncthreads();
}

// Re-reads chunk c: appends its non-history elements with value >= th to the list.
template <bool BF16, int VEC>
__device__ __forceinline__ void rescan_collect(const KArgs& a, Smem& sm, const RowCtx& C, uint32_t c, float th,
                                               bool sorted) {
    const PenSrc P{true, nullptr, nullptr, nullptr};
    span_pass<BF16, VEC, true>(a, sm, C, P, chunk_lo(a, c), chunk_hi(a, c), [&](uint32_t id, float v) {
        if (v >= th && v > -__builtin_inff()) {
            const uint32_t slot = lds_add(&sm.misc[MISC_N], 1u);
            if (slot < NMAX) sm.u.cb.keys[slot] = sorted ? key64(v, id) : (((uint64_t)(~id) << 32) | ord32(v));
        }
    });
}

enum { CB_DONE = 0, CB_RADIX = 1 };

// N in (64, NMAX] candidates: one bitonic sort in LDS, then f64 scans. Returns CB_DONE, or
// -1 when the list does not decide the cut (nothing has been written then).
__device__ __forceinline__ int combine_list(const KArgs& a, Smem& sm, const RowCtx& C, int N, bool sorted, float M,
                                            float S, ArgMax rawmax, bool exhaustive, bool minp_complete,
                                            int64_t tb) {
    const int tid = threadIdx.x;
    sort_list(sm, N);
    BFI_TRACE(a, tb, 5);
    // probabilities of the sorted positions: p = expf(s - M) / S (sample.rs:383, 388)
    for (int j = tid; j < N; j += BLOCK) {
        const uint64_t k = sm.u.cb.keys[j];
        const float s = sorted ? key_s(k) : unord32((uint32_t)k);
        sm.u.cb.p[j] = expf(s - M) / S;
    }
    __syncthreads();
    auto idx_at = [&](int j) -> uint32_t {
        const uint64_t k = sm.u.cb.keys[j];
        return sorted ? key_idx(k) : ~(uint32_t)(k >> 32);
    };
    const float* p = sm.u.cb.p;

    const int64_t Lk = C.kmode ? C.k : a.V;
    int64_t Lp = Lk, Lm = L_UNKNOWN;
    const int lim = (int)(Lk < N ? Lk : N);
    if (sorted && C.pmode) {  // sample.rs:397-409
        const uint32_t j = first_cum_ge(sm, lim, [&](int i) { return (double)p[i]; }, [](int) { return true; },
                                        (double)C.top_p);
        if (j != 0xFFFFFFFFu) Lp = (int64_t)j + 1;
        else if (!(Lk <= N || exhaustive)) Lp = L_UNKNOWN;
    }
    float thresh = 0.0f;
    if (C.mmode) {  // sample.rs:411-414
        thresh = C.min_p * (1.0f / S);
        if (sorted) {
            const int64_t trunc = min(Lk, Lp);
            const int n_in = (int)(trunc < N ? trunc : N);
            const uint32_t j = first_cum_ge(sm, n_in, [&](int i) { return p[i] >= thresh ? 0.0 : 1.0; },
                                            [](int) { return true; }, 0.5);
            if (j != 0xFFFFFFFFu) Lm = (int64_t)j;
            else if (trunc <= N) Lm = trunc;
            else if (minp_complete || exhaustive) Lm = N;
        } else {
            uint32_t c = 0;
            for (int j = tid; j < N; j += BLOCK) c += p[j] >= thresh;
            c = block_sum_u(c, sm.ru);
            if (minp_complete || exhaustive) Lm = c;
        }
        if (Lm == 0) {  // sample.rs:415-422: argmax of the masked, un-penalized logits
            const uint32_t tok = rawmax.v > -__builtin_inff() ? rawmax.i : 0u;
            finish_token(a, sm, C, tok);
            return CB_DONE;
        }
    }
    int64_t L;
    if (sorted) {
        if (!resolve_L(Lk, Lp, C.mmode ? Lm : L_UNKNOWN, N, exhaustive, L)) return -1;
    } else {
        if (Lm == L_UNKNOWN) return -1;
        L = Lm;
    }
    const int nl = sorted ? (int)(L < N ? L : N) : N;  // list positions that can be kept
    auto kept = [&](int j) -> bool { return sorted ? j < nl : (p[j] >= thresh); };
    auto wk = [&](int j) -> double { return kept(j) ? (double)p[j] : 0.0; };

    // target introspection: kept entries with p > 0 in draw order
    if (a.t_kind) {
        if (tid == 0) {
            a.t_kind[C.row] = BFI_SMP_TARGET_WEIGHTS;
            a.t_kept[C.row] = (int32_t)L;
        }
        uint32_t c = 0;
        for (int j = tid * PT; j < tid * PT + PT; j++) c += (j < nl && kept(j) && p[j] > 0.0f);
        uint32_t tc;
        uint32_t o = block_excl_scan<uint32_t>(c, sm.ru, tc);
        for (int j = tid * PT; j < tid * PT + PT; j++) {
            if (j < nl && kept(j) && p[j] > 0.0f) {
                if ((int64_t)o < a.t_cap) {
                    a.t_ids[(int64_t)C.row * a.t_cap + o] = idx_at(j);
                    a.t_probs[(int64_t)C.row * a.t_cap + o] = p[j];
                }
                o++;
            }
        }
        if (tid == 0) a.t_listed[C.row] = (int32_t)(tc < a.t_cap ? tc : a.t_cap);
    }

    const double sum = list_sum(sm, nl, wk);
    if (!C.judged) {  // draw (sample.rs:312-323)
        const double r = (double)C.u * sum;
        const uint32_t j = first_cum_ge(sm, nl, wk, kept, r);
        const uint32_t tok = j == 0xFFFFFFFFu ? 0u : idx_at((int)j);
        if (a.t_kind && tid == 0 && a.out_tok) a.out_tok[C.row] = tok;
        emit(a, sm, C, tok, 1u);
        return CB_DONE;
    }
    // judge (spec.rs:83-95)
    uint32_t pd = 0xFFFFFFFFu;
    for (int j = tid; j < nl; j += BLOCK)
        if (kept(j) && idx_at(j) == C.draft) pd = (uint32_t)j;
    pd = block_min_u(pd, sm.ru);
    const double p_d = pd == 0xFFFFFFFFu ? 0.0 : (double)p[pd];
    if (sum > 0.0 && (double)C.u < p_d / sum) {
        emit(a, sm, C, C.draft, 1u);
        return CB_DONE;
    }
    uint32_t pos = 0;
    for (int j = tid; j < nl; j += BLOCK) pos += (kept(j) && (uint32_t)j != pd && p[j] > 0.0f);
    pos = block_sum_u(pos, sm.ru);
    if (pos == 0) {  // residual empty or all <= 0: Accept (spec.rs:90-93)
        emit(a, sm, C, C.draft, 1u);
        return CB_DONE;
    }
    auto wr = [&](int j) -> double { return (kept(j) && (uint32_t)j != pd) ? (double)p[j] : 0.0; };
    const double r2 = (double)C.u2 * (sum - p_d);
    const uint32_t j = first_cum_ge(sm, nl, wr, [&](int i) { return kept(i) && (uint32_t)i != pd; }, r2);
    emit(a, sm, C, j == 0xFFFFFFFFu ? 0u : idx_at((int)j), 0u);
    return CB_DONE;
}



// Exclusive prefix of the chunks' candidate counts into sm.cpre (sm.cpre[nc] = total).
// Rows of at most 64 chunks use wave 0 alone. Needs a barrier before sm.cpre is read.
__device__ __forceinline__ void chunk_prefix(Smem& sm, int nc, uint32_t myn) {
    const int tid = threadIdx.x;
    if (nc <= WAVE) {
        if (wave_id() == 0) {
            const uint32_t incl = wave_scan_incl(myn, 0u, [](uint32_t x, uint32_t y) { return x + y; });
            if (tid < nc) sm.cpre[tid] = incl - myn;
            const uint32_t tot = lane63(incl);
            if (tid == 0) sm.cpre[nc] = tot;
        }
    } else {
        uint32_t tot;
        const uint32_t off = block_excl_scan<uint32_t>(myn, sm.ru, tot);
        if (tid < nc) sm.cpre[tid] = off;
        if (tid == 0) sm.cpre[nc] = tot;
    }
}

// Appends the history ids whose penalized value is >= th. Every thread calls it.
__device__ __forceinline__ void append_hist(Smem& sm, const RowCtx& C, float th, bool sorted) {
    if (!C.pen_hash) return;
    const int nh = (int)sm.misc[MISC_HN];
    for (int j0 = 0; j0 < nh; j0 += BLOCK) {  // uniform trip count: wave_append below
        const int j = j0 + threadIdx.x;
        const int k = j < nh ? sm.hlist[j] : 0;
        const uint32_t id = sm.hkey[k];
        const float v = sm.hpen[k];
        const bool take = j < nh && v >= th && v > -__builtin_inff();
        const uint32_t slot = wave_append(&sm.misc[MISC_N], take);
        if (take && slot < NMAX) sm.u.cb.keys[slot] = sorted ? key64(v, id) : (((uint64_t)(~id) << 32) | ord32(v));
    }
}


// Top-k rows whose list above th holds more than NMAX entries: a bound t >= th with at least
// k entries at or above it (and, buckets being narrow, usually few more), from a histogram
// of the entries' values in 1/32-wide buckets below M (2048 buckets). The entries are the
// current candidate ranges (sm.cpre) and the history ids. Returns th when the k-th largest
// lies in the last bucket.
__device__ __forceinline__ float topk_bound(const KArgs& a, Smem& sm, const RowCtx& C, float M, float th) {
    constexpr int NBK = 2048;
    constexpr float R = 32.0f;
    constexpr int BPT = NBK / BLOCK;
    const int tid = threadIdx.x;
    const int nc = a.n_chunks;
    uint32_t* cnt = reinterpret_cast<uint32_t*>(sm.u.cb.keys);  // the list is rebuilt afterwards
    for (int b = tid; b < NBK; b += BLOCK) cnt[b] = 0u;
    __syncthreads();
    auto bucket = [&](float v) -> uint32_t {
        const float d = (M - v) * R;
        return d < (float)(NBK - 1) ? (uint32_t)d : (uint32_t)(NBK - 1);
    };
    for (uint32_t b0 = 0; b0 < sm.cpre[nc]; b0 += GU * BLOCK) {  // uniform trip count
        const CandBatch B = load_cands(a, sm, C.row, nc, b0);
#pragma unroll
        for (int g = 0; g < GU; g++) {
            const float v = raw_value(C, B.cd[g].x, true);
            if (v >= th && v > -__builtin_inff() && !(C.pen_hash && hist_find(sm, B.cd[g].idx) >= 0))
                lds_add(&cnt[bucket(v)], 1u);
        }
    }
    if (C.pen_hash) {
        for (int j = tid; j < (int)sm.misc[MISC_HN]; j += BLOCK) {
            const float v = sm.hpen[sm.hlist[j]];
            if (v >= th && v > -__builtin_inff()) lds_add(&cnt[bucket(v)], 1u);
        }
    }
    __syncthreads();
    uint32_t loc[BPT], run = 0;
#pragma unroll
    for (int i = 0; i < BPT; i++) {
        run += cnt[tid * BPT + i];
        loc[i] = run;
    }
    uint32_t tot;
    const uint32_t pre = block_excl_scan<uint32_t>(run, sm.ru, tot);
    uint32_t hit = 0xFFFFFFFFu;
#pragma unroll
    for (int i = 0; i < BPT; i++)
        if (hit == 0xFFFFFFFFu && pre + loc[i] >= (uint32_t)C.k) hit = (uint32_t)(tid * BPT + i);
    hit = block_min_u(hit, sm.ru);
    if (hit >= (uint32_t)(NBK - 1)) return th;
    // every entry of buckets 0..hit is >= this (the margins cover the rounding of the index)
    const float t = M - ((float)(hit + 1) / R) * (1.0f + 1e-6f) - 1e-6f * (fabsf(M) + 1.0f);
    return fmaxf(th, t);
}

// `th_raw`: every non-history element >= th_raw is some chunk's candidate (the largest chunk
// bound). `list_ready`: the first pass's list (complete above max(th_raw, min-p bound)) is
// already in sm.u.cb.keys with its length in MISC_N. `need_hash()` runs before the second
// pass, whose chunk re-reads take the penalties from the LDS history hash.
template <bool BF16, int VEC, typename F>
__device__ __forceinline__ int combine_bounded(const KArgs& a, Smem& sm, const RowCtx& C, const ChunkPart& mine,
                                               float M, float S, ArgMax rawmax, float th_raw, bool list_ready,
                                               int64_t tb, F need_hash) {
    const int tid = threadIdx.x;
    const int nc = a.n_chunks;
    const bool sorted = C.kmode || C.pmode;  // else min-p only: index order (sample.rs:411-414)
    const float th_m = minp_bound(C, M);
    float th = fmaxf(th_raw, th_m);
    for (int pass = 0; pass < 2; pass++) {
        if (pass) need_hash();
        // ---- the list: complete above th
        if (!(pass == 0 && list_ready)) {
            chunk_prefix(sm, nc, tid < nc ? chunk_take(mine, th) : 0u);
            if (tid == 0) sm.misc[MISC_N] = 0;
            __syncthreads();
            for (uint32_t b0 = 0; b0 < sm.cpre[nc]; b0 += GU * BLOCK)  // uniform trip count
                append_cands(sm, C, load_cands(a, sm, C.row, nc, b0), th, sorted, HistExcl{sm, C});
            append_hist(sm, C, th, sorted);
            __syncthreads();
            // re-read the chunks whose candidates stop above th (repair pass)
            if (pass) {
                for (int c = 0; c < nc; c++) {
                    const float tc = sm.cm[c] >= th ? a.parts[(int64_t)C.row * nc + c].theta : -__builtin_inff();
                    if (tc > th) rescan_collect<BF16, VEC>(a, sm, C, (uint32_t)c, th, sorted);
                }
                __syncthreads();
            }
        }
        int N = (int)sm.misc[MISC_N];
        if (N > NMAX && pass == 0 && C.kmode && C.k <= NMAX / 2) {
            // top-k needs only the k largest: raise th to a bound holding about k entries
            th = topk_bound(a, sm, C, M, th);
            if (tid == 0) sm.misc[MISC_N] = 0;
            __syncthreads();
            for (uint32_t b0 = 0; b0 < sm.cpre[nc]; b0 += GU * BLOCK)  // uniform trip count
                append_cands(sm, C, load_cands(a, sm, C.row, nc, b0), th, sorted, HistExcl{sm, C});
            append_hist(sm, C, th, sorted);
            __syncthreads();
            N = (int)sm.misc[MISC_N];
        }
        BFI_TRACE(a, tb, 4);
        if (a.trace && tid == 0) sm.tr[6] = ((uint64_t)sm.cpre[nc] << 32) | (uint32_t)N;
        if (N > NMAX) return CB_RADIX;
        const bool exhaustive = !(th > -__builtin_inff());
        const bool minp_complete = th <= th_m;
        if (N <= WAVE) {
            if (combine_wave<1>(a, sm, C, N, sorted, M, S, rawmax, exhaustive, minp_complete)) return CB_DONE;
        } else if (N <= 8 * WAVE) {
            if (N <= BLOCK) sort_list_regs(sm, N);
            else sort_list(sm, N);
            BFI_TRACE(a, tb, 5);
            if (combine_wave<8>(a, sm, C, N, sorted, M, S, rawmax, exhaustive, minp_complete)) return CB_DONE;
        } else {
            const int r = combine_list(a, sm, C, N, sorted, M, S, rawmax, exhaustive, minp_complete, tb);
            if (r >= 0) return r;
        }
        // the cut lies below th: list down to the min-p bound, or everything
        th = C.mmode ? th_m : -__builtin_inff();
    }
    return CB_RADIX;
}

// ---- combine: draws in index order (no top-k/top-p) ------------------------------------
//
// Rows without top-k/top-p keep every element (or, with min-p, the retained ones) in index
// order (sample.rs:411-414). The draw finds its chunk from per-chunk kept masses, then
// re-reads that one chunk.

// Kept weights of one tile of [t0, t1): p = expf(s - M) / S when p >= thresh, else 0
// (and 0 outside the tile and for `excl`).
template <bool BF16, int VEC>
__device__ __forceinline__ void tile_weights(const KArgs& a, const Smem& sm, const RowCtx& C, const PenSrc& P,
                                             uint32_t t0, uint32_t t1, float M, float S, float thresh, uint32_t excl,
                                             float (&x)[VEC][Elem<BF16>::EPV]) {
    constexpr int EPV = Elem<BF16>::EPV;
    RawTile<BF16, VEC> r;
    load_raw<BF16, VEC>(a, C, P, t0, t1, r);
#pragma unroll
    for (int q = 0; q < VEC; q++) unpack16<BF16, VEC>(r.w[q], x[q]);
    transform_raw<BF16, VEC>(sm, C, P, t0, t1, r, x);
#pragma unroll
    for (int q = 0; q < VEC; q++)
#pragma unroll
        for (int e = 0; e < EPV; e++) {
            const uint32_t id = t0 + (uint32_t)(q * BLOCK + threadIdx.x) * EPV + e;
            const float p = expf(x[q][e] - M) / S;
            x[q][e] = (id < t1 && id != excl && p >= thresh) ? p : 0.0f;
        }
}

// Re-reads chunk [c0, c1) and returns the first index (in index order) with a positive
// weight where the cumulative weight reaches frac * (chunk total).
template <bool BF16, int VEC>
__device__ __forceinline__ uint32_t scan_chunk_index_order(const KArgs& a, Smem& sm, const RowCtx& C,
                                                           const PenSrc& P, uint32_t c0, uint32_t c1, float M, float S,
                                                           float thresh, uint32_t excl, double frac) {
    constexpr int EPV = Elem<BF16>::EPV;
    constexpr uint32_t TILE = (uint32_t)BLOCK * VEC * EPV;
    const int tid = threadIdx.x;
    float x[VEC][EPV];
    double tsum = 0.0;
    for (uint32_t t0 = c0; t0 < c1; t0 += TILE) {
        tile_weights<BF16, VEC>(a, sm, C, P, t0, min(t0 + TILE, c1), M, S, thresh, excl, x);
#pragma unroll
        for (int q = 0; q < VEC; q++)
#pragma unroll
            for (int e = 0; e < EPV; e++) tsum += x[q][e];
    }
    const double target = frac * block_sum_d(tsum, sm.rd);
    double carry = 0.0;
    uint32_t found = 0xFFFFFFFFu, lastpos = 0;
    for (uint32_t t0 = c0; t0 < c1 && found == 0xFFFFFFFFu; t0 += TILE) {
        const uint32_t t1 = min(t0 + TILE, c1);
        tile_weights<BF16, VEC>(a, sm, C, P, t0, t1, M, S, thresh, excl, x);
#pragma unroll
        for (int q = 0; q < VEC; q++) {  // VEC slabs in index order
            double ts = 0.0;
#pragma unroll
            for (int e = 0; e < EPV; e++) {
                ts += x[q][e];
                const uint32_t id = t0 + (uint32_t)(q * BLOCK + tid) * EPV + e;
                if (x[q][e] > 0.0f) lastpos = max(lastpos, id + 1);
            }
            double tot;
            const double pre = block_excl_scan<double>(ts, sm.rd, tot);
            if (found == 0xFFFFFFFFu && carry + tot >= target) {
                uint32_t best = 0xFFFFFFFFu;
                double c = carry + pre;
#pragma unroll
                for (int e = 0; e < EPV; e++) {
                    const uint32_t id = t0 + (uint32_t)(q * BLOCK + tid) * EPV + e;
                    c += x[q][e];
                    if (best == 0xFFFFFFFFu && x[q][e] > 0.0f && c >= target) best = id;
                }
                found = block_min_u(best, sm.ru);
            }
            carry += tot;
        }
    }
    if (found == 0xFFFFFFFFu) {  // rounding at the chunk end: last positive element
        const uint32_t l = (uint32_t)block_max_u64(lastpos, sm.r64);
        found = l ? l - 1 : c0;
    }
    return found;
}

// Penalized value s of one element (the draft of a judged row).
__device__ __forceinline__ float element_s(const KArgs& a, Smem& sm, const RowCtx& C, uint32_t id, bool bf16,
                                           bool hashed) {
    const int tid = threadIdx.x;
    if (id >= (uint32_t)a.V) return -__builtin_inff();  // a draft outside the vocabulary
    float x;
    if (bf16)
        x = __uint_as_float((uint32_t)((const uint16_t*)a.logits)[(int64_t)C.row * a.row_stride + id] << 16);
    else
        x = ((const float*)a.logits)[(int64_t)C.row * a.row_stride + id];
    const bool allowed = !C.mrow || ((C.mrow[id >> 5] >> (id & 31)) & 1u);
    uint32_t c = 0;
    if (C.pen_on) {
        if (hashed && C.pen_hash) {
            const int k = hist_find(sm, id);
            c = k >= 0 ? sm.hcnt[k] : 0u;
        } else {
            const int64_t H = C.h.size();
            for (int64_t j = tid; j < H; j += BLOCK) c += C.h.at(j) == id;
            c = block_sum_u(c, sm.ru);
        }
    }
    return c ? pen_value(C, x, allowed, c) : raw_value(C, x, allowed);
}

// `mc` = this thread's chunk (tid < n_chunks) kept mass, normalized by S; `n_kept` = the
// kept count (sample.rs:411-414; V when nothing is filtered).
template <bool BF16, int VEC>
__device__ __forceinline__ void combine_index_order(const KArgs& a, Smem& sm, const RowCtx& C, const PenSrc& P,
                                                    bool hashed, float M, float S, float thresh, double mc,
                                                    uint32_t n_kept) {
    const int tid = threadIdx.x;
    const int nc = a.n_chunks;
    uint32_t pd_chunk = 0xFFFFFFFFu;
    double p_d = 0.0;
    if (C.judged && C.draft < (uint32_t)a.V) {
        const float sd = element_s(a, sm, C, C.draft, BF16, hashed);
        const float pf = expf(sd - M) / S;
        if (pf >= thresh) {  // the draft is kept
            p_d = (double)pf;
            pd_chunk = C.draft / (uint32_t)a.chunk;
            if ((uint32_t)tid == pd_chunk) mc = mc > p_d ? mc - p_d : 0.0;
        }
    }
    double total;
    const double pre = block_excl_scan<double>(tid < nc ? mc : 0.0, sm.rd, total);
    const double sum = total + p_d;  // sum of kept weights
    if (a.t_kind && tid == 0) {
        a.t_kind[C.row] = BFI_SMP_TARGET_WEIGHTS;
        a.t_kept[C.row] = (int32_t)n_kept;
        a.t_listed[C.row] = 0;
    }
    float u = C.u;
    bool resid = false;
    if (C.judged) {  // spec.rs:83-95
        if (sum > 0.0 && (double)C.u < p_d / sum) {
            emit(a, sm, C, C.draft, 1u);
            return;
        }
        if (!(total > 0.0)) {  // residual empty or all <= 0
            emit(a, sm, C, C.draft, 1u);
            return;
        }
        u = C.u2;
        resid = true;
    }
    const double r = (double)u * total;
    uint32_t tok;
    if (r <= 0.0 && thresh == 0.0f) {
        // r = 0 picks the first element of the list, whatever its weight (sample.rs:314-319)
        tok = (resid && C.draft == 0) ? 1u : 0u;
    } else {
        uint32_t c = 0xFFFFFFFFu;
        if (tid < nc && mc > 0.0 && pre + mc >= r) c = (uint32_t)tid;
        c = block_min_u(c, sm.ru);
        if (c == 0xFFFFFFFFu) {  // rounding: last chunk with mass
            uint32_t l = (tid < nc && mc > 0.0) ? (uint32_t)tid + 1 : 0u;
            l = (uint32_t)block_max_u64(l, sm.r64);
            c = l ? l - 1 : 0;
        }
        // mass before chunk c and the chunk's own mass
        if ((uint32_t)tid == c) {
            sm.rd[0] = pre;
            sm.rd[1] = mc;
        }
        __syncthreads();
        const double before = sm.rd[0], mass = sm.rd[1];
        __syncthreads();
        double frac = mass > 0.0 ? (r - before) / mass : 0.0;
        frac = frac < 0.0 ? 0.0 : (frac > 1.0 ? 1.0 : frac);
        tok = scan_chunk_index_order<BF16, VEC>(a, sm, C, P, chunk_lo(a, c), chunk_hi(a, c), M, S, thresh,
                                                resid ? C.draft : 0xFFFFFFFFu, frac);
    }
    if (a.t_kind && tid == 0 && a.out_tok) a.out_tok[C.row] = tok;
    emit(a, sm, C, tok, resid ? 0u : 1u);
}

// Index-order rows. `known` = this thread's chunk mass `mc` (normalized by S) is given
// (unfiltered rows, from the streaming pass); otherwise one pass per chunk computes each
// chunk's kept mass and count (min-p rows the candidate lists do not cover, rows with an
// oversized history).
template <bool BF16, int VEC>
__device__ __forceinline__ void combine_index_order_passes(const KArgs& a, Smem& sm, const RowCtx& C, const PenSrc& P,
                                                           bool hashed, float M, float S, ArgMax rawmax, bool known,
                                                           double mc) {
    const int tid = threadIdx.x;
    const int nc = a.n_chunks;
    const float thresh = C.mmode ? C.min_p * (1.0f / S) : 0.0f;  // sample.rs:411-414
    uint32_t cnt = (uint32_t)a.V;
    if (!known) {
        mc = 0.0;
        cnt = 0;
        for (int c = 0; c < nc; c++) {
            double w = 0.0;
            span_pass<BF16, VEC, false>(a, sm, C, P, chunk_lo(a, c), chunk_hi(a, c), [&](uint32_t, float s) {
                const float p = expf(s - M) / S;
                if (p >= thresh) {
                    w += (double)p;
                    cnt++;
                }
            });
            w = block_sum_d(w, sm.rd);
            if (tid == c) mc = w;
        }
        cnt = block_sum_u(cnt, sm.ru);
        if (C.mmode && cnt == 0) {  // sample.rs:415-422
            finish_token(a, sm, C, rawmax.v > -__builtin_inff() ? rawmax.i : 0u);
            return;
        }
    }
    combine_index_order<BF16, VEC>(a, sm, C, P, hashed, M, S, thresh, mc, cnt);
}

// ---- combine: radix select over the row ------------------------------------------------

struct Sel {
    uint64_t key;       // selected element
    uint64_t pos;       // its 0-based position in the sorted order
    uint64_t cum_mass;  // fixed-point mass through it (inclusive)
};

// One pass over the whole row: f(id, s) for every element (s = penalized value).
template <bool BF16, int VEC, typename F>
__device__ __forceinline__ void row_pass(const KArgs& a, Smem& sm, const RowCtx& C, const PenSrc& P, F f) {
    span_pass<BF16, VEC, false>(a, sm, C, P, 0u, (uint32_t)a.V, f);
}

// Finds the element at a sorted position (kind 0: 0-based position `target`) or the first
// element whose inclusive fixed-point cumulative mass reaches `target` (kind 1), over the
// order of key64 descending, skipping the element with key `excl`: 10-bit key digits from
// the top, one row pass per digit. The general fallback of vsel_query (targets among -inf
// elements, value buckets too dense to sort in LDS).
template <bool BF16, int VEC>
__device__ __forceinline__ Sel radix_select(const KArgs& a, Smem& sm, const RowCtx& C, const PenSrc& P, float M,
                            double scale, int kind, uint64_t target, uint64_t excl, uint64_t excl_mass) {
    const int tid = threadIdx.x;
    uint64_t prefix = 0;
    int pbits = 0;
    uint64_t before_cnt = 0, before_mass = 0;
    (void)excl_mass;
    for (;;) {  // one 10-bit digit of the key per round
        const int w = (64 - pbits) >= 10 ? 10 : 64 - pbits;
        const int shift = 64 - pbits - w;
        const uint32_t nb = 1u << w;
        {
            for (uint32_t b = tid; b < NBUCKET; b += BLOCK) {
                sm.u.hs.mass[b] = 0;
                sm.u.hs.cnt[b] = 0;
            }
            __syncthreads();
            row_pass<BF16, VEC>(a, sm, C, P, [&](uint32_t id, float s) __attribute__((always_inline)) {
                uint64_t k = key64(s, id);
                if (k == excl) return;
                if (pbits && (k >> (64 - pbits)) != prefix) return;
                uint32_t b = (uint32_t)(k >> shift) & (nb - 1);
                lds_add(&sm.u.hs.cnt[b], 1u);
                uint64_t m = efix_of(s, M, scale);
                if (m) lds_add64(&sm.u.hs.mass[b], m);
            });
            __syncthreads();
        }
        // scan buckets from the top (o = 0 is bucket nb-1); BPT buckets per thread
        constexpr int BPT = NBUCKET / BLOCK;
        uint64_t lc[BPT], lm[BPT];
        uint64_t rc = 0, rm = 0;
#pragma unroll
        for (int i = 0; i < BPT; i++) {
            uint32_t o = (uint32_t)tid * BPT + i;
            uint32_t b = nb - 1 - o;
            uint64_t c = o < nb ? sm.u.hs.cnt[b] : 0, m = o < nb ? sm.u.hs.mass[b] : 0;
            rc += c;
            rm += m;
            lc[i] = rc;
            lm[i] = rm;
        }
        uint64_t tc, tm;
        uint64_t pc = block_excl_scan<uint64_t>(rc, sm.r64, tc);
        uint64_t pm = block_excl_scan<uint64_t>(rm, sm.r64b, tm);
        uint32_t hit = 0xFFFFFFFFu;
#pragma unroll
        for (int i = 0; i < BPT; i++) {
            uint32_t o = (uint32_t)tid * BPT + i;
            const uint32_t bc = o < nb ? sm.u.hs.cnt[nb - 1 - o] : 0u;
            bool ok = kind == 0 ? (before_cnt + pc + lc[i] > target)
                                : (bc > 0 && before_mass + pm + lm[i] >= target);
            if (hit == 0xFFFFFFFFu && o < nb && ok) hit = o;
        }
        hit = block_min_u(hit, sm.ru);
        if (hit == 0xFFFFFFFFu) {  // target beyond the total: the last non-empty bucket
            uint32_t l = 0;
            for (uint32_t o = tid; o < nb; o += BLOCK)
                if (sm.u.hs.cnt[nb - 1 - o] > 0) l = max(l, o + 1);
            l = (uint32_t)block_max_u64(l, sm.r64);
            hit = l ? l - 1 : nb - 1;
        }
        // counts/mass above the chosen bucket
        if ((uint32_t)tid == hit / BPT) {
            const int i = (int)(hit % BPT);
            uint64_t cab = pc, mab = pm;
#pragma unroll
            for (int ii = 0; ii < BPT; ii++) {
                if (ii + 1 == i) {
                    cab = pc + lc[ii];
                    mab = pm + lm[ii];
                }
            }
            sm.r64[0] = cab;
            sm.r64b[0] = mab;
            sm.r64[1] = sm.u.hs.cnt[nb - 1 - hit];
        }
        __syncthreads();
        before_cnt += sm.r64[0];
        before_mass += sm.r64b[0];
        const uint64_t nbk = sm.r64[1];
        __syncthreads();
        prefix = (prefix << w) | (uint64_t)(nb - 1 - hit);
        pbits += w;
        if (nbk <= (uint64_t)NMAX || pbits >= 64) {
            // gather the bucket, sort it, walk it
            if (tid == 0) sm.misc[MISC_N] = 0;
            __syncthreads();
            row_pass<BF16, VEC>(a, sm, C, P, [&](uint32_t id, float s) __attribute__((always_inline)) {
                uint64_t k = key64(s, id);
                if (k == excl) return;
                if ((k >> (64 - pbits)) != prefix) return;
                uint32_t slot = lds_add(&sm.misc[MISC_N], 1u);
                if (slot < NMAX) sm.u.cb.keys[slot] = k;
            });
            __syncthreads();
            int N = (int)min(sm.misc[MISC_N], (uint32_t)NMAX);
            int n2 = 64;
            while (n2 < N) n2 <<= 1;
            for (int j = N + tid; j < n2; j += BLOCK) sm.u.cb.keys[j] = 0ull;
            __syncthreads();
            bitonic_sort_desc(sm.u.cb.keys, n2);
            // masses of the sorted bucket
            uint64_t loc[PT];
            uint64_t run = 0;
#pragma unroll
            for (int i = 0; i < PT; i++) {
                int j = tid * PT + i;
                run += j < N ? efix_of(key_s(sm.u.cb.keys[j]), M, scale) : 0ull;
                loc[i] = run;
            }
            uint64_t tot;
            uint64_t pre = block_excl_scan<uint64_t>(run, sm.r64, tot);
            uint32_t best = 0xFFFFFFFFu;
#pragma unroll
            for (int i = 0; i < PT; i++) {
                int j = tid * PT + i;
                if (best != 0xFFFFFFFFu || j >= N) continue;
                bool ok = kind == 0 ? (before_cnt + (uint64_t)j >= target)
                                    : (before_mass + pre + loc[i] >= target);
                if (ok) best = (uint32_t)j;
            }
            best = block_min_u(best, sm.ru);
            if (best == 0xFFFFFFFFu) best = N > 0 ? (uint32_t)N - 1 : 0u;
            Sel r;
            if ((uint32_t)tid == best / PT) {
                const int i = (int)(best % PT);
                uint64_t li = 0;
#pragma unroll
                for (int ii = 0; ii < PT; ii++)
                    if (ii == i) li = loc[ii];
                sm.r64[0] = sm.u.cb.keys[best];
                sm.r64[1] = before_mass + pre + li;
            }
            __syncthreads();
            r.key = sm.r64[0];
            r.cum_mass = sm.r64[1];
            r.pos = before_cnt + best;
            __syncthreads();
            return r;
        }
    }
}

// ---- row select by value buckets ------------------------------------------------------
//
// Bucket b holds the elements with (M - s) * 32 in [b, b + 1); the last bucket also takes
// everything further below M. -inf elements (mass 0, last in the order) are in none. A
// query finds its bucket from the bucket prefix, then gathers that bucket in one row pass,
// sorts it in LDS and walks it.

__device__ __forceinline__ uint32_t vbucket(float s, float M) {
    const float d = (M - s) * 32.0f;
    return d < (float)(NVB - 1) ? (uint32_t)d : (uint32_t)(NVB - 1);
}

// The row's value histogram (count, fixed-point mass), saved to global scratch for every
// query of this row; returns the total fixed-point mass. *n_finite receives the count.
template <bool BF16, int VEC>
__device__ __forceinline__ uint64_t vsel_l1(const KArgs& a, Smem& sm, const RowCtx& C, const PenSrc& P, float M,
                                            double scale, uint64_t* n_finite) {
    const int tid = threadIdx.x;
    for (uint32_t b = tid; b < NVB; b += BLOCK) {
        sm.u.hs.mass[b] = 0;
        sm.u.hs.cnt[b] = 0;
    }
    __syncthreads();
    row_pass<BF16, VEC>(a, sm, C, P, [&](uint32_t, float s) __attribute__((always_inline)) {
        if (!(s > -__builtin_inff())) return;
        const uint32_t b = vbucket(s, M);
        lds_add(&sm.u.hs.cnt[b], 1u);
        const uint64_t m = efix_of(s, M, scale);
        if (m) lds_add64(&sm.u.hs.mass[b], m);
    });
    __syncthreads();
    uint64_t* saved = a.row_hist + (int64_t)C.row * NVB * 2;
    uint64_t m = 0, c = 0;
    for (uint32_t b = tid; b < NVB; b += BLOCK) {
        saved[2 * b] = sm.u.hs.mass[b];
        saved[2 * b + 1] = sm.u.hs.cnt[b];
        m += sm.u.hs.mass[b];
        c += sm.u.hs.cnt[b];
    }
    uint64_t tot, ctot;
    block_excl_scan<uint64_t>(m, sm.r64, tot);
    block_excl_scan<uint64_t>(c, sm.r64b, ctot);
    *n_finite = ctot;
    __syncthreads();
    return tot;
}

// The query expected after a top-p cut, whose buckets the cut's gather collects ahead:
// mode 1, the draw at ceil(u * kept); mode 2, the residual draw of a verify row at
// ceil(u * (kept - md)) without the draft (bucket bd, mass md) when the draft is kept, at
// ceil(u * kept) when it is not.
struct SpecReq {
    int mode;
    double u;
    uint64_t md;
    uint32_t bd;
};

// radix_select's query by value buckets (vsel_l1 must have run for this row). With `sr`, the
// gather also collects the buckets the following query can need (the kept mass lies between
// the cut bucket's exclusive and inclusive cumulative masses); a query whose bucket lies in
// the collected range takes it from LDS instead of a pass over the row.
template <bool BF16, int VEC>
__device__ __forceinline__ Sel vsel_query(const KArgs& a, Smem& sm, const RowCtx& C, const PenSrc& P, float M,
                                          double scale, int kind, uint64_t target, uint64_t excl, uint64_t excl_mass,
                                          SpecReq sr = SpecReq{0, 0.0, 0, 0}) {
    constexpr int BPT = NVB / BLOCK;
    const int tid = threadIdx.x;
    const uint64_t* saved = a.row_hist + (int64_t)C.row * NVB * 2;
    const float xs = excl != ~0ull ? key_s(excl) : -__builtin_inff();
    const uint32_t xb = xs > -__builtin_inff() ? vbucket(xs, M) : 0xFFFFFFFFu;
    uint64_t lc[BPT], lm[BPT], bc[BPT];
    uint64_t rc = 0, rm = 0;
#pragma unroll
    for (int i = 0; i < BPT; i++) {
        const uint32_t b = (uint32_t)tid * BPT + i;
        uint64_t m = saved[2 * b], c = saved[2 * b + 1];
        if (b == xb) {  // the excluded element
            c -= 1;
            m -= excl_mass;
        }
        bc[i] = c;
        rc += c;
        rm += m;
        lc[i] = rc;
        lm[i] = rm;
    }
    uint64_t tc, tm;
    const uint64_t pc = block_excl_scan<uint64_t>(rc, sm.r64, tc);
    const uint64_t pm = block_excl_scan<uint64_t>(rm, sm.r64b, tm);
    if (kind == 0 && target >= tc)  // among the -inf elements
        return radix_select<BF16, VEC>(a, sm, C, P, M, scale, kind, target, excl, excl_mass);
    uint32_t hit = 0xFFFFFFFFu;
#pragma unroll
    for (int i = 0; i < BPT; i++) {
        const bool ok = kind == 0 ? (pc + lc[i] > target) : (bc[i] > 0 && pm + lm[i] >= target);
        if (hit == 0xFFFFFFFFu && ok) hit = (uint32_t)tid * BPT + i;
    }
    hit = block_min_u(hit, sm.ru);
    if (hit == 0xFFFFFFFFu) {  // target beyond the total (rounding): the last non-empty bucket
        uint32_t l = 0;
#pragma unroll
        for (int i = 0; i < BPT; i++)
            if (bc[i] > 0) l = (uint32_t)tid * BPT + i + 1;
        l = (uint32_t)block_max_u64(l, sm.r64);
        hit = l ? l - 1 : 0;
    }
    if ((uint32_t)tid == hit / BPT) {
        const int i = (int)(hit % BPT);
        uint64_t cab = pc, mab = pm, nbk = 0;
#pragma unroll
        for (int ii = 0; ii < BPT; ii++) {
            if (ii + 1 == i) {
                cab = pc + lc[ii];
                mab = pm + lm[ii];
            }
            if (ii == i) nbk = bc[ii];
        }
        sm.r64[0] = cab;
        sm.r64b[0] = mab;
        sm.r64[1] = nbk;
        sm.r64b[1] = pm + lm[i];  // inclusive cumulative mass through the bucket
    }
    __syncthreads();
    const uint64_t before_cnt = sm.r64[0], before_mass = sm.r64b[0], nbk = sm.r64[1], incl_mass = sm.r64b[1];
    const bool cached = sm.spec_lo <= hit && hit <= sm.spec_hi;
    __syncthreads();
    if (nbk > (uint64_t)NMAX || nbk == 0)  // too dense to sort in LDS
        return radix_select<BF16, VEC>(a, sm, C, P, M, scale, kind, target, excl, excl_mass);
    // the bucket of mass target t (as `hit` above) when element mass xm in bucket xb is
    // left out
    auto mass_bucket = [&](uint64_t t, uint32_t xb2, uint64_t xm2) __attribute__((always_inline)) {
        uint32_t h = 0xFFFFFFFFu, l = 0;
#pragma unroll
        for (int i = 0; i < BPT; i++) {
            const uint32_t b = (uint32_t)tid * BPT + i;
            const uint64_t c = bc[i] - (b == xb2 ? 1u : 0u);
            const uint64_t cm = pm + lm[i] - (b >= xb2 ? xm2 : 0ull);
            if (h == 0xFFFFFFFFu && c > 0 && cm >= t) h = b;
            if (c > 0) l = b + 1;
        }
        h = block_min_u(h, sm.ru);
        if (h == 0xFFFFFFFFu) {
            l = (uint32_t)block_max_u64(l, sm.r64);
            h = l ? l - 1 : 0;
        }
        return h;
    };
    // inclusive cumulative count through bucket b
    auto cum_cnt = [&](uint32_t b) __attribute__((always_inline)) {
        if ((uint32_t)tid == b / BPT) {
            uint64_t v = 0;
#pragma unroll
            for (int ii = 0; ii < BPT; ii++)
                if ((uint32_t)ii == b % BPT) v = pc + lc[ii];
            sm.r64[2] = v;
        }
        __syncthreads();
        const uint64_t v = sm.r64[2];
        __syncthreads();
        return v;
    };
    uint32_t slo = 1u, shi = 0u;
    if (sr.mode && !cached && excl == ~0ull) {
        const bool can_drop = sr.mode == 1 || sr.bd >= hit;  // the draft may be outside the kept set
        const bool can_keep = sr.mode == 2 && sr.bd <= hit;
        slo = 0xFFFFFFFFu;
        shi = 0u;
        if (can_drop) {  // ceil(u * kept), kept in [before, incl]
            slo = min(slo, mass_bucket((uint64_t)ceil(sr.u * (double)before_mass), 0xFFFFFFFFu, 0ull));
            shi = max(shi, mass_bucket((uint64_t)ceil(sr.u * (double)incl_mass), 0xFFFFFFFFu, 0ull));
        }
        if (can_keep) {  // ceil(u * (kept - md)) without the draft, kept - md in [lo, incl - md]
            const uint64_t lo = sr.bd < hit ? before_mass - sr.md : before_mass;
            slo = min(slo, mass_bucket((uint64_t)ceil(sr.u * (double)lo), sr.bd, sr.md));
            shi = max(shi, mass_bucket((uint64_t)ceil(sr.u * (double)(incl_mass - sr.md)), sr.bd, sr.md));
        }
        if (slo <= shi) {  // only a range that fits
            const uint64_t n_in = cum_cnt(shi) - (slo ? cum_cnt(slo - 1) : 0ull);
            if (n_in > (uint64_t)NSPEC) {
                slo = 1u;
                shi = 0u;
            }
        }
    }
    const bool spec_on = slo <= shi;
    // the bucket (without `excl`) into the list: from the buckets gathered ahead, or a pass
    if (tid == 0) {
        sm.misc[MISC_N] = 0;
        if (spec_on) sm.spec_n = 0;
    }
    __syncthreads();
    if (cached) {
        const int ns = (int)sm.spec_n;
        for (int j = tid; j < ns; j += BLOCK) {
            const uint64_t k = sm.spec[j];
            if (vbucket(key_s(k), M) != hit || k == excl) continue;
            const uint32_t slot = lds_add(&sm.misc[MISC_N], 1u);
            if (slot < NMAX) sm.u.cb.keys[slot] = k;
        }
    } else {
        row_pass<BF16, VEC>(a, sm, C, P, [&](uint32_t id, float s) __attribute__((always_inline)) {
            if (!(s > -__builtin_inff())) return;
            const uint32_t b = vbucket(s, M);
            const bool in_spec = spec_on && b - slo <= shi - slo;
            if (b != hit && !in_spec) return;
            const uint64_t k = key64(s, id);
            if (b == hit && k != excl) {
                const uint32_t slot = lds_add(&sm.misc[MISC_N], 1u);
                if (slot < NMAX) sm.u.cb.keys[slot] = k;
            }
            if (in_spec) {
                const uint32_t slot = lds_add(&sm.spec_n, 1u);
                if (slot < NSPEC) sm.spec[slot] = k;
            }
        });
    }
    __syncthreads();
    if (spec_on && tid == 0) {  // complete, or unusable
        const bool fits = sm.spec_n <= (uint32_t)NSPEC;
        sm.spec_lo = fits ? slo : 1u;
        sm.spec_hi = fits ? shi : 0u;
    }
    const int N = (int)min(sm.misc[MISC_N], (uint32_t)NMAX);
    if (N <= BLOCK && N > WAVE) sort_list_regs(sm, N);
    else sort_list(sm, N);
    uint64_t loc[PT];
    uint64_t run = 0;
#pragma unroll
    for (int i = 0; i < PT; i++) {
        const int j = tid * PT + i;
        run += j < N ? efix_of(key_s(sm.u.cb.keys[j]), M, scale) : 0ull;
        loc[i] = run;
    }
    uint64_t tot;
    const uint64_t pre = block_excl_scan<uint64_t>(run, sm.r64, tot);
    uint32_t best = 0xFFFFFFFFu;
#pragma unroll
    for (int i = 0; i < PT; i++) {
        const int j = tid * PT + i;
        if (best != 0xFFFFFFFFu || j >= N) continue;
        const bool ok = kind == 0 ? (before_cnt + (uint64_t)j >= target) : (before_mass + pre + loc[i] >= target);
        if (ok) best = (uint32_t)j;
    }
    best = block_min_u(best, sm.ru);
    if (best == 0xFFFFFFFFu) best = N > 0 ? (uint32_t)N - 1 : 0u;
    if ((uint32_t)tid == best / PT) {
        const int i = (int)(best % PT);
        uint64_t li = 0;
#pragma unroll
        for (int ii = 0; ii < PT; ii++)
            if (ii == i) li = loc[ii];
        sm.r64[0] = sm.u.cb.keys[best];
        sm.r64[1] = before_mass + pre + li;
    }
    __syncthreads();
    Sel r;
    r.key = sm.r64[0];
    r.cum_mass = sm.r64[1];
    r.pos = before_cnt + best;
    __syncthreads();
    return r;
}

// Rows the candidate lists do not cover, in sorted order: top-k / top-p / min-p cuts and
// the draw (sample.rs:392-426, 312-323) by radix queries over the row. The queries run
// from one call site (a small state machine), which keeps the inlined code compact.
template <bool BF16, int VEC>
__device__ __forceinline__ void combine_radix(const KArgs& a, Smem& sm, const RowCtx& C, const PenSrc& P, bool hashed,
                                              float M, float S, ArgMax rawmax) {
    const int tid = threadIdx.x;
    const double scale = ldexp(1.0, a.fix_bits);
    const uint64_t V = (uint64_t)a.V;

    uint64_t n_finite;
    BFI_TRACE(a, 0, 4);
    if (tid == 0) {
        sm.spec_lo = 1u;
        sm.spec_hi = 0u;
        sm.spec_n = 0u;
    }
    // the draft's value, for the judge and the bound of its mass in the residual's buckets
    const float sd = C.judged ? element_s(a, sm, C, C.draft, BF16, hashed) : -__builtin_inff();
    const uint64_t S_fix = vsel_l1<BF16, VEC>(a, sm, C, P, M, scale, &n_finite);
    BFI_TRACE(a, 0, 5);
    int nq = 0;
    const uint64_t Lk = C.kmode ? (uint64_t)C.k : V;
    uint64_t Lp = ~0ull, Lm = ~0ull, L = 0, T = 0, kept_mass = 0, kd = ~0ull, md = 0;
    Sel selp{0, 0, 0}, last{0, 0, 0};
    if (C.pmode) {
        const double tp = ceil((double)C.top_p * (double)S_fix);
        T = tp <= 0.0 ? 0ull : (uint64_t)tp;
    }
    enum { Q_K, Q_P, Q_LAST, Q_DRAW, Q_RESID, ST_MINP, ST_LIST };
    int st = C.pmode ? (C.kmode ? Q_K : Q_P) : ST_MINP;
    for (;;) {
        if (st == ST_MINP) {
            if (C.mmode) {  // sample.rs:411-414: count p >= min_p * max_p
                const float thresh = C.min_p * (1.0f / S);
                uint32_t c = 0;
                row_pass<BF16, VEC>(a, sm, C, P, [&](uint32_t, float s) { c += (expf(s - M) / S >= thresh) ? 1u : 0u; });
                Lm = block_sum_u(c, sm.ru);
                if (Lm == 0) {  // sample.rs:415-422
                    finish_token(a, sm, C, rawmax.v > -__builtin_inff() ? rawmax.i : 0u);
                    return;
                }
            }
            L = Lk < Lp ? Lk : Lp;
            L = L < Lm ? L : Lm;
            if (C.pmode && L == Lp) {
                last = selp;
                st = ST_LIST;
            } else {
                st = Q_LAST;
            }
            continue;
        }
        if (st == ST_LIST) {
            kept_mass = last.cum_mass;
            if (a.t_kind && tid == 0) {
                a.t_kind[C.row] = BFI_SMP_TARGET_WEIGHTS;
                a.t_kept[C.row] = (int32_t)L;
                a.t_listed[C.row] = 0;
            }
            // introspection listing: gather keys >= last.key when they fit
            if (a.t_kind && a.t_cap > 0 && L <= (uint64_t)NMAX) {
                if (tid == 0) sm.misc[MISC_N] = 0;
                __syncthreads();
                row_pass<BF16, VEC>(a, sm, C, P, [&](uint32_t id, float s) {
                    const uint64_t k = key64(s, id);
                    if (k >= last.key) {
                        const uint32_t slot = lds_add(&sm.misc[MISC_N], 1u);
                        if (slot < NMAX) sm.u.cb.keys[slot] = k;
                    }
                });
                __syncthreads();
                const int N = (int)min(sm.misc[MISC_N], (uint32_t)NMAX);
                int n2 = 64;
                while (n2 < N) n2 <<= 1;
                for (int j = N + tid; j < n2; j += BLOCK) sm.u.cb.keys[j] = 0ull;
                __syncthreads();
                bitonic_sort_desc(sm.u.cb.keys, n2);
                uint32_t c = 0;
                for (int j = tid * PT; j < tid * PT + PT; j++)
                    if (j < N) c += (expf(key_s(sm.u.cb.keys[j]) - M) / S) > 0.0f;
                uint32_t tc;
                uint32_t o = block_excl_scan<uint32_t>(c, sm.ru, tc);
                for (int j = tid * PT; j < tid * PT + PT; j++) {
                    if (j < N) {
                        const float pj = expf(key_s(sm.u.cb.keys[j]) - M) / S;
                        if (pj > 0.0f) {
                            if ((int64_t)o < a.t_cap) {
                                a.t_ids[(int64_t)C.row * a.t_cap + o] = key_idx(sm.u.cb.keys[j]);
                                a.t_probs[(int64_t)C.row * a.t_cap + o] = pj;
                            }
                            o++;
                        }
                    }
                }
                if (tid == 0) a.t_listed[C.row] = (int32_t)(tc < a.t_cap ? tc : a.t_cap);
                __syncthreads();
            }
            if (!C.judged) {
                st = Q_DRAW;
                continue;
            }
            // judge (spec.rs:83-95)
            const bool kept_d = C.draft < V && key64(sd, C.draft) >= last.key;
            kd = kept_d ? key64(sd, C.draft) : ~0ull;
            md = kept_d ? efix_of(sd, M, scale) : 0ull;
            if (kept_mass > 0 && (double)C.u < (double)md / (double)kept_mass) {
                emit(a, sm, C, C.draft, 1u);
                return;
            }
            if (kept_mass - md == 0) {  // residual empty or all <= 0
                emit(a, sm, C, C.draft, 1u);
                return;
            }
            st = Q_RESID;
            continue;
        }
        // one radix query
        int kind = 1;
        uint64_t target = 0, ex = ~0ull, exm = 0;
        if (st == Q_K) {
            kind = 0;
            target = Lk - 1;
        } else if (st == Q_P) {
            target = T;
        } else if (st == Q_LAST) {
            kind = 0;
            target = L - 1;
        } else if (st == Q_DRAW) {
            target = (uint64_t)ceil((double)C.u * (double)kept_mass);
        } else {
            target = (uint64_t)ceil((double)C.u2 * (double)(kept_mass - md));
            ex = kd;
            exm = md;
        }
        SpecReq sr{0, 0.0, 0, 0};
        if (st == Q_P) {
            if (!C.judged) sr = SpecReq{1, (double)C.u, 0, 0};
            else if (sd > -__builtin_inff()) sr = SpecReq{2, (double)C.u2, efix_of(sd, M, scale), vbucket(sd, M)};
            else sr = SpecReq{2, (double)C.u2, 0, 0xFFFFFFFFu};
        }
        const Sel r = vsel_query<BF16, VEC>(a, sm, C, P, M, scale, kind, target, ex, exm, sr);
        if (nq < 3) BFI_TRACE(a, 0, 12 + nq);
        nq++;
        if (st == Q_K) {  // top-p runs over the top-k list: cut inside it, or keep all k
            if (r.cum_mass < T) {
                Lp = Lk;
                selp = r;
                st = ST_MINP;
            } else {
                st = Q_P;
            }
        } else if (st == Q_P) {
            selp = r;
            Lp = r.pos + 1;
            st = ST_MINP;
        } else if (st == Q_LAST) {
            last = r;
            st = ST_LIST;
        } else {
            const uint32_t tok = key_idx(r.key);
            if (st == Q_DRAW && a.t_kind && tid == 0 && a.out_tok) a.out_tok[C.row] = tok;
            emit(a, sm, C, tok, st == Q_DRAW ? 1u : 0u);
            return;
        }
    }
}

// ---- select kernel: one workgroup per row ----------------------------------------------
//
// The streaming pass saw every element at its un-penalized value. The select kernel puts
// the row's history ids (at most HMAX distinct) in an LDS hash, computes their penalized
// values, and corrects the chunk statistics: a history id's term exp(s - m_c) is taken out
// of its chunk's sum (recomputed exactly as the streaming pass did, accumulated in fixed
// point so the result does not depend on the order), and its penalized term is added. A
// chunk whose maximum is a history id ("dirty") is re-read for the maximum and sum of its
// other elements, so that no subtraction loses precision. Rows with a larger history take
// whole-row passes with the history tables in global memory.


// Every logit is -inf: the reference's weights are NaN and its outcome is deterministic
// (the min-p fallback argmax, or the last kept id of the draw).
__device__ __forceinline__ void finish_all_masked(const KArgs& a, Smem& sm, const RowCtx& C, ArgMax rawmax) {
    if (C.mmode) {
        finish_token(a, sm, C, rawmax.v > -__builtin_inff() ? rawmax.i : 0u);
        return;
    }
    const uint32_t L = C.kmode ? (uint32_t)C.k : (uint32_t)a.V;
    if (a.t_kind && threadIdx.x == 0) {
        a.t_kind[C.row] = BFI_SMP_TARGET_WEIGHTS;
        a.t_kept[C.row] = (int32_t)L;
        a.t_listed[C.row] = 0;
    }
    if (C.judged) {
        // residual = kept minus d; a draw over NaN weights returns its last id
        const uint32_t lastid = (C.draft == L - 1) ? L - 2 : L - 1;
        const bool empty = (L == 1 && C.draft == 0);
        emit(a, sm, C, empty ? C.draft : lastid, empty ? 1u : 0u);
        return;
    }
    if (a.t_kind && threadIdx.x == 0 && a.out_tok) a.out_tok[C.row] = L - 1;
    emit(a, sm, C, L - 1, 1u);
}

// Rows whose history does not fit the hash: M (greedy: the argmax) and S by whole-row
// passes with the history tables in global memory. Returns false when the row is done.
template <bool BF16, int VEC>
__device__ __forceinline__ bool stats_full(const KArgs& a, Smem& sm, const RowCtx& C, const PenSrc& P, ArgMax rawmax,
                                           float& M, float& S) {
    ArgMax am{-__builtin_inff(), 0xFFFFFFFFu};
    row_pass<BF16, VEC>(a, sm, C, P, [&](uint32_t id, float s) { am = argmax_merge(am, ArgMax{s, id}); });
    am = block_argmax(am, sm.rf, sm.ru);
    if (C.greedy) {  // sample.rs:369-371, 429-439
        finish_token(a, sm, C, am.v > -__builtin_inff() ? am.i : 0u);
        return false;
    }
    M = am.v;
    if (!(M > -__builtin_inff())) {
        finish_all_masked(a, sm, C, rawmax);
        return false;
    }
    double ls = 0.0;
    row_pass<BF16, VEC>(a, sm, C, P, [&](uint32_t, float s) { ls += (double)expf(s - M); });
    S = (float)block_sum_d(ls, sm.rd);
    return true;
}

// Row handled by this workgroup: rows grouped per XCD (dispatch is round-robin over the 8
// XCDs).
__device__ __forceinline__ int select_row_id() {
    const uint32_t G = gridDim.x, bid = blockIdx.x;
    const uint32_t q8 = G / 8, r8 = G % 8, xcd = bid % 8, slot = bid / 8;
    return (int)(xcd < r8 ? xcd * (q8 + 1) + slot : r8 * (q8 + 1) + (xcd - r8) * q8 + slot);
}

template <bool BF16>
__device__ __forceinline__ void select_row(const KArgs& a, Smem& sm) {
    constexpr int VEC = BF16 ? 2 : 4;  // row passes walk 8192-element tiles
    const int tid = threadIdx.x;
    const int row = select_row_id();
    const int64_t tb = 0;
    BFI_TRACE(a, tb, 0);
    if (row >= a.n_rows) return;
    RowCtx C = make_ctx(a, row);
    if (!C.active) return;
    BFI_TRACE(a, tb, 8);
    const bool track_raw = !C.greedy && C.min_p > 1.0f;
    const bool cand_row = !C.greedy && (C.kmode || C.pmode || C.mmode);  // may have candidate lists

    const int nc = a.n_chunks;
    ChunkPart mine;
    if (tid < nc) {
        mine = a.parts[(int64_t)row * nc + tid];
    } else {
        mine.m = -__builtin_inff();
        mine.sum = 0.0;
        mine.arg = 0xFFFFFFFFu;
        mine.ncand = 0;
        mine.theta = -__builtin_inff();
        mine.raw_m = -__builtin_inff();
        mine.raw_arg = 0xFFFFFFFFu;
    }
    // ---- A: history hash; chunk results into LDS and the row aggregates (one pair of
    // barriers; the history loads are issued while the chunk results are in flight)
    if (tid < nc) {
        sm.cflag[tid] = 0u;
        sm.craw[tid] = 0ull;
        sm.cpen[tid] = 0ull;
    }
    if (tid == 0) {
        sm.ag.gkey = 0ull;
        sm.ag.rawkey = 0ull;
        sm.ag.sfix = 0ull;
        sm.ag.mmax = 0u;
        sm.ag.hmax = 0u;
        sm.ag.thr = 0u;
        sm.ag.flags = 0u;
        sm.ag.nd = 0u;
        sm.ag.kth = 0u;
    }
    HistOwn ho;
    const bool hashed = hist_build<BF16>(a, sm, C, ho, [&]() {
        BFI_TRACE(a, tb, 9);
        if (tid < nc) {
            sm.cm[tid] = mine.m;
            sm.cxm[tid] = mine.raw_m;
            sm.carg[tid] = mine.arg;
            sm.csum[tid] = mine.sum;
        }
        if (wave_id() * WAVE < nc) {  // waves holding chunks
            const bool in = tid < nc;
            wave_lds_max(&sm.ag.mmax, in && mine.m > -__builtin_inff() ? ord32(mine.m) : 0u);
            wave_lds_max(&sm.ag.thr, in ? ord32(mine.theta) : 0u);
            wave_lds_add(&sm.ag.flags, in && (mine.ncand == NCAND_UNBOUNDED || mine.ncand == NCAND_OVERFLOW));
            if (C.greedy) wave_lds_max64(&sm.ag.gkey, in ? argmax_key(mine.m, mine.arg) : 0ull);
            if (track_raw) wave_lds_max64(&sm.ag.rawkey, in ? argmax_key(mine.raw_m, mine.raw_arg) : 0ull);
        }
        // prefix over every chunk's candidate list (the first pass filters them later)
        if (cand_row) chunk_prefix(sm, nc, tid < nc && mine.ncand <= (uint32_t)CAND_CAP ? mine.ncand : 0u);
        if (tid == 0) sm.misc[MISC_N] = 0;
        BFI_TRACE(a, tb, 10);
    });
    BFI_TRACE(a, tb, 1);
    // bounded rows: the first candidate loads go out now and land during the history work
    const bool unfiltered = !C.kmode && !C.pmode && !C.mmode;
    const bool bounded = cand_row && hashed && C.stream_ok && sm.ag.flags == 0u;
    CandBatch first;
    if (bounded) first = load_cands(a, sm, row, nc, 0);
    BFI_TRACE(a, tb, 2);
    // masked, un-penalized argmax (min-p fallback, sample.rs:415-422)
    const ArgMax rawmax = track_raw ? argmax_of_key(sm.ag.rawkey) : ArgMax{-__builtin_inff(), 0xFFFFFFFFu};
    const PenSrc H{true, nullptr, nullptr, nullptr};
    // Rows whose penalties the stream pass applied have an empty hash; the passes that
    // re-read logits (repairs, index-order draws) build it first. Its values do not change
    // M or S, which are final by then.
    auto need_hash = [&]() __attribute__((always_inline)) {
        if (C.prepen && !C.pen_hash) {
            C.pen_hash = true;
            HistOwn h2;
            hist_build<BF16>(a, sm, C, h2, []() {});
            hist_values(a, sm, C, h2);
        }
    };
    const int nw = a.bm_words;
    const uint32_t* gbm = a.row_pen + (int64_t)row * (2 * nw + GDCAP);
    const PenSrc GT{false, gbm, gbm + nw, gbm + 2 * nw};
    float M, S;
    double wc = 0.0;  // this thread's chunk: sum of exp(s - M) over it (hashed rows)
    enum { R_INDEX, R_RADIX };
    int route;
    if (!hashed || (!C.greedy && !C.stream_ok)) {
        // an oversized history, or a temperature whose streaming values are not usable
        build_row_pen(a, sm, C);
        if (!stats_full<BF16, VEC>(a, sm, C, GT, rawmax, M, S)) return;
        if (a.t_stats && tid == 0) a.t_stats[row * 4 + 3] = 4.0f;
        route = (C.kmode || C.pmode) ? R_RADIX : R_INDEX;
    } else {
        // ---- B: history values (sample.rs:331-375) and the streaming terms they replace
        uint32_t dirty = 0;
        if (C.pen_hash) {
            hist_values(a, sm, C, ho);
            if (sm.ag.nd) {
                // rare: a chunk whose maximum is a history id; re-read it for the max and
                // sum of its other elements, then refresh the aggregates
                dirty = tid < nc ? sm.cflag[tid] : 0u;
                for (int c = 0; c < nc; c++) {
                    if (!sm.cflag[c]) continue;
                    ArgMax am{-__builtin_inff(), 0xFFFFFFFFu};
                    span_pass<BF16, VEC, true>(a, sm, C, H, chunk_lo(a, c), chunk_hi(a, c),
                                               [&](uint32_t id, float v) { am = argmax_merge(am, ArgMax{v, id}); });
                    am = block_argmax(am, sm.rf, sm.ru);
                    double ls = 0.0;
                    if (!C.greedy && am.v > -__builtin_inff())
                        span_pass<BF16, VEC, true>(a, sm, C, H, chunk_lo(a, c), chunk_hi(a, c),
                                                   [&](uint32_t, float v) { ls += (double)__expf(v - am.v); });
                    ls = block_sum_d(ls, sm.rd);
                    if (tid == 0) {
                        sm.cm[c] = am.v;
                        sm.carg[c] = am.i;
                        sm.csum[c] = ls;
                        sm.ag.mmax = 0u;
                        if (C.greedy) sm.ag.gkey = 0ull;
                    }
                }
                __syncthreads();
                if (tid < nc && dirty) {
                    mine.m = sm.cm[tid];
                    mine.arg = sm.carg[tid];
                    mine.sum = sm.csum[tid];
                }
                const bool in = tid < nc;
                wave_lds_max(&sm.ag.mmax, in && mine.m > -__builtin_inff() ? ord32(mine.m) : 0u);
                if (C.greedy) {
                    uint64_t gk = in ? argmax_key(mine.m, mine.arg) : 0ull;
                    for (int j = tid; j < (int)sm.misc[MISC_HN]; j += BLOCK) {
                        const int k = sm.hlist[j];
                        const uint64_t key = argmax_key(sm.hpen[k], sm.hkey[k]);
                        gk = key > gk ? key : gk;
                    }
                    wave_lds_max64(&sm.ag.gkey, gk);
                }
                __syncthreads();
            }
        }
        if (C.greedy) {  // sample.rs:369-371, 429-439
            const ArgMax am = argmax_of_key(sm.ag.gkey);
            finish_token(a, sm, C, am.v > -__builtin_inff() ? am.i : 0u);
            return;
        }
        M = fmaxf(unord_or_ninf(sm.ag.mmax), unord_or_ninf(sm.ag.hmax));
        if (!(M > -__builtin_inff())) {
            finish_all_masked(a, sm, C, rawmax);
            return;
        }
        // ---- C: S (penalized terms of the history ids + the chunks' corrected sums, in
        // 2^-44 fixed point) and, for bounded rows, the candidate prefix of the first pass
        constexpr double FIX44 = 17592186044416.0;
        uint64_t sf = 0;  // this thread's share of S, fixed point
        if (C.pen_hash) {
            for (int j = tid; j < (int)sm.misc[MISC_HN]; j += BLOCK) {
                const int k = sm.hlist[j];
                const uint32_t c = sm.hkey[k] / (uint32_t)a.chunk;
                const double tp = (double)expf(sm.hpen[k] - M);
                lds_add64(&sm.cpen[c], (uint64_t)(tp * FIX52));
                sf += (uint64_t)(tp * FIX44);
            }
        }
        if (tid < nc && mine.m > -__builtin_inff()) {
            const double rc = mine.sum - (C.pen_hash && !dirty ? (double)sm.craw[tid] / FIX52 : 0.0);
            wc = rc * (double)expf(mine.m - M);
            sf += (uint64_t)(wc * FIX44);
        }
        wave_lds_add64(&sm.ag.sfix, sf);
        // Top-k rows with k <= chunks: the chunk maxima are k distinct elements at or above the
        // k-th largest of them (kth), so the row's k-th largest value is too. The reference
        // orders by p = expf(s - M) / S with ties in index order (sample.rs:392-395), so an
        // element just below kth can tie in p with one above it: the bound is lowered by the
        // streaming pass's margin (1e-4 + 1e-5 |s|, far above an ulp of s - M while
        // s - M > -64), and not used at all further below M, where p nears underflow and
        // ties at zero. It raises the list bound when the chunk bounds are loose (short
        // chunks: one row over many chunks).
        if (C.kmode && (uint32_t)C.k <= (uint32_t)nc) {
            if (tid < nc && mine.m > -__builtin_inff()) {
                uint32_t rank = 0;
                for (int c = 0; c < nc; c++) {
                    const float o = sm.cm[c];
                    rank += (o > mine.m || (o == mine.m && c < tid)) ? 1u : 0u;
                }
                if (rank == (uint32_t)C.k - 1u) sm.ag.kth = ord32(mine.m);
            }
            __syncthreads();
        }
        const float kth = unord_or_ninf(sm.ag.kth);
        const float th_k = kth > M - 64.0f ? kth - (1e-4f + 1e-5f * fabsf(kth)) : -__builtin_inff();
        const float th_raw = fmaxf(unord_or_ninf(sm.ag.thr), th_k);
        if (bounded) {  // the first pass's list: complete above max(th_raw, min-p bound)
            const float th = fmaxf(th_raw, minp_bound(C, M));
            const bool sorted = C.kmode || C.pmode;
            BFI_TRACE(a, tb, 11);
            append_cands(sm, C, first, th, sorted, HistExcl{sm, C});
            BFI_TRACE(a, tb, 12);
            for (uint32_t b0 = GU * BLOCK; b0 < sm.cpre[nc]; b0 += GU * BLOCK)  // uniform trip count
                append_cands(sm, C, load_cands(a, sm, row, nc, b0), th, sorted, HistExcl{sm, C});
            append_hist(sm, C, th, sorted);
        }
        __syncthreads();
        S = (float)((double)sm.ag.sfix / FIX44);
        if (tid < nc && C.pen_hash) wc += (double)sm.cpen[tid] / FIX52;
        BFI_TRACE(a, tb, 3);
        if (a.t_stats && tid == 0) {
            a.t_stats[row * 4 + 0] = M;
            a.t_stats[row * 4 + 1] = S;
            a.t_stats[row * 4 + 3] = unfiltered ? 2.0f : (bounded ? 1.0f : 3.0f);
        }
        if (bounded) {
            if (combine_bounded<BF16, VEC>(a, sm, C, mine, M, S, rawmax, th_raw, true, tb, need_hash) == CB_DONE)
                return;
            if (a.t_stats && tid == 0) a.t_stats[row * 4 + 3] = 3.0f;
        }
        route = (C.kmode || C.pmode) ? R_RADIX : R_INDEX;
    }
    if (a.t_stats && tid == 0) {
        a.t_stats[row * 4 + 0] = M;
        a.t_stats[row * 4 + 1] = S;
    }
    const bool full = !hashed || !C.stream_ok;  // the global history tables are built
    if (!full) need_hash();
    if (route == R_RADIX) {
        if (!full) build_row_pen(a, sm, C);
        combine_radix<BF16, VEC>(a, sm, C, GT, hashed, M, S, rawmax);
    } else {
        const bool known = !full && !C.kmode && !C.pmode && !C.mmode;
        combine_index_order_passes<BF16, VEC>(a, sm, C, hashed ? H : GT, hashed, M, S, rawmax, known,
                                              known ? wc / (double)S : 0.0);
    }
}

// One workgroup per row and usually one per CU: registers up to 256 per lane (two waves
// per SIMD) rather than spills for a third. The fast finish goes first; a row it leaves
// starts over on the general path.
template <bool BF16>
__global__ __launch_bounds__(BLOCK) __attribute__((amdgpu_waves_per_eu(1, 2))) void k_select(KArgs a) {
    __shared__ Smem sm;
    if (a.trace && threadIdx.x == 0)
        for (int i = 0; i < 16; i++) sm.tr[i] = 0;
    BFI_TRACE(a, 0, 0);
    const int row = select_row_id();
    if (row >= a.n_rows) return;
    if (!select_fast<true>(a, sm, row, [&]() { return make_ctx(a, row); })) {
        __syncthreads();
        select_row<BF16>(a, sm);
    }
    if (a.trace && threadIdx.x == 0 && row < a.n_rows) {
        sm.tr[7] = wall_clock64();
        uint64_t* t = a.trace + (int64_t)a.n_rows * a.n_chunks * 8 + (int64_t)row * 16;
        for (int i = 0; i < 16; i++) t[i] = sm.tr[i];
    }
}

// ---- launch ----------------------------------------------------------------------------

hipError_t launch_select(const KArgs& a, int bf16, hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
    const dim3 grid((unsigned)a.n_rows), block(BLOCK);
    if (bf16)
        hipExtLaunchKernelGGL((k_select<true>), grid, block, 0, stream, start, stop, 0, a);
    else
        hipExtLaunchKernelGGL((k_select<false>), grid, block, 0, stream, start, stop, 0, a);
    return hipGetLastError();
}

}  // namespace bfi
