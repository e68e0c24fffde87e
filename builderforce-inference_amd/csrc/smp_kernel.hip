// smp_kernel.hip — the gfx950 token-sampling kernel.
//
// One launch samples every row of a batch (generate_batch's per-step call, engine/mod.rs:
// 316-322) or judges every draft of a spec-verify step (engine/spec.rs:137-162).
//
// Stream phase: workgroup (row, chunk) holds `chunk` logits of one row in VGPRs, read once
// from HBM with 16-byte loads. It applies the allow-mask, repeat/presence/frequency
// penalties and the temperature division (sample.rs:331-375) in registers. It then reduces
// max and sum(exp(s - max)) and writes the elements that can still belong to the kept set:
// those above the chunk's top-k or min-p bound. The last workgroup of a row to finish (an
// atomic ticket, no spinning) runs the combine phase for the row:
//   - greedy: argmax (sample.rs:369-371, 429-439);
//   - bounded candidates (top-k <= 512 or min-p > 0): gather, one bitonic sort in LDS, then
//     top-k / top-p / min-p and the draw by f64 scans (sample.rs:392-426, 312-323);
//   - unfiltered rows (no top-k/top-p/min-p): the draw in index order from per-chunk masses
//     plus one chunk re-read;
//   - unbounded rows (top-p without top-k/min-p, or candidate overflow): radix select over
//     the row (10-bit digits of a 64-bit (value, index) key, with counts and fixed-point
//     masses), re-reading the row.
// Spec verify applies judge() (spec.rs:79-97) to each row's target; the last row of a
// sequence to finish computes the accepted prefix.
#include "smp_device.h"

namespace bfi {

// ---- shared memory ---------------------------------------------------------------------

struct __align__(16) Smem {
    union {
        struct {
            uint32_t bm[CHUNK_MAX / 32];   // history bitmap of the chunk
            uint32_t pre[CHUNK_MAX / 32];  // popcount prefix of bm
            uint32_t cnt[DCAP];            // occurrences per distinct history id
        } st;
        struct {
            uint64_t keys[NMAX];
            float p[NMAX];
        } cb;
        struct {
            uint64_t mass[NBUCKET];
            uint32_t cnt[NBUCKET];
        } hs;
    } u;
    uint32_t cpre[BLOCK + 1];  // per-chunk candidate prefix (combine)
    float rf[NWAVE];
    float rf2[NWAVE];
    uint32_t ru[NWAVE];
    uint32_t ru2[NWAVE];
    double rd[NWAVE];
    uint64_t r64[NWAVE];
    uint64_t r64b[NWAVE];
    uint32_t misc[8];
};

// The stream kernel needs only the history tables and the reduction scratch.
struct __align__(16) StreamSmem {
    union {
        struct {
            uint32_t bm[CHUNK_MAX / 32];
            uint32_t pre[CHUNK_MAX / 32];
            uint32_t cnt[DCAP];
        } st;
    } u;
    float rf[NWAVE];
    uint32_t ru[NWAVE];
    double rd[NWAVE];
    uint32_t misc[8];
};

enum { MISC_LAST = 0, MISC_N = 1, MISC_NDIST = 2, MISC_OVF = 3 };

// ---- per-row context -------------------------------------------------------------------

struct RowCtx {
    int row, seq, ri, dl;
    bool active, verify, judged;
    uint32_t draft;
    float u, u2;
    float T, rT, top_p, min_p;
    bool fast_div;  // T in [2^-20, 2^20]: FMA-corrected reciprocal division is exact
    int32_t k;
    bool greedy, kmode, pmode, mmode;
    Pen pen;
    bool pen_on;
    HistView h;
    const uint32_t* mrow;
    const char* lrow;
};

__device__ __forceinline__ RowCtx make_ctx(const KArgs& a, int row) {
    RowCtx C;
    C.row = row;
    C.verify = a.rows_per_seq > 0;
    if (C.verify) {
        int rps = a.rows_per_seq;
        C.seq = row / rps;
        C.ri = row % rps;
        int dl = a.draft_len[C.seq];
        dl = dl < 0 ? 0 : (dl > rps - 1 ? rps - 1 : dl);
        C.dl = dl;
        C.active = C.ri <= dl;
        C.judged = C.ri < dl;
        const int64_t dbase = (int64_t)C.seq * (rps - 1);
        C.draft = C.judged ? a.drafts[dbase + C.ri] : 0u;
        if (C.judged) {
            C.u = a.u_pairs[(dbase + C.ri) * 2];
            C.u2 = a.u_pairs[(dbase + C.ri) * 2 + 1];
        } else {
            C.u = a.u_bonus[C.seq];
            C.u2 = 0.0f;
        }
        C.h.extra = a.drafts + dbase;
        C.h.nextra = C.ri;
    } else {
        C.seq = row;
        C.ri = 0;
        C.dl = 0;
        C.active = true;
        C.judged = false;
        C.draft = 0;
        C.u = a.u ? a.u[row] : 0.0f;
        C.u2 = 0.0f;
        C.h.extra = nullptr;
        C.h.nextra = 0;
    }
    const bfi_smp_row_params P = a.params[C.seq];
    if (a.hist_off) {
        int64_t o0 = a.hist_off[C.seq], o1 = a.hist_off[C.seq + 1];
        C.h.base = a.hist + o0;
        C.h.nbase = o1 > o0 ? o1 - o0 : 0;
    } else {
        C.h.base = nullptr;
        C.h.nbase = 0;
    }
    const int64_t H = C.h.size();
    C.T = P.temperature;
    C.rT = 1.0f / P.temperature;  // IEEE, once per row
    C.fast_div = P.temperature >= 0x1p-20f && P.temperature <= 0x1p20f;
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
    C.pen.rep_on = fabsf(P.repeat_penalty - 1.0f) > F32_EPS && H > 0;  // sample.rs:346
    C.pen.pres_on = P.presence_penalty != 0.0f && H > 0;               // sample.rs:360
    C.pen.freq_on = P.frequency_penalty != 0.0f && H > 0;
    C.pen_on = C.pen.rep_on || C.pen.pres_on || C.pen.freq_on;
    C.mrow = a.mask ? a.mask + (int64_t)row * a.mask_stride : nullptr;
    const int esz = 4;  // overridden by the loader for bf16
    (void)esz;
    C.lrow = (const char*)a.logits;
    return C;
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

// ---- history structures ----------------------------------------------------------------

// The first 2*BLOCK history ids of a row, loaded into registers before the logits so that
// their latency overlaps the HBM stream (UINT32_MAX past the end).
struct HistPre {
    uint32_t v0, v1;
};
__device__ __forceinline__ HistPre hist_prefetch(const RowCtx& C) {
    const int64_t H = C.h.size();
    const int tid = threadIdx.x;
    HistPre p;
    p.v0 = (C.pen_on && tid < H) ? C.h.at(tid) : 0xFFFFFFFFu;
    p.v1 = (C.pen_on && tid + BLOCK < H) ? C.h.at(tid + BLOCK) : 0xFFFFFFFFu;
    return p;
}

// Chunk-local history bitmap + dense occurrence counts in LDS (ids in [c0, c1)).
template <typename SM>
__device__ __forceinline__ void build_chunk_pen(SM& sm, const RowCtx& C, uint32_t c0, uint32_t c1,
                                                HistPre hp) {
    const int tid = threadIdx.x;
    const uint32_t nw = (c1 - c0 + 31) / 32;
    for (uint32_t w = tid; w < CHUNK_MAX / 32; w += BLOCK) sm.u.st.bm[w] = 0;
    if (C.pen.freq_on)
        for (uint32_t w = tid; w < DCAP; w += BLOCK) sm.u.st.cnt[w] = 0;
    __syncthreads();
    const int64_t H = C.h.size();
    if (hp.v0 >= c0 && hp.v0 < c1) lds_or(&sm.u.st.bm[(hp.v0 - c0) >> 5], 1u << ((hp.v0 - c0) & 31));
    if (hp.v1 >= c0 && hp.v1 < c1) lds_or(&sm.u.st.bm[(hp.v1 - c0) >> 5], 1u << ((hp.v1 - c0) & 31));
    for (int64_t j = tid + 2 * BLOCK; j < H; j += BLOCK) {
        uint32_t id = C.h.at(j);
        if (id >= c0 && id < c1) lds_or(&sm.u.st.bm[(id - c0) >> 5], 1u << ((id - c0) & 31));
    }
    __syncthreads();
    if (C.pen.freq_on) {
        uint32_t c = (uint32_t)tid < nw ? __popc(sm.u.st.bm[tid]) : 0u;
        uint32_t tot;
        uint32_t pre = block_excl_scan<uint32_t>(c, sm.ru, tot);
        if ((uint32_t)tid < CHUNK_MAX / 32) sm.u.st.pre[tid] = pre;
        if (tid == 0) sm.misc[MISC_NDIST] = tot;
        __syncthreads();
        if (tot <= DCAP) {
            auto count = [&](uint32_t id) {
                if (id >= c0 && id < c1) {
                    uint32_t o = id - c0, w = o >> 5;
                    lds_add(&sm.u.st.cnt[dense_rank(sm.u.st.pre[w], sm.u.st.bm[w], o & 31)], 1u);
                }
            };
            count(hp.v0);
            count(hp.v1);
            for (int64_t j = tid + 2 * BLOCK; j < H; j += BLOCK) count(C.h.at(j));
        }
        __syncthreads();
    }
}

template <typename SM>
__device__ __forceinline__ uint32_t chunk_count(const SM& sm, const RowCtx& C, uint32_t c0,
                                                uint32_t id) {
    if (!C.pen.freq_on) return 0;
    if (sm.misc[MISC_NDIST] > DCAP) return C.h.count_scan(id);
    uint32_t o = id - c0, w = o >> 5;
    return sm.u.st.cnt[dense_rank(sm.u.st.pre[w], sm.u.st.bm[w], o & 31)];
}

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

// ---- the element transform (sample.rs:331-375) -----------------------------------------

// Where the penalty membership/counts of an element come from.
struct PenSrc {
    bool global;
    uint32_t c0;                // chunk base (LDS tables)
    const uint32_t* gbm;        // row tables (global)
    const uint32_t* gpre;
    const uint32_t* gcnt;
};

template <typename SM>
__device__ __forceinline__ uint32_t pen_bits(const SM& sm, const PenSrc& S, uint32_t id0, int epv) {
    const uint32_t em = (1u << epv) - 1u;
    if (!S.global) {
        uint32_t o = id0 - S.c0;
        return (sm.u.st.bm[o >> 5] >> (o & 31)) & em;
    }
    return (S.gbm[id0 >> 5] >> (id0 & 31)) & em;
}
template <typename SM>
__device__ __forceinline__ uint32_t pen_count(const SM& sm, const PenSrc& S, const RowCtx& C,
                                              uint32_t id) {
    if (!C.pen.freq_on) return 0;
    if (!S.global) return chunk_count(sm, C, S.c0, id);
    if (sm.misc[MISC_NDIST] > GDCAP) return C.h.count_scan(id);
    return S.gcnt[dense_rank(S.gpre[id >> 5], S.gbm[id >> 5], id & 31)];
}

// x / T rounded like IEEE division (sample.rs:373-375). With r = RN(1/T), q = RN(x*r) is
// within one ulp of x/T, e = x - q*T is exact under FMA, and RN(q + e*r) is the correctly
// rounded quotient while no step underflows or overflows (Markstein's correction). This was
// checked bit-exhaustively against IEEE division over all f32 x with |x| in [2^-100, 2^100]
// for temperatures across [2^-20, 2^20]. Zeros give +-0 and infinities/NaN pass through (e
// is NaN there, and q is already the quotient). `div_ok` says whether x is in the checked
// range; a wave with any other value takes IEEE division for its whole tile.
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

// In place: masked -> penalized -> (/T unless greedy). Tracks the masked, un-penalized
// argmax when RAW (min-p fallback, sample.rs:415-422).
template <bool BF16, int VEC, bool RAW = false, typename SM>
__device__ __forceinline__ ArgMax transform_tile(const SM& sm, const RowCtx& C, const PenSrc& S,
                                                 uint32_t c0, uint32_t c1,
                                                 float (&x)[VEC][Elem<BF16>::EPV]) {
    constexpr int EPV = Elem<BF16>::EPV;
    const int tid = threadIdx.x;
    const uint32_t em = (1u << EPV) - 1u;
    ArgMax raw{-__builtin_inff(), 0xFFFFFFFFu};
    bool bad = false;
#pragma unroll
    for (int q = 0; q < VEC; q++) {
        const uint32_t id0 = c0 + (uint32_t)(q * BLOCK + tid) * EPV;
        if (id0 >= c1) continue;  // all -inf already
        if (C.mrow) {             // sample.rs:331-337
            const uint32_t mb = (C.mrow[id0 >> 5] >> (id0 & 31)) & em;
#pragma unroll
            for (int e = 0; e < EPV; e++) x[q][e] = ((mb >> e) & 1u) ? x[q][e] : -__builtin_inff();
        }
        if (RAW) {
#pragma unroll
            for (int e = 0; e < EPV; e++)
                if (id0 + e < c1) raw = argmax_merge(raw, ArgMax{x[q][e], id0 + e});
        }
        const uint32_t pb = C.pen_on ? pen_bits(sm, S, id0, EPV) : 0u;
        if (pb) {  // rare: an id of the history in this vector
#pragma unroll
            for (int e = 0; e < EPV; e++)
                if ((pb >> e) & 1u) x[q][e] = penalize(x[q][e], pen_count(sm, S, C, id0 + e), C.pen);
        }
        if (!C.greedy) {
#pragma unroll
            for (int e = 0; e < EPV; e++) bad = bad || !div_ok(x[q][e]);
        }
    }
    if (!C.greedy) {  // sample.rs:373-375
        if (C.fast_div && __ballot(bad) == 0) {
#pragma unroll
            for (int q = 0; q < VEC; q++)
#pragma unroll
                for (int e = 0; e < EPV; e++) x[q][e] = div_T_fast(x[q][e], C);
        } else {
#pragma unroll
            for (int q = 0; q < VEC; q++)
#pragma unroll
                for (int e = 0; e < EPV; e++) x[q][e] = x[q][e] / C.T;
        }
    }
    return raw;
}

// ---- small helpers ---------------------------------------------------------------------

template <bool BF16, int VEC>
__device__ __forceinline__ uint32_t tile_count_ge(const float (&x)[VEC][Elem<BF16>::EPV], float th) {
    constexpr int EPV = Elem<BF16>::EPV;
    uint32_t c = 0;
#pragma unroll
    for (int q = 0; q < VEC; q++)
#pragma unroll
        for (int e = 0; e < EPV; e++) c += (x[q][e] >= th && x[q][e] > -__builtin_inff()) ? 1u : 0u;
    return c;
}

__device__ __forceinline__ uint64_t efix_of(float s, float M, double scale) {
    float e = expf(s - M);
    return (uint64_t)((double)e * scale);
}

// ---- result emission (sample / target / verify) ----------------------------------------

// Stores the row's outcome. For spec verify, `verdict` is 1 = Accept, 0 = Reject(token),
// and the last row of a sequence to finish resolves the accepted prefix (spec.rs:140-162).
__device__ __forceinline__ void emit(const KArgs& a, Smem& sm, const RowCtx& C, uint32_t token, uint32_t verdict) {
    const int tid = threadIdx.x;
    if (!C.verify) {
        if (tid == 0) {
            if (a.out_tok) a.out_tok[C.row] = token;
        }
        return;
    }
    if (tid == 0) {
        a.row_res[2 * C.row] = C.judged ? verdict : 2u;
        a.row_res[2 * C.row + 1] = token;
    }
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        uint32_t prev = glb_add(&a.seq_ctr[C.seq], 1u);
        sm.misc[MISC_LAST] = prev == (uint32_t)C.dl;
    }
    __syncthreads();
    if (!sm.misc[MISC_LAST]) return;
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

__device__ __forceinline__ void emit_target_token(const KArgs& a, const RowCtx& C, uint32_t tok) {
    if (threadIdx.x == 0 && a.t_kind) {
        a.t_kind[C.row] = BFI_SMP_TARGET_TOKEN;
        a.t_kept[C.row] = 0;
        a.t_listed[C.row] = 0;
        if (a.out_tok) a.out_tok[C.row] = tok;
    }
}

// Token target (greedy, min-p fallback): judge is exact equality (spec.rs:81-82).
__device__ __forceinline__ void finish_token(const KArgs& a, Smem& sm, const RowCtx& C, uint32_t tok) {
    emit_target_token(a, C, tok);
    if (C.judged)
        emit(a, sm, C, tok, tok == C.draft ? 1u : 0u);
    else
        emit(a, sm, C, tok, 1u);
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

__device__ __forceinline__ void bitonic_sort_desc(uint64_t* k, int n) {
    for (int size = 2; size <= n; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = threadIdx.x; i < n / 2; i += BLOCK) {
                int lo = 2 * i - (i & (stride - 1));
                int hi = lo + stride;
                bool desc = (lo & size) == 0;
                uint64_t x = k[lo], y = k[hi];
                if ((x < y) == desc) {
                    k[lo] = y;
                    k[hi] = x;
                }
            }
            __syncthreads();
        }
    }
}

// ---- combine: bounded candidates -------------------------------------------------------

// The bounded combine for N <= 64 candidates (in sm.u.cb.keys): wave 0 does all of it in
// registers with shuffles and ballots, no barrier; the others wait for the result.
__device__ __forceinline__ void combine_wave(const KArgs& a, Smem& sm, const RowCtx& C, int N, bool sorted, float M,
                                             float S, ArgMax rawmax) {
    enum { R_TOK = 0, R_VERDICT = 1, R_TOKEN_TARGET = 2 };
    if (wave_id() == 0) {
        const int lane = lane_id();
        const bool valid = lane < N;
        uint64_t key = valid ? sm.u.cb.keys[lane] : 0ull;
        key = wave_sort_desc(key);
        const float s = sorted ? key_s(key) : unord32((uint32_t)key);
        const uint32_t idx = sorted ? key_idx(key) : ~(uint32_t)(key >> 32);
        const float p = valid ? expf(s - M) / S : 0.0f;  // sample.rs:383, 388
        const int64_t Lk = C.kmode ? C.k : a.V;
        const int lim = (int)(Lk < N ? Lk : N);
        int64_t Lp = INT64_MAX, Lm = INT64_MAX;
        if (sorted && C.pmode) {  // sample.rs:397-409
            const double cum = wave_incl_scan_d((double)p);
            const uint64_t hit = __ballot(lane < lim && cum >= (double)C.top_p);
            Lp = hit ? (int64_t)__ffsll((unsigned long long)hit) : Lk;
        }
        float thresh = 0.0f;
        bool token_target = false;
        uint32_t tok = 0, verdict = 1;
        if (C.mmode) {  // sample.rs:411-414
            thresh = C.min_p * (1.0f / S);
            if (sorted) {
                const int lim2 = (int)(Lp < lim ? Lp : lim);
                const uint64_t fail = __ballot(lane < lim2 && p < thresh);
                Lm = fail ? (int64_t)__ffsll((unsigned long long)fail) - 1 : lim2;
            } else {
                Lm = __popcll(__ballot(valid && p >= thresh));
            }
            if (Lm == 0) {  // sample.rs:415-422
                token_target = true;
                tok = rawmax.v > -__builtin_inff() ? rawmax.i : 0u;
                verdict = C.judged ? (tok == C.draft) : 1u;
            }
        }
        if (!token_target) {
            const int64_t L = sorted ? min(Lk, min(Lp, Lm)) : Lm;
            const int nl = sorted ? (int)(L < N ? L : N) : N;
            const bool kept = sorted ? lane < nl : (valid && p >= thresh);
            if (a.t_kind) {
                const bool listed = kept && p > 0.0f;
                const uint64_t lm = __ballot(listed);
                const int o = __popcll(lm & lanes_below());
                if (listed && o < a.t_cap) {
                    a.t_ids[(int64_t)C.row * a.t_cap + o] = idx;
                    a.t_probs[(int64_t)C.row * a.t_cap + o] = p;
                }
                if (lane == 0) {
                    a.t_kind[C.row] = BFI_SMP_TARGET_WEIGHTS;
                    a.t_kept[C.row] = (int32_t)L;
                    a.t_listed[C.row] = (int32_t)min((int64_t)__popcll(lm), a.t_cap);
                }
            }
            const double w = kept ? (double)p : 0.0;
            const double cumk = wave_incl_scan_d(w);
            const double sum = __shfl(cumk, WAVE - 1);
            if (!C.judged) {  // draw, sample.rs:312-323
                const double r = (double)C.u * sum;
                const uint64_t hit = __ballot(kept && cumk >= r);
                const int j = hit ? __ffsll((unsigned long long)hit) - 1 : 0;
                tok = __shfl(idx, j);
            } else {  // judge, spec.rs:83-95
                const uint64_t dm = __ballot(kept && idx == C.draft);
                const int pd = dm ? __ffsll((unsigned long long)dm) - 1 : -1;
                const double p_d = pd >= 0 ? (double)__shfl(p, pd) : 0.0;
                if (sum > 0.0 && (double)C.u < p_d / sum) {
                    tok = C.draft;
                    verdict = 1;
                } else {
                    const bool res = kept && lane != pd;
                    if (__ballot(res && p > 0.0f) == 0) {  // residual empty or all <= 0
                        tok = C.draft;
                        verdict = 1;
                    } else {
                        const double cum2 = wave_incl_scan_d(res ? (double)p : 0.0);
                        const double r2 = (double)C.u2 * (sum - p_d);
                        const uint64_t hit = __ballot(res && cum2 >= r2);
                        const int j = hit ? __ffsll((unsigned long long)hit) - 1 : 0;
                        tok = __shfl(idx, j);
                        verdict = 0;
                    }
                }
            }
        }
        if (lane == 0) {
            sm.misc[4 + R_TOK] = tok;
            sm.misc[4 + R_VERDICT] = verdict;
            sm.misc[4 + R_TOKEN_TARGET] = token_target;
        }
    }
    __syncthreads();
    const uint32_t tok = sm.misc[4 + R_TOK], verdict = sm.misc[4 + R_VERDICT];
    const bool token_target = sm.misc[4 + R_TOKEN_TARGET] != 0;
    __syncthreads();
    if (token_target) {
        finish_token(a, sm, C, tok);
        return;
    }
    if (a.t_kind && threadIdx.x == 0 && a.out_tok) a.out_tok[C.row] = tok;
    emit(a, sm, C, tok, verdict);
}

// Returns false when the candidates do not fit (caller falls back to the radix select).
__device__ __forceinline__ bool combine_bounded(const KArgs& a, Smem& sm, const RowCtx& C, const ChunkPart& mine,
                                float M, float S, ArgMax rawmax, int64_t tb) {
    const int tid = threadIdx.x;
    const int nc = a.n_chunks;
    const bool sorted = C.kmode || C.pmode;  // else min-p only: index order (sample.rs:411-414)
    // global candidate threshold: tightest chunk bound, and the min-p bound at the row max
    float theta = tid < nc ? mine.theta : -__builtin_inff();
    theta = block_max(theta, sm.rf);
    if (C.mmode) {
        float lm = logf(C.min_p);
        float margin = 1e-4f + 1e-5f * (fabsf(M) + fabsf(lm));
        theta = fmaxf(theta, M + lm - margin);
    }
    // prefix of candidate counts over chunks (a chunk whose max is below theta has none)
    uint32_t myn = (tid < nc && mine.m >= theta) ? mine.ncand : 0u;
    uint32_t tot;
    uint32_t off = block_excl_scan<uint32_t>(myn, sm.ru, tot);
    if (tid < nc) sm.cpre[tid] = off;
    if (tid == 0) {
        sm.cpre[nc] = tot;
        sm.misc[MISC_N] = 0;
    }
    __syncthreads();
    const Cand* cands = a.cands + (int64_t)C.row * nc * CAND_CAP;
    constexpr int GU = 4;  // loads in flight per thread
    for (uint32_t f0 = tid; f0 < tot; f0 += GU * BLOCK) {
        Cand cd[GU];
#pragma unroll
        for (int g = 0; g < GU; g++) {
            const uint32_t f = f0 + g * BLOCK;
            cd[g].idx = 0;
            cd[g].s = -__builtin_inff();
            if (f < tot) {
                int lo = 0, hi = nc;  // largest c with cpre[c] <= f
                while (hi - lo > 1) {
                    int mid = (lo + hi) >> 1;
                    if (sm.cpre[mid] <= f) lo = mid;
                    else hi = mid;
                }
                cd[g] = cands[(int64_t)lo * CAND_CAP + (f - sm.cpre[lo])];
            }
        }
#pragma unroll
        for (int g = 0; g < GU; g++) {
            if (cd[g].s >= theta && cd[g].s > -__builtin_inff()) {
                uint32_t slot = lds_add(&sm.misc[MISC_N], 1u);
                if (slot < NMAX)
                    sm.u.cb.keys[slot] = sorted ? key64(cd[g].s, cd[g].idx)
                                                : (((uint64_t)(~cd[g].idx) << 32) | ord32(cd[g].s));
            }
        }
    }
    __syncthreads();
    const int N = (int)sm.misc[MISC_N];
    BFI_TRACE(a, tb, 2);
    if (a.trace && tid == 0) a.trace[tb + 6] = ((uint64_t)tot << 32) | (uint32_t)N;
    if (N > NMAX) return false;
    if (N <= WAVE) {
        combine_wave(a, sm, C, N, sorted, M, S, rawmax);
        return true;
    }
    int n2 = 64;
    while (n2 < N) n2 <<= 1;
    for (int j = N + tid; j < n2; j += BLOCK) sm.u.cb.keys[j] = 0ull;
    __syncthreads();
    bitonic_sort_desc(sm.u.cb.keys, n2);
    BFI_TRACE(a, tb, 3);
    // probabilities of the sorted positions: p = expf(s - M) / S (sample.rs:383, 388)
    for (int j = tid; j < N; j += BLOCK) {
        uint64_t k = sm.u.cb.keys[j];
        float s = sorted ? key_s(k) : unord32((uint32_t)k);
        sm.u.cb.p[j] = expf(s - M) / S;
    }
    __syncthreads();
    auto idx_at = [&](int j) -> uint32_t {
        uint64_t k = sm.u.cb.keys[j];
        return sorted ? key_idx(k) : ~(uint32_t)(k >> 32);
    };
    const float* p = sm.u.cb.p;

    int64_t Lk = C.kmode ? C.k : a.V;
    int64_t Lp = INT64_MAX, Lm = INT64_MAX;
    int lim = (int)(Lk < N ? Lk : N);
    if (sorted && C.pmode) {  // sample.rs:397-409
        uint32_t j = first_cum_ge(sm, lim, [&](int i) { return (double)p[i]; }, [](int) { return true; },
                                  (double)C.top_p);
        Lp = j == 0xFFFFFFFFu ? Lk : (int64_t)j + 1;
    }
    float thresh = 0.0f;
    if (C.mmode) {  // sample.rs:411-414
        float pmax = 1.0f / S;
        thresh = C.min_p * pmax;
        if (sorted) {
            int lim2 = (int)(Lp < lim ? Lp : lim);
            uint32_t j = first_cum_ge(sm, lim2, [&](int i) { return p[i] >= thresh ? 0.0 : 1.0; },
                                      [](int) { return true; }, 0.5);
            Lm = j == 0xFFFFFFFFu ? lim2 : (int64_t)j;
        } else {
            uint32_t c = 0;
            for (int j = tid; j < N; j += BLOCK) c += p[j] >= thresh;
            Lm = block_sum_u(c, sm.ru);
        }
        if (Lm == 0) {  // sample.rs:415-422: argmax of the masked, un-penalized logits
            uint32_t tok = rawmax.v > -__builtin_inff() ? rawmax.i : 0u;
            finish_token(a, sm, C, tok);
            return true;
        }
    }
    const int64_t L = sorted ? min(Lk, min(Lp, Lm)) : Lm;
    const int nl = sorted ? (int)(L < N ? L : N) : N;  // list positions that can be kept
    auto kept = [&](int j) -> bool { return sorted ? j < nl : (p[j] >= thresh); };
    auto wk = [&](int j) -> double { return kept(j) ? (double)p[j] : 0.0; };

    // target introspection
    if (a.t_kind) {
        if (tid == 0) {
            a.t_kind[C.row] = BFI_SMP_TARGET_WEIGHTS;
            a.t_kept[C.row] = (int32_t)L;
        }
        // list kept entries with p > 0 in draw order
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

    BFI_TRACE(a, tb, 4);
    const double sum = list_sum(sm, nl, wk);
    if (!C.judged) {  // draw (sample.rs:312-323)
        double r = (double)C.u * sum;
        uint32_t j = first_cum_ge(sm, nl, wk, kept, r);
        uint32_t tok = j == 0xFFFFFFFFu ? 0u : idx_at((int)j);
        if (a.t_kind && tid == 0 && a.out_tok) a.out_tok[C.row] = tok;
        emit(a, sm, C, tok, 1u);
        return true;
    }
    // judge (spec.rs:83-95)
    uint32_t pd = 0xFFFFFFFFu;
    for (int j = tid; j < nl; j += BLOCK)
        if (kept(j) && idx_at(j) == C.draft) pd = (uint32_t)j;
    pd = block_min_u(pd, sm.ru);
    const double p_d = pd == 0xFFFFFFFFu ? 0.0 : (double)p[pd];
    if (sum > 0.0 && (double)C.u < p_d / sum) {
        emit(a, sm, C, C.draft, 1u);
        return true;
    }
    uint32_t pos = 0;
    for (int j = tid; j < nl; j += BLOCK) pos += (kept(j) && (uint32_t)j != pd && p[j] > 0.0f);
    pos = block_sum_u(pos, sm.ru);
    if (pos == 0) {  // residual empty or all <= 0: Accept (spec.rs:90-93)
        emit(a, sm, C, C.draft, 1u);
        return true;
    }
    auto wr = [&](int j) -> double { return (kept(j) && (uint32_t)j != pd) ? (double)p[j] : 0.0; };
    double r2 = (double)C.u2 * (sum - p_d);
    uint32_t j = first_cum_ge(sm, nl, wr, [&](int i) { return kept(i) && (uint32_t)i != pd; }, r2);
    uint32_t tok = j == 0xFFFFFFFFu ? 0u : idx_at((int)j);
    emit(a, sm, C, tok, 0u);
    return true;
}

// ---- combine: unfiltered rows, draw in index order -------------------------------------

// Weights p = expf(s - M) / S of one tile of [t0, t1) (0 outside it and for `excl`).
template <bool BF16, int VEC>
__device__ __forceinline__ void tile_weights(const KArgs& a, Smem& sm, const RowCtx& C, uint32_t c0, uint32_t t0,
                                             uint32_t t1, float M, float S, uint32_t excl,
                                             float (&x)[VEC][Elem<BF16>::EPV]) {
    constexpr int EPV = Elem<BF16>::EPV;
    load_tile<BF16, VEC>(a, C.row, t0, t1, x);
    PenSrc S0{false, c0, nullptr, nullptr, nullptr};
    transform_tile<BF16, VEC>(sm, C, S0, t0, t1, x);
#pragma unroll
    for (int q = 0; q < VEC; q++)
#pragma unroll
        for (int e = 0; e < EPV; e++) {
            uint32_t id = t0 + (uint32_t)(q * BLOCK + threadIdx.x) * EPV + e;
            x[q][e] = (id < t1 && id != excl) ? expf(x[q][e] - M) / S : 0.0f;
        }
}

// Re-reads chunk [c0, c1) and returns the first index (in index order) where the
// cumulative weight reaches frac * (chunk total); d is excluded when excl != UINT32_MAX.
template <bool BF16, int VEC>
__device__ __forceinline__ uint32_t scan_chunk_index_order(const KArgs& a, Smem& sm, const RowCtx& C, uint32_t c0,
                                                           uint32_t c1, float M, float S, uint32_t excl,
                                                           double frac) {
    constexpr int EPV = Elem<BF16>::EPV;
    constexpr uint32_t TILE = (uint32_t)BLOCK * VEC * EPV;
    const int tid = threadIdx.x;
    if (C.pen_on) build_chunk_pen(sm, C, c0, c1, hist_prefetch(C));
    float x[VEC][EPV];
    double tsum = 0.0;
    for (uint32_t t0 = c0; t0 < c1; t0 += TILE) {
        tile_weights<BF16, VEC>(a, sm, C, c0, t0, min(t0 + TILE, c1), M, S, excl, x);
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
        tile_weights<BF16, VEC>(a, sm, C, c0, t0, t1, M, S, excl, x);
#pragma unroll
        for (int q = 0; q < VEC; q++) {  // VEC slabs in index order
            double ts = 0.0;
#pragma unroll
            for (int e = 0; e < EPV; e++) {
                ts += x[q][e];
                uint32_t id = t0 + (uint32_t)(q * BLOCK + tid) * EPV + e;
                if (x[q][e] > 0.0f) lastpos = max(lastpos, id + 1);
            }
            double tot;
            double pre = block_excl_scan<double>(ts, sm.rd, tot);
            if (found == 0xFFFFFFFFu && carry + tot >= target) {
                uint32_t best = 0xFFFFFFFFu;
                double c = carry + pre;
#pragma unroll
                for (int e = 0; e < EPV; e++) {
                    uint32_t id = t0 + (uint32_t)(q * BLOCK + tid) * EPV + e;
                    c += x[q][e];
                    if (best == 0xFFFFFFFFu && x[q][e] > 0.0f && c >= target) best = id;
                }
                found = block_min_u(best, sm.ru);
            }
            carry += tot;
        }
    }
    if (found == 0xFFFFFFFFu) {  // rounding at the chunk end: last positive element
        uint32_t l = (uint32_t)block_max_u64(lastpos, sm.r64);
        found = l ? l - 1 : c0;
    }
    return found;
}

// s of one element (penalties computed by scanning the history).
__device__ __forceinline__ float element_s(const KArgs& a, Smem& sm, const RowCtx& C, uint32_t id, bool bf16) {
    const int tid = threadIdx.x;
    if (id >= (uint32_t)a.V) return -__builtin_inff();  // a draft outside the vocabulary
    float x;
    if (bf16)
        x = __uint_as_float((uint32_t)((const uint16_t*)a.logits)[(int64_t)C.row * a.row_stride + id] << 16);
    else
        x = ((const float*)a.logits)[(int64_t)C.row * a.row_stride + id];
    if (C.mrow && !((C.mrow[id >> 5] >> (id & 31)) & 1u)) x = -__builtin_inff();
    uint32_t c = 0;
    if (C.pen_on) {
        const int64_t H = C.h.size();
        for (int64_t j = tid; j < H; j += BLOCK) c += C.h.at(j) == id;
        c = block_sum_u(c, sm.ru);
        if (c) x = penalize(x, c, C.pen);
    }
    return C.greedy ? x : div_T(x, C);
}

template <bool BF16, int VEC>
__device__ __forceinline__ void combine_unfiltered(const KArgs& a, Smem& sm, const RowCtx& C, const ChunkPart& mine,
                                   float M, float S) {
    const int tid = threadIdx.x;
    const int nc = a.n_chunks;
    // chunk masses: sum_c exp(m_c - M) / S ~ sum of p over the chunk
    double mc = (tid < nc && mine.m > -__builtin_inff()) ? (double)mine.sum * (double)expf(mine.m - M) / (double)S
                                                       : 0.0;
    uint32_t pd_chunk = 0xFFFFFFFFu;
    double p_d = 0.0;
    if (C.judged) {
        float sd = element_s(a, sm, C, C.draft, BF16);
        p_d = (double)(expf(sd - M) / S);
        pd_chunk = C.draft / (uint32_t)a.chunk;
        if ((uint32_t)tid == pd_chunk) mc = mc > p_d ? mc - p_d : 0.0;
    }
    double total;
    double pre = block_excl_scan<double>(mc, sm.rd, total);
    const double sum = total + p_d;  // sum of kept weights (all of V)
    if (a.t_kind && tid == 0) {
        a.t_kind[C.row] = BFI_SMP_TARGET_WEIGHTS;
        a.t_kept[C.row] = a.V;
        a.t_listed[C.row] = 0;
    }
    float u = C.u;
    bool resid = false;
    if (C.judged) {
        if (sum > 0.0 && (double)C.u < p_d / sum) {
            emit(a, sm, C, C.draft, 1u);
            return;
        }
        if (!(total > 0.0)) {
            emit(a, sm, C, C.draft, 1u);
            return;
        }
        u = C.u2;
        resid = true;
    }
    const double r = (double)u * total;
    uint32_t tok;
    if (r <= 0.0 && !resid) {
        tok = 0;  // r = 0: the first element of index order (sample.rs:314-319)
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
        double before = sm.rd[0], mass = sm.rd[1];
        __syncthreads();
        double frac = mass > 0.0 ? (r - before) / mass : 0.0;
        frac = frac < 0.0 ? 0.0 : (frac > 1.0 ? 1.0 : frac);
        uint32_t c0 = c * (uint32_t)a.chunk, c1 = min(c0 + (uint32_t)a.chunk, (uint32_t)a.V);
        tok = scan_chunk_index_order<BF16, VEC>(a, sm, C, c0, c1, M, S, resid ? C.draft : 0xFFFFFFFFu, frac);
    }
    if (a.t_kind && tid == 0 && a.out_tok) a.out_tok[C.row] = tok;
    emit(a, sm, C, tok, resid ? 0u : 1u);
}

// ---- combine: radix select over the row ------------------------------------------------

struct Sel {
    uint64_t key;       // selected element
    uint64_t pos;       // its 0-based position in the sorted order
    uint64_t cum_mass;  // fixed-point mass through it (inclusive)
};

// One pass over the whole row: f(id, s) for every element (s = transformed value).
template <bool BF16, int VEC, typename F>
__device__ __forceinline__ void row_pass(const KArgs& a, Smem& sm, const RowCtx& C, const PenSrc& P, F f) {
    constexpr int EPV = Elem<BF16>::EPV;
    const uint32_t tile = (uint32_t)BLOCK * EPV * VEC;
    for (uint32_t t0 = 0; t0 < (uint32_t)a.V; t0 += tile) {
        const uint32_t t1 = min(t0 + tile, (uint32_t)a.V);
        float x[VEC][EPV];
        load_tile<BF16, VEC>(a, C.row, t0, t1, x);
        transform_tile<BF16, VEC>(sm, C, P, t0, t1, x);
#pragma unroll
        for (int q = 0; q < VEC; q++)
#pragma unroll
            for (int e = 0; e < EPV; e++) {
                uint32_t id = t0 + (uint32_t)(q * BLOCK + threadIdx.x) * EPV + e;
                if (id < t1) f(id, x[q][e]);
            }
    }
}

// Finds the element at a sorted position (kind 0: 0-based position `target`) or the first
// element whose inclusive fixed-point cumulative mass reaches `target` (kind 1), over the
// order of key64 descending, skipping the element with key `excl`.
template <bool BF16, int VEC>
__device__ __forceinline__ Sel radix_select(const KArgs& a, Smem& sm, const RowCtx& C, const PenSrc& P, float M,
                            double scale, int kind, uint64_t target, uint64_t excl, uint64_t excl_mass) {
    const int tid = threadIdx.x;
    uint64_t prefix = 0;
    int pbits = 0;
    uint64_t before_cnt = 0, before_mass = 0;
    uint64_t* saved = a.row_hist + (int64_t)C.row * NBUCKET * 2;
    for (int level = 0;; level++) {
        const int w = (64 - pbits) >= 10 ? 10 : 64 - pbits;
        const int shift = 64 - pbits - w;
        const uint32_t nb = 1u << w;
        if (level == 0) {  // the level-1 histogram saved by radix_l1 (minus `excl`)
            for (uint32_t b = tid; b < NBUCKET; b += BLOCK) {
                sm.u.hs.mass[b] = saved[2 * b];
                sm.u.hs.cnt[b] = (uint32_t)saved[2 * b + 1];
            }
            __syncthreads();
            if (excl != ~0ull && tid == 0) {
                uint32_t b = (uint32_t)(excl >> 54);
                sm.u.hs.cnt[b] -= 1;
                sm.u.hs.mass[b] -= excl_mass;
            }
            __syncthreads();
        } else {
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
        // scan buckets from the top (o = 0 is bucket nb-1); 4 buckets per thread
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

// Level-1 histogram (top 10 key bits) of the whole row, saved to global scratch for every
// later query of this row; returns the total fixed-point mass.
template <bool BF16, int VEC>
__device__ __forceinline__ uint64_t radix_l1(const KArgs& a, Smem& sm, const RowCtx& C, const PenSrc& P, float M, double scale) {
    const int tid = threadIdx.x;
    for (uint32_t b = tid; b < NBUCKET; b += BLOCK) {
        sm.u.hs.mass[b] = 0;
        sm.u.hs.cnt[b] = 0;
    }
    __syncthreads();
    row_pass<BF16, VEC>(a, sm, C, P, [&](uint32_t id, float s) __attribute__((always_inline)) {
        uint32_t b = (uint32_t)(key64(s, id) >> 54);
        lds_add(&sm.u.hs.cnt[b], 1u);
        uint64_t m = efix_of(s, M, scale);
        if (m) lds_add64(&sm.u.hs.mass[b], m);
    });
    __syncthreads();
    uint64_t* saved = a.row_hist + (int64_t)C.row * NBUCKET * 2;
    uint64_t m = 0;
    for (uint32_t b = tid; b < NBUCKET; b += BLOCK) {
        saved[2 * b] = sm.u.hs.mass[b];
        saved[2 * b + 1] = sm.u.hs.cnt[b];
        m += sm.u.hs.mass[b];
    }
    uint64_t tot;
    block_excl_scan<uint64_t>(m, sm.r64, tot);
    __threadfence_block();
    __syncthreads();
    return tot;
}

template <bool BF16, int VEC>
__device__ __forceinline__ void combine_radix(const KArgs& a, Smem& sm, const RowCtx& C, float M, float S, ArgMax rawmax) {
    const int tid = threadIdx.x;
    build_row_pen(a, sm, C);
    const int nw = a.bm_words;
    const uint32_t* gbm = a.row_pen + (int64_t)C.row * (2 * nw + GDCAP);
    PenSrc P{true, 0u, gbm, gbm + nw, gbm + 2 * nw};
    const double scale = ldexp(1.0, a.fix_bits);
    const uint64_t V = (uint64_t)a.V;

    const uint64_t S_fix = radix_l1<BF16, VEC>(a, sm, C, P, M, scale);
    uint64_t Lk = C.kmode ? (uint64_t)C.k : V;
    uint64_t Lp = ~0ull, Lm = ~0ull;
    Sel selp{0, 0, 0};
    if (C.pmode) {  // sample.rs:397-409
        double tp = ceil((double)C.top_p * (double)S_fix);
        uint64_t T = tp <= 0.0 ? 0ull : (uint64_t)tp;
        if (C.kmode) {
            // top-p runs over the top-k list: cut inside it, or keep all k
            Sel sk = radix_select<BF16, VEC>(a, sm, C, P, M, scale, 0, Lk - 1, ~0ull, 0);
            if (sk.cum_mass < T) {
                Lp = Lk;
                selp = sk;
            } else {
                selp = radix_select<BF16, VEC>(a, sm, C, P, M, scale, 1, T, ~0ull, 0);
                Lp = selp.pos + 1;
            }
        } else {
            selp = radix_select<BF16, VEC>(a, sm, C, P, M, scale, 1, T, ~0ull, 0);
            Lp = selp.pos + 1;
        }
    }
    float thresh = 0.0f;
    if (C.mmode) {  // sample.rs:411-414: count p >= min_p * max_p
        thresh = C.min_p * (1.0f / S);
        uint32_t c = 0;
        row_pass<BF16, VEC>(a, sm, C, P, [&](uint32_t, float s) __attribute__((always_inline)) { c += (expf(s - M) / S >= thresh) ? 1u : 0u; });
        Lm = block_sum_u(c, sm.ru);
        if (Lm == 0) {
            uint32_t tok = rawmax.v > -__builtin_inff() ? rawmax.i : 0u;
            finish_token(a, sm, C, tok);
            return;
        }
    }
    uint64_t L = Lk < Lp ? Lk : Lp;
    L = L < Lm ? L : Lm;
    Sel last;
    if (C.pmode && L == Lp) {
        last = selp;
    } else {
        last = radix_select<BF16, VEC>(a, sm, C, P, M, scale, 0, L - 1, ~0ull, 0);
    }
    const uint64_t kept_mass = last.cum_mass;
    if (a.t_kind && tid == 0) {
        a.t_kind[C.row] = BFI_SMP_TARGET_WEIGHTS;
        a.t_kept[C.row] = (int32_t)L;
        a.t_listed[C.row] = 0;
    }
    // introspection listing: gather keys >= last.key when they fit
    if (a.t_kind && a.t_cap > 0 && L <= (uint64_t)NMAX) {
        if (tid == 0) sm.misc[MISC_N] = 0;
        __syncthreads();
        row_pass<BF16, VEC>(a, sm, C, P, [&](uint32_t id, float s) __attribute__((always_inline)) {
            uint64_t k = key64(s, id);
            if (k >= last.key) {
                uint32_t slot = lds_add(&sm.misc[MISC_N], 1u);
                if (slot < NMAX) sm.u.cb.keys[slot] = k;
            }
        });
        __syncthreads();
        int N = (int)min(sm.misc[MISC_N], (uint32_t)NMAX);
        int n2 = 64;
        while (n2 < N) n2 <<= 1;
        for (int j = N + tid; j < n2; j += BLOCK) sm.u.cb.keys[j] = 0ull;
        __syncthreads();
        bitonic_sort_desc(sm.u.cb.keys, n2);
        uint32_t c = 0;
        for (int j = tid * PT; j < tid * PT + PT; j++) {
            if (j < N) {
                float pj = expf(key_s(sm.u.cb.keys[j]) - M) / S;
                c += pj > 0.0f;
            }
        }
        uint32_t tc;
        uint32_t o = block_excl_scan<uint32_t>(c, sm.ru, tc);
        for (int j = tid * PT; j < tid * PT + PT; j++) {
            if (j < N) {
                float pj = expf(key_s(sm.u.cb.keys[j]) - M) / S;
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
        double r = ceil((double)C.u * (double)kept_mass);
        Sel d = radix_select<BF16, VEC>(a, sm, C, P, M, scale, 1, (uint64_t)r, ~0ull, 0);
        uint32_t tok = key_idx(d.key);
        if (a.t_kind && tid == 0 && a.out_tok) a.out_tok[C.row] = tok;
        emit(a, sm, C, tok, 1u);
        return;
    }
    // judge
    float sd = element_s(a, sm, C, C.draft, BF16);
    uint64_t kd = key64(sd, C.draft);
    bool kept_d = C.draft < V && kd >= last.key;
    uint64_t md = kept_d ? efix_of(sd, M, scale) : 0ull;
    if (kept_mass > 0 && (double)C.u < (double)md / (double)kept_mass) {
        emit(a, sm, C, C.draft, 1u);
        return;
    }
    uint64_t resid = kept_mass - md;
    if (resid == 0) {
        emit(a, sm, C, C.draft, 1u);
        return;
    }
    double r2 = ceil((double)C.u2 * (double)resid);
    Sel d = radix_select<BF16, VEC>(a, sm, C, P, M, scale, 1, (uint64_t)r2, kept_d ? kd : ~0ull, md);
    emit(a, sm, C, key_idx(d.key), 0u);
}

// ---- the kernel ------------------------------------------------------------------------

template <bool BF16, int VEC>
__global__ __launch_bounds__(BLOCK, 5) void k_stream(KArgs a) {
    constexpr int EPV = Elem<BF16>::EPV;
    __shared__ StreamSmem sm;
    const int tid = threadIdx.x;

    // workgroups are dispatched round-robin over the 8 XCDs: give each XCD a contiguous
    // range of (row, chunk) so a row's chunks share one L2
    const uint32_t G = gridDim.x, bid = blockIdx.x;
    const uint32_t q8 = G / 8, r8 = G % 8, xcd = bid % 8, slot = bid / 8;
    const uint32_t logical = xcd < r8 ? xcd * (q8 + 1) + slot : r8 * (q8 + 1) + (xcd - r8) * q8 + slot;
    const int row = (int)(logical / (uint32_t)a.n_chunks);
    const int chunk = (int)(logical % (uint32_t)a.n_chunks);
    const int64_t tb = (int64_t)logical * 8;
    BFI_TRACE(a, tb, 0);
    if (row >= a.n_rows) return;
    const RowCtx C = make_ctx(a, row);
    if (!C.active) return;

    const uint32_t V = (uint32_t)a.V;
    const uint32_t c0 = (uint32_t)chunk * (uint32_t)a.chunk;
    const uint32_t c1 = min(c0 + (uint32_t)a.chunk, V);

    // ---- stream phase
    const HistPre hp = hist_prefetch(C);
    float x[VEC][EPV];
    load_tile<BF16, VEC>(a, row, c0, c1, x);
    if (C.pen_on) build_chunk_pen(sm, C, c0, c1, hp);
    BFI_TRACE(a, tb, 1);
    const bool track_raw = !C.greedy && C.min_p > 1.0f;
    ArgMax raw{-__builtin_inff(), 0xFFFFFFFFu};
    PenSrc S0{false, c0, nullptr, nullptr, nullptr};
    if (track_raw)
        raw = transform_tile<BF16, VEC, true>(sm, C, S0, c0, c1, x);
    else
        transform_tile<BF16, VEC, false>(sm, C, S0, c0, c1, x);
    if (track_raw) raw = block_argmax(raw, sm.rf, sm.ru);
    if (a.trace) {  // force the transform to complete before the stamp
        float t = 0.0f;
#pragma unroll
        for (int q = 0; q < VEC; q++) t += x[q][0];
        if (t == 12345.678f) a.trace[tb + 7] = 1;
    }
    BFI_TRACE(a, tb, 2);

    ChunkPart part;
    part.pad = 0;
    part.raw_m = raw.v;
    part.raw_arg = raw.i;
    if (C.greedy) {
        ArgMax best{-__builtin_inff(), 0xFFFFFFFFu};
#pragma unroll
        for (int q = 0; q < VEC; q++)
#pragma unroll
            for (int e = 0; e < EPV; e++)
                best = argmax_merge(best, ArgMax{x[q][e], c0 + (uint32_t)(q * BLOCK + tid) * EPV + e});
        best = block_argmax(best, sm.rf, sm.ru);
        part.m = best.v;
        part.arg = best.i;
        part.sum = 0.0f;
        part.ncand = 0;
        part.theta = -__builtin_inff();
    } else {
        float lm = -__builtin_inff();
#pragma unroll
        for (int q = 0; q < VEC; q++)
#pragma unroll
            for (int e = 0; e < EPV; e++) lm = fmaxf(lm, x[q][e]);
        const float mc = block_max(lm, sm.rf);
        BFI_TRACE(a, tb, 3);
        part.m = mc;
        part.arg = 0;
        const bool kb = C.kmode && C.k <= CAND_CAP;
        const float margin = 1e-4f + 1e-5f * fabsf(mc);
        // min-p bound of this chunk: p >= min_p * max p needs s >= max_s + ln(min_p)
        float th = __builtin_inff();
        if (C.mmode && mc > -__builtin_inff()) {
            const float lmp = logf(C.min_p);
            th = mc + lmp - (margin + 1e-5f * fabsf(lmp));
        }
        // one pass: sum of exp(s - max) and the candidate count at th
        float ls = 0.0f;
        uint32_t lc = 0;
        if (mc > -__builtin_inff()) {
#pragma unroll
            for (int q = 0; q < VEC; q++)
#pragma unroll
                for (int e = 0; e < EPV; e++) {
                    const float v = x[q][e];
                    ls += __expf(v - mc);
                    lc += (v >= th) ? 1u : 0u;
                }
        }
        uint32_t cnt;
        part.sum = block_sum_fu(ls, lc, cnt, sm.rf, sm.ru);
        BFI_TRACE(a, tb, 4);
        if (!(mc > -__builtin_inff())) {
            part.ncand = 0;
            part.theta = -__builtin_inff();
        } else if (!(C.mmode || kb)) {
            part.ncand = NCAND_UNBOUNDED;
            part.theta = __builtin_inff();
        } else {
            if (!C.mmode) {
                th = -__builtin_inff();
                cnt = 0xFFFFFFFFu;
            }
            if (kb && cnt > (uint32_t)CAND_CAP) {
                // smallest power-of-two distance below the chunk max holding k elements,
                // then bisection toward <= CAND_CAP candidates
                float d = 0.25f, lo = 0.0f;
                uint32_t c = 0;
                int it = 0;
                for (; it < 18; it++) {
                    c = block_sum_u(tile_count_ge<BF16, VEC>(x, mc - d), sm.ru);
                    if (c >= (uint32_t)C.k) break;
                    lo = d;
                    d *= 2.0f;
                }
                float tk;
                if (c < (uint32_t)C.k) {
                    tk = -__builtin_inff();
                } else {
                    float hi = d;
                    const uint32_t want = max(2u * (uint32_t)C.k, 64u);  // a tight bound keeps the gather small
                    for (int j = 0; j < 12 && c > want; j++) {
                        float mid = 0.5f * (lo + hi);
                        uint32_t cm = block_sum_u(tile_count_ge<BF16, VEC>(x, mc - mid), sm.ru);
                        if (cm >= (uint32_t)C.k) {
                            hi = mid;
                            c = cm;
                        } else {
                            lo = mid;
                        }
                    }
                    tk = mc - hi - margin;
                }
                th = C.mmode ? fmaxf(th, tk) : tk;
                cnt = block_sum_u(tile_count_ge<BF16, VEC>(x, th), sm.ru);
            }
            part.theta = th;
            if (cnt > (uint32_t)CAND_CAP) {
                part.ncand = NCAND_OVERFLOW;
            } else {
                part.ncand = cnt;
                uint32_t my = tile_count_ge<BF16, VEC>(x, th), tot;
                uint32_t o = block_excl_scan<uint32_t>(my, sm.ru, tot);
                if (my) {
                    Cand* dst = a.cands + ((int64_t)row * a.n_chunks + chunk) * CAND_CAP;
#pragma unroll
                    for (int q = 0; q < VEC; q++)
#pragma unroll
                        for (int e = 0; e < EPV; e++) {
                            float v = x[q][e];
                            if (v >= th && v > -__builtin_inff()) {
                                dst[o].idx = c0 + (uint32_t)(q * BLOCK + tid) * EPV + e;
                                dst[o].s = v;
                                o++;
                            }
                        }
                }
            }
        }
    }
    if (tid == 0) a.parts[(int64_t)row * a.n_chunks + chunk] = part;
    BFI_TRACE(a, tb, 5);
}

// ---- select kernel: one workgroup per row ----------------------------------------------

template <bool BF16>
__global__ __launch_bounds__(BLOCK) void k_select(KArgs a) {
    constexpr int VEC = BF16 ? 2 : 4;  // row passes walk 4096-element tiles
    __shared__ Smem sm;
    const int tid = threadIdx.x;
    // rows grouped per XCD (dispatch is round-robin over the 8 XCDs)
    const uint32_t G = gridDim.x, bid = blockIdx.x;
    const uint32_t q8 = G / 8, r8 = G % 8, xcd = bid % 8, slot = bid / 8;
    const int row = (int)(xcd < r8 ? xcd * (q8 + 1) + slot : r8 * (q8 + 1) + (xcd - r8) * q8 + slot);
    const int64_t tb = ((int64_t)a.n_rows * a.n_chunks + row) * 8;
    BFI_TRACE(a, tb, 0);
    if (row >= a.n_rows) return;
    const RowCtx C = make_ctx(a, row);
    if (!C.active) return;
    const uint32_t V = (uint32_t)a.V;
    const bool track_raw = !C.greedy && C.min_p > 1.0f;

    const int nc = a.n_chunks;
    ChunkPart mine;
    if (tid < nc) {
        mine = a.parts[(int64_t)row * nc + tid];
    } else {
        mine.m = -__builtin_inff();
        mine.sum = 0.0f;
        mine.arg = 0xFFFFFFFFu;
        mine.ncand = 0;
        mine.theta = -__builtin_inff();
        mine.raw_m = -__builtin_inff();
        mine.raw_arg = 0xFFFFFFFFu;
    }
    if (C.greedy) {  // sample.rs:369-371
        ArgMax am = block_argmax(ArgMax{mine.m, mine.arg}, sm.rf, sm.ru);
        uint32_t tok = (am.v > -__builtin_inff()) ? am.i : 0u;
        finish_token(a, sm, C, tok);
        return;
    }
    ArgMax rawmax{-__builtin_inff(), 0xFFFFFFFFu};
    if (track_raw) rawmax = block_argmax(ArgMax{mine.raw_m, mine.raw_arg}, sm.rf, sm.ru);
    const float M = block_max(mine.m, sm.rf);
    if (!(M > -__builtin_inff())) {
        // every logit is -inf: NaN weights in the reference; its outcome is deterministic
        uint32_t tok;
        if (C.mmode) {
            tok = rawmax.v > -__builtin_inff() ? rawmax.i : 0u;
            finish_token(a, sm, C, tok);
            return;
        }
        const uint32_t L = C.kmode ? (uint32_t)C.k : V;
        if (a.t_kind && tid == 0) {
            a.t_kind[row] = BFI_SMP_TARGET_WEIGHTS;
            a.t_kept[row] = (int32_t)L;
            a.t_listed[row] = 0;
        }
        if (C.judged) {
            // residual = kept minus d; draw over NaN weights returns its last id
            uint32_t lastid = (C.draft == L - 1) ? L - 2 : L - 1;
            bool empty = (L == 1 && C.draft == 0);
            emit(a, sm, C, empty ? C.draft : lastid, empty ? 1u : 0u);
            return;
        }
        tok = L - 1;
        if (a.t_kind && tid == 0 && a.out_tok) a.out_tok[row] = tok;
        emit(a, sm, C, tok, 1u);
        return;
    }
    // S = sum exp(s - M): chunk sums rescaled to the row max, accumulated in f64
    double sc = (tid < nc && mine.m > -__builtin_inff()) ? (double)mine.sum * (double)expf(mine.m - M) : 0.0;
    const float S = (float)block_sum_d(sc, sm.rd);
    if (a.t_stats && tid == 0) {
        a.t_stats[row * 4 + 0] = M;
        a.t_stats[row * 4 + 1] = S;
    }

    BFI_TRACE(a, tb, 1);
    uint32_t flags = 0;  // 1 = some chunk unbounded/overflowed
    if (tid < nc && (mine.ncand == NCAND_UNBOUNDED || mine.ncand == NCAND_OVERFLOW)) flags = 1;
    flags = block_sum_u(flags, sm.ru);
    if (!C.kmode && !C.pmode && !C.mmode) {
        if (a.t_stats && tid == 0) a.t_stats[row * 4 + 3] = 2.0f;
        combine_unfiltered<BF16, VEC>(a, sm, C, mine, M, S);
        return;
    }
    if (flags == 0) {
        if (a.t_stats && tid == 0) a.t_stats[row * 4 + 3] = 1.0f;
        if (combine_bounded(a, sm, C, mine, M, S, rawmax, tb)) {
            BFI_TRACE(a, tb, 7);
            return;
        }
    }
    if (a.t_stats && tid == 0) a.t_stats[row * 4 + 3] = 3.0f;
    combine_radix<BF16, VEC>(a, sm, C, M, S, rawmax);
}


// ---- launch ----------------------------------------------------------------------------

hipError_t launch_stream(const KArgs& a, int bf16, int vec, hipStream_t stream) {
    const dim3 grid((unsigned)((int64_t)a.n_rows * a.n_chunks)), block(BLOCK);
#define BFI_LAUNCH(B, VV) hipLaunchKernelGGL((k_stream<B, VV>), grid, block, 0, stream, a)
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

hipError_t launch_select(const KArgs& a, int bf16, hipStream_t stream) {
    const dim3 grid((unsigned)a.n_rows), block(BLOCK);
    if (bf16)
        hipLaunchKernelGGL((k_select<true>), grid, block, 0, stream, a);
    else
        hipLaunchKernelGGL((k_select<false>), grid, block, 0, stream, a);
    return hipGetLastError();
}

}  // namespace bfi
