// smp_api.cpp — the C ABI of include/bfi_sampler.h: contexts, argument checks, device
// workspace, launch-shape choice. No exception or abort crosses the boundary; every
// failure is a status code plus a message (bfi_smp_last_error).
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <new>
#include <string>

#include "../../include/bfi_sampler.h"
#include "smp_device.h"

#include <mutex>
#include <vector>

// ---- the allocation-free entry point's workspace ---------------------------------------
//
// bfi_smp_sample_rows_noalloc runs the same kernels in a fixed device array instead of the
// context's allocated workspace (for callers that cannot allocate: graph capture, serving
// loops). Each device holds its own copy of the array from the library's load until the
// process ends; its address on a device comes from hipGetSymbolAddress (the array's name in
// host code is only a stand-in). Every call on a device shares it.
static __device__ __align__(256) unsigned char scratch[BFI_SMP_NOALLOC_BYTES];

namespace {
constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[MAX_DEVICES];  // per device: the array's device address (null: not yet)

// Resolves the array's address on `device` (the current device) once; 0 on success.
hipError_t scratch_setup(int device) {
    if (device < 0 || device >= MAX_DEVICES) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch_ptr[device]) return hipSuccess;
    void* ptr = nullptr;
    hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    g_scratch_ptr[device] = ptr;
    return hipSuccess;
}
void* scratch_ptr(int device) {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    return device >= 0 && device < MAX_DEVICES ? g_scratch_ptr[device] : nullptr;
}

// Zero-fill of counters that must start at zero (a kernel, not a memset: callers may capture
// the call into a graph).
__global__ void k_fill_zero(uint32_t* p, uint32_t n) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0u;
}
}  // namespace

namespace bfi {
hipError_t launch_stream(const KArgs& a, int bf16, int vec, hipStream_t stream, hipEvent_t start, hipEvent_t stop);
hipError_t launch_quant(const KArgs& a, int bf16, int vec, hipStream_t stream, hipEvent_t start, hipEvent_t stop);
hipError_t launch_row(const KArgs& a, int bf16, hipStream_t stream, hipEvent_t start, hipEvent_t stop);
hipError_t launch_head(const float* x, const float* norm_w, int norm_per_row, float eps, const float* W, int64_t n_tok,
                       int64_t d, int64_t n_out, int vec, int blocked, float* xn, float* out, hipStream_t stream);
hipError_t launch_dequant(int type, const void* src, int64_t n, float* dst, hipStream_t stream);
}

struct bfi_smp_ctx {
    int device = 0;
    std::string err;
    char* ws = nullptr;  // parts | vhist | row_res | row_pen | spill | rinfo | qpre | qhead | qitem
    size_t ws_size = 0;
    uint32_t* ctr = nullptr;  // arrival counters (per row), then seq_ctr; kept zero between launches
    size_t ctr_words = 0;
    bool ctr_dirty = false;
    // staging for bfi_smp_sample_host
    char* stage = nullptr;
    size_t stage_size = 0;
    // the output head's workspace: normalized rows, then (head_sample_rows) the logits
    char* head = nullptr;
    size_t head_size = 0;
    // phase trace of the last launch (diagnostics)
    uint64_t* trace = nullptr;
    size_t trace_words = 0, trace_used = 0;
    bool tracing = false;
    // profiling: per launch, start/stop events recorded in the dispatches of its three kernels
    bool profiling = false;
    std::vector<hipEvent_t> ev_pool;
    size_t ev_used = 0;
};

namespace {

thread_local std::string g_err;

int fail(bfi_smp_ctx* ctx, int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    if (ctx)
        ctx->err = buf;
    else
        g_err = buf;
    return code;
}

int hip_fail(bfi_smp_ctx* ctx, hipError_t e, const char* what) {
    if (ctx) ctx->ctr_dirty = true;
    return fail(ctx, BFI_SMP_EHIP, "%s: %s", what, hipGetErrorString(e));
}

struct DeviceGuard {
    int prev = -1;
    hipError_t err = hipSuccess;
    explicit DeviceGuard(int dev) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        if (prev != dev) err = hipSetDevice(dev);
    }
    ~DeviceGuard() {
        int cur = -1;
        if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
    }
};

size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

constexpr int EV_PER_LAUNCH = 6;  // start/stop of k_stream, k_quant, k_row


// Launch shape: 16-byte vectors per thread -> chunk of BLOCK*VEC*EPV elements. The largest
// chunk that still gives >= 1024 workgroups (4 per CU on 256 CUs); at most 256 chunks/row.
struct Shape {
    int vec, chunk, n_chunks;
};

bool choose_shape(int64_t n_rows, int64_t V, int bf16, Shape& s) {
    const int epv = bf16 ? 8 : 4;
    const int vecs_f32[3] = {8, 4, 2}, vecs_bf16[3] = {4, 2, 1};
    const int* vecs = bf16 ? vecs_bf16 : vecs_f32;
    bool found = false;
    for (int i = 0; i < 3; i++) {
        int chunk = bfi::BLOCK * vecs[i] * epv;
        int64_t nc = (V + chunk - 1) / chunk;
        if (nc > bfi::NCMAX) continue;
        s = Shape{vecs[i], chunk, (int)nc};
        found = true;
        if (n_rows * nc >= 1024) break;
    }
    return found;
}

// Window elements a chunk may list (beyond: it is streamed exactly).
size_t qcap_of(const Shape& s) { return (size_t)(s.chunk < bfi::QWIN ? s.chunk : bfi::QWIN); }

struct Layout {
    size_t parts, vhist, row_res, row_pen, spill, rinfo, qpre, qhead, qitem, rowcnt, total;
};

Layout layout(int64_t n_rows, int64_t V, const Shape& s, int bm_words) {
    Layout L;
    size_t off = 0;
    L.parts = off;
    off = align_up(off + (size_t)n_rows * s.n_chunks * sizeof(bfi::ChunkPart), 256);
    L.vhist = off;
    off = align_up(off + (size_t)n_rows * s.n_chunks * 2 * bfi::HBINS * sizeof(uint32_t), 256);
    L.row_res = off;
    off = align_up(off + (size_t)n_rows * 2 * sizeof(uint32_t), 256);
    L.row_pen = off;
    off = align_up(off + (size_t)n_rows * (2 * (size_t)bm_words + bfi::GDCAP) * sizeof(uint32_t), 256);
    L.spill = off;
    off = align_up(off + (size_t)n_rows * 4 * (size_t)V * sizeof(uint64_t), 256);
    L.rinfo = off;
    off = align_up(off + (size_t)n_rows * sizeof(bfi::RowInfo), 256);
    L.qpre = off;
    off = align_up(off + (size_t)n_rows * s.n_chunks * sizeof(bfi::QPre), 256);
    L.qhead = off;
    off = align_up(off + (size_t)n_rows * s.n_chunks * sizeof(bfi::QHead), 256);
    L.qitem = off;
    off = align_up(off + (size_t)n_rows * s.n_chunks * (qcap_of(s) + 1) * sizeof(bfi::QItem), 256);
    L.rowcnt = off;
    off = align_up(off + (size_t)n_rows * sizeof(uint32_t), 256);
    L.total = off;
    return L;
}

int ensure_ws(bfi_smp_ctx* ctx, size_t bytes, size_t ctr_words, hipStream_t stream) {
    if (bytes > ctx->ws_size) {
        if (ctx->ws) (void)hipFree(ctx->ws);
        ctx->ws = nullptr;
        ctx->ws_size = 0;
        size_t want = bytes + bytes / 4;
        if (hipMalloc((void**)&ctx->ws, want) != hipSuccess) {
            ctx->ws = nullptr;
            return fail(ctx, BFI_SMP_ENOMEM, "workspace allocation of %zu bytes failed", want);
        }
        ctx->ws_size = want;
    }
    if (ctr_words > ctx->ctr_words || ctx->ctr_dirty) {
        if (ctr_words > ctx->ctr_words) {
            if (ctx->ctr) (void)hipFree(ctx->ctr);
            ctx->ctr = nullptr;
            ctx->ctr_words = 0;
            size_t want = ctr_words < 4096 ? 4096 : ctr_words * 2;
            if (hipMalloc((void**)&ctx->ctr, want * sizeof(uint32_t)) != hipSuccess) {
                ctx->ctr = nullptr;
                return fail(ctx, BFI_SMP_ENOMEM, "counter allocation failed");
            }
            ctx->ctr_words = want;
        }
        hipError_t e = hipMemsetAsync(ctx->ctr, 0, ctx->ctr_words * sizeof(uint32_t), stream);
        if (e != hipSuccess) return hip_fail(ctx, e, "hipMemsetAsync(counters)");
        ctx->ctr_dirty = false;
    }
    return BFI_SMP_OK;
}

struct Call {
    const void* logits;
    int dtype;
    int64_t n_rows, V, row_stride;
    const bfi_smp_row_params* params;
    const uint32_t* hist;
    const int64_t* hist_off;
    const uint32_t* mask;
    int64_t mask_stride;
    const float* u;
    uint32_t* out;
    // target
    int32_t *kind = nullptr, *kept = nullptr, *listed = nullptr;
    uint32_t* ids = nullptr;
    float* probs = nullptr;
    int64_t cap = 0;
    float* stats = nullptr;
    // verify
    int64_t rows_per_seq = 0, n_seq = 0;
    const uint32_t* drafts = nullptr;
    const int32_t* draft_len = nullptr;
    const float *u_pairs = nullptr, *u_bonus = nullptr;
    int32_t* out_acc = nullptr;
    uint32_t* out_next = nullptr;
};

// A workspace the caller provides (the allocation-free entry point): base and capacity.
struct Fixed {
    char* base;
    size_t cap;
};

int run(bfi_smp_ctx* ctx, const Call& c, hipStream_t stream, const Fixed* fixed = nullptr) {
    if (c.dtype != BFI_SMP_F32 && c.dtype != BFI_SMP_BF16)
        return fail(ctx, BFI_SMP_EINVAL, "dtype %d is not BFI_SMP_F32 or BFI_SMP_BF16", c.dtype);
    if (c.n_rows < 0 || c.V < 0) return fail(ctx, BFI_SMP_EINVAL, "negative n_rows or n_vocab");
    if (c.n_rows == 0) return BFI_SMP_OK;
    if (c.V > (int64_t)1 << 21)
        return fail(ctx, BFI_SMP_EINVAL, "n_vocab %lld exceeds the supported 2097152", (long long)c.V);
    if (c.n_rows > (int64_t)1 << 24) return fail(ctx, BFI_SMP_EINVAL, "too many rows");
    if (!c.params) return fail(ctx, BFI_SMP_EINVAL, "params is NULL");
    if (c.V > 0 && !c.logits) return fail(ctx, BFI_SMP_EINVAL, "logits is NULL");
    if (c.V > 0 && c.row_stride < c.V) return fail(ctx, BFI_SMP_EINVAL, "row_stride < n_vocab");
    if (c.hist_off && !c.hist) return fail(ctx, BFI_SMP_EINVAL, "hist_off given without hist");
    const int bm_words = (int)((c.V + 31) / 32);
    if (c.mask && c.mask_stride < bm_words)
        return fail(ctx, BFI_SMP_EINVAL, "mask_stride %lld < ceil(n_vocab/32) = %d", (long long)c.mask_stride, bm_words);
    const bool verify = c.rows_per_seq > 0;
    if (verify) {
        if (!c.drafts && c.rows_per_seq > 1) return fail(ctx, BFI_SMP_EINVAL, "drafts is NULL");
        if (!c.draft_len || !c.u_bonus || !c.out_acc || !c.out_next)
            return fail(ctx, BFI_SMP_EINVAL, "verify output/input pointer is NULL");
        if (c.rows_per_seq > 1 && !c.u_pairs) return fail(ctx, BFI_SMP_EINVAL, "u_pairs is NULL");
    } else {
        if (!c.u) return fail(ctx, BFI_SMP_EINVAL, "u is NULL");
        if (!c.out) return fail(ctx, BFI_SMP_EINVAL, "out is NULL");
        if (c.kind && (!c.kept || !c.listed || (c.cap > 0 && (!c.ids || !c.probs))))
            return fail(ctx, BFI_SMP_EINVAL, "target outputs incomplete");
        if (c.cap < 0) return fail(ctx, BFI_SMP_EINVAL, "cap < 0");
    }
    if (c.V == 0) {
        // sample.rs:327-329: empty logits -> Token(0)
        return fail(ctx, BFI_SMP_EINVAL, "n_vocab == 0 on the device path (use bfi_smp_sample_host)");
    }
    DeviceGuard g(ctx->device);
    if (g.err != hipSuccess) return hip_fail(ctx, g.err, "hipSetDevice");

    Shape s;
    if (!choose_shape(c.n_rows, c.V, c.dtype == BFI_SMP_BF16, s))
        return fail(ctx, BFI_SMP_EINVAL, "no launch shape for n_vocab %lld", (long long)c.V);
    const Layout L = layout(c.n_rows, c.V, s, bm_words);
    const size_t ctr_words = (size_t)c.n_rows + (verify ? (size_t)c.n_seq : 0);
    char* ws = nullptr;
    uint32_t* ctr = nullptr;
    if (fixed) {
        const size_t need = L.total + align_up(ctr_words * sizeof(uint32_t), 256);
        if (need > fixed->cap)
            return fail(ctx, BFI_SMP_EINVAL,
                        "%lld rows of %lld logits need %zu bytes of workspace; the allocation-free entry point "
                        "holds %zu (BFI_SMP_NOALLOC_BYTES)",
                        (long long)c.n_rows, (long long)c.V, need, fixed->cap);
        ws = fixed->base;
        ctr = (uint32_t*)(fixed->base + L.total);
        // the counters start at zero (the kernels leave them so, but an earlier call may have
        // failed midway)
        const uint32_t n = (uint32_t)ctr_words;
        hipLaunchKernelGGL(k_fill_zero, dim3((n + 255) / 256), dim3(256), 0, stream, ctr, n);
        hipError_t e0 = hipGetLastError();
        if (e0 != hipSuccess) return hip_fail(ctx, e0, "counter fill launch");
    } else {
        int rc = ensure_ws(ctx, L.total, ctr_words, stream);
        if (rc) return rc;
        ws = ctx->ws;
        ctr = ctx->ctr;
    }

    bfi::KArgs a;
    memset(&a, 0, sizeof a);
    a.logits = c.logits;
    a.row_stride = c.row_stride;
    a.V = (int32_t)c.V;
    a.n_rows = (int32_t)c.n_rows;
    a.n_chunks = s.n_chunks;
    a.chunk = s.chunk;
    const size_t esz = c.dtype == BFI_SMP_BF16 ? 2 : 4;
    a.vec_ok = ((uintptr_t)c.logits % 16 == 0) && ((size_t)c.row_stride * esz % 16 == 0);
    a.params = c.params;
    a.hist = c.hist;
    a.hist_off = c.hist_off;
    a.mask = c.mask;
    a.mask_stride = c.mask_stride;
    a.u = c.u;
    a.out_tok = c.out;
    a.t_kind = c.kind;
    a.t_kept = c.kept;
    a.t_listed = c.listed;
    a.t_ids = c.ids;
    a.t_probs = c.probs;
    a.t_cap = c.cap;
    a.t_stats = c.stats;
    a.rows_per_seq = (int32_t)c.rows_per_seq;
    a.drafts = c.drafts;
    a.draft_len = c.draft_len;
    a.u_pairs = c.u_pairs;
    a.u_bonus = c.u_bonus;
    a.out_accepted = c.out_acc;
    a.out_next = c.out_next;
    a.parts = (bfi::ChunkPart*)(ws + L.parts);
    a.vhist = (uint32_t*)(ws + L.vhist);
    a.row_res = (uint32_t*)(ws + L.row_res);
    a.row_pen = (uint32_t*)(ws + L.row_pen);
    a.spill = (uint64_t*)(ws + L.spill);
    a.rinfo = (bfi::RowInfo*)(ws + L.rinfo);
    a.qpre = (bfi::QPre*)(ws + L.qpre);
    a.qhead = (bfi::QHead*)(ws + L.qhead);
    a.qitem = (bfi::QItem*)(ws + L.qitem);
    a.rowcnt = (uint32_t*)(ws + L.rowcnt);
    a.arrive = ctr;
    a.seq_ctr = ctr + c.n_rows;
    a.bm_words = bm_words;
    a.qcap = (int32_t)qcap_of(s);
    a.trace = nullptr;
    if (ctx->tracing && !fixed) {
        // the quantizing pass's workgroups (8 words), the rows (16), the streaming pass's
        // workgroups (8)
        size_t words = (size_t)c.n_rows * s.n_chunks * 16 + (size_t)c.n_rows * 16;
        if (words > ctx->trace_words) {
            if (ctx->trace) (void)hipFree(ctx->trace);
            ctx->trace = nullptr;
            ctx->trace_words = 0;
            if (hipMalloc((void**)&ctx->trace, words * 8) != hipSuccess)
                return fail(ctx, BFI_SMP_ENOMEM, "trace allocation failed");
            ctx->trace_words = words;
        }
        hipError_t e0 = hipMemsetAsync(ctx->trace, 0, words * 8, stream);
        if (e0 != hipSuccess) return hip_fail(ctx, e0, "hipMemsetAsync(trace)");
        ctx->trace_used = words;
        a.trace = ctx->trace;
    }

    hipEvent_t ev[EV_PER_LAUNCH] = {};
    if (ctx->profiling && !fixed) {
        if (ctx->ev_used + EV_PER_LAUNCH > ctx->ev_pool.size()) {
            if (ctx->ev_pool.size() >= EV_PER_LAUNCH * 65536)
                return fail(ctx, BFI_SMP_EINVAL, "profiling record full: read it");
            for (int i = 0; i < EV_PER_LAUNCH * 256; i++) {
                hipEvent_t x;
                hipError_t ee = hipEventCreate(&x);
                if (ee != hipSuccess) return hip_fail(ctx, ee, "hipEventCreate");
                ctx->ev_pool.push_back(x);
            }
        }
        for (int i = 0; i < EV_PER_LAUNCH; i++) ev[i] = ctx->ev_pool[ctx->ev_used + i];
        ctx->ev_used += EV_PER_LAUNCH;
    }
    const int bf16 = c.dtype == BFI_SMP_BF16;
    hipError_t e = hipSuccess;
    if ((e = bfi::launch_stream(a, bf16, s.vec, stream, ev[0], ev[1])) != hipSuccess)
        return hip_fail(ctx, e, "k_stream launch");
    if ((e = bfi::launch_quant(a, bf16, s.vec, stream, ev[2], ev[3])) != hipSuccess)
        return hip_fail(ctx, e, "k_quant launch");
    if ((e = bfi::launch_row(a, bf16, stream, ev[4], ev[5])) != hipSuccess)
        return hip_fail(ctx, e, "k_row launch");
    return BFI_SMP_OK;
}

}  // namespace

extern "C" {

int bfi_smp_abi_version(void) { return BFI_SMP_ABI_VERSION; }

int bfi_smp_create(int device, bfi_smp_ctx** out) {
    if (!out) return fail(nullptr, BFI_SMP_EINVAL, "out is NULL");
    *out = nullptr;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0) return fail(nullptr, BFI_SMP_EHIP, "no HIP device available");
    if (device < 0 || device >= n) return fail(nullptr, BFI_SMP_EINVAL, "device %d out of range (%d devices)", device, n);
    bfi_smp_ctx* ctx = new (std::nothrow) bfi_smp_ctx();
    if (!ctx) return fail(nullptr, BFI_SMP_ENOMEM, "context allocation failed");
    ctx->device = device;
    DeviceGuard g(device);
    if (g.err != hipSuccess) {
        delete ctx;
        return fail(nullptr, BFI_SMP_EHIP, "hipSetDevice(%d): %s", device, hipGetErrorString(g.err));
    }
    // the allocation-free entry point's array on this device (once per device)
    if ((e = scratch_setup(device)) != hipSuccess) {
        delete ctx;
        return fail(nullptr, BFI_SMP_EHIP, "hipGetSymbolAddress(scratch) on device %d: %s", device,
                    hipGetErrorString(e));
    }
    *out = ctx;
    return BFI_SMP_OK;
}

void bfi_smp_destroy(bfi_smp_ctx* ctx) {
    if (!ctx) return;
    {
        DeviceGuard g(ctx->device);
        for (hipEvent_t e : ctx->ev_pool) (void)hipEventDestroy(e);
        if (ctx->ws) (void)hipFree(ctx->ws);
        if (ctx->ctr) (void)hipFree(ctx->ctr);
        if (ctx->stage) (void)hipFree(ctx->stage);
        if (ctx->head) (void)hipFree(ctx->head);
    }
    delete ctx;
}

int bfi_smp_set_tracing(bfi_smp_ctx* ctx, int enabled) {
    if (!ctx) return fail(nullptr, BFI_SMP_EINVAL, "ctx is NULL");
    ctx->tracing = enabled != 0;
    return BFI_SMP_OK;
}

int64_t bfi_smp_trace(bfi_smp_ctx* ctx, uint64_t* out, int64_t max_words) {
    if (!ctx || !out || max_words < 0) return -1;
    DeviceGuard g(ctx->device);
    size_t n = ctx->trace_used < (size_t)max_words ? ctx->trace_used : (size_t)max_words;
    if (n && hipMemcpy(out, ctx->trace, n * 8, hipMemcpyDeviceToHost) != hipSuccess) return -1;
    return (int64_t)n;
}

int bfi_smp_set_profiling(bfi_smp_ctx* ctx, int enabled) {
    if (!ctx) return fail(nullptr, BFI_SMP_EINVAL, "ctx is NULL");
    ctx->profiling = enabled != 0;  // the record persists until bfi_smp_profile reads it
    return BFI_SMP_OK;
}

int bfi_smp_profile(bfi_smp_ctx* ctx, double* kernel_ms, int64_t* launches) {
    if (!ctx || !kernel_ms || !launches) return fail(ctx, BFI_SMP_EINVAL, "NULL argument");
    DeviceGuard g(ctx->device);
    double acc[4] = {0.0, 0.0, 0.0, 0.0};
    const size_t n = ctx->ev_used / EV_PER_LAUNCH;
    for (size_t i = 0; i < n; i++) {
        hipEvent_t* e = &ctx->ev_pool[EV_PER_LAUNCH * i];
        hipError_t r = hipEventSynchronize(e[5]);
        if (r != hipSuccess) return hip_fail(ctx, r, "hipEventSynchronize");
        const int pairs[4][2] = {{0, 1}, {2, 3}, {4, 5}, {0, 5}};
        for (int k = 0; k < 4; k++) {
            float t = 0.0f;
            if ((r = hipEventElapsedTime(&t, e[pairs[k][0]], e[pairs[k][1]])) != hipSuccess)
                return hip_fail(ctx, r, "hipEventElapsedTime");
            acc[k] += t;
        }
    }
    for (int k = 0; k < 4; k++) kernel_ms[k] = acc[k];
    *launches = (int64_t)n;
    ctx->ev_used = 0;
    return BFI_SMP_OK;
}

const char* bfi_smp_last_error(const bfi_smp_ctx* ctx) {
    return ctx ? ctx->err.c_str() : g_err.c_str();
}

int bfi_smp_sample_rows(bfi_smp_ctx* ctx, const void* d_logits, int dtype, int64_t n_rows, int64_t n_vocab,
                        int64_t row_stride, const bfi_smp_row_params* d_params, const uint32_t* d_hist,
                        const int64_t* d_hist_off, const uint32_t* d_mask, int64_t mask_stride, const float* d_u,
                        uint32_t* d_out, void* stream) {
    if (!ctx) return fail(nullptr, BFI_SMP_EINVAL, "ctx is NULL");
    Call c{};
    c.logits = d_logits;
    c.dtype = dtype;
    c.n_rows = n_rows;
    c.V = n_vocab;
    c.row_stride = row_stride;
    c.params = d_params;
    c.hist = d_hist;
    c.hist_off = d_hist_off;
    c.mask = d_mask;
    c.mask_stride = mask_stride;
    c.u = d_u;
    c.out = d_out;
    return run(ctx, c, (hipStream_t)stream);
}

int bfi_smp_sample_rows_noalloc(bfi_smp_ctx* ctx, const void* d_logits, int dtype, int64_t n_rows, int64_t n_vocab,
                                int64_t row_stride, const bfi_smp_row_params* d_params, const uint32_t* d_hist,
                                const int64_t* d_hist_off, const uint32_t* d_mask, int64_t mask_stride,
                                const float* d_u, uint32_t* d_out, void* stream) {
    if (!ctx) return fail(nullptr, BFI_SMP_EINVAL, "ctx is NULL");
    void* ptr = scratch_ptr(ctx->device);
    if (!ptr) return fail(ctx, BFI_SMP_EHIP, "the fixed workspace of device %d is not set up", ctx->device);
    Call c{};
    c.logits = d_logits;
    c.dtype = dtype;
    c.n_rows = n_rows;
    c.V = n_vocab;
    c.row_stride = row_stride;
    c.params = d_params;
    c.hist = d_hist;
    c.hist_off = d_hist_off;
    c.mask = d_mask;
    c.mask_stride = mask_stride;
    c.u = d_u;
    c.out = d_out;
    const Fixed f{(char*)ptr, (size_t)BFI_SMP_NOALLOC_BYTES};
    return run(ctx, c, (hipStream_t)stream, &f);
}

int bfi_smp_target_rows(bfi_smp_ctx* ctx, const void* d_logits, int dtype, int64_t n_rows, int64_t n_vocab,
                        int64_t row_stride, const bfi_smp_row_params* d_params, const uint32_t* d_hist,
                        const int64_t* d_hist_off, const uint32_t* d_mask, int64_t mask_stride, const float* d_u,
                        uint32_t* d_token, int32_t* d_kind, int32_t* d_kept_len, int32_t* d_listed,
                        uint32_t* d_ids, float* d_probs, int64_t cap, float* d_stats, void* stream) {
    if (!ctx) return fail(nullptr, BFI_SMP_EINVAL, "ctx is NULL");
    if (!d_kind) return fail(ctx, BFI_SMP_EINVAL, "kind is NULL");
    Call c{};
    c.logits = d_logits;
    c.dtype = dtype;
    c.n_rows = n_rows;
    c.V = n_vocab;
    c.row_stride = row_stride;
    c.params = d_params;
    c.hist = d_hist;
    c.hist_off = d_hist_off;
    c.mask = d_mask;
    c.mask_stride = mask_stride;
    c.u = d_u;
    c.out = d_token;
    c.kind = d_kind;
    c.kept = d_kept_len;
    c.listed = d_listed;
    c.ids = d_ids;
    c.probs = d_probs;
    c.cap = cap;
    c.stats = d_stats;
    return run(ctx, c, (hipStream_t)stream);
}

int bfi_smp_verify(bfi_smp_ctx* ctx, const void* d_logits, int dtype, int64_t n_seq, int64_t rows_per_seq,
                   int64_t n_vocab, int64_t row_stride, const bfi_smp_row_params* d_params, const uint32_t* d_hist,
                   const int64_t* d_hist_off, const uint32_t* d_drafts, const int32_t* d_draft_len,
                   const uint32_t* d_mask, int64_t mask_stride, const float* d_u_pairs, const float* d_u_bonus,
                   int32_t* d_out_accepted, uint32_t* d_out_next, void* stream) {
    if (!ctx) return fail(nullptr, BFI_SMP_EINVAL, "ctx is NULL");
    if (rows_per_seq < 1) return fail(ctx, BFI_SMP_EINVAL, "rows_per_seq must be >= 1");
    if (n_seq < 0) return fail(ctx, BFI_SMP_EINVAL, "n_seq < 0");
    Call c{};
    c.logits = d_logits;
    c.dtype = dtype;
    c.n_rows = n_seq * rows_per_seq;
    c.V = n_vocab;
    c.row_stride = row_stride;
    c.params = d_params;
    c.hist = d_hist;
    c.hist_off = d_hist_off;
    c.mask = d_mask;
    c.mask_stride = mask_stride;
    c.rows_per_seq = rows_per_seq;
    c.n_seq = n_seq;
    c.drafts = d_drafts;
    c.draft_len = d_draft_len;
    c.u_pairs = d_u_pairs;
    c.u_bonus = d_u_bonus;
    c.out_acc = d_out_accepted;
    c.out_next = d_out_next;
    return run(ctx, c, (hipStream_t)stream);
}

namespace {

// The output head into `out` (n_tok x n_out f32), the normalized rows in the context's head
// workspace (whose first `lead` bytes the caller may use too).
int run_head(bfi_smp_ctx* ctx, const float* x, const float* norm_w, int norm_per_row, float eps, const float* W,
             int64_t n_tok, int64_t d, int64_t n_out, float* out, size_t lead, hipStream_t stream, int blocked = 0) {
    if (!x || !norm_w || !W) return fail(ctx, BFI_SMP_EINVAL, "x, norm_w or W is NULL");
    if (n_tok < 0 || d <= 0 || n_out <= 0 || n_tok > (1 << 20) || n_out > ((int64_t)1 << 31) / 64)
        return fail(ctx, BFI_SMP_EINVAL, "head sizes out of range (n_tok %lld, d %lld, n_out %lld)", (long long)n_tok,
                    (long long)d, (long long)n_out);
    DeviceGuard g(ctx->device);
    if (g.err != hipSuccess) return hip_fail(ctx, g.err, "hipSetDevice");
    const size_t need = align_up(lead, 256) + (size_t)n_tok * (size_t)d * sizeof(float);
    if (need > ctx->head_size) {
        if (ctx->head) (void)hipFree(ctx->head);
        ctx->head = nullptr;
        ctx->head_size = 0;
        if (hipMalloc((void**)&ctx->head, need) != hipSuccess) {
            ctx->head = nullptr;
            return fail(ctx, BFI_SMP_ENOMEM, "head workspace allocation failed (%zu bytes)", need);
        }
        ctx->head_size = need;
    }
    float* xn = (float*)(ctx->head + align_up(lead, 256));
    if (!out) out = (float*)ctx->head;
    const int vec = (d % 4 == 0) && ((uintptr_t)W % 16 == 0);
    const hipError_t e = bfi::launch_head(x, norm_w, norm_per_row, eps, W, n_tok, d, n_out, vec, blocked, xn, out, stream);
    return e == hipSuccess ? BFI_SMP_OK : hip_fail(ctx, e, "head launch");
}

// Weights a block of each GGML type this head takes holds (0: a type it does not take).
int64_t ggml_block_elems(int32_t type) {
    switch (type) {
        case 0: case 1: case 30: return 1;  // F32, F16, BF16
        case 2: case 8: return 32;           // Q4_0, Q8_0
        case 12: case 13: case 14: return 256;  // Q4_K, Q5_K, Q6_K
        case 41: case 142: case 143: return 128;  // Q1_0, PQ2_0, PTQ1_0
        default: return 0;
    }
}

// The head's dot order for a type (cpu.rs:515-563): a format with a fused block dot sums by
// blocks when the row is whole blocks (1: 32-weight blocks, 2: 128-weight blocks, 3: Q1_0's
// signed blocks); every other type, and a row of partial blocks, is one dot over the row (0).
int head_mode(int32_t type, int64_t n_embd) {
    if ((type == 8 || type == 2) && n_embd % 32 == 0) return 1;
    if ((type == 142 || type == 143) && n_embd % 128 == 0) return 2;
    if (type == 41 && n_embd % 128 == 0) return 3;
    return 0;
}

}  // namespace

int bfi_smp_dequant(bfi_smp_ctx* ctx, int32_t ggml_type, const void* d_src, int64_t n_weights, float* d_dst,
                    void* stream) {
    if (!ctx) return fail(nullptr, BFI_SMP_EINVAL, "ctx is NULL");
    const int64_t be = ggml_block_elems(ggml_type);
    if (be == 0 || ggml_type == 0)
        return fail(ctx, BFI_SMP_EINVAL, "GGML type %d is not one this head dequantizes", (int)ggml_type);
    if (n_weights < 0 || n_weights % be != 0)
        return fail(ctx, BFI_SMP_EINVAL, "%lld weights is not a whole number of %lld-weight blocks",
                    (long long)n_weights, (long long)be);
    if (n_weights > 0 && (!d_src || !d_dst)) return fail(ctx, BFI_SMP_EINVAL, "d_src or d_dst is NULL");
    DeviceGuard g(ctx->device);
    if (g.err != hipSuccess) return hip_fail(ctx, g.err, "hipSetDevice");
    const hipError_t e = bfi::launch_dequant(ggml_type, d_src, n_weights, d_dst, (hipStream_t)stream);
    return e == hipSuccess ? BFI_SMP_OK : hip_fail(ctx, e, "dequant launch");
}

int bfi_smp_head_typed(bfi_smp_ctx* ctx, const float* d_x, const float* d_norm_w, int norm_per_row, float eps,
                       const float* d_w, int32_t ggml_type, int64_t n_tokens, int64_t n_embd, int64_t n_vocab,
                       float* d_logits, void* stream) {
    if (!ctx) return fail(nullptr, BFI_SMP_EINVAL, "ctx is NULL");
    if (!d_logits) return fail(ctx, BFI_SMP_EINVAL, "d_logits is NULL");
    if (ggml_block_elems(ggml_type) == 0)
        return fail(ctx, BFI_SMP_EINVAL, "GGML type %d is not one this head takes", (int)ggml_type);
    const int blocked = head_mode(ggml_type, n_embd);
    return run_head(ctx, d_x, d_norm_w, norm_per_row, eps, d_w, n_tokens, n_embd, n_vocab, d_logits, 0,
                    (hipStream_t)stream, blocked);
}

int bfi_smp_head(bfi_smp_ctx* ctx, const float* d_x, const float* d_norm_w, int norm_per_row, float eps,
                 const float* d_w, int64_t n_tokens, int64_t n_embd, int64_t n_vocab, float* d_logits, void* stream) {
    if (!ctx) return fail(nullptr, BFI_SMP_EINVAL, "ctx is NULL");
    if (!d_logits) return fail(ctx, BFI_SMP_EINVAL, "d_logits is NULL");
    return run_head(ctx, d_x, d_norm_w, norm_per_row, eps, d_w, n_tokens, n_embd, n_vocab, d_logits, 0,
                    (hipStream_t)stream);
}

int bfi_smp_head_sample_rows(bfi_smp_ctx* ctx, const float* d_x, const float* d_norm_w, int norm_per_row, float eps,
                             const float* d_w, int64_t n_tokens, int64_t n_embd, int64_t n_vocab,
                             const bfi_smp_row_params* d_params, const uint32_t* d_hist, const int64_t* d_hist_off,
                             const uint32_t* d_mask, int64_t mask_stride, const float* d_u, uint32_t* d_out,
                             void* stream) {
    return bfi_smp_head_typed_sample_rows(ctx, d_x, d_norm_w, norm_per_row, eps, d_w, 0, n_tokens, n_embd, n_vocab,
                                          d_params, d_hist, d_hist_off, d_mask, mask_stride, d_u, d_out, stream);
}

int bfi_smp_head_typed_sample_rows(bfi_smp_ctx* ctx, const float* d_x, const float* d_norm_w, int norm_per_row,
                                   float eps, const float* d_w, int32_t ggml_type, int64_t n_tokens, int64_t n_embd,
                                   int64_t n_vocab, const bfi_smp_row_params* d_params, const uint32_t* d_hist,
                                   const int64_t* d_hist_off, const uint32_t* d_mask, int64_t mask_stride,
                                   const float* d_u, uint32_t* d_out, void* stream) {
    if (!ctx) return fail(nullptr, BFI_SMP_EINVAL, "ctx is NULL");
    if (ggml_block_elems(ggml_type) == 0)
        return fail(ctx, BFI_SMP_EINVAL, "GGML type %d is not one this head takes", (int)ggml_type);
    const int blocked = head_mode(ggml_type, n_embd);
    const size_t lbytes = (size_t)(n_tokens > 0 ? n_tokens : 0) * (size_t)(n_vocab > 0 ? n_vocab : 0) * sizeof(float);
    int rc = run_head(ctx, d_x, d_norm_w, norm_per_row, eps, d_w, n_tokens, n_embd, n_vocab, nullptr, lbytes,
                      (hipStream_t)stream, blocked);
    if (rc != BFI_SMP_OK) return rc;
    return bfi_smp_sample_rows(ctx, ctx->head, BFI_SMP_F32, n_tokens, n_vocab, n_vocab, d_params, d_hist, d_hist_off,
                               d_mask, mask_stride, d_u, d_out, stream);
}

int bfi_smp_sample_host(bfi_smp_ctx* ctx, const float* logits, int64_t n_vocab, const uint32_t* prev,
                        int64_t n_prev, const bfi_smp_row_params* params, const uint32_t* allow_mask, float u,
                        uint32_t* out_token) {
    if (!ctx) return fail(nullptr, BFI_SMP_EINVAL, "ctx is NULL");
    if (!out_token || !params) return fail(ctx, BFI_SMP_EINVAL, "out_token or params is NULL");
    if (n_vocab < 0 || n_prev < 0) return fail(ctx, BFI_SMP_EINVAL, "negative size");
    if (n_vocab == 0) {  // sample.rs:327-329
        *out_token = 0;
        return BFI_SMP_OK;
    }
    if (!logits) return fail(ctx, BFI_SMP_EINVAL, "logits is NULL");
    if (n_prev > 0 && !prev) return fail(ctx, BFI_SMP_EINVAL, "prev is NULL");
    DeviceGuard g(ctx->device);
    if (g.err != hipSuccess) return hip_fail(ctx, g.err, "hipSetDevice");
    const int64_t mw = (n_vocab + 31) / 32;
    size_t off = 0;
    const size_t o_log = off;
    off = align_up(off + (size_t)n_vocab * 4, 256);
    const size_t o_hist = off;
    off = align_up(off + (size_t)(n_prev ? n_prev : 1) * 4, 256);
    const size_t o_off = off;
    off = align_up(off + 2 * 8, 256);
    const size_t o_mask = off;
    off = align_up(off + (size_t)mw * 4, 256);
    const size_t o_par = off;
    off = align_up(off + sizeof(bfi_smp_row_params), 256);
    const size_t o_u = off;
    off = align_up(off + 4, 256);
    const size_t o_out = off;
    off = align_up(off + 4, 256);
    if (off > ctx->stage_size) {
        if (ctx->stage) (void)hipFree(ctx->stage);
        ctx->stage = nullptr;
        ctx->stage_size = 0;
        if (hipMalloc((void**)&ctx->stage, off) != hipSuccess) {
            ctx->stage = nullptr;
            return fail(ctx, BFI_SMP_ENOMEM, "staging allocation failed");
        }
        ctx->stage_size = off;
    }
    char* d = ctx->stage;
    int64_t hoff[2] = {0, n_prev};
    hipError_t e;
    if ((e = hipMemcpy(d + o_log, logits, (size_t)n_vocab * 4, hipMemcpyHostToDevice)) != hipSuccess ||
        (n_prev && (e = hipMemcpy(d + o_hist, prev, (size_t)n_prev * 4, hipMemcpyHostToDevice)) != hipSuccess) ||
        (e = hipMemcpy(d + o_off, hoff, sizeof hoff, hipMemcpyHostToDevice)) != hipSuccess ||
        (allow_mask && (e = hipMemcpy(d + o_mask, allow_mask, (size_t)mw * 4, hipMemcpyHostToDevice)) != hipSuccess) ||
        (e = hipMemcpy(d + o_par, params, sizeof *params, hipMemcpyHostToDevice)) != hipSuccess ||
        (e = hipMemcpy(d + o_u, &u, 4, hipMemcpyHostToDevice)) != hipSuccess)
        return hip_fail(ctx, e, "hipMemcpy to device");
    Call c{};
    c.logits = d + o_log;
    c.dtype = BFI_SMP_F32;
    c.n_rows = 1;
    c.V = n_vocab;
    c.row_stride = n_vocab;
    c.params = (const bfi_smp_row_params*)(d + o_par);
    c.hist = (const uint32_t*)(d + o_hist);
    c.hist_off = (const int64_t*)(d + o_off);
    c.mask = allow_mask ? (const uint32_t*)(d + o_mask) : nullptr;
    c.mask_stride = mw;
    c.u = (const float*)(d + o_u);
    c.out = (uint32_t*)(d + o_out);
    int rc = run(ctx, c, nullptr);
    if (rc) return rc;
    if ((e = hipMemcpy(out_token, d + o_out, 4, hipMemcpyDeviceToHost)) != hipSuccess)
        return hip_fail(ctx, e, "hipMemcpy to host");
    return BFI_SMP_OK;
}

}  // extern "C"
