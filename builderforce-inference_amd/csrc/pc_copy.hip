// pc_copy.hip — the prefix cache's device copies in one launch: a batch of (copy, then zero)
// ranges, each block working on one range, 16-byte loads and stores in flight four at a time
// per thread. A restore (every K/V tensor's kept rows copied back and the rest of its capacity
// zeroed, the recurrent tensors and the logits) or an insert (the kept rows gathered into the
// entry's block) is HBM-bound work: one pass over the bytes, no reuse.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "pc_copy.h"

namespace bfi {

namespace {

constexpr int PC_BLOCK = 256;
constexpr int PC_UNROLL = 4;

struct PcBatch {
    PcRange r[PC_MAX_RANGES];
    uint32_t first_block[PC_MAX_RANGES + 1];  // blocks of range i: [first_block[i], first_block[i + 1])
    int n;
};

__global__ __launch_bounds__(PC_BLOCK) void k_pc_copy(const PcBatch b) {
    // the range of this block (uniform: a scalar search over the kernel arguments)
    int lo = 0, hi = b.n;
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (b.first_block[mid] <= blockIdx.x) lo = mid;
        else hi = mid;
    }
    const PcRange r = b.r[lo];
    const uint64_t nb = b.first_block[lo + 1] - b.first_block[lo];
    const uint64_t units_copy = r.copy_bytes >> 4, units = (r.copy_bytes + r.zero_bytes) >> 4;
    const uint4* src = reinterpret_cast<const uint4*>(r.src);
    uint4* dst = reinterpret_cast<uint4*>(r.dst);
    const uint64_t stride = nb * PC_BLOCK;
    uint64_t u = (blockIdx.x - b.first_block[lo]) * (uint64_t)PC_BLOCK + threadIdx.x;
    for (; u + (PC_UNROLL - 1) * stride < units; u += PC_UNROLL * stride) {
        uint4 v[PC_UNROLL];
#pragma unroll
        for (int k = 0; k < PC_UNROLL; k++) {
            const uint64_t x = u + k * stride;
            v[k] = x < units_copy ? src[x] : make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int k = 0; k < PC_UNROLL; k++) dst[u + k * stride] = v[k];
    }
    for (; u < units; u += stride) dst[u] = u < units_copy ? src[u] : make_uint4(0u, 0u, 0u, 0u);
}

}  // namespace

// Ranges must be 16-byte aligned with sizes in multiples of 16 (pc_ranges_aligned); at most
// PC_MAX_RANGES a launch.
hipError_t pc_copy_launch(const PcRange* ranges, int n, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    PcBatch b{};
    b.n = n;
    uint64_t total = 0;
    for (int i = 0; i < n; i++) total += ranges[i].copy_bytes + ranges[i].zero_bytes;
    // about 2048 blocks over the batch, shared by bytes (at least one per range)
    constexpr uint64_t TARGET = 2048;
    uint32_t blk = 0;
    for (int i = 0; i < n; i++) {
        b.r[i] = ranges[i];
        b.first_block[i] = blk;
        const uint64_t bytes = ranges[i].copy_bytes + ranges[i].zero_bytes;
        uint64_t want = total ? (bytes * TARGET + total - 1) / total : 1;
        const uint64_t most = (bytes / 16 + PC_BLOCK - 1) / PC_BLOCK;  // no block without a unit
        want = want > most ? most : want;
        blk += (uint32_t)(want ? want : 1);
    }
    b.first_block[n] = blk;
    hipLaunchKernelGGL(k_pc_copy, dim3(blk), dim3(PC_BLOCK), 0, stream, b);
    return hipGetLastError();
}

}  // namespace bfi
