// pc_copy.h — batched device copies of the prefix cache (pc_copy.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace bfi {

constexpr int PC_MAX_RANGES = 48;  // ranges a launch takes as kernel arguments

// dst[0, copy_bytes) = src[0, copy_bytes), then dst[copy_bytes, copy_bytes + zero_bytes) = 0.
struct PcRange {
    const void* src;
    void* dst;
    uint64_t copy_bytes;
    uint64_t zero_bytes;
};

inline bool pc_range_aligned(const PcRange& r) {
    return ((uintptr_t)r.src % 16u) == 0 && ((uintptr_t)r.dst % 16u) == 0 && r.copy_bytes % 16u == 0 &&
           r.zero_bytes % 16u == 0;
}

hipError_t pc_copy_launch(const PcRange* ranges, int n, hipStream_t stream);

}  // namespace bfi
