// Small device helpers shared by the kernels: wave64 lane ranks and index
// loads whose element type (int32 or int64) is known only at run time.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace ekv {

// Number of set bits of `mask` below the calling lane (wave64).
__device__ __forceinline__ uint32_t lanes_below(uint64_t mask) {
    return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                     __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0u));
}

// Element `offset` of an int32 (is64 = 0) or int64 array, widened to int64,
// without a branch on the element type: the low word and the high word (for
// an int32 array the element itself again, replaced by its sign). With a
// branch per element the compiler waits for each load before the next one is
// issued, so a batch of index loads would not be in flight together.
__device__ __forceinline__ int64_t load_index(const void* base, int32_t is64, int64_t offset) {
    const char* at = static_cast<const char*>(base) + offset * (is64 ? 8 : 4);
    const int32_t lo = *reinterpret_cast<const int32_t*>(at);
    const int32_t high = *reinterpret_cast<const int32_t*>(at + (is64 ? 4 : 0));
    return static_cast<int64_t>((static_cast<uint64_t>(static_cast<uint32_t>(is64 ? high : lo >> 31)) << 32) |
                                static_cast<uint32_t>(lo));
}

}  // namespace ekv
