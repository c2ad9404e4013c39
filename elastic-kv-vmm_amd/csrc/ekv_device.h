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

// Element `offset` of an int32 (is64 = 0) or int64 array, widened to int64.
__device__ __forceinline__ int64_t load_index(const void* base, int32_t is64, int64_t offset) {
    return is64 ? static_cast<const int64_t*>(base)[offset]
                : static_cast<int64_t>(static_cast<const int32_t*>(base)[offset]);
}

}  // namespace ekv
