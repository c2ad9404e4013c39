// Host-side validation of ekv_tensor descriptors and small device helpers for
// reading int32/int64 index tensors whose dtype is known only at run time.
#pragma once

#include "../../include/ekv_kernels.h"
#include "ekv_common.h"

#include <string>

namespace ekv {

inline int64_t itemsize(int32_t dtype) {
    switch (dtype) {
        case EKV_INT32: return 4;
        case EKV_INT64: return 8;
        case EKV_UINT8: return 1;
        case EKV_INT8: return 1;
        case EKV_INT16: return 2;
        case EKV_BFLOAT16: return 2;
        case EKV_FLOAT16: return 2;
        case EKV_FLOAT32: return 4;
        default: throw std::invalid_argument("unknown dtype code " + std::to_string(dtype));
    }
}

inline const ekv_tensor& need(const ekv_tensor* t, const char* name) {
    if (t == nullptr) {
        throw std::invalid_argument(std::string(name) + " is required");
    }
    if (t->ndim < 0 || t->ndim > 4) {
        throw std::invalid_argument(std::string(name) + " must have 0..4 dimensions");
    }
    for (int i = 0; i < t->ndim; ++i) {
        if (t->shape[i] < 0) {
            throw std::invalid_argument(std::string(name) + " has a negative extent");
        }
    }
    (void)itemsize(t->dtype);
    return *t;
}

inline int64_t numel(const ekv_tensor& t) {
    int64_t n = 1;
    for (int i = 0; i < t.ndim; ++i) {
        n *= t.shape[i];
    }
    return n;
}

inline void need_ndim(const ekv_tensor& t, int ndim, const char* name) {
    if (t.ndim != ndim) {
        throw std::invalid_argument(std::string(name) + " must have " + std::to_string(ndim) +
                                    " dimensions, got " + std::to_string(t.ndim));
    }
}

inline void need_index(const ekv_tensor& t, const char* name) {
    if (t.dtype != EKV_INT32 && t.dtype != EKV_INT64) {
        throw std::invalid_argument(std::string(name) + " must be int32 or int64");
    }
}

inline void need_dim(const ekv_tensor& t, int dim, int64_t extent, const char* name) {
    if (t.shape[dim] != extent) {
        throw std::invalid_argument(std::string(name) + " dimension " + std::to_string(dim) + " is " +
                                    std::to_string(t.shape[dim]) + ", expected " + std::to_string(extent));
    }
}

inline void need_data(const ekv_tensor& t, const char* name) {
    if (numel(t) > 0 && t.data == nullptr) {
        throw std::invalid_argument(std::string(name) + " has a null data pointer");
    }
}

// An int32/int64 index array read through one stride, dtype chosen at run time.
struct IndexRef {
    const void* data = nullptr;
    int64_t stride = 0;
    int32_t is64 = 0;

#if defined(__HIPCC__)
    __device__ __forceinline__ int64_t operator[](int64_t i) const {
        return is64 ? static_cast<const int64_t*>(data)[i * stride]
                    : static_cast<int64_t>(static_cast<const int32_t*>(data)[i * stride]);
    }

    // The same value without a branch on the element type: the low word and
    // the high word (for int32 arrays the element itself again, then replaced
    // by its sign) are read from in-bounds addresses chosen by selects. For
    // workgroup-uniform reads in a kernel's prologue, where a branch per index
    // load would keep consecutive loads from being in flight together.
    __device__ __forceinline__ int64_t fetch(int64_t i) const {
        const char* at = static_cast<const char*>(data) + i * stride * (is64 ? 8 : 4);
        const int32_t lo = *reinterpret_cast<const int32_t*>(at);
        const int32_t high = *reinterpret_cast<const int32_t*>(at + (is64 ? 4 : 0));
        const int32_t hi = is64 ? high : (lo >> 31);
        return static_cast<int64_t>((static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) |
                                    static_cast<uint32_t>(lo));
    }

    // The element's low 32 bits (its value truncated to int32), one load and
    // no branch: for batches of independent loads that must all be in flight
    // before any is waited for.
    __device__ __forceinline__ int32_t low(int64_t i) const {
        return *reinterpret_cast<const int32_t*>(static_cast<const char*>(data) + i * stride * (is64 ? 8 : 4));
    }
#endif
};

#if defined(__HIPCC__)
// Index reads for a kernel's prologue, as vector loads. The compiler makes a
// workgroup-uniform read a scalar load, and it waits for every outstanding
// scalar load before the first use of any of them, so a prologue's
// independent index reads (and the kernel-argument reloads between them)
// become a chain of memory round trips. Vector loads complete in issue order:
// a batch of them is waited for once, and scalar waits do not wait for them.
// An opaque per-lane zero in the address keeps them vector loads; index_value
// reads a uniform value back as a scalar, lane_value a per-lane one.
struct PendingIndex {
    int32_t lo, hi;
};

__device__ __forceinline__ uint32_t opaque_zero() {
    uint32_t zero;
    asm volatile("v_mov_b32 %0, 0" : "=v"(zero));
    return zero;
}

// Element i of `r`: its low word and, for int64 arrays, its high word (for
// int32 arrays the element again); no branch on the element type.
__device__ __forceinline__ PendingIndex issue_index(const IndexRef& r, int64_t i, uint32_t zero) {
    const char* at = static_cast<const char*>(r.data) + i * r.stride * (r.is64 ? 8 : 4) + zero;
    return PendingIndex{*reinterpret_cast<const int32_t*>(at), *reinterpret_cast<const int32_t*>(at + (r.is64 ? 4 : 0))};
}

__device__ __forceinline__ int64_t index_value(const IndexRef& r, const PendingIndex& p) {
    // Both words are read back unconditionally: a read under the element-type
    // test let the compiler move the high word's load into that branch and
    // wait there for every load in flight.
    const int32_t lo = __builtin_amdgcn_readfirstlane(p.lo);
    const int32_t high = __builtin_amdgcn_readfirstlane(p.hi);
    const int32_t hi = r.is64 ? high : (lo >> 31);
    return static_cast<int64_t>((static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) | static_cast<uint32_t>(lo));
}

// The same element read by a per-thread load (any value per lane).
__device__ __forceinline__ int64_t lane_value(const IndexRef& r, const PendingIndex& p) {
    const int32_t hi = r.is64 ? p.hi : (p.lo >> 31);
    return static_cast<int64_t>((static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) |
                                static_cast<uint32_t>(p.lo));
}

#endif

inline IndexRef index_ref(const ekv_tensor& t, int dim) {
    IndexRef r;
    r.data = t.data;
    r.stride = t.ndim > dim ? t.stride[dim] : 0;
    r.is64 = t.dtype == EKV_INT64;
    return r;
}

}  // namespace ekv
