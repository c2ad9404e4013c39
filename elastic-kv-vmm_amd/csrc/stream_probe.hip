// Streaming bandwidth probes (gfx950): read-only, write-only and copy
// kernels over dense device buffers. They give the on-box ceilings that the
// row-copy engine and the lookup are judged against, measured with the same
// access style: 16-byte lanes, kUnroll independent loads in flight per lane
// before any store, non-temporal stores, one tile per workgroup, tiles dealt
// to the 8 XCDs in contiguous ranges, and an optional LDS reservation that
// caps the workgroups resident per CU. Variants the ceiling is also taken
// over: non-temporal loads, and 16 KiB tiles (4 loads per lane) instead of
// 32 KiB (8).
#include "../../include/ekv_kernels.h"
#include "ekv_common.h"
#include "ekv_vec.h"

#include <algorithm>
#include <type_traits>

namespace ekv {
namespace {

constexpr int kThreads = 256;
constexpr uint32_t kXcds = 8;
constexpr size_t kLdsPerCu = 160 * 1024;

// Tile of workgroup b: XCD b % 8 takes tiles [x * per_xcd, (x + 1) * per_xcd).
__device__ __forceinline__ uint64_t tile_of(uint32_t per_xcd) {
    return uint64_t{blockIdx.x % kXcds} * per_xcd + blockIdx.x / kXcds;
}

// kUnroll 16-byte words per lane: a tile is kThreads * kUnroll words (8: 32 KiB, 4: 16 KiB).
template <int kMode, int kUnroll, bool kNtLoad>
__global__ __launch_bounds__(kThreads) void stream_kernel(const u32x4* __restrict__ src, u32x4* __restrict__ dst,
                                                          uint64_t words, uint32_t per_xcd) {
    extern __shared__ unsigned char reserve[];   // sized by the host to cap workgroups per CU; unused
    constexpr uint64_t kTileWords = uint64_t{kThreads} * kUnroll;
    const uint64_t first = tile_of(per_xcd) * kTileWords + threadIdx.x;
    if (kMode == EKV_PROBE_WRITE) {
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const uint64_t i = first + static_cast<uint64_t>(u) * kThreads;
            if (i < words) {
                __builtin_nontemporal_store(u32x4{0u, 0u, 0u, 0u}, dst + i);
            }
        }
        return;
    }
    u32x4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const uint64_t i = first + static_cast<uint64_t>(u) * kThreads;
        const u32x4* at = src + (i < words ? i : words - 1);
        if constexpr (kNtLoad) {
            v[u] = __builtin_nontemporal_load(at);
        } else {
            v[u] = *at;
        }
    }
    if (kMode == EKV_PROBE_COPY) {
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const uint64_t i = first + static_cast<uint64_t>(u) * kThreads;
            if (i < words) {
                __builtin_nontemporal_store(v[u], dst + i);
            }
        }
    } else {
        // Read only: fold the words and store only when the fold hits a value
        // the host never plants, so the loads cannot be dropped.
        u32x4 acc = v[0];
#pragma unroll
        for (int u = 1; u < kUnroll; ++u) {
            acc ^= v[u];
        }
        if (acc.x == 0x9e3779b9u && acc.y == 0x7f4a7c15u && acc.z == 0x85ebca6bu && acc.w == 0xc2b2ae35u) {
            dst[blockIdx.x] = acc;
        }
    }
}

int stream_probe(int mode_flags, const void* src, void* dst, uint64_t bytes, int per_cu, void* stream) {
    const int mode = mode_flags & 0xf;
    const int flags = mode_flags & ~0xf;
    if (mode != EKV_PROBE_READ && mode != EKV_PROBE_WRITE && mode != EKV_PROBE_COPY) {
        throw std::invalid_argument("mode must be EKV_PROBE_READ, EKV_PROBE_WRITE or EKV_PROBE_COPY");
    }
    if ((flags & ~(EKV_PROBE_NT_LOAD | EKV_PROBE_HALF_TILE)) != 0) {
        throw std::invalid_argument("unknown stream probe flags");
    }
    if (bytes % 16 != 0 || (reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) % 16 != 0) {
        throw std::invalid_argument("buffers must be 16-byte aligned and a multiple of 16 bytes long");
    }
    if (per_cu < 0 || per_cu > 32) {
        throw std::invalid_argument("workgroups_per_cu must be 0 (no cap) .. 32");
    }
    const uint64_t words = bytes / 16;
    if (words == 0) {
        return 0;
    }
    if ((mode != EKV_PROBE_WRITE && src == nullptr) || dst == nullptr) {
        throw std::invalid_argument("null buffer");
    }
    const bool half = (flags & EKV_PROBE_HALF_TILE) != 0;
    const bool nt_load = (flags & EKV_PROBE_NT_LOAD) != 0;
    const uint64_t tile_words = uint64_t{kThreads} * (half ? 4 : 8);
    const uint64_t tiles = (words + tile_words - 1) / tile_words;
    const uint64_t per_xcd = (tiles + kXcds - 1) / kXcds;
    if (per_xcd * kXcds > 0xffffffffull) {
        throw std::invalid_argument("buffer too large for one launch");
    }
    // The read probe may write one 16-byte word per workgroup into dst.
    if (mode == EKV_PROBE_READ && bytes < per_xcd * kXcds * 16) {
        throw std::invalid_argument("the read probe needs dst of at least 16 bytes per tile of src");
    }
    const size_t lds = per_cu > 0 ? (kLdsPerCu / static_cast<size_t>(per_cu)) & ~size_t{1023} : 0;
    const dim3 grid(static_cast<uint32_t>(per_xcd * kXcds));
    const auto s = static_cast<hipStream_t>(stream);
    const auto* in = static_cast<const u32x4*>(src);
    auto* out = static_cast<u32x4*>(dst);
    const auto launch = [&](auto kernel) {
        if (lds > 64 * 1024) {
            check_hip(hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)),
                      "raise the probe LDS limit");
        }
        kernel<<<grid, dim3(kThreads), lds, s>>>(in, out, words, static_cast<uint32_t>(per_xcd));
    };
    const auto by_load = [&](auto unroll) {
        constexpr int kU = decltype(unroll)::value;
        if (mode == EKV_PROBE_WRITE) {
            launch(stream_kernel<EKV_PROBE_WRITE, kU, false>);
        } else if (mode == EKV_PROBE_READ) {
            nt_load ? launch(stream_kernel<EKV_PROBE_READ, kU, true>) : launch(stream_kernel<EKV_PROBE_READ, kU, false>);
        } else {
            nt_load ? launch(stream_kernel<EKV_PROBE_COPY, kU, true>) : launch(stream_kernel<EKV_PROBE_COPY, kU, false>);
        }
    };
    if (half) {
        by_load(std::integral_constant<int, 4>{});
    } else {
        by_load(std::integral_constant<int, 8>{});
    }
    check_hip(hipGetLastError(), "launch stream probe");
    return 0;
}

}  // namespace
}  // namespace ekv

extern "C" int ekv_stream_probe(int mode, const void* src, void* dst, uint64_t bytes, int workgroups_per_cu,
                                void* stream) {
    return ekv::guarded(-1, [&] { return ekv::stream_probe(mode, src, dst, bytes, workgroups_per_cu, stream); });
}
