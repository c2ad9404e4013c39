// One sparse-KV decode step in one call: resident lookup with miss
// compaction, batch-token LRU swap-in, promotion of the misses from mapped
// pinned host memory, and the Top-K K/V gather - the sequence the
// reference's decode path runs per layer (adaptive_sparse/
// request_residency.py:805-832: lookup, then the host-backed swap, then the
// attention read of the gathered rows).
//
// The four launches are the library's own entry points, queued in order on
// the caller's stream, after one small kernel that zeroes the miss counts
// (the lookup writes the counts of selected rows only, and the move reads
// every row's). Their intermediates - the miss list and counts that the
// lookup hands to the swap-in, and the promotion lists that the swap-in hands
// to the move - live in a workspace the caller brings (layout below); nothing
// is allocated, no stream is synchronized and no memset node is recorded, so
// the step can be captured in a HIP graph.
#include "../../include/ekv_kernels.h"
#include "ekv_common.h"
#include "ekv_tensor_util.h"

#include <algorithm>
#include <mutex>
#include <string>

// The allocation-free form (ekv_decode_step_static) keeps its workspace in
// this file-scope device array: every GPU the library runs on holds one copy
// (32 MiB) until the process ends, and every call on that GPU shares it. In
// host code `scratch` names a host-side stand-in, never the device memory:
// its device address is taken once per device with hipGetSymbolAddress
// (static_address below) and only that address is used.
constexpr uint64_t kStaticWorkspaceBytes = uint64_t{32} << 20;
static __device__ __align__(256) unsigned char scratch[kStaticWorkspaceBytes];

namespace ekv {
namespace {

constexpr uint64_t kAlign = 256;

uint64_t aligned(uint64_t bytes) { return (bytes + kAlign - 1) / kAlign * kAlign; }

// Workspace of a step over L layers x B rows x W lanes: misses, promote_src
// and promote_dst ([L, B, W] int32 each), then counts ([L, B] int32), each
// region 256-byte aligned.
uint64_t step_workspace_bytes(int64_t layers, int64_t batch, int64_t width) {
    if (layers < 0 || batch < 0 || width < 0) {
        throw std::invalid_argument("negative step dimensions");
    }
    const uint64_t lanes = static_cast<uint64_t>(layers) * static_cast<uint64_t>(batch) * static_cast<uint64_t>(width);
    return 3 * aligned(lanes * 4) + aligned(static_cast<uint64_t>(layers) * static_cast<uint64_t>(batch) * 4);
}

ekv_tensor int32_view(void* data, int64_t layers, int64_t batch, int64_t width, int ndim) {
    ekv_tensor t{};
    t.data = data;
    t.dtype = EKV_INT32;
    t.ndim = ndim;
    t.shape[0] = layers;
    t.shape[1] = batch;
    t.shape[2] = width;
    t.stride[2] = 1;
    t.stride[1] = ndim == 3 ? width : 1;
    t.stride[0] = ndim == 3 ? batch * width : batch;
    return t;
}

__global__ __launch_bounds__(256) void zero_words_kernel(int32_t* __restrict__ words, uint64_t count) {
    const uint64_t stride = uint64_t{gridDim.x} * blockDim.x;
    for (uint64_t i = uint64_t{blockIdx.x} * blockDim.x + threadIdx.x; i < count; i += stride) {
        words[i] = 0;
    }
}

void check_step(int status, const char* stage) {
    if (status != 0) {
        throw std::runtime_error(std::string(stage) + ": " + last_error());
    }
}

int decode_step(const ekv_step_args& s, void* workspace, uint64_t workspace_bytes, void* stream) {
    const ekv_tensor& topk = need(s.topk, "topk");
    need_ndim(topk, 3, "topk");
    if (s.block_size < 1) {
        throw std::invalid_argument("block_size must be positive");
    }
    const int64_t layers = topk.shape[0], batch = topk.shape[1], width = topk.shape[2] * s.block_size;
    const uint64_t needed = step_workspace_bytes(layers, batch, width);
    if (workspace_bytes < needed) {
        throw std::invalid_argument("the step needs " + std::to_string(needed) + " workspace bytes, got " +
                                    std::to_string(workspace_bytes));
    }
    if (needed == 0) {
        return 0;
    }
    if (workspace == nullptr || reinterpret_cast<uintptr_t>(workspace) % kAlign != 0) {
        throw std::invalid_argument("the workspace must be a 256-byte aligned device buffer");
    }
    if ((s.step_counter == nullptr) == (s.step < 0)) {
        throw std::invalid_argument("give either a step (>= 0) or a device step counter");
    }
    const uint64_t list = aligned(static_cast<uint64_t>(layers * batch * width) * 4);
    char* base = static_cast<char*>(workspace);
    const ekv_tensor misses = int32_view(base, layers, batch, width, 3);
    const ekv_tensor src = int32_view(base + list, layers, batch, width, 3);
    const ekv_tensor dst = int32_view(base + 2 * list, layers, batch, width, 3);
    const ekv_tensor counts = int32_view(base + 3 * list, layers, batch, 1, 2);
    const ekv_tensor& table = need(s.table, "table");
    // The four stages, queued in order. Every stage is checked first without
    // launching (CheckOnly), so an argument a later stage refuses fails the
    // call before the lookup has written its slots.
    const auto stages = [&] {
        if (table.dtype == EKV_INT16) {
            check_step(ekv_resolve_resident_local(s.topk, s.table, s.slot_base, s.resident_bits, s.bits_shift,
                                                  s.rows, s.lengths, s.selected, s.slots, &misses, &counts,
                                                  s.block_size, stream),
                       "lookup");
        } else if (s.resident_bits != nullptr) {
            check_step(ekv_resolve_resident_bits(s.topk, s.table, s.resident_bits, s.bits_shift, s.rows, s.lengths,
                                                 s.selected, s.slots, &misses, &counts, s.block_size, stream),
                       "lookup");
        } else {
            check_step(ekv_resolve_resident(s.topk, s.table, nullptr, s.rows, s.lengths, s.selected, s.slots,
                                            &misses, &counts, s.block_size, stream),
                       "lookup");
        }
        if (s.step_counter != nullptr) {
            check_step(ekv_swap_in_counted(s.topk, s.block_size, s.rows, s.selected, s.slots, &misses, &counts,
                                           s.table, s.resident_bits, s.bits_shift, s.resident_counts, s.slot_token,
                                           s.stamps, s.slot_base, s.host_table, &src, &dst, s.step_counter,
                                           s.status, stream),
                       "swap-in");
        } else {
            check_step(ekv_swap_in(s.topk, s.block_size, s.rows, s.selected, s.slots, &misses, &counts, s.table,
                                   s.resident_bits, s.bits_shift, s.resident_counts, s.slot_token, s.stamps,
                                   s.slot_base, s.host_table, &src, &dst, s.step, s.status, stream),
                       "swap-in");
        }
        check_step(ekv_move_kv(s.host, &src, s.pool, &dst, &counts, 1, stream), "promote");
        check_step(ekv_gather_kv(s.pool, s.slots, s.out, 1, stream), "gather");
    };
    {
        CheckOnly checking;
        stages();
    }
    const uint64_t rows_total = static_cast<uint64_t>(layers * batch);
    const uint32_t zero_blocks = static_cast<uint32_t>(std::min<uint64_t>((rows_total + 255) / 256, 1024));
    zero_words_kernel<<<dim3(zero_blocks), dim3(256), 0, static_cast<hipStream_t>(stream)>>>(
        static_cast<int32_t*>(counts.data), rows_total);
    check_hip(hipGetLastError(), "launch count reset");
    stages();
    return 0;
}

constexpr int kMaxDevices = 64;

// Device address of the current device's `scratch` (taken on the first call on
// that device, with the device current).
void* static_address() {
    static std::mutex lock;
    static void* address[kMaxDevices] = {};
    int device = -1;
    check_hip(hipGetDevice(&device), "hipGetDevice");
    if (device < 0 || device >= kMaxDevices) {
        throw std::runtime_error("device ordinal " + std::to_string(device) + " out of range");
    }
    std::lock_guard<std::mutex> guard(lock);
    if (address[device] == nullptr) {
        void* found = nullptr;
        check_hip(hipGetSymbolAddress(&found, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
        if (found == nullptr) {
            throw std::runtime_error("hipGetSymbolAddress(scratch) returned no address");
        }
        address[device] = found;
    }
    return address[device];
}

int decode_step_static(const ekv_step_args& s, void* stream) {
    const ekv_tensor& topk = need(s.topk, "topk");
    need_ndim(topk, 3, "topk");
    if (s.block_size < 1) {
        throw std::invalid_argument("block_size must be positive");
    }
    const uint64_t needed = step_workspace_bytes(topk.shape[0], topk.shape[1], topk.shape[2] * s.block_size);
    if (needed > kStaticWorkspaceBytes) {
        throw std::invalid_argument("the step needs " + std::to_string(needed) +
                                    " workspace bytes, more than the static workspace's " +
                                    std::to_string(kStaticWorkspaceBytes) + "; split it over fewer layers or rows");
    }
    return decode_step(s, static_address(), kStaticWorkspaceBytes, stream);
}

}  // namespace
}  // namespace ekv

extern "C" int ekv_decode_step_static(const ekv_step_args* args, void* stream) {
    return ekv::guarded(-1, [&] {
        if (args == nullptr) {
            throw std::invalid_argument("args is required");
        }
        return ekv::decode_step_static(*args, stream);
    });
}

extern "C" uint64_t ekv_decode_step_workspace_bytes(int64_t layers, int64_t batch, int64_t width) {
    return ekv::guarded(~uint64_t{0}, [&] { return ekv::step_workspace_bytes(layers, batch, width); });
}

extern "C" int ekv_decode_step(const ekv_step_args* args, void* workspace, uint64_t workspace_bytes,
                               void* stream) {
    return ekv::guarded(-1, [&] {
        if (args == nullptr) {
            throw std::invalid_argument("args is required");
        }
        return ekv::decode_step(*args, workspace, workspace_bytes, stream);
    });
}
