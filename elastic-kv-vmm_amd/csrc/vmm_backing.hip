// Demand-backed virtual KV range on HIP virtual memory management.
//
// Behaviour follows the reference's native/elastic_vmm.cpp (semantics of
// Backing::initialize :50-86, ensure_impl :97-153, drop :166-184, close
// :186-215, normalize :235-256, release :258-274 and the ABI :316-369); the
// implementation is HIP-native:
//   * the reservation is aligned to the chunk size when the chunk size is a
//     power of two, so every 2 MiB chunk can use a 2 MiB GPU page;
//   * access is granted per chunk and new chunks are zero-filled by our own
//     fill kernel over each contiguous run of new chunks, on a private
//     non-blocking stream (a kernel does not care that a run spans several
//     physical allocations);
//   * a failed close keeps the object alive so the close can be retried.
#include "../../include/elastic_vmm.h"
#include "ekv_common.h"

#include <algorithm>
#include <limits>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace ekv {

std::string& last_error() {
    thread_local std::string message;
    return message;
}

namespace {

// Zero `words` 16-byte words starting at `base` (grid-stride, 16 B per lane).
__global__ __launch_bounds__(256) void zero_fill_kernel(uint4* __restrict__ base, uint64_t words) {
    const uint64_t stride = uint64_t{gridDim.x} * blockDim.x;
    for (uint64_t i = uint64_t{blockIdx.x} * blockDim.x + threadIdx.x; i < words; i += stride) {
        base[i] = make_uint4(0u, 0u, 0u, 0u);
    }
}

struct Chunk {
    hipMemGenericAllocationHandle_t handle{};
    bool created = false;
    bool mapped = false;
};

class VmmBacking {
public:
    VmmBacking(int device, uint64_t capacity_bytes, uint64_t chunk_bytes) : device_(device) {
        if (capacity_bytes == 0 || chunk_bytes == 0) {
            throw std::invalid_argument("capacity and chunk size must be positive");
        }
        if (chunk_bytes % 16 != 0) {
            throw std::invalid_argument("chunk size must be a multiple of 16 bytes");
        }
        const uint64_t chunks = capacity_bytes / chunk_bytes + (capacity_bytes % chunk_bytes != 0);
        if (chunks > std::numeric_limits<uint64_t>::max() / chunk_bytes) {
            throw std::invalid_argument("aligned capacity overflows 64 bits");
        }
        chunk_bytes_ = chunk_bytes;
        reserved_bytes_ = chunks * chunk_bytes;

        int count = 0;
        check_hip(hipGetDeviceCount(&count), "hipGetDeviceCount");
        if (device < 0 || device >= count) {
            throw std::invalid_argument("device ordinal " + std::to_string(device) + " out of range (" +
                                        std::to_string(count) + " devices)");
        }
        DeviceGuard guard(device_);
        int supported = 0;
        check_hip(hipDeviceGetAttribute(&supported, hipDeviceAttributeVirtualMemoryManagementSupported,
                                        device_),
                  "query VMM support");
        if (!supported) {
            throw std::runtime_error("device does not support HIP virtual memory management");
        }
        prop_.type = hipMemAllocationTypePinned;
        prop_.location.type = hipMemLocationTypeDevice;
        prop_.location.id = device_;
        size_t granularity = 0;
        check_hip(hipMemGetAllocationGranularity(&granularity, &prop_, hipMemAllocationGranularityMinimum),
                  "hipMemGetAllocationGranularity");
        granularity_ = granularity;
        if (granularity_ == 0 || chunk_bytes_ % granularity_ != 0) {
            throw std::invalid_argument("chunk_bytes must be a multiple of VMM granularity " +
                                        std::to_string(granularity_));
        }
        const bool power_of_two = (chunk_bytes_ & (chunk_bytes_ - 1)) == 0;
        const size_t alignment = power_of_two ? static_cast<size_t>(chunk_bytes_) : granularity_;
        void* base = nullptr;
        check_hip(hipMemAddressReserve(&base, reserved_bytes_, alignment, nullptr, 0), "hipMemAddressReserve");
        base_ = reinterpret_cast<uintptr_t>(base);
        const hipError_t stream_status = hipStreamCreateWithFlags(&zero_stream_, hipStreamNonBlocking);
        if (stream_status != hipSuccess) {
            (void)hipMemAddressFree(base, reserved_bytes_);
            base_ = 0;
            fail_hip(stream_status, "hipStreamCreateWithFlags");
        }
        open_ = true;
    }

    ~VmmBacking() { (void)close(); }

    VmmBacking(const VmmBacking&) = delete;
    VmmBacking& operator=(const VmmBacking&) = delete;

    // ensure (wait = true) and precommit (wait = false).
    void commit(const uint64_t* ids, size_t count, bool wait) {
        const std::vector<uint64_t> fresh = pending(ids, count, /*want_mapped=*/false);
        DeviceGuard guard(device_);
        if (fresh.empty()) {
            if (wait) {
                wait_for_zero();
            }
            return;
        }
        size_t touched = 0;  // chunks of this batch that may own resources
        try {
            for (const uint64_t id : fresh) {
                Chunk& chunk = chunks_[id];
                ++touched;
                check_hip(hipMemCreate(&chunk.handle, chunk_bytes_, &prop_, 0), "hipMemCreate");
                chunk.created = true;
                check_hip(hipMemMap(address(id), chunk_bytes_, 0, chunk.handle, 0), "hipMemMap");
                chunk.mapped = true;
                hipMemAccessDesc access{};
                access.location = prop_.location;
                access.flags = hipMemAccessFlagsProtReadWrite;
                check_hip(hipMemSetAccess(address(id), chunk_bytes_, &access, 1), "hipMemSetAccess");
            }
            // Zero each contiguous run of new chunks with one fill launch.
            for (size_t begin = 0; begin < fresh.size();) {
                size_t end = begin + 1;
                while (end < fresh.size() && fresh[end] == fresh[end - 1] + 1) {
                    ++end;
                }
                const uint64_t words = (end - begin) * chunk_bytes_ / 16;
                const uint64_t blocks = std::min<uint64_t>((words + 255) / 256, 65536);
                zero_fill_kernel<<<dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, zero_stream_>>>(
                    static_cast<uint4*>(address(fresh[begin])), words);
                check_hip(hipGetLastError(), "launch zero fill");
                zero_pending_ = true;
                begin = end;
            }
            if (wait) {
                wait_for_zero();
            }
        } catch (...) {
            // Never release memory whose zero-fill might still be running.
            if (zero_pending_) {
                if (hipStreamSynchronize(zero_stream_) != hipSuccess) {
                    poisoned_ = true;
                    throw;
                }
                zero_pending_ = false;
            }
            while (touched > 0) {
                const uint64_t id = fresh[--touched];
                auto it = chunks_.find(id);
                if (release(id, it->second) == hipSuccess) {
                    chunks_.erase(it);
                } else {
                    poisoned_ = true;
                }
            }
            throw;
        }
    }

    void decommit(const uint64_t* ids, size_t count) {
        const std::vector<uint64_t> mapped = pending(ids, count, /*want_mapped=*/true);
        if (mapped.empty()) {
            return;
        }
        DeviceGuard guard(device_);
        wait_for_zero();
        for (const uint64_t id : mapped) {
            auto it = chunks_.find(id);
            const hipError_t status = release(id, it->second);
            if (status != hipSuccess) {
                // Earlier chunks of this call are gone already; the caller
                // must tear the object down.
                poisoned_ = true;
                fail_hip(status, "decommit chunk");
            }
            chunks_.erase(it);
        }
    }

    // Releases everything; returns the first failure. Safe to call again.
    hipError_t close() noexcept {
        if (!open_) {
            return hipSuccess;
        }
        hipError_t first = hipSuccess;
        auto record = [&first](hipError_t status) {
            if (first == hipSuccess && status != hipSuccess) {
                first = status;
            }
        };
        int previous = 0;
        record(hipGetDevice(&previous));
        record(hipSetDevice(device_));
        if (first == hipSuccess) {
            record(hipDeviceSynchronize());
        }
        if (first == hipSuccess) {
            zero_pending_ = false;
            for (auto it = chunks_.begin(); it != chunks_.end();) {
                const hipError_t status = release(it->first, it->second);
                record(status);
                it = status == hipSuccess ? chunks_.erase(it) : std::next(it);
            }
            if (chunks_.empty() && base_) {
                const hipError_t status = hipMemAddressFree(reinterpret_cast<void*>(base_), reserved_bytes_);
                record(status);
                if (status == hipSuccess) {
                    base_ = 0;
                }
            }
            if (base_ == 0 && zero_stream_) {
                const hipError_t status = hipStreamDestroy(zero_stream_);
                record(status);
                if (status == hipSuccess) {
                    zero_stream_ = nullptr;
                }
            }
            if (base_ == 0 && zero_stream_ == nullptr) {
                open_ = false;
            }
        }
        (void)hipSetDevice(previous);
        if (first != hipSuccess) {
            poisoned_ = true;
        }
        return first;
    }

    uint64_t base() const { return base_; }
    uint64_t granularity() const { return granularity_; }
    uint64_t reserved() const { return reserved_bytes_; }
    bool poisoned() const { return poisoned_; }

    uint64_t backed() const {
        uint64_t committed = 0;
        for (const auto& entry : chunks_) {
            committed += entry.second.created || entry.second.mapped;
        }
        return committed * chunk_bytes_;
    }

private:
    void* address(uint64_t id) const { return reinterpret_cast<void*>(base_ + id * chunk_bytes_); }

    void wait_for_zero() {
        if (!zero_pending_) {
            return;
        }
        check_hip(hipStreamSynchronize(zero_stream_), "wait for backing initialization");
        zero_pending_ = false;
    }

    // Sorted, de-duplicated ids whose mapped state equals `want_mapped`.
    std::vector<uint64_t> pending(const uint64_t* ids, size_t count, bool want_mapped) const {
        if (!open_) {
            throw std::runtime_error("backing is closed");
        }
        if (poisoned_) {
            throw std::runtime_error("backing is poisoned after a partial HIP failure");
        }
        if (count != 0 && ids == nullptr) {
            throw std::invalid_argument("chunk index array is null");
        }
        const uint64_t limit = reserved_bytes_ / chunk_bytes_;
        std::vector<uint64_t> result;
        result.reserve(count);
        for (size_t i = 0; i < count; ++i) {
            if (ids[i] >= limit) {
                throw std::out_of_range("chunk index outside reserved range");
            }
            if ((chunks_.count(ids[i]) != 0) == want_mapped) {
                result.push_back(ids[i]);
            }
        }
        std::sort(result.begin(), result.end());
        result.erase(std::unique(result.begin(), result.end()), result.end());
        return result;
    }

    hipError_t release(uint64_t id, Chunk& chunk) noexcept {
        if (chunk.mapped) {
            const hipError_t status = hipMemUnmap(address(id), chunk_bytes_);
            if (status != hipSuccess) {
                return status;
            }
            chunk.mapped = false;
        }
        if (chunk.created) {
            const hipError_t status = hipMemRelease(chunk.handle);
            if (status != hipSuccess) {
                return status;
            }
            chunk.created = false;
        }
        return hipSuccess;
    }

    int device_ = 0;
    uintptr_t base_ = 0;
    hipStream_t zero_stream_ = nullptr;
    hipMemAllocationProp prop_{};
    uint64_t reserved_bytes_ = 0;
    uint64_t chunk_bytes_ = 0;
    uint64_t granularity_ = 0;
    bool zero_pending_ = false;
    bool poisoned_ = false;
    bool open_ = false;
    std::map<uint64_t, Chunk> chunks_;
};

VmmBacking& require(void* handle) {
    if (handle == nullptr) {
        throw std::invalid_argument("null backing handle");
    }
    return *static_cast<VmmBacking*>(handle);
}

constexpr uint64_t kInvalid = std::numeric_limits<uint64_t>::max();

}  // namespace
}  // namespace ekv

using ekv::guarded;
using ekv::require;

extern "C" {

void* ev_create(int device, uint64_t capacity_bytes, uint64_t chunk_bytes) {
    return guarded(static_cast<void*>(nullptr), [&] {
        auto backing = std::make_unique<ekv::VmmBacking>(device, capacity_bytes, chunk_bytes);
        return static_cast<void*>(backing.release());
    });
}

int ev_ensure(void* handle, const uint64_t* indices, size_t count) {
    return guarded(-1, [&] {
        require(handle).commit(indices, count, true);
        return 0;
    });
}

int ev_precommit(void* handle, const uint64_t* indices, size_t count) {
    return guarded(-1, [&] {
        require(handle).commit(indices, count, false);
        return 0;
    });
}

int ev_drop(void* handle, const uint64_t* indices, size_t count) {
    return guarded(-1, [&] {
        require(handle).decommit(indices, count);
        return 0;
    });
}

uint64_t ev_base(void* handle) {
    return guarded(ekv::kInvalid, [&] { return require(handle).base(); });
}

uint64_t ev_backed(void* handle) {
    return guarded(ekv::kInvalid, [&] { return require(handle).backed(); });
}

uint64_t ev_reserved(void* handle) {
    return guarded(ekv::kInvalid, [&] { return require(handle).reserved(); });
}

uint64_t ev_granularity(void* handle) {
    return guarded(ekv::kInvalid, [&] { return require(handle).granularity(); });
}

int ev_poisoned(void* handle) {
    return guarded(-1, [&] { return require(handle).poisoned() ? 1 : 0; });
}

const char* ev_error(void) { return ekv::last_error().c_str(); }

int ev_close(void* handle) {
    return guarded(-1, [&] {
        if (handle == nullptr) {
            return 0;
        }
        auto* backing = static_cast<ekv::VmmBacking*>(handle);
        const hipError_t status = backing->close();
        if (status != hipSuccess) {
            ekv::fail_hip(status, "close backing");
        }
        delete backing;
        return 0;
    });
}

}  // extern "C"
