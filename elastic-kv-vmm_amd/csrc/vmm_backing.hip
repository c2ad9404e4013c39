// Demand-backed virtual KV range on HIP virtual memory management: the HIP
// driver of vmm_core.h (whose Backing holds the reference's semantics,
// native/elastic_vmm.cpp) and the ev_* C ABI over it. HIP-native parts:
//   * the reservation is aligned to the chunk size when the chunk size is a
//     power of two, so every 2 MiB chunk can use a 2 MiB GPU page;
//   * access is granted per chunk and new chunks are zero-filled by our own
//     fill kernel over each contiguous run of new chunks, on a private
//     non-blocking stream (a kernel does not care that a run spans several
//     physical allocations);
//   * a failed close keeps the object alive so the close can be retried.
#include "../../include/elastic_vmm.h"
#include "ekv_common.h"
#include "vmm_core.h"

#include <algorithm>
#include <string>

namespace ekv {
namespace {

// Zero `words` 16-byte words starting at `base` (grid-stride, 16 B per lane).
__global__ __launch_bounds__(256) void zero_fill_kernel(uint4* __restrict__ base, uint64_t words) {
    const uint64_t stride = uint64_t{gridDim.x} * blockDim.x;
    for (uint64_t i = uint64_t{blockIdx.x} * blockDim.x + threadIdx.x; i < words; i += stride) {
        base[i] = make_uint4(0u, 0u, 0u, 0u);
    }
}

// The HIP side of vmm::Backing: physical chunks are pinned device allocations
// (hipMemCreate) of the object's device, granted read/write per chunk and
// zero-filled by zero_fill_kernel on a private non-blocking stream. Statuses
// are hipError_t values.
class HipDriver {
public:
    class Scope {
    public:
        explicit Scope(HipDriver& driver) {
            status_ = hipGetDevice(&previous_);
            if (status_ == hipSuccess && previous_ != driver.device_) {
                status_ = hipSetDevice(driver.device_);
                switched_ = status_ == hipSuccess;
            }
        }
        ~Scope() {
            if (switched_) {
                (void)hipSetDevice(previous_);
            }
        }
        Scope(const Scope&) = delete;
        Scope& operator=(const Scope&) = delete;
        int status() const { return status_; }

    private:
        int previous_ = 0;
        int status_ = hipSuccess;
        bool switched_ = false;
    };

    int init(int device, uint64_t* granularity) {
        int count = 0;
        hipError_t status = hipGetDeviceCount(&count);
        if (status != hipSuccess) {
            return status;
        }
        if (device < 0 || device >= count) {
            throw std::invalid_argument("device ordinal " + std::to_string(device) + " out of range (" +
                                        std::to_string(count) + " devices)");
        }
        device_ = device;
        int supported = 0;
        status = hipDeviceGetAttribute(&supported, hipDeviceAttributeVirtualMemoryManagementSupported, device);
        if (status != hipSuccess) {
            return status;
        }
        if (!supported) {
            throw std::runtime_error("device does not support HIP virtual memory management");
        }
        prop_.type = hipMemAllocationTypePinned;
        prop_.location.type = hipMemLocationTypeDevice;
        prop_.location.id = device;
        size_t bytes = 0;
        status = hipMemGetAllocationGranularity(&bytes, &prop_, hipMemAllocationGranularityMinimum);
        *granularity = bytes;
        return status;
    }

    int reserve(uint64_t bytes, uint64_t alignment, uintptr_t* base) {
        void* address = nullptr;
        const hipError_t status = hipMemAddressReserve(&address, bytes, alignment, nullptr, 0);
        *base = reinterpret_cast<uintptr_t>(address);
        return status;
    }
    int free_range(uintptr_t base, uint64_t bytes) {
        return hipMemAddressFree(reinterpret_cast<void*>(base), bytes);
    }
    int open_stream() { return hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking); }
    int close_stream() {
        const hipError_t status = hipStreamDestroy(stream_);
        if (status == hipSuccess) {
            stream_ = nullptr;
        }
        return status;
    }
    int create(uint64_t bytes, uint64_t* handle) {
        hipMemGenericAllocationHandle_t created{};
        const hipError_t status = hipMemCreate(&created, bytes, &prop_, 0);
        *handle = reinterpret_cast<uint64_t>(created);
        return status;
    }
    int map(uintptr_t address, uint64_t bytes, uint64_t handle) {
        return hipMemMap(reinterpret_cast<void*>(address), bytes, 0,
                         reinterpret_cast<hipMemGenericAllocationHandle_t>(handle), 0);
    }
    int set_access(uintptr_t address, uint64_t bytes) {
        hipMemAccessDesc access{};
        access.location = prop_.location;
        access.flags = hipMemAccessFlagsProtReadWrite;
        return hipMemSetAccess(reinterpret_cast<void*>(address), bytes, &access, 1);
    }
    int unmap(uintptr_t address, uint64_t bytes) { return hipMemUnmap(reinterpret_cast<void*>(address), bytes); }
    int release(uint64_t handle) {
        return hipMemRelease(reinterpret_cast<hipMemGenericAllocationHandle_t>(handle));
    }
    int zero_async(uintptr_t address, uint64_t bytes) {
        const uint64_t words = bytes / 16;
        const uint64_t blocks = std::min<uint64_t>((words + 255) / 256, 65536);
        zero_fill_kernel<<<dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, stream_>>>(
            reinterpret_cast<uint4*>(address), words);
        return hipGetLastError();
    }
    int wait_zero() { return hipStreamSynchronize(stream_); }
    int synchronize_device() { return hipDeviceSynchronize(); }
    std::string describe(int status) const {
        const auto code = static_cast<hipError_t>(status);
        return std::string(hipGetErrorName(code)) + " (" + hipGetErrorString(code) + ")";
    }

private:
    int device_ = 0;
    hipStream_t stream_ = nullptr;
    hipMemAllocationProp prop_{};
};

}  // namespace
}  // namespace ekv

EKV_DEFINE_VMM_ABI(ekv::HipDriver)
