// Shared host-side plumbing of libelastic_vmm: HIP status checks, a
// current-device guard and (from ekv_errors.h) error capture across the C ABI.
#pragma once

#include "ekv_errors.h"

#include <hip/hip_runtime.h>

#include <cstdint>
#include <stdexcept>
#include <string>

namespace ekv {

[[noreturn]] inline void fail_hip(hipError_t status, const char* what) {
    throw std::runtime_error(std::string(what) + ": " + hipGetErrorName(status) + " (" +
                             hipGetErrorString(status) + ")");
}

inline void check_hip(hipError_t status, const char* what) {
    if (status != hipSuccess) {
        fail_hip(status, what);
    }
}

// Makes `device` current for the lifetime of the guard and restores the
// caller's current device afterwards (HIP's current device is per thread).
class DeviceGuard {
public:
    explicit DeviceGuard(int device) {
        check_hip(hipGetDevice(&previous_), "hipGetDevice");
        if (previous_ != device) {
            check_hip(hipSetDevice(device), "hipSetDevice");
            switched_ = true;
        }
    }
    ~DeviceGuard() {
        if (switched_) {
            (void)hipSetDevice(previous_);
        }
    }
    DeviceGuard(const DeviceGuard&) = delete;
    DeviceGuard& operator=(const DeviceGuard&) = delete;

private:
    int previous_ = 0;
    bool switched_ = false;
};

}  // namespace ekv
