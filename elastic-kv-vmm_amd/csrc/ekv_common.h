// Shared host-side plumbing of libelastic_vmm: error capture across the C ABI,
// HIP status checks and a current-device guard.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <stdexcept>
#include <string>

namespace ekv {

// Thread-local message of the last failed ABI call (read by ev_error()).
std::string& last_error();

[[noreturn]] inline void fail_hip(hipError_t status, const char* what) {
    throw std::runtime_error(std::string(what) + ": " + hipGetErrorName(status) + " (" +
                             hipGetErrorString(status) + ")");
}

inline void check_hip(hipError_t status, const char* what) {
    if (status != hipSuccess) {
        fail_hip(status, what);
    }
}

// Runs `body` and converts any C++ exception into `error_value` plus a message.
template <typename Result, typename Body>
Result guarded(Result error_value, Body&& body) noexcept {
    try {
        last_error().clear();
        return body();
    } catch (const std::exception& e) {
        last_error() = e.what();
    } catch (...) {
        last_error() = "unknown native error";
    }
    return error_value;
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
