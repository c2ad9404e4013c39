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

// Checking without launching: while a CheckOnly guard lives on this thread,
// the kernel entry points run all of their argument checks and return before
// their first launch. ekv_decode_step checks its four stages this way before
// it queues any of them, so a bad argument to a later stage fails the call
// with nothing queued instead of after the earlier stages have written their
// outputs.
inline bool& check_only_flag() {
    static thread_local bool flag = false;
    return flag;
}

inline bool check_only() { return check_only_flag(); }

class CheckOnly {
public:
    CheckOnly() : previous_(check_only_flag()) { check_only_flag() = true; }
    ~CheckOnly() { check_only_flag() = previous_; }
    CheckOnly(const CheckOnly&) = delete;
    CheckOnly& operator=(const CheckOnly&) = delete;

private:
    bool previous_;
};

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
