// Error capture across the C ABI, shared by every entry point of
// libelastic_vmm. Free of HIP headers, so host-only builds (the VMM core under
// a fault-injecting driver) can use it too.
#pragma once

#include <stdexcept>
#include <string>

namespace ekv {

// Thread-local message of the last failed ABI call (read by ev_error()).
// Defined once per binary: in the library by vmm_backing.hip.
std::string& last_error();

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

}  // namespace ekv
