// Division of 32-bit unsigned numerators by a divisor fixed at launch time,
// by multiply-high and shift (round-up reciprocal method of Granlund and
// Montgomery, "Division by invariant integers using multiplication", 1994).
// For d >= 1 let s = ceil(log2 d) and m = floor(2^32 * (2^s - d) / d) + 1;
// then for every n < 2^31:  n / d == (mulhi32(n, m) + n) >> s.
// The sum stays below 2^32 because n < 2^31 and mulhi32(n, m) <= n.
#pragma once

#include <cstdint>

#if defined(__HIPCC__)
#define EKV_HD __host__ __device__
#else
#define EKV_HD
#endif

namespace ekv {

struct FastDiv {
    uint32_t divisor = 1;
    uint32_t multiplier = 1;
    uint32_t shift = 0;

    FastDiv() = default;

    explicit FastDiv(uint32_t d) : divisor(d) {
        uint32_t s = 0;
        while ((uint64_t{1} << s) < d) {
            ++s;
        }
        shift = s;
        multiplier = static_cast<uint32_t>(((uint64_t{1} << 32) * ((uint64_t{1} << s) - d)) / d + 1);
    }

    // Valid for n < 2^31.
    EKV_HD uint32_t div(uint32_t n) const {
#if defined(__HIP_DEVICE_COMPILE__)
        const uint32_t high = __umulhi(n, multiplier);
#else
        const uint32_t high = static_cast<uint32_t>((uint64_t{n} * multiplier) >> 32);
#endif
        return (high + n) >> shift;
    }
};

}  // namespace ekv
