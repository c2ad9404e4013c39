// Vector types for byte-moving kernels and the host-side choice of their width.
#pragma once

#include <cstdint>
#include <initializer_list>

namespace ekv {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

// Vec<VW>::type moves VW bytes with one lane access.
template <int VW> struct Vec;
template <> struct Vec<16> { using type = u32x4; };
template <> struct Vec<8> { using type = u32x2; };
template <> struct Vec<4> { using type = uint32_t; };
template <> struct Vec<2> { using type = uint16_t; };
template <> struct Vec<1> { using type = uint8_t; };

// Largest power of two <= 16 that divides every value (addresses, strides, sizes).
inline int pick_vector_width(std::initializer_list<int64_t> values) {
    int vw = 16;
    for (const int64_t v : values) {
        while (vw > 1 && (v % vw) != 0) {
            vw >>= 1;
        }
    }
    return vw;
}

}  // namespace ekv
