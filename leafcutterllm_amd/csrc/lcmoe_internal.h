// Internal declarations shared by the host utilities (lcmoe_host.cpp) and the
// HIP implementation (lcmoe.hip).  Not part of the ABI.
#pragma once

#include <cstdarg>
#include <cstddef>
#include <cstdint>
#include <cstring>

#include "../../include/lcmoe.h"

namespace lcmoe {

// Sets the calling thread's last-error message and returns `st`.
lcmoe_status fail(lcmoe_status st, const char *fmt, ...);
void clear_error();

// GGUF block geometry (QuantType::block_size / block_bytes,
// rust/src/model/quant.rs:170-239) for the types this library handles.
inline int64_t block_size(int32_t type) {
    switch (type) {
    case LCMOE_TYPE_F32: return 1;
    case LCMOE_TYPE_Q8_0: return 32;
    case LCMOE_TYPE_Q4_K:
    case LCMOE_TYPE_Q6_K: return 256;
    default: return 0;
    }
}
inline int64_t block_bytes(int32_t type) {
    switch (type) {
    case LCMOE_TYPE_F32: return 4;
    case LCMOE_TYPE_Q8_0: return 34;
    case LCMOE_TYPE_Q4_K: return 144;
    case LCMOE_TYPE_Q6_K: return 210;
    default: return 0;
    }
}

// IEEE binary16 <-> binary32, bit level (exact widening, RNE narrowing).
inline float half_to_float(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu, u;
    if (e == 0) {
        if (m == 0) {
            u = sign;
        } else {
            int sh = 0;
            while (!(m & 0x400u)) { m <<= 1; sh++; }
            u = sign | ((uint32_t)(113 - sh) << 23) | ((m & 0x3ffu) << 13);
        }
    } else if (e == 31) {
        u = sign | 0x7f800000u | (m << 13);
    } else {
        u = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

inline uint16_t float_to_half(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
    if (ax < 0x38800000u) {
        if (ax < 0x33000000u) return sign;
        uint32_t e = ax >> 23, mant = (ax & 0x7fffffu) | 0x800000u;
        int shift = 126 - (int)e;
        uint32_t q = mant >> shift, rem = mant & ((1u << shift) - 1u), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t h = ((((ax >> 23) - 112u) << 10) | ((ax & 0x7fffffu) >> 13));
    uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

// Host-side validation of a descriptor (no GPU).  Returns LCMOE_OK or an
// error with the message set.
lcmoe_status validate_desc(const lcmoe_desc *d);
// Host-side scan of every expert tensor's block scales.
lcmoe_status scan_weights(const lcmoe_desc *d, const lcmoe_weights *w);
// RPL64 repack (defined in lcmoe_host.cpp, layout documented there).
void repack_rpl64_q4k(const uint8_t *src, uint8_t *dst, int64_t rows, int64_t cols);
// RPL64 repack of Q6_K (defined in lcmoe_host.cpp, layout documented there).
void repack_rpl64_q6k(const uint8_t *src, uint8_t *dst, int64_t rows, int64_t cols);
// RPL64 repack of Q8_0 (lcmoe_host.cpp).
void repack_rpl64_q8(const uint8_t *src, uint8_t *dst, int64_t rows, int64_t cols);
// Split repack of Q4_K with cols an odd multiple of 128 (lcmoe_host.cpp).
void repack_rpl64_q4k_split(const uint8_t *src, uint8_t *dst, int64_t rows, int64_t cols);

}  // namespace lcmoe
