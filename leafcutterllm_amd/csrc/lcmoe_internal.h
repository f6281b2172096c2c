// Internal declarations shared by the host utilities (lcmoe_host.cpp) and the
// HIP implementation (lcmoe.hip).  Not part of the ABI.
#pragma once

#include <cstdarg>
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <vector>

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

// Weights the reference's sanitize_weights (rust/src/model/loader.rs:241-249)
// zeroes in `count` elements of GGUF bytes of `type` (lcmoe_sanitize.cpp);
// *unzeroable: how many of them a Q4_K block cannot encode as zero in place.
int64_t count_outliers(int32_t type, const uint8_t *data, int64_t count, int64_t *unzeroable);

// A stack of n expert matrices [rows, cols] as the library uploads them
// after sanitising: the caller's bytes where no weight trips the rule, a
// zero-coded copy where every outlier can be written as zero in place, and
// the sanitised f32 dequantisation of every expert when some Q4_K outlier
// cannot (the stored type is then LCMOE_TYPE_F32).  Experts [0, na) come
// from a, [na, na + nb) from b.
struct SanitizedStack {
    const uint8_t *a = nullptr, *b = nullptr;
    int na = 0, nb = 0;
    int32_t qt_in = 0, qt = 0;  // the caller's type, the stored type
    int64_t rows = 0, cols = 0;
    std::vector<uint8_t> fix;   // per expert: needs a zero-coded copy
    // Scans every expert and fills `fix`; true when some Q4_K outlier cannot
    // be zero-coded, so the stack must be stored as f32 (qt = F32; the
    // caller decides, since gate and up share one stored type).
    bool analyse();
    // expert e's bytes as stored (`buf` may hold them)
    const uint8_t *get(int e, std::vector<uint8_t> &buf) const;
    int64_t stored_bytes() const;  // per expert
};

}  // namespace lcmoe
