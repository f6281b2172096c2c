// The reference ingest's weight sanitising on GGUF bytes.
//
// The reference dequantises every tensor it loads and then zeroes each
// weight that is NaN, +-Inf or larger than 100 in magnitude
// (sanitize_weights, rust/src/model/loader.rs:241-249, applied by load_layer
// at loader.rs:161 and by load_special at loader.rs:188).  This library keeps
// weights in their GGUF bytes, so the same rule is applied to the bytes at
// upload:
//  * Q8_0 (v = q*d) and Q6_K (v = (d*sc)*q) encode an exact zero for any
//    single element (q = 0; the 6-bit code 32), so an outlier element gets
//    that code in place;
//  * a Q4_K element decodes to (d*sc)*q - dmin*m, and q = 0 yields zero only
//    where dmin*m is zero; an outlier elsewhere cannot be written in Q4_K,
//    and the caller stores that tensor as its sanitised f32 dequantisation
//    (lcmoe_dequantize with sanitize = 1) instead;
//  * a block whose scale is not finite decodes to non-finite values only, so
//    all of it becomes zero: its scales are set to +0;
//  * f32 tensors are sanitised element by element.
// The host decoders below restate rust/src/kernels/mod.rs:37-180 (two
// roundings per K-quant element, no fused multiply-add; this file is built
// with -ffp-contract=off).

#include <algorithm>
#include <atomic>
#include <cmath>
#include <thread>
#include <vector>

#include "lcmoe_internal.h"

namespace lcmoe {
namespace {

// sanitize_weights' test (loader.rs:245): NaN, +-Inf, |v| > 100.
inline bool outlier(float v) { return std::isnan(v) || std::isinf(v) || std::fabs(v) > 100.0f; }

inline float ld_half(const uint8_t *p) { return half_to_float((uint16_t)(p[0] | (p[1] << 8))); }
inline void st_zero_half(uint8_t *p) { p[0] = p[1] = 0; }

// get_scale_min_k4, rust/src/kernels/mod.rs:54-63.
inline void scale_min_k4(int j, const uint8_t *q, int *sc, int *m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

// dequantize_q8_0, kernels/mod.rs:37-51: v = (q as f32) * d.
void dec_q8_0(const uint8_t *b, float *o) {
    const float d = ld_half(b);
    for (int j = 0; j < 32; j++) o[j] = (float)(int8_t)b[2 + j] * d;
}

// dequantize_q4_k, kernels/mod.rs:66-98: sub-block pair (2g, 2g+1) takes the
// low / high nibbles of qs[32g .. 32g + 32]; v = (d*sc)*q - dmin*m.
void dec_q4_k(const uint8_t *b, float *o) {
    const float d = ld_half(b), dmin = ld_half(b + 2);
    const uint8_t *scales = b + 4, *qs = b + 16;
    for (int g = 0; g < 4; g++) {
        int sc1, m1, sc2, m2;
        scale_min_k4(2 * g, scales, &sc1, &m1);
        scale_min_k4(2 * g + 1, scales, &sc2, &m2);
        const float dl1 = d * (float)sc1, dl2 = d * (float)sc2;
        const float mn1 = dmin * (float)m1, mn2 = dmin * (float)m2;
        for (int l = 0; l < 32; l++) {
            const uint8_t q = qs[32 * g + l];
            o[64 * g + l] = dl1 * (float)(q & 0x0F) - mn1;
            o[64 * g + 32 + l] = dl2 * (float)(q >> 4) - mn2;
        }
    }
}

// Q6_K element i (0..255) of a block: byte positions of its low nibble and
// high bits, the scale index, and the shifts (dequantize_q6_k,
// kernels/mod.rs:145-180).  Half n = i / 128; within it r = i % 128,
// l = r % 32, quarter c = r / 32: ql byte 64n + l + 32 (c & 1), nibble
// c >> 1; qh byte 128 + 32n + l, bits 2c; scale 192 + 8n + l / 16 + 2c.
struct Q6Pos {
    int ql, qh, sc, nib_shift, qh_shift;
};
inline Q6Pos q6_pos(int i) {
    const int n = i / 128, r = i % 128, l = r % 32, c = r / 32;
    return {64 * n + l + 32 * (c & 1), 128 + 32 * n + l, 192 + 8 * n + l / 16 + 2 * c,
            4 * (c >> 1), 2 * c};
}

// dequantize_q6_k: v = (d * sc) * q with q = (nibble | hi2 << 4) - 32.
void dec_q6_k(const uint8_t *b, float *o) {
    const float d = ld_half(b + 208);
    for (int i = 0; i < 256; i++) {
        const Q6Pos p = q6_pos(i);
        const int q = (int)(((b[p.ql] >> p.nib_shift) & 0x0F) | (((b[p.qh] >> p.qh_shift) & 3) << 4)) - 32;
        o[i] = d * (float)(int8_t)b[p.sc] * (float)q;
    }
}

void dec_block(int32_t type, const uint8_t *b, float *o) {
    switch (type) {
    case LCMOE_TYPE_Q8_0: dec_q8_0(b, o); break;
    case LCMOE_TYPE_Q4_K: dec_q4_k(b, o); break;
    case LCMOE_TYPE_Q6_K: dec_q6_k(b, o); break;
    default: break;
    }
}

// Scale fields of a block: all finite?
bool scales_finite(int32_t type, const uint8_t *b) {
    switch (type) {
    case LCMOE_TYPE_Q8_0: return std::isfinite(ld_half(b));
    case LCMOE_TYPE_Q4_K: return std::isfinite(ld_half(b)) && std::isfinite(ld_half(b + 2));
    case LCMOE_TYPE_Q6_K: return std::isfinite(ld_half(b + 208));
    default: return true;
    }
}

// Can any element of this block (finite scales) be an outlier?  Each decode
// is monotone in q for fixed scales (every step is one rounded operation
// monotone in its varying operand), so the extreme codes bound a group:
// Q8_0 by max |q|, Q4_K by q = 0 and 15 per sub-block, Q6_K by q = -32 per
// 16-element group (|(d*sc) * -32| >= |(d*sc) * 31|).
bool block_may_have_outlier(int32_t type, const uint8_t *b) {
    switch (type) {
    case LCMOE_TYPE_Q8_0: {
        int mx = 0;
        for (int j = 0; j < 32; j++) mx = std::max(mx, std::abs((int)(int8_t)b[2 + j]));
        return outlier((float)mx * ld_half(b));
    }
    case LCMOE_TYPE_Q4_K: {
        const float d = ld_half(b), dmin = ld_half(b + 2);
        for (int j = 0; j < 8; j++) {
            int sc, m;
            scale_min_k4(j, b + 4, &sc, &m);
            const float dl = d * (float)sc, mn = dmin * (float)m;
            if (outlier(dl * 0.0f - mn) || outlier(dl * 15.0f - mn)) return true;
        }
        return false;
    }
    case LCMOE_TYPE_Q6_K: {
        const float d = ld_half(b + 208);
        for (int j = 0; j < 16; j++)
            if (outlier(d * (float)(int8_t)b[192 + j] * -32.0f)) return true;
        return false;
    }
    default: return false;
    }
}

struct BlockResult {
    int64_t zeroed = 0, unzeroable = 0;
};

// One block: zero every outlier in place where the type can encode it
// (modify), and count the outliers that cannot be.
BlockResult sanitize_block(int32_t type, uint8_t *b, bool modify) {
    BlockResult r;
    const int bs = (int)block_size(type);
    if (!scales_finite(type, b)) {  // every element decodes non-finite
        r.zeroed = bs;
        if (modify) {
            if (type == LCMOE_TYPE_Q6_K) {
                st_zero_half(b + 208);
            } else {
                st_zero_half(b);
                if (type == LCMOE_TYPE_Q4_K) st_zero_half(b + 2);
            }
        }
        return r;
    }
    if (!block_may_have_outlier(type, b)) return r;
    float v[256];
    dec_block(type, b, v);
    for (int i = 0; i < bs; i++) {
        if (!outlier(v[i])) continue;
        switch (type) {
        case LCMOE_TYPE_Q8_0:
            r.zeroed++;
            if (modify) b[2 + i] = 0;
            break;
        case LCMOE_TYPE_Q6_K: {
            r.zeroed++;
            if (modify) {  // code 32: low nibble 0, high bits 2
                const Q6Pos p = q6_pos(i);
                b[p.ql] = (uint8_t)(b[p.ql] & ~(0x0F << p.nib_shift));
                b[p.qh] = (uint8_t)((b[p.qh] & ~(3 << p.qh_shift)) | (2 << p.qh_shift));
            }
            break;
        }
        case LCMOE_TYPE_Q4_K: {
            int sc, m;
            scale_min_k4(i / 32, b + 4, &sc, &m);
            if (ld_half(b + 2) * (float)m == 0.0f) {  // q = 0 decodes to +-0
                r.zeroed++;
                if (modify) {
                    uint8_t &q = b[16 + 32 * (i / 64) + i % 32];
                    q = (i / 32) % 2 ? (uint8_t)(q & 0x0F) : (uint8_t)(q & 0xF0);
                }
            } else {
                r.unzeroable++;
            }
            break;
        }
        default: break;
        }
    }
    return r;
}

template <class Fn>
void parallel_blocks(int64_t nb, Fn fn) {
    const unsigned nth = nb < 4096 ? 1u : std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    if (nth == 1) {
        fn(0, nb);
        return;
    }
    std::vector<std::thread> th;
    const int64_t per = (nb + nth - 1) / nth;
    for (unsigned t = 0; t < nth; t++) {
        const int64_t b0 = t * per, b1 = std::min(nb, b0 + per);
        if (b0 < b1) th.emplace_back([=] { fn(b0, b1); });
    }
    for (auto &x : th) x.join();
}

BlockResult sanitize_bytes(int32_t type, uint8_t *data, int64_t count, bool modify) {
    BlockResult total;
    if (type == LCMOE_TYPE_F32) {
        for (int64_t i = 0; i < count; i++) {
            float v;
            std::memcpy(&v, data + 4 * i, 4);
            if (!outlier(v)) continue;
            total.zeroed++;
            if (modify) std::memset(data + 4 * i, 0, 4);
        }
        return total;
    }
    const int64_t bs = block_size(type), bb = block_bytes(type), nb = count / bs;
    std::atomic<int64_t> zeroed{0}, unz{0};
    parallel_blocks(nb, [&](int64_t b0, int64_t b1) {
        int64_t z = 0, u = 0;
        for (int64_t i = b0; i < b1; i++) {
            const BlockResult r = sanitize_block(type, data + i * bb, modify);
            z += r.zeroed;
            u += r.unzeroable;
        }
        zeroed += z;
        unz += u;
    });
    total.zeroed = zeroed;
    total.unzeroable = unz;
    return total;
}

bool sanitizable_type(int32_t t) {
    return t == LCMOE_TYPE_F32 || t == LCMOE_TYPE_Q8_0 || t == LCMOE_TYPE_Q4_K ||
           t == LCMOE_TYPE_Q6_K;
}

}  // namespace

int64_t count_outliers(int32_t type, const uint8_t *data, int64_t count, int64_t *unzeroable) {
    // modify == false never writes through the pointer
    const BlockResult r = sanitize_bytes(type, const_cast<uint8_t *>(data), count, false);
    if (unzeroable) *unzeroable = r.unzeroable;
    return r.zeroed + r.unzeroable;
}

bool SanitizedStack::analyse() {
    const size_t sz = lcmoe_tensor_size(qt_in, rows * cols);
    fix.assign((size_t)(na + nb), 0);
    bool need_f32 = false;
    for (int e = 0; e < na + nb; e++) {
        const uint8_t *src = e < na ? a + (size_t)e * sz : b + (size_t)(e - na) * sz;
        int64_t unz = 0;
        fix[e] = count_outliers(qt_in, src, rows * cols, &unz) > 0;
        need_f32 = need_f32 || unz > 0;
    }
    return need_f32;
}

const uint8_t *SanitizedStack::get(int e, std::vector<uint8_t> &buf) const {
    const size_t sz = lcmoe_tensor_size(qt_in, rows * cols);
    const uint8_t *src = e < na ? a + (size_t)e * sz : b + (size_t)(e - na) * sz;
    if (qt == LCMOE_TYPE_F32 && qt_in != LCMOE_TYPE_F32) {
        buf.resize((size_t)(rows * cols) * 4);
        lcmoe_dequantize(qt_in, src, rows * cols, reinterpret_cast<float *>(buf.data()), 1);
        return buf.data();
    }
    if (fix.empty() || !fix[e]) return src;
    buf.assign(src, src + sz);
    sanitize_bytes(qt_in, buf.data(), rows * cols, true);
    return buf.data();
}

int64_t SanitizedStack::stored_bytes() const { return (int64_t)lcmoe_tensor_size(qt, rows * cols); }

}  // namespace lcmoe

using namespace lcmoe;

extern "C" int64_t lcmoe_dequantize(int32_t type, const uint8_t *data, int64_t count, float *out,
                                    int32_t sanitize) {
    if (!data || !out || count < 0 || !sanitizable_type(type)) return -1;
    if (type == LCMOE_TYPE_F32) {
        std::memcpy(out, data, 4 * (size_t)count);
    } else {
        // whole blocks only, as the reference decoders (num_blocks =
        // out.len() / block size; the rest of `out` stays zero)
        const int64_t bs = block_size(type), bb = block_bytes(type), nb = count / bs;
        parallel_blocks(nb, [&](int64_t b0, int64_t b1) {
            for (int64_t i = b0; i < b1; i++) dec_block(type, data + i * bb, out + i * bs);
        });
        std::fill(out + nb * bs, out + count, 0.0f);
    }
    if (!sanitize) return 0;
    int64_t n = 0;
    for (int64_t i = 0; i < count; i++)
        if (outlier(out[i])) {
            out[i] = 0.0f;
            n++;
        }
    return n;
}

extern "C" int64_t lcmoe_sanitize_blocks(int32_t type, uint8_t *data, int64_t count,
                                         int64_t *unzeroable) {
    if (unzeroable) *unzeroable = 0;
    if (!data || count < 0 || !sanitizable_type(type)) return -1;
    const BlockResult r = sanitize_bytes(type, data, count, true);
    if (unzeroable) *unzeroable = r.unzeroable;
    return r.zeroed;
}
