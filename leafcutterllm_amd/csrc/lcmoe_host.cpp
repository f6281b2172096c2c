// Host-side utilities of the MoE library: error state, block geometry,
// descriptor validation, block-scale scan, GGUF encoders and the synthetic
// data generator.  None of this touches the GPU, so all of it runs (and is
// tested) on machines without one.
//
// Built with -ffp-contract=off: the encoders' a*b+c are two roundings, so
// their bytes do not depend on the compiler's contraction choices.

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <string>
#include <thread>
#include <vector>

#include "lcmoe_internal.h"

namespace lcmoe {

static thread_local std::string g_last_error;

lcmoe_status fail(lcmoe_status st, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return st;
}

void clear_error() { g_last_error.clear(); }

static bool type_ok(int32_t t) {
    return t == LCMOE_TYPE_F32 || t == LCMOE_TYPE_Q8_0 || t == LCMOE_TYPE_Q4_K ||
           t == LCMOE_TYPE_Q6_K;
}

lcmoe_status validate_desc(const lcmoe_desc *d) {
    if (!d) return fail(LCMOE_ERR_INVALID_ARG, "desc is NULL");
    if (d->d_model <= 0 || d->d_model % 32)
        return fail(LCMOE_ERR_INVALID_ARG, "d_model=%d must be a positive multiple of 32", d->d_model);
    if (d->d_model > 16384) return fail(LCMOE_ERR_INVALID_ARG, "d_model=%d exceeds 16384", d->d_model);
    if (d->d_ff <= 0 || d->d_ff % 32)
        return fail(LCMOE_ERR_INVALID_ARG, "d_ff=%d must be a positive multiple of 32", d->d_ff);
    if (d->n_expert < 1 || d->n_expert > 256)
        return fail(LCMOE_ERR_INVALID_ARG, "n_expert=%d outside [1, 256]", d->n_expert);
    if (d->n_expert_used < 1 || d->n_expert_used > 16 || d->n_expert_used > d->n_expert)
        return fail(LCMOE_ERR_INVALID_ARG, "n_expert_used=%d outside [1, min(16, n_expert)]",
                    d->n_expert_used);
    if (d->n_shared < 0 || d->n_shared > 8)
        return fail(LCMOE_ERR_INVALID_ARG, "n_shared=%d outside [0, 8]", d->n_shared);
    if (d->n_shared > 0 && (d->d_ff_shared <= 0 || d->d_ff_shared % 32))
        return fail(LCMOE_ERR_INVALID_ARG, "d_ff_shared=%d must be a positive multiple of 32",
                    d->d_ff_shared);
    if (d->max_tokens < 1 || d->max_tokens > 65536)
        return fail(LCMOE_ERR_INVALID_ARG, "max_tokens=%d outside [1, 65536]", d->max_tokens);
    if (!(d->routed_scale == d->routed_scale) || std::isinf(d->routed_scale))
        return fail(LCMOE_ERR_INVALID_ARG, "routed_scale is not finite");
    switch (d->route_kind) {
    case LCMOE_ROUTE_SOFTMAX_RENORM:
    case LCMOE_ROUTE_SOFTMAX: break;
    case LCMOE_ROUTE_SIGMOID_GROUP:
        if (d->n_group < 1 || d->n_group > 64 || d->n_expert % d->n_group)
            return fail(LCMOE_ERR_INVALID_ARG, "n_group=%d must be <= 64 and divide n_expert=%d", d->n_group,
                        d->n_expert);
        if (d->topk_group < 1 || d->topk_group > d->n_group)
            return fail(LCMOE_ERR_INVALID_ARG, "topk_group=%d outside [1, n_group]", d->topk_group);
        if (d->n_expert_used > d->topk_group * (d->n_expert / d->n_group))
            return fail(LCMOE_ERR_INVALID_ARG, "n_expert_used exceeds the experts of the kept groups");
        break;
    default: return fail(LCMOE_ERR_UNSUPPORTED, "route_kind=%d unknown", d->route_kind);
    }
    const int32_t types[3] = {d->type_gate, d->type_up, d->type_down};
    for (int32_t t : types)
        if (!type_ok(t)) return fail(LCMOE_ERR_UNSUPPORTED, "expert quant type %d unsupported", t);
    if (d->n_shared > 0) {
        const int32_t st[3] = {d->type_gate_sh, d->type_up_sh, d->type_down_sh};
        for (int32_t t : st)
            if (!type_ok(t)) return fail(LCMOE_ERR_UNSUPPORTED, "shared quant type %d unsupported", t);
    }
    return LCMOE_OK;
}

}  // namespace lcmoe

using namespace lcmoe;

extern "C" const char *lcmoe_last_error(void) { return g_last_error.c_str(); }

extern "C" size_t lcmoe_tensor_size(int32_t type, int64_t count) {
    int64_t bs = block_size(type), bb = block_bytes(type);
    if (!bs || count < 0) return 0;
    return (size_t)((count + bs - 1) / bs * bb);
}

static inline float ld_half(const uint8_t *p) { return half_to_float((uint16_t)(p[0] | (p[1] << 8))); }

static inline bool bad_scale(float v) { return std::isnan(v) || std::isinf(v) || std::fabs(v) > 1e4f; }

// Per-block test of scan_for_corruption (rust/src/model/loader.rs:389-398):
// d (Q6_K: bytes 208..209; others: 0..1) and, for Q4_K, dmin (2..3).
extern "C" int64_t lcmoe_scan_blocks(int32_t type, const uint8_t *data, int64_t count) {
    int64_t bs = block_size(type), bb = block_bytes(type);
    if (!data || !bs || count <= 0 || type == LCMOE_TYPE_F32) return 0;
    int64_t nb = (count + bs - 1) / bs, bad = 0;
    for (int64_t i = 0; i < nb; i++) {
        const uint8_t *b = data + i * bb;
        bool is_bad;
        if (type == LCMOE_TYPE_Q6_K) {
            is_bad = bad_scale(ld_half(b + 208));
        } else {
            is_bad = bad_scale(ld_half(b));
            if (type == LCMOE_TYPE_Q4_K) is_bad = is_bad || bad_scale(ld_half(b + 2));
        }
        bad += is_bad ? 1 : 0;
    }
    return bad;
}

namespace lcmoe {

static lcmoe_status scan_tensor(const char *name, int32_t type, const uint8_t *p, int64_t per_count,
                                int n) {
    if (!p) return fail(LCMOE_ERR_INVALID_ARG, "%s is NULL", name);
    if (type == LCMOE_TYPE_F32) return LCMOE_OK;
    size_t sz = lcmoe_tensor_size(type, per_count);
    for (int e = 0; e < n; e++) {
        int64_t bad = lcmoe_scan_blocks(type, p + (size_t)e * sz, per_count);
        if (bad)
            return fail(LCMOE_ERR_CORRUPT, "%s[%d]: %lld block(s) with a non-finite or |scale|>1e4",
                        name, e, (long long)bad);
    }
    return LCMOE_OK;
}

lcmoe_status scan_weights(const lcmoe_desc *d, const lcmoe_weights *w) {
    if (!w) return fail(LCMOE_ERR_INVALID_ARG, "weights is NULL");
    if (!w->router) return fail(LCMOE_ERR_INVALID_ARG, "router is NULL");
    if (d->has_bias && !w->bias) return fail(LCMOE_ERR_INVALID_ARG, "has_bias set but bias is NULL");
    // (non-finite router weights are not refused: the upload sanitises
    // them to 0 as load_layer does, rust/src/model/loader.rs:161)
    int64_t D = d->d_model, F = d->d_ff, FS = d->d_ff_shared;
    lcmoe_status st;
    if ((st = scan_tensor("gate", d->type_gate, w->gate, F * D, d->n_expert))) return st;
    if ((st = scan_tensor("up", d->type_up, w->up, F * D, d->n_expert))) return st;
    if ((st = scan_tensor("down", d->type_down, w->down, D * F, d->n_expert))) return st;
    if (d->n_shared > 0) {
        if ((st = scan_tensor("gate_sh", d->type_gate_sh, w->gate_sh, FS * D, d->n_shared))) return st;
        if ((st = scan_tensor("up_sh", d->type_up_sh, w->up_sh, FS * D, d->n_shared))) return st;
        if ((st = scan_tensor("down_sh", d->type_down_sh, w->down_sh, D * FS, d->n_shared))) return st;
    }
    return LCMOE_OK;
}

// ------------------------------------------------------------------------
// Encoders
// ------------------------------------------------------------------------

static inline void st_half(uint8_t *p, uint16_t h) {
    p[0] = (uint8_t)(h & 0xff);
    p[1] = (uint8_t)(h >> 8);
}
static inline float clampf(float v, float lo, float hi) { return v < lo ? lo : (v > hi ? hi : v); }
// f32::max of the Rust reference: the non-NaN argument wins.
static inline float nan_max(float a, float b) {
    if (a != a) return b;
    if (b != b) return a;
    return a > b ? a : b;
}

// quantize_f32_to_q8_0, rust/src/kernels/q8_0.rs:90-122.
static void enc_q8_0(const float *v, uint8_t *o) {
    float max_abs = 0.0f;
    for (int i = 0; i < 32; i++) max_abs = nan_max(max_abs, std::fabs(v[i]));
    float scale = max_abs > 0.0f ? max_abs / 127.0f : 0.0f;
    st_half(o, float_to_half(scale));
    for (int i = 0; i < 32; i++) {
        int8_t q = 0;
        if (scale > 0.0f) {
            float r = clampf(std::round(v[i] / scale), -127.0f, 127.0f);
            q = (r != r) ? 0 : (int8_t)r;
        }
        o[2 + i] = (uint8_t)q;
    }
}

// Q4_K encoder (this project's own; the decoder is dequantize_q4_k,
// rust/src/kernels/mod.rs:66-98).  Sub-block j of 32: lo = min(0, min v),
// scale_j = (max v - lo) / 15, min_j = -lo; d = max scale / 63 and dmin =
// max min / 63 stored as f16; sc_j, m_j = nearest 6-bit multiples;
// q = round((v + dmin*m_j) / (d*sc_j)) in [0, 15].
static void enc_q4_k(const float *v, uint8_t *o) {
    float scale[8], mn[8], max_scale = 0.0f, max_min = 0.0f;
    for (int j = 0; j < 8; j++) {
        float lo = v[32 * j], hi = v[32 * j];
        for (int l = 1; l < 32; l++) {
            float t = v[32 * j + l];
            if (t < lo) lo = t;
            if (t > hi) hi = t;
        }
        if (lo > 0.0f) lo = 0.0f;
        scale[j] = (hi - lo) / 15.0f;
        mn[j] = -lo;
        if (scale[j] > max_scale) max_scale = scale[j];
        if (mn[j] > max_min) max_min = mn[j];
    }
    uint16_t d16 = float_to_half(max_scale / 63.0f), m16 = float_to_half(max_min / 63.0f);
    float df = half_to_float(d16), mf = half_to_float(m16);
    uint8_t sc[8], m[8];
    for (int j = 0; j < 8; j++) {
        sc[j] = df > 0.0f ? (uint8_t)clampf(std::round(scale[j] / df), 0.0f, 63.0f) : 0;
        m[j] = mf > 0.0f ? (uint8_t)clampf(std::round(mn[j] / mf), 0.0f, 63.0f) : 0;
    }
    st_half(o, d16);
    st_half(o + 2, m16);
    uint8_t *s = o + 4;
    for (int j = 0; j < 4; j++) {
        s[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
        s[j + 4] = (uint8_t)((m[j] & 63) | ((m[j + 4] >> 4) << 6));
        s[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((m[j + 4] & 15) << 4));
    }
    uint8_t *qs = o + 16;
    for (int j = 0; j < 4; j++) {
        float dl0 = df * (float)sc[2 * j], ml0 = mf * (float)m[2 * j];
        float dl1 = df * (float)sc[2 * j + 1], ml1 = mf * (float)m[2 * j + 1];
        for (int l = 0; l < 32; l++) {
            float a = v[64 * j + l], b = v[64 * j + 32 + l];
            uint8_t qa = dl0 > 0.0f ? (uint8_t)clampf(std::round((a + ml0) / dl0), 0.0f, 15.0f) : 0;
            uint8_t qb = dl1 > 0.0f ? (uint8_t)clampf(std::round((b + ml1) / dl1), 0.0f, 15.0f) : 0;
            qs[32 * j + l] = (uint8_t)(qa | (qb << 4));
        }
    }
}

// Q6_K encoder (project's own; decoder dequantize_q6_k,
// rust/src/kernels/mod.rs:145-180).  Sub-block i of 16: scale_i = max|v|/31;
// d = max scale / 127 (f16); sc_i = round(scale_i / d);
// q = round(v / (d*sc_i)) in [-32, 31], stored as q + 32.
static void enc_q6_k(const float *v, uint8_t *o) {
    float scale[16], max_scale = 0.0f;
    for (int i = 0; i < 16; i++) {
        float a = 0.0f;
        for (int l = 0; l < 16; l++) {
            float t = std::fabs(v[16 * i + l]);
            if (t > a) a = t;
        }
        scale[i] = a / 31.0f;
        if (scale[i] > max_scale) max_scale = scale[i];
    }
    uint16_t d16 = float_to_half(max_scale / 127.0f);
    float df = half_to_float(d16);
    int8_t sc[16];
    for (int i = 0; i < 16; i++)
        sc[i] = df > 0.0f ? (int8_t)clampf(std::round(scale[i] / df), -128.0f, 127.0f) : 0;
    std::memset(o, 0, 210);
    uint8_t *ql = o, *qh = o + 128;
    for (int e = 0; e < 256; e++) {
        float step = df * (float)sc[e / 16];
        int qi = step != 0.0f ? (int)clampf(std::round(v[e] / step), -32.0f, 31.0f) : 0;
        uint8_t c = (uint8_t)(qi + 32);
        int n = e / 128, w = e % 128, s = w / 32, l = w % 32;
        uint8_t *lb = &ql[64 * n + l + 32 * (s & 1)];
        *lb |= (s < 2) ? (uint8_t)(c & 15) : (uint8_t)((c & 15) << 4);
        qh[32 * n + l] |= (uint8_t)((c >> 4) << (2 * s));
    }
    for (int i = 0; i < 16; i++) o[192 + i] = (uint8_t)sc[i];
    st_half(o + 208, d16);
}

template <class Fn>
static void parallel_for(int64_t n, Fn fn) {
    unsigned hw = std::thread::hardware_concurrency();
    int64_t nt = std::min<int64_t>(std::max(1u, std::min(hw, 16u)), n);
    if (nt <= 1 || n < 4096) {
        fn(0, n);
        return;
    }
    std::vector<std::thread> th;
    int64_t chunk = (n + nt - 1) / nt;
    for (int64_t t = 0; t < nt; t++) {
        int64_t a = t * chunk, b = std::min(n, a + chunk);
        if (a < b) th.emplace_back([=] { fn(a, b); });
    }
    for (auto &t : th) t.join();
}

static inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

// RPL64 repack of a GGUF Q4_K [rows, cols] matrix (rows % 64 == 0,
// cols % 256 == 0): per 64-row tile and 256-column super-block, the 144-byte
// blocks of the 64 rows are cut into nine 16-byte chunks and chunk c of all
// 64 rows is stored contiguously.  Same bytes, new order.
void repack_rpl64_q4k(const uint8_t *src, uint8_t *dst, int64_t rows, int64_t cols) {
    const int64_t NB = cols / 256, row_bytes = NB * 144;
    for (int64_t rt = 0; rt < rows / 64; rt++)
        for (int64_t kb = 0; kb < NB; kb++)
            for (int c = 0; c < 9; c++) {
                uint8_t *o = dst + ((rt * NB + kb) * 9 + c) * 1024;
                for (int r = 0; r < 64; r++)
                    std::memcpy(o + r * 16, src + (rt * 64 + r) * row_bytes + kb * 144 + c * 16, 16);
            }
}

// The 6-bit scales and mins of a Q4_K block's 12 packed bytes
// (get_scale_min_k4, rust/src/kernels/mod.rs:54-63), and the inverse.
static void unpack_scales_k4(const uint8_t *q, uint8_t sc[8], uint8_t m[8]) {
    for (int j = 0; j < 4; j++) {
        sc[j] = q[j] & 63;
        m[j] = q[j + 4] & 63;
    }
    for (int j = 4; j < 8; j++) {
        sc[j] = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        m[j] = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

static void pack_scales_k4(const uint8_t sc[8], const uint8_t m[8], uint8_t *q) {
    for (int j = 0; j < 4; j++) {
        q[j] = (uint8_t)(sc[j] | ((sc[j + 4] >> 4) << 6));
        q[j + 4] = (uint8_t)(m[j] | ((m[j + 4] >> 4) << 6));
        q[j + 8] = (uint8_t)((sc[j + 4] & 0xF) | ((m[j + 4] & 0xF) << 4));
    }
}

// Split repack of a GGUF Q4_K [rows, cols] matrix with cols an odd multiple
// of 128, whose 256-element blocks straddle rows: each row gets
// ceil(cols / 256) virtual super-blocks of its own columns 256 kb .. +255.
// A virtual block's halves (sub-blocks 0-3 and 4-7) are half blocks of the
// original (the first or second half of one block each; a half past the row
// end is zero).  Its header holds the first half's (d, dmin) and the eight
// (scale, min) pairs packed as in Q4_K; its qs are the halves' qs bytes (a
// half is two 32-byte pairs of qs); the second half's (d, dmin) goes to a
// 4-byte entry per row after the nine 1 KiB chunks of the RPL64 layout:
// 9,472 bytes per 64-row tile and virtual block.  The decoded values are the
// original ones, with zeros past the row end.
void repack_rpl64_q4k_split(const uint8_t *src, uint8_t *dst, int64_t rows, int64_t cols) {
    const int64_t NB = (cols + 255) / 256, tb = 9 * 1024 + 256;
    for (int64_t rt = 0; rt < rows / 64; rt++)
        for (int64_t kb = 0; kb < NB; kb++) {
            uint8_t *o = dst + (rt * NB + kb) * tb;
            for (int r = 0; r < 64; r++) {
                uint8_t vb[144] = {0}, db[4] = {0}, sc[8] = {0}, mm[8] = {0};
                for (int part = 0; part < 2; part++) {
                    const int64_t c0 = 256 * kb + 128 * part;
                    if (c0 >= cols) break;
                    const int64_t e = (rt * 64 + r) * cols + c0, half = (e % 256) / 128;
                    const uint8_t *blk = src + (e / 256) * 144;
                    uint8_t bs[8], bm[8];
                    unpack_scales_k4(blk + 4, bs, bm);
                    for (int k = 0; k < 4; k++) {
                        sc[4 * part + k] = bs[4 * half + k];
                        mm[4 * part + k] = bm[4 * half + k];
                    }
                    std::memcpy(vb + 16 + 64 * part, blk + 16 + 64 * half, 64);
                    std::memcpy(part ? db : vb, blk, 4);
                }
                pack_scales_k4(sc, mm, vb + 4);
                for (int c = 0; c < 9; c++) std::memcpy(o + c * 1024 + r * 16, vb + c * 16, 16);
                std::memcpy(o + 9 * 1024 + r * 4, db, 4);
            }
        }
}

// RPL64 repack of a GGUF Q8_0 [rows, cols] matrix (rows % 64 == 0,
// cols % 256 == 0): per 64-row tile and 256-column group (eight 34-byte
// blocks per row), chunk 0 holds each row's eight f16 d (16 bytes) and
// chunks 1-16 its 256 quants, 16 per chunk, each chunk's 64 rows
// contiguous: 17 KiB per tile and group.  Same bytes, new order.
void repack_rpl64_q8(const uint8_t *src, uint8_t *dst, int64_t rows, int64_t cols) {
    const int64_t NG = cols / 256, row_bytes = cols / 32 * 34;
    for (int64_t rt = 0; rt < rows / 64; rt++)
        for (int64_t g = 0; g < NG; g++) {
            uint8_t *o = dst + (rt * NG + g) * 17 * 1024;
            for (int r = 0; r < 64; r++) {
                const uint8_t *grp = src + (rt * 64 + r) * row_bytes + g * 8 * 34;
                for (int b = 0; b < 8; b++) {
                    std::memcpy(o + r * 16 + 2 * b, grp + 34 * b, 2);
                    std::memcpy(o + (1 + 2 * b) * 1024 + r * 16, grp + 34 * b + 2, 16);
                    std::memcpy(o + (2 + 2 * b) * 1024 + r * 16, grp + 34 * b + 18, 16);
                }
            }
        }
}

// RPL64 repack of a GGUF Q6_K [rows, cols] matrix (rows % 64 == 0,
// cols % 256 == 0): per 64-row tile and super-block, the 210-byte blocks of
// the 64 rows are cut into thirteen 16-byte chunks (ql: 0-7, qh: 8-11,
// scales: 12) stored chunk by chunk as for Q4_K, followed by the 64 rows'
// 2-byte d: 13,440 bytes per tile and super-block.  Same bytes, new order.
void repack_rpl64_q6k(const uint8_t *src, uint8_t *dst, int64_t rows, int64_t cols) {
    const int64_t NB = cols / 256, row_bytes = NB * 210, tb = 13 * 1024 + 128;
    for (int64_t rt = 0; rt < rows / 64; rt++)
        for (int64_t kb = 0; kb < NB; kb++) {
            uint8_t *o = dst + (rt * NB + kb) * tb;
            for (int r = 0; r < 64; r++) {
                const uint8_t *blk = src + (rt * 64 + r) * row_bytes + kb * 210;
                for (int c = 0; c < 13; c++) std::memcpy(o + c * 1024 + r * 16, blk + c * 16, 16);
                std::memcpy(o + 13 * 1024 + r * 2, blk + 208, 2);
            }
        }
}

}  // namespace lcmoe

extern "C" lcmoe_status lcmoe_quantize(int32_t type, const float *src, uint8_t *dst, int64_t count) {
    clear_error();
    if (!src || !dst || count < 0) return fail(LCMOE_ERR_INVALID_ARG, "null pointer or negative count");
    int64_t bs = block_size(type), bb = block_bytes(type);
    if (!bs) return fail(LCMOE_ERR_UNSUPPORTED, "quant type %d unsupported", type);
    if (count % bs) return fail(LCMOE_ERR_INVALID_ARG, "count %% %lld != 0", (long long)bs);
    if (type == LCMOE_TYPE_F32) {
        std::memcpy(dst, src, (size_t)count * 4);
        return LCMOE_OK;
    }
    void (*enc)(const float *, uint8_t *) =
        type == LCMOE_TYPE_Q8_0 ? enc_q8_0 : (type == LCMOE_TYPE_Q4_K ? enc_q4_k : enc_q6_k);
    parallel_for(count / bs, [&](int64_t a, int64_t b) {
        for (int64_t i = a; i < b; i++) enc(src + i * bs, dst + i * bb);
    });
    return LCMOE_OK;
}

extern "C" void lcmoe_synth_normal(uint64_t seed, uint64_t stream, float stddev, float *out, int64_t n) {
    if (!out || n <= 0) return;
    const uint64_t G = 0x9E3779B97F4A7C15ULL;
    uint64_t key = mix64(seed ^ mix64(stream + G));
    parallel_for((n + 1) / 2, [&](int64_t a, int64_t b) {
        for (int64_t j = a; j < b; j++) {
            uint64_t r1 = mix64(key + (uint64_t)(2 * j + 1) * G);
            uint64_t r2 = mix64(key + (uint64_t)(2 * j + 2) * G);
            double u1 = (double)((r1 >> 11) + 1) * 0x1.0p-53;
            double u2 = (double)(r2 >> 11) * 0x1.0p-53;
            double rad = std::sqrt(-2.0 * std::log(u1));
            double th = 6.283185307179586 * u2;
            out[2 * j] = (float)(rad * std::cos(th) * (double)stddev);
            if (2 * j + 1 < n) out[2 * j + 1] = (float)(rad * std::sin(th) * (double)stddev);
        }
    });
}
