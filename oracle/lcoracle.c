/*
 * lcoracle.c -- CPU oracle for the MoE feed-forward hot path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the product): see lcoracle.h
 * for who may load it and for the pinning status of each function.
 *
 * Build: oracle/Makefile (gcc, -O2 -mavx2 -mfma -ffp-contract=off -fopenmp).
 * -ffp-contract=off matters: every a*b+c below that is not an explicit fmaf /
 * _mm256_fmadd_ps is two roundings, exactly as the Rust reference computes it.
 */
#include "lcoracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#if defined(__AVX2__) && defined(__FMA__)
#include <immintrin.h>
#define LCO_HAVE_AVX2 1
#endif
#ifdef _OPENMP
#include <omp.h>
#endif

/* ====================================================================== */
/* f16 <-> f32 (crate `half` 2.7.1 semantics: exact widening, RNE narrowing). */
/* Used by every reference decoder: kernels/mod.rs:24, :45, :72-73, :154.    */
/* ====================================================================== */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float lco_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0) {
        if (m == 0) return u2f(sign);
        int sh = 0;
        while (!(m & 0x400u)) { m <<= 1; sh++; }
        m &= 0x3ffu;
        return u2f(sign | ((uint32_t)(113 - sh) << 23) | (m << 13));
    }
    if (e == 31) return u2f(sign | 0x7f800000u | (m << 13));
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

uint16_t lco_f32_to_f16(float f) {
    uint32_t x = f2u(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 -> inf */
    if (ax < 0x38800000u) {                                      /* f16 subnormal / 0 */
        if (ax < 0x33000000u) return sign;                       /* < 2^-25 -> 0 */
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

void lco_f16_to_f32_n(const uint16_t *h, float *f, size_t n) {
    for (size_t i = 0; i < n; i++) f[i] = lco_f16_to_f32(h[i]);
}
void lco_f32_to_f16_n(const float *f, uint16_t *h, size_t n) {
    for (size_t i = 0; i < n; i++) h[i] = lco_f32_to_f16(f[i]);
}

static inline float ld_f16(const uint8_t *p) { return lco_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }
static inline void st_f16(uint8_t *p, uint16_t h) { p[0] = (uint8_t)(h & 0xff); p[1] = (uint8_t)(h >> 8); }

/* ====================================================================== */
/* Block geometry: QuantType::block_size / block_bytes / tensor_size       */
/* (rust/src/model/quant.rs:170-183, :186-239, :256-261).                   */
/* ====================================================================== */

size_t lco_block_size(int type) {
    switch (type) {
    case LCO_F32: case LCO_F16: return 1;
    case LCO_Q8_0: return 32;
    case LCO_Q4_K: case LCO_Q6_K: return 256;
    default: return 0;
    }
}
size_t lco_block_bytes(int type) {
    switch (type) {
    case LCO_F32: return 4;
    case LCO_F16: return 2;
    case LCO_Q8_0: return 34;
    case LCO_Q4_K: return 144;
    case LCO_Q6_K: return 210;
    default: return 0;
    }
}
size_t lco_tensor_size(int type, size_t count) {
    size_t bs = lco_block_size(type), bb = lco_block_bytes(type);
    if (!bs) return 0;
    return (count + bs - 1) / bs * bb;
}

/* ====================================================================== */
/* Decoders                                                                  */
/* ====================================================================== */

/* dequantize_q8_0, rust/src/kernels/mod.rs:37-51: v = (int8)q * d. */
void lco_dequant_q8_0(const uint8_t *src, float *dst, size_t count) {
    size_t nb = count / 32;
    for (size_t i = 0; i < nb; i++) {
        const uint8_t *b = src + i * 34;
        float scale = ld_f16(b);
        for (int j = 0; j < 32; j++) dst[i * 32 + j] = (float)(int8_t)b[2 + j] * scale;
    }
}

/* get_scale_min_k4, rust/src/kernels/mod.rs:54-63. */
void lco_scale_min_k4(int j, const uint8_t *q, uint8_t *sc, uint8_t *m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* dequantize_q4_k, rust/src/kernels/mod.rs:66-98.  Decodes the flattened
 * buffer (num_blocks = count / 256), so rows that straddle super-blocks
 * (d_ff = 1408) decode exactly as the reference decodes them. */
void lco_dequant_q4_k(const uint8_t *src, float *dst, size_t count) {
    size_t nb = count / 256;
    for (size_t i = 0; i < nb; i++) {
        const uint8_t *b = src + i * 144;
        float d = ld_f16(b), dmin = ld_f16(b + 2);
        const uint8_t *scales = b + 4, *qs = b + 16;
        float *o = dst + i * 256;
        for (int j = 0; j < 4; j++) {
            uint8_t sc1, m1, sc2, m2;
            lco_scale_min_k4(2 * j, scales, &sc1, &m1);
            lco_scale_min_k4(2 * j + 1, scales, &sc2, &m2);
            float dl1 = d * (float)sc1, dl2 = d * (float)sc2;
            float ml1 = dmin * (float)m1, ml2 = dmin * (float)m2;
            for (int l = 0; l < 32; l++) {
                o[64 * j + l] = dl1 * (float)(qs[32 * j + l] & 0x0F) - ml1;
                o[64 * j + l + 32] = dl2 * (float)(qs[32 * j + l] >> 4) - ml2;
            }
        }
    }
}

/* dequantize_q6_k, rust/src/kernels/mod.rs:145-180. */
void lco_dequant_q6_k(const uint8_t *src, float *dst, size_t count) {
    size_t nb = count / 256;
    for (size_t i = 0; i < nb; i++) {
        const uint8_t *b = src + i * 210;
        const uint8_t *ql = b, *qh = b + 128;
        const int8_t *sc = (const int8_t *)(b + 192);
        float d = ld_f16(b + 208);
        float *o = dst + i * 256;
        for (int n = 0; n < 2; n++) {
            const uint8_t *l8 = ql + 64 * n, *h8 = qh + 32 * n;
            const int8_t *s8 = sc + 8 * n;
            for (int l = 0; l < 32; l++) {
                int is = l / 16;
                int q1 = (int)((l8[l] & 0xF) | (((h8[l] >> 0) & 3) << 4)) - 32;
                int q2 = (int)((l8[l + 32] & 0xF) | (((h8[l] >> 2) & 3) << 4)) - 32;
                int q3 = (int)((l8[l] >> 4) | (((h8[l] >> 4) & 3) << 4)) - 32;
                int q4 = (int)((l8[l + 32] >> 4) | (((h8[l] >> 6) & 3) << 4)) - 32;
                o[128 * n + l + 0] = d * (float)s8[is + 0] * (float)q1;
                o[128 * n + l + 32] = d * (float)s8[is + 2] * (float)q2;
                o[128 * n + l + 64] = d * (float)s8[is + 4] * (float)q3;
                o[128 * n + l + 96] = d * (float)s8[is + 6] * (float)q4;
            }
        }
    }
}

/* GGUFModel::dequantize dispatch, rust/src/model/loader.rs:205-235. */
int lco_dequant(int type, const uint8_t *src, float *dst, size_t count) {
    switch (type) {
    case LCO_F32: memcpy(dst, src, count * 4); return 0;
    case LCO_F16:
        for (size_t i = 0; i < count; i++) dst[i] = ld_f16(src + 2 * i);
        return 0;
    case LCO_Q8_0: lco_dequant_q8_0(src, dst, count); return 0;
    case LCO_Q4_K: lco_dequant_q4_k(src, dst, count); return 0;
    case LCO_Q6_K: lco_dequant_q6_k(src, dst, count); return 0;
    default: return -1;
    }
}

/* sanitize_weights, rust/src/model/loader.rs:241-249 (threshold 100). */
void lco_sanitize(float *v, size_t n) {
    for (size_t i = 0; i < n; i++)
        if (isnan(v[i]) || isinf(v[i]) || fabsf(v[i]) > 100.0f) v[i] = 0.0f;
}

/* scan_for_corruption's per-block test, rust/src/model/loader.rs:301-422:
 * d (and dmin where present) non-finite or |.| > 1e4 marks the block bad.
 * Q6_K keeps d in bytes 208..209; Q8_0/Q4_K keep d at 0..1; Q4_K also has
 * dmin at 2..3.  Deliberate deviation: the reference also reads bytes 2..3
 * of a Q8_0 block as "dmin" (loader.rs:374-382), but there they are the
 * first two int8 quants, so valid Q8_0 data (e.g. qs[1] in -4..-1) would be
 * flagged; only real scale fields are checked here. */
size_t lco_scan_blocks(int type, const uint8_t *src, size_t count) {
    size_t bs = lco_block_size(type), bb = lco_block_bytes(type);
    if (type == LCO_F32 || type == LCO_F16 || !bs) return 0;
    size_t nb = (count + bs - 1) / bs, bad = 0;
    for (size_t i = 0; i < nb; i++) {
        const uint8_t *b = src + i * bb;
        float d, dmin = 0.0f;
        int has_dmin = 0;
        if (type == LCO_Q6_K) {
            d = ld_f16(b + 208);
        } else {
            d = ld_f16(b);
            if (type == LCO_Q4_K) {
                dmin = ld_f16(b + 2);
                has_dmin = 1;
            }
        }
        int is_bad = isnan(d) || isinf(d) || fabsf(d) > 1e4f;
        if (has_dmin && (isnan(dmin) || isinf(dmin) || fabsf(dmin) > 1e4f)) is_bad = 1;
        bad += (size_t)is_bad;
    }
    return bad;
}

/* ====================================================================== */
/* Encoders                                                                  */
/* ====================================================================== */

/* Rust f32::max: returns the non-NaN argument when one is NaN. */
static inline float rust_fmax(float a, float b) {
    if (isnan(a)) return b;
    if (isnan(b)) return a;
    return a > b ? a : b;
}
/* Rust `f as i8` after clamp: NaN -> 0. */
static inline int8_t rust_to_i8(float v) {
    if (isnan(v)) return 0;
    if (v >= 127.0f) return 127;
    if (v <= -128.0f) return -128;
    return (int8_t)v;
}

/* quantize_f32_to_q8_0, rust/src/kernels/q8_0.rs:90-122:
 * scale = max|v| / 127 (f32), stored as f16 (RNE); q = round_half_away(v /
 * scale) clamped to +-127, divided by the f32 scale, not the stored f16. */
void lco_quantize_q8_0(const float *src, uint8_t *dst, size_t count) {
    size_t nb = count / 32;
    for (size_t b = 0; b < nb; b++) {
        const float *v = src + b * 32;
        uint8_t *o = dst + b * 34;
        float max_abs = 0.0f;
        for (int i = 0; i < 32; i++) max_abs = rust_fmax(max_abs, fabsf(v[i]));
        float scale = max_abs > 0.0f ? max_abs / 127.0f : 0.0f;
        st_f16(o, lco_f32_to_f16(scale));
        for (int i = 0; i < 32; i++) {
            int8_t q = 0;
            if (scale > 0.0f) {
                float r = roundf(v[i] / scale);
                r = r < -127.0f ? -127.0f : (r > 127.0f ? 127.0f : r);
                q = rust_to_i8(r);
            }
            o[2 + i] = (uint8_t)q;
        }
    }
}

static inline float clampf(float v, float lo, float hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* Q4_K encoder.  The reference has none; this one is the project's own and
 * its bytes are the synthetic-data contract.  Per 32-element sub-block j:
 * lo = min(0, min v), hi = max v, scale_j = (hi - lo) / 15, min_j = -lo.
 * Super-block d = max scale_j / 63 and dmin = max min_j / 63, stored f16.
 * sc_j = round(scale_j / d), m_j = round(min_j / dmin) in [0, 63];
 * q = round((v + dmin*m_j) / (d*sc_j)) in [0, 15].  Packing is the inverse
 * of get_scale_min_k4 (kernels/mod.rs:54-63) and the qs order of
 * dequantize_q4_k (kernels/mod.rs:86-93). */
void lco_quantize_q4_k(const float *src, uint8_t *dst, size_t count) {
    size_t nb = count / 256;
    for (size_t ib = 0; ib < nb; ib++) {
        const float *v = src + ib * 256;
        uint8_t *o = dst + ib * 144;
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
        uint16_t d16 = lco_f32_to_f16(max_scale / 63.0f);
        uint16_t m16 = lco_f32_to_f16(max_min / 63.0f);
        float df = lco_f16_to_f32(d16), mf = lco_f16_to_f32(m16);
        uint8_t sc[8], m[8];
        for (int j = 0; j < 8; j++) {
            sc[j] = df > 0.0f ? (uint8_t)clampf(roundf(scale[j] / df), 0.0f, 63.0f) : 0;
            m[j] = mf > 0.0f ? (uint8_t)clampf(roundf(mn[j] / mf), 0.0f, 63.0f) : 0;
        }
        st_f16(o, d16);
        st_f16(o + 2, m16);
        uint8_t *s = o + 4;
        for (int j = 0; j < 4; j++) {
            s[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
            s[j + 4] = (uint8_t)((m[j] & 63) | ((m[j + 4] >> 4) << 6));
            s[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((m[j + 4] & 15) << 4));
        }
        uint8_t q[256];
        for (int j = 0; j < 8; j++) {
            float dl = df * (float)sc[j], ml = mf * (float)m[j];
            for (int l = 0; l < 32; l++) {
                float t = v[32 * j + l];
                q[32 * j + l] = dl > 0.0f ? (uint8_t)clampf(roundf((t + ml) / dl), 0.0f, 15.0f) : 0;
            }
        }
        uint8_t *qs = o + 16;
        for (int j = 0; j < 4; j++)
            for (int l = 0; l < 32; l++)
                qs[32 * j + l] = (uint8_t)(q[64 * j + l] | (q[64 * j + 32 + l] << 4));
    }
}

/* Q6_K encoder (project's own; the reference has none).  Per 16-element
 * sub-block i: scale_i = max|v| / 31; super-block d = max scale_i / 127
 * (f16); sc_i = round(scale_i / d) in [-128, 127];
 * q = round(v / (d*sc_i)) in [-32, 31], stored as q+32 in the ql/qh layout
 * that dequantize_q6_k (kernels/mod.rs:145-180) reads. */
void lco_quantize_q6_k(const float *src, uint8_t *dst, size_t count) {
    size_t nb = count / 256;
    for (size_t ib = 0; ib < nb; ib++) {
        const float *v = src + ib * 256;
        uint8_t *o = dst + ib * 210;
        float scale[16], max_scale = 0.0f;
        for (int i = 0; i < 16; i++) {
            float a = 0.0f;
            for (int l = 0; l < 16; l++) {
                float t = fabsf(v[16 * i + l]);
                if (t > a) a = t;
            }
            scale[i] = a / 31.0f;
            if (scale[i] > max_scale) max_scale = scale[i];
        }
        uint16_t d16 = lco_f32_to_f16(max_scale / 127.0f);
        float df = lco_f16_to_f32(d16);
        int8_t sc[16];
        for (int i = 0; i < 16; i++)
            sc[i] = df > 0.0f ? (int8_t)clampf(roundf(scale[i] / df), -128.0f, 127.0f) : 0;
        uint8_t q[256];
        for (int e = 0; e < 256; e++) {
            float step = df * (float)sc[e / 16];
            int qi = step != 0.0f ? (int)clampf(roundf(v[e] / step), -32.0f, 31.0f) : 0;
            q[e] = (uint8_t)(qi + 32);
        }
        uint8_t *ql = o, *qh = o + 128;
        memset(o, 0, 210);
        for (int e = 0; e < 256; e++) {
            int n = e / 128, w = e % 128, s = w / 32, l = w % 32;
            uint8_t *lb = &ql[64 * n + l + 32 * (s & 1)];
            if (s < 2) *lb |= (uint8_t)(q[e] & 15);
            else *lb |= (uint8_t)((q[e] & 15) << 4);
            qh[32 * n + l] |= (uint8_t)((q[e] >> 4) << (2 * s));
        }
        for (int i = 0; i < 16; i++) o[192 + i] = (uint8_t)sc[i];
        st_f16(o + 208, d16);
    }
}

int lco_quantize(int type, const float *src, uint8_t *dst, size_t count) {
    switch (type) {
    case LCO_F32: memcpy(dst, src, count * 4); return 0;
    case LCO_Q8_0: lco_quantize_q8_0(src, dst, count); return 0;
    case LCO_Q4_K: lco_quantize_q4_k(src, dst, count); return 0;
    case LCO_Q6_K: lco_quantize_q6_k(src, dst, count); return 0;
    default: return -1;
    }
}

/* ====================================================================== */
/* Synthetic data: counter-based splitmix64 + Box-Muller (float64).          */
/* ====================================================================== */

static inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

/* Element i of stream (seed, stream) is a deterministic function of
 * (seed, stream, i) alone, so any slice can be generated independently. */
void lco_synth_normal(uint64_t seed, uint64_t stream, float stddev, float *out, size_t n) {
    const uint64_t G = 0x9E3779B97F4A7C15ULL;
    uint64_t key = mix64(seed ^ mix64(stream + G));
    long long np = (long long)((n + 1) / 2);
#pragma omp parallel for schedule(static)
    for (long long j = 0; j < np; j++) {
        uint64_t r1 = mix64(key + (uint64_t)(2 * j + 1) * G);
        uint64_t r2 = mix64(key + (uint64_t)(2 * j + 2) * G);
        double u1 = (double)((r1 >> 11) + 1) * 0x1.0p-53;
        double u2 = (double)(r2 >> 11) * 0x1.0p-53;
        double rad = sqrt(-2.0 * log(u1));
        double th = 6.283185307179586 * u2;
        out[2 * j] = (float)(rad * cos(th) * (double)stddev);
        if ((size_t)(2 * j + 1) < n) out[2 * j + 1] = (float)(rad * sin(th) * (double)stddev);
    }
}

/* ====================================================================== */
/* f32 GEMM in the reference's accumulation order.                          */
/* avx2_matmul, rust/src/kernels/simd.rs:226-249: for each row i and each     */
/* 8-column block, acc = fma(a[i,l], b[l, j..j+8], acc) over ascending l      */
/* starting from 0; columns n - n%8 .. n are a scalar tail with sum +=        */
/* a*b as two roundings.  simd_matmul_par_avx2 (:298-311) splits rows         */
/* recursively down to <= 4 rows per task; that changes no arithmetic.        */
/* ====================================================================== */

static void mm_block(const float *a, const float *b, float *c, int m, int k, int n, int j0, int j1) {
    /* columns [j0, j1) of the FMA region (multiples of 8) */
    for (int i = 0; i < m; i++) {
        const float *ar = a + (size_t)i * k;
        for (int j = j0; j < j1; j += 8) {
#ifdef LCO_HAVE_AVX2
            __m256 acc = _mm256_setzero_ps();
            for (int l = 0; l < k; l++)
                acc = _mm256_fmadd_ps(_mm256_set1_ps(ar[l]), _mm256_loadu_ps(b + (size_t)l * n + j), acc);
            _mm256_storeu_ps(c + (size_t)i * n + j, acc);
#else
            float acc[8] = {0};
            for (int l = 0; l < k; l++)
                for (int q = 0; q < 8; q++) acc[q] = fmaf(ar[l], b[(size_t)l * n + j + q], acc[q]);
            memcpy(c + (size_t)i * n + j, acc, sizeof acc);
#endif
        }
    }
}

static void mm_tail(const float *a, const float *b, float *c, int m, int k, int n, int j0) {
    for (int i = 0; i < m; i++)
        for (int j = j0; j < n; j++) {
            float sum = 0.0f;
            for (int l = 0; l < k; l++) {
                float p = a[(size_t)i * k + l] * b[(size_t)l * n + j];
                sum = sum + p;
            }
            c[(size_t)i * n + j] = sum;
        }
}

static void mm_rows(const float *a, const float *b, float *c, int m, int k, int n) {
    int n8 = n & ~7;
    mm_block(a, b, c, m, k, n, 0, n8);
    mm_tail(a, b, c, m, k, n, n8);
}

/* leaves of the rayon recursion (m <= 4 rows each) */
static int row_leaves(int r0, int m, int *starts, int *lens, int cnt) {
    if (m <= 4) { starts[cnt] = r0; lens[cnt] = m; return cnt + 1; }
    int mid = m / 2;
    cnt = row_leaves(r0, mid, starts, lens, cnt);
    return row_leaves(r0 + mid, m - mid, starts, lens, cnt);
}

/* threads <= 0: reference-faithful row split (rayon, >= 1 leaf per <= 4 rows,
 * single-threaded below 4096 outputs as CpuBackend::matmul, cpu.rs:13-23).
 * threads >= 1: the same per-element arithmetic split over column blocks
 * across `threads` threads (the "all-cores" CPU baseline). */
void lco_matmul(const float *a, const float *b, float *c, int m, int k, int n, int threads) {
    if (m <= 0 || n <= 0) return;
    if (threads <= 0) {
        if ((long long)m * n < 4096 || m <= 4) { mm_rows(a, b, c, m, k, n); return; }
        int cap = m / 2 + 2;
        int *st = (int *)malloc(sizeof(int) * cap * 2), *ln = st + cap;
        int nl = row_leaves(0, m, st, ln, 0);
#pragma omp parallel for schedule(dynamic, 1)
        for (int q = 0; q < nl; q++)
            mm_rows(a + (size_t)st[q] * k, b, c + (size_t)st[q] * n, ln[q], k, n);
        free(st);
        return;
    }
    int n8 = n & ~7, nblk = n8 / 8;
    if (threads == 1 || nblk < 2) { mm_rows(a, b, c, m, k, n); return; }
#pragma omp parallel for schedule(static) num_threads(threads)
    for (int q = 0; q < nblk; q++) mm_block(a, b, c, m, k, n, 8 * q, 8 * q + 8);
    mm_tail(a, b, c, m, k, n, n8);
}

/* Tensor::transpose (rust/src/model/tensor.rs:175-188): b[c][r] = a[r][c].
 * Tiled only for cache behaviour; a pure data movement. */
void lco_transpose(const float *a, float *b, int rows, int cols) {
    const int TB = 32;
#pragma omp parallel for schedule(static) if ((long long)rows * cols > (1 << 20))
    for (int r0 = 0; r0 < rows; r0 += TB)
        for (int c0 = 0; c0 < cols; c0 += TB)
            for (int r = r0; r < r0 + TB && r < rows; r++)
                for (int c = c0; c < c0 + TB && c < cols; c++)
                    b[(size_t)c * rows + r] = a[(size_t)r * cols + c];
}

/* CpuBackend::silu, rust/src/backend/cpu.rs:62-64: v * (1 / (1 + exp(-v))). */
float lco_silu(float v) { return v * (1.0f / (1.0f + expf(-v))); }

/* CpuBackend::rms_norm, rust/src/backend/cpu.rs:49-60, on the x86_64 SIMD
 * paths it calls: simd_sum_sq (rust/src/kernels/simd.rs:390-409) keeps four
 * lane sums, lane j adding x[i]*x[i] (multiply, then add) for i = j, j+4,
 * ... up to the last full group of four; the lanes are summed in order from
 * 0.0 (Iterator::sum) and the remaining elements added one by one.
 * mean_sq = sum / hidden; scale = 1 / sqrt(mean_sq + eps); then
 * simd_vec_scale_mul (simd.rs:353-369) writes (x[i] * scale) * w[i]. */
void lco_rms_norm(const float *x, const float *w, float eps, int T, int d, float *out) {
    for (int t = 0; t < T; t++) {
        const float *r = x + (size_t)t * d;
        float lane[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        int i = 0;
        for (; i + 4 <= d; i += 4)
            for (int j = 0; j < 4; j++) {
                const float p = r[i + j] * r[i + j];
                lane[j] = p + lane[j];
            }
        float sum = 0.0f;
        for (int j = 0; j < 4; j++) sum = sum + lane[j];
        for (; i < d; i++) {
            const float p = r[i] * r[i];
            sum = sum + p;
        }
        const float mean_sq = sum / (float)d;
        const float scale = 1.0f / sqrtf(mean_sq + eps);
        for (int k = 0; k < d; k++) {
            const float a = r[k] * scale;
            out[(size_t)t * d + k] = a * w[k];
        }
    }
}

/* CpuBackend::softmax, rust/src/backend/cpu.rs:66-79 (one row): max folded
 * from -inf with f32::max, sum of exp(x - max) in order, then divide. */
void lco_softmax(const float *x, float *y, int n) {
    float mx = -INFINITY;
    for (int i = 0; i < n; i++) mx = rust_fmax(mx, x[i]);
    float s = 0.0f;
    for (int i = 0; i < n; i++) s = s + expf(x[i] - mx);
    for (int i = 0; i < n; i++) y[i] = expf(x[i] - mx) / s;
}

/* exp for the sigmoid router, written so that the host and the device
 * evaluate it to the same bits: Cody-Waite range reduction (Cody & Waite,
 * "Software Manual for the Elementary Functions", 1980) with the fdlibm
 * two-part ln2, then the degree-7 Taylor polynomial of e^r on |r| <= ln2/2
 * in Horner form with fused multiply-adds, then exact scaling by 2^k.
 * Only IEEE basic operations and fma are used.  Error <= 2 ulp. */
float lco_expf_cw(float x) {
    if (isnan(x)) return x;
    if (x > 88.7228394f) return INFINITY;
    if (x < -103.972084f) return 0.0f;
    const float shifter = 12582912.0f; /* 1.5 * 2^23 */
    float kf = fmaf(x, 1.44269502f, shifter) - shifter;
    float r = fmaf(-kf, 0.693145751953125f, x);
    r = fmaf(-kf, 1.42860677e-06f, r);
    float p = 1.98412701e-04f;             /* 1/5040 */
    p = fmaf(p, r, 1.38888892e-03f);       /* 1/720  */
    p = fmaf(p, r, 8.33333377e-03f);       /* 1/120  */
    p = fmaf(p, r, 4.16666679e-02f);       /* 1/24   */
    p = fmaf(p, r, 1.66666672e-01f);       /* 1/6    */
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    int k = (int)kf;
    if (k < -125) { p = p * 5.42101086e-20f; k += 64; } /* * 2^-64, exact */
    if (k > 127) { p = p * 2.0f; k -= 1; }
    return p * u2f((uint32_t)(k + 127) << 23);
}

float lco_sigmoid_cw(float x) { return 1.0f / (1.0f + lco_expf_cw(-x)); }

/* The largest dip of lco_sigmoid_cw below its running maximum, in units in
 * the last place: max over x <= y of bits(s(x)) - bits(s(y)) (s >= 0, so
 * bit patterns order as values), over every non-NaN float taken in
 * increasing order, -inf .. -0, +0 .. +inf.  A certified router may treat
 * the function as monotone within this many ulps.  The ordered inputs are
 * cut into chunks; a dip across chunks is the maximum before a chunk minus
 * a value inside it. */
#define LCO_NFLOAT 4278190082ull /* 2 * (0x7f800000 + 1) */
static float lco_ordered_float(uint64_t n) {
    return n <= 0x7f800000ull ? u2f((uint32_t)(0xff800000ull - n))
                              : u2f((uint32_t)(n - 0x7f800001ull));
}
int64_t lco_sigmoid_max_dip(int threads) {
    enum { NCH = 256 };
    static uint32_t cmax[NCH], cmin[NCH];
    static int64_t cdip[NCH];
    if (threads < 1) threads = 1;
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads)
    for (int c = 0; c < NCH; c++) {
        const uint64_t n0 = LCO_NFLOAT * (uint64_t)c / NCH, n1 = LCO_NFLOAT * (uint64_t)(c + 1) / NCH;
        uint32_t run = 0, mn = 0xffffffffu;
        int64_t dip = 0;
        for (uint64_t n = n0; n < n1; n++) {
            const uint32_t b = f2u(lco_sigmoid_cw(lco_ordered_float(n)));
            if (b > run) run = b;
            if (b < mn) mn = b;
            if ((int64_t)run - (int64_t)b > dip) dip = (int64_t)run - (int64_t)b;
        }
        cmax[c] = run;
        cmin[c] = mn;
        cdip[c] = dip;
    }
    int64_t dip = 0;
    uint32_t before = 0;
    for (int c = 0; c < NCH; c++) {
        if (cdip[c] > dip) dip = cdip[c];
        if ((int64_t)before - (int64_t)cmin[c] > dip) dip = (int64_t)before - (int64_t)cmin[c];
        if (cmax[c] > before) before = cmax[c];
    }
    return dip;
}

/* ====================================================================== */
/* Routing.  The reference has no router; the rules below are this          */
/* project's written semantics (router logits reuse Tensor::matmul,          */
/* tensor.rs:107-135, so they follow the avx2_matmul order above).           */
/* ====================================================================== */

void lco_router_logits(const float *x, const float *w, float *l, int T, int d, int E) {
    mm_rows(x, w, l, T, d, E);
}

/* a beats b: larger value, NaN treated as -inf, ties -> lower index. */
static inline int beats(float za, int a, float zb, int b) {
    if (isnan(za)) za = -INFINITY;
    if (isnan(zb)) zb = -INFINITY;
    return za > zb || (za == zb && a < b);
}

/* select the K best of z[0..n) among allowed[] (NULL = all) in rank order */
static void topk_select(const float *z, int n, const unsigned char *allowed, int K, int *out) {
    unsigned char *used = (unsigned char *)calloc((size_t)n, 1);
    for (int s = 0; s < K; s++) {
        int best = -1;
        for (int e = 0; e < n; e++) {
            if (used[e] || (allowed && !allowed[e])) continue;
            if (best < 0 || beats(z[e], e, z[best], best)) best = e;
        }
        out[s] = best;
        if (best >= 0) used[best] = 1;
    }
    free(used);
}

int lco_route(const lco_desc *desc, const float *logits, const float *bias, int T,
              int32_t *topk_idx, float *topk_w) {
    int E = desc->n_expert, K = desc->n_expert_used;
    if (K <= 0 || K > E) return -1;
    float *z = (float *)malloc(sizeof(float) * E * 3);
    float *s = z + E, *p = z + 2 * E;
    int *sel = (int *)malloc(sizeof(int) * (E + 1));
    for (int t = 0; t < T; t++) {
        const float *l = logits + (size_t)t * E;
        if (desc->route_kind == LCO_ROUTE_SIGMOID_GROUP) {
            int G = desc->n_group, TG = desc->topk_group, gs = E / G;
            for (int e = 0; e < E; e++) {
                s[e] = lco_sigmoid_cw(l[e]);
                z[e] = (desc->has_bias && bias) ? s[e] + bias[e] : s[e];
            }
            float *gsc = (float *)malloc(sizeof(float) * G);
            for (int g = 0; g < G; g++) {
                int two[2];
                topk_select(z + g * gs, gs, NULL, gs >= 2 ? 2 : 1, two);
                gsc[g] = gs >= 2 ? z[g * gs + two[0]] + z[g * gs + two[1]] : z[g * gs + two[0]];
            }
            int *gk = (int *)malloc(sizeof(int) * TG);
            topk_select(gsc, G, NULL, TG, gk);
            unsigned char *allowed = (unsigned char *)calloc((size_t)E, 1);
            for (int i = 0; i < TG; i++)
                for (int e = 0; e < gs; e++) allowed[gk[i] * gs + e] = 1;
            topk_select(z, E, allowed, K, sel);
            float sum = 0.0f;
            for (int k = 0; k < K; k++) sum = sum + s[sel[k]];
            for (int k = 0; k < K; k++) {
                topk_idx[(size_t)t * K + k] = sel[k];
                topk_w[(size_t)t * K + k] = (s[sel[k]] / sum) * desc->routed_scale;
            }
            free(gsc); free(gk); free(allowed);
        } else {
            for (int e = 0; e < E; e++) z[e] = (desc->has_bias && bias) ? l[e] + bias[e] : l[e];
            topk_select(z, E, NULL, K, sel);
            if (desc->route_kind == LCO_ROUTE_SOFTMAX_RENORM) {
                float zs[256 + 8], ws[256 + 8];
                for (int k = 0; k < K; k++) zs[k] = z[sel[k]];
                lco_softmax(zs, ws, K);
                for (int k = 0; k < K; k++) p[k] = ws[k];
            } else {
                float *full = (float *)malloc(sizeof(float) * E);
                lco_softmax(z, full, E);
                for (int k = 0; k < K; k++) p[k] = full[sel[k]];
                free(full);
            }
            for (int k = 0; k < K; k++) {
                topk_idx[(size_t)t * K + k] = sel[k];
                topk_w[(size_t)t * K + k] = p[k] * desc->routed_scale;
            }
        }
    }
    free(z);
    free(sel);
    return 0;
}

/* Stable counting sort of assignments a = t*K + k by expert. */
int lco_dispatch(const int32_t *topk_idx, int T, int K, int E, int32_t *counts,
                 int32_t *offsets, int32_t *perm, int32_t *inv) {
    int A = T * K;
    if (E <= 0 || T < 0 || K <= 0) return -1;
    for (int e = 0; e < E; e++) counts[e] = 0;
    for (int a = 0; a < A; a++) {
        int e = topk_idx[a];
        if (e < 0 || e >= E) return -1;
        counts[e]++;
    }
    offsets[0] = 0;
    for (int e = 0; e < E; e++) offsets[e + 1] = offsets[e] + counts[e];
    int32_t *fill = (int32_t *)calloc((size_t)E, sizeof(int32_t));
    for (int a = 0; a < A; a++) {
        int e = topk_idx[a];
        int pos = offsets[e] + fill[e]++;
        perm[pos] = a;
        inv[a] = pos;
    }
    free(fill);
    return 0;
}

/* ====================================================================== */
/* Expert FFN and the whole layer.                                           */
/* ====================================================================== */

/* ffn_forward, rust/src/inference/engine.rs:146-164, on post-load weights
 * wg_t/wu_t [d, F] and wd_t [F, d]. */
void lco_ffn_dense(const float *x, int m, int d, int F, const float *wg_t,
                   const float *wu_t, const float *wd_t, float *y, int threads) {
    float *g = (float *)malloc(sizeof(float) * (size_t)m * F * 2);
    float *u = g + (size_t)m * F;
    lco_matmul(x, wg_t, g, m, d, F, threads);
    lco_matmul(x, wu_t, u, m, d, F, threads);
    for (size_t i = 0; i < (size_t)m * F; i++) g[i] = lco_silu(g[i]) * u[i];
    lco_matmul(g, wd_t, y, m, F, d, threads);
    free(g);
}

/* load_layer's per-tensor ingest, rust/src/model/loader.rs:145-168:
 * GGUF ne=[cols, rows] -> shape [rows, cols] -> dequantize -> transpose to
 * [cols, rows] -> sanitize. */
static float *ingest(int type, const uint8_t *bytes, int rows, int cols) {
    size_t n = (size_t)rows * cols;
    float *tmp = (float *)malloc(sizeof(float) * n * 2), *out = tmp + n;
    lco_dequant(type, bytes, tmp, n);
    lco_transpose(tmp, out, rows, cols);
    lco_sanitize(out, n);
    memmove(tmp, out, sizeof(float) * n);
    return (float *)realloc(tmp, sizeof(float) * n);
}

/* The router and bias as load_layer ingests them (loader.rs:161: every
 * layer tensor is sanitised, :241-249); NULL in, NULL out. */
static float *ingest_f32(const float *v, size_t n) {
    if (!v) return NULL;
    float *o = (float *)malloc(sizeof(float) * (n ? n : 1));
    memcpy(o, v, sizeof(float) * n);
    lco_sanitize(o, n);
    return o;
}

static int desc_ok(const lco_desc *d) {
    if (d->d_model <= 0 || d->d_ff <= 0 || d->n_expert <= 0 || d->n_expert_used <= 0) return 0;
    if (d->n_expert_used > d->n_expert || d->n_expert > 256 || d->n_expert_used > 16) return 0;
    if (d->n_shared < 0 || (d->n_shared > 0 && d->d_ff_shared <= 0)) return 0;
    if (d->route_kind == LCO_ROUTE_SIGMOID_GROUP &&
        (d->n_group <= 0 || d->n_expert % d->n_group || d->topk_group <= 0 || d->topk_group > d->n_group))
        return 0;
    return 1;
}

static void combine(const lco_desc *desc, int T, const float *Y, const float *Ysh,
                    const int32_t *inv, const float *topk_w, float *y) {
    int K = desc->n_expert_used, D = desc->d_model, S = desc->n_shared;
    for (int t = 0; t < T; t++)
        for (int c = 0; c < D; c++) {
            float acc = 0.0f;
            for (int k = 0; k < K; k++) {
                float p = topk_w[(size_t)t * K + k] * Y[(size_t)inv[(size_t)t * K + k] * D + c];
                acc = acc + p;
            }
            for (int s = 0; s < S; s++) acc = acc + Ysh[((size_t)s * T + t) * D + c];
            y[(size_t)t * D + c] = acc;
        }
}

int lco_moe_forward(const lco_desc *desc, const lco_weights *w, const float *x, int T,
                    float *y, int32_t *topk_idx_o, float *topk_w_o, int32_t *counts_o,
                    int32_t *offsets_o, int32_t *perm_o, int32_t *inv_o, int threads) {
    if (!desc_ok(desc) || T < 0) return -1;
    int D = desc->d_model, F = desc->d_ff, E = desc->n_expert, K = desc->n_expert_used;
    int S = desc->n_shared, FS = desc->d_ff_shared;
    if (T == 0) return 0;
    size_t A = (size_t)T * K;
    float *logits = (float *)malloc(sizeof(float) * (size_t)T * E);
    int32_t *idx = (int32_t *)malloc(sizeof(int32_t) * A);
    float *tw = (float *)malloc(sizeof(float) * A);
    int32_t *counts = (int32_t *)malloc(sizeof(int32_t) * E);
    int32_t *offsets = (int32_t *)malloc(sizeof(int32_t) * (E + 1));
    int32_t *perm = (int32_t *)malloc(sizeof(int32_t) * A);
    int32_t *inv = (int32_t *)malloc(sizeof(int32_t) * A);
    float *Y = (float *)malloc(sizeof(float) * A * D);
    float *Ysh = (float *)malloc(sizeof(float) * ((size_t)S * T * D + 1));
    float *router = ingest_f32(w->router, (size_t)D * E);
    float *bias = desc->has_bias ? ingest_f32(w->bias, (size_t)E) : NULL;
    lco_router_logits(x, router, logits, T, D, E);
    lco_route(desc, logits, bias, T, idx, tw);
    lco_dispatch(idx, T, K, E, counts, offsets, perm, inv);
    free(router);
    free(bias);

    size_t szg = lco_tensor_size(desc->type_gate, (size_t)F * D);
    size_t szu = lco_tensor_size(desc->type_up, (size_t)F * D);
    size_t szd = lco_tensor_size(desc->type_down, (size_t)D * F);
    float *xe = (float *)malloc(sizeof(float) * A * D);
    /* threads > 1: experts in parallel, each expert's products on one thread
     * (the per-element arithmetic does not depend on the split) */
    const int par = threads > 1;
#pragma omp parallel for schedule(dynamic, 1) num_threads(par ? threads : 1) if (par)
    for (int e = 0; e < E; e++) {
        int n = counts[e];
        if (!n) continue;
        float *xr = xe + (size_t)offsets[e] * D;
        for (int r = 0; r < n; r++)
            memcpy(xr + (size_t)r * D, x + (size_t)(perm[offsets[e] + r] / K) * D, sizeof(float) * D);
        float *wg = ingest(desc->type_gate, w->gate + (size_t)e * szg, F, D);
        float *wu = ingest(desc->type_up, w->up + (size_t)e * szu, F, D);
        float *wd = ingest(desc->type_down, w->down + (size_t)e * szd, D, F);
        lco_ffn_dense(xr, n, D, F, wg, wu, wd, Y + (size_t)offsets[e] * D, par ? 1 : threads);
        free(wg); free(wu); free(wd);
    }
    if (S > 0) {
        size_t sg = lco_tensor_size(desc->type_gate_sh, (size_t)FS * D);
        size_t su = lco_tensor_size(desc->type_up_sh, (size_t)FS * D);
        size_t sd = lco_tensor_size(desc->type_down_sh, (size_t)D * FS);
        for (int s = 0; s < S; s++) {
            float *wg = ingest(desc->type_gate_sh, w->gate_sh + (size_t)s * sg, FS, D);
            float *wu = ingest(desc->type_up_sh, w->up_sh + (size_t)s * su, FS, D);
            float *wd = ingest(desc->type_down_sh, w->down_sh + (size_t)s * sd, D, FS);
            lco_ffn_dense(x, T, D, FS, wg, wu, wd, Ysh + (size_t)s * T * D, threads);
            free(wg); free(wu); free(wd);
        }
    }
    combine(desc, T, Y, Ysh, inv, tw, y);
    if (topk_idx_o) memcpy(topk_idx_o, idx, sizeof(int32_t) * A);
    if (topk_w_o) memcpy(topk_w_o, tw, sizeof(float) * A);
    if (counts_o) memcpy(counts_o, counts, sizeof(int32_t) * E);
    if (offsets_o) memcpy(offsets_o, offsets, sizeof(int32_t) * (E + 1));
    if (perm_o) memcpy(perm_o, perm, sizeof(int32_t) * A);
    if (inv_o) memcpy(inv_o, inv, sizeof(int32_t) * A);
    free(logits); free(idx); free(tw); free(counts); free(offsets); free(perm); free(inv);
    free(Y); free(Ysh); free(xe);
    return 0;
}

/* ---- resident CPU baseline ------------------------------------------- */

typedef struct {
    lco_desc desc;
    const float *router, *bias;
    float **wg, **wu, **wd; /* E + S each, post-load [in,out] f32 */
} lco_resident;

void *lco_resident_create(const lco_desc *desc, const lco_weights *w, int threads) {
    (void)threads;
    if (!desc_ok(desc)) return NULL;
    lco_resident *r = (lco_resident *)calloc(1, sizeof *r);
    r->desc = *desc;
    int E = desc->n_expert, S = desc->n_shared, D = desc->d_model, F = desc->d_ff, FS = desc->d_ff_shared;
    r->router = ingest_f32(w->router, (size_t)D * E);
    r->bias = desc->has_bias ? ingest_f32(w->bias, (size_t)E) : NULL;
    r->wg = (float **)calloc((size_t)(E + S) * 3, sizeof(float *));
    r->wu = r->wg + (E + S);
    r->wd = r->wu + (E + S);
    size_t szg = lco_tensor_size(desc->type_gate, (size_t)F * D);
    size_t szu = lco_tensor_size(desc->type_up, (size_t)F * D);
    size_t szd = lco_tensor_size(desc->type_down, (size_t)D * F);
    size_t sg = S ? lco_tensor_size(desc->type_gate_sh, (size_t)FS * D) : 0;
    size_t su = S ? lco_tensor_size(desc->type_up_sh, (size_t)FS * D) : 0;
    size_t sd = S ? lco_tensor_size(desc->type_down_sh, (size_t)D * FS) : 0;
#pragma omp parallel for schedule(dynamic, 1)
    for (int e = 0; e < E + S; e++) {
        if (e < E) {
            r->wg[e] = ingest(desc->type_gate, w->gate + (size_t)e * szg, F, D);
            r->wu[e] = ingest(desc->type_up, w->up + (size_t)e * szu, F, D);
            r->wd[e] = ingest(desc->type_down, w->down + (size_t)e * szd, D, F);
        } else {
            int s = e - E;
            r->wg[e] = ingest(desc->type_gate_sh, w->gate_sh + (size_t)s * sg, FS, D);
            r->wu[e] = ingest(desc->type_up_sh, w->up_sh + (size_t)s * su, FS, D);
            r->wd[e] = ingest(desc->type_down_sh, w->down_sh + (size_t)s * sd, D, FS);
        }
    }
    return r;
}

int lco_resident_forward(void *h, const float *x, int T, float *y, int threads) {
    lco_resident *r = (lco_resident *)h;
    const lco_desc *desc = &r->desc;
    int D = desc->d_model, F = desc->d_ff, E = desc->n_expert, K = desc->n_expert_used;
    int S = desc->n_shared, FS = desc->d_ff_shared;
    size_t A = (size_t)T * K;
    float *logits = (float *)malloc(sizeof(float) * (size_t)T * E);
    int32_t *idx = (int32_t *)malloc(sizeof(int32_t) * A * 3);
    int32_t *perm = idx + A, *inv = perm + A;
    float *tw = (float *)malloc(sizeof(float) * A);
    int32_t *counts = (int32_t *)malloc(sizeof(int32_t) * (2 * E + 1)), *offsets = counts + E;
    float *Y = (float *)malloc(sizeof(float) * A * D);
    float *Ysh = (float *)malloc(sizeof(float) * ((size_t)S * T * D + 1));
    float *xe = (float *)malloc(sizeof(float) * A * D);
    lco_router_logits(x, r->router, logits, T, D, E);
    lco_route(desc, logits, r->bias, T, idx, tw);
    lco_dispatch(idx, T, K, E, counts, offsets, perm, inv);
    for (int e = 0; e < E; e++) {
        int n = counts[e];
        if (!n) continue;
        for (int q = 0; q < n; q++)
            memcpy(xe + (size_t)q * D, x + (size_t)(perm[offsets[e] + q] / K) * D, sizeof(float) * D);
        lco_ffn_dense(xe, n, D, F, r->wg[e], r->wu[e], r->wd[e], Y + (size_t)offsets[e] * D, threads);
    }
    for (int s = 0; s < S; s++)
        lco_ffn_dense(x, T, D, FS, r->wg[E + s], r->wu[E + s], r->wd[E + s], Ysh + (size_t)s * T * D, threads);
    combine(desc, T, Y, Ysh, inv, tw, y);
    free(logits); free(idx); free(tw); free(counts); free(Y); free(Ysh); free(xe);
    return 0;
}

void lco_resident_destroy(void *h) {
    lco_resident *r = (lco_resident *)h;
    if (!r) return;
    int n = r->desc.n_expert + r->desc.n_shared;
    for (int e = 0; e < n; e++) { free(r->wg[e]); free(r->wu[e]); free(r->wd[e]); }
    free(r->wg);
    free((void *)r->router);
    free((void *)r->bias);
    free(r);
}

/* The shard engine's quantised GEMM, C[m,n] = A[m,k] B[k,n], B in blocks of
 * 32 along n, row-major over k (rust/src/kernels/int8_gemm.rs).  n is a
 * whole number of blocks, so x86 always takes the AVX2 path
 * (q8_0_matmul :172-194 -> q8_0_matmul_avx2_inner :47-98; the Q4_0 twin
 * q4_0_matmul_avx2_inner follows :240-290): C starts at 0; for each k-row l
 * every block is dequantised to f32 (q * scale, one rounding) and
 * c = fma(a[i,l], deq, c).  Blocks come from bytes as q8_0.rs:24-32 /
 * q4_0.rs Block::from_bytes read them: Q8_0 = f16 scale + 32 int8 (34 B);
 * Q4_0 = f16 scale + 16 bytes, element 2t the low nibble of byte t, 2t+1
 * the high one, value nibble - 8 (q4_0.rs:36-46; not GGUF's order).
 * type: LCO_Q8_0 or LCO_Q4_0_SHARD.  Returns -1 on a bad type or shape. */
int lco_shard_matmul(int type, const float *a, const uint8_t *b, float *c, int m, int k,
                     int n) {
    if ((type != LCO_Q8_0 && type != LCO_Q4_0_SHARD) || m < 0 || k < 0 || n < 0 || n % 32)
        return -1;
    const int bpr = n / 32;
    const size_t bb = type == LCO_Q8_0 ? 34 : 18;
    float *deq = (float *)malloc(sizeof(float) * (size_t)(n ? n : 1));
    if (!deq) return -1;
    for (int i = 0; i < m; i++) {
        float *cr = c + (size_t)i * n;
        for (int j = 0; j < n; j++) cr[j] = 0.0f;
        for (int l = 0; l < k; l++) {
            for (int blk = 0; blk < bpr; blk++) {
                const uint8_t *p = b + ((size_t)l * bpr + blk) * bb;
                const float sc = lco_f16_to_f32((uint16_t)(p[0] | (p[1] << 8)));
                for (int t = 0; t < 32; t++) {
                    float q;
                    if (type == LCO_Q8_0) {
                        q = (float)(int8_t)p[2 + t];
                    } else {
                        const uint8_t byte = p[2 + t / 2];
                        q = (float)((t & 1) ? (byte >> 4) : (byte & 15)) - 8.0f;
                    }
                    deq[blk * 32 + t] = q * sc;
                }
            }
            const float av = a[(size_t)i * k + l];
            for (int j = 0; j < n; j++) cr[j] = fmaf(av, deq[j], cr[j]);
        }
    }
    free(deq);
    return 0;
}

/* ====================================================================== */
/* Decoder-layer pieces around the MoE FFN, for the end-to-end engine      */
/* (rust/src/inference/engine.rs:78-132).  Same arithmetic as the Rust:     */
/* every a*b+c rounds twice (-ffp-contract=off), f32 libm calls.           */
/* ====================================================================== */

/* apply_rotary_emb, rust/src/inference/attention.rs:13-34, on x [seq, heads,
 * hd]: pair (d, d + hd/2) of token i rotates by angle (pos0 + i) * freq_d,
 * freq_d = 1 / theta^(2d / hd).  The reference passes pos0 = 0 on every
 * forward (positions restart at each call: a decode token rotates by 0). */
void lco_rope(float *x, int seq, int heads, int hd, float theta, int pos0) {
    for (int i = 0; i < seq; i++)
        for (int h = 0; h < heads; h++)
            for (int d = 0; d < hd / 2; d++) {
                float freq = 1.0f / powf(theta, 2.0f * (float)d / (float)hd);
                float angle = (float)(pos0 + i) * freq;
                float cos_a = cosf(angle), sin_a = sinf(angle);
                size_t base = (size_t)i * heads * hd + (size_t)h * hd;
                float x1 = x[base + d], x2 = x[base + d + hd / 2];
                x[base + d] = x1 * cos_a - x2 * sin_a;
                x[base + d + hd / 2] = x1 * sin_a + x2 * cos_a;
            }
}

/* The attention core of attention_forward, attention.rs:56-115, for one
 * forward of seq tokens whose K/V were just appended to a cache of `total`
 * positions (so cache_len = total - seq came before): q [seq, heads, hd]
 * after RoPE; k, v [total, kv_heads, hd] the cache decompressed to f32
 * (cache/mod.rs:66-78); out [seq, heads * hd].  Head h reads kv head
 * h / (heads / kv_heads).  Score = (sum_d q*k in order) / sqrt(hd), t past
 * cache_len + s masked to -inf; softmax as max, sum of exp, then
 * exp / sum; out = sum_t p_t * v_t in order. */
void lco_attention_core(const float *q, const float *k, const float *v, int seq, int total,
                        int heads, int kv_heads, int hd, float *out) {
    const int groups = heads / kv_heads, cache_len = total - seq;
    float *scores = (float *)malloc(sizeof(float) * (size_t)(total > 0 ? total : 1));
    const float sq = sqrtf((float)hd);
    for (int h = 0; h < heads; h++) {
        const int kvh = h / groups;
        for (int s = 0; s < seq; s++) {
            for (int t = 0; t < total; t++) {
                if (t > cache_len + s) {
                    scores[t] = -INFINITY;
                } else {
                    float dot = 0.0f;
                    for (int d = 0; d < hd; d++) {
                        float p = q[(size_t)s * heads * hd + (size_t)h * hd + d] *
                                  k[(size_t)t * kv_heads * hd + (size_t)kvh * hd + d];
                        dot = dot + p;
                    }
                    scores[t] = dot / sq;
                }
            }
            float mx = -INFINITY;
            for (int t = 0; t < total; t++) mx = rust_fmax(mx, scores[t]);
            float sum = 0.0f;
            for (int t = 0; t < total; t++) sum = sum + expf(scores[t] - mx);
            for (int t = 0; t < total; t++) scores[t] = expf(scores[t] - mx) / sum;
            for (int d = 0; d < hd; d++) {
                float acc = 0.0f;
                for (int t = 0; t < total; t++) {
                    float p = scores[t] * v[(size_t)t * kv_heads * hd + (size_t)kvh * hd + d];
                    acc = acc + p;
                }
                out[(size_t)s * heads * hd + (size_t)h * hd + d] = acc;
            }
        }
    }
    free(scores);
}

/* Greedy sampling, sample_top_p with temperature <= 0
 * (rust/src/inference/sampler.rs:8-10): Iterator::max_by over f32::total_cmp,
 * which keeps the LAST of equal maxima; total order -NaN < -inf < ... < -0 <
 * +0 < ... < +inf < +NaN.  Returns 0 for n == 0 (unwrap_or(0)). */
int lco_argmax_last(const float *x, int n) {
    int best = -1;
    int32_t bk = 0;
    for (int i = 0; i < n; i++) {
        int32_t b = (int32_t)f2u(x[i]);
        b ^= (int32_t)(((uint32_t)(b >> 31)) >> 1);
        if (best < 0 || b >= bk) { best = i; bk = b; }
    }
    return best < 0 ? 0 : best;
}
