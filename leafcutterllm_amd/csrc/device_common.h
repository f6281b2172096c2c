// Device helpers shared by the kernel translation units (HIP, gfx950).
//
// Every TU that includes this is compiled with -ffp-contract=off: fused
// multiply-adds are explicit (__builtin_fmaf); a*b+c otherwise rounds twice.
#pragma once

#include <hip/hip_runtime.h>

#include <climits>
#include <cstdint>

#include "../../include/lcmoe.h"

namespace lcmoe {

constexpr int kMaxE = 256;
constexpr int kMaxK = 16;

__device__ __forceinline__ float dh2f(uint32_t h) {
    _Float16 v;
    uint16_t b = (uint16_t)h;
    __builtin_memcpy(&v, &b, 2);
    return (float)v;
}

// get_scale_min_k4, rust/src/kernels/mod.rs:54-63.
__device__ __forceinline__ void scale_min_k4(int j, const uint8_t *q, int &sc, int &m) {
    if (j < 4) {
        sc = q[j] & 63;
        m = q[j + 4] & 63;
    } else {
        sc = (q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4);
        m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

// Decode 8 consecutive elements starting at flat element index idx (a
// multiple of 8) of a GGUF tensor into f32, bit-identical to the reference
// decoders.  Flat indexing is what those decoders do (num_blocks =
// out.len() / QK), so rows that start inside a super-block decode correctly.
template <int QT>
struct Dec;

template <>
struct Dec<LCMOE_TYPE_F32> {
    __device__ __forceinline__ static void run(const uint8_t *__restrict__ base, int64_t idx,
                                               float (&o)[8]) {
        const float4 *p = reinterpret_cast<const float4 *>(base + idx * 4);
        float4 a = p[0], b = p[1];
        o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
        o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
    }
};

// dequantize_q8_0, rust/src/kernels/mod.rs:37-51: v = (int8)q * d.
template <>
struct Dec<LCMOE_TYPE_Q8_0> {
    __device__ __forceinline__ static void run(const uint8_t *__restrict__ base, int64_t idx,
                                               float (&o)[8]) {
        const uint8_t *b = base + (idx >> 5) * 34;
        float d = dh2f(*reinterpret_cast<const uint16_t *>(b));
        const uint16_t *q = reinterpret_cast<const uint16_t *>(b + 2 + (idx & 31));
#pragma unroll
        for (int i = 0; i < 4; i++) {
            uint32_t u = q[i];
            o[2 * i] = (float)(int8_t)(u & 0xff) * d;
            o[2 * i + 1] = (float)(int8_t)(u >> 8) * d;
        }
    }
};

// dequantize_q4_k, rust/src/kernels/mod.rs:66-98: v = (d*sc)*q - dmin*m.
template <>
struct Dec<LCMOE_TYPE_Q4_K> {
    __device__ __forceinline__ static void run(const uint8_t *__restrict__ base, int64_t idx,
                                               float (&o)[8]) {
        const uint8_t *b = base + (idx >> 8) * 144;
        int e = (int)(idx & 255), j = e >> 6, hi = (e >> 5) & 1, l = e & 31;
        uint32_t dd = *reinterpret_cast<const uint32_t *>(b);
        float d = dh2f(dd & 0xffff), dmin = dh2f(dd >> 16);
        int sc, m;
        scale_min_k4(2 * j + hi, b + 4, sc, m);
        float dl = d * (float)sc, ml = dmin * (float)m;
        uint2 q = *reinterpret_cast<const uint2 *>(b + 16 + 32 * j + l);
        uint32_t w0 = hi ? q.x >> 4 : q.x, w1 = hi ? q.y >> 4 : q.y;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            o[i] = dl * (float)((w0 >> (8 * i)) & 15) - ml;
            o[4 + i] = dl * (float)((w1 >> (8 * i)) & 15) - ml;
        }
    }
};

// dequantize_q6_k, rust/src/kernels/mod.rs:145-180: v = (d*sc)*(q - 32).
template <>
struct Dec<LCMOE_TYPE_Q6_K> {
    __device__ __forceinline__ static void run(const uint8_t *__restrict__ base, int64_t idx,
                                               float (&o)[8]) {
        const uint8_t *b = base + (idx >> 8) * 210;
        int e = (int)(idx & 255), n = e >> 7, w = e & 127, s = w >> 5, l = w & 31;
        const uint16_t *ql = reinterpret_cast<const uint16_t *>(b + 64 * n + 32 * (s & 1) + l);
        const uint16_t *qh = reinterpret_cast<const uint16_t *>(b + 128 + 32 * n + l);
        float d = dh2f(*reinterpret_cast<const uint16_t *>(b + 208));
        float dsc = d * (float)(int8_t)b[192 + (e >> 4)];
        int lsh = (s < 2) ? 0 : 4, hsh = 2 * s;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            uint32_t lo = ql[i], hb = qh[i];
            int q0 = (int)((((lo >> lsh) & 15) | (((hb >> hsh) & 3) << 4))) - 32;
            int q1 = (int)((((lo >> (8 + lsh)) & 15) | (((hb >> (8 + hsh)) & 3) << 4))) - 32;
            o[2 * i] = dsc * (float)q0;
            o[2 * i + 1] = dsc * (float)q1;
        }
    }
};

// Router sigmoid: 1 / (1 + e^-x) with e^x evaluated by Cody-Waite range
// reduction and a degree-7 Taylor polynomial (Horner, fused multiply-adds),
// then exact scaling by 2^k.  Only IEEE basic operations and fma, so the
// host oracle and the device produce identical bits.
__device__ __forceinline__ float expf_cw(float x) {
    if (x != x) return x;
    if (x > 88.7228394f) return __builtin_inff();
    if (x < -103.972084f) return 0.0f;
    const float shifter = 12582912.0f;
    float kf = __builtin_fmaf(x, 1.44269502f, shifter) - shifter;
    float r = __builtin_fmaf(-kf, 0.693145751953125f, x);
    r = __builtin_fmaf(-kf, 1.42860677e-06f, r);
    float p = 1.98412701e-04f;
    p = __builtin_fmaf(p, r, 1.38888892e-03f);
    p = __builtin_fmaf(p, r, 8.33333377e-03f);
    p = __builtin_fmaf(p, r, 4.16666679e-02f);
    p = __builtin_fmaf(p, r, 1.66666672e-01f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    int k = (int)kf;
    if (k < -125) {
        p = p * 5.42101086e-20f;
        k += 64;
    }
    if (k > 127) {
        p = p * 2.0f;
        k -= 1;
    }
    return p * __uint_as_float((uint32_t)(k + 127) << 23);
}

__device__ __forceinline__ float sigmoid_cw(float x) { return 1.0f / (1.0f + expf_cw(-x)); }

// silu as CpuBackend::silu, rust/src/backend/cpu.rs:62-64.
__device__ __forceinline__ float silu(float v) { return v * (1.0f / (1.0f + expf(-v))); }

// f32::max of the reference: the non-NaN argument wins.
__device__ __forceinline__ float nan_max(float a, float b) {
    if (a != a) return b;
    if (b != b) return a;
    return a > b ? a : b;
}

__device__ __forceinline__ float sel_key(float z) { return z != z ? -__builtin_inff() : z; }
__device__ __forceinline__ bool better(float ka, int a, float kb, int b) {
    return ka > kb || (ka == kb && a < b);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// f64 move across lanes by DPP (both 32-bit halves); lanes whose source is
// outside the pattern, or whose row the mask leaves out, read +0
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ double dpp_f64(double v) {
    const int lo = __builtin_amdgcn_update_dpp(0, __double2loint(v), CTRL, ROW_MASK, 0xf, true);
    const int hi = __builtin_amdgcn_update_dpp(0, __double2hiint(v), CTRL, ROW_MASK, 0xf, true);
    return __hiloint2double(hi, lo);
}

// inclusive prefix sum over the 64 lanes (row shifts 1, 2, 4, 8 inside each
// row of 16, then row broadcasts 15 and 31 across rows): register moves only,
// no LDS round trips
__device__ __forceinline__ double wave_incl_scan_f64(double v) {
    v += dpp_f64<0x111, 0xf>(v);  // row_shr:1
    v += dpp_f64<0x112, 0xf>(v);  // row_shr:2
    v += dpp_f64<0x114, 0xf>(v);  // row_shr:4
    v += dpp_f64<0x118, 0xf>(v);  // row_shr:8
    v += dpp_f64<0x142, 0xa>(v);  // row_bcast:15 into rows 1 and 3
    v += dpp_f64<0x143, 0xc>(v);  // row_bcast:31 into rows 2 and 3
    return v;
}

__device__ __forceinline__ double readlane_f64(double v, int lane) {
    const int lo = __builtin_amdgcn_readlane(__double2loint(v), lane);
    const int hi = __builtin_amdgcn_readlane(__double2hiint(v), lane);
    return __hiloint2double(hi, lo);
}

// the sum over the 64 lanes, in every lane
__device__ __forceinline__ double wave_total_f64(double v) {
    return readlane_f64(wave_incl_scan_f64(v), 63);
}

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROW_MASK, 0xf, true);
}

// the maximum over the 64 lanes, in every lane (0 is the identity); the same
// row-shift / row-broadcast pattern as wave_incl_scan_f64
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, dpp_u32<0x111, 0xf>(v));
    v = max(v, dpp_u32<0x112, 0xf>(v));
    v = max(v, dpp_u32<0x114, 0xf>(v));
    v = max(v, dpp_u32<0x118, 0xf>(v));
    v = max(v, dpp_u32<0x142, 0xa>(v));
    v = max(v, dpp_u32<0x143, 0xc>(v));
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint64_t max_dpp_u64(uint64_t v) {
    const uint64_t o = ((uint64_t)dpp_u32<CTRL, ROW_MASK>((uint32_t)(v >> 32)) << 32) |
                       dpp_u32<CTRL, ROW_MASK>((uint32_t)v);
    return o > v ? o : v;
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
    v = max_dpp_u64<0x111, 0xf>(v);
    v = max_dpp_u64<0x112, 0xf>(v);
    v = max_dpp_u64<0x114, 0xf>(v);
    v = max_dpp_u64<0x118, 0xf>(v);
    v = max_dpp_u64<0x142, 0xa>(v);
    v = max_dpp_u64<0x143, 0xc>(v);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(v >> 32), 63);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
    return ((uint64_t)hi << 32) | lo;
}

// order-preserving unsigned encoding of a non-NaN float, -0 and +0 equal:
// a < b  <=>  ord_key(a) < ord_key(b); every value encodes above 0
__device__ __forceinline__ uint32_t ord_key(float f) {
    const uint32_t u = __float_as_uint(f == 0.0f ? 0.0f : f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Matrix-core activation format of one 32-column sub-block sbi of row t
// (row width d, a multiple of 256): the f16 hi = f16(v) and lo = f16(v - hi)
// halves at columns 32 (sbi % 8) .. +31 of the row's super-block piece sbi / 8
// (hi[256] then lo[256], columns at act16_pos), and the sub-block's sum of (hi + lo) -- of hi
// alone when !lo, for products that take only the hi halves -- added in
// column order, as a (hi, lo) pair.  v: the 32 values, 16-byte aligned.
// Position of column c (0..255) inside its piece of the matrix-core
// activation format: columns are stored permuted within each group of four
// as (c0, c2, c1, c3), the order in which one and-or pulls two nibbles out of
// a packed weight word as f16 magic values (bytes 0 and 2, then 1 and 3).
// The permutation is applied to both operands of every product, so the sums
// are unchanged.
__device__ __forceinline__ int act16_pos(int c) { return (c & ~3) | ((c & 1) << 1) | ((c >> 1) & 1); }

__device__ inline void act16_subblock(const float *v, int64_t t, int d, int sbi,
                                      _Float16 *__restrict__ x16, _Float16 *__restrict__ xs,
                                      bool lo_sum = true) {
    typedef _Float16 h8 __attribute__((ext_vector_type(8)));
    const float4 *v4 = reinterpret_cast<const float4 *>(v);
    _Float16 *piece = x16 + (t * (d >> 8) + (sbi >> 3)) * 512 + 32 * (sbi & 7);
    h8 *oh = reinterpret_cast<h8 *>(piece);
    h8 *ol = reinterpret_cast<h8 *>(piece + 256);
    float sum = 0.0f;
#pragma unroll
    for (int g = 0; g < 4; g++) {
        const float4 a = v4[2 * g], b = v4[2 * g + 1];
        const float f[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        h8 hv, lv;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const _Float16 hi = (_Float16)f[i], lo = (_Float16)(f[i] - (float)hi);
            hv[act16_pos(i)] = hi;
            lv[act16_pos(i)] = lo;
            sum = sum + (lo_sum ? (float)hi + (float)lo : (float)hi);
        }
        oh[g] = hv;
        ol[g] = lv;
    }
    const _Float16 shi = (_Float16)sum, slo = (_Float16)(sum - (float)shi);
    const int64_t q = t * (d >> 5) + sbi;
    xs[q * 2] = shi;
    xs[q * 2 + 1] = slo;
}

// Which expert a block of an expert-product launch serves.  Routed launch:
// slot i < nr serves touched[i] (nothing when i >= number touched) over
// positions p in [offsets[e], offsets[e] + counts[e]) whose token is
// perm[p] / K; slot nr + s*ns + c serves tokens [c*sl, c*sl + sl) of shared
// expert s < S, stored as expert E + s, at positions sbase + s*T + t (shared
// experts fused into the routed launch, in ns slices of sl tokens).  With
// pslots, routed slot i < nr is pass slot i instead: pass p of expert e
// (pslots[1 + i] = 256 p + e; nothing when i >= pslots[0]), positions
// offsets[e] + 32 p onward, at most 32.  Shared launch (shared = 1): slot s
// is shared expert s over all T tokens, positions s*T + t.
struct SlotArgs {
    const int32_t *perm, *counts, *offsets, *touched;
    int E, K, T, shared;
    int nr, S, sbase, ns, sl;
    const int32_t *pslots;  // pass slots (RouterArgs::pass_slots) or null
};

constexpr int kPassTokens = 32;  // tokens per pass slot

__device__ __forceinline__ bool slot_info(const SlotArgs &sa, int slot, int &e, int &p0, int &n) {
    if (sa.shared) {
        e = slot;
        p0 = slot * sa.T;
        n = sa.T;
        return true;
    }
    if (slot >= sa.nr) {
        const int v = slot - sa.nr, s = v / sa.ns, c = v - s * sa.ns;
        if (s >= sa.S) return false;
        e = sa.E + s;
        p0 = sa.sbase + s * sa.T + c * sa.sl;
        n = min(sa.sl, sa.T - c * sa.sl);
        return n > 0;
    }
    if (sa.pslots) {  // one 32-token pass of one expert
        if (slot >= sa.pslots[0]) return false;
        const int v = sa.pslots[1 + slot], pass = v >> 8;
        e = v & 255;
        p0 = sa.offsets[e] + kPassTokens * pass;
        n = min(kPassTokens, sa.counts[e] - kPassTokens * pass);
        return true;
    }
    if (slot >= sa.touched[sa.E]) return false;
    e = sa.touched[slot];
    p0 = sa.offsets[e];
    n = sa.counts[e];
    return true;
}

// token of position p0 + q; positions from sbase on belong to fused shared
// experts and follow the tokens (T per expert)
__device__ __forceinline__ int slot_token(const SlotArgs &sa, int p0, int q) {
    if (sa.shared) return q;
    return p0 >= sa.sbase ? (p0 - sa.sbase) % sa.T + q : sa.perm[p0 + q] / sa.K;
}

// Two-limb int8 quantisation of 32 values held one per lane in a 32-lane
// half-wave: v ~= s * (128*hi + lo), hi in [-127,127], lo in [-64,63],
// s = max|v| / 16256.  Returns the limbs and, in *sum_out (same in all 32
// lanes), s * sum(128*hi + lo), the quantised values' sum.
__device__ __forceinline__ void quant2_half(float v, int &hi, int &lo, float &s, float &sum_out) {
    float a = fabsf(v);
#pragma unroll
    for (int off = 16; off >= 1; off >>= 1) a = fmaxf(a, __shfl_xor(a, off, 64));
    s = a * (1.0f / 16256.0f);
    int xi = 0;
    if (a > 0.0f) {
        xi = (int)rintf(v / s);
        xi = xi > 16256 ? 16256 : (xi < -16256 ? -16256 : xi);
    }
    hi = (xi + 64) >> 7;
    lo = xi - 128 * hi;
    int isum = xi;
#pragma unroll
    for (int off = 16; off >= 1; off >>= 1) isum += __shfl_xor(isum, off, 64);
    sum_out = s * (float)isum;
}

}  // namespace lcmoe
