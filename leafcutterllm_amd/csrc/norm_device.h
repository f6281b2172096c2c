// CpuBackend::rms_norm, bit for bit, as a per-wave device function shared by
// the stand-alone norm kernel (kern_generic.hip) and the router entry kernel
// that fuses it (kern_route.hip).
#pragma once

#include "device_common.h"

namespace lcmoe {
namespace rmsnorm_detail {

// CpuBackend::rms_norm (rust/src/backend/cpu.rs:49-60) on x86, where the sum
// of squares is simd_sum_sq (rust/src/kernels/simd.rs:390-409): four running
// sums, lane j taking columns j, j+4, j+8, ... (each product rounded, then
// added), folded into 0 in lane order; mean = sum / d and scale =
// 1 / sqrt(mean + eps), each correctly rounded; out = (x * scale) * w, two
// roundings (simd_vec_scale_mul, simd.rs:353-369).  d % 4 == 0, so there is
// no tail.  The four sums are sequential chains whose order fixes the bits:
// one wave per token squares up to kNormChunk columns at a time into LDS,
// lane j's terms contiguous, and lanes 0-3 advance the chains from there,
// four terms per LDS read (each chain is padded with zeros to a multiple of
// 32 terms, which adds exactly nothing: the sums are never -0); then the
// whole wave scales the row (with one chunk, d <= 4096, the row and the
// weights are still in registers).
constexpr int kNormChunk = 4096;

// Round-to-nearest-even f32 results from a double estimate, corrected by
// exact midpoint tests: the midpoint of two adjacent floats has at most 25
// significant bits, so its product with a float (24 bits) or with itself is
// exact in double.  The estimate only has to land within a float ulp or two.
__device__ inline float next_up(float q) { return __uint_as_float(__float_as_uint(q) + 1u); }
__device__ inline float next_dn(float q) { return __uint_as_float(__float_as_uint(q) - 1u); }
__device__ inline bool odd(float q) { return __float_as_uint(q) & 1u; }

// a / b for a >= 0, b > 0, both finite
__device__ float div_rn_pos(float a, float b) {
    float q = (float)((double)a / (double)b);
    if (!(q > 0.0f) || __float_as_uint(q) >= 0x7f800000u) return q;  // 0 or overflow
    for (int it = 0; it < 4; it++) {
        const double pu = 0.5 * ((double)q + (double)next_up(q)) * (double)b;
        const double pd = 0.5 * ((double)q + (double)next_dn(q)) * (double)b;
        if ((double)a > pu || ((double)a == pu && odd(q))) q = next_up(q);
        else if ((double)a < pd || ((double)a == pd && odd(q))) q = next_dn(q);
        else break;
    }
    return q;
}

// sqrt(m) for m >= 0
__device__ float sqrt_rn(float m) {
    float s = (float)__builtin_sqrt((double)m);
    if (!(s > 0.0f) || __float_as_uint(s) >= 0x7f800000u) return s;  // 0, inf, NaN
    for (int it = 0; it < 4; it++) {
        const double mu = 0.5 * ((double)s + (double)next_up(s));
        const double md = 0.5 * ((double)s + (double)next_dn(s));
        if ((double)m > mu * mu || ((double)m == mu * mu && odd(s))) s = next_up(s);
        else if ((double)m < md * md || ((double)m == md * md && odd(s))) s = next_dn(s);
        else break;
    }
    return s;
}
// LDS floats rmsnorm_wave<CHUNK> needs
template <int CHUNK = kNormChunk>
constexpr int rmsnorm_lds() { return 4 * (CHUNK / 4 + 4); }
constexpr int kRmsnormLds = rmsnorm_lds<>();

// LDS stores of the wave visible to its own later reads
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

// One wave: out = rms_norm(x) * w for the row x (d % 4 == 0; x, w and out
// 16-byte aligned; out may not alias x), s_sq = rmsnorm_lds<CHUNK>() floats
// of LDS.  CHUNK columns are squared per LDS pass (a multiple of 256; fewer
// registers for a smaller one, the same bits either way).
template <int CHUNK = kNormChunk>
__device__ inline void rmsnorm_wave(const float *__restrict__ x, const float *__restrict__ w,
                                    float eps, int d, float *__restrict__ out, float *s_sq) {
    constexpr int kNormChunk = CHUNK;
    constexpr int ld = kNormChunk / 4 + 4, kV = kNormChunk / 256;  // kV: float4s per lane
    const int lane = threadIdx.x & 63;
    const float4 *r = reinterpret_cast<const float4 *>(x);
    const int n4 = d >> 2;
    const float4 *g = reinterpret_cast<const float4 *>(w);
    float4 v[kV], gw[kV];
    float acc = 0.0f;
    for (int c0 = 0; c0 < n4; c0 += kNormChunk / 4) {
        // q: the chunk's float4 count rounded up to whole groups of 8 per chain
        const int n = min(kNormChunk / 4, n4 - c0), q = (n + 31) & ~31;
#pragma unroll
        for (int k = 0; k < kV; k++) {  // every load of the chunk in flight at once
            const int i = lane + 64 * k;
            v[k] = i < n ? r[c0 + i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
        if (n4 <= kNormChunk / 4) {  // one chunk: the weights load during the chain
#pragma unroll
            for (int k = 0; k < kV; k++) {
                const int i = lane + 64 * k;
                if (i < n) gw[k] = g[i];
            }
        }
#pragma unroll
        for (int k = 0; k < kV; k++) {
            const int i = lane + 64 * k;
            if (i < q) {
                s_sq[i] = v[k].x * v[k].x;
                s_sq[ld + i] = v[k].y * v[k].y;
                s_sq[2 * ld + i] = v[k].z * v[k].z;
                s_sq[3 * ld + i] = v[k].w * v[k].w;
            }
        }
        wave_lds_sync();
        if (lane < 4) {  // groups of 8 float4s, the next group's reads in flight
            const float4 *c = reinterpret_cast<const float4 *>(s_sq + lane * ld);
            float4 cur[8], nxt[8];
#pragma unroll
            for (int u = 0; u < 8; u++) cur[u] = c[u];
            for (int gi = 8; gi <= q / 4; gi += 8) {
                if (gi < q / 4) {
#pragma unroll
                    for (int u = 0; u < 8; u++) nxt[u] = c[gi + u];
                }
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    acc = acc + cur[u].x;
                    acc = acc + cur[u].y;
                    acc = acc + cur[u].z;
                    acc = acc + cur[u].w;
                }
#pragma unroll
                for (int u = 0; u < 8; u++) cur[u] = nxt[u];
            }
        }
        wave_lds_sync();
    }
    float sum = 0.0f;
    for (int j = 0; j < 4; j++) sum = sum + __shfl(acc, j);
    // sum >= 0; inf or NaN rows go through the double route unchanged
    const float mean = div_rn_pos(sum, (float)d);
    const float root = sqrt_rn(mean + eps);
    const float scale = root > 0.0f ? div_rn_pos(1.0f, root) : 1.0f / root;
    float4 *o = reinterpret_cast<float4 *>(out);
    for (int c0 = 0; c0 < n4; c0 += kNormChunk / 4) {
        const int n = min(kNormChunk / 4, n4 - c0);
        if (n4 > kNormChunk / 4) {  // one chunk: the row and weights are still in v, gw
#pragma unroll
            for (int k = 0; k < kV; k++) {
                const int i = lane + 64 * k;
                if (i < n) {
                    v[k] = r[c0 + i];
                    gw[k] = g[c0 + i];
                }
            }
        }
#pragma unroll
        for (int k = 0; k < kV; k++) {
            const int i = lane + 64 * k;
            if (i < n) {
                float4 a;
                a.x = v[k].x * scale; a.y = v[k].y * scale;
                a.z = v[k].z * scale; a.w = v[k].w * scale;
                a.x = a.x * gw[k].x; a.y = a.y * gw[k].y; a.z = a.z * gw[k].z; a.w = a.w * gw[k].w;
                o[c0 + i] = a;
            }
        }
    }
}

}  // namespace rmsnorm_detail

using rmsnorm_detail::kRmsnormLds;
using rmsnorm_detail::rmsnorm_lds;
using rmsnorm_detail::rmsnorm_wave;

}  // namespace lcmoe
