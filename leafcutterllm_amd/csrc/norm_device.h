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
// 64 terms, which adds exactly nothing: the sums are never -0); then the
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
__device__ __forceinline__ float div_rn_pos(float a, float b) {
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
__device__ __forceinline__ float sqrt_rn(float m) {
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
// One lane's chain: acc + c[0].x + c[0].y + ... + c[n16 - 1].w in order
// (n16 a positive multiple of 16 float4s).  Each step issues 16 LDS reads at
// once and adds their 64 terms as they land (the waits count down the reads
// in order), so one read latency is exposed per 64 dependent adds.  Reads
// carried in registers from one step into the next would hide that latency
// too, but the register allocator then copies them between steps, behind
// waits, which costs more than it saves.
__device__ __forceinline__ float chain_sum(const float4 *c, int n16, float acc) {
    for (int gi = 0; gi < n16; gi += 16) {
        float4 a[16];
#pragma unroll
        for (int u = 0; u < 16; u++) a[u] = c[gi + u];
#pragma unroll
        for (int u = 0; u < 16; u++) {
            acc = acc + a[u].x;
            acc = acc + a[u].y;
            acc = acc + a[u].z;
            acc = acc + a[u].w;
        }
    }
    return acc;
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
        // q: the chunk's float4 count rounded up to whole pairs of groups of 8
        // per chain
        const int n = min(kNormChunk / 4, n4 - c0), q = (n + 63) & ~63;
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
        if (lane < 4) acc = chain_sum(reinterpret_cast<const float4 *>(s_sq + lane * ld), q / 4, acc);
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

// The same norm by a block of NT threads (a multiple of 64, >= 64): every
// thread loads, squares and later scales its float4s i = tid, tid + NT, ...
// (held in registers: at most kBlockPer per thread, d <= 4 NT kBlockPer),
// and the chains run on lanes 0-3 of the first wave exactly as
// rmsnorm_wave's (the same LDS layout, the same padding, the same order), so
// the bits are the same.  s_sq: rmsnorm_block_lds(d) floats; s_scale: one
// float of LDS.  x may be a row the block has just written (callers fence).
constexpr int kBlockPer = 8;  // d <= 8192 with 256 threads
__host__ __device__ constexpr int rmsnorm_block_lds(int d) { return 4 * (d / 4 + 64 + 4); }

template <int NT>
__device__ __attribute__((always_inline)) inline void rmsnorm_block(const float *__restrict__ x, const float *__restrict__ w,
                                     float eps, int d, float *__restrict__ out, float *s_sq,
                                     float *s_scale) {
    const int tid = threadIdx.x, n4 = d >> 2, q = (n4 + 63) & ~63, ld = n4 + 64 + 4;
    const float4 *r = reinterpret_cast<const float4 *>(x);
    const float4 *g = reinterpret_cast<const float4 *>(w);
    // the row and the weights in flight together; a thread past the end
    // re-reads the last float4 (branch-free loads keep the waits partial)
    float4 v[kBlockPer], gw[kBlockPer];
#pragma unroll
    for (int k = 0; k < kBlockPer; k++)
        if (NT * k < n4) v[k] = r[min(tid + NT * k, n4 - 1)];
#pragma unroll
    for (int k = 0; k < kBlockPer; k++)
        if (NT * k < n4) gw[k] = g[min(tid + NT * k, n4 - 1)];
#pragma unroll
    for (int k = 0; k < kBlockPer; k++) {
        const int i = tid + NT * k;
        if (i < n4) {
            s_sq[i] = v[k].x * v[k].x;
            s_sq[ld + i] = v[k].y * v[k].y;
            s_sq[2 * ld + i] = v[k].z * v[k].z;
            s_sq[3 * ld + i] = v[k].w * v[k].w;
        } else if (i < q) {  // chain padding: adds exactly nothing
            s_sq[i] = s_sq[ld + i] = s_sq[2 * ld + i] = s_sq[3 * ld + i] = 0.0f;
        }
    }
    if (NT * kBlockPer < q)  // padding past the threads' float4s (d close to the limit)
        for (int i = NT * kBlockPer + tid; i < q; i += NT)
            s_sq[i] = s_sq[ld + i] = s_sq[2 * ld + i] = s_sq[3 * ld + i] = 0.0f;
    __syncthreads();
    if (tid < 64) {
        const int lane = tid;
        float acc = 0.0f;
        if (lane < 4 && q > 0)
            acc = chain_sum(reinterpret_cast<const float4 *>(s_sq + lane * ld), q / 4, acc);
        float sum = 0.0f;
        for (int j = 0; j < 4; j++) sum = sum + __shfl(acc, j);
        if (lane == 0) {
            const float mean = div_rn_pos(sum, (float)d);
            const float root = sqrt_rn(mean + eps);
            *s_scale = root > 0.0f ? div_rn_pos(1.0f, root) : 1.0f / root;
        }
    }
    __syncthreads();
    const float scale = *s_scale;
    float4 *o = reinterpret_cast<float4 *>(out);
#pragma unroll
    for (int k = 0; k < kBlockPer; k++) {
        const int i = tid + NT * k;
        if (i < n4) {
            float4 a;
            a.x = v[k].x * scale; a.y = v[k].y * scale;
            a.z = v[k].z * scale; a.w = v[k].w * scale;
            a.x = a.x * gw[k].x; a.y = a.y * gw[k].y; a.z = a.z * gw[k].z; a.w = a.w * gw[k].w;
            o[i] = a;
        }
    }
}

}  // namespace rmsnorm_detail

using rmsnorm_detail::kRmsnormLds;
using rmsnorm_detail::rmsnorm_lds;
using rmsnorm_detail::rmsnorm_wave;
using rmsnorm_detail::rmsnorm_block;
using rmsnorm_detail::rmsnorm_block_lds;
using rmsnorm_detail::kBlockPer;

}  // namespace lcmoe
