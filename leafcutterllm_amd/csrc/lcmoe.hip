// MoE feed-forward layer for MI355X (gfx950): device kernels and the C ABI
// entry points that launch them.
//
// One forward on one stream:
//   k_router    logits (the reference f32 GEMM order) + top-k + weights
//   k_dispatch  histogram + per-wave stable ranking -> counts/offsets/perm/inv
//   k_gateup    fused dequant-dot gate & up rows + SwiGLU -> H     (per expert)
//   k_down      fused dequant-dot down rows -> Y                   (per expert)
//   k_combine   y[t] = sum_k w[t,k] * Y[inv[t,k]] + sum_s Ysh[s,t] (no atomics)
//
// Compiled with -ffp-contract=off: every fused multiply-add is written as
// __builtin_fmaf, every other a*b+c is two roundings.  That is what makes the
// router logits and the decoders bit-identical to the reference arithmetic.

#include <hip/hip_runtime.h>

#include <climits>
#include <cmath>
#include <mutex>
#include <new>
#include <vector>

#include "lcmoe_internal.h"

using namespace lcmoe;

#define HIP_TRY(expr)                                                                    \
    do {                                                                                 \
        hipError_t e_ = (expr);                                                          \
        if (e_ != hipSuccess)                                                            \
            return fail(LCMOE_ERR_HIP, "%s: %s", #expr, hipGetErrorString(e_));          \
    } while (0)

namespace {

constexpr int kMaxE = 256;
constexpr int kMaxK = 16;

// ---------------------------------------------------------------------------
// device helpers
// ---------------------------------------------------------------------------

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
// multiple of 8) of a GGUF tensor into f32.  Flat indexing is what the
// reference decoders do (kernels/mod.rs: num_blocks = out.len() / QK), so a
// row that starts inside a super-block (d_ff = 1408) decodes correctly.
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

// ---------------------------------------------------------------------------
// k_router: one block per token.
// Logits follow Tensor::matmul -> avx2_matmul (rust/src/kernels/simd.rs:
// 226-249): ascending-k accumulation from 0 with fma for the first 8*(E/8)
// experts, mul-then-add for the rest.  One thread owns one expert's chain.
// ---------------------------------------------------------------------------

struct RouteParams {
    int kind, n_group, topk_group, has_bias;
    float scale;
};

__global__ __launch_bounds__(256) void k_router(const float *__restrict__ x,
                                                const float *__restrict__ wr,
                                                const float *__restrict__ bias, int d, int E, int K,
                                                RouteParams rp, int32_t *__restrict__ topk_idx,
                                                float *__restrict__ topk_w) {
    extern __shared__ float s_x[];
    __shared__ float s_z[kMaxE], s_s[kMaxE], s_g[kMaxE];
    __shared__ unsigned char s_ok[kMaxE];
    __shared__ int s_sel[kMaxK];
    const int t = blockIdx.x, tid = threadIdx.x;
    const float *xr = x + (int64_t)t * d;
    for (int i = tid; i < d; i += blockDim.x) s_x[i] = xr[i];
    __syncthreads();

    if (tid < E) {
        const float *w = wr + tid;
        float acc = 0.0f;
        if (tid < (E & ~7)) {
            for (int k = 0; k < d; k++) acc = __builtin_fmaf(s_x[k], w[(int64_t)k * E], acc);
        } else {
            for (int k = 0; k < d; k++) {
                float p = s_x[k] * w[(int64_t)k * E];
                acc = acc + p;
            }
        }
        float z;
        if (rp.kind == LCMOE_ROUTE_SIGMOID_GROUP) {
            float s = sigmoid_cw(acc);
            s_s[tid] = s;
            z = rp.has_bias ? s + bias[tid] : s;
        } else {
            z = rp.has_bias ? acc + bias[tid] : acc;
        }
        s_z[tid] = z;
        s_ok[tid] = 1;
    }
    __syncthreads();

    if (rp.kind == LCMOE_ROUTE_SIGMOID_GROUP) {
        const int G = rp.n_group, gs = E / G;
        if (tid < G) {  // group score = top-1 z + top-2 z of the group
            int b1 = -1, b2 = -1;
            for (int i = 0; i < gs; i++) {
                int e = tid * gs + i;
                float k = sel_key(s_z[e]);
                if (b1 < 0 || better(k, e, sel_key(s_z[b1]), b1)) {
                    b2 = b1;
                    b1 = e;
                } else if (b2 < 0 || better(k, e, sel_key(s_z[b2]), b2)) {
                    b2 = e;
                }
            }
            s_g[tid] = gs >= 2 ? s_z[b1] + s_z[b2] : s_z[b1];
        }
        __syncthreads();
        if (tid == 0) {  // keep the topk_group best groups (ties -> lower g)
            unsigned char keep[kMaxE];
            for (int g = 0; g < G; g++) keep[g] = 0;
            for (int i = 0; i < rp.topk_group; i++) {
                int best = -1;
                for (int g = 0; g < G; g++) {
                    if (keep[g]) continue;
                    if (best < 0 || better(sel_key(s_g[g]), g, sel_key(s_g[best]), best)) best = g;
                }
                keep[best] = 1;
            }
            for (int g = 0; g < G; g++) s_g[g] = keep[g] ? 1.0f : 0.0f;
        }
        __syncthreads();
        if (tid < E) s_ok[tid] = s_g[tid / gs] != 0.0f;
        __syncthreads();
    }

    if (tid < 64) {  // wave 0: K rounds of wave-wide argmax, ties -> lower e
        const int lane = tid;
        unsigned used = 0;  // bit i: expert lane + 64*i already taken
        for (int slot = 0; slot < K; slot++) {
            float bk = -__builtin_inff();
            int be = INT_MAX;
            for (int i = 0, e = lane; e < E; i++, e += 64) {
                if (!s_ok[e] || (used >> i) & 1u) continue;
                float k = sel_key(s_z[e]);
                if (better(k, e, bk, be)) {
                    bk = k;
                    be = e;
                }
            }
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) {
                float ok = __shfl_xor(bk, off, 64);
                int oe = __shfl_xor(be, off, 64);
                if (better(ok, oe, bk, be)) {
                    bk = ok;
                    be = oe;
                }
            }
            if (be >= E) be = 0;  // unreachable: K <= candidates is validated on the host
            if ((be & 63) == lane) used |= 1u << (be >> 6);
            if (lane == 0) s_sel[slot] = be;
        }
        if (lane == 0) {
            float w[kMaxK];
            if (rp.kind == LCMOE_ROUTE_SIGMOID_GROUP) {
                float sum = 0.0f;
                for (int k = 0; k < K; k++) sum = sum + s_s[s_sel[k]];
                for (int k = 0; k < K; k++) w[k] = (s_s[s_sel[k]] / sum) * rp.scale;
            } else if (rp.kind == LCMOE_ROUTE_SOFTMAX_RENORM) {  // cpu.rs:66-79 over the K
                float mx = -__builtin_inff(), sum = 0.0f;
                for (int k = 0; k < K; k++) mx = nan_max(mx, s_z[s_sel[k]]);
                for (int k = 0; k < K; k++) sum = sum + expf(s_z[s_sel[k]] - mx);
                for (int k = 0; k < K; k++) w[k] = (expf(s_z[s_sel[k]] - mx) / sum) * rp.scale;
            } else {  // full-E softmax probabilities of the selected experts
                float mx = -__builtin_inff(), sum = 0.0f;
                for (int e = 0; e < E; e++) mx = nan_max(mx, s_z[e]);
                for (int e = 0; e < E; e++) sum = sum + expf(s_z[e] - mx);
                for (int k = 0; k < K; k++) w[k] = (expf(s_z[s_sel[k]] - mx) / sum) * rp.scale;
            }
            for (int k = 0; k < K; k++) {
                topk_idx[(int64_t)t * K + k] = s_sel[k];
                topk_w[(int64_t)t * K + k] = w[k];
            }
        }
    }
}

// ---------------------------------------------------------------------------
// k_dispatch: one block of 16 waves.  Stable counting sort of the A = T*K
// assignments by expert.  Each wave owns a contiguous chunk of assignments:
// pass 1 counts per (wave, expert) in LDS, a prefix over waves and experts
// gives every wave its base per expert, pass 2 ranks equal experts inside
// each 64-assignment group with ballots (lower lane = lower a) and advances
// the wave's private counter.  Integer-only, deterministic.
// ---------------------------------------------------------------------------

constexpr int kDispWaves = 16;

__global__ __launch_bounds__(1024) void k_dispatch(const int32_t *__restrict__ topk_idx, int A,
                                                   int E, int32_t *__restrict__ counts,
                                                   int32_t *__restrict__ offsets,
                                                   int32_t *__restrict__ perm,
                                                   int32_t *__restrict__ inv,
                                                   int32_t *__restrict__ touched) {
    __shared__ int s_cw[kDispWaves][kMaxE];
    __shared__ int s_off[kMaxE + 1];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    for (int i = tid; i < kDispWaves * kMaxE; i += blockDim.x) (&s_cw[0][0])[i] = 0;
    __syncthreads();
    const int chunk = (((A + kDispWaves - 1) / kDispWaves) + 63) & ~63;
    const int a0 = min(A, wave * chunk), a1 = min(A, a0 + chunk);
    for (int a = a0 + lane; a < a1; a += 64) atomicAdd(&s_cw[wave][topk_idx[a]], 1);
    __syncthreads();
    if (tid < E) {
        int run = 0;
        for (int w = 0; w < kDispWaves; w++) {
            int c = s_cw[w][tid];
            s_cw[w][tid] = run;
            run += c;
        }
        counts[tid] = run;
        s_off[tid] = run;
    }
    __syncthreads();
    if (tid == 0) {
        int run = 0, nt = 0;
        for (int e = 0; e < E; e++) {
            int c = s_off[e];
            s_off[e] = run;
            offsets[e] = run;
            run += c;
            if (c) touched[nt++] = e;
        }
        s_off[E] = run;
        offsets[E] = run;
        touched[E] = nt;
    }
    __syncthreads();
    for (int base = a0; base < a1; base += 64) {
        const int a = base + lane;
        const bool valid = a < a1;
        const int e = valid ? topk_idx[a] : 0;
        uint64_t mask = __ballot(valid);
#pragma unroll
        for (int b = 0; b < 8; b++) {
            uint64_t bb = __ballot(valid && ((e >> b) & 1));
            mask &= ((e >> b) & 1) ? bb : ~bb;
        }
        if (valid) {
            const int rank = __popcll(mask & ((1ull << lane) - 1ull));
            const int pos = s_off[e] + s_cw[wave][e] + rank;
            perm[pos] = a;
            inv[a] = pos;
            if (rank == 0) s_cw[wave][e] += __popcll(mask);
        }
    }
}

// ---------------------------------------------------------------------------
// Expert products.  Grid (row blocks, slots).  Routed launch: slot i serves
// touched[i] (skips when i >= number touched) over its counts[e] positions
// p in [offsets[e], offsets[e] + counts[e]) whose token is perm[p] / K.
// Shared launch: slot s is shared expert s over all T tokens.
// Each wave owns RB/4 consecutive output rows; its lanes stride the input
// dimension 8 elements at a time, decode those weights to registers and
// accumulate up to NT tokens, then reduce across the wave.
// ---------------------------------------------------------------------------

struct SlotArgs {
    const int32_t *perm, *counts, *offsets, *touched;
    int E, K, T, shared;
};

__device__ __forceinline__ bool slot_info(const SlotArgs &sa, int slot, int &e, int &p0, int &n) {
    if (sa.shared) {
        e = slot;
        p0 = slot * sa.T;
        n = sa.T;
        return true;
    }
    if (slot >= sa.touched[sa.E]) return false;
    e = sa.touched[slot];
    p0 = sa.offsets[e];
    n = sa.counts[e];
    return true;
}

constexpr int kRB = 16;  // output rows per block (4 per wave)
constexpr int kNT = 4;   // tokens per pass

template <int QT>
__global__ __launch_bounds__(256) void k_gateup(const uint8_t *__restrict__ gate,
                                                const uint8_t *__restrict__ up, int64_t estride,
                                                const float *__restrict__ x, SlotArgs sa, int d,
                                                int F, float *__restrict__ H) {
    int e, p0, n;
    if (!slot_info(sa, blockIdx.y, e, p0, n)) return;
    const uint8_t *G = gate + (int64_t)e * estride, *U = up + (int64_t)e * estride;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int ng = d >> 3;
    for (int r = 0; r < kRB / 4; r++) {
        const int f = blockIdx.x * kRB + wave * (kRB / 4) + r;
        if (f >= F) break;
        const int64_t rowbase = (int64_t)f * d;
        for (int c = 0; c < n; c += kNT) {
            const float *xr[kNT];
#pragma unroll
            for (int t = 0; t < kNT; t++) {
                int q = min(c + t, n - 1);
                int tok = sa.shared ? q : sa.perm[p0 + q] / sa.K;
                xr[t] = x + (int64_t)tok * d;
            }
            float ag[kNT] = {}, au[kNT] = {};
            for (int g = lane; g < ng; g += 64) {
                float wg[8], wu[8];
                Dec<QT>::run(G, rowbase + 8 * g, wg);
                Dec<QT>::run(U, rowbase + 8 * g, wu);
#pragma unroll
                for (int t = 0; t < kNT; t++) {
                    const float4 *xp = reinterpret_cast<const float4 *>(xr[t] + 8 * g);
                    float4 a = xp[0], b = xp[1];
                    float xv[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
                    for (int i = 0; i < 8; i++) {
                        ag[t] = __builtin_fmaf(wg[i], xv[i], ag[t]);
                        au[t] = __builtin_fmaf(wu[i], xv[i], au[t]);
                    }
                }
            }
#pragma unroll
            for (int t = 0; t < kNT; t++) {
                float gs = wave_sum(ag[t]), us = wave_sum(au[t]);
                if (lane == 0 && c + t < n) H[(int64_t)(p0 + c + t) * F + f] = silu(gs) * us;
            }
        }
    }
}

template <int QT>
__global__ __launch_bounds__(256) void k_down(const uint8_t *__restrict__ down, int64_t estride,
                                              const float *__restrict__ H, SlotArgs sa, int d,
                                              int F, float *__restrict__ Y) {
    int e, p0, n;
    if (!slot_info(sa, blockIdx.y, e, p0, n)) return;
    const uint8_t *W = down + (int64_t)e * estride;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int ng = F >> 3;
    for (int r = 0; r < kRB / 4; r++) {
        const int row = blockIdx.x * kRB + wave * (kRB / 4) + r;
        if (row >= d) break;
        const int64_t rowbase = (int64_t)row * F;
        for (int c = 0; c < n; c += kNT) {
            float acc[kNT] = {};
            for (int g = lane; g < ng; g += 64) {
                float w[8];
                Dec<QT>::run(W, rowbase + 8 * g, w);
#pragma unroll
                for (int t = 0; t < kNT; t++) {
                    int q = min(c + t, n - 1);
                    const float4 *hp = reinterpret_cast<const float4 *>(H + (int64_t)(p0 + q) * F + 8 * g);
                    float4 a = hp[0], b = hp[1];
                    float hv[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
                    for (int i = 0; i < 8; i++) acc[t] = __builtin_fmaf(w[i], hv[i], acc[t]);
                }
            }
#pragma unroll
            for (int t = 0; t < kNT; t++) {
                float s = wave_sum(acc[t]);
                if (lane == 0 && c + t < n) Y[(int64_t)(p0 + c + t) * d + row] = s;
            }
        }
    }
}

// y[t] = sum_k w[t,k] * Yr[inv[t*K+k]] + sum_s Ysh[s*T + t], slot order then
// shared order, each term rounded then added.
__global__ __launch_bounds__(256) void k_combine(const float *__restrict__ Yr,
                                                 const float *__restrict__ Ys,
                                                 const int32_t *__restrict__ inv,
                                                 const float *__restrict__ topk_w, int T, int K,
                                                 int S, int d, float *__restrict__ y) {
    const int t = blockIdx.x;
    int pos[kMaxK];
    float w[kMaxK];
    for (int k = 0; k < K; k++) {
        pos[k] = inv[(int64_t)t * K + k];
        w[k] = topk_w[(int64_t)t * K + k];
    }
    for (int c = threadIdx.x; c < d; c += blockDim.x) {
        float acc = 0.0f;
        for (int k = 0; k < K; k++) {
            float p = w[k] * Yr[(int64_t)pos[k] * d + c];
            acc = acc + p;
        }
        for (int s = 0; s < S; s++) acc = acc + Ys[((int64_t)s * T + t) * d + c];
        y[(int64_t)t * d + c] = acc;
    }
}

template <int QT>
__global__ void k_debug_dequant(const uint8_t *__restrict__ src, int64_t count,
                                float *__restrict__ out) {
    int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (8 * g >= count) return;
    float o[8];
    Dec<QT>::run(src, 8 * g, o);
    for (int i = 0; i < 8; i++) out[8 * g + i] = o[i];
}

__global__ void k_debug_sigmoid(const float *__restrict__ x, int64_t n, float *__restrict__ out) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = sigmoid_cw(x[i]);
}

// ---------------------------------------------------------------------------
// launch helpers
// ---------------------------------------------------------------------------

enum Slot { kSlotRouter, kSlotDispatch, kSlotGateUp, kSlotGateUpSh, kSlotDown, kSlotDownSh,
            kSlotCombine, kNumSlots };
const char *kSlotNames[kNumSlots] = {"router", "dispatch", "gateup", "gateup_shared",
                                     "down", "down_shared", "combine"};

template <template <int> class K, class... Args>
hipError_t launch_typed(int qt, dim3 grid, dim3 block, hipStream_t st, Args... args) {
    switch (qt) {
    case LCMOE_TYPE_F32: hipLaunchKernelGGL(K<LCMOE_TYPE_F32>::fn, grid, block, 0, st, args...); break;
    case LCMOE_TYPE_Q8_0: hipLaunchKernelGGL(K<LCMOE_TYPE_Q8_0>::fn, grid, block, 0, st, args...); break;
    case LCMOE_TYPE_Q4_K: hipLaunchKernelGGL(K<LCMOE_TYPE_Q4_K>::fn, grid, block, 0, st, args...); break;
    case LCMOE_TYPE_Q6_K: hipLaunchKernelGGL(K<LCMOE_TYPE_Q6_K>::fn, grid, block, 0, st, args...); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int QT> struct GateUpK { static constexpr auto fn = k_gateup<QT>; };
template <int QT> struct DownK { static constexpr auto fn = k_down<QT>; };
template <int QT> struct DeqK { static constexpr auto fn = k_debug_dequant<QT>; };

}  // namespace

// ---------------------------------------------------------------------------
// handle
// ---------------------------------------------------------------------------

struct lcmoe_handle {
    lcmoe_desc desc{};
    int device = 0;
    hipStream_t stream = nullptr;
    std::vector<void *> allocs;
    float *router = nullptr, *bias = nullptr;
    uint8_t *gate = nullptr, *up = nullptr, *down = nullptr;
    uint8_t *gate_sh = nullptr, *up_sh = nullptr, *down_sh = nullptr;
    int64_t sz_g = 0, sz_u = 0, sz_d = 0, sz_gs = 0, sz_us = 0, sz_ds = 0;
    float *x_dev = nullptr, *y_dev = nullptr;
    int32_t *topk_idx = nullptr, *counts = nullptr, *offsets = nullptr, *perm = nullptr,
            *inv = nullptr, *touched = nullptr;
    float *topk_w = nullptr, *Hr = nullptr, *Hs = nullptr, *Yr = nullptr, *Ys = nullptr;
    int last_T = -1;
    hipStream_t last_stream = nullptr;
    bool timing = false;
    struct Pending { int slot; hipEvent_t a, b; };
    std::vector<Pending> pending;
    std::vector<hipEvent_t> event_pool;
    double t_ms[kNumSlots] = {};
    int64_t t_n[kNumSlots] = {};
};

namespace {

lcmoe_status dev_alloc(lcmoe_handle *h, void **p, size_t bytes) {
    *p = nullptr;
    if (bytes == 0) bytes = 256;
    hipError_t e = hipMalloc(p, bytes);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return fail(e == hipErrorOutOfMemory ? LCMOE_ERR_OUT_OF_MEMORY : LCMOE_ERR_HIP,
                    "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
    }
    h->allocs.push_back(*p);
    return LCMOE_OK;
}

template <class T>
lcmoe_status upload(lcmoe_handle *h, T **dst, const void *src, size_t bytes) {
    void *p;
    lcmoe_status st = dev_alloc(h, &p, bytes);
    if (st) return st;
    *dst = static_cast<T *>(p);
    if (src && bytes) HIP_TRY(hipMemcpy(p, src, bytes, hipMemcpyHostToDevice));
    return LCMOE_OK;
}

void free_handle(lcmoe_handle *h) {
    if (!h) return;
    if (h->stream) (void)hipStreamSynchronize(h->stream);
    for (auto &p : h->pending) {
        (void)hipEventDestroy(p.a);
        (void)hipEventDestroy(p.b);
    }
    for (auto ev : h->event_pool) (void)hipEventDestroy(ev);
    for (void *p : h->allocs) (void)hipFree(p);
    if (h->stream) (void)hipStreamDestroy(h->stream);
    delete h;
}

hipEvent_t take_event(lcmoe_handle *h) {
    if (!h->event_pool.empty()) {
        hipEvent_t e = h->event_pool.back();
        h->event_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

// Wraps one launch with timing events when timing is on.
template <class Fn>
hipError_t timed(lcmoe_handle *h, hipStream_t st, int slot, Fn fn) {
    if (!h->timing) return fn();
    hipEvent_t a = take_event(h), b = take_event(h);
    if (!a || !b) return fn();
    (void)hipEventRecord(a, st);
    hipError_t e = fn();
    (void)hipEventRecord(b, st);
    h->pending.push_back({slot, a, b});
    return e;
}

}  // namespace

extern "C" lcmoe_status lcmoe_create(const lcmoe_desc *desc, const lcmoe_weights *w,
                                     lcmoe_handle **out) {
    clear_error();
    if (!out) return fail(LCMOE_ERR_INVALID_ARG, "out is NULL");
    *out = nullptr;
    lcmoe_status st = validate_desc(desc);
    if (st) return st;
    if (desc->type_gate != desc->type_up || (desc->n_shared && desc->type_gate_sh != desc->type_up_sh))
        return fail(LCMOE_ERR_UNSUPPORTED, "gate and up must share a quant type");
    if ((st = scan_weights(desc, w))) return st;

    int ndev = 0;
    hipError_t he = hipGetDeviceCount(&ndev);
    if (he != hipSuccess || ndev < 1) {
        (void)hipGetLastError();
        return fail(LCMOE_ERR_HIP, "no HIP device available (%s)", hipGetErrorString(he));
    }
    lcmoe_handle *h = new (std::nothrow) lcmoe_handle();
    if (!h) return fail(LCMOE_ERR_OUT_OF_MEMORY, "host allocation failed");
    h->desc = *desc;
    const lcmoe_desc &D = h->desc;
    auto bail = [&](lcmoe_status s) {
        free_handle(h);
        return s;
    };
    if (hipGetDevice(&h->device) != hipSuccess) return bail(fail(LCMOE_ERR_HIP, "hipGetDevice failed"));
    if (hipStreamCreateWithFlags(&h->stream, hipStreamNonBlocking) != hipSuccess)
        return bail(fail(LCMOE_ERR_HIP, "hipStreamCreate failed"));

    const int64_t d = D.d_model, F = D.d_ff, E = D.n_expert, K = D.n_expert_used, S = D.n_shared,
                  FS = D.d_ff_shared, Tm = D.max_tokens;
    h->sz_g = (int64_t)lcmoe_tensor_size(D.type_gate, F * d);
    h->sz_u = (int64_t)lcmoe_tensor_size(D.type_up, F * d);
    h->sz_d = (int64_t)lcmoe_tensor_size(D.type_down, d * F);
    if ((st = upload(h, &h->router, w->router, sizeof(float) * d * E))) return bail(st);
    if (D.has_bias && (st = upload(h, &h->bias, w->bias, sizeof(float) * E))) return bail(st);
    if ((st = upload(h, &h->gate, w->gate, h->sz_g * E))) return bail(st);
    if ((st = upload(h, &h->up, w->up, h->sz_u * E))) return bail(st);
    if ((st = upload(h, &h->down, w->down, h->sz_d * E))) return bail(st);
    if (S > 0) {
        h->sz_gs = (int64_t)lcmoe_tensor_size(D.type_gate_sh, FS * d);
        h->sz_us = (int64_t)lcmoe_tensor_size(D.type_up_sh, FS * d);
        h->sz_ds = (int64_t)lcmoe_tensor_size(D.type_down_sh, d * FS);
        if ((st = upload(h, &h->gate_sh, w->gate_sh, h->sz_gs * S))) return bail(st);
        if ((st = upload(h, &h->up_sh, w->up_sh, h->sz_us * S))) return bail(st);
        if ((st = upload(h, &h->down_sh, w->down_sh, h->sz_ds * S))) return bail(st);
    }
    const int64_t A = Tm * K;
    if ((st = upload(h, &h->x_dev, nullptr, sizeof(float) * Tm * d))) return bail(st);
    if ((st = upload(h, &h->y_dev, nullptr, sizeof(float) * Tm * d))) return bail(st);
    if ((st = upload(h, &h->topk_idx, nullptr, sizeof(int32_t) * A))) return bail(st);
    if ((st = upload(h, &h->topk_w, nullptr, sizeof(float) * A))) return bail(st);
    if ((st = upload(h, &h->counts, nullptr, sizeof(int32_t) * E))) return bail(st);
    if ((st = upload(h, &h->offsets, nullptr, sizeof(int32_t) * (E + 1)))) return bail(st);
    if ((st = upload(h, &h->perm, nullptr, sizeof(int32_t) * A))) return bail(st);
    if ((st = upload(h, &h->inv, nullptr, sizeof(int32_t) * A))) return bail(st);
    if ((st = upload(h, &h->touched, nullptr, sizeof(int32_t) * (E + 1)))) return bail(st);
    if ((st = upload(h, &h->Hr, nullptr, sizeof(float) * A * F))) return bail(st);
    if ((st = upload(h, &h->Yr, nullptr, sizeof(float) * A * d))) return bail(st);
    if (S > 0) {
        if ((st = upload(h, &h->Hs, nullptr, sizeof(float) * S * Tm * FS))) return bail(st);
        if ((st = upload(h, &h->Ys, nullptr, sizeof(float) * S * Tm * d))) return bail(st);
    }
    *out = h;
    return LCMOE_OK;
}

extern "C" void lcmoe_destroy(lcmoe_handle *h) { free_handle(h); }

static lcmoe_status enqueue_forward(lcmoe_handle *h, const float *x, int32_t T, float *y,
                                    hipStream_t st) {
    const lcmoe_desc &D = h->desc;
    const int d = D.d_model, F = D.d_ff, E = D.n_expert, K = D.n_expert_used, S = D.n_shared,
              FS = D.d_ff_shared;
    RouteParams rp{D.route_kind, D.n_group, D.topk_group, D.has_bias, D.routed_scale};
    HIP_TRY(timed(h, st, kSlotRouter, [&] {
        hipLaunchKernelGGL(k_router, dim3(T), dim3(256), sizeof(float) * d, st, x, h->router,
                           h->bias, d, E, K, rp, h->topk_idx, h->topk_w);
        return hipGetLastError();
    }));
    HIP_TRY(timed(h, st, kSlotDispatch, [&] {
        hipLaunchKernelGGL(k_dispatch, dim3(1), dim3(1024), 0, st, h->topk_idx, T * K, E,
                           h->counts, h->offsets, h->perm, h->inv, h->touched);
        return hipGetLastError();
    }));
    const int slots = std::min(E, T * K);
    SlotArgs sr{h->perm, h->counts, h->offsets, h->touched, E, K, T, 0};
    SlotArgs ss{h->perm, h->counts, h->offsets, h->touched, E, K, T, 1};
    HIP_TRY(timed(h, st, kSlotGateUp, [&] {
        return launch_typed<GateUpK>(D.type_gate, dim3((F + kRB - 1) / kRB, slots), dim3(256), st,
                                     (const uint8_t *)h->gate, (const uint8_t *)h->up, h->sz_g, x,
                                     sr, d, F, h->Hr);
    }));
    if (S > 0)
        HIP_TRY(timed(h, st, kSlotGateUpSh, [&] {
            return launch_typed<GateUpK>(D.type_gate_sh, dim3((FS + kRB - 1) / kRB, S), dim3(256),
                                         st, (const uint8_t *)h->gate_sh, (const uint8_t *)h->up_sh,
                                         h->sz_gs, x, ss, d, FS, h->Hs);
        }));
    HIP_TRY(timed(h, st, kSlotDown, [&] {
        return launch_typed<DownK>(D.type_down, dim3((d + kRB - 1) / kRB, slots), dim3(256), st,
                                   (const uint8_t *)h->down, h->sz_d, (const float *)h->Hr, sr, d,
                                   F, h->Yr);
    }));
    if (S > 0)
        HIP_TRY(timed(h, st, kSlotDownSh, [&] {
            return launch_typed<DownK>(D.type_down_sh, dim3((d + kRB - 1) / kRB, S), dim3(256), st,
                                       (const uint8_t *)h->down_sh, h->sz_ds, (const float *)h->Hs,
                                       ss, d, FS, h->Ys);
        }));
    HIP_TRY(timed(h, st, kSlotCombine, [&] {
        hipLaunchKernelGGL(k_combine, dim3(T), dim3(256), 0, st, (const float *)h->Yr,
                           (const float *)h->Ys, h->inv, h->topk_w, T, K, S, d, y);
        return hipGetLastError();
    }));
    h->last_T = T;
    h->last_stream = st;
    return LCMOE_OK;
}

extern "C" lcmoe_status lcmoe_forward_dev(lcmoe_handle *h, const float *x_dev, int32_t T,
                                          float *y_dev, void *stream) {
    clear_error();
    if (!h) return fail(LCMOE_ERR_INVALID_ARG, "handle is NULL");
    if (T < 0 || T > h->desc.max_tokens)
        return fail(LCMOE_ERR_INVALID_ARG, "T=%d outside [0, max_tokens=%d]", T, h->desc.max_tokens);
    if (T > 0 && (!x_dev || !y_dev)) return fail(LCMOE_ERR_INVALID_ARG, "x or y is NULL");
    HIP_TRY(hipSetDevice(h->device));
    hipStream_t st = stream ? (hipStream_t)stream : h->stream;
    if (T == 0) {
        h->last_T = 0;
        h->last_stream = st;
        return LCMOE_OK;
    }
    return enqueue_forward(h, x_dev, T, y_dev, st);
}

extern "C" lcmoe_status lcmoe_forward(lcmoe_handle *h, const float *x, int32_t T, float *y,
                                      int32_t *topk_idx, float *topk_w) {
    clear_error();
    if (!h) return fail(LCMOE_ERR_INVALID_ARG, "handle is NULL");
    if (T < 0 || T > h->desc.max_tokens)
        return fail(LCMOE_ERR_INVALID_ARG, "T=%d outside [0, max_tokens=%d]", T, h->desc.max_tokens);
    HIP_TRY(hipSetDevice(h->device));
    if (T == 0) {
        h->last_T = 0;
        h->last_stream = h->stream;
        return LCMOE_OK;
    }
    if (!x || !y) return fail(LCMOE_ERR_INVALID_ARG, "x or y is NULL");
    const size_t xb = sizeof(float) * (size_t)T * h->desc.d_model;
    const size_t kb = (size_t)T * h->desc.n_expert_used;
    HIP_TRY(hipMemcpyAsync(h->x_dev, x, xb, hipMemcpyHostToDevice, h->stream));
    lcmoe_status st = enqueue_forward(h, h->x_dev, T, h->y_dev, h->stream);
    if (st) return st;
    HIP_TRY(hipMemcpyAsync(y, h->y_dev, xb, hipMemcpyDeviceToHost, h->stream));
    if (topk_idx)
        HIP_TRY(hipMemcpyAsync(topk_idx, h->topk_idx, kb * 4, hipMemcpyDeviceToHost, h->stream));
    if (topk_w) HIP_TRY(hipMemcpyAsync(topk_w, h->topk_w, kb * 4, hipMemcpyDeviceToHost, h->stream));
    HIP_TRY(hipStreamSynchronize(h->stream));
    return LCMOE_OK;
}

extern "C" lcmoe_status lcmoe_get_dispatch(lcmoe_handle *h, int32_t *T_out, int32_t *topk_idx,
                                           float *topk_w, int32_t *counts, int32_t *offsets,
                                           int32_t *perm, int32_t *inv) {
    clear_error();
    if (!h) return fail(LCMOE_ERR_INVALID_ARG, "handle is NULL");
    if (h->last_T < 0) return fail(LCMOE_ERR_STATE, "no forward has run on this handle");
    HIP_TRY(hipSetDevice(h->device));
    HIP_TRY(hipStreamSynchronize(h->last_stream));
    const int T = h->last_T, K = h->desc.n_expert_used, E = h->desc.n_expert;
    if (T_out) *T_out = T;
    const size_t A = (size_t)T * K;
    if (T == 0) {
        if (counts) std::memset(counts, 0, sizeof(int32_t) * E);
        if (offsets) std::memset(offsets, 0, sizeof(int32_t) * (E + 1));
        return LCMOE_OK;
    }
    if (topk_idx) HIP_TRY(hipMemcpy(topk_idx, h->topk_idx, A * 4, hipMemcpyDeviceToHost));
    if (topk_w) HIP_TRY(hipMemcpy(topk_w, h->topk_w, A * 4, hipMemcpyDeviceToHost));
    if (counts) HIP_TRY(hipMemcpy(counts, h->counts, (size_t)E * 4, hipMemcpyDeviceToHost));
    if (offsets) HIP_TRY(hipMemcpy(offsets, h->offsets, (size_t)(E + 1) * 4, hipMemcpyDeviceToHost));
    if (perm) HIP_TRY(hipMemcpy(perm, h->perm, A * 4, hipMemcpyDeviceToHost));
    if (inv) HIP_TRY(hipMemcpy(inv, h->inv, A * 4, hipMemcpyDeviceToHost));
    return LCMOE_OK;
}

extern "C" lcmoe_status lcmoe_set_timing(lcmoe_handle *h, int32_t enable) {
    clear_error();
    if (!h) return fail(LCMOE_ERR_INVALID_ARG, "handle is NULL");
    h->timing = enable != 0;
    return LCMOE_OK;
}

extern "C" lcmoe_status lcmoe_get_timing(lcmoe_handle *h, int32_t n_slots, double *ms,
                                         int64_t *launches) {
    clear_error();
    if (!h) return fail(LCMOE_ERR_INVALID_ARG, "handle is NULL");
    HIP_TRY(hipSetDevice(h->device));
    for (auto &p : h->pending) {
        HIP_TRY(hipEventSynchronize(p.b));
        float t = 0.0f;
        HIP_TRY(hipEventElapsedTime(&t, p.a, p.b));
        h->t_ms[p.slot] += t;
        h->t_n[p.slot] += 1;
        h->event_pool.push_back(p.a);
        h->event_pool.push_back(p.b);
    }
    h->pending.clear();
    for (int i = 0; i < n_slots && i < kNumSlots; i++) {
        if (ms) ms[i] = h->t_ms[i];
        if (launches) launches[i] = h->t_n[i];
        h->t_ms[i] = 0.0;
        h->t_n[i] = 0;
    }
    return LCMOE_OK;
}

extern "C" const char *lcmoe_timing_name(int32_t slot) {
    return (slot >= 0 && slot < kNumSlots) ? kSlotNames[slot] : "";
}

extern "C" int32_t lcmoe_timing_slots(void) { return kNumSlots; }

extern "C" lcmoe_status lcmoe_debug_dequant(int32_t type, const uint8_t *data, int64_t count,
                                            float *out) {
    clear_error();
    if (!data || !out || count <= 0 || count % 8)
        return fail(LCMOE_ERR_INVALID_ARG, "bad arguments");
    int64_t bs = block_size(type);
    if (!bs) return fail(LCMOE_ERR_UNSUPPORTED, "type %d", type);
    if (count % bs) return fail(LCMOE_ERR_INVALID_ARG, "count not a whole number of blocks");
    size_t nbytes = lcmoe_tensor_size(type, count);
    void *src = nullptr, *dst = nullptr;
    HIP_TRY(hipMalloc(&src, nbytes + 16));
    hipError_t e = hipMalloc(&dst, sizeof(float) * count);
    if (e == hipSuccess) e = hipMemcpy(src, data, nbytes, hipMemcpyHostToDevice);
    if (e == hipSuccess) {
        int64_t groups = count / 8;
        e = launch_typed<DeqK>(type, dim3((unsigned)((groups + 255) / 256)), dim3(256), nullptr,
                               (const uint8_t *)src, count, (float *)dst);
    }
    if (e == hipSuccess) e = hipMemcpy(out, dst, sizeof(float) * count, hipMemcpyDeviceToHost);
    (void)hipFree(src);
    if (dst) (void)hipFree(dst);
    if (e != hipSuccess) return fail(LCMOE_ERR_HIP, "debug_dequant: %s", hipGetErrorString(e));
    return LCMOE_OK;
}

extern "C" lcmoe_status lcmoe_debug_sigmoid(const float *x, int64_t n, float *out) {
    clear_error();
    if (!x || !out || n <= 0) return fail(LCMOE_ERR_INVALID_ARG, "bad arguments");
    void *a = nullptr, *b = nullptr;
    HIP_TRY(hipMalloc(&a, sizeof(float) * n));
    hipError_t e = hipMalloc(&b, sizeof(float) * n);
    if (e == hipSuccess) e = hipMemcpy(a, x, sizeof(float) * n, hipMemcpyHostToDevice);
    if (e == hipSuccess) {
        hipLaunchKernelGGL(k_debug_sigmoid, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, nullptr,
                           (const float *)a, n, (float *)b);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipMemcpy(out, b, sizeof(float) * n, hipMemcpyDeviceToHost);
    (void)hipFree(a);
    if (b) (void)hipFree(b);
    if (e != hipSuccess) return fail(LCMOE_ERR_HIP, "debug_sigmoid: %s", hipGetErrorString(e));
    return LCMOE_OK;
}
