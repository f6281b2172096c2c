// Router, activation quantisation, top-k and dispatch: one launch.
//
// Grid (token groups, expert groups).  A block owns TB tokens x EG experts:
//   1. stages its x rows and its experts' router rows in LDS
//      (router transposed to [E, d] at upload so an expert's row is
//      contiguous);
//   2. one thread per (token, expert) runs the logit as the reference GEMM
//      does (Tensor::matmul -> avx2_matmul, rust/src/kernels/simd.rs:226-249):
//      ascending k from 0, fma for experts < 8*(E/8), mul-then-add for the
//      rest; the order is sequential by definition, so this chain is the
//      latency floor of the launch;
//   3. the expert-group-0 block also writes x as two int8 limbs per
//      32-element sub-block for the integer decode kernels;
//   4. the last block to finish a token group (atomic counter) selects top-k
//      for those tokens, one wave per token;
//   5. the last token group to finish runs the stable counting-sort dispatch.
// Counters are reset by the blocks that consume them, so the next launch on
// the stream starts from zero.

#include "device_common.h"
#include "kernels.h"

namespace lcmoe {
namespace {

constexpr int kThreads = 256;
constexpr int kEG = 8;             // max experts per block
constexpr int kPad = 4;            // LDS row padding (floats) against bank conflicts
constexpr int kSlack = 16;         // floats past the last LDS row (chain prefetch overrun)
constexpr int kLdsFloats = 32768;  // dynamic LDS budget: x rows + router rows

__device__ void select_token(const RouterArgs &a, int t, float *s_z, float *s_s, float *s_g,
                             unsigned char *s_ok, int *s_sel) {
    // one wave: lane-strided over experts; s_* are this wave's LDS rows
    const int lane = threadIdx.x & 63, E = a.E, K = a.K;
    const RouteParams &rp = a.rp;
    const float *l = a.logits + (int64_t)t * E;
    for (int e = lane; e < E; e += 64) {
        float v = l[e], z;
        if (rp.kind == LCMOE_ROUTE_SIGMOID_GROUP) {
            float s = sigmoid_cw(v);
            s_s[e] = s;
            z = rp.has_bias ? s + a.bias[e] : s;
        } else {
            z = rp.has_bias ? v + a.bias[e] : v;
        }
        s_z[e] = z;
        s_ok[e] = 1;
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    if (rp.kind == LCMOE_ROUTE_SIGMOID_GROUP) {
        const int G = rp.n_group, gs = E / G;
        for (int g = lane; g < G; g += 64) {  // group score = top-1 z + top-2 z
            int b1 = -1, b2 = -1;
            for (int i = 0; i < gs; i++) {
                int e = g * gs + i;
                float k = sel_key(s_z[e]);
                if (b1 < 0 || better(k, e, sel_key(s_z[b1]), b1)) {
                    b2 = b1;
                    b1 = e;
                } else if (b2 < 0 || better(k, e, sel_key(s_z[b2]), b2)) {
                    b2 = e;
                }
            }
            s_g[g] = gs >= 2 ? s_z[b1] + s_z[b2] : s_z[b1];
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        // keep the topk_group best groups (ties -> lower group index)
        unsigned long long keep = 0;  // G <= 64 groups supported here
        for (int i = 0; i < rp.topk_group; i++) {
            float bk = -__builtin_inff();
            int bg = INT_MAX;
            for (int g = lane; g < G; g += 64) {
                if ((keep >> g) & 1ull) continue;
                float k = sel_key(s_g[g]);
                if (better(k, g, bk, bg)) {
                    bk = k;
                    bg = g;
                }
            }
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) {
                float ok = __shfl_xor(bk, off, 64);
                int og = __shfl_xor(bg, off, 64);
                if (better(ok, og, bk, bg)) {
                    bk = ok;
                    bg = og;
                }
            }
            if (bg < G) keep |= 1ull << bg;
        }
        for (int e = lane; e < E; e += 64) s_ok[e] = (keep >> (e / gs)) & 1ull;
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    }
    // K rounds of wave-wide argmax, ties -> lower expert index
    unsigned used = 0;  // bit i: expert lane + 64*i taken
    for (int slot = 0; slot < K; slot++) {
        float bk = -__builtin_inff();
        int be = INT_MAX;
        for (int i = 0, e = lane; e < E; i++, e += 64) {
            if (!s_ok[e] || ((used >> i) & 1u)) continue;
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
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    if (lane == 0) {
        int32_t *oi = a.topk_idx + (int64_t)t * K;
        float *ow = a.topk_w + (int64_t)t * K;
        if (rp.kind == LCMOE_ROUTE_SIGMOID_GROUP) {
            float sum = 0.0f;
            for (int k = 0; k < K; k++) sum = sum + s_s[s_sel[k]];
            for (int k = 0; k < K; k++) ow[k] = (s_s[s_sel[k]] / sum) * rp.scale;
        } else if (rp.kind == LCMOE_ROUTE_SOFTMAX_RENORM) {  // cpu.rs:66-79 over the K
            float mx = -__builtin_inff(), sum = 0.0f;
            for (int k = 0; k < K; k++) mx = nan_max(mx, s_z[s_sel[k]]);
            for (int k = 0; k < K; k++) sum = sum + expf(s_z[s_sel[k]] - mx);
            for (int k = 0; k < K; k++) ow[k] = (expf(s_z[s_sel[k]] - mx) / sum) * rp.scale;
        } else {  // full-E softmax probabilities of the selected experts
            float mx = -__builtin_inff(), sum = 0.0f;
            for (int e = 0; e < E; e++) mx = nan_max(mx, s_z[e]);
            for (int e = 0; e < E; e++) sum = sum + expf(s_z[e] - mx);
            for (int k = 0; k < K; k++) ow[k] = (expf(s_z[s_sel[k]] - mx) / sum) * rp.scale;
        }
        for (int k = 0; k < K; k++) oi[k] = s_sel[k];
    }
}

// Stable counting sort of the A = T*K assignments a = t*K + k by expert, by
// the 4 waves of one block.  Each wave owns a contiguous chunk: pass 1 counts
// per (wave, expert), prefixes over waves and experts give each wave its base
// per expert, pass 2 ranks equal experts inside each 64-assignment group with
// ballots (lower lane = lower a) and advances the wave's private counters.
__device__ void dispatch_block(const RouterArgs &a, int (*s_cw)[kMaxE], int *s_off) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int A = a.T * a.K, E = a.E;
    constexpr int W = kThreads / 64;
    for (int i = tid; i < W * kMaxE; i += kThreads) (&s_cw[0][0])[i] = 0;
    __syncthreads();
    const int chunk = (((A + W - 1) / W) + 63) & ~63;
    const int a0 = min(A, wave * chunk), a1 = min(A, a0 + chunk);
    for (int q = a0 + lane; q < a1; q += 64) atomicAdd(&s_cw[wave][a.topk_idx[q]], 1);
    __syncthreads();
    if (tid < E) {
        int run = 0;
        for (int w = 0; w < W; w++) {
            int c = s_cw[w][tid];
            s_cw[w][tid] = run;
            run += c;
        }
        a.counts[tid] = run;
        s_off[tid] = run;
    }
    __syncthreads();
    if (tid == 0) {
        int run = 0, nt = 0;
        for (int e = 0; e < E; e++) {
            int c = s_off[e];
            s_off[e] = run;
            a.offsets[e] = run;
            run += c;
            if (c) a.touched[nt++] = e;
        }
        s_off[E] = run;
        a.offsets[E] = run;
        a.touched[E] = nt;
    }
    __syncthreads();
    for (int base = a0; base < a1; base += 64) {
        const int q = base + lane;
        const bool valid = q < a1;
        const int e = valid ? a.topk_idx[q] : 0;
        uint64_t mask = __ballot(valid);
#pragma unroll
        for (int b = 0; b < 8; b++) {
            uint64_t bb = __ballot(valid && ((e >> b) & 1));
            mask &= ((e >> b) & 1) ? bb : ~bb;
        }
        if (valid) {
            const int rank = __popcll(mask & ((1ull << lane) - 1ull));
            const int pos = s_off[e] + s_cw[wave][e] + rank;
            a.perm[pos] = q;
            a.inv[q] = pos;
            if (rank == 0) s_cw[wave][e] += __popcll(mask);
        }
    }
}

// rows x d floats from global (row-major) into LDS rows of `stride` floats
__device__ __forceinline__ void stage_rows(const float *__restrict__ src, float *dst, int rows,
                                           int d, int stride, int tid) {
    const int d4 = d / 4, n = rows * d4;
    for (int base = 0; base < n; base += 8 * kThreads) {
        float4 v[8];
#pragma unroll
        for (int i = 0; i < 8; i++)
            v[i] = reinterpret_cast<const float4 *>(src)[min(base + tid + i * kThreads, n - 1)];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int q = base + tid + i * kThreads;
            if (q < n) *reinterpret_cast<float4 *>(&dst[(q / d4) * stride + 4 * (q % d4)]) = v[i];
        }
    }
}

template <bool FMA>
__device__ __forceinline__ float step4(float4 x, float4 w, float acc) {
    if (FMA) {
        acc = __builtin_fmaf(x.x, w.x, acc);
        acc = __builtin_fmaf(x.y, w.y, acc);
        acc = __builtin_fmaf(x.z, w.z, acc);
        return __builtin_fmaf(x.w, w.w, acc);
    }
    float p;
    p = x.x * w.x; acc = acc + p;
    p = x.y * w.y; acc = acc + p;
    p = x.z * w.z; acc = acc + p;
    p = x.w * w.w; acc = acc + p;
    return acc;
}

// Ascending-k chain over n4 float4 steps (n4 % 8 == 0), operands fetched in
// groups of 4 float4 (16 k) one group ahead of use.
template <bool FMA>
__device__ __forceinline__ float chain16(const float4 *xr, const float4 *wr, int n4, float acc) {
    float4 xa[4], wa[4], xb[4], wb[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        xa[i] = xr[i];
        wa[i] = wr[i];
    }
    // the last iteration prefetches 4 float4 past the row: the LDS rows are
    // padded (kSlack) so those reads stay inside the allocation and are unused
    for (int q = 0; q < n4; q += 8) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            xb[i] = xr[q + 4 + i];
            wb[i] = wr[q + 4 + i];
        }
#pragma unroll
        for (int i = 0; i < 4; i++) acc = step4<FMA>(xa[i], wa[i], acc);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            xa[i] = xr[q + 8 + i];
            wa[i] = wr[q + 8 + i];
        }
#pragma unroll
        for (int i = 0; i < 4; i++) acc = step4<FMA>(xb[i], wb[i], acc);
    }
    return acc;
}

__global__ __launch_bounds__(kThreads) void k_router(RouterArgs a, int TB, int EG) {
    extern __shared__ float smem[];
    const int d = a.d, E = a.E, stride = d + kPad;
    float *s_x = smem;                // [TB][d + pad]
    float *s_w = smem + TB * stride;  // [EG][d + pad], this block's router rows
    __shared__ float s_z[4][kMaxE], s_s[4][kMaxE], s_g[4][kMaxE];
    __shared__ unsigned char s_ok[4][kMaxE];
    __shared__ int s_sel[4][kMaxK];
    __shared__ int s_cw[kThreads / 64][kMaxE];
    __shared__ int s_off[kMaxE + 1];
    __shared__ int s_flag;

    const int tid = threadIdx.x, tg = blockIdx.x, eg = blockIdx.y;
    const int t0 = tg * TB, nt = min(TB, a.T - t0);
    const int e0 = eg * EG, ne = min(EG, E - e0);

    // stage x rows and router rows; 8 loads in flight per thread
    stage_rows(a.x + (int64_t)t0 * d, s_x, nt, d, stride, tid);
    stage_rows(a.wrt + (int64_t)e0 * d, s_w, ne, d, stride, tid);
    __syncthreads();

    // x limbs for the integer decode path (expert group 0 only)
    if (eg == 0 && a.xh) {
        const int nsb = d / 32;
        for (int q = tid; q < nt * nsb; q += kThreads) {
            int t = q / nsb, sb = q % nsb;
            const float *v = &s_x[t * stride + 32 * sb];
            float amax = 0.0f;
            for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(v[i]));
            float s = amax * (1.0f / 16256.0f), inv = amax > 0.0f ? 16256.0f / amax : 0.0f;
            int isum = 0;
            uint32_t hw[8], lw[8];
#pragma unroll
            for (int i = 0; i < 8; i++) hw[i] = lw[i] = 0;
#pragma unroll
            for (int i = 0; i < 32; i++) {
                int xi = (int)rintf(v[i] * inv);  // inv == 0 when the sub-block is all zero
                xi = xi > 16256 ? 16256 : (xi < -16256 ? -16256 : xi);
                int hi = (xi + 64) >> 7, lo = xi - 128 * hi;
                isum += xi;
                hw[i >> 2] |= (uint32_t)(hi & 0xff) << (8 * (i & 3));
                lw[i >> 2] |= (uint32_t)(lo & 0xff) << (8 * (i & 3));
            }
            int64_t off = (int64_t)(t0 + t) * d + 32 * sb;
            uint4 *ph = reinterpret_cast<uint4 *>(a.xh + off), *pl = reinterpret_cast<uint4 *>(a.xl + off);
            ph[0] = make_uint4(hw[0], hw[1], hw[2], hw[3]);
            ph[1] = make_uint4(hw[4], hw[5], hw[6], hw[7]);
            pl[0] = make_uint4(lw[0], lw[1], lw[2], lw[3]);
            pl[1] = make_uint4(lw[4], lw[5], lw[6], lw[7]);
            a.xs[(int64_t)(t0 + t) * nsb + sb] = s;
            a.xm[(int64_t)(t0 + t) * nsb + sb] = s * (float)isum;
        }
    }

    // one thread per (token, expert): the sequential logit chain
    const bool chain = tid < nt * EG && (tid % EG) < ne;
    const int ct = tid / EG, ce = tid % EG, e = e0 + ce;
    float acc = 0.0f;
    if (chain) {
        const float4 *xr = reinterpret_cast<const float4 *>(&s_x[ct * stride]);
        const float4 *wr = reinterpret_cast<const float4 *>(&s_w[ce * stride]);
        if (e < (E & ~7))
            acc = chain16<true>(xr, wr, d / 4, acc);
        else
            acc = chain16<false>(xr, wr, d / 4, acc);
    }
    if (chain) a.logits[(int64_t)(t0 + ct) * E + e] = acc;

    // ---- last expert-group block of this token group selects top-k
    const int n_eg = gridDim.y, n_tg = gridDim.x;
    __threadfence();  // every writer releases at device scope before the count
    __syncthreads();
    if (tid == 0) {
        unsigned old = atomicAdd(&a.sync[tg], 1u);
        s_flag = (old == (unsigned)(n_eg - 1));
    }
    __syncthreads();
    if (!s_flag) return;
    __threadfence();
    const int wave = tid >> 6;
    for (int t = wave; t < nt; t += kThreads / 64)
        select_token(a, t0 + t, s_z[wave], s_s[wave], s_g[wave], s_ok[wave], s_sel[wave]);

    // ---- last token group runs the dispatch
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        a.sync[tg] = 0;
        unsigned old = atomicAdd(&a.sync[n_tg], 1u);
        s_flag = (old == (unsigned)(n_tg - 1));
    }
    __syncthreads();
    if (!s_flag) return;
    __threadfence();
    dispatch_block(a, s_cw, s_off);
    if (tid == 0) a.sync[n_tg] = 0;
}

__global__ void k_debug_sigmoid(const float *__restrict__ x, int64_t n, float *__restrict__ out) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = sigmoid_cw(x[i]);
}

// tokens and experts per block so that their x rows and router rows fit in
// 128 KB of LDS together
void block_shape(int d, int E, int &TB, int &EG) {
    const int row = d + kPad, budget = kLdsFloats - kSlack;
    TB = budget / 2 / row;
    TB = TB < 1 ? 1 : (TB > 4 ? 4 : TB);
    EG = (budget - TB * row) / row;
    EG = EG < 1 ? 1 : (EG > kEG ? kEG : EG);
    if (EG > E) EG = E;
}

}  // namespace

int router_token_groups(int T, int d, int E) {
    int TB, EG;
    block_shape(d, E, TB, EG);
    return (T + TB - 1) / TB;
}

hipError_t launch_router(const RouterArgs &a, hipStream_t st) {
    int TB, EG;
    block_shape(a.d, a.E, TB, EG);
    const int ntg = (a.T + TB - 1) / TB, neg = (a.E + EG - 1) / EG;
    const size_t lds = sizeof(float) * ((size_t)(TB + EG) * (a.d + kPad) + kSlack);
    static bool attr_set = false;
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&k_router),
                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)(sizeof(float) * kLdsFloats));
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    hipLaunchKernelGGL(k_router, dim3(ntg, neg), dim3(kThreads), lds, st, a, TB, EG);
    return hipGetLastError();
}

hipError_t launch_debug_sigmoid(const float *x, int64_t n, float *out, hipStream_t st) {
    hipLaunchKernelGGL(k_debug_sigmoid, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x, n,
                       out);
    return hipGetLastError();
}

}  // namespace lcmoe
