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

#include "chains.h"
#include "device_common.h"
#include "kernels.h"
#include "norm_device.h"

namespace lcmoe {
namespace {

// native 4-float vector: HIP's float4 is a struct, and arrays of it held in
// registers lower to memcpy through scratch memory
using chain_detail::f32x4;

constexpr int kThreads = 256;
constexpr int kEG = 8;             // max experts per block
constexpr int kPad = 4;            // LDS row padding (floats) against bank conflicts
constexpr int kSlack = 16;         // floats past the last LDS row (chain prefetch overrun)
constexpr int kLdsFloats = 32768;  // dynamic LDS budget: x rows + router rows

// Device-coherent (all XCDs) store and load of one int: agent-scope relaxed
// atomics write through / read past the XCD-private L2, so a value published
// this way needs no cache write-back fence, only the store's completion.
__device__ __forceinline__ void store_agent(int32_t *p, int32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int32_t load_agent(const int32_t *p) {
    return __hip_atomic_load(const_cast<int32_t *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Routing weights of token t from its scores s_z (sigmoid scores s_s for the
// group router) and its selection sel[0..K), in slot order, by one wave: the
// full-E softmax's maximum and exps across the lanes (the exps into s_s,
// which the softmax kinds leave free), every sum on lane 0 in item order.
__device__ void token_weights(const RouterArgs &a, int t, const float *s_z, float *s_s,
                              const int *sel) {
    const int lane = threadIdx.x & 63, E = a.E, K = a.K;
    const RouteParams &rp = a.rp;
    float *ow = a.topk_w + (int64_t)t * K;
    if (rp.kind == LCMOE_ROUTE_SOFTMAX) {  // full-E softmax probabilities of the selected
        float mx = -__builtin_inff();
        for (int e = lane; e < E; e += 64) mx = nan_max(mx, s_z[e]);
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) mx = nan_max(mx, __shfl_xor(mx, off, 64));
        for (int e = lane; e < E; e += 64) s_s[e] = expf(s_z[e] - mx);
        chain_detail::wave_lds_sync();
        if (lane == 0) {
            float sum = 0.0f;
            for (int e = 0; e < E; e++) sum = sum + s_s[e];
            for (int k = 0; k < K; k++) ow[k] = (s_s[sel[k]] / sum) * rp.scale;
        }
        return;
    }
    if (lane != 0) return;
    if (rp.kind == LCMOE_ROUTE_SIGMOID_GROUP) {
        float sum = 0.0f;
        for (int k = 0; k < K; k++) sum = sum + s_s[sel[k]];
        for (int k = 0; k < K; k++) ow[k] = (s_s[sel[k]] / sum) * rp.scale;
    } else {  // cpu.rs:66-79 over the K
        float mx = -__builtin_inff(), sum = 0.0f;
        for (int k = 0; k < K; k++) mx = nan_max(mx, s_z[sel[k]]);
        for (int k = 0; k < K; k++) sum = sum + expf(s_z[sel[k]] - mx);
        for (int k = 0; k < K; k++) ow[k] = (expf(s_z[sel[k]] - mx) / sum) * rp.scale;
    }
}

// v from lane l ^ off for off = 1, 2 (quad permutes), or from a lane of the
// partner block of size off = 4, 8 (half-row and row mirrors: lane j of an
// 8- or 16-lane block reads lane 7 - j or 15 - j); 16 and 32 by shuffle.
// A butterfly only needs the partner block, whose lanes agree.
template <int OFF>
__device__ __forceinline__ float xchg_block(float v) {
    constexpr int ctrl = OFF == 1 ? 0xB1 : OFF == 2 ? 0x4E : OFF == 4 ? 0x141 : 0x140;
    if constexpr (OFF >= 16) {
        return __shfl_xor(v, OFF, 64);
    } else {
        return __int_as_float(
            __builtin_amdgcn_update_dpp(0, __float_as_int(v), ctrl, 0xf, 0xf, false));
    }
}

// (largest, second largest) over aligned lane blocks of size 2 OFF, from
// blocks of size OFF whose lanes agree; NA x 4 independent pairs interleaved
template <int OFF, int NA>
__device__ __forceinline__ void top2_step(float (&k1)[NA][4], float (&k2)[NA][4]) {
#pragma unroll
    for (int arr = 0; arr < NA; arr++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float o1 = xchg_block<OFF>(k1[arr][i]), o2 = xchg_block<OFF>(k2[arr][i]);
            const float hi1 = fmaxf(k1[arr][i], o1), lo1 = fminf(k1[arr][i], o1);
            k2[arr][i] = fmaxf(lo1, fmaxf(k2[arr][i], o2));
            k1[arr][i] = hi1;
        }
}

// the largest two of every aligned block of gs lanes (gs a power of two up
// to 64) in every lane of the block, for the NA x 4 key sets
template <int NA>
__device__ __forceinline__ void block_top2(int gs, float (&k1)[NA][4], float (&k2)[NA][4]) {
    if (gs > 1) top2_step<1>(k1, k2);
    if (gs > 2) top2_step<2>(k1, k2);
    if (gs > 4) top2_step<4>(k1, k2);
    if (gs > 8) top2_step<8>(k1, k2);
    if (gs > 16) top2_step<16>(k1, k2);
    if (gs > 32) top2_step<32>(k1, k2);
}

// the lowest expert e = l + 64 i whose lane flag is set in slice i, or -1
__device__ __forceinline__ int lowest_flagged(const bool (&f)[4]) {
    int w = -1;
#pragma unroll
    for (int i = 3; i >= 0; i--) {
        const uint64_t b = __ballot(f[i]);
        if (b) w = 64 * i + __builtin_ctzll(b);
    }
    return w;
}

// The exact selection of token t from its chain logits, by one wave (the
// reference's route order, ties to the lower index): keys z_e = logit (the
// sigmoid score for the group kind) + bias, expert l + 64 i in lane l; for
// the group kind the topk_group groups with the largest sums of their two
// largest keys, by argmax rounds; then K argmax rounds over the kept
// experts, each a 32-bit wave maximum of the order keys and a ballot per
// slice for the lowest index at it.  s_z, s_s: this wave's E scores and
// sigmoid scores (for the weights); s_g: group scores; s_sel: K.
__device__ void select_token(const RouterArgs &a, int t, float *s_z, float *s_s, float *s_g,
                             int *s_sel) {
    const int lane = threadIdx.x & 63, E = a.E, K = a.K;
    const RouteParams &rp = a.rp;
    const bool grouped = rp.kind == LCMOE_ROUTE_SIGMOID_GROUP;
    const float *l = a.logits + (int64_t)t * E;
    float lv[4], bv[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {  // every load of the lane in flight at once
        const int e = min(lane + 64 * i, E - 1);
        lv[i] = l[e];
        bv[i] = rp.has_bias ? a.bias[e] : 0.0f;
    }
    bool valid[4];
    float z[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int e = lane + 64 * i;
        valid[i] = e < E;
        float v = lv[i];
        if (grouped) {
            const float sg = sigmoid_cw(v);
            if (valid[i]) s_s[e] = sg;
            v = sg;
        }
        z[i] = rp.has_bias ? v + bv[i] : v;
        if (valid[i]) s_z[e] = z[i];
    }
    chain_detail::wave_lds_sync();
    uint64_t kmask = ~0ull;  // kept groups (one for the softmax kinds)
    const int G = grouped ? rp.n_group : 1, gs = E / G;
    if (grouped) {
        // group score = the rounded sum of the group's two largest keys (a
        // NaN key ranks as -inf and counts as one; group scores are only
        // compared through sel_key, where NaN and -inf are the same)
        if (gs <= 64 && (gs & (gs - 1)) == 0) {
            float k1[1][4], k2[1][4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                k1[0][i] = valid[i] ? sel_key(z[i]) : -__builtin_inff();
                k2[0][i] = -__builtin_inff();
            }
            block_top2<1>(gs, k1, k2);
            if ((lane & (gs - 1)) == 0) {
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (valid[i])
                        s_g[(lane + 64 * i) / gs] = gs >= 2 ? k1[0][i] + k2[0][i] : k1[0][i];
            }
        } else if (lane < G) {
            float k1 = -__builtin_inff(), k2 = -__builtin_inff();
            int e1 = INT_MAX, e2 = INT_MAX;
            for (int i = 0; i < gs; i++) {
                const int e = lane * gs + i;
                const float k = sel_key(s_z[e]);
                if (better(k, e, k1, e1)) {
                    k2 = k1;
                    e2 = e1;
                    k1 = k;
                    e1 = e;
                } else if (better(k, e, k2, e2)) {
                    k2 = k;
                    e2 = e;
                }
            }
            s_g[lane] = gs >= 2 ? s_z[e1] + s_z[min(e2, E - 1)] : s_z[e1];
        }
        chain_detail::wave_lds_sync();
        // keep the topk_group best groups (ties to the lower group index)
        uint32_t gkey = lane < G ? ord_key(sel_key(s_g[lane])) : 0u;
        bool kept = false;
        for (int r = 0; r < rp.topk_group; r++) {
            const uint32_t m = wave_max_u32(gkey);
            const uint64_t b = __ballot(gkey == m && m != 0u);
            if (!b) break;
            if (lane == __builtin_ctzll(b)) {
                kept = true;
                gkey = 0u;
            }
        }
        kmask = __ballot(kept);
    }
    uint32_t ck[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int e = lane + 64 * i;
        ck[i] = valid[i] && ((kmask >> (e / gs)) & 1ull) ? ord_key(sel_key(z[i])) : 0u;
    }
    for (int r = 0; r < K; r++) {
        const uint32_t m = wave_max_u32(max(max(ck[0], ck[1]), max(ck[2], ck[3])));
        bool at[4];
#pragma unroll
        for (int i = 0; i < 4; i++) at[i] = ck[i] == m && m != 0u;
        int f = lowest_flagged(at);
        if (f < 0) f = 0;  // unreachable: K <= candidates is validated on the host
#pragma unroll
        for (int i = 0; i < 4; i++)
            if (lane + 64 * i == f) ck[i] = 0u;
        if (lane == 0) s_sel[r] = f;
    }
    chain_detail::wave_lds_sync();
    token_weights(a, t, s_z, s_s, s_sel);
    if (lane < K) store_agent(a.topk_idx + (int64_t)t * K + lane, s_sel[lane]);
}

// Inclusive scan across the wave
__device__ __forceinline__ int wave_incl_scan(int v) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int u = __shfl_up(v, off, 64);
        if (lane >= off) v += u;
    }
    return v;
}

// Exclusive scan of s_off[0..E) (per-expert counts) into offsets by one
// wave, writing offsets[0..E], touched[] and s_off[E] = total, and with
// a.pass_slots the pass slots: expert e's ceil(count / 32) passes, in
// expert order, after the count of them.
__device__ void scan_experts(const RouterArgs &a, int *s_off) {
    const int lane = threadIdx.x & 63, E = a.E;
    int run = 0, nt = 0, np = 0;
    for (int e0 = 0; e0 < E; e0 += 64) {
        const int e = e0 + lane;
        const int c = e < E ? s_off[e] : 0;
        const int incl = wave_incl_scan(c);
        const uint64_t m = __ballot(c > 0);
        if (e < E) {
            s_off[e] = run + incl - c;
            a.offsets[e] = run + incl - c;
        }
        if (c > 0) a.touched[nt + __popcll(m & ((1ull << lane) - 1ull))] = e;
        run += __shfl(incl, 63, 64);
        nt += __popcll(m);
        if (a.pass_slots) {
            const int passes = (c + kPassTokens - 1) / kPassTokens;
            const int pincl = wave_incl_scan(passes);
            for (int j = 0; j < passes; j++)
                a.pass_slots[1 + np + pincl - passes + j] = j * 256 + e;
            np += __shfl(pincl, 63, 64);
        }
    }
    if (lane == 0) {
        s_off[E] = run;
        a.offsets[E] = run;
        a.touched[E] = nt;
        if (a.pass_slots) a.pass_slots[0] = np;
    }
}

// Stable counting sort of the A = T*K assignments a = t*K + k by expert, by
// the NT/64 waves of one block.  Each wave owns a contiguous chunk: pass 1
// counts per (wave, expert), prefixes over waves and experts give each wave
// its base per expert, pass 2 ranks equal experts inside each 64-assignment
// group with ballots (lower lane = lower a) and advances the wave's private
// counters.  The selections are read with device-coherent loads, kDispBatch
// groups in flight per lane; when a wave's chunk is one such batch (A <=
// 64 kDispBatch NT / 64), pass 2 takes them from registers.
constexpr int kDispBatch = 8;

template <int NT>
__device__ void dispatch_block(const RouterArgs &a, int (*s_cw)[kMaxE], int *s_off) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int A = a.T * a.K, E = a.E;
    constexpr int W = NT / 64;
    for (int i = tid; i < W * kMaxE; i += NT) (&s_cw[0][0])[i] = 0;
    __syncthreads();
    const int chunk = (((A + W - 1) / W) + 63) & ~63;
    const int a0 = min(A, wave * chunk), a1 = min(A, a0 + chunk);
    const bool one = chunk <= 64 * kDispBatch;
    int keep[kDispBatch];
    for (int base = a0; base < a1; base += 64 * kDispBatch) {
        int ev[kDispBatch];
#pragma unroll
        for (int j = 0; j < kDispBatch; j++) {
            const int q = base + 64 * j + lane;
            ev[j] = q < a1 ? load_agent(a.topk_idx + q) : -1;
            keep[j] = ev[j];
        }
#pragma unroll
        for (int j = 0; j < kDispBatch; j++)
            if (ev[j] >= 0) atomicAdd(&s_cw[wave][ev[j]], 1);
    }
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
    if (wave == 0) scan_experts(a, s_off);
    __syncthreads();
    for (int base = a0; base < a1; base += 64 * kDispBatch) {
        int ev[kDispBatch];
#pragma unroll
        for (int j = 0; j < kDispBatch; j++) {
            const int q = base + 64 * j + lane;
            ev[j] = q >= a1 ? 0 : one ? keep[j] : load_agent(a.topk_idx + q);
        }
#pragma unroll
        for (int j = 0; j < kDispBatch; j++) {
            const int q = base + 64 * j + lane;
            const bool valid = q < a1;
            const int e = ev[j];
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
}

// The same dispatch for one token, by one wave, from its selection sel[0..K)
// in LDS: its K assignments a = k sorted by expert (the experts are distinct).
__device__ void dispatch_one(const RouterArgs &a, const int *sel) {
    const int lane = threadIdx.x & 63, E = a.E, K = a.K;
    int sk[kMaxK];
#pragma unroll
    for (int k = 0; k < kMaxK; k++) sk[k] = k < K ? sel[k] : -1;
    int run = 0;
    for (int e0 = 0; e0 < E; e0 += 64) {
        const int e = e0 + lane;
        int kpos = -1;
#pragma unroll
        for (int k = 0; k < kMaxK; k++)
            if (sk[k] == e) kpos = k;
        const bool hit = kpos >= 0 && e < E;
        const uint64_t m = __ballot(hit);
        const int pos = run + __popcll(m & ((1ull << lane) - 1ull));
        if (e < E) {
            a.counts[e] = hit ? 1 : 0;
            a.offsets[e] = pos;
        }
        if (hit) {
            a.perm[pos] = kpos;
            a.inv[kpos] = pos;
            a.touched[pos] = e;
            if (a.pass_slots) a.pass_slots[1 + pos] = e;  // one pass per expert
        }
        run += __popcll(m);
    }
    if (lane == 0) {
        a.offsets[E] = run;
        a.touched[E] = run;
        if (a.pass_slots) a.pass_slots[0] = run;
    }
}

// rows x d floats from global (row-major) into LDS rows of `stride` floats
__device__ __forceinline__ void stage_rows(const float *__restrict__ src, float *dst, int rows,
                                           int d, int stride, int tid) {
    const int d4 = d / 4, n = rows * d4;
    for (int base = 0; base < n; base += 8 * kThreads) {
        f32x4 v[8];
#pragma unroll
        for (int i = 0; i < 8; i++)
            v[i] = reinterpret_cast<const f32x4 *>(src)[min(base + tid + i * kThreads, n - 1)];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int q = base + tid + i * kThreads;
            if (q < n) *reinterpret_cast<f32x4 *>(&dst[(q / d4) * stride + 4 * (q % d4)]) = v[i];
        }
    }
}

template <bool FMA>
__device__ __forceinline__ float step4(f32x4 x, f32x4 w, float acc) {
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
__device__ __forceinline__ float chain16(const f32x4 *xr, const f32x4 *wr, int n4, float acc) {
    f32x4 xa[4], wa[4], xb[4], wb[4];
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

// Exact logits, x limbs, top-k and dispatch (the whole router).
__global__ __launch_bounds__(kThreads) void k_router(RouterArgs a, int TB, int EG) {
    extern __shared__ float smem[];
    const int d = a.d, E = a.E, stride = d + kPad;
    float *s_x = smem;                // [TB][d + pad]
    float *s_w = smem + TB * stride;  // [EG][d + pad], this block's router rows
    __shared__ float s_z[4][kMaxE], s_s[4][kMaxE], s_g[4][kMaxE];
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
        const f32x4 *xr = reinterpret_cast<const f32x4 *>(&s_x[ct * stride]);
        const f32x4 *wr = reinterpret_cast<const f32x4 *>(&s_w[ce * stride]);
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
        select_token(a, t0 + t, s_z[wave], s_s[wave], s_g[wave], s_sel[wave]);

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
    dispatch_block<kThreads>(a, s_cw, s_off);
    if (tid == 0) a.sync[n_tg] = 0;
}

// ---------------------------------------------------------------------------
// Certified fast router (softmax kinds).  One block per token.
//
// The reference logit is the sequential f32 chain s_k = fl(s_{k-1} + x_k w_k)
// (one rounding per step on the FMA lanes; two on the mul+add tail lanes).
// Its final value c differs from the exact sum S_d = sum_k x_k w_k by at most
//   u (1 + 1.01 d u) sum_k |S_k|                      (FMA lanes)
//   + u (1+u)(1 + 1.01 d u) sum_k |x_k w_k|           (tail lanes, extra)
// with u = 2^-24 and S_k the exact prefix sums: each step adds at most
// u |S_k + e_{k-1}| to the error e.  Each wave computes, for one expert, S_d
// and sum_k |S_k| in float64 (products of two floats are exact in float64;
// a 64-lane scan gives every lane its chunk's prefix), plus a margin for the
// float64 roundings.  That bounds the chain's value to [S_d - B, S_d + B],
// hence the score z = fl(c + bias) to [zlo, zhi] (rounding is monotone).
// If the intervals order the top-k experts strictly (rank by rank, and the
// k-th against every unselected expert), the reference chain selects exactly
// those experts in that order, and the selection is final.  Otherwise the
// block runs the exact chains for that token and selects from them.  The
// routing weights need the chain values themselves: extra blocks of this
// launch and of the routed gate/up launch compute them (chains.h), and the
// combine turns them into weights.
// ---------------------------------------------------------------------------

// next float toward +inf / -inf (finite, non-NaN arguments)
__device__ __forceinline__ float next_up(float f) {
    if (f == 0.0f) return __uint_as_float(1u);
    const uint32_t b = __float_as_uint(f);
    return __uint_as_float(f > 0.0f ? b + 1u : b - 1u);
}
__device__ __forceinline__ float next_down(float f) { return -next_up(-f); }
// smallest float >= v, largest float <= v (finite v)
__device__ __forceinline__ float ceil_f32(double v) {
    const float f = (float)v;
    return (double)f < v ? next_up(f) : f;
}
__device__ __forceinline__ float floor_f32(double v) {
    const float f = (float)v;
    return (double)f > v ? next_down(f) : f;
}

constexpr int kFastThreads = 512;  // 8 waves: one expert per wave for E = 8

// Activations of token t for the expert products: int8 limbs for the
// row-per-lane kernels and f16 hi/lo pieces + sub-block sums for the
// matrix-core kernels.  Four threads share a 32-column sub-block, eight
// columns each, and meet through lane shuffles (NTHR threads, a multiple
// of 64).  With s_x, the same reads stage the token row into LDS for the
// logits: lane l's chunk of C = 4*NC4 columns is row l of C + 4 floats,
// which keeps 8 consecutive lanes' b128 reads on distinct banks.  With
// nshare > 1 this block takes share `share` of the work (NTHR-thread slices
// share, share + nshare, ...).
template <int NC4, int NTHR = kFastThreads>
__device__ void quantise_token(const RouterArgs &a, int t, float *s_x, int share = 0,
                               int nshare = 1) {
    constexpr int C = 4 * NC4;
    const int d = a.d, nsb = d / 32;
    for (int q = share * NTHR + threadIdx.x; q < 4 * nsb; q += nshare * NTHR) {
        const int sb = q >> 2, part = q & 3, col0 = 32 * sb + 8 * part;
        const f32x4 *v = reinterpret_cast<const f32x4 *>(a.x + (int64_t)t * d + col0);
        const f32x4 v0 = v[0], v1 = v[1];
        if (s_x) {
            const int q4 = col0 / 4;
            *reinterpret_cast<f32x4 *>(s_x + (q4 / NC4) * (C + 4) + 4 * (q4 % NC4)) = v0;
            *reinterpret_cast<f32x4 *>(s_x + ((q4 + 1) / NC4) * (C + 4) + 4 * ((q4 + 1) % NC4)) =
                v1;
        }
        const float f[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
        if (a.xh) {
            float amax = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; i++) amax = fmaxf(amax, fabsf(f[i]));
            amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
            amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
            const float sc = amax * (1.0f / 16256.0f), inv = amax > 0.0f ? 16256.0f / amax : 0.0f;
            int isum = 0;
            uint32_t hw[2] = {0, 0}, lw[2] = {0, 0};
#pragma unroll
            for (int i = 0; i < 8; i++) {
                int xi = (int)rintf(f[i] * inv);  // inv == 0 when the sub-block is all zero
                xi = xi > 16256 ? 16256 : (xi < -16256 ? -16256 : xi);
                const int hi = (xi + 64) >> 7, lo = xi - 128 * hi;
                isum += xi;
                hw[i >> 2] |= (uint32_t)(hi & 0xff) << (8 * (i & 3));
                lw[i >> 2] |= (uint32_t)(lo & 0xff) << (8 * (i & 3));
            }
            isum += __shfl_xor(isum, 1, 64);
            isum += __shfl_xor(isum, 2, 64);
            const int64_t off = (int64_t)t * d + col0;
            *reinterpret_cast<uint2 *>(a.xh + off) = make_uint2(hw[0], hw[1]);
            *reinterpret_cast<uint2 *>(a.xl + off) = make_uint2(lw[0], lw[1]);
            if (part == 0) {
                a.xs[(int64_t)t * nsb + sb] = sc;
                a.xm[(int64_t)t * nsb + sb] = sc * (float)isum;
            }
        }
        if (a.x16) {
            typedef _Float16 half8v __attribute__((ext_vector_type(8)));
            half8v hv, lv;
            float sum = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const _Float16 hi = (_Float16)f[i];
                const _Float16 lo = (_Float16)(f[i] - (float)hi);
                hv[act16_pos(i)] = hi;  // the format's column order
                lv[act16_pos(i)] = lo;
                // the sum of what the products take: hi + lo, or hi alone
                sum = sum + (a.x16_lo ? (float)hi + (float)lo : (float)hi);
            }
            // the sub-block sum in column order: (c0..7 + c8..15) + (c16..23 + c24..31)
            sum = sum + __shfl_xor(sum, 1, 64);
            sum = sum + __shfl_xor(sum, 2, 64);
            _Float16 *piece = a.x16 + ((int64_t)t * (d >> 8) + (sb >> 3)) * 512 + 32 * (sb & 7) +
                              8 * part;
            *reinterpret_cast<half8v *>(piece) = hv;
            *reinterpret_cast<half8v *>(piece + 256) = lv;
            if (part == 0) {
                const _Float16 shi = (_Float16)sum, slo = (_Float16)(sum - (float)shi);
                a.x16s[((int64_t)t * nsb + sb) * 2] = shi;
                a.x16s[((int64_t)t * nsb + sb) * 2 + 1] = slo;
            }
        }
    }
}

// float64 logit S_d and chain error bound of every expert for token t; wave
// w takes experts w, w+8, ...; lane l holds columns [l*C, l*C + C) with
// C = 4*NC4 in registers.  sum_k |S_k| is bounded by groups of 4 columns:
// for k in group g, |S_k| <= |S_g| + sum_{i in g} |p_i| with S_g the prefix
// before the group, so sum_k |S_k| <= 4 sum_g |S_g| + 4 sum_i |p_i|.
template <int NC4>
struct LogitRegs {
    f32x4 wv[NC4];
    const float *xs;  // this lane's token chunk in LDS
};

// this wave's first expert's router chunk, one coalesced KiB per load (the
// lane-chunk order a.wlc)
template <int NC4>
__device__ __forceinline__ void load_wchunk(const RouterArgs &a, int e, f32x4 (&wv)[NC4]) {
    const int lane = threadIdx.x & 63;
    const f32x4 *wr = reinterpret_cast<const f32x4 *>(a.wlc) + (int64_t)e * NC4 * 64 + lane;
#pragma unroll
    for (int i = 0; i < NC4; i++) wv[i] = wr[64 * i];
}

template <int NC4>
__device__ __forceinline__ void logit_bounds(const RouterArgs &a, LogitRegs<NC4> &R, double *s_a,
                                             double *s_b) {
    constexpr int W = kFastThreads / 64;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int d = a.d, E = a.E, E8 = E & ~7;
    // up to d = 2048 the next expert's chunk loads while this one is summed
    // (a second register set; at larger d it would spill)
    constexpr bool kAhead = NC4 <= 8;
    for (int e = wave; e < E; e += W) {
        f32x4 wn[kAhead ? NC4 : 1];
        const bool more = kAhead && e + W < E;
        if constexpr (kAhead) {
            if (more) load_wchunk<NC4>(a, e + W, wn);
        } else {
            if (e != wave) load_wchunk<NC4>(a, e, R.wv);
        }
        double l2[2] = {0.0, 0.0}, ab2[2] = {0.0, 0.0}, qg[NC4];
#pragma unroll
        for (int g = 0; g < NC4; g++) {  // products are exact in float64
            const f32x4 x = *reinterpret_cast<const f32x4 *>(R.xs + 4 * g), w = R.wv[g];
            const double p0 = (double)x.x * (double)w.x, p1 = (double)x.y * (double)w.y;
            const double p2 = (double)x.z * (double)w.z, p3 = (double)x.w * (double)w.w;
            qg[g] = (p0 + p1) + (p2 + p3);  // group sum, kept for the prefix pass
            l2[g & 1] += qg[g];
            ab2[g & 1] += (fabs(p0) + fabs(p1)) + (fabs(p2) + fabs(p3));
        }
        const double loc = l2[0] + l2[1];
        double absp = ab2[0] + ab2[1];
        const double incl = wave_incl_scan_f64(loc);
        double run = incl - loc, sg = 0.0;
#pragma unroll
        for (int g = 0; g < NC4; g++) {  // the prefix before each group, in order
            sg += fabs(run);
            run += qg[g];
        }
        sg = wave_total_f64(sg);
        absp = wave_total_f64(absp);
        const double total = readlane_f64(incl, 63);
        if (lane == 0) {
            // float64 rounding of the sums above is covered, with a wide
            // margin, by the 2^-36 * sum|p| term
            const double u = 0x1p-24, g = 1.0 + 1.01 * (double)d * u;
            const double sabs = 4.0 * sg + 4.0 * absp;  // >= sum_k |S_k|
            double B = u * g * sabs + 0x1p-36 * absp + (double)d * 0x1p-149;
            if (e >= E8) B += u * (1.0 + u) * g * absp;
            s_a[e] = total;
            s_b[e] = B;
        }
        if constexpr (kAhead) {
            if (more) {
#pragma unroll
                for (int i = 0; i < NC4; i++) R.wv[i] = wn[i];
            }
        }
    }
}

// columns per LDS pass of the fused norm: small, so that its registers fit
// beside the router chunk already in flight
constexpr int kFusedNormChunk = 1024;

template <int NC4>
__device__ __forceinline__ void logits_and_activations(const RouterArgs &a, int t, float *s_x,
                                                       double *s_a, double *s_b) {
    LogitRegs<NC4> R;
    load_wchunk<NC4>(a, min((int)(threadIdx.x >> 6), a.E - 1), R.wv);
    if (a.xin) {  // the fused norm, while the router chunks load
        if ((threadIdx.x >> 6) == 0) {
            const int64_t row = (int64_t)t * a.d;
            rmsnorm_wave<kFusedNormChunk>(a.xin + row, a.norm_w, a.norm_eps, a.d, a.xn + row, s_x);
        }
        __threadfence_block();
        __syncthreads();
    }
    quantise_token<NC4>(a, t, s_x);  // while the router chunks load
    __syncthreads();
    R.xs = s_x + (threadIdx.x & 63) * (4 * NC4 + 4);
    logit_bounds<NC4>(a, R, s_a, s_b);
}

// grid (T [+ chain blocks]): block t routes token t; with ch.tiles, the
// blocks past T run the first column range of the exact router chains
// (wave 0, one tile at a time)
template <int FBW>
__global__ __launch_bounds__(kFastThreads) void k_route_fast(RouterArgs a, ChainArgs ch) {
    __shared__ double s_a[kMaxE], s_b[kMaxE];
    __shared__ float s_z[kMaxE], s_zlo[kMaxE], s_zhi[kMaxE], s_s[kMaxE], s_g[kMaxE];
    __shared__ int s_sel[kMaxK];
    __shared__ int s_cw[kFastThreads / 64][kMaxE];
    __shared__ int s_off[kMaxE + 1];
    __shared__ int s_flag;
    // x row for the logits (C <= 64 floats per lane), later the fallback's
    // chain stream (one token, 8 experts)
    // (and first, with the fused norm, its squares: kRmsnormLds floats)
    // the fallback's chain streams: one region for each of its FBW waves
    constexpr int kXFloats = 64 * (64 + 4), kFbFloats = chain_lds_floats(1 + 8, 256);
    constexpr int kFbAll = kFbFloats * FBW;
    constexpr int kS1 = kXFloats > kFbAll ? kXFloats : kFbAll;
    constexpr int kS2 = rmsnorm_lds<kFusedNormChunk>();
    __shared__ __attribute__((aligned(16))) float s_x[kS1 > kS2 ? kS1 : kS2];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int t = blockIdx.x, d = a.d, E = a.E, K = a.K;
    if (t >= a.T) {
        if (wave == 0)
            for (int tile = t - a.T; tile < ch.tiles; tile += gridDim.x - a.T) {
                if (ch.nt == 1)
                    chain_tile<1, 256, 1>(ch, tile, s_x);
                else
                    chain_tile<8, 128, 1>(ch, tile, s_x);
            }
        return;
    }

    // bias into LDS while the logits run
    for (int e = tid; e < E; e += kFastThreads) s_g[e] = a.rp.has_bias ? a.bias[e] : 0.0f;

    // 1. activations for the expert products; float64 logit and chain error
    //    bound per expert, one wave each
    switch (d >> 8) {
    case 1: logits_and_activations<1>(a, t, s_x, s_a, s_b); break;
    case 2: logits_and_activations<2>(a, t, s_x, s_a, s_b); break;
    case 4: logits_and_activations<4>(a, t, s_x, s_a, s_b); break;
    case 8: logits_and_activations<8>(a, t, s_x, s_a, s_b); break;
    default: logits_and_activations<16>(a, t, s_x, s_a, s_b); break;
    }
    __syncthreads();

    // 2. score intervals, ranks on the float64 scores (lane = expert,
    //    E <= 64), certification
    if (wave == 0) {
        const int e = lane;
        const bool valid = e < E;
        bool ok = true;
        if (valid) {
            const double lo = s_a[e] - s_b[e], hi = s_a[e] + s_b[e];
            ok = __builtin_isfinite(lo) && __builtin_isfinite(hi);
            const float bias = s_g[e];
            float zlo = ceil_f32(lo), zhi = floor_f32(hi), zm = (float)s_a[e];
            if (a.rp.has_bias) {
                zlo = zlo + bias;
                zhi = zhi + bias;
                zm = zm + bias;
            }
            s_zlo[e] = zlo;
            s_zhi[e] = zhi;
            s_z[e] = zm;
        }
        // Selection: K rounds of a wave argmax over 64-bit keys (score in an
        // order-preserving encoding, then the inverted index: a larger key
        // is a better expert, ties to the lower index, as better()).
        const float zm_e = valid ? s_z[e] : 0.0f, lo_e = valid ? s_zlo[e] : 0.0f;
        const float hi_e = valid ? s_zhi[e] : 0.0f;
        uint64_t key = valid ? ((uint64_t)ord_key(sel_key(zm_e)) << 32) | (uint32_t)~e : 0;
        int rank = -1;
        for (int r = 0; r < K; r++) {
            const uint64_t best = wave_max_u64(key);
            const int be = (int)~(uint32_t)best;
            if (e == be) {
                rank = r;
                key = 0;
            }
        }
        // Certification: a selected expert must rank certainly before every
        // expert ranked below it (interval ends apart, or touching with the
        // lower index first).  Below it: all unselected experts -- whose
        // highest interval end Mx, and the lowest index among those at Mx,
        // two wave reductions give -- and the selected experts of later rank.
        const bool unsel = valid && rank < 0;
        const uint32_t mx = wave_max_u32(unsel ? ord_key(hi_e) : 0u);
        const uint32_t fmin = 64u - wave_max_u32(unsel && ord_key(hi_e) == mx ? 64u - e : 0u);
        if (rank >= 0 && mx != 0) {
            const uint32_t ol = ord_key(lo_e);
            ok = ok && (ol > mx || (ol == mx && (uint32_t)e < fmin));
        }
        for (int r2 = 1; r2 < K; r2++) {  // the selected expert of rank r2, by ballot
            const int f = __builtin_ctzll(__ballot(rank == r2));
            const float hi_f = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(hi_e), f));
            if (rank >= 0 && rank < r2) ok = ok && (lo_e > hi_f || (lo_e == hi_f && e < f));
        }
        ok = __all(ok);
        if (lane == 0) s_flag = ok;
        if (ok && rank >= 0) {
            s_sel[rank] = e;
            store_agent(a.topk_idx + (int64_t)t * K + rank, e);
            if (a.T > 1) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
    }
    __syncthreads();
    if (!s_flag) {  // 3. fallback: exact chains, exact selection
        // the token's tiles of 8 experts side by side on FBW waves: a tile's
        // time is its d / 256 chunk loads one after another, so the eight
        // tiles of E = 60 on one wave took ~112 us
        const int ne = (E + 7) / 8;
        if (wave < FBW) {
            const ChainArgs ca = make_chains(a.x, a.wrt, a.logits, nullptr, a.T, d, E, 0, d, 1);
            for (int g = wave; g < ne; g += FBW)
                chain_tile<1, 256, 1>(ca, t * ne + g, s_x + wave * kFbFloats);
        }
        __threadfence_block();
        __syncthreads();
        if (wave == 0) {
            select_token(a, t, s_z, s_s, s_g, s_sel);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        __syncthreads();
    }

    // 4. one token: this block holds the whole selection and dispatches it
    //    from LDS (no publication wait, no counter)
    if (a.T == 1) {
        if (wave == 0) dispatch_one(a, s_sel);
        return;
    }
    // the last block to finish runs the dispatch (the selections were
    // published with coherent stores and have completed)
    if (tid == 0) {
        const unsigned old = atomicAdd(&a.sync[0], 1u);
        s_flag = (old == (unsigned)a.T - 1);
    }
    __syncthreads();
    if (!s_flag) return;
    dispatch_block<kFastThreads>(a, s_cw, s_off);
    if (tid == 0) a.sync[0] = 0;
}

// ---------------------------------------------------------------------------
// Certified router with parallel bounds.  The sigmoid-group kind (lco_route
// kind 2, the DeepSeek-V3 noaux_tc rule): score s_e = sigmoid(c_e) of the
// reference chain logit c_e, key z_e = s_e + bias_e; each of the G groups
// of E/G experts scores the rounded sum of its two largest keys; the
// topk_group best groups are kept and the K largest keys among their
// experts selected, ties to the lower index throughout.  The softmax kinds
// (at one token, for wide routers): key z_e = c_e + bias_e, the K largest
// over all experts (one group, kept).
//
// Grid (E / kSigWaves [+ chain blocks], T): wave w of block (b, t) bounds
// the chain logit of expert kSigWaves b + w for token t in float64, as the
// fast router does (c_e in [S_d - B, S_d + B], hence in [zlo, zhi] as
// floats); the blocks also write t's activations, a slice each.  The last
// block of token t to finish (a per-token counter) certifies it in one wave:
//   * sigmoid_cw dips below its running maximum by at most one ulp (an
//     exhaustive check over every float input, lco_sigmoid_max_dip in the
//     oracle), so s_e lies in [down(sigmoid(zlo)), up(sigmoid(zhi))], and
//     the key in the rounded sums with the bias (rounding is monotone; for
//     the softmax kinds the key interval is [zlo + b, zhi + b] directly);
//   * a group score is monotone in every key, so the group scores of the
//     low and the high keys bound it;
//   * the kept groups stand when every kept group's low score beats every
//     dropped group's high score (or ties it with a lower index);
//   * the selection stands rank by rank as in the fast router, over the
//     kept groups' experts.
// A certified token's selection is final here.  With one token the
// certifying wave also runs the exact path for an uncertified token (the
// chains over all d columns, select_token) and the dispatch; with more, the
// uncertified tokens are marked for the exact chains (k_route_chains) and
// selection (k_route_select) that follow, which also dispatch every token.
// The routing weights come from the exact logits (chains beside the
// bounds and the gate/up products) in the combine.
// ---------------------------------------------------------------------------
constexpr int kSigWaves = 4;

// d / 256 values with an instantiation (the lane's chunk fully unrolled,
// so all of its loads are in flight at once)
__host__ __device__ constexpr bool sig_nc4_ok(int n) {
    return n == 1 || n == 2 || n == 4 || n == 8 || n == 16 || n == 28 || n == 32;
}

__device__ __forceinline__ void store_agent_u64(uint64_t *p, uint64_t v) {
    __hip_atomic_store(reinterpret_cast<unsigned long long *>(p), (unsigned long long)v,
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t load_agent_u64(const uint64_t *p) {
    return __hip_atomic_load(reinterpret_cast<unsigned long long *>(const_cast<uint64_t *>(p)),
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The certification keys of one expert from its chain logit interval
// [S - B, S + B]: the interval's float ends zlo = up(S - B), zhi = down(S + B)
// and the point zm = (float)S, as scores (sigmoid_cw for the group kind,
// whose dips are at most one ulp, so the low and high scores widen by one
// step each way) plus the bias, rounded to nearest (monotone).  Returns
// whether every key is finite (a NaN bias or an overflowing bound goes to
// the exact path).
__device__ __forceinline__ bool interval_keys(bool grouped, bool has_bias, float bias, double S,
                                              double B, float &klo, float &khi, float &km) {
    const double lo = S - B, hi = S + B;
    const bool fin = __builtin_isfinite(lo) && __builtin_isfinite(hi);
    const float zlo = fin ? ceil_f32(lo) : 0.0f, zhi = fin ? floor_f32(hi) : 0.0f;
    const float zm = fin ? (float)S : 0.0f;
    float kl = zlo, kh = zhi, kp = zm;
    if (grouped) {  // scores lie in [0, 1]
        kl = sigmoid_cw(zlo);
        kh = next_up(sigmoid_cw(zhi));
        kp = sigmoid_cw(zm);
        kl = kl > 0.0f ? next_down(kl) : 0.0f;
    }
    if (has_bias) {
        kl = kl + bias;
        kh = kh + bias;
        kp = kp + bias;
    }
    klo = kl;
    khi = kh;
    km = kp;
    return fin && __builtin_isfinite(kl) && __builtin_isfinite(kh) && __builtin_isfinite(kp);
}

// float64 chain logit and error bound of (t, e), as logit_bounds(): lane l
// holds columns [l C, l C + C) (C = 4 NC4) of the token row (read through
// the cache: every wave of the token reads it) and of the router row in
// lane-chunk order (a.wlc).  The expert's certification keys (klo, khi)
// and (km, finite) go to a.bnd[(t E + e) 2 + {0, 1}] as float pairs.
template <int NC4>
__device__ void sig_bounds(const RouterArgs &a, int t, int e) {
    constexpr int C = 4 * NC4;
    const int lane = threadIdx.x & 63, d = a.d;
    const float bias = a.rp.has_bias ? a.bias[e] : 0.0f;
    const f32x4 *xr = reinterpret_cast<const f32x4 *>(a.x + (int64_t)t * d + lane * C);
    const f32x4 *wr = reinterpret_cast<const f32x4 *>(a.wlc) + (int64_t)e * NC4 * 64 + lane;
    f32x4 wv[NC4], xv[NC4];
#pragma unroll
    for (int g = 0; g < NC4; g++) {  // the whole chunk in flight
        wv[g] = wr[64 * g];
        xv[g] = xr[g];
    }
    double l2[2] = {0.0, 0.0}, ab2[2] = {0.0, 0.0}, qg[NC4];
#pragma unroll
    for (int g = 0; g < NC4; g++) {  // products are exact in float64
        const f32x4 x = xv[g], w = wv[g];
        const double p0 = (double)x.x * (double)w.x, p1 = (double)x.y * (double)w.y;
        const double p2 = (double)x.z * (double)w.z, p3 = (double)x.w * (double)w.w;
        qg[g] = (p0 + p1) + (p2 + p3);
        l2[g & 1] += qg[g];
        ab2[g & 1] += (fabs(p0) + fabs(p1)) + (fabs(p2) + fabs(p3));
    }
    const double loc = l2[0] + l2[1];
    double absp = ab2[0] + ab2[1];
    const double incl = wave_incl_scan_f64(loc);
    double run = incl - loc, sg = 0.0;
#pragma unroll
    for (int g = 0; g < NC4; g++) {
        sg += fabs(run);
        run += qg[g];
    }
    sg = wave_total_f64(sg);
    absp = wave_total_f64(absp);
    const double total = readlane_f64(incl, 63);
    if (lane == 0) {
        const double u = 0x1p-24, gm = 1.0 + 1.01 * (double)d * u;
        const double sabs = 4.0 * sg + 4.0 * absp;
        double B = u * gm * sabs + 0x1p-36 * absp + (double)d * 0x1p-149;
        if (e >= (a.E & ~7)) B += u * (1.0 + u) * gm * absp;
        float klo, khi, km;
        const bool fin = interval_keys(a.rp.kind == LCMOE_ROUTE_SIGMOID_GROUP, a.rp.has_bias != 0,
                                       bias, total, B, klo, khi, km);
        uint64_t *out = a.bnd + ((int64_t)t * a.E + e) * 2;
        store_agent_u64(out, ((uint64_t)__float_as_uint(khi) << 32) | __float_as_uint(klo));
        store_agent_u64(out + 1, ((uint64_t)(fin ? 1u : 0u) << 32) | __float_as_uint(km));
    }
}

// Certification of token t by one wave (E <= 256, G <= 64);
// s_lo / s_hi / s_m: E floats each (the low, high and point keys, for the
// group scores of sizes the lane butterfly does not cover), s_g: 3 x 64
// group scores, s_sel: K.  Writes topk_idx[t] when certified and flag[t]
// (0 certified, 1 for the exact path); returns the verdict, with the
// selection in s_sel when certified.  The softmax kinds select the K largest
// keys z = c + bias over all experts (select_token): one group, kept.
//
// Lane l holds experts l + 64 i (i < 4) and keeps their three keys in
// registers.  An argmax round is a 32-bit wave maximum of the order keys and
// a ballot per slice for the lowest index at that maximum (the tie rule of
// better()).

__device__ bool sig_certify(const RouterArgs &a, int t, float *s_lo, float *s_hi, float *s_m,
                            float *s_g, int *s_sel) {
    const int lane = threadIdx.x & 63, E = a.E, K = a.K;
    const RouteParams &rp = a.rp;
    const bool grouped = rp.kind == LCMOE_ROUTE_SIGMOID_GROUP;
    const int G = grouped ? rp.n_group : 1, gs = E / G;
    bool ok = true;
    // the keys the bound waves stored, every load of the lane in flight
    uint64_t kv[4][2];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint64_t *src = a.bnd + ((int64_t)t * E + min(lane + 64 * i, E - 1)) * 2;
        kv[i][0] = load_agent_u64(src);
        kv[i][1] = load_agent_u64(src + 1);
    }
    bool valid[4];
    float klo[4], khi[4], km[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        valid[i] = lane + 64 * i < E;
        klo[i] = __uint_as_float((uint32_t)kv[i][0]);
        khi[i] = __uint_as_float((uint32_t)(kv[i][0] >> 32));
        km[i] = __uint_as_float((uint32_t)kv[i][1]);
        if (valid[i]) ok = ok && (kv[i][1] >> 32) != 0;
    }
    uint64_t kmask = ~0ull;  // kept groups (one for the softmax kinds)
    if (grouped) {
        // group scores of the three key sets: the rounded sum of the group's
        // two largest keys (select_token's expression; only the values
        // matter, and the keys are finite when they count).  Groups of a
        // power-of-two size up to 64 are aligned lane blocks of each
        // 64-expert slice: a butterfly over the block merges (largest,
        // second) pairs.
        if (gs <= 64 && (gs & (gs - 1)) == 0) {
            float k1[3][4], k2[3][4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float ninf = -__builtin_inff();
                k1[0][i] = valid[i] ? klo[i] : ninf;
                k1[1][i] = valid[i] ? khi[i] : ninf;
                k1[2][i] = valid[i] ? km[i] : ninf;
                k2[0][i] = k2[1][i] = k2[2][i] = ninf;
            }
            block_top2<3>(gs, k1, k2);
            if ((lane & (gs - 1)) == 0) {
#pragma unroll
                for (int arr = 0; arr < 3; arr++)
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        if (valid[i])
                            s_g[64 * arr + (lane + 64 * i) / gs] =
                                gs >= 2 ? k1[arr][i] + k2[arr][i] : k1[arr][i];
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++)
                if (valid[i]) {
                    s_lo[lane + 64 * i] = klo[i];
                    s_hi[lane + 64 * i] = khi[i];
                    s_m[lane + 64 * i] = km[i];
                }
            chain_detail::wave_lds_sync();
            if (lane < G) {
                for (int arr = 0; arr < 3; arr++) {
                    const float *v = arr == 0 ? s_lo : arr == 1 ? s_hi : s_m;
                    float k1 = -__builtin_inff(), k2 = -__builtin_inff();
                    int e1 = INT_MAX, e2 = INT_MAX;
                    for (int i = 0; i < gs; i++) {
                        const int e = lane * gs + i;
                        const float k = sel_key(v[e]);
                        if (better(k, e, k1, e1)) {
                            k2 = k1;
                            e2 = e1;
                            k1 = k;
                            e1 = e;
                        } else if (better(k, e, k2, e2)) {
                            k2 = k;
                            e2 = e;
                        }
                    }
                    s_g[64 * arr + lane] = gs >= 2 ? v[e1] + v[min(e2, E - 1)] : v[e1];
                }
            }
        }
        chain_detail::wave_lds_sync();
        // kept groups by the point scores: topk_group argmax rounds, ties to
        // the lower group index
        const bool gv = lane < G;
        const float glo = gv ? s_g[lane] : 0.0f, ghi = gv ? s_g[64 + lane] : 0.0f;
        uint32_t gkey = gv ? ord_key(sel_key(s_g[128 + lane])) : 0u;
        bool kept = false;
        for (int r = 0; r < rp.topk_group; r++) {
            const uint32_t m = wave_max_u32(gkey);
            const uint64_t b = __ballot(gkey == m && m != 0u);
            if (!b) break;
            if (lane == __builtin_ctzll(b)) {
                kept = true;
                gkey = 0u;
            }
        }
        // every kept group above every dropped one: the dropped groups'
        // highest score Mx and the lowest index at it
        {
            const bool dropped = gv && !kept;
            const uint32_t mx = wave_max_u32(dropped ? ord_key(ghi) : 0u);
            const uint64_t b = __ballot(dropped && ord_key(ghi) == mx);
            const uint32_t fmin = b ? (uint32_t)__builtin_ctzll(b) : 64u;
            if (kept && mx != 0) {
                const uint32_t ol = ord_key(glo);
                ok = ok && (ol > mx || (ol == mx && (uint32_t)lane < fmin));
            }
        }
        kmask = __ballot(kept);
    }
    // K argmax rounds over the kept groups' experts (point keys)
    uint32_t ck[4];
    int rank[4];
    bool cand[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int e = lane + 64 * i;
        cand[i] = valid[i] && ((kmask >> (e / gs)) & 1ull);
        ck[i] = cand[i] ? ord_key(sel_key(km[i])) : 0u;
        rank[i] = -1;
    }
    for (int r = 0; r < K; r++) {
        const uint32_t m = wave_max_u32(max(max(ck[0], ck[1]), max(ck[2], ck[3])));
        bool at[4];
#pragma unroll
        for (int i = 0; i < 4; i++) at[i] = ck[i] == m && m != 0u;
        const int f = lowest_flagged(at);
        if (f < 0) {  // fewer candidates than K: left to the exact path
            ok = false;
            break;
        }
#pragma unroll
        for (int i = 0; i < 4; i++)
            if (lane + 64 * i == f) {
                rank[i] = r;
                ck[i] = 0u;
            }
        if (lane == 0) s_sel[r] = f;
    }
    // every selected expert certainly above every unselected candidate (their
    // highest interval end Mx and the lowest index at it) ...
    {
        uint32_t ml = 0;
        bool un[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            un[i] = cand[i] && rank[i] < 0;
            if (un[i]) ml = max(ml, ord_key(khi[i]));
        }
        const uint32_t mx = wave_max_u32(ml);
        bool at[4];
#pragma unroll
        for (int i = 0; i < 4; i++) at[i] = un[i] && ord_key(khi[i]) == mx;
        const int w = lowest_flagged(at);
        const uint32_t fmin = w < 0 ? (uint32_t)E : (uint32_t)w;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int e = lane + 64 * i;
            if (rank[i] >= 0 && mx != 0) {
                const uint32_t ol = ord_key(klo[i]);
                ok = ok && (ol > mx || (ol == mx && (uint32_t)e < fmin));
            }
            // the selected experts' interval ends by rank, for the pair checks
            if (rank[i] >= 0) {
                s_lo[rank[i]] = klo[i];
                s_hi[rank[i]] = khi[i];
            }
        }
    }
    chain_detail::wave_lds_sync();
    // ... and above every selected expert of a later rank (interval ends
    // apart, or touching with the lower index first): pair (r1, r2) per lane
    if (ok) {
        for (int q = lane; q < K * K; q += 64) {
            const int r1 = q / K, r2 = q % K;
            if (r1 < r2) {
                const float le = s_lo[r1], hf = s_hi[r2];
                ok = ok && (le > hf || (le == hf && s_sel[r1] < s_sel[r2]));
            }
        }
    }
    ok = __all(ok);
    if (ok) {
#pragma unroll
        for (int i = 0; i < 4; i++)
            if (rank[i] >= 0) store_agent(a.topk_idx + (int64_t)t * K + rank[i], lane + 64 * i);
    }
    if (lane == 0) store_agent(a.flag + t, ok ? 0 : 1);
    chain_detail::wave_lds_sync();  // s_sel for the caller's wave
    return ok;
}

template <int NC4, int FBW>
__global__ __launch_bounds__(64 * kSigWaves) void k_route_sig(RouterArgs a, ChainArgs ch) {
    __shared__ float s_f[3 * kMaxE + 3 * 64];  // certification: keys, group scores
    // one wave's chain stream: the chain blocks', or the one-token fallback's
    // streams, one for each of its FBW waves
    constexpr int kChainFloats = chain_lds_floats(1 + 8, 256);
    __shared__ __attribute__((aligned(16))) float s_chain[kChainFloats * FBW];
    __shared__ int s_last;
    const int t = blockIdx.y, tid = threadIdx.x, wave = tid >> 6;
    const int nsig = a.E / kSigWaves;  // bound blocks per token
    if ((int)blockIdx.x >= nsig) {
        // blocks past them (row 0): the first column range of the exact
        // chains, wave 0, one tile at a time, two chunks of loads ahead
        if (t == 0 && wave == 0) {
            for (int tile = blockIdx.x - nsig; tile < ch.tiles; tile += gridDim.x - nsig)
                chain_tile<1, 256, 2>(ch, tile, s_chain);
        }
        return;
    }
    sig_bounds<NC4>(a, t, blockIdx.x * kSigWaves + wave);
    // the token's activations, a slice per block
    quantise_token<1, 64 * kSigWaves>(a, t, nullptr, blockIdx.x, nsig);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's bounds have landed
    __syncthreads();
    if (tid == 0) s_last = atomicAdd(&a.tsync[t], 1u) == (unsigned)nsig - 1;
    __syncthreads();
    if (!s_last) return;
    // the last block of token t: every bound of t is stored
    __shared__ int s_sel[kMaxK];
    __shared__ int s_ok;
    if (wave == 0) {
        if (tid == 0) a.tsync[t] = 0;
        const bool ok = sig_certify(a, t, s_f, s_f + a.E, s_f + 2 * a.E, s_f + 3 * a.E, s_sel);
        if (tid == 0) s_ok = ok;
    }
    if (a.T > 1) return;  // the chains, selection and dispatch launches follow
    // one token: this block finishes the routing itself (no launches
    // follow): for an uncertified token the exact chains over all d columns
    // (its tiles of 8 experts spread over FBW waves) and the exact
    // selection, then the dispatch from LDS
    __syncthreads();
    if (!s_ok) {
        if (wave < FBW) {
            const ChainArgs ca = make_chains(a.x, a.wrt, a.logits, nullptr, a.T, a.d, a.E, 0,
                                             a.d, 1);
            for (int g = wave; g < ca.tiles; g += FBW)
                chain_tile<1, 256, 1>(ca, g, s_chain + wave * kChainFloats);
        }
        __threadfence_block();
        __syncthreads();
        if (wave == 0) {
            float *s_z = s_f, *s_s = s_f + kMaxE, *s_g = s_f + 2 * kMaxE;
            select_token(a, t, s_z, s_s, s_g, s_sel);
            chain_detail::wave_lds_sync();
        }
    }
    if (wave == 0) dispatch_one(a, s_sel);
}

// ---------------------------------------------------------------------------
// Chain router: exact logits for every (token, expert) as chain tiles
// (chains.h), spread over the whole chip, then selection and dispatch.  It
// serves the sigmoid-group kind, more than 64 experts, and batches whose
// T*E*d makes the per-token fast router re-read the router matrix too often.
//
// Launch 1, grid (chain blocks + activation blocks): wave w of chain block b
// runs tile 4b + w (8 tokens x 8 experts over all d columns); activation
// block T0 + t prepares token t's limbs and/or f16 pieces.
// Launch 2, grid (ceil(T / 8)): wave w selects token 8b + w from its logits
// (select_token); the last block to finish dispatches (one token: the
// selecting wave dispatches from LDS).
// ---------------------------------------------------------------------------

constexpr int kChainWaves = 4;
constexpr int kChainLds = chain_lds_floats(9, 256) > chain_lds_floats(16, 128)
                              ? chain_lds_floats(9, 256)
                              : chain_lds_floats(16, 128);
constexpr int kSelWaves = 8;

__global__ __launch_bounds__(64 * kChainWaves) void k_route_chains(RouterArgs a, ChainArgs ch,
                                                                   int chain_blocks) {
    __shared__ __attribute__((aligned(16))) float s_lds[kChainWaves][kChainLds];
    if ((int)blockIdx.x < chain_blocks) {
        const int wave = threadIdx.x >> 6, tile = blockIdx.x * kChainWaves + wave;
        // after the certified sigmoid router: only tokens it marked
        bool need = true;
        if (a.flag && tile < ch.tiles) {
            const int t0 = (tile / ((ch.E + 7) / 8)) * ch.nt;
            need = false;
            for (int t = t0; t < min(t0 + ch.nt, ch.T); t++) need = need || a.flag[t] != 0;
        }
        if (tile < ch.tiles && need) {
            if (ch.nt == 1)  // fewer than 8 tokens: 1-token tiles, 256-column chunks
                chain_tile<1, 256, 2>(ch, tile, s_lds[wave]);
            else
                chain_tile<8, 128, 4>(ch, tile, s_lds[wave]);
        }
        return;
    }
    quantise_token<1, 64 * kChainWaves>(a, blockIdx.x - chain_blocks, nullptr);
}

__global__ __launch_bounds__(64 * kSelWaves) void k_route_select(RouterArgs a) {
    __shared__ float s_z[kSelWaves][kMaxE], s_s[kSelWaves][kMaxE], s_g[kSelWaves][kMaxE];
    __shared__ int s_sel[kSelWaves][kMaxK];
    __shared__ int s_cw[kSelWaves][kMaxE];
    __shared__ int s_off[kMaxE + 1];
    __shared__ int s_flag;
    const int tid = threadIdx.x, wave = tid >> 6, t = blockIdx.x * kSelWaves + wave;
    // after the certified sigmoid router: only the tokens it marked
    const bool sel = t < a.T && (!a.flag || a.flag[t] != 0);
    if (sel) select_token(a, t, s_z[wave], s_s[wave], s_g[wave], s_sel[wave]);
    if (a.T == 1) {
        if (wave == 0) {
            if (!sel) {  // certified: the selection is in topk_idx
                if ((tid & 63) < a.K) s_sel[0][tid & 63] = load_agent(a.topk_idx + (tid & 63));
                chain_detail::wave_lds_sync();
            }
            dispatch_one(a, s_sel[0]);
        }
        return;
    }
    // the selections were published with coherent stores (store_agent) and
    // dispatch_block reads them with coherent loads: once every wave's
    // stores have completed the count may advance, with no L2 write-back or
    // invalidate (a device-scope fence in each of the T / 8 blocks costs
    // tens of us)
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0) {
        const unsigned old = atomicAdd(&a.sync[0], 1u);
        s_flag = (old == gridDim.x - 1);
    }
    __syncthreads();
    if (!s_flag) return;
    dispatch_block<64 * kSelWaves>(a, s_cw, s_off);
    if (tid == 0) a.sync[0] = 0;
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

bool route_chains_ok(const RouterArgs &a) { return a.d % 128 == 0 && (a.T >= 8 || a.d % 256 == 0); }

hipError_t launch_route_chains(const RouterArgs &a, hipStream_t st) {
    const ChainArgs ch =
        make_chains(a.x, a.wrt, a.logits, nullptr, a.T, a.d, a.E, 0, a.d, a.T < 8 ? 1 : 8);
    const int cb = (ch.tiles + kChainWaves - 1) / kChainWaves;
    const int ab = (a.xh || a.x16) ? a.T : 0;
    hipLaunchKernelGGL(k_route_chains, dim3(cb + ab), dim3(64 * kChainWaves), 0, st, a, ch, cb);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_route_select, dim3((a.T + kSelWaves - 1) / kSelWaves),
                       dim3(64 * kSelWaves), 0, st, a);
    return hipGetLastError();
}

// softmax kinds, at most 64 experts, d = 64 * 4 * NC4 with NC4 in
// {1, 2, 4, 8, 16}

bool route_fast_ok(const RouterArgs &a) {
    const int c4 = a.d / 256;
    return a.rp.kind != LCMOE_ROUTE_SIGMOID_GROUP && a.wlc && a.E <= 64 && a.d % 256 == 0 &&
           (c4 == 1 || c4 == 2 || c4 == 4 || c4 == 8 || c4 == 16);
}

hipError_t launch_route_fast(const RouterArgs &a, const ChainArgs &ch, hipStream_t st) {
    ChainArgs c = ch;
    int cb = 0;
    if (c.tiles) {
        if (c.k0 % 256 || c.k1 % 256) return hipErrorInvalidValue;
        c = with_nt(ch, ch.T == 1 ? 1 : 8);
        cb = c.tiles < 64 ? c.tiles : 64;
    }
    // E > 8: the fallback's tiles on 4 waves (LDS for 4 chain streams, ~75
    // KB; 8 do not fit beside the rest), which leaves one block per CU, so
    // only while the grid fits one round of the CUs; E <= 8 has one tile and
    // keeps the small LDS footprint
    if (a.E > 8 && a.T <= 256)
        hipLaunchKernelGGL(k_route_fast<4>, dim3(a.T + cb), dim3(kFastThreads), 0, st, a, c);
    else
        hipLaunchKernelGGL(k_route_fast<1>, dim3(a.T + cb), dim3(kFastThreads), 0, st, a, c);
    return hipGetLastError();
}

bool route_sig_ok(const RouterArgs &a) {
    const int G = a.rp.n_group;
    const bool groups = a.rp.kind != LCMOE_ROUTE_SIGMOID_GROUP ||
                        (G >= 1 && G <= 64 && a.E % G == 0);
    return a.wlc && a.bnd && a.tsync && a.flag && a.E % kSigWaves == 0 && a.E <= 256 &&
           a.d % 256 == 0 && sig_nc4_ok(a.d / 256) && groups && a.K <= kMaxK &&
           route_chains_ok(a);
}

template <int FBW>
static void launch_sig(int c4, dim3 grid, dim3 block, hipStream_t st, const RouterArgs &a,
                       const ChainArgs &c) {
    switch (c4) {
    case 1: hipLaunchKernelGGL((k_route_sig<1, FBW>), grid, block, 0, st, a, c); break;
    case 2: hipLaunchKernelGGL((k_route_sig<2, FBW>), grid, block, 0, st, a, c); break;
    case 4: hipLaunchKernelGGL((k_route_sig<4, FBW>), grid, block, 0, st, a, c); break;
    case 8: hipLaunchKernelGGL((k_route_sig<8, FBW>), grid, block, 0, st, a, c); break;
    case 16: hipLaunchKernelGGL((k_route_sig<16, FBW>), grid, block, 0, st, a, c); break;
    case 28: hipLaunchKernelGGL((k_route_sig<28, FBW>), grid, block, 0, st, a, c); break;
    default: hipLaunchKernelGGL((k_route_sig<32, FBW>), grid, block, 0, st, a, c); break;
    }
}

hipError_t launch_route_sig(const RouterArgs &a, const ChainArgs &ch, hipStream_t st) {
    if (!route_sig_ok(a)) return hipErrorInvalidValue;
    static_assert(64 % kSigWaves == 0, "blocks of whole expert groups");
    ChainArgs c = ch;
    int cb = 0;
    if (c.tiles) {  // one-token tiles, 256-column chunks
        if (c.k0 % 256 || c.k1 % 256) return hipErrorInvalidValue;
        c = with_nt(ch, 1);
        cb = c.tiles < 64 ? c.tiles : 64;
    }
    const dim3 grid(a.E / kSigWaves + cb, a.T), block(64 * kSigWaves);
    // one token: its fallback chains on every wave of the block (LDS for
    // kSigWaves chain streams); more tokens keep the small LDS footprint
    if (a.T == 1)
        launch_sig<kSigWaves>(a.d / 256, grid, block, st, a, c);
    else
        launch_sig<1>(a.d / 256, grid, block, st, a, c);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.T == 1) return e;  // one token: the launch dispatched it
    // the exact chains and selection for the marked tokens; the activations
    // are written already
    RouterArgs b = a;
    b.xh = nullptr;
    b.x16 = nullptr;
    return launch_route_chains(b, st);
}

hipError_t launch_debug_sigmoid(const float *x, int64_t n, float *out, hipStream_t st) {
    hipLaunchKernelGGL(k_debug_sigmoid, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x, n,
                       out);
    return hipGetLastError();
}

}  // namespace lcmoe
