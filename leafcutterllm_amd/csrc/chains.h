// Exact router-logit chains in the reference summation order, run by whole
// waves with their operand rows streamed through LDS.
//
// logit[t][e] = sum_k x[t][k] * w[e][k] accumulated strictly in ascending k,
// one rounding per step: fused multiply-add for experts of the 8-wide blocks
// (e < E & ~7), multiply then add for the tail, as the reference router GEMM
// does (Tensor::matmul -> avx2_matmul, rust/src/kernels/simd.rs:226-249).
// Each chain is
// sequential, so a chain occupies one lane; a wave runs the NT x 8
// (token, expert) chains of one tile, lane l taking token t0 + l / 8 (NT = 8)
// or t0 (NT = 1) and expert e0 + l % 8.  Indices past T or E are clamped to
// the last valid one for the loads and their results are dropped.
//
// The NT x rows and 8 router rows advance together in chunks of CH columns:
// the wave's lanes load each chunk with coalesced 16-byte loads DEPTH chunks
// ahead, store it to one of two LDS buffers and synchronise at wave level
// only; every lane then reads its two rows from LDS, four float4 per operand
// one group ahead of use.  The wave raises its issue priority: the expert
// waves it shares a SIMD with would otherwise stretch each dependent step.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace lcmoe {

// The chains of one launch cover columns [k0, k1): from zero (k0 == 0) or
// from the running sums `part` a previous launch left, to `part` (k1 < d) or
// to the logits (k1 == d).  tiles == 0: the launch computes no chains.
struct ChainArgs {
    const float *x;    // [T, d]
    const float *wrt;  // [E, d]
    float *logits;     // [T, E] out
    float *part;       // [T, E] running sums between launches
    int T, d, E;
    int k0, k1;        // column range, multiples of 256
    int nt;            // tokens per tile: 1 or 8
    int tiles;         // ceil(T / nt) * ceil(E / 8)
};

__host__ __device__ inline ChainArgs make_chains(const float *x, const float *wrt, float *logits,
                                                 float *part, int T, int d, int E, int k0, int k1,
                                                 int nt) {
    return ChainArgs{x, wrt, logits, part, T, d, E, k0, k1, nt,
                     ((T + nt - 1) / nt) * ((E + 7) / 8)};
}

// the same chains tiled nt tokens at a time
__host__ __device__ inline ChainArgs with_nt(ChainArgs c, int nt) {
    c.nt = nt;
    c.tiles = ((c.T + nt - 1) / nt) * ((c.E + 7) / 8);
    return c;
}

// LDS floats of one wave's two chunk buffers (rows padded by 4 floats so that
// rows start on different banks), plus the 16 floats the operand prefetch
// reads past the last row
constexpr int chain_lds_floats(int NR, int CH) { return 2 * NR * (CH + 4) + 16; }

namespace chain_detail {

// native vector (HIP's float4 is a struct whose copies lower to memcpy
// through scratch memory when held in arrays)
typedef float f32x4 __attribute__((ext_vector_type(4)));

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

// ascending chain over n4 float4 of LDS rows xr, wr (n4 % 8 == 0); groups of
// 4 float4 are read one group ahead, the last read lands past the rows
template <bool FMA>
__device__ __forceinline__ float chain_lds(const f32x4 *xr, const f32x4 *wr, int n4, float acc) {
    f32x4 xa[4], wa[4], xb[4], wb[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        xa[i] = xr[i];
        wa[i] = wr[i];
    }
    for (int q = 0; q < n4; q += 8) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            xb[i] = xr[q + 4 + i];
            wb[i] = wr[q + 4 + i];
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < 4; i++) acc = step4<FMA>(xa[i], wa[i], acc);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            xa[i] = xr[q + 8 + i];
            wa[i] = wr[q + 8 + i];
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < 4; i++) acc = step4<FMA>(xb[i], wb[i], acc);
        __builtin_amdgcn_sched_barrier(0);
    }
    return acc;
}

__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

}  // namespace chain_detail

// One wave's tile `tile` of chains over columns [a.k0, a.k1); lds:
// chain_lds_floats(NT + 8, CH) floats private to this wave.  Requires k0 and
// k1 to be multiples of CH.
template <int NT, int CH, int DEPTH>
__device__ void chain_tile(const ChainArgs &a, int tile, float *lds) {
    using namespace chain_detail;
    constexpr int NR = NT + 8, ROW = CH + 4, F4 = CH / 4;  // float4 per row per chunk
    constexpr int NL = NR * F4 / 64;                       // loads per lane per chunk
    static_assert(NR * F4 % 64 == 0, "chunk must split evenly over the wave");
    const int lane = threadIdx.x & 63, ne = (a.E + 7) / 8;
    const int t0 = (tile / ne) * NT, e0 = (tile % ne) * 8;
    const int nch = (a.k1 - a.k0) / CH;
    // the chain is one long dependency: issue its instructions ahead of the
    // streaming waves that share this SIMD
    __builtin_amdgcn_s_setprio(3);
    // this lane's share of every chunk: float4 j = i * 64 + lane -> (row, col4)
    const f32x4 *src[NL];
    int dst[NL];
#pragma unroll
    for (int i = 0; i < NL; i++) {
        const int j = i * 64 + lane, r = j / F4, c4 = j % F4;
        const float *row = r < NT ? a.x + (int64_t)min(t0 + r, a.T - 1) * a.d
                                  : a.wrt + (int64_t)min(e0 + r - NT, a.E - 1) * a.d;
        src[i] = reinterpret_cast<const f32x4 *>(row + a.k0) + c4;
        dst[i] = r * ROW + 4 * c4;
    }
    f32x4 v[DEPTH][NL];
#pragma unroll
    for (int s = 0; s < DEPTH; s++)
#pragma unroll
        for (int i = 0; i < NL; i++) v[s][i] = src[i][min(s, nch - 1) * F4];
#pragma unroll
    for (int i = 0; i < NL; i++) *reinterpret_cast<f32x4 *>(lds + dst[i]) = v[0][i];
#pragma unroll
    for (int i = 0; i < NL; i++) v[0][i] = src[i][min(DEPTH, nch - 1) * F4];
    wave_lds_sync();

    const int tb = NT == 1 ? 0 : lane / 8, eg = lane % 8;
    const bool fma = min(e0 + eg, a.E - 1) < (a.E & ~7);
    const int xoff = tb * ROW, woff = (NT + eg) * ROW;
    const int t = t0 + tb, e = e0 + eg;
    float acc = a.k0 > 0 ? a.part[(int64_t)min(t, a.T - 1) * a.E + min(e, a.E - 1)] : 0.0f;
    // chunk c sits in buffer c % 2; registers slot (c + 1 + s) % DEPTH holds
    // chunk c + 1 + s for s < DEPTH (unrolled by DEPTH so slots are static)
    for (int c0 = 0; c0 < nch; c0 += DEPTH) {
#pragma unroll
        for (int s = 0; s < DEPTH; s++) {
            const int c = c0 + s;
            if (c < nch) {
                const float *cur = lds + (c & 1) * NR * ROW;
                float *nxt = lds + ((c + 1) & 1) * NR * ROW;
                const f32x4 *xr = reinterpret_cast<const f32x4 *>(cur + xoff);
                const f32x4 *wr = reinterpret_cast<const f32x4 *>(cur + woff);
                acc = fma ? chain_lds<true>(xr, wr, F4, acc) : chain_lds<false>(xr, wr, F4, acc);
                // chunk c + 1 is in slot (s + 1) % DEPTH: store it, refill the
                // slot with chunk c + 1 + DEPTH (clamped, unused past the end)
                const int slot = (s + 1) % DEPTH;
                if (c + 1 < nch) {
#pragma unroll
                    for (int i = 0; i < NL; i++)
                        *reinterpret_cast<f32x4 *>(nxt + dst[i]) = v[slot][i];
                }
#pragma unroll
                for (int i = 0; i < NL; i++) v[slot][i] = src[i][min(c + 1 + DEPTH, nch - 1) * F4];
                wave_lds_sync();
            }
        }
    }
    float *out = a.k1 < a.d ? a.part : a.logits;
    if (t < a.T && e < a.E && (NT == 8 || lane < 8)) out[(int64_t)t * a.E + e] = acc;
    __builtin_amdgcn_s_setprio(0);
}

}  // namespace lcmoe
