// Matrix-core (MFMA) expert products for Q4_K weights in the RPL64 layout,
// for experts that receive many tokens (decode batches of tens of tokens,
// prefill).  Same weight bytes and layout as the row-per-lane kernels.
//
// One v_mfma_f32_16x16x32_f16 computes C[16 tokens][16 weight rows] over 32
// input columns (one Q4_K sub-block).  Lane l holds
//   A (activations): token l%16, columns 8*(l/16) + slot
//   B (weights):     row   l%16, columns 8*(l/16) + slot
//   C (result):      tokens 4*(l/16)+s, row l%16
// so the row a lane dequantises is the row whose results it owns, and the
// per-row super-block scale d / dmin apply lane-locally.
//
// Exact operands: B = sc_j * q (6-bit * 4-bit integers, exact in f16), built
// from the nibbles with (0x6400 | q) = 1024 + q and one packed-f16 fma
// (1024+q)*sc - 1024*sc.  Activations enter as two f16 halves hi + lo
// (v - hi rounded again), about 22 significant bits.  Per super-block
//   sum_k w_k v_k = d * sum_k (sc*q)_k v_k - dmin * sum_j m_j * V_j
// with V_j the sub-block sums of v; the second sum is one
// v_mfma_f32_16x16x16_f16 with k' = (sub-block, half).
//
// Slot order: nibble extraction pairs bytes (0,2),(1,3) of a dword, so MFMA
// slot s of a lane holds column 8*(l/16) + kPerm[s]; activations are stored
// pre-permuted the same way (an involution inside each group of 8).

#include "device_common.h"
#include "kernels.h"

namespace lcmoe {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float4v __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;

__device__ __forceinline__ half2v as_h2(uint32_t u) {
    half2v h;
    __builtin_memcpy(&h, &u, 4);
    return h;
}
__device__ __forceinline__ uint32_t as_u(half2v h) {
    uint32_t u;
    __builtin_memcpy(&u, &h, 4);
    return u;
}

// 8 nibbles (low or high half of 8 bytes) -> 8 f16 values sc*q in MFMA slot
// order.  w0, w1 hold the bytes already shifted so the wanted nibble is in
// bits 0..3 of each byte.
__device__ __forceinline__ half8 nib8(uint32_t w0, uint32_t w1, half2v sc2, half2v c2) {
    const uint32_t m = 0x000F000Fu, o = 0x64006400u;
    half2v p0 = as_h2((w0 & m) | o), p1 = as_h2(((w0 >> 8) & m) | o);
    half2v p2 = as_h2((w1 & m) | o), p3 = as_h2(((w1 >> 8) & m) | o);
    p0 = __builtin_elementwise_fma(p0, sc2, c2);
    p1 = __builtin_elementwise_fma(p1, sc2, c2);
    p2 = __builtin_elementwise_fma(p2, sc2, c2);
    p3 = __builtin_elementwise_fma(p3, sc2, c2);
    half8 r;
    r[0] = p0[0]; r[1] = p0[1]; r[2] = p1[0]; r[3] = p1[1];
    r[4] = p2[0]; r[5] = p2[1]; r[6] = p3[0]; r[7] = p3[1];
    return r;
}

// (sc, sc) and (-1024*sc, -1024*sc) as packed f16 for a 6-bit scale
__device__ __forceinline__ void sc_pair(uint32_t sc, half2v &sc2, half2v &c2) {
    const _Float16 s = (_Float16)(float)sc;
    sc2 = half2v{s, s};
    const _Float16 c = (_Float16)(-1024.0f * (float)sc);
    c2 = half2v{c, c};
}

// 6-bit (sc, m) of all 8 sub-blocks from the 12 scale bytes (get_scale_min_k4,
// rust/src/kernels/mod.rs:54-63), one byte per sub-block.
__device__ __forceinline__ void unpack_sm(uint4 h, uint32_t &sc03, uint32_t &sc47, uint32_t &m03,
                                          uint32_t &m47) {
    sc03 = h.y & 0x3F3F3F3Fu;
    m03 = h.z & 0x3F3F3F3Fu;
    sc47 = (h.w & 0x0F0F0F0Fu) | ((h.y >> 2) & 0x30303030u);
    m47 = ((h.w >> 4) & 0x0F0F0F0Fu) | ((h.z >> 2) & 0x30303030u);
}
__device__ __forceinline__ uint32_t byte_of(uint32_t w03, uint32_t w47, int j) {
    return ((j < 4 ? w03 : w47) >> (8 * (j & 3))) & 0xffu;
}

struct Scales {  // one matrix, one 16-row group, this lane's row
    uint32_t sc03, sc47, m03, m47;
    float d, dmin;
};

__device__ __forceinline__ Scales load_scales(const uint8_t *blk, int row) {
    const uint4 hdr = *reinterpret_cast<const uint4 *>(blk + row * 16);
    Scales S;
    unpack_sm(hdr, S.sc03, S.sc47, S.m03, S.m47);
    S.d = dh2f(hdr.x & 0xffff);
    S.dmin = dh2f(hdr.x >> 16);
    return S;
}

// B operands (weights) of sub-blocks 2j, 2j+1 for one 16-row group
__device__ __forceinline__ void weights_pair(const uint8_t *blk, int row, int j, int c4,
                                             const Scales &S, half8 &b0, half8 &b1) {
    const uint2 q = *reinterpret_cast<const uint2 *>(
        blk + (1 + 2 * j + (c4 >> 1)) * 1024 + row * 16 + 8 * (c4 & 1));
    half2v s0, c0, s1, c1;
    sc_pair(byte_of(S.sc03, S.sc47, 2 * j), s0, c0);
    sc_pair(byte_of(S.sc03, S.sc47, 2 * j + 1), s1, c1);
    b0 = nib8(q.x, q.y, s0, c0);
    b1 = nib8(q.x >> 4, q.y >> 4, s1, c1);
}

__device__ __forceinline__ float4v mfma4(const half8 &h0, const half8 &l0, const half8 &h1,
                                         const half8 &l1, const half8 &b0, const half8 &b1,
                                         float4v S) {
    S = __builtin_amdgcn_mfma_f32_16x16x32_f16(h0, b0, S, 0, 0, 0);
    S = __builtin_amdgcn_mfma_f32_16x16x32_f16(l0, b0, S, 0, 0, 0);
    S = __builtin_amdgcn_mfma_f32_16x16x32_f16(h1, b1, S, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(l1, b1, S, 0, 0, 0);
}

// acc += d * S - dmin * (sum_j m_j V_j) for one 16-row group
__device__ __forceinline__ void finish_group(const Scales &S, int c4, const half4 &amin,
                                             const float4v &Ssum, float4v &acc) {
    const _Float16 mA = (_Float16)(float)byte_of(S.m03, S.m47, 2 * c4);
    const _Float16 mB = (_Float16)(float)byte_of(S.m03, S.m47, 2 * c4 + 1);
    const half4 bmin = half4{mA, mA, mB, mB};
    const float4v Smin = __builtin_amdgcn_mfma_f32_16x16x16f16(
        amin, bmin, float4v{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
    for (int s = 0; s < 4; s++) {
        acc[s] = __builtin_fmaf(S.d, Ssum[s], acc[s]);
        acc[s] = __builtin_fmaf(-S.dmin, Smin[s], acc[s]);
    }
}

// activations of sub-blocks 2j, 2j+1 of super-block kb for this lane's row
__device__ __forceinline__ void act_pair(const _Float16 *vh, const _Float16 *vl, int64_t base,
                                         int j, half8 &h0, half8 &l0, half8 &h1, half8 &l1) {
    h0 = *reinterpret_cast<const half8 *>(vh + base + 64 * j);
    l0 = *reinterpret_cast<const half8 *>(vl + base + 64 * j);
    h1 = *reinterpret_cast<const half8 *>(vh + base + 64 * j + 32);
    l1 = *reinterpret_cast<const half8 *>(vl + base + 64 * j + 32);
}

struct H16Out {
    _Float16 *h, *l, *s;  // [positions, F] halves (permuted), sums [positions, F/32, 2]
    float *f;             // optional f32 H [positions, F]
};

// split v into f16 hi + lo
__device__ __forceinline__ void split16(float v, _Float16 &hi, _Float16 &lo) {
    hi = (_Float16)v;
    lo = (_Float16)(v - (float)hi);
}

// position of column f inside its permuted group of 8
__device__ __forceinline__ int perm_col(int f) {
    const int s = f & 7;
    return (f & ~7) | (s == 1 ? 2 : (s == 2 ? 1 : (s == 5 ? 6 : (s == 6 ? 5 : s))));
}

// LDS: partials of the 4 waves' K slices, [dst group][src slot][matrix][4][64],
// then the 16-row sub-block partials [group][16 tokens]
constexpr int kRedFloats = 4 * 3 * 2 * 4 * 64 + 4 * 16;

// deterministic sum over the 4 waves' K slices of one value of group r = wave
__device__ __forceinline__ float wave_total(const float *s_red, int r, int mat, int s, int lane,
                                            float own) {
    float v = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; w++) {
        const float part =
            w == r ? own : s_red[(((r * 3 + (w < r ? w : w - 1)) * 2 + mat) * 4 + s) * 64 + lane];
        v = v + part;
    }
    return v;
}

__device__ __forceinline__ void post_partials(float *s_red, int wave, int mat, int lane,
                                              const float4v (&acc)[4]) {
#pragma unroll
    for (int r = 0; r < 4; r++) {
        if (r == wave) continue;
        const int slot = wave < r ? wave : wave - 1;
#pragma unroll
        for (int s = 0; s < 4; s++) s_red[(((r * 3 + slot) * 2 + mat) * 4 + s) * 64 + lane] = acc[r][s];
    }
}

// Row group R of the tile: totals over the 4 K slices, SwiGLU, H out.
template <int R>
__device__ __forceinline__ void gateup_epilogue(const float4v &og, const float4v &ou,
                                                float *s_red, const SlotArgs &sa, int p0, int n,
                                                int c, int F, int rt, const H16Out &out) {
    const int lane = threadIdx.x & 63, i16 = lane & 15, c4 = lane >> 4;
    const int f = rt * 64 + 16 * R + i16;
    float *s_part = s_red + 4 * 3 * 2 * 4 * 64;
#pragma unroll
    for (int s = 0; s < 4; s++) {
        const float g = wave_total(s_red, R, 0, s, lane, og[s]);
        const float u = wave_total(s_red, R, 1, s, lane, ou[s]);
        const int q = c + 4 * c4 + s;  // token index within the slot
        const float h = silu(g) * u;
        // this group's 16-row share of the token's sub-block sum
        _Float16 hi, lo;
        split16(h, hi, lo);
        float part = (float)hi + (float)lo;
        part += __shfl_xor(part, 1, 64);
        part += __shfl_xor(part, 2, 64);
        part += __shfl_xor(part, 4, 64);
        part += __shfl_xor(part, 8, 64);
        if (q < n) {
            const int64_t p = p0 + q;
            if (out.f) out.f[p * F + f] = h;
            out.h[p * F + perm_col(f)] = hi;
            out.l[p * F + perm_col(f)] = lo;
        }
        if (i16 == 0) s_part[R * 16 + 4 * c4 + s] = part;
    }
}

template <int R>
__device__ __forceinline__ void down_epilogue(const float4v &own, const float *s_red, int p0,
                                              int n, int c, int d, int rt, float *Y) {
    const int lane = threadIdx.x & 63, i16 = lane & 15, c4 = lane >> 4;
    const int row = rt * 64 + 16 * R + i16;
#pragma unroll
    for (int s = 0; s < 4; s++) {
        const float v = wave_total(s_red, R, 0, s, lane, own[s]);
        const int q = c + 4 * c4 + s;
        if (q < n) Y[(int64_t)(p0 + q) * d + row] = v;
    }
}

// 16 token rows starting at position c of the slot, one 64-row gate/up tile
__device__ __forceinline__ void gateup_pass(const uint8_t *G, const uint8_t *U, int kb0, int kb1,
                                            const _Float16 *xh, const _Float16 *xl,
                                            const _Float16 *xs, int d, const SlotArgs &sa, int p0,
                                            int n, int c, int F, int rt, const H16Out &out,
                                            float *s_red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, i16 = lane & 15, c4 = lane >> 4;
    const int xrow = slot_token(sa, p0, min(c + i16, n - 1));
    float4v ag[4], au[4];
#pragma unroll
    for (int r = 0; r < 4; r++) ag[r] = au[r] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
    for (int kb = kb0; kb < kb1; kb++) {
        const uint8_t *bg = G + (int64_t)kb * 9 * 1024, *bu = U + (int64_t)kb * 9 * 1024;
        const int64_t abase = (int64_t)xrow * d + (int64_t)kb * 256 + 8 * c4;
        Scales sg[4], su[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            sg[r] = load_scales(bg, 16 * r + i16);
            su[r] = load_scales(bu, 16 * r + i16);
        }
        float4v Sg[4], Su[4];
#pragma unroll
        for (int r = 0; r < 4; r++) Sg[r] = Su[r] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            half8 h0, l0, h1, l1;
            act_pair(xh, xl, abase, j, h0, l0, h1, l1);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                half8 b0, b1;
                weights_pair(bg, 16 * r + i16, j, c4, sg[r], b0, b1);
                Sg[r] = mfma4(h0, l0, h1, l1, b0, b1, Sg[r]);
                weights_pair(bu, 16 * r + i16, j, c4, su[r], b0, b1);
                Su[r] = mfma4(h0, l0, h1, l1, b0, b1, Su[r]);
            }
        }
        const half4 amin = *reinterpret_cast<const half4 *>(
            xs + ((int64_t)xrow * (d >> 5) + (int64_t)kb * 8 + 2 * c4) * 2);
#pragma unroll
        for (int r = 0; r < 4; r++) {
            finish_group(sg[r], c4, amin, Sg[r], ag[r]);
            finish_group(su[r], c4, amin, Su[r], au[r]);
        }
    }
    post_partials(s_red, wave, 0, lane, ag);
    post_partials(s_red, wave, 1, lane, au);
    __syncthreads();
    // wave w finishes row group w (compile-time index into the accumulators)
    switch (__builtin_amdgcn_readfirstlane(wave)) {
    case 0: gateup_epilogue<0>(ag[0], au[0], s_red, sa, p0, n, c, F, rt, out); break;
    case 1: gateup_epilogue<1>(ag[1], au[1], s_red, sa, p0, n, c, F, rt, out); break;
    case 2: gateup_epilogue<2>(ag[2], au[2], s_red, sa, p0, n, c, F, rt, out); break;
    default: gateup_epilogue<3>(ag[3], au[3], s_red, sa, p0, n, c, F, rt, out); break;
    }
    __syncthreads();
    float *s_part = s_red + 4 * 3 * 2 * 4 * 64;
    // sub-block sums: groups (0,1) and (2,3) of the tile are sub-blocks 2rt, 2rt+1
    if (threadIdx.x < 32) {
        const int half = threadIdx.x >> 4, tok = threadIdx.x & 15, q = c + tok;
        const float v = s_part[(2 * half) * 16 + tok] + s_part[(2 * half + 1) * 16 + tok];
        if (q < n) {
            _Float16 hi, lo;
            split16(v, hi, lo);
            const int64_t p = p0 + q, sb = 2 * rt + half;
            out.s[(p * (F >> 5) + sb) * 2] = hi;
            out.s[(p * (F >> 5) + sb) * 2 + 1] = lo;
        }
    }
    __syncthreads();
}

__device__ __forceinline__ void down_pass(const uint8_t *W, int kb0, int kb1, const _Float16 *hh,
                                          const _Float16 *hl, const _Float16 *hs, int F, int p0,
                                          int n, int c, int d, int rt, float *Y, float *s_red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, i16 = lane & 15, c4 = lane >> 4;
    const int hrow = p0 + min(c + i16, n - 1);
    float4v acc[4];
#pragma unroll
    for (int r = 0; r < 4; r++) acc[r] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
    for (int kb = kb0; kb < kb1; kb++) {
        const uint8_t *bw = W + (int64_t)kb * 9 * 1024;
        const int64_t abase = (int64_t)hrow * F + (int64_t)kb * 256 + 8 * c4;
        Scales sw[4];
#pragma unroll
        for (int r = 0; r < 4; r++) sw[r] = load_scales(bw, 16 * r + i16);
        float4v Sw[4];
#pragma unroll
        for (int r = 0; r < 4; r++) Sw[r] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            half8 h0, l0, h1, l1;
            act_pair(hh, hl, abase, j, h0, l0, h1, l1);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                half8 b0, b1;
                weights_pair(bw, 16 * r + i16, j, c4, sw[r], b0, b1);
                Sw[r] = mfma4(h0, l0, h1, l1, b0, b1, Sw[r]);
            }
        }
        const half4 amin = *reinterpret_cast<const half4 *>(
            hs + ((int64_t)hrow * (F >> 5) + (int64_t)kb * 8 + 2 * c4) * 2);
#pragma unroll
        for (int r = 0; r < 4; r++) finish_group(sw[r], c4, amin, Sw[r], acc[r]);
    }
    post_partials(s_red, wave, 0, lane, acc);
    __syncthreads();
    switch (__builtin_amdgcn_readfirstlane(wave)) {
    case 0: down_epilogue<0>(acc[0], s_red, p0, n, c, d, rt, Y); break;
    case 1: down_epilogue<1>(acc[1], s_red, p0, n, c, d, rt, Y); break;
    case 2: down_epilogue<2>(acc[2], s_red, p0, n, c, d, rt, Y); break;
    default: down_epilogue<3>(acc[3], s_red, p0, n, c, d, rt, Y); break;
    }
    __syncthreads();
}

__global__ __launch_bounds__(256) void k_mfma_gateup(
    const uint8_t *__restrict__ gate, const uint8_t *__restrict__ up, int64_t estride,
    const _Float16 *__restrict__ xh, const _Float16 *__restrict__ xl,
    const _Float16 *__restrict__ xs, SlotArgs sa, int d, int F, _Float16 *__restrict__ oh,
    _Float16 *__restrict__ ol, _Float16 *__restrict__ os, float *__restrict__ of) {
    __shared__ float s_red[kRedFloats];
    int e, p0, n;
    if (!slot_info(sa, blockIdx.y, e, p0, n)) return;
    const int NB = d >> 8, rt = blockIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int kb0 = NB * wave / kWaves, kb1 = NB * (wave + 1) / kWaves;
    const int64_t tile = (int64_t)rt * NB * 9 * 1024;
    const uint8_t *G = gate + (int64_t)e * estride + tile, *U = up + (int64_t)e * estride + tile;
    const H16Out out{oh, ol, os, of};
    for (int c = 0; c < n; c += 16)
        gateup_pass(G, U, kb0, kb1, xh, xl, xs, d, sa, p0, n, c, F, rt, out, s_red);
}

// grid (d/64 tiles, slots, ksplit) as the row-per-lane down kernel
__global__ __launch_bounds__(256) void k_mfma_down(
    const uint8_t *__restrict__ down, int64_t estride, const _Float16 *__restrict__ hh,
    const _Float16 *__restrict__ hl, const _Float16 *__restrict__ hs, SlotArgs sa, int d, int F,
    float *__restrict__ Y, int64_t split_stride) {
    __shared__ float s_red[kRedFloats];
    int e, p0, n;
    if (!slot_info(sa, blockIdx.y, e, p0, n)) return;
    const int NB = F >> 8, rt = blockIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int slices = kWaves * gridDim.z, s = blockIdx.z * kWaves + wave;
    const int kb0 = (int)((int64_t)NB * s / slices), kb1 = (int)((int64_t)NB * (s + 1) / slices);
    const uint8_t *W = down + (int64_t)e * estride + (int64_t)rt * NB * 9 * 1024;
    float *Yz = Y + (int64_t)blockIdx.z * split_stride;
    for (int c = 0; c < n; c += 16) down_pass(W, kb0, kb1, hh, hl, hs, F, p0, n, c, d, rt, Yz, s_red);
}

// x rows -> permuted f16 hi/lo halves + per-sub-block sums (hi, lo)
__global__ __launch_bounds__(256) void k_act16(const float *__restrict__ x, int T, int d,
                                               _Float16 *__restrict__ xh, _Float16 *__restrict__ xl,
                                               _Float16 *__restrict__ xs) {
    const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // sub-block index
    const int nsb = d >> 5;
    if (q >= (int64_t)T * nsb) return;
    const int64_t t = q / nsb, sb = q % nsb;
    const float *v = x + t * d + 32 * sb;
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; i++) {
        _Float16 hi, lo;
        split16(v[i], hi, lo);
        const int64_t o = t * d + perm_col(32 * (int)sb + i);
        xh[o] = hi;
        xl[o] = lo;
        sum = sum + ((float)hi + (float)lo);
    }
    _Float16 hi, lo;
    split16(sum, hi, lo);
    xs[(t * nsb + sb) * 2] = hi;
    xs[(t * nsb + sb) * 2 + 1] = lo;
}

SlotArgs dev_slots(const SlotArgsHost &s) {
    return SlotArgs{s.perm, s.counts, s.offsets, s.touched, s.E, s.K, s.T, s.shared};
}

}  // namespace

hipError_t launch_act16(const float *x, int T, int d, _Float16 *xh, _Float16 *xl, _Float16 *xs,
                        hipStream_t st) {
    const int64_t n = (int64_t)T * (d / 32);
    hipLaunchKernelGGL(k_act16, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x, T, d, xh,
                       xl, xs);
    return hipGetLastError();
}

hipError_t launch_mfma_gateup(const uint8_t *gate, const uint8_t *up, int64_t estride,
                              const _Float16 *xh, const _Float16 *xl, const _Float16 *xs,
                              const SlotArgsHost &sa, int slots, int d, int F, _Float16 *oh,
                              _Float16 *ol, _Float16 *os, float *of, hipStream_t st) {
    hipLaunchKernelGGL(k_mfma_gateup, dim3(F / 64, slots), dim3(256), 0, st, gate, up, estride, xh,
                       xl, xs, dev_slots(sa), d, F, oh, ol, os, of);
    return hipGetLastError();
}

hipError_t launch_mfma_down(const uint8_t *down, int64_t estride, const _Float16 *hh,
                            const _Float16 *hl, const _Float16 *hs, const SlotArgsHost &sa,
                            int slots, int d, int F, int ksplit, float *Y, int64_t split_stride,
                            hipStream_t st) {
    hipLaunchKernelGGL(k_mfma_down, dim3(d / 64, slots, ksplit), dim3(256), 0, st, down, estride,
                       hh, hl, hs, dev_slots(sa), d, F, Y, split_stride);
    return hipGetLastError();
}

}  // namespace lcmoe
