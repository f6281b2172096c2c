// Matrix-core (MFMA) expert products for Q4_K weights in the RPL64 layout,
// for experts that receive many tokens (decode batches of tens of tokens,
// prefill).  Same weight bytes and layout as the row-per-lane kernels.
//
// One v_mfma_f32_32x32x16_f16 computes C[32 tokens][32 weight rows] over 16
// input columns.  Lane l (r = l % 32, h = l / 32) holds
//   A (activations): token r, columns 8h .. 8h+7 of the 16
//   B (weights):     row   r, columns 8h .. 8h+7
//   C (result):      row r, tokens 8*(i/4) + 4h + i%4 for register i = 0..15
// so every per-row quantity (super-block scales d / dmin, 6-bit sub-block
// scales and mins) is lane-local.
//
// Exact operands: B = sc_j * q (6-bit * 4-bit integers, exact in f16), built
// from the nibbles as the f16 bit pattern 0x6400 | q = 1024 + q and one
// packed-f16 fma (1024+q)*sc - 1024*sc.  Activations enter as two f16 halves
// hi + lo (lo = v - hi rounded again), about 22 significant bits.  Per
// super-block
//   sum_k w_k v_k = d * sum_k (sc*q)_k v_k - dmin * sum_j m_j * V_j
// with V_j the sub-block sums of v; the second sum is one more MFMA whose 16
// input columns are (sub-block, half).
//
// Work split: a wave owns 32 weight rows and ALL tokens of its expert (32 per
// pass), so every weight byte is read and decoded once per 32 tokens.  Waves
// are independent (no barriers); four consecutive row groups of one expert
// form a block so that their activation reads share the CU's L1.  The next
// super-block's weights are loaded into registers while the current one is
// computed, and each activation unit one step ahead.

#include "device_common.h"
#include "kernels.h"

namespace lcmoe {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float16v __attribute__((ext_vector_type(16)));

constexpr int kWaves = 4;  // waves per block = 4 groups of 32 rows
constexpr int kTok = 32;   // tokens per pass
constexpr uint32_t kMagic = 0x64646464u;

__device__ __forceinline__ half2v as_h2(uint32_t u) {
    half2v h;
    __builtin_memcpy(&h, &u, 4);
    return h;
}

__device__ __forceinline__ float16v mfma32(const half8 &a, const half8 &b, const float16v &c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// bytes (b_i, b_j) of w -> f16 pair (1024 + b_i, 1024 + b_j); the bytes must
// already be nibbles
__device__ __forceinline__ half2v magic2(uint32_t w, uint32_t sel) {
    return as_h2(__builtin_amdgcn_perm(kMagic, w, sel));
}
constexpr uint32_t kSel01 = 0x04010400u;  // bytes 0, 1
constexpr uint32_t kSel23 = 0x04030402u;  // bytes 2, 3
constexpr uint32_t kSel00 = 0x04000400u;  // byte 0 twice
constexpr uint32_t kSel11 = 0x04010401u;
constexpr uint32_t kSel22 = 0x04020402u;
constexpr uint32_t kSel33 = 0x04030403u;

// 8 nibbles (one per byte of w0, w1, already masked) -> 8 f16 values sc*q,
// natural column order
__device__ __forceinline__ half8 dec8(uint32_t w0, uint32_t w1, half2v sc2, half2v c2) {
    const half2v p0 = __builtin_elementwise_fma(magic2(w0, kSel01), sc2, c2);
    const half2v p1 = __builtin_elementwise_fma(magic2(w0, kSel23), sc2, c2);
    const half2v p2 = __builtin_elementwise_fma(magic2(w1, kSel01), sc2, c2);
    const half2v p3 = __builtin_elementwise_fma(magic2(w1, kSel23), sc2, c2);
    half8 r;
    r[0] = p0[0]; r[1] = p0[1]; r[2] = p1[0]; r[3] = p1[1];
    r[4] = p2[0]; r[5] = p2[1]; r[6] = p3[0]; r[7] = p3[1];
    return r;
}

// Per-row super-block header (d, dmin, 12 packed scale bytes) unpacked.
struct Hdr {
    uint32_t sc03, sc47, m03, m47;
    float d, dmin;
};

// get_scale_min_k4 (rust/src/kernels/mod.rs:54-63) for all 8 sub-blocks,
// one byte per sub-block
__device__ __forceinline__ Hdr unpack_hdr16(uint4 h) {
    Hdr s;
    s.sc03 = h.y & 0x3F3F3F3Fu;
    s.m03 = h.z & 0x3F3F3F3Fu;
    s.sc47 = (h.w & 0x0F0F0F0Fu) | ((h.y >> 2) & 0x30303030u);
    s.m47 = ((h.w >> 4) & 0x0F0F0F0Fu) | ((h.z >> 2) & 0x30303030u);
    s.d = dh2f(h.x & 0xffff);
    s.dmin = dh2f(h.x >> 16);
    return s;
}

// (sc, sc) and (-1024 sc, -1024 sc) for the two sub-blocks of pair p
__device__ __forceinline__ void pair_scales(const Hdr &s, int p, half2v &sa, half2v &ca,
                                            half2v &sb, half2v &cb) {
    const uint32_t w = p < 2 ? s.sc03 : s.sc47;
    const half2v k1024 = half2v{(_Float16)1024.0f, (_Float16)1024.0f};
    const half2v km = half2v{(_Float16)-1024.0f, (_Float16)-1024.0f};
    sa = magic2(w, (p & 1) ? kSel22 : kSel00) - k1024;
    sb = magic2(w, (p & 1) ? kSel33 : kSel11) - k1024;
    ca = sa * km;
    cb = sb * km;
}

// B operand of the min MFMA: (m_j, m_j) for sub-blocks j = 4h .. 4h+3
__device__ __forceinline__ half8 min_operand(const Hdr &s, int h) {
    const uint32_t w = h ? s.m47 : s.m03;
    const half2v k1024 = half2v{(_Float16)1024.0f, (_Float16)1024.0f};
    const half2v a = magic2(w, kSel00) - k1024, b = magic2(w, kSel11) - k1024;
    const half2v c = magic2(w, kSel22) - k1024, e = magic2(w, kSel33) - k1024;
    half8 r;
    r[0] = a[0]; r[1] = a[1]; r[2] = b[0]; r[3] = b[1];
    r[4] = c[0]; r[5] = c[1]; r[6] = e[0]; r[7] = e[1];
    return r;
}

// Activation format (x for gate/up, H for down): per token and super-block,
// 1 KiB = hi[256] then lo[256] halves; sub-block sums as (hi, lo) pairs in a
// separate [token][cols/32][2] array.
//
// LDS stage of one super-block for the pass's 32 tokens: token rows of 1040
// bytes (the 1 KiB piece + 16 bytes of pad: b128 reads by 8 consecutive
// tokens hit distinct banks), then the 32 tokens' sums (32 bytes each).
// Two stages live in two distinct arrays so that the compiler can tell the
// DMA into one from the reads of the other.
constexpr int kTokBytes = 1040;
constexpr int kSumsOff = kTok * kTokBytes;
constexpr int kStageBytes = kSumsOff + kTok * 32;

__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

typedef __attribute__((address_space(3))) void lds_void;

// Per-pass source addresses for the block's staging DMA: wave w moves the
// 1 KiB pieces of tokens w + 4i (i = 0..7); wave 0 also moves the 32 sums
// pieces (lane l: token l/2, half l%2).
struct StageSrc {
    const uint8_t *tok[8];  // token row bases (wave-uniform)
    const uint8_t *sums;    // this lane's sums row base
};

// DMA super-block kb of the pass's activations into stage (1 KiB per token
// per wave instruction, lane l -> bytes 16l..16l+15)
__device__ __forceinline__ void stage_dma(uint8_t *stage, const StageSrc &src, int kb, int wave,
                                          int lane) {
#pragma unroll
    for (int i = 0; i < 8; i++)
        __builtin_amdgcn_global_load_lds(src.tok[i] + (int64_t)kb * 1024 + 16 * lane,
                                         (lds_void *)(stage + (wave + 4 * i) * kTokBytes), 16, 0, 0);
    if (wave == 0)
        __builtin_amdgcn_global_load_lds(src.sums + (int64_t)kb * 32 + 16 * (lane & 1),
                                         (lds_void *)(stage + kSumsOff), 16, 0, 0);
}

// Raw weight registers of one super-block for one matrix: this lane's row
// header and, per unit u = 2p + s, 8 bytes of chunk 1 + u.
struct WRaw {
    uint4 hdr;
    uint2 q[8];
};

__device__ __forceinline__ void load_w(WRaw &w, const uint8_t *row, int kb, int h) {
    const uint8_t *b = row + (int64_t)kb * 9 * 1024;
    w.hdr = *reinterpret_cast<const uint4 *>(b);
#pragma unroll
    for (int u = 0; u < 8; u++)
        w.q[u] = *reinterpret_cast<const uint2 *>(b + (1 + u) * 1024 + 8 * h);
}

// Activation operands of one (pair p, k-step s) unit from the LDS stage:
// sub-blocks 2p, 2p+1, hi and lo halves.
struct AUnit {
    half8 h0, l0, h1, l1;
};

__device__ __forceinline__ void read_a(AUnit &a, const uint8_t *tokrow, int u, int h) {
    const int col = 2 * (64 * (u >> 1) + 16 * (u & 1) + 8 * h);  // bytes
    a.h0 = *reinterpret_cast<const half8 *>(tokrow + col);
    a.l0 = *reinterpret_cast<const half8 *>(tokrow + 512 + col);
    a.h1 = *reinterpret_cast<const half8 *>(tokrow + col + 64);
    a.l1 = *reinterpret_cast<const half8 *>(tokrow + 512 + col + 64);
}

// One unit of MATS matrices: decode B for sub-blocks 2p (low nibbles) and
// 2p+1 (high nibbles), four MFMAs per matrix.
template <int MATS>
__device__ __forceinline__ void unit_mfma(const WRaw (&w)[MATS], const Hdr (&hd)[MATS], int u,
                                          const AUnit &a, float16v (&S)[MATS]) {
    const int p = u >> 1;
#pragma unroll
    for (int m = 0; m < MATS; m++) {
        half2v sa, ca, sb, cb;
        pair_scales(hd[m], p, sa, ca, sb, cb);
        const uint32_t w0 = w[m].q[u].x, w1 = w[m].q[u].y;
        const half8 blo = dec8(w0 & 0x0F0F0F0Fu, w1 & 0x0F0F0F0Fu, sa, ca);
        const half8 bhi = dec8((w0 >> 4) & 0x0F0F0F0Fu, (w1 >> 4) & 0x0F0F0F0Fu, sb, cb);
        S[m] = mfma32(a.h0, blo, S[m]);
        S[m] = mfma32(a.l0, blo, S[m]);
        S[m] = mfma32(a.h1, bhi, S[m]);
        S[m] = mfma32(a.l1, bhi, S[m]);
    }
}

// acc += d * S - dmin * (sum_j m_j V_j) for one matrix
__device__ __forceinline__ void finish_sb(const Hdr &hd, const half8 &amin, int h,
                                          const float16v &S, float16v &acc) {
    const float16v Smin = mfma32(amin, min_operand(hd, h), float16v{});
#pragma unroll
    for (int i = 0; i < 16; i++) {
        acc[i] = __builtin_fmaf(hd.d, S[i], acc[i]);
        acc[i] = __builtin_fmaf(-hd.dmin, Smin[i], acc[i]);
    }
}

// One super-block step: start the DMA of super-block kn into `nxt` and the
// loads of its weights into wn, compute kb from `cur` and wc, then wait for
// everything at the barrier.
template <int MATS>
__device__ __forceinline__ void step(const uint8_t *const (&wr)[MATS], int kb, int kn,
                                     const uint8_t *cur, uint8_t *nxt, const StageSrc &src,
                                     WRaw (&wc)[MATS], WRaw (&wn)[MATS], float16v (&acc)[MATS],
                                     int wave, int lane) {
    const int r = lane & 31, h = lane >> 5;
    // Wait for this step's weights (loaded one step ago) before issuing the
    // next step's loads, so that the wait cannot cover the new loads.
#pragma unroll
    for (int m = 0; m < MATS; m++) {
        asm volatile("" ::"v"(wc[m].hdr.x), "v"(wc[m].hdr.y), "v"(wc[m].hdr.z), "v"(wc[m].hdr.w));
#pragma unroll
        for (int u = 0; u < 8; u++) asm volatile("" ::"v"(wc[m].q[u].x), "v"(wc[m].q[u].y));
    }
    stage_dma(nxt, src, kn, wave, lane);
#pragma unroll
    for (int m = 0; m < MATS; m++) load_w(wn[m], wr[m], kn, h);
    Hdr hd[MATS];
#pragma unroll
    for (int m = 0; m < MATS; m++) hd[m] = unpack_hdr16(wc[m].hdr);
    float16v S[MATS];
#pragma unroll
    for (int m = 0; m < MATS; m++) S[m] = float16v{};
    const uint8_t *tokrow = cur + r * kTokBytes;
#pragma unroll
    for (int u = 0; u < 8; u++) {
        AUnit a;
        read_a(a, tokrow, u, h);
        unit_mfma<MATS>(wc, hd, u, a, S);
    }
    const half8 amin = *reinterpret_cast<const half8 *>(cur + kSumsOff + r * 32 + 16 * h);
#pragma unroll
    for (int m = 0; m < MATS; m++) finish_sb(hd[m], amin, h, S[m], acc[m]);
    lds_barrier();
}

__shared__ __attribute__((aligned(1024))) uint8_t s_stage0[kStageBytes];
__shared__ __attribute__((aligned(1024))) uint8_t s_stage1[kStageBytes];

// One pass of the block over super-blocks [kb0, kb1) for its 32 tokens.
// wr[m]: this lane's row of chunk 0, super-block 0 of matrix m.  Double
// buffered: the DMA of the next super-block's activations and the loads of
// its weights are in flight while the current one is computed.  The last
// step re-fetches its own super-block (in bounds, unused) so that every
// step has the same shape.
template <int MATS>
__device__ __forceinline__ void block_pass(const uint8_t *const (&wr)[MATS], int kb0, int kb1,
                                           const StageSrc &src, float16v (&acc)[MATS]) {
    const int lane = threadIdx.x & 63, h = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    WRaw w0[MATS], w1[MATS];
    stage_dma(s_stage0, src, kb0, wave, lane);
#pragma unroll
    for (int m = 0; m < MATS; m++) load_w(w0[m], wr[m], kb0, h);
    lds_barrier();
    int kb = kb0;
    for (; kb + 2 <= kb1; kb += 2) {
        step<MATS>(wr, kb, kb + 1, s_stage0, s_stage1, src, w0, w1, acc, wave, lane);
        step<MATS>(wr, kb + 1, min(kb + 2, kb1 - 1), s_stage1, s_stage0, src, w1, w0, acc, wave,
                   lane);
    }
    if (kb < kb1) step<MATS>(wr, kb, kb, s_stage0, s_stage1, src, w0, w1, acc, wave, lane);
}

// split v into f16 hi + lo
__device__ __forceinline__ void split16(float v, _Float16 &hi, _Float16 &lo) {
    hi = (_Float16)v;
    lo = (_Float16)(v - (float)hi);
}

// token (within the pass) held in C register i by half h
__device__ __forceinline__ int c_token(int i, int h) { return 8 * (i >> 2) + 4 * h + (i & 3); }

// grid (F/128 row blocks, slots); block = 4 waves x 32 weight rows
__global__ __launch_bounds__(256, 2) void k_mfma_gateup(
    const uint8_t *__restrict__ gate, const uint8_t *__restrict__ up, int64_t estride,
    const _Float16 *__restrict__ x16, const _Float16 *__restrict__ xs, SlotArgs sa, int d, int F,
    _Float16 *__restrict__ h16, _Float16 *__restrict__ hs, float *__restrict__ hf) {
    int e, p0, n;
    if (!slot_info(sa, blockIdx.y, e, p0, n)) return;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, r = lane & 31, h = lane >> 5;
    const int ngrp = F >> 5, grp0 = blockIdx.x * kWaves + wave;
    const int grp = min(grp0, ngrp - 1);  // duplicate the last group past the end
    const int NB = d >> 8, tile = grp >> 1, nsb = d >> 5;
    const int64_t rowoff = (int64_t)tile * NB * 9 * 1024 + (32 * (grp & 1) + r) * 16;
    const uint8_t *const wr[2] = {gate + (int64_t)e * estride + rowoff,
                                  up + (int64_t)e * estride + rowoff};
    const int f = grp * 32 + r, nkb = F >> 8;
    const uint8_t *xb = reinterpret_cast<const uint8_t *>(x16);
    const uint8_t *sb = reinterpret_cast<const uint8_t *>(xs);
    for (int c = 0; c < n; c += kTok) {
        StageSrc src;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int tok = slot_token(sa, p0, min(c + wave + 4 * i, n - 1));
            src.tok[i] = xb + (int64_t)tok * d * 4;
        }
        src.sums = sb + (int64_t)slot_token(sa, p0, min(c + (lane >> 1), n - 1)) * nsb * 4;
        float16v acc[2] = {float16v{}, float16v{}};
        block_pass<2>(wr, 0, NB, src, acc);
        if (grp0 >= ngrp) continue;
        // SwiGLU, H out (f16 hi/lo pieces and/or f32), 32-row sub-block sums
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int q = c + c_token(i, h);
            const float v = silu(acc[0][i]) * acc[1][i];
            _Float16 hi, lo;
            split16(v, hi, lo);
            float part = (float)hi + (float)lo;
#pragma unroll
            for (int off = 1; off < 32; off <<= 1) part += __shfl_xor(part, off, 64);
            if (q < n) {
                const int64_t p = p0 + q;
                if (hf) hf[p * F + f] = v;
                if (h16) {
                    _Float16 *piece = h16 + (p * nkb + (f >> 8)) * 512 + (f & 255);
                    piece[0] = hi;
                    piece[256] = lo;
                    if (r == 0) {
                        _Float16 shi, slo;
                        split16(part, shi, slo);
                        hs[(p * (F >> 5) + grp) * 2] = shi;
                        hs[(p * (F >> 5) + grp) * 2 + 1] = slo;
                    }
                }
            }
        }
    }
}

// grid (d/128 row blocks, slots, ksplit); partial sums of K slice z go to
// Y + z * split_stride
__global__ __launch_bounds__(256, 2) void k_mfma_down(
    const uint8_t *__restrict__ down, int64_t estride, const _Float16 *__restrict__ h16,
    const _Float16 *__restrict__ hs, SlotArgs sa, int d, int F, float *__restrict__ Y,
    int64_t split_stride) {
    int e, p0, n;
    if (!slot_info(sa, blockIdx.y, e, p0, n)) return;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, r = lane & 31, h = lane >> 5;
    const int ngrp = d >> 5, grp0 = blockIdx.x * kWaves + wave;
    const int grp = min(grp0, ngrp - 1);
    const int NB = F >> 8, tile = grp >> 1, nsb = F >> 5;
    const int kb0 = (int)((int64_t)NB * blockIdx.z / gridDim.z);
    const int kb1 = (int)((int64_t)NB * (blockIdx.z + 1) / gridDim.z);
    const int64_t rowoff = (int64_t)tile * NB * 9 * 1024 + (32 * (grp & 1) + r) * 16;
    const uint8_t *const wr[1] = {down + (int64_t)e * estride + rowoff};
    float *Yz = Y + (int64_t)blockIdx.z * split_stride;
    const int row = grp * 32 + r;
    const uint8_t *hb = reinterpret_cast<const uint8_t *>(h16);
    const uint8_t *sb = reinterpret_cast<const uint8_t *>(hs);
    for (int c = 0; c < n; c += kTok) {
        StageSrc src;
#pragma unroll
        for (int i = 0; i < 8; i++)
            src.tok[i] = hb + (int64_t)(p0 + min(c + wave + 4 * i, n - 1)) * F * 4;
        src.sums = sb + (int64_t)(p0 + min(c + (lane >> 1), n - 1)) * nsb * 4;
        float16v acc[1] = {float16v{}};
        block_pass<1>(wr, kb0, kb1, src, acc);
        if (grp0 >= ngrp) continue;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int q = c + c_token(i, h);
            if (q < n) Yz[(int64_t)(p0 + q) * d + row] = acc[0][i];
        }
    }
}

// x rows -> f16 hi/lo pieces (per super-block: hi[256] then lo[256]) and
// per-sub-block sums (hi, lo); one thread per 32-column sub-block
__global__ __launch_bounds__(256) void k_act16(const float *__restrict__ x, int T, int d,
                                               _Float16 *__restrict__ x16,
                                               _Float16 *__restrict__ xs) {
    const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // sub-block index
    const int nsb = d >> 5;
    if (q >= (int64_t)T * nsb) return;
    const int64_t t = q / nsb;
    const int sbi = (int)(q % nsb);
    const float4 *v = reinterpret_cast<const float4 *>(x + q * 32);
    _Float16 *piece = x16 + (t * (d >> 8) + (sbi >> 3)) * 512 + 32 * (sbi & 7);
    half8 *oh = reinterpret_cast<half8 *>(piece);
    half8 *ol = reinterpret_cast<half8 *>(piece + 256);
    float sum = 0.0f;
#pragma unroll
    for (int g = 0; g < 4; g++) {
        const float4 a = v[2 * g], b = v[2 * g + 1];
        const float f[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        half8 hv, lv;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            _Float16 hi, lo;
            split16(f[i], hi, lo);
            hv[i] = hi;
            lv[i] = lo;
            sum = sum + ((float)hi + (float)lo);
        }
        oh[g] = hv;
        ol[g] = lv;
    }
    _Float16 hi, lo;
    split16(sum, hi, lo);
    xs[q * 2] = hi;
    xs[q * 2 + 1] = lo;
}

SlotArgs dev_slots(const SlotArgsHost &s) {
    return SlotArgs{s.perm, s.counts, s.offsets, s.touched, s.E, s.K, s.T, s.shared};
}

}  // namespace

hipError_t launch_act16(const float *x, int T, int d, _Float16 *x16, _Float16 *xs,
                        hipStream_t st) {
    const int64_t n = (int64_t)T * (d / 32);
    hipLaunchKernelGGL(k_act16, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x, T, d, x16,
                       xs);
    return hipGetLastError();
}

hipError_t launch_mfma_gateup(const uint8_t *gate, const uint8_t *up, int64_t estride,
                              const _Float16 *x16, const _Float16 *xs, const SlotArgsHost &sa,
                              int slots, int d, int F, _Float16 *h16, _Float16 *hs, float *hf,
                              hipStream_t st) {
    const int groups = F / 32;
    hipLaunchKernelGGL(k_mfma_gateup, dim3((groups + kWaves - 1) / kWaves, slots), dim3(256), 0,
                       st, gate, up, estride, x16, xs, dev_slots(sa), d, F, h16, hs, hf);
    return hipGetLastError();
}

hipError_t launch_mfma_down(const uint8_t *down, int64_t estride, const _Float16 *h16,
                            const _Float16 *hs, const SlotArgsHost &sa, int slots, int d, int F,
                            int ksplit, float *Y, int64_t split_stride, hipStream_t st) {
    const int groups = d / 32;
    hipLaunchKernelGGL(k_mfma_down, dim3((groups + kWaves - 1) / kWaves, slots, ksplit), dim3(256),
                       0, st, down, estride, h16, hs, dev_slots(sa), d, F, Y, split_stride);
    return hipGetLastError();
}

}  // namespace lcmoe
