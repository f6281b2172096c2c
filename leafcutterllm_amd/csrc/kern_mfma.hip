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
// packed-f16 fma (1024+q)*sc - 1024*sc.  Activations enter as one f16 per
// element (LO = false, the default mode) or as two f16 halves hi + lo
// (lo = v - hi rounded again, about 22 significant bits).  Per
// super-block
//   sum_k w_k v_k = d * sum_k (sc*q)_k v_k - dmin * sum_j m_j * V_j
// with V_j the sub-block sums of v; the second sum is one more MFMA whose 16
// input columns are (sub-block, half), V_j the sums of what the products take.
//
// Work split: a wave owns 32 weight rows and ALL tokens of its expert (32 per
// pass), so every weight byte is read and decoded once per 32 tokens.  Four
// consecutive row groups of one expert form a block: they stage each
// super-block's activations in LDS together and meet at one barrier per
// super-block step.  The next super-block's weights are loaded into
// registers while the current one is computed, and each activation unit one
// step ahead.

#include "device_common.h"
#include "kernels.h"

namespace lcmoe {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float16v __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));  // native vectors: copies of HIP's
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));  // uint4 struct become memcpy

// Global-memory bytes: an explicit address space keeps loads through
// pointers rebuilt from integers as global (not flat) loads.
typedef __attribute__((address_space(1))) const uint8_t g_u8;

template <class T>
__device__ __forceinline__ T gload(g_u8 *p) {
    return *reinterpret_cast<const __attribute__((address_space(1))) T *>(p);
}

// p as a wave-uniform (scalar register) global pointer; p must be the same in
// all lanes
__device__ __forceinline__ g_u8 *uniform(const void *p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return reinterpret_cast<g_u8 *>(((uint64_t)hi << 32) | lo);
}

constexpr int kWaves = 4;  // waves per block = 4 groups of 32 rows
constexpr int kXcds = 8;   // MI355X: accelerator complex dies, one L2 each
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

// 16-token passes use v_mfma_f32_16x16x32_f16 on two 16-row tiles per wave:
// lane l (r16 = l % 16, c4 = l / 16) holds A: token r16, columns 8*c4..+8 of
// a 32-column sub-block; B: row r16 of the tile, the same columns; C: row
// r16, tokens 4*c4 + i.
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float float4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float4v mfma16(const half8 &a, const half8 &b, const float4v &c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// bytes (b_i, b_j) of w -> f16 pair (1024 + b_i, 1024 + b_j); the bytes must
// already be nibbles
__device__ __forceinline__ half2v magic2(uint32_t w, uint32_t sel) {
    return as_h2(__builtin_amdgcn_perm(kMagic, w, sel));
}
constexpr uint32_t kSel01 = 0x04010400u;  // bytes 0, 1
constexpr uint32_t kSel23 = 0x04030402u;  // bytes 2, 3
constexpr uint32_t kSel02 = 0x04020400u;  // bytes 0, 2
constexpr uint32_t kSel13 = 0x04030401u;  // bytes 1, 3
constexpr uint32_t kSel00 = 0x04000400u;  // byte 0 twice
constexpr uint32_t kSel11 = 0x04010401u;
constexpr uint32_t kSel22 = 0x04020402u;
constexpr uint32_t kSel33 = 0x04030403u;

// Per-row super-block header (d, dmin, 12 packed scale bytes) unpacked;
// d2, dmin2: the scales of sub-blocks 4-7 in the split layout.
struct Hdr {
    uint32_t sc03, sc47, m03, m47;
    float d, dmin, d2, dmin2;
};

// get_scale_min_k4 (rust/src/kernels/mod.rs:54-63) for all 8 sub-blocks,
// one byte per sub-block
__device__ __forceinline__ Hdr unpack_hdr16(u32x4 h) {
    Hdr s;
    s.sc03 = h.y & 0x3F3F3F3Fu;
    s.m03 = h.z & 0x3F3F3F3Fu;
    s.sc47 = (h.w & 0x0F0F0F0Fu) | ((h.y >> 2) & 0x30303030u);
    s.m47 = ((h.w >> 4) & 0x0F0F0F0Fu) | ((h.z >> 2) & 0x30303030u);
    s.d = dh2f(h.x & 0xffff);
    s.dmin = dh2f(h.x >> 16);
    s.d2 = s.d;
    s.dmin2 = s.dmin;
    return s;
}

__device__ __forceinline__ Hdr unpack_hdr_split(u32x4 h, uint32_t db) {
    Hdr s = unpack_hdr16(h);
    s.d2 = dh2f(db & 0xffff);
    s.dmin2 = dh2f(db >> 16);
    return s;
}

// Scales of pair p: s2 = (sc_2p, sc_2p+1 / 16) and c2 = -1024 * s2.  The
// low-nibble sub-block 2p decodes as (1024 + q) * sc_2p - 1024 * sc_2p; the
// high-nibble sub-block 2p+1 is decoded unshifted, from the byte 16q, as
// (1024 + 16q) * (sc / 16) - 64 * sc.  Every step is exact in f16 (the fmas
// round only their final, integer results <= 945).
__device__ __forceinline__ void pair_scales(const Hdr &s, int p, half2v &s2, half2v &c2) {
    const uint32_t w = p < 2 ? s.sc03 : s.sc47;
    const half2v mag = magic2(w, (p & 1) ? kSel23 : kSel01);  // 1024 + sc
    s2 = __builtin_elementwise_fma(mag, half2v{(_Float16)1.0f, (_Float16)0.0625f},
                                   half2v{(_Float16)-1024.0f, (_Float16)-64.0f});
    c2 = s2 * half2v{(_Float16)-1024.0f, (_Float16)-1024.0f};
}

// Two f16 magic values from the nibbles of bytes 0 and 2 of w, one and-or:
// the low nibbles (mask 0x000F000F) as 1024 + q, the high ones (0x00F000F0)
// as 1024 + 16 q
// mg: kMagicH held in a vector register (magic_reg()), so that the and-or
// takes the mask as its one constant operand
constexpr uint32_t kMagicH = 0x64006400u;
__device__ __forceinline__ half2v nib2(uint32_t w, uint32_t mask, uint32_t mg) {
    return as_h2((w & mask) | mg);
}
__device__ __forceinline__ uint32_t magic_reg() {
    uint32_t mg = kMagicH;
    asm volatile("" : "+v"(mg));
    return mg;
}

// B operands (sc*q, 8 columns each) of pair p's two sub-blocks from one
// lane's 8 qs bytes w0, w1 (bytes j = columns j), in the activation format's
// column order (act16_pos): bytes 0, 2, 1, 3, 4, 6, 5, 7.  Per pair of
// weights one and-or and one packed fma; the shifted words w >> 8 bring
// bytes 1 and 3 down to the places of 0 and 2.
__device__ __forceinline__ void dec_pair(const Hdr &s, int p, uint32_t w0, uint32_t w1,
                                         uint32_t mg, half8 &blo, half8 &bhi) {
    half2v s2, c2;
    pair_scales(s, p, s2, c2);
    const uint32_t w[4] = {w0, w0 >> 8, w1, w1 >> 8};
    const half2v sl{s2[0], s2[0]}, cl{c2[0], c2[0]}, sh{s2[1], s2[1]}, ch{c2[1], c2[1]};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const half2v a = __builtin_elementwise_fma(nib2(w[i], 0x000F000Fu, mg), sl, cl);
        const half2v b = __builtin_elementwise_fma(nib2(w[i], 0x00F000F0u, mg), sh, ch);
        blo[2 * i] = a[0];
        blo[2 * i + 1] = a[1];
        bhi[2 * i] = b[0];
        bhi[2 * i + 1] = b[1];
    }
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
constexpr int kTokBytes = 1040;
constexpr int kSumsOff = kTok * kTokBytes;
constexpr int kStageBytes = kSumsOff + kTok * 32;
// Stages of activations without their lo halves (LO = false: the gate/up
// products take x as one f16 per element): token rows of 512 + 16 bytes.
template <bool LO>
constexpr int kTokB = LO ? kTokBytes : 528;
template <bool LO>
constexpr int kSumsOffT = kTok * kTokB<LO>;

// Per-pass source addresses of the block's activation staging: wave w moves
// the 1 KiB pieces of tokens w + 4i (i = 0..7); wave 0 also moves the 32
// sums pieces (lane l: token l/2, half l%2).
struct StageSrc {
    g_u8 *tok[8];   // token row bases (wave-uniform)
    g_u8 *sums;     // sums array base (wave-uniform)
    uint32_t soff;  // this lane's byte offset of its sums row
};

// One super-block of activations on its way to LDS through this wave's
// registers: loaded at the start of a step, stored to the other LDS stage at
// its end.  Ordinary loads (not LDS DMA), so that every wait in the pipeline
// is an in-order vmcnt wait that leaves younger weight loads in flight.
template <int NI, bool LO = true>
struct StageRegs {
    typename std::conditional<LO, u32x4, u32x2>::type tok[NI];
    u32x4 sums;
};

// LO: the whole 1 KiB piece (16 bytes per lane); otherwise its hi half
// (8 bytes per lane)
template <int NI, bool LO = true>
__device__ __forceinline__ void stage_load(StageRegs<NI, LO> &s, const StageSrc &src, int kb,
                                           int wave, int lane) {
#pragma unroll
    for (int i = 0; i < NI; i++) {
        if constexpr (LO)
            s.tok[i] = gload<u32x4>(src.tok[i] + (uint32_t)(kb * 1024 + 16 * lane));
        else
            s.tok[i] = gload<u32x2>(src.tok[i] + (uint32_t)(kb * 1024 + 8 * lane));
    }
    // every wave loads and stores the same sums (identical bytes), which
    // keeps the staging free of branches
    s.sums = gload<u32x4>(src.sums + (src.soff + (uint32_t)kb * 32));
}

template <int NI, bool LO = true>
__device__ __forceinline__ void stage_store(uint8_t *stage, const StageRegs<NI, LO> &s, int wave,
                                            int lane) {
#pragma unroll
    for (int i = 0; i < NI; i++) {
        if constexpr (LO)
            *reinterpret_cast<u32x4 *>(stage + (wave + 4 * i) * kTokBytes + 16 * lane) = s.tok[i];
        else
            *reinterpret_cast<u32x2 *>(stage + (wave + 4 * i) * kTokB<false> + 8 * lane) = s.tok[i];
    }
    *reinterpret_cast<u32x4 *>(stage + kSumsOffT<LO> + 16 * lane) = s.sums;
}

__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// B operand of the 16x16x16 min MFMA: (m_j, m_j) for sub-blocks 2*c4, 2*c4+1
__device__ __forceinline__ half4 min_operand16(const Hdr &s, int c4) {
    const uint32_t w = c4 < 2 ? s.m03 : s.m47;
    const half2v k1024 = half2v{(_Float16)1024.0f, (_Float16)1024.0f};
    const half2v a = magic2(w, (c4 & 1) ? kSel22 : kSel00) - k1024;
    const half2v b = magic2(w, (c4 & 1) ? kSel33 : kSel11) - k1024;
    return half4{a[0], a[1], b[0], b[1]};
}

// Raw weight registers of one super-block for one matrix: this lane's row
// header and, per unit u = 2p + s, 8 bytes of chunk 1 + u.
struct WRaw {
    u32x4 hdr;
    uint32_t db;  // split layout: the second (d, dmin)
    u32x2 q[8];
};

// Bytes per 64-row tile and super-block: nine 1 KiB chunks; the split
// layout (rows whose length is an odd multiple of 128 columns, lcmoe_host.cpp)
// adds the 64 rows' second (d, dmin) pair, 4 bytes each.
template <bool SPLIT>
constexpr int kTileSB = SPLIT ? 9 * 1024 + 256 : 9 * 1024;

// Weight addressing: a wave-uniform base (the wave's row group, chunk 0 of
// super-block 0) plus this lane's 32-bit row offset `lo`.
template <bool SPLIT = false>
__device__ __forceinline__ u32x4 load_hdr(g_u8 *base, uint32_t lo, int kb, int off = 0) {
    return gload<u32x4>(base + (lo + (uint32_t)(kb * kTileSB<SPLIT> + off)));
}

template <bool SPLIT = false>
__device__ __forceinline__ u32x2 load_q(g_u8 *base, uint32_t lo, int kb, int chunk, int off) {
    return gload<u32x2>(base + (lo + (uint32_t)(kb * kTileSB<SPLIT> + chunk * 1024 + off)));
}

// the second (d, dmin) of a split-layout row; dbo: the row's offset from
// `base` into the pair area
template <bool SPLIT>
__device__ __forceinline__ uint32_t load_db(g_u8 *base, uint32_t dbo, int kb) {
    if (!SPLIT) return 0;
    return gload<uint32_t>(base + (dbo + (uint32_t)(kb * kTileSB<SPLIT>)));
}

template <bool SPLIT = false>
__device__ __forceinline__ void load_w(WRaw &w, g_u8 *base, uint32_t lo, uint32_t dbo, int kb,
                                       int h) {
    w.hdr = load_hdr<SPLIT>(base, lo, kb);
    w.db = load_db<SPLIT>(base, dbo, kb);
#pragma unroll
    for (int u = 0; u < 8; u++) w.q[u] = load_q<SPLIT>(base, lo, kb, 1 + u, 8 * h);
}

// Activation operands of one (pair p, k-step s) unit from the LDS stage:
// sub-blocks 2p, 2p+1, hi and lo halves.
struct AUnit {
    half8 h0, l0, h1, l1;
};

template <bool LO = true>
__device__ __forceinline__ void read_a(AUnit &a, const uint8_t *tokrow, int u, int h) {
    const int col = 2 * (64 * (u >> 1) + 16 * (u & 1) + 8 * h);  // bytes
    a.h0 = *reinterpret_cast<const half8 *>(tokrow + col);
    a.h1 = *reinterpret_cast<const half8 *>(tokrow + col + 64);
    if constexpr (LO) {
        a.l0 = *reinterpret_cast<const half8 *>(tokrow + 512 + col);
        a.l1 = *reinterpret_cast<const half8 *>(tokrow + 512 + col + 64);
    }
}

// One unit of MATS matrices: decode B for sub-blocks 2p (low nibbles) and
// 2p+1 (high nibbles), four MFMAs per matrix (two without lo halves).
template <int MATS, bool LO = true>
__device__ __forceinline__ void unit_mfma(const WRaw (&w)[MATS], const Hdr (&hd)[MATS], int u,
                                          const AUnit &a, uint32_t mg, float16v (&S)[MATS]) {
    const int p = u >> 1;
#pragma unroll
    for (int m = 0; m < MATS; m++) {
        half8 blo, bhi;
        dec_pair(hd[m], p, w[m].q[u].x, w[m].q[u].y, mg, blo, bhi);
        S[m] = mfma32(a.h0, blo, S[m]);
        if constexpr (LO) S[m] = mfma32(a.l0, blo, S[m]);
        S[m] = mfma32(a.h1, bhi, S[m]);
        if constexpr (LO) S[m] = mfma32(a.l1, bhi, S[m]);
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

// The split layout's finish (sub-blocks 0-3 scaled by d, dmin; 4-7 by d2,
// dmin2).  Mid-step, after sub-blocks 0-3: acc += d * S.  At the end:
// acc += d2 * S and the min terms -dmin * SA - dmin2 * SB, computed as
// (dmin2 - dmin) * SA - dmin2 * (SA + SB): SA from an MFMA whose lanes of
// sub-blocks 4-7 supply zero mins, SA + SB from the unmasked MFMA, one
// result live at a time.
__device__ __forceinline__ void finish_first(const Hdr &hd, const float16v &S, float16v &acc) {
#pragma unroll
    for (int i = 0; i < 16; i++) acc[i] = __builtin_fmaf(hd.d, S[i], acc[i]);
}

__device__ __forceinline__ void finish_split(const Hdr &hd, const half8 &amin, int h,
                                             const float16v &S, float16v &acc) {
#pragma unroll
    for (int i = 0; i < 16; i++) acc[i] = __builtin_fmaf(hd.d2, S[i], acc[i]);
    const half8 mo = min_operand(hd, h);
    const _Float16 k0 = h == 0 ? (_Float16)1.0f : (_Float16)0.0f;
    const float16v SA = mfma32(amin, mo * k0, float16v{});
    const float ddm = hd.dmin2 - hd.dmin;  // exact: two f16 values
#pragma unroll
    for (int i = 0; i < 16; i++) acc[i] = __builtin_fmaf(ddm, SA[i], acc[i]);
    const float16v ST = mfma32(amin, mo, float16v{});
#pragma unroll
    for (int i = 0; i < 16; i++) acc[i] = __builtin_fmaf(-hd.dmin2, ST[i], acc[i]);
}

// Pipeline of a pass over super-blocks [kb0, kb1).  One register set of
// weights: step k computes super-block k from it and from LDS stage k % 2,
// and reloads each weight register with super-block k+1 right after its
// decode has read it, so every weight load has about one step to arrive and
// the loads stream steadily instead of in a burst per step.  The step also
// loads super-block k+1's activations at its start and stores them to the
// other stage at its end.  Only ordinary vector loads are used; they
// complete in issue order, so each wait the compiler places (for the
// activations before their store, for a weight register at its next use)
// leaves the younger loads in flight, and no wait drains the queue at the
// barrier.  Indices past the end are clamped to kb1 - 1 (in bounds, unused).

// One step of a 32-token pass: super-block k from `cur` and w; activations
// of super-block kn into `nxt`; w reloaded with super-block kn.
template <int MATS, bool SPLIT = false, bool LO = true>
__device__ __forceinline__ void step(g_u8 *const (&wb)[MATS], uint32_t lo,
                                     const uint32_t (&dbo)[MATS], int kn, const uint8_t *cur,
                                     uint8_t *nxt, const StageSrc &src, WRaw (&w)[MATS],
                                     float16v (&acc)[MATS], int wave, int lane) {
    const int r = lane & 31, h = lane >> 5;
    StageRegs<8, LO> act;
    stage_load<8, LO>(act, src, kn, wave, lane);
    __builtin_amdgcn_sched_barrier(0);  // keep the activation loads first
    Hdr hd[MATS];
#pragma unroll
    for (int m = 0; m < MATS; m++) {
        hd[m] = SPLIT ? unpack_hdr_split(w[m].hdr, w[m].db) : unpack_hdr16(w[m].hdr);
        w[m].hdr = load_hdr<SPLIT>(wb[m], lo, kn);
        w[m].db = load_db<SPLIT>(wb[m], dbo[m], kn);
    }
    float16v S[MATS];
#pragma unroll
    for (int m = 0; m < MATS; m++) S[m] = float16v{};
    const uint8_t *tokrow = cur + r * kTokB<LO>;
    const half8 *aminp = reinterpret_cast<const half8 *>(cur + kSumsOffT<LO> + r * 32 + 16 * h);
    AUnit a[2];  // unit u's operands, and unit u+1's read ahead
    read_a<LO>(a[0], tokrow, 0, h);
    const uint32_t mg = magic_reg();
#pragma unroll
    for (int u = 0; u < 8; u++) {
        if (u + 1 < 8) read_a<LO>(a[(u + 1) & 1], tokrow, u + 1, h);
        unit_mfma<MATS, LO>(w, hd, u, a[u & 1], mg, S);
#pragma unroll
        for (int m = 0; m < MATS; m++) w[m].q[u] = load_q<SPLIT>(wb[m], lo, kn, 1 + u, 8 * h);
        if (SPLIT && u == 3) {  // sub-blocks 0-3 done: their own d
#pragma unroll
            for (int m = 0; m < MATS; m++) {
                finish_first(hd[m], S[m], acc[m]);
                S[m] = float16v{};
            }
        }
        __builtin_amdgcn_sched_barrier(0);  // bounds the live operands to two units
    }
    const half8 amin = *aminp;
#pragma unroll
    for (int m = 0; m < MATS; m++) {
        if (SPLIT)
            finish_split(hd[m], amin, h, S[m], acc[m]);
        else
            finish_sb(hd[m], amin, h, S[m], acc[m]);
    }
    stage_store<8, LO>(nxt, act, wave, lane);
    lds_barrier();
}

__shared__ __attribute__((aligned(1024))) uint8_t s_stage0[kStageBytes];
__shared__ __attribute__((aligned(1024))) uint8_t s_stage1[kStageBytes];

// One pass of the block over super-blocks [kb0, kb1) for its 32 tokens.
// wb[m]: the wave's row group of matrix m (uniform); lo: this lane's row offset.
template <int MATS, bool SPLIT = false, bool LO = true>
__device__ __forceinline__ void block_pass(g_u8 *const (&wb)[MATS], uint32_t lo,
                                           const uint32_t (&dbo)[MATS], int kb0, int kb1,
                                           const StageSrc &src, float16v (&acc)[MATS]) {
    const int lane = threadIdx.x & 63, h = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int last = kb1 - 1;
    // opaque start: keeps the prologue's loads in base + 32-bit offset form
    // instead of per-lane 64-bit addresses folded and kept across passes
    asm volatile("" : "+s"(kb0));
    WRaw w[MATS];
    StageRegs<8, LO> act;
    stage_load<8, LO>(act, src, kb0, wave, lane);
#pragma unroll
    for (int m = 0; m < MATS; m++) load_w<SPLIT>(w[m], wb[m], lo, dbo[m], kb0, h);
    stage_store<8, LO>(s_stage0, act, wave, lane);
    lds_barrier();
    int kb = kb0;
    for (; kb + 2 <= kb1; kb += 2) {
        step<MATS, SPLIT, LO>(wb, lo, dbo, kb + 1, s_stage0, s_stage1, src, w, acc, wave, lane);
        step<MATS, SPLIT, LO>(wb, lo, dbo, min(kb + 2, last), s_stage1, s_stage0, src, w, acc,
                              wave, lane);
    }
    if (kb < kb1)
        step<MATS, SPLIT, LO>(wb, lo, dbo, kb, s_stage0, s_stage1, src, w, acc, wave, lane);
}

// ---- 16-token passes -------------------------------------------------------
// The wave's 32 rows are two 16-row tiles t = 0, 1.  Lane l (r16 = l % 16,
// c4 = l / 16) loads, for tile t, row 16t + r16's header and the 8 qs bytes
// 32p + 8*c4 .. +7 of each pair p: chunk 1 + 2p + c4/2, byte 8*(c4 % 2).
struct WRaw16 {
    u32x4 hdr[2];
    uint32_t db[2];  // split layout: the second (d, dmin) per tile
    u32x2 q[4][2];   // [pair][tile]
};

// lo: offset of this lane's row r16 of tile 0; tile 1 is the 16 rows after
// it, 256 bytes further in every chunk (64 bytes further in the pair area)
template <bool SPLIT = false>
__device__ __forceinline__ u32x2 load_q16(g_u8 *base, uint32_t lo, int kb, int p, int t, int c4) {
    return load_q<SPLIT>(base, lo, kb, 1 + 2 * p + (c4 >> 1), 256 * t + 8 * (c4 & 1));
}

template <bool SPLIT = false>
__device__ __forceinline__ void load_w16(WRaw16 &w, g_u8 *base, uint32_t lo, uint32_t dbo, int kb,
                                         int c4) {
#pragma unroll
    for (int t = 0; t < 2; t++) {
        w.hdr[t] = load_hdr<SPLIT>(base, lo, kb, 256 * t);
        w.db[t] = load_db<SPLIT>(base, dbo + 64 * t, kb);
    }
#pragma unroll
    for (int p = 0; p < 4; p++)
#pragma unroll
        for (int t = 0; t < 2; t++) w.q[p][t] = load_q16<SPLIT>(base, lo, kb, p, t, c4);
}

__device__ __forceinline__ void finish16(const Hdr &hd, const half4 &amin, int c4,
                                         const float4v &S, float4v &acc) {
    const float4v Smin =
        __builtin_amdgcn_mfma_f32_16x16x16f16(amin, min_operand16(hd, c4), float4v{}, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        acc[i] = __builtin_fmaf(hd.d, S[i], acc[i]);
        acc[i] = __builtin_fmaf(-hd.dmin, Smin[i], acc[i]);
    }
}

// finish16 for one half of a split-layout super-block: lanes c4 = 2 part,
// 2 part + 1 hold that half's mins
__device__ __forceinline__ void finish16_part(const Hdr &hd, const half4 &amin, int c4, int part,
                                              const float4v &S, float4v &acc) {
    const half4 mop = (c4 >> 1) == part ? min_operand16(hd, c4) : half4{};
    const float4v Smin = __builtin_amdgcn_mfma_f32_16x16x16f16(amin, mop, float4v{}, 0, 0, 0);
    const float dd = part ? hd.d2 : hd.d, dm = part ? hd.dmin2 : hd.dmin;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        acc[i] = __builtin_fmaf(dd, S[i], acc[i]);
        acc[i] = __builtin_fmaf(-dm, Smin[i], acc[i]);
    }
}

// Activation operands of pair p for a 16-token pass: token r16, columns
// 8*c4 .. +7 of sub-blocks 2p and 2p+1, hi and lo halves
template <bool LO = true>
__device__ __forceinline__ void read_a16(AUnit &a, const uint8_t *tokrow, int p, int c4) {
    const int col = 2 * (64 * p + 8 * c4);  // bytes
    a.h0 = *reinterpret_cast<const half8 *>(tokrow + col);
    a.h1 = *reinterpret_cast<const half8 *>(tokrow + col + 64);
    if constexpr (LO) {
        a.l0 = *reinterpret_cast<const half8 *>(tokrow + 512 + col);
        a.l1 = *reinterpret_cast<const half8 *>(tokrow + 512 + col + 64);
    }
}

// One step of a 16-token pass (same pipeline as step()).  Per pair p the
// activations of sub-blocks 2p and 2p+1 (hi, lo) are read once and shared by
// both tiles and all matrices.
template <int MATS, bool SPLIT = false, bool LO = true>
__device__ __forceinline__ void step16(g_u8 *const (&wb)[MATS], uint32_t lo,
                                       const uint32_t (&dbo)[MATS], int kn, const uint8_t *cur,
                                       uint8_t *nxt, const StageSrc &src, WRaw16 (&w)[MATS],
                                       float4v (&acc)[MATS][2], int wave, int lane) {
    const int r16 = lane & 15, c4 = lane >> 4;
    StageRegs<4, LO> act;
    stage_load<4, LO>(act, src, kn, wave, lane);
    __builtin_amdgcn_sched_barrier(0);  // keep the activation loads first
    Hdr hd[MATS][2];
#pragma unroll
    for (int m = 0; m < MATS; m++)
#pragma unroll
        for (int t = 0; t < 2; t++) {
            hd[m][t] = SPLIT ? unpack_hdr_split(w[m].hdr[t], w[m].db[t]) : unpack_hdr16(w[m].hdr[t]);
            w[m].hdr[t] = load_hdr<SPLIT>(wb[m], lo, kn, 256 * t);
            w[m].db[t] = load_db<SPLIT>(wb[m], dbo[m] + 64 * t, kn);
        }
    float4v S[MATS][2];
#pragma unroll
    for (int m = 0; m < MATS; m++) S[m][0] = S[m][1] = float4v{};
    const uint8_t *tokrow = cur + r16 * kTokB<LO>;
    const half4 *aminp = reinterpret_cast<const half4 *>(cur + kSumsOffT<LO> + r16 * 32 + 8 * c4);
    AUnit a[2];  // pair p's operands, and pair p+1's read ahead
    read_a16<LO>(a[0], tokrow, 0, c4);
    const uint32_t mg = magic_reg();
#pragma unroll
    for (int p = 0; p < 4; p++) {
        if (p + 1 < 4) read_a16<LO>(a[(p + 1) & 1], tokrow, p + 1, c4);
        const half8 h0 = a[p & 1].h0, l0 = a[p & 1].l0, h1 = a[p & 1].h1, l1 = a[p & 1].l1;
#pragma unroll
        for (int m = 0; m < MATS; m++)
#pragma unroll
            for (int t = 0; t < 2; t++) {
                half8 blo, bhi;
                dec_pair(hd[m][t], p, w[m].q[p][t].x, w[m].q[p][t].y, mg, blo, bhi);
                w[m].q[p][t] = load_q16<SPLIT>(wb[m], lo, kn, p, t, c4);
                S[m][t] = mfma16(h0, blo, S[m][t]);
                if constexpr (LO) S[m][t] = mfma16(l0, blo, S[m][t]);
                S[m][t] = mfma16(h1, bhi, S[m][t]);
                if constexpr (LO) S[m][t] = mfma16(l1, bhi, S[m][t]);
            }
        if (SPLIT && p == 1) {  // sub-blocks 0-3 done: their own d, dmin
            const half4 amin = *aminp;
#pragma unroll
            for (int m = 0; m < MATS; m++)
#pragma unroll
                for (int t = 0; t < 2; t++) {
                    finish16_part(hd[m][t], amin, c4, 0, S[m][t], acc[m][t]);
                    S[m][t] = float4v{};
                }
        }
        __builtin_amdgcn_sched_barrier(0);  // bounds the live operands to two pairs
    }
    const half4 amin = *aminp;
#pragma unroll
    for (int m = 0; m < MATS; m++)
#pragma unroll
        for (int t = 0; t < 2; t++) {
            if (SPLIT)
                finish16_part(hd[m][t], amin, c4, 1, S[m][t], acc[m][t]);
            else
                finish16(hd[m][t], amin, c4, S[m][t], acc[m][t]);
        }
    stage_store<4, LO>(nxt, act, wave, lane);
    lds_barrier();
}

// block_pass() for a pass of at most 16 tokens; lo is the offset of this
// lane's row r16 of the wave's first tile
template <int MATS, bool SPLIT = false, bool LO = true>
__device__ __forceinline__ void block_pass16(g_u8 *const (&wb)[MATS], uint32_t lo,
                                             const uint32_t (&dbo)[MATS], int kb0, int kb1,
                                             const StageSrc &src, float4v (&acc)[MATS][2]) {
    const int lane = threadIdx.x & 63, c4 = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int last = kb1 - 1;
    asm volatile("" : "+s"(kb0));  // see block_pass()
    WRaw16 w[MATS];
    StageRegs<4, LO> act;
    stage_load<4, LO>(act, src, kb0, wave, lane);
#pragma unroll
    for (int m = 0; m < MATS; m++) load_w16<SPLIT>(w[m], wb[m], lo, dbo[m], kb0, c4);
    stage_store<4, LO>(s_stage0, act, wave, lane);
    lds_barrier();
    int kb = kb0;
    for (; kb + 2 <= kb1; kb += 2) {
        step16<MATS, SPLIT, LO>(wb, lo, dbo, kb + 1, s_stage0, s_stage1, src, w, acc, wave, lane);
        step16<MATS, SPLIT, LO>(wb, lo, dbo, min(kb + 2, last), s_stage1, s_stage0, src, w, acc,
                                wave, lane);
    }
    if (kb < kb1)
        step16<MATS, SPLIT, LO>(wb, lo, dbo, kb, s_stage0, s_stage1, src, w, acc, wave, lane);
}

// split v into f16 hi + lo
__device__ __forceinline__ void split16(float v, _Float16 &hi, _Float16 &lo) {
    hi = (_Float16)v;
    lo = (_Float16)(v - (float)hi);
}

// token (within the pass) held in C register i by half h
__device__ __forceinline__ int c_token(int i, int h) { return 8 * (i >> 2) + 4 * h + (i & 3); }

// Each wave of a chain block streams its chain tiles through its own half
// of one activation stage.
static_assert(kStageBytes / 8 >= chain_lds_floats(16, 128), "chain tile LDS");

// grid (F/128 row blocks, [chain row +] slots, pass groups); block = 4 waves
// x 32 weight rows.  With ch.tiles, row y = 0 runs the exact router chains
// (a wave per 8 x 8 tile, blocks of z = 0) and slot s is row s + 1.
// LO: x enters as two f16 (hi + lo); otherwise as its hi half alone.  H
// leaves in the format the down products of the same mode take (with LO
// its lo halves and the sums of hi + lo, without it sums of hi alone).
template <bool LO>
__global__ __launch_bounds__(256, 2) void k_mfma_gateup(
    const uint8_t *__restrict__ gate, const uint8_t *__restrict__ up, int64_t estride,
    const _Float16 *__restrict__ x16, const _Float16 *__restrict__ xs, SlotArgs sa, int d, int F,
    _Float16 *__restrict__ h16, _Float16 *__restrict__ hs, float *__restrict__ hf, ChainArgs ch) {
    int slot = blockIdx.y;
    if (ch.tiles) {
        if (slot == 0) {
            if (blockIdx.z) return;
            const int cw = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
            float *lds = reinterpret_cast<float *>(cw < 2 ? s_stage0 : s_stage1) +
                         (cw & 1) * (kStageBytes / 8);
            for (int tile = blockIdx.x * kWaves + cw; tile < ch.tiles; tile += gridDim.x * kWaves)
                chain_tile<8, 128, 1>(ch, tile, lds);
            return;
        }
        slot -= 1;
    }
    int e, p0, n;
    if (!slot_info(sa, slot, e, p0, n)) return;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, r = lane & 31, h = lane >> 5;
    const int ngrp = F >> 5, grp0 = blockIdx.x * kWaves + wave;
    const int grp = min(grp0, ngrp - 1);  // duplicate the last group past the end
    const int NB = d >> 8, tile = grp >> 1, nsb = d >> 5;
    const int64_t grpoff = (int64_t)tile * NB * 9 * 1024 + 32 * (grp & 1) * 16;
    g_u8 *const wb[2] = {uniform(gate + (int64_t)e * estride + grpoff),
                                  uniform(up + (int64_t)e * estride + grpoff)};
    // H rows: ceil(F / 256) pieces and 8 sums per piece (zero past F)
    const int f = grp * 32 + r, nkb = (F + 255) >> 8, hsr = nkb * 8;
    const uint32_t nodb[2] = {0, 0};
    const uint8_t *xb = reinterpret_cast<const uint8_t *>(x16);
    const uint8_t *sb = reinterpret_cast<const uint8_t *>(xs);
    for (int c = blockIdx.z * kTok; c < n; c += gridDim.z * kTok) {
        StageSrc src;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int tok = slot_token(sa, p0, min(c + wave + 4 * i, n - 1));
            src.tok[i] = uniform(xb + (int64_t)tok * d * 4);
        }
        src.sums = uniform(sb);
        src.soff = (uint32_t)slot_token(sa, p0, min(c + (lane >> 1), n - 1)) * nsb * 4 +
                   16 * (lane & 1);
        if (n - c <= 16) {
            const int r16 = lane & 15, c4 = lane >> 4;
            float4v acc[2][2] = {};
            block_pass16<2, false, LO>(wb, r16 * 16, nodb, 0, NB, src, acc);
            if (grp0 >= ngrp) continue;
            // output addresses are formed here from an opaque row index, so
            // that the compiler does not keep them live across the pass
            int fb = grp * 32 + r16;
            asm volatile("" : "+v"(fb));
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int q = c + 4 * c4 + i;
                _Float16 hi[2], lo[2];
                float v[2], part = 0.0f;
#pragma unroll
                for (int t = 0; t < 2; t++) {
                    v[t] = silu(acc[0][t][i]) * acc[1][t][i];
                    split16(v[t], hi[t], lo[t]);
                    // the sums of what the down products take
                    part += LO ? (float)hi[t] + (float)lo[t] : (float)hi[t];
                }
#pragma unroll
                for (int off = 1; off < 16; off <<= 1) part += __shfl_xor(part, off, 64);
                if (q < n) {
                    const int64_t p = p0 + q;
#pragma unroll
                    for (int t = 0; t < 2; t++) {
                        const int ft = fb + 16 * t;
                        if (hf) hf[p * F + ft] = v[t];
                        if (h16) {
                            _Float16 *piece = h16 + (p * nkb + (ft >> 8)) * 512 + act16_pos(ft & 255);
                            piece[0] = hi[t];
                            if (LO) piece[256] = lo[t];
                        }
                    }
                    if (h16 && r16 == 0) {
                        _Float16 shi, slo;
                        split16(part, shi, slo);
                        hs[(p * hsr + grp) * 2] = shi;
                        hs[(p * hsr + grp) * 2 + 1] = slo;
                    }
                }
            }
            continue;
        }
        float16v acc[2] = {float16v{}, float16v{}};
        block_pass<2, false, LO>(wb, r * 16, nodb, 0, NB, src, acc);
        if (grp0 >= ngrp) continue;
        int fo = f;  // opaque copy: output addresses are formed here (see above)
        asm volatile("" : "+v"(fo));
        // SwiGLU, H out (f16 hi/lo pieces and/or f32), 32-row sub-block sums
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int q = c + c_token(i, h);
            const float v = silu(acc[0][i]) * acc[1][i];
            _Float16 hi, lo;
            split16(v, hi, lo);
            float part = LO ? (float)hi + (float)lo : (float)hi;
#pragma unroll
            for (int off = 1; off < 32; off <<= 1) part += __shfl_xor(part, off, 64);
            if (q < n) {
                const int64_t p = p0 + q;
                if (hf) hf[p * F + fo] = v;
                if (h16) {
                    _Float16 *piece = h16 + (p * nkb + (fo >> 8)) * 512 + act16_pos(fo & 255);
                    piece[0] = hi;
                    if (LO) piece[256] = lo;
                    if (r == 0) {
                        _Float16 shi, slo;
                        split16(part, shi, slo);
                        hs[(p * hsr + grp) * 2] = shi;
                        hs[(p * hsr + grp) * 2 + 1] = slo;
                    }
                }
            }
        }
    }
}

// grid (d/256 row blocks, slots, ksplit x pass groups); z = split + ksplit *
// group.  Partial sums of K split z go to Y + z * split_stride.  A wave owns
// one 64-row RPL tile as two 32-row halves that share every activation read
// (the two "matrices" of the pipeline), so each LDS read feeds twice the
// weight bytes of a 32-row wave.  SPLIT: F is an odd multiple of 128 and the
// weights are in the split layout (ceil(F / 256) super-blocks per row).
template <bool SPLIT, bool LO>
__global__ __launch_bounds__(256, 2) void k_mfma_down(
    const uint8_t *__restrict__ down, int64_t estride, const _Float16 *__restrict__ h16,
    const _Float16 *__restrict__ hs, SlotArgs sa, int d, int F, int ksplit, float *__restrict__ Y,
    int64_t split_stride) {
    // Workgroups go to the 8 XCDs round-robin in dispatch order and each XCD
    // has its own L2.  Every (slot, split) pair reads one slice of H, shared
    // by its row blocks: remap the grid so that each XCD runs whole pairs and
    // keeps only its pairs' slices.  Pair p goes to XCD p % 8, so the pairs of
    // slot rows that exit at once (pass slots past the realised count) spread
    // over the XCDs (identity when the pair count is not a multiple of 8).
    int bx = blockIdx.x, by = blockIdx.y, bz = blockIdx.z;
    {
        const int nx = gridDim.x, ny = gridDim.y;
        const int id = bx + nx * (by + ny * bz), pairs = ny * gridDim.z;
        if (pairs % kXcds == 0) {  // pair p on XCD p % 8, all of its row blocks
            const int j = id / kXcds, pair = id % kXcds + kXcds * (j / nx);
            bx = j % nx;
            by = pair % ny;
            bz = pair / ny;
        }
    }
    const int cz = bz / ksplit, nz = gridDim.z / ksplit;  // pass group
    bz -= cz * ksplit;                                     // K split
    int e, p0, n;
    if (!slot_info(sa, by, e, p0, n)) return;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, r = lane & 31, h = lane >> 5;
    const int ntile = d >> 6, tile0 = bx * kWaves + wave;
    const int tile = min(tile0, ntile - 1);  // duplicate the last tile past the end
    const int NB = (F + 255) >> 8, nsb = NB * 8;
    const int kb0 = (int)((int64_t)NB * bz / ksplit);
    const int kb1 = (int)((int64_t)NB * (bz + 1) / ksplit);
    const uint8_t *tb = down + (int64_t)e * estride + (int64_t)tile * NB * kTileSB<SPLIT>;
    g_u8 *const wb[2] = {uniform(tb), uniform(tb + 32 * 16)};
    float *Yz = Y + (int64_t)bz * split_stride;
    const uint8_t *hb = reinterpret_cast<const uint8_t *>(h16);
    const uint8_t *sb = reinterpret_cast<const uint8_t *>(hs);
    for (int c = cz * kTok; c < n; c += nz * kTok) {
        StageSrc src;
#pragma unroll
        for (int i = 0; i < 8; i++)
            src.tok[i] = uniform(hb + (int64_t)(p0 + min(c + wave + 4 * i, n - 1)) * NB * 1024);
        src.sums = uniform(sb);
        src.soff = (uint32_t)(p0 + min(c + (lane >> 1), n - 1)) * nsb * 4 + 16 * (lane & 1);
        if (n - c <= 16) {
            const int r16 = lane & 15, c4 = lane >> 4;
            // pair-area offsets of rows r16 (half 0) and 32 + r16 (half 1),
            // from each half's base
            const uint32_t dbo[2] = {9 * 1024 + 4 * (uint32_t)r16,
                                     9 * 1024 + 4 * (32 + (uint32_t)r16) - 32 * 16};
            float4v acc[2][2] = {};
            block_pass16<2, SPLIT, LO>(wb, r16 * 16, dbo, kb0, kb1, src, acc);
            if (tile0 >= ntile) continue;
            int rb = tile * 64 + r16;  // opaque: output addresses are formed here
            asm volatile("" : "+v"(rb));
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int q = c + 4 * c4 + i;
                if (q < n) {
                    float *yrow = Yz + (int64_t)(p0 + q) * d + rb;
#pragma unroll
                    for (int m = 0; m < 2; m++)
#pragma unroll
                        for (int t = 0; t < 2; t++) yrow[32 * m + 16 * t] = acc[m][t][i];
                }
            }
            continue;
        }
        const uint32_t dbo[2] = {9 * 1024 + 4 * (uint32_t)r,
                                 9 * 1024 + 4 * (32 + (uint32_t)r) - 32 * 16};
        float16v acc[2] = {float16v{}, float16v{}};
        block_pass<2, SPLIT, LO>(wb, r * 16, dbo, kb0, kb1, src, acc);
        if (tile0 >= ntile) continue;
        int rb = tile * 64 + r;  // opaque: output addresses are formed here
        asm volatile("" : "+v"(rb));
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int q = c + c_token(i, h);
            if (q < n) {
                float *yrow = Yz + (int64_t)(p0 + q) * d + rb;
                yrow[0] = acc[0][i];
                yrow[32] = acc[1][i];
            }
        }
    }
}

// ---- Q6_K down ------------------------------------------------------------
// Weights in the RPL64 Q6_K layout (lcmoe_host.cpp): per 64-row tile and
// super-block, thirteen 1 KiB chunks (chunk c = bytes 16c .. 16c+15 of every
// row's 210-byte block: ql in 0-7, qh in 8-11, the 16 int8 scales in 12) and
// then the 64 rows' f16 d.
//
// Element 128n + 32j + l of a block (half n, group j, l < 32) has the 6-bit
// code q = (4 bits of ql) | (2 bits of qh) << 4 (dequantize_q6_k,
// rust/src/kernels/mod.rs:145-180):
//   j = 0: ql[64n + l] low,  qh[32n + l] bits 0-1    j = 1: ql[64n+32+l] low,  bits 2-3
//   j = 2: ql[64n + l] high, qh[32n + l] bits 4-5    j = 3: ql[64n+32+l] high, bits 6-7
// and the value d * sc[8n + 2j + l/16] * (q - 32).  A 16-column K-step is
// one scale group.  sc * (q - 32) reaches 4096, past the integers f16 holds
// exactly, so the scale is split as sc = 16 sh + sl (sh = sc >> 4 in
// [-8, 7], sl = sc & 15): B1 = sh (q - 32) and B2 = sl (q - 32) are exact
// f16 values, and S = 16 S1 + S2 with S1 = A B1, S2 = A B2 (four MFMAs per
// K-step with the activations' hi/lo halves).  Lane (r, h) of a 32-row half
// takes, per unit v = 2n + i, the 8 bytes at 8h of ql chunks 4n+i and
// 4n+2+i and of qh chunk 8+2n+i: columns 128n + 32j + 16i + 8h .. +7 of the
// four groups j.
constexpr int kQ6Chunks = 13;
constexpr int kQ6Stride = kQ6Chunks * 1024 + 128;

struct W6 {
    u32x4 sc;        // the row's 16 scales
    uint32_t d;      // the row's d (f16 bits)
    u32x2 q[4][3];   // per unit: ql (groups 0, 2), ql (groups 1, 3), qh
};

__device__ __forceinline__ u32x2 load_q6(g_u8 *base, uint32_t lo, int kb, int chunk) {
    return gload<u32x2>(base + (lo + (uint32_t)(kb * kQ6Stride + chunk * 1024)));
}

// lo: this lane's row offset (row * 16) plus 8h; dlo: the row's d offset
__device__ __forceinline__ void load_w6_unit(W6 &w, g_u8 *base, uint32_t lo, int kb, int v) {
    const int n = v >> 1, i = v & 1;
    w.q[v][0] = load_q6(base, lo, kb, 4 * n + i);
    w.q[v][1] = load_q6(base, lo, kb, 4 * n + 2 + i);
    w.q[v][2] = load_q6(base, lo, kb, 8 + 2 * n + i);
}

__device__ __forceinline__ void load_w6_head(W6 &w, g_u8 *base, uint32_t rlo, uint32_t dlo,
                                             int kb) {
    w.sc = gload<u32x4>(base + (rlo + (uint32_t)(kb * kQ6Stride + 12 * 1024)));
    w.d = gload<uint16_t>(base + (dlo + (uint32_t)(kb * kQ6Stride + kQ6Chunks * 1024)));
}

// 6-bit codes of group j from one unit's words (one code per byte)
__device__ __forceinline__ uint32_t q6_group(uint32_t qa, uint32_t qb, uint32_t qh, int j) {
    switch (j) {
    case 0: return (qa & 0x0F0F0F0Fu) | ((qh << 4) & 0x30303030u);
    case 1: return (qb & 0x0F0F0F0Fu) | ((qh << 2) & 0x30303030u);
    case 2: return ((qa >> 4) & 0x0F0F0F0Fu) | (qh & 0x30303030u);
    default: return ((qb >> 4) & 0x0F0F0F0Fu) | ((qh >> 2) & 0x30303030u);
    }
}

// byte b of w twice, as the f16 pair (1024 + byte, 1024 + byte)
__device__ __forceinline__ half2v magic_bb(uint32_t w, int b) {
    const uint32_t sel = 0x04000400u | ((uint32_t)b << 16) | (uint32_t)b;
    return magic2(w, sel);
}

// B1 = sh (q - 32), B2 = sl (q - 32) for 8 codes (bytes of g0, g1):
// (1024 + q) s - 1056 s, one rounding of an exact integer result
__device__ __forceinline__ void dec6(uint32_t g0, uint32_t g1, half2v sh2, half2v c1, half2v sl2,
                                     half2v c2, half8 &b1, half8 &b2) {
    // the activation format's column order (act16_pos): bytes 0, 2, 1, 3, ...
    const half2v m[4] = {magic2(g0, kSel02), magic2(g0, kSel13), magic2(g1, kSel02),
                         magic2(g1, kSel13)};
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const half2v x = __builtin_elementwise_fma(m[k], sh2, c1);
        const half2v y = __builtin_elementwise_fma(m[k], sl2, c2);
        b1[2 * k] = x[0];
        b1[2 * k + 1] = x[1];
        b2[2 * k] = y[0];
        b2[2 * k + 1] = y[1];
    }
}

// One step of a 32-token pass over Q6_K: super-block k of both 32-row halves
// from `cur` and w; activations of super-block kn into `nxt`; w reloaded
// with kn unit by unit after each unit's decode.
template <bool LO>
__device__ __forceinline__ void step_q6(g_u8 *wb, const uint32_t (&lo)[2], const uint32_t (&rlo)[2],
                                        const uint32_t (&dlo)[2], int kn, const uint8_t *cur,
                                        uint8_t *nxt, const StageSrc &src, W6 (&w)[2],
                                        float16v (&acc)[2], int wave, int lane) {
    const int r = lane & 31, h = lane >> 5;
    StageRegs<8, LO> act;
    stage_load<8, LO>(act, src, kn, wave, lane);
    __builtin_amdgcn_sched_barrier(0);
    u32x4 sc[2];
    float dd[2];
#pragma unroll
    for (int m = 0; m < 2; m++) {
        sc[m] = w[m].sc;
        dd[m] = dh2f(w[m].d & 0xffff);
        load_w6_head(w[m], wb, rlo[m], dlo[m], kn);
    }
    float16v S1[2], S2[2];
#pragma unroll
    for (int m = 0; m < 2; m++) S1[m] = S2[m] = float16v{};
    const uint8_t *tokrow = cur + r * kTokB<LO>;
    const half2v k1024 = half2v{(_Float16)-1024.0f, (_Float16)-1024.0f};
    const half2v k1032 = half2v{(_Float16)-1032.0f, (_Float16)-1032.0f};
    const half2v k1056 = half2v{(_Float16)-1056.0f, (_Float16)-1056.0f};
#pragma unroll
    for (int v = 0; v < 4; v++) {
        const int n = v >> 1, i = v & 1;
        // scale nibbles of this unit's four groups: bytes i, i + 2 of words
        // 2n (groups 0, 1) and 2n + 1 (groups 2, 3)
        uint32_t sl_w[2][2], sh_w[2][2];
#pragma unroll
        for (int m = 0; m < 2; m++)
#pragma unroll
            for (int k = 0; k < 2; k++) {
                const uint32_t wv = sc[m][2 * n + k];
                sl_w[m][k] = wv & 0x0F0F0F0Fu;
                sh_w[m][k] = ((wv >> 4) & 0x0F0F0F0Fu) ^ 0x08080808u;  // sh + 8
            }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int col = 2 * (128 * n + 32 * j + 16 * i + 8 * h);  // bytes
            const half8 ah = *reinterpret_cast<const half8 *>(tokrow + col);
            half8 al{};
            if constexpr (LO) al = *reinterpret_cast<const half8 *>(tokrow + 512 + col);
#pragma unroll
            for (int m = 0; m < 2; m++) {
                const int b = i + 2 * (j & 1);
                const half2v sl2 = magic_bb(sl_w[m][j >> 1], b) + k1024;
                const half2v sh2 = magic_bb(sh_w[m][j >> 1], b) + k1032;
                const half2v c1 = sh2 * k1056, c2 = sl2 * k1056;
                const uint32_t g0 = q6_group(w[m].q[v][0].x, w[m].q[v][1].x, w[m].q[v][2].x, j);
                const uint32_t g1 = q6_group(w[m].q[v][0].y, w[m].q[v][1].y, w[m].q[v][2].y, j);
                half8 b1, b2;
                dec6(g0, g1, sh2, c1, sl2, c2, b1, b2);
                S1[m] = mfma32(ah, b1, S1[m]);
                if constexpr (LO) S1[m] = mfma32(al, b1, S1[m]);
                S2[m] = mfma32(ah, b2, S2[m]);
                if constexpr (LO) S2[m] = mfma32(al, b2, S2[m]);
            }
        }
#pragma unroll
        for (int m = 0; m < 2; m++) load_w6_unit(w[m], wb, lo[m], kn, v);
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int m = 0; m < 2; m++) {
        const float d16 = 16.0f * dd[m];
#pragma unroll
        for (int t = 0; t < 16; t++) {
            acc[m][t] = __builtin_fmaf(d16, S1[m][t], acc[m][t]);
            acc[m][t] = __builtin_fmaf(dd[m], S2[m][t], acc[m][t]);
        }
    }
    stage_store<8, LO>(nxt, act, wave, lane);
    lds_barrier();
}

template <bool LO>
__device__ __forceinline__ void block_pass_q6(g_u8 *wb, const uint32_t (&lo)[2],
                                              const uint32_t (&rlo)[2], const uint32_t (&dlo)[2],
                                              int kb0, int kb1, const StageSrc &src,
                                              float16v (&acc)[2]) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int last = kb1 - 1;
    asm volatile("" : "+s"(kb0));  // see block_pass()
    W6 w[2];
    StageRegs<8, LO> act;
    stage_load<8, LO>(act, src, kb0, wave, lane);
#pragma unroll
    for (int m = 0; m < 2; m++) {
        load_w6_head(w[m], wb, rlo[m], dlo[m], kb0);
#pragma unroll
        for (int v = 0; v < 4; v++) load_w6_unit(w[m], wb, lo[m], kb0, v);
    }
    stage_store<8, LO>(s_stage0, act, wave, lane);
    lds_barrier();
    int kb = kb0;
    for (; kb + 2 <= kb1; kb += 2) {
        step_q6<LO>(wb, lo, rlo, dlo, kb + 1, s_stage0, s_stage1, src, w, acc, wave, lane);
        step_q6<LO>(wb, lo, rlo, dlo, min(kb + 2, last), s_stage1, s_stage0, src, w, acc, wave,
                    lane);
    }
    if (kb < kb1) step_q6<LO>(wb, lo, rlo, dlo, kb, s_stage0, s_stage1, src, w, acc, wave, lane);
}

// ---- Q6_K down, 16-token passes (v_mfma_f32_16x16x32_f16) ------------------
// A wave's 64 rows are four 16-row tiles (half m, tile t: rows 32m + 16t ..).
// Lane (r16, c4) takes row r16 of each tile and, per 32-column group j of
// block half n, columns 8c4 .. 8c4+7: the 8 bytes at 8(c4 & 1) of ql chunks
// 4n + c4/2 (groups 0, 2) and 4n + 2 + c4/2 (groups 1, 3) and of qh chunk
// 8 + 2n + c4/2; its scale is sc[8n + 2j + c4/2].  The split B1, B2 of the
// 32-token kernel is per element, so one MFMA may span two scale groups.
struct W6t {
    u32x4 sc;
    uint32_t d;
    u32x2 q[2][3];  // per half n: ql (groups 0, 2), ql (groups 1, 3), qh
};

__device__ __forceinline__ void load_w6t_head(W6t &w, g_u8 *base, uint32_t rlo, uint32_t dlo,
                                              int kb) {
    w.sc = gload<u32x4>(base + (rlo + (uint32_t)(kb * kQ6Stride + 12 * 1024)));
    w.d = gload<uint16_t>(base + (dlo + (uint32_t)(kb * kQ6Stride + kQ6Chunks * 1024)));
}

// lo: row offset (row * 16) + 8 (c4 & 1); cb = c4 / 2
__device__ __forceinline__ void load_w6t_half(W6t &w, g_u8 *base, uint32_t lo, int kb, int n,
                                              int cb) {
    w.q[n][0] = load_q6(base, lo, kb, 4 * n + cb);
    w.q[n][1] = load_q6(base, lo, kb, 4 * n + 2 + cb);
    w.q[n][2] = load_q6(base, lo, kb, 8 + 2 * n + cb);
}

template <bool LO>
__device__ __forceinline__ void step16_q6(g_u8 *wb, const uint32_t (&lo)[2][2],
                                          const uint32_t (&rlo)[2][2], const uint32_t (&dlo)[2][2],
                                          int kn, const uint8_t *cur, uint8_t *nxt,
                                          const StageSrc &src, W6t (&w)[2][2],
                                          float4v (&acc)[2][2], int wave, int lane) {
    const int r16 = lane & 15, c4 = lane >> 4, cb = c4 >> 1;
    StageRegs<4, LO> act;
    stage_load<4, LO>(act, src, kn, wave, lane);
    __builtin_amdgcn_sched_barrier(0);
    // scales are read from w and reloaded with kn after the last group
    float dd[2][2];
#pragma unroll
    for (int m = 0; m < 2; m++)
#pragma unroll
        for (int t = 0; t < 2; t++) dd[m][t] = dh2f(w[m][t].d & 0xffff);
    float4v S1[2][2], S2[2][2];
#pragma unroll
    for (int m = 0; m < 2; m++)
#pragma unroll
        for (int t = 0; t < 2; t++) S1[m][t] = S2[m][t] = float4v{};
    const uint8_t *tokrow = cur + r16 * kTokB<LO>;
    const half2v k1024 = half2v{(_Float16)-1024.0f, (_Float16)-1024.0f};
    const half2v k1032 = half2v{(_Float16)-1032.0f, (_Float16)-1032.0f};
    const half2v k1056 = half2v{(_Float16)-1056.0f, (_Float16)-1056.0f};
#pragma unroll
    for (int n = 0; n < 2; n++) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int col = 2 * (128 * n + 32 * j + 8 * c4);  // bytes
            const half8 ah = *reinterpret_cast<const half8 *>(tokrow + col);
            half8 al{};
            if constexpr (LO) al = *reinterpret_cast<const half8 *>(tokrow + 512 + col);
            const int b = 2 * (j & 1) + cb;  // scale byte within word 2n + j/2
#pragma unroll
            for (int m = 0; m < 2; m++)
#pragma unroll
                for (int t = 0; t < 2; t++) {
                    const uint32_t wv = w[m][t].sc[2 * n + (j >> 1)];
                    const half2v sl2 = magic_bb(wv & 0x0F0F0F0Fu, b) + k1024;
                    const half2v sh2 = magic_bb(((wv >> 4) & 0x0F0F0F0Fu) ^ 0x08080808u, b) + k1032;
                    const half2v c1 = sh2 * k1056, c2 = sl2 * k1056;
                    const u32x2 qa = w[m][t].q[n][0], qb = w[m][t].q[n][1], qh = w[m][t].q[n][2];
                    const uint32_t g0 = q6_group(qa.x, qb.x, qh.x, j);
                    const uint32_t g1 = q6_group(qa.y, qb.y, qh.y, j);
                    half8 b1, b2;
                    dec6(g0, g1, sh2, c1, sl2, c2, b1, b2);
                    S1[m][t] = mfma16(ah, b1, S1[m][t]);
                    if constexpr (LO) S1[m][t] = mfma16(al, b1, S1[m][t]);
                    S2[m][t] = mfma16(ah, b2, S2[m][t]);
                    if constexpr (LO) S2[m][t] = mfma16(al, b2, S2[m][t]);
                }
        }
#pragma unroll
        for (int m = 0; m < 2; m++)
#pragma unroll
            for (int t = 0; t < 2; t++) {
                load_w6t_half(w[m][t], wb, lo[m][t], kn, n, cb);
                if (n == 1) load_w6t_head(w[m][t], wb, rlo[m][t], dlo[m][t], kn);
            }
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int m = 0; m < 2; m++)
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const float d16 = 16.0f * dd[m][t];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                acc[m][t][i] = __builtin_fmaf(d16, S1[m][t][i], acc[m][t][i]);
                acc[m][t][i] = __builtin_fmaf(dd[m][t], S2[m][t][i], acc[m][t][i]);
            }
        }
    stage_store<4, LO>(nxt, act, wave, lane);
    lds_barrier();
}

template <bool LO>
__device__ __forceinline__ void block_pass16_q6(g_u8 *wb, const uint32_t (&lo)[2][2],
                                                const uint32_t (&rlo)[2][2],
                                                const uint32_t (&dlo)[2][2], int kb0, int kb1,
                                                const StageSrc &src, float4v (&acc)[2][2]) {
    const int lane = threadIdx.x & 63, cb = (lane >> 4) >> 1;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int last = kb1 - 1;
    asm volatile("" : "+s"(kb0));  // see block_pass()
    W6t w[2][2];
    StageRegs<4, LO> act;
    stage_load<4, LO>(act, src, kb0, wave, lane);
#pragma unroll
    for (int m = 0; m < 2; m++)
#pragma unroll
        for (int t = 0; t < 2; t++) {
            load_w6t_head(w[m][t], wb, rlo[m][t], dlo[m][t], kb0);
#pragma unroll
            for (int n = 0; n < 2; n++) load_w6t_half(w[m][t], wb, lo[m][t], kb0, n, cb);
        }
    stage_store<4, LO>(s_stage0, act, wave, lane);
    lds_barrier();
    int kb = kb0;
    for (; kb + 2 <= kb1; kb += 2) {
        step16_q6<LO>(wb, lo, rlo, dlo, kb + 1, s_stage0, s_stage1, src, w, acc, wave, lane);
        step16_q6<LO>(wb, lo, rlo, dlo, min(kb + 2, last), s_stage1, s_stage0, src, w, acc, wave,
                      lane);
    }
    if (kb < kb1)
        step16_q6<LO>(wb, lo, rlo, dlo, kb, s_stage0, s_stage1, src, w, acc, wave, lane);
}

// grid (d/256 row blocks, slots, ksplit x pass groups), as k_mfma_down.
// PASS 0: each slot takes passes of 32 tokens (32x32x16 MFMAs: one decode
// per weight for up to 32 tokens) while more than 16 remain, the rest as
// one pass of up to 16 (16x16x32 MFMAs: half the matrix-core work).  With
// two f16 per activation that kernel outgrows the register file, so LO
// takes one kind per kernel: PASS 16 or 32.
template <bool LO, int PASS>
__global__ __launch_bounds__(256, 2) void k_mfma_down_q6(
    const uint8_t *__restrict__ down, int64_t estride, const _Float16 *__restrict__ h16,
    SlotArgs sa, int d, int F, int ksplit, float *__restrict__ Y, int64_t split_stride) {
    int bx = blockIdx.x, by = blockIdx.y, bz = blockIdx.z;
    {
        const int nx = gridDim.x, ny = gridDim.y;
        const int id = bx + nx * (by + ny * bz), pairs = ny * gridDim.z;
        if (pairs % kXcds == 0) {  // pair p on XCD p % 8, all of its row blocks
            const int j = id / kXcds, pair = id % kXcds + kXcds * (j / nx);
            bx = j % nx;
            by = pair % ny;
            bz = pair / ny;
        }
    }
    const int cz = bz / ksplit, nz = gridDim.z / ksplit;
    bz -= cz * ksplit;
    int e, p0, n;
    if (!slot_info(sa, by, e, p0, n)) return;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, r = lane & 31, h = lane >> 5;
    const int ntile = d >> 6, tile0 = bx * kWaves + wave;
    const int tile = min(tile0, ntile - 1);  // duplicate the last tile past the end
    const int NB = F >> 8;
    const int kb0 = (int)((int64_t)NB * bz / ksplit);
    const int kb1 = (int)((int64_t)NB * (bz + 1) / ksplit);
    g_u8 *const wb = uniform(down + (int64_t)e * estride + (int64_t)tile * NB * kQ6Stride);
    const uint32_t rlo[2] = {(uint32_t)r * 16, (uint32_t)(32 + r) * 16};
    const uint32_t lo[2] = {rlo[0] + 8 * h, rlo[1] + 8 * h};
    const uint32_t dlo[2] = {(uint32_t)r * 2, (uint32_t)(32 + r) * 2};
    float *Yz = Y + (int64_t)bz * split_stride;
    const uint8_t *hb = reinterpret_cast<const uint8_t *>(h16);
    constexpr int kPass = PASS == 16 ? 16 : kTok;
    for (int c = cz * kPass; c < n; c += nz * kPass) {
        StageSrc src;
#pragma unroll
        for (int i = 0; i < 8; i++)
            src.tok[i] = uniform(hb + (int64_t)(p0 + min(c + wave + 4 * i, n - 1)) * F * 4);
        // the sums are not used (Q6_K has no mins): stage a valid row
        src.sums = uniform(hb);
        src.soff = 16 * (uint32_t)lane;
        if (PASS == 16 || (PASS == 0 && n - c <= 16)) {
            const int r16 = lane & 15, c4 = lane >> 4;
            uint32_t lo16[2][2], rlo16[2][2], dlo16[2][2];
#pragma unroll
            for (int m = 0; m < 2; m++)
#pragma unroll
                for (int t = 0; t < 2; t++) {
                    const uint32_t row = 32 * m + 16 * t + r16;
                    rlo16[m][t] = row * 16;
                    lo16[m][t] = row * 16 + 8 * (c4 & 1);
                    dlo16[m][t] = row * 2;
                }
            float4v acc[2][2] = {};
            block_pass16_q6<LO>(wb, lo16, rlo16, dlo16, kb0, kb1, src, acc);
            if (tile0 >= ntile) continue;
            int rb = tile * 64 + r16;  // opaque: output addresses are formed here
            asm volatile("" : "+v"(rb));
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int q = c + 4 * c4 + i;
                if (q < n) {
                    float *yrow = Yz + (int64_t)(p0 + q) * d + rb;
#pragma unroll
                    for (int m = 0; m < 2; m++)
#pragma unroll
                        for (int t = 0; t < 2; t++) yrow[32 * m + 16 * t] = acc[m][t][i];
                }
            }
        } else if constexpr (PASS != 16) {
        float16v acc[2] = {float16v{}, float16v{}};
        block_pass_q6<LO>(wb, lo, rlo, dlo, kb0, kb1, src, acc);
        if (tile0 >= ntile) continue;
        int rb = tile * 64 + r;  // opaque: output addresses are formed here
        asm volatile("" : "+v"(rb));
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int q = c + c_token(i, h);
            if (q < n) {
                float *yrow = Yz + (int64_t)(p0 + q) * d + rb;
                yrow[0] = acc[0][i];
                yrow[32] = acc[1][i];
            }
        }
        }
    }
}

// ---- Q8_0 on the matrix cores ---------------------------------------------
// Weights in the RPL64 Q8_0 layout (lcmoe_host.cpp repack_rpl64_q8): per
// 64-row tile and 256-column group, chunk 0 holds each row's eight f16
// block scales (16 bytes) and chunk 1 + j the row's columns 16j .. 16j+15.
// A Q8_0 block (32 columns) is exactly the K of one v_mfma_f32_16x16x32_f16:
// each block's product S_b = sum_k x_k q_k starts from zero and its scale is
// applied once, acc += d_b * S_b in f32 (dequantize_q8_0,
// rust/src/kernels/mod.rs:37-51: w = q * d).  B = q is exact in f16: the
// biased byte q ^ 0x80 under the 0x64 exponent byte is 1152 + q, and one
// packed add leaves q.  Activations enter as one f16 per element (the
// default mode).  A block is one wave of 32 rows (two 16-row tiles) of its
// MATS matrices and one 16-token pass: small layers (config 1: F = 2816,
// d = 1024) need the many blocks, and the wave stages its own tokens'
// activations, eight tokens at a time.
//
// H between the products: f16 pieces in the format of k_mfma_gateup, each
// token's 32-column block (one gate/up wave's rows, one down MFMA's K)
// scaled by 2^-e with e the smallest exponent that keeps the block's largest
// magnitude below 2^15, and e in a byte per token and block.  e = 0 for
// every block that f16 holds as it is (such blocks are the plain
// conversion); the down scales each block's product back by 2^e.  Q8_0
// weights up to the loader's |w| <= 100 can drive H past f16's range.
constexpr int kQ8Group = 17 * 1024;  // bytes per 64-row tile and group
constexpr int kQ8Tok = 16;
constexpr int kQ8Exp = kQ8Tok * kTokB<false>;  // 16 token rows of 528 bytes
constexpr int kQ8Stage = kQ8Exp + 8 * kQ8Tok * 4;  // then the scales 2^e, [block][token]
constexpr int kQ8Lds = 2 * kQ8Stage > 4 * chain_lds_floats(16, 128)
                           ? 2 * kQ8Stage : 4 * chain_lds_floats(16, 128);
__shared__ __attribute__((aligned(1024))) uint8_t s_q8[kQ8Lds];

// One matrix's NTL 16-row tiles for one group: lane (r16, c4) holds row r16
// of tile t's eight scales and, per block b, the row's columns 32b + 8c4 .. +7.
template <int NTL>
struct WQ8 {
    u32x4 d[NTL];
    u32x2 q[8][NTL];  // [block][tile]
};

// lo: this lane's row offset r16 * 16 from the wave's row base; tile 1 is
// the 16 rows after tile 0 (256 bytes further in every chunk)
__device__ __forceinline__ u32x4 load_q8d(g_u8 *base, uint32_t lo, int g, int t) {
    return gload<u32x4>(base + (lo + (uint32_t)(g * kQ8Group + 256 * t)));
}
__device__ __forceinline__ u32x2 load_q8q(g_u8 *base, uint32_t lo, int g, int b, int t, int c4) {
    return gload<u32x2>(base + (lo + (uint32_t)(g * kQ8Group + (1 + 2 * b + (c4 >> 1)) * 1024 +
                                                256 * t + 8 * (c4 & 1))));
}

// B operand of 8 quants in the activation format's column order
// (act16_pos: bytes 0, 2, 1, 3, 4, 6, 5, 7)
__device__ __forceinline__ half8 dec_q8(u32x2 q) {
    const uint32_t w0 = q.x ^ 0x80808080u, w1 = q.y ^ 0x80808080u;
    const half2v k = half2v{(_Float16)-1152.0f, (_Float16)-1152.0f};
    const half2v a = magic2(w0, kSel02) + k, b = magic2(w0, kSel13) + k;
    const half2v c = magic2(w1, kSel02) + k, e = magic2(w1, kSel13) + k;
    return half8{a[0], a[1], b[0], b[1], c[0], c[1], e[0], e[1]};
}

// Eight tokens' activations of one group (their f16 pieces' hi halves)
// through this wave's registers, and (down) lane i < 16's 8 block exponents
// of token i.
struct Q8Act {
    u32x2 tok[kQ8Tok / 2];
    u32x2 ex;
};

template <bool EXP>
__device__ __forceinline__ void q8_act_load(Q8Act &s, g_u8 *const (&tok)[kQ8Tok], g_u8 *exb,
                                            uint32_t exo, int g, int lane, int half) {
#pragma unroll
    for (int i = 0; i < kQ8Tok / 2; i++)
        s.tok[i] = gload<u32x2>(tok[kQ8Tok / 2 * half + i] + (uint32_t)(g * 1024 + 8 * lane));
    if (EXP && half == 0) s.ex = gload<u32x2>(exb + (exo + (uint32_t)(8 * g)));
}

template <bool EXP>
__device__ __forceinline__ void q8_act_store(uint8_t *stage, const Q8Act &s, int lane, int half) {
#pragma unroll
    for (int i = 0; i < kQ8Tok / 2; i++)
        *reinterpret_cast<u32x2 *>(stage + (kQ8Tok / 2 * half + i) * kTokB<false> + 8 * lane) =
            s.tok[i];
    if (EXP && half == 1 && lane < kQ8Tok) {
#pragma unroll
        for (int b = 0; b < 8; b++) {
            const int e = (int)(((b < 4 ? s.ex.x : s.ex.y) >> (8 * (b & 3))) & 0xff);
            *reinterpret_cast<float *>(stage + kQ8Exp + (b * kQ8Tok + lane) * 4) =
                __builtin_amdgcn_ldexpf(1.0f, e);
        }
    }
}

// One group: the blocks of `cur`'s activations against w; w reloaded with
// group gn block by block, and gn's activations staged into `nxt` in two
// halves.  MATS = 1 (down): each block's product scaled by 2^e of its token.
template <int MATS, int NTL>
__device__ __forceinline__ void q8_step(g_u8 *const (&wb)[MATS], uint32_t lo, int gn,
                                        const uint8_t *cur, uint8_t *nxt,
                                        g_u8 *const (&tok)[kQ8Tok], g_u8 *exb, uint32_t exo,
                                        WQ8<NTL> (&w)[MATS], float4v (&acc)[MATS][NTL], int lane) {
    constexpr bool EXP = MATS == 1;
    const int r16 = lane & 15, c4 = lane >> 4;
    Q8Act act;
    q8_act_load<EXP>(act, tok, exb, exo, gn, lane, 0);
    __builtin_amdgcn_sched_barrier(0);  // keep the activation loads first
    uint32_t dw[MATS][NTL][4];  // this group's scales; the next group's load in their place
#pragma unroll
    for (int m = 0; m < MATS; m++)
#pragma unroll
        for (int t = 0; t < NTL; t++) {
            const u32x4 v = w[m].d[t];
            dw[m][t][0] = v.x;
            dw[m][t][1] = v.y;
            dw[m][t][2] = v.z;
            dw[m][t][3] = v.w;
            w[m].d[t] = load_q8d(wb[m], lo, gn, t);
        }
    const uint8_t *tokrow = cur + r16 * kTokB<false>;
    half8 a[2];  // block b's activations, and b + 1's read ahead
    a[0] = *reinterpret_cast<const half8 *>(tokrow + 16 * c4);
#pragma unroll
    for (int b = 0; b < 8; b++) {
        if (b + 1 < 8)
            a[(b + 1) & 1] = *reinterpret_cast<const half8 *>(tokrow + 64 * (b + 1) + 16 * c4);
        float4v S[MATS][NTL];
#pragma unroll
        for (int m = 0; m < MATS; m++)
#pragma unroll
            for (int t = 0; t < NTL; t++) {
                const half8 bq = dec_q8(w[m].q[b][t]);
                w[m].q[b][t] = load_q8q(wb[m], lo, gn, b, t, c4);
                S[m][t] = mfma16(a[b & 1], bq, float4v{});
            }
        // down: the scales 2^e of this lane's result tokens 4 c4 + i for block
        // b (d_b 2^e is exact, so the fma rounds d_b S_b 2^e once, as before)
        float4v sc = float4v{1.0f, 1.0f, 1.0f, 1.0f};
        if constexpr (EXP)
            sc = *reinterpret_cast<const float4v *>(cur + kQ8Exp + (b * kQ8Tok + 4 * c4) * 4);
#pragma unroll
        for (int m = 0; m < MATS; m++)
#pragma unroll
            for (int t = 0; t < NTL; t++) {
                const float db = dh2f(dw[m][t][b >> 1] >> (16 * (b & 1)));
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float dbs = EXP ? db * sc[i] : db;
                    acc[m][t][i] = __builtin_fmaf(dbs, S[m][t][i], acc[m][t][i]);
                }
            }
        if (b == 3) {  // the first half of gn's activations to LDS, the second half in flight
            q8_act_store<EXP>(nxt, act, lane, 0);
            q8_act_load<EXP>(act, tok, exb, exo, gn, lane, 1);
        }
        __builtin_amdgcn_sched_barrier(0);  // bounds the live operands to one block
    }
    q8_act_store<EXP>(nxt, act, lane, 1);
    chain_detail::wave_lds_sync();
}

// grid (rows / (16 NTL) row groups, [chain row +] slots, token groups);
// block = one wave.  MATS = 2, NTL = 2: the gate/up products (w0 = gate, w1 = up, cols = d,
// rows = F) from the f16 pieces of x, with the SwiGLU into H (scaled f16
// pieces and their exponents, no sub-block sums); with ch.tiles, row 0 runs
// the exact router chains.  MATS = 1, NTL = 1: the down product (w0 = down, cols = F,
// rows = d) from H, grid z = K split + ksplit * token group, partial sums
// of split z into Y + z * split_stride.  Token group z takes the slot's
// 16-token passes z, z + groups, ...  hexp: one byte per position and
// 32-column block of H.
template <int MATS, int NTL>
__global__ __launch_bounds__(64, 2) void k_mfma_q8(
    const uint8_t *__restrict__ w0, const uint8_t *__restrict__ w1, int64_t estride,
    const _Float16 *__restrict__ act, uint8_t *__restrict__ hexp, SlotArgs sa, int cols, int rows,
    int ksplit, _Float16 *__restrict__ h16, float *__restrict__ Y, int64_t split_stride,
    ChainArgs ch) {
    int slot = blockIdx.y;
    if (MATS == 2 && ch.tiles) {
        if (slot == 0) {
            if (blockIdx.z) return;
            float *lds = reinterpret_cast<float *>(s_q8);
            for (int tile = blockIdx.x; tile < ch.tiles; tile += gridDim.x)
                chain_tile<8, 128, 1>(ch, tile, lds);
            return;
        }
        slot -= 1;
    }
    int e, p0, n;
    if (!slot_info(sa, slot, e, p0, n)) return;
    const int lane = threadIdx.x & 63, r16 = lane & 15, c4 = lane >> 4;
    const int rg = blockIdx.x, NG = cols >> 8;
    const int ks = MATS == 1 ? ksplit : 1;
    const int cz = blockIdx.z / ks, nz = gridDim.z / ks, bz = blockIdx.z - cz * ks;
    const int g0 = (int)((int64_t)NG * bz / ks), g1 = (int)((int64_t)NG * (bz + 1) / ks);
    constexpr int kPerTile = 4 / NTL;  // row groups per 64-row tile
    const int64_t rbase = (int64_t)e * estride + (int64_t)(rg / kPerTile) * NG * kQ8Group +
                          16 * NTL * (rg % kPerTile) * 16;
    g_u8 *wbm[MATS];
    wbm[0] = uniform(w0 + rbase);
    if constexpr (MATS == 2) wbm[1] = uniform(w1 + rbase);
    const uint32_t lo = r16 * 16;
    const uint8_t *ab = reinterpret_cast<const uint8_t *>(act);
    g_u8 *const exb = uniform(hexp);
    uint8_t *const st0 = s_q8, *const st1 = s_q8 + kQ8Stage;
    for (int c = cz * kQ8Tok; c < n; c += nz * kQ8Tok) {
        g_u8 *tok[kQ8Tok];
#pragma unroll
        for (int i = 0; i < kQ8Tok; i++) {
            const int q = min(c + i, n - 1);
            const int64_t row = MATS == 2 ? slot_token(sa, p0, q) : p0 + q;
            tok[i] = uniform(ab + row * (int64_t)cols * 4);
        }
        // down: lane i < 16's exponents row (token i of the pass)
        const uint32_t exo = MATS == 1 ? (uint32_t)(p0 + min(c + (lane & 15), n - 1)) * (cols >> 5) : 0;
        float4v acc[MATS][NTL];
#pragma unroll
        for (int m = 0; m < MATS; m++)
#pragma unroll
            for (int t = 0; t < NTL; t++) acc[m][t] = float4v{};
        WQ8<NTL> w[MATS];
        Q8Act a0;
        q8_act_load<MATS == 1>(a0, tok, exb, exo, g0, lane, 0);
#pragma unroll
        for (int m = 0; m < MATS; m++)
#pragma unroll
            for (int t = 0; t < NTL; t++) {
                w[m].d[t] = load_q8d(wbm[m], lo, g0, t);
#pragma unroll
                for (int b = 0; b < 8; b++) w[m].q[b][t] = load_q8q(wbm[m], lo, g0, b, t, c4);
            }
        q8_act_store<MATS == 1>(st0, a0, lane, 0);
        q8_act_load<MATS == 1>(a0, tok, exb, exo, g0, lane, 1);
        q8_act_store<MATS == 1>(st0, a0, lane, 1);
        chain_detail::wave_lds_sync();
        const int last = g1 - 1;
        int g = g0;
        for (; g + 2 <= g1; g += 2) {
            q8_step<MATS, NTL>(wbm, lo, g + 1, st0, st1, tok, exb, exo, w, acc, lane);
            q8_step<MATS, NTL>(wbm, lo, min(g + 2, last), st1, st0, tok, exb, exo, w, acc, lane);
        }
        if (g < g1) q8_step<MATS, NTL>(wbm, lo, g, st0, st1, tok, exb, exo, w, acc, lane);
        if constexpr (MATS == 2) {
            // SwiGLU; per token the 32 values of this wave (a block of H)
            // scaled into f16's range and written as pieces, the exponent
            // beside them
            const int F = rows, nkb = (F + 255) >> 8, neb = F >> 5;
            static_assert(MATS != 2 || NTL == 2, "a gate/up wave covers one H block");
            int fb = rg * 32 + r16;  // opaque: output addresses are formed here
            asm volatile("" : "+v"(fb));
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int q = c + 4 * c4 + i;
                float v[2];
#pragma unroll
                for (int t = 0; t < 2; t++) v[t] = silu(acc[0][t][i]) * acc[1][t][i];
                float mx = fmaxf(fabsf(v[0]), fabsf(v[1]));
#pragma unroll
                for (int off = 1; off < 16; off <<= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
                // mx >= 2^15: e = ilogb(mx) - 14 puts the block's largest below 2^15
                const int ex = mx >= 32768.0f ? (int)((__float_as_uint(mx) >> 23) & 0xff) - 141 : 0;
                if (q < n) {
                    const int64_t p = p0 + q;
#pragma unroll
                    for (int t = 0; t < 2; t++) {
                        const int ft = fb + 16 * t;
                        h16[(p * nkb + (ft >> 8)) * 512 + act16_pos(ft & 255)] =
                            (_Float16)__builtin_amdgcn_ldexpf(v[t], -ex);
                    }
                    if (r16 == 0) hexp[p * neb + rg] = (uint8_t)ex;
                }
            }
        } else {
            float *Yz = Y + (int64_t)bz * split_stride;
            int rb = rg * 16 * NTL + r16;  // opaque: output addresses are formed here
            asm volatile("" : "+v"(rb));
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int q = c + 4 * c4 + i;
                if (q < n) {
                    float *yrow = Yz + (int64_t)(p0 + q) * rows + rb;
#pragma unroll
                    for (int t = 0; t < NTL; t++) yrow[16 * t] = acc[0][t][i];
                }
            }
        }
    }
}

// x rows -> f16 hi/lo pieces (per super-block: hi[256] then lo[256]) and
// per-sub-block sums (hi, lo); one thread per 32-column sub-block
__global__ __launch_bounds__(256) void k_act16(const float *__restrict__ x, int T, int d,
                                               _Float16 *__restrict__ x16,
                                               _Float16 *__restrict__ xs, bool lo) {
    const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // sub-block index
    const int nsb = d >> 5;
    if (q >= (int64_t)T * nsb) return;
    act16_subblock(x + q * 32, q / nsb, d, (int)(q % nsb), x16, xs, lo);
}

SlotArgs dev_slots(const SlotArgsHost &s) {
    return SlotArgs{s.perm, s.counts, s.offsets, s.touched, s.E, s.K, s.T, s.shared, s.nr, s.S, s.sbase, s.ns, s.sl, s.pslots};
}

}  // namespace

hipError_t launch_mfma_down_q6(const uint8_t *down, int64_t estride, const _Float16 *h16,
                               const SlotArgsHost &sa, int slots, int chunks, int d, int F,
                               int ksplit, float *Y, int64_t split_stride, hipStream_t st,
                               bool h_lo, bool p16) {
    const int tiles = d / 64;
    if (chunks < 1 || ksplit < 1 || (int64_t)chunks * ksplit > 65535) return hipErrorInvalidValue;
    const dim3 grid((tiles + kWaves - 1) / kWaves, slots, ksplit * chunks);
    auto *kern = !h_lo ? k_mfma_down_q6<false, 0>
                       : p16 ? k_mfma_down_q6<true, 16> : k_mfma_down_q6<true, 32>;
    hipLaunchKernelGGL(kern, grid, dim3(256), 0, st, down, estride, h16, dev_slots(sa), d, F,
                       ksplit, Y, split_stride);
    return hipGetLastError();
}

hipError_t launch_act16(const float *x, int T, int d, _Float16 *x16, _Float16 *xs,
                        hipStream_t st, bool lo) {
    const int64_t n = (int64_t)T * (d / 32);
    hipLaunchKernelGGL(k_act16, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x, T, d, x16,
                       xs, lo);
    return hipGetLastError();
}

hipError_t launch_mfma_gateup(const uint8_t *gate, const uint8_t *up, int64_t estride,
                              const _Float16 *x16, const _Float16 *xs, const SlotArgsHost &sa,
                              int slots, int chunks, int d, int F, _Float16 *h16, _Float16 *hs,
                              float *hf, const ChainArgs &ch, hipStream_t st, bool x_lo) {
    const int groups = F / 32;
    ChainArgs c = ch;
    if (c.tiles) {
        if (c.k0 % 256 || c.k1 % 256) return hipErrorInvalidValue;
        c = with_nt(ch, 8);
    }
    if (chunks < 1 || chunks > 65535) return hipErrorInvalidValue;
    hipLaunchKernelGGL(x_lo ? k_mfma_gateup<true> : k_mfma_gateup<false>,
                       dim3((groups + kWaves - 1) / kWaves, slots + (c.tiles ? 1 : 0), chunks),
                       dim3(256), 0, st, gate, up, estride, x16, xs, dev_slots(sa), d, F, h16, hs,
                       hf, c);
    return hipGetLastError();
}

hipError_t launch_mfma_gateup_q8(const uint8_t *gate, const uint8_t *up, int64_t estride,
                                 const _Float16 *x16, const SlotArgsHost &sa, int slots,
                                 int groups, int d, int F, _Float16 *h16, uint8_t *hexp,
                                 const ChainArgs &ch, hipStream_t st) {
    if (F % 64 || d % 256 || groups < 1 || groups > 65535) return hipErrorInvalidValue;
    ChainArgs c = ch;
    if (c.tiles) {
        if (c.k0 % 128 || c.k1 % 128) return hipErrorInvalidValue;
        c = with_nt(ch, 8);
    }
    hipLaunchKernelGGL((k_mfma_q8<2, 2>), dim3(F / 32, slots + (c.tiles ? 1 : 0), groups), dim3(64), 0,
                       st, gate, up, estride, x16, hexp, dev_slots(sa), d, F, 1, h16, nullptr,
                       (int64_t)0, c);
    return hipGetLastError();
}

hipError_t launch_mfma_down_q8(const uint8_t *down, int64_t estride, const _Float16 *h16,
                               const uint8_t *hexp, const SlotArgsHost &sa, int slots, int groups,
                               int d, int F, int ksplit, float *Y, int64_t split_stride,
                               hipStream_t st) {
    if (d % 64 || F % 256 || ksplit < 1 || groups < 1 || (int64_t)groups * ksplit > 65535)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL((k_mfma_q8<1, 1>), dim3(d / 16, slots, groups * ksplit), dim3(64), 0, st, down,
                       nullptr, estride, h16, const_cast<uint8_t *>(hexp), dev_slots(sa), F, d,
                       ksplit, nullptr, Y, split_stride, ChainArgs{});
    return hipGetLastError();
}

hipError_t launch_mfma_down(const uint8_t *down, int64_t estride, const _Float16 *h16,
                            const _Float16 *hs, const SlotArgsHost &sa, int slots, int chunks,
                            int d, int F, int ksplit, float *Y, int64_t split_stride,
                            hipStream_t st, bool h_lo) {
    const int tiles = d / 64;
    if (chunks < 1 || ksplit < 1 || (int64_t)chunks * ksplit > 65535) return hipErrorInvalidValue;
    if (F % 128) return hipErrorInvalidValue;
    const dim3 grid((tiles + kWaves - 1) / kWaves, slots, ksplit * chunks);
    auto *kern = F % 256 ? (h_lo ? k_mfma_down<true, true> : k_mfma_down<true, false>)
                         : (h_lo ? k_mfma_down<false, true> : k_mfma_down<false, false>);
    hipLaunchKernelGGL(kern, grid, dim3(256), 0, st, down, estride, h16, hs, dev_slots(sa), d, F,
                       ksplit, Y, split_stride);
    return hipGetLastError();
}

}  // namespace lcmoe
