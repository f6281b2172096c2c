// Decode-regime expert products for Q4_K weights in the RPL64 layout.
//
// RPL64: a Q4_K matrix [rows, cols] is stored as 64-row tiles; inside a tile,
// for each 256-column super-block kb, its 144-byte blocks are split into nine
// 16-byte chunks and chunk c of the 64 rows is contiguous (1 KB):
//   byte offset = ((tile * NB + kb) * 9 + c) * 1024 + row_in_tile * 16.
// A wave owns one tile, one lane one row, so each 16-byte load instruction
// moves 1 KB of contiguous HBM.  The byte count equals the GGUF tensor's.
//
// Activations arrive as two int8 limbs per 32-element sub-block
// (v ~= s * (128*hi + lo), exact to 1/32512 of the sub-block's max|v|), with
// s and s*sum(128*hi+lo) per sub-block.  They are wave-uniform (every lane of
// the wave needs the same token and columns), so they are scalar loads and
// v_dot4 takes them as its SGPR operand.  With q the 4-bit quants of a
// sub-block j of a row, d*sc_j and dmin*m_j its scale and min:
//   sum_k w_k v_k = (d*sc_j) * s * sum_k q_k (128*hi_k + lo_k) - (dmin*m_j) * s*sum(...)
// The integer part is exact (|.| < 2^24); only the last two products round.
//
// The four waves of a block split the super-blocks of the row; their partial
// sums meet in LDS in a fixed order, so results are deterministic.

#include "device_common.h"
#include "kernels.h"

namespace lcmoe {
namespace {

constexpr int kWaves = 4;

// (d2, dmin2) scale sub-blocks 4-7: the split layout's second half block
// (lcmoe_host.cpp repack_rpl64_q4k_split); the header's own pair otherwise
__device__ __forceinline__ void unpack_hdr(uint4 h, float (&dl)[8], float (&ml)[8],
                                           const uint32_t *db = nullptr) {
    const float d = dh2f(h.x & 0xffff), dmin = dh2f(h.x >> 16);
    const float d2 = db ? dh2f(*db & 0xffff) : d, dmin2 = db ? dh2f(*db >> 16) : dmin;
    // get_scale_min_k4 (rust/src/kernels/mod.rs:54-63) for all 8 sub-blocks
    const uint32_t sc03 = h.y & 0x3F3F3F3Fu, m03 = h.z & 0x3F3F3F3Fu;
    const uint32_t sc47 = (h.w & 0x0F0F0F0Fu) | ((h.y >> 2) & 0x30303030u);
    const uint32_t m47 = ((h.w >> 4) & 0x0F0F0F0Fu) | ((h.z >> 2) & 0x30303030u);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        dl[i] = d * (float)((sc03 >> (8 * i)) & 0xffu);
        dl[4 + i] = d2 * (float)((sc47 >> (8 * i)) & 0xffu);
        ml[i] = dmin * (float)((m03 >> (8 * i)) & 0xffu);
        ml[4 + i] = dmin2 * (float)((m47 >> (8 * i)) & 0xffu);
    }
}

// One 256-element super-block of this lane's row against NT token rows.
// xh/xl point at the tokens' limbs for this super-block (as ints), xs/xm at
// their 8 sub-block scales / quantised sums.
// With db (split layout), sub-blocks 4-7 take the second (d, dmin); with
// first_half, only sub-blocks 0-3 exist (the last block of a row whose length
// is an odd multiple of 128: the rest lies past the row).
template <int NT>
__device__ __forceinline__ void q4_block_dot(const uint4 (&c)[9], const int *const (&xh)[NT],
                                             const int *const (&xl)[NT],
                                             const float *const (&xs)[NT],
                                             const float *const (&xm)[NT], float (&acc)[NT],
                                             const uint32_t *db = nullptr,
                                             bool first_half = false) {
    float dl[8], ml[8];
    unpack_hdr(c[0], dl, ml, db);
#pragma unroll
    for (int j = 0; j < 4; j++) {
        if (j >= 2 && first_half) break;
        const uint4 a = c[1 + 2 * j], b = c[2 + 2 * j];
        const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        int lo[8], hi[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            lo[i] = (int)(w[i] & 0x0F0F0F0Fu);
            hi[i] = (int)((w[i] >> 4) & 0x0F0F0F0Fu);
        }
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const int *ph = xh[t] + 16 * j, *pl = xl[t] + 16 * j;
            int sh0 = 0, sl0 = 0, sh1 = 0, sl1 = 0;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                sh0 = __builtin_amdgcn_sdot4(lo[i], ph[i], sh0, false);
                sl0 = __builtin_amdgcn_sdot4(lo[i], pl[i], sl0, false);
                sh1 = __builtin_amdgcn_sdot4(hi[i], ph[8 + i], sh1, false);
                sl1 = __builtin_amdgcn_sdot4(hi[i], pl[8 + i], sl1, false);
            }
            const float f0 = (float)(sh0 * 128 + sl0), f1 = (float)(sh1 * 128 + sl1);
            acc[t] = __builtin_fmaf(dl[2 * j] * xs[t][2 * j], f0, acc[t]);
            acc[t] = __builtin_fmaf(-ml[2 * j], xm[t][2 * j], acc[t]);
            acc[t] = __builtin_fmaf(dl[2 * j + 1] * xs[t][2 * j + 1], f1, acc[t]);
            acc[t] = __builtin_fmaf(-ml[2 * j + 1], xm[t][2 * j + 1], acc[t]);
        }
    }
}

struct Limbs {
    const int8_t *h, *l;
    const float *s, *m;
    int len;  // row length (elements) of the limb arrays
};

template <int NT>
__device__ __forceinline__ void token_ptrs(const Limbs &X, const int (&row)[NT], int kb,
                                           const int *(&xh)[NT], const int *(&xl)[NT],
                                           const float *(&xs)[NT], const float *(&xm)[NT]) {
    const int nsb = X.len >> 5;
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const int64_t off = (int64_t)row[t] * X.len + 256 * kb;
        xh[t] = reinterpret_cast<const int *>(X.h + off);
        xl[t] = reinterpret_cast<const int *>(X.l + off);
        xs[t] = X.s + (int64_t)row[t] * nsb + 8 * kb;
        xm[t] = X.m + (int64_t)row[t] * nsb + 8 * kb;
    }
}

// gate and up rows of this lane over super-blocks [kb0, kb1).
template <int NT>
__device__ __forceinline__ void pass2(const uint4 *__restrict__ G, const uint4 *__restrict__ U,
                                      int kb0, int kb1, const Limbs &X, const int (&row)[NT],
                                      float (&ag)[NT], float (&au)[NT]) {
    for (int kb = kb0; kb < kb1; kb++) {
        uint4 cg[9], cu[9];
        const uint4 *pg = G + (int64_t)kb * 9 * 64, *pu = U + (int64_t)kb * 9 * 64;
#pragma unroll
        for (int i = 0; i < 9; i++) {
            cg[i] = pg[i * 64];
            cu[i] = pu[i * 64];
        }
        const int *xh[NT], *xl[NT];
        const float *xs[NT], *xm[NT];
        token_ptrs<NT>(X, row, kb, xh, xl, xs, xm);
        q4_block_dot<NT>(cg, xh, xl, xs, xm, ag);
        q4_block_dot<NT>(cu, xh, xl, xs, xm, au);
    }
}

// this lane's 9 chunks of super-block kb
__device__ __forceinline__ void load_chunks(uint4 (&c)[9], const uint4 *W, int kb) {
    const uint4 *p = W + (int64_t)kb * 9 * 64;
#pragma unroll
    for (int i = 0; i < 9; i++) c[i] = p[i * 64];
}

template <int NT>
__device__ __forceinline__ void dot_sb(const uint4 (&c)[9], int kb, const Limbs &X,
                                       const int (&row)[NT], float (&acc)[NT]) {
    const int *xh[NT], *xl[NT];
    const float *xs[NT], *xm[NT];
    token_ptrs<NT>(X, row, kb, xh, xl, xs, xm);
    q4_block_dot<NT>(c, xh, xl, xs, xm, acc);
}

// Rows of this lane over super-blocks [kb0, kb1), the next super-block's
// chunks loaded while the current one is computed (two register sets; the
// loads complete in issue order, so waiting for the current set leaves the
// next one in flight).
template <int NT>
__device__ __forceinline__ void pass1(const uint4 *__restrict__ W, int kb0, int kb1,
                                      const Limbs &X, const int (&row)[NT], float (&acc)[NT]) {
    if (kb0 >= kb1) return;
    uint4 c0[9], c1[9];
    load_chunks(c0, W, kb0);
    int kb = kb0;
    for (; kb + 2 <= kb1; kb += 2) {
        load_chunks(c1, W, kb + 1);
        dot_sb<NT>(c0, kb, X, row, acc);
        load_chunks(c0, W, min(kb + 2, kb1 - 1));
        dot_sb<NT>(c1, kb + 1, X, row, acc);
    }
    if (kb < kb1) dot_sb<NT>(c0, kb, X, row, acc);
}

// ---- Q4_K down in the split layout ----------------------------------------
// Rows whose length F is an odd multiple of 128 (repack_rpl64_q4k_split): per
// 64-row tile and virtual super-block (256 of the row's own columns), the
// nine 1 KiB chunks of the RPL64 layout, then the 64 rows' second (d, dmin)
// for sub-blocks 4-7: 592 uint4.  The last virtual block of a row holds only
// sub-blocks 0-3 (the rest would lie past F and is never read, neither are
// the activations there).
constexpr int kSplitUint4 = (9 * 1024 + 256) / 16;

__device__ __forceinline__ void load_split(uint4 (&c)[9], uint32_t &db, const uint4 *W, int kb,
                                           int lane) {
    const uint4 *p = W + (int64_t)kb * kSplitUint4;
#pragma unroll
    for (int i = 0; i < 9; i++) c[i] = p[i * 64];
    db = reinterpret_cast<const uint32_t *>(p - lane + 9 * 64)[lane];
}

template <int NT>
__device__ __forceinline__ void pass1_split(const uint4 *__restrict__ W, int kb0, int kb1, int nkb,
                                            bool half_last, const Limbs &X, const int (&row)[NT],
                                            float (&acc)[NT]) {
    if (kb0 >= kb1) return;
    const int lane = threadIdx.x & 63;
    uint4 c0[9], c1[9];
    uint32_t d0, d1;
    load_split(c0, d0, W, kb0, lane);
    auto dot = [&](const uint4 (&c)[9], const uint32_t &db, int kb) {
        const int *xh[NT], *xl[NT];
        const float *xs[NT], *xm[NT];
        token_ptrs<NT>(X, row, kb, xh, xl, xs, xm);
        q4_block_dot<NT>(c, xh, xl, xs, xm, acc, &db, half_last && kb == nkb - 1);
    };
    int kb = kb0;
    for (; kb + 2 <= kb1; kb += 2) {
        load_split(c1, d1, W, kb + 1, lane);
        dot(c0, d0, kb);
        load_split(c0, d0, W, min(kb + 2, kb1 - 1), lane);
        dot(c1, d1, kb + 1);
    }
    if (kb < kb1) dot(c0, d0, kb);
}

// ---- Q6_K down in the RPL64 Q6_K layout -----------------------------------
// Per 64-row tile and super-block: thirteen chunks of 64 rows x 16 bytes (ql
// in 0-7, qh in 8-11, the 16 int8 scales in 12), then the rows' f16 d; 840
// uint4 in all.  Element 128n + 32j + l (l < 32) of a row's block has the
// code q = (ql nibble) | (qh bits 2j, 2j+1) << 4 with the nibble the low (j
// < 2) or high half of ql[64n + 32(j & 1) + l] and the qh byte qh[32n + l],
// and the value d * sc[8n + 2j + l/16] * (q - 32) (dequantize_q6_k,
// rust/src/kernels/mod.rs:145-180).  Per 16-element scale group the integer
// sum sc * sum (q - 32) (128 hi + lo) is exact in int32 (|.| <= 2^30.99 for a
// 32-element sub-block).
constexpr int kQ6Uint4 = (13 * 1024 + 128) / 16;

struct Q6Regs {
    uint4 c[13];
    uint32_t d;
};

__device__ __forceinline__ void load_q6(Q6Regs &w, const uint4 *W, const uint16_t *D, int kb) {
    const uint4 *p = W + (int64_t)kb * kQ6Uint4;
#pragma unroll
    for (int i = 0; i < 13; i++) w.c[i] = p[i * 64];
    w.d = D[(int64_t)kb * (kQ6Uint4 * 8)];
}

// q - 32 of four 6-bit codes (one per byte) as signed bytes
__device__ __forceinline__ int q6_signed(uint32_t q) {
    const uint32_t v = q ^ 0x20202020u, b = v & 0x20202020u;
    return (int)(v | (b << 1) | (b << 2));
}

template <int NT>
__device__ __forceinline__ void q6_block_dot(const Q6Regs &w, const int *const (&xh)[NT],
                                             const int *const (&xl)[NT],
                                             const float *const (&xs)[NT], float (&acc)[NT]) {
    const float d = dh2f(w.d & 0xffff);
    const uint32_t scw[4] = {w.c[12].x, w.c[12].y, w.c[12].z, w.c[12].w};
#pragma unroll
    for (int n = 0; n < 2; n++) {
        const uint4 ha = w.c[8 + 2 * n], hb = w.c[9 + 2 * n];
        const uint32_t qh[8] = {ha.x, ha.y, ha.z, ha.w, hb.x, hb.y, hb.z, hb.w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint4 qa = w.c[4 * n + 2 * (j & 1)], qb = w.c[4 * n + 2 * (j & 1) + 1];
            const uint32_t ql[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
            int sq[8];
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const uint32_t nib = j < 2 ? ql[i] & 0x0F0F0F0Fu : (ql[i] >> 4) & 0x0F0F0F0Fu;
                const uint32_t hi2 = ((qh[i] >> (2 * j)) & 0x03030303u) << 4;
                sq[i] = q6_signed(nib | hi2);
            }
            const int sb = 4 * n + j, k0 = 8 * n + 2 * j;
            const int s0 = (int)(int8_t)(scw[k0 >> 2] >> (8 * (k0 & 3)));
            const int s1 = (int)(int8_t)(scw[(k0 + 1) >> 2] >> (8 * ((k0 + 1) & 3)));
#pragma unroll
            for (int t = 0; t < NT; t++) {
                const int *ph = xh[t] + 8 * sb, *pl = xl[t] + 8 * sb;
                int h0 = 0, l0 = 0, h1 = 0, l1 = 0;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    h0 = __builtin_amdgcn_sdot4(sq[i], ph[i], h0, false);
                    l0 = __builtin_amdgcn_sdot4(sq[i], pl[i], l0, false);
                    h1 = __builtin_amdgcn_sdot4(sq[4 + i], ph[4 + i], h1, false);
                    l1 = __builtin_amdgcn_sdot4(sq[4 + i], pl[4 + i], l1, false);
                }
                const int isb = (h0 * 128 + l0) * s0 + (h1 * 128 + l1) * s1;
                acc[t] = __builtin_fmaf(d * xs[t][sb], (float)isb, acc[t]);
            }
        }
    }
}

template <int NT>
__device__ __forceinline__ void dot_sb_q6(const Q6Regs &w, int kb, const Limbs &X,
                                          const int (&row)[NT], float (&acc)[NT]) {
    const int *xh[NT], *xl[NT];
    const float *xs[NT], *xm[NT];
    token_ptrs<NT>(X, row, kb, xh, xl, xs, xm);
    q6_block_dot<NT>(w, xh, xl, xs, acc);
}

// pass1() for Q6_K: two register sets, the next super-block loading while
// the current one is computed
template <int NT>
__device__ __forceinline__ void pass1_q6(const uint4 *__restrict__ W, const uint16_t *D, int kb0,
                                         int kb1, const Limbs &X, const int (&row)[NT],
                                         float (&acc)[NT]) {
    if (kb0 >= kb1) return;
    Q6Regs c0, c1;
    load_q6(c0, W, D, kb0);
    int kb = kb0;
    for (; kb + 2 <= kb1; kb += 2) {
        load_q6(c1, W, D, kb + 1);
        dot_sb_q6<NT>(c0, kb, X, row, acc);
        load_q6(c0, W, D, min(kb + 2, kb1 - 1));
        dot_sb_q6<NT>(c1, kb + 1, X, row, acc);
    }
    if (kb < kb1) dot_sb_q6<NT>(c0, kb, X, row, acc);
}

// ---- Q8_0 in the RPL64 Q8_0 layout ----------------------------------------
// Per 64-row tile and 256-column group (eight Q8_0 blocks of 32): chunk 0
// holds each row's eight f16 d (16 bytes), chunks 1-16 its 256 int8 quants
// in column order, 16 bytes per chunk: 1,088 uint4 per tile and group, the
// GGUF bytes permuted.  A Q8_0 block is one 32-column activation sub-block,
// so sum_k q_k (128 hi_k + lo_k) is one exact int32 per block and token
// (|.| <= 32 * 127 * 16256): value d * s * that (dequantize_q8_0,
// rust/src/kernels/mod.rs:37-51, times the activation limbs).
constexpr int kQ8Chunks = 17;

template <int NT>
__device__ __forceinline__ void q8_block_dot(const uint4 (&c)[kQ8Chunks], const int *const (&xh)[NT],
                                             const int *const (&xl)[NT],
                                             const float *const (&xs)[NT], float (&acc)[NT]) {
    const uint32_t dw[4] = {c[0].x, c[0].y, c[0].z, c[0].w};
#pragma unroll
    for (int b = 0; b < 8; b++) {
        const float d = dh2f((dw[b >> 1] >> (16 * (b & 1))) & 0xffff);
        const uint4 qa = c[1 + 2 * b], qb = c[2 + 2 * b];
        const int q[8] = {(int)qa.x, (int)qa.y, (int)qa.z, (int)qa.w,
                          (int)qb.x, (int)qb.y, (int)qb.z, (int)qb.w};
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const int *ph = xh[t] + 8 * b, *pl = xl[t] + 8 * b;
            int h = 0, l = 0;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                h = __builtin_amdgcn_sdot4(q[i], ph[i], h, false);
                l = __builtin_amdgcn_sdot4(q[i], pl[i], l, false);
            }
            acc[t] = __builtin_fmaf(d * xs[t][b], (float)(h * 128 + l), acc[t]);
        }
    }
}

__device__ __forceinline__ void load_q8(uint4 (&c)[kQ8Chunks], const uint4 *W, int kb) {
    const uint4 *p = W + (int64_t)kb * kQ8Chunks * 64;
#pragma unroll
    for (int i = 0; i < kQ8Chunks; i++) c[i] = p[i * 64];
}

template <int NT>
__device__ __forceinline__ void dot_sb_q8(const uint4 (&c)[kQ8Chunks], int kb, const Limbs &X,
                                          const int (&row)[NT], float (&acc)[NT]) {
    const int *xh[NT], *xl[NT];
    const float *xs[NT], *xm[NT];
    token_ptrs<NT>(X, row, kb, xh, xl, xs, xm);
    q8_block_dot<NT>(c, xh, xl, xs, acc);
}

template <int NT>
__device__ __forceinline__ void pass1_q8(const uint4 *__restrict__ W, int kb0, int kb1,
                                         const Limbs &X, const int (&row)[NT], float (&acc)[NT]) {
    if (kb0 >= kb1) return;
    uint4 c0[kQ8Chunks], c1[kQ8Chunks];
    load_q8(c0, W, kb0);
    int kb = kb0;
    for (; kb + 2 <= kb1; kb += 2) {
        load_q8(c1, W, kb + 1);
        dot_sb_q8<NT>(c0, kb, X, row, acc);
        load_q8(c0, W, min(kb + 2, kb1 - 1));
        dot_sb_q8<NT>(c1, kb + 1, X, row, acc);
    }
    if (kb < kb1) dot_sb_q8<NT>(c0, kb, X, row, acc);
}

// gate and up rows of this lane, Q8_0
template <int NT>
__device__ __forceinline__ void pass2_q8(const uint4 *__restrict__ G, const uint4 *__restrict__ U,
                                         int kb0, int kb1, const Limbs &X, const int (&row)[NT],
                                         float (&ag)[NT], float (&au)[NT]) {
    for (int kb = kb0; kb < kb1; kb++) {
        uint4 cg[kQ8Chunks], cu[kQ8Chunks];
        load_q8(cg, G, kb);
        load_q8(cu, U, kb);
        dot_sb_q8<NT>(cg, kb, X, row, ag);
        dot_sb_q8<NT>(cu, kb, X, row, au);
    }
}

struct HOut {
    float *f;       // H f32 [positions, F] or null
    int8_t *h, *l;  // H limbs [positions, F] or null
    float *s, *m;   // [positions, F/32]
    // H as f16 hi/lo pieces [positions][F/256][hi 256 | lo 256] and 32-row
    // sums (hi, lo) [positions][F/32][2] for the matrix-core down, or null
    _Float16 *h16, *hs16;
};

// Tokens per pass.  This path runs when experts average fewer than two
// tokens (the matrix-core kernels take larger batches), so passes of at most
// four keep the tokens' limbs within the scalar register file; an expert
// with more tokens takes several passes.
constexpr int kMaxNT = 4;

// Token rows c .. c+NT-1 of one gate/up tile (rows past n repeat the last
// token and are not written): the 4 waves' partial sums meet in LDS, then
// wave w finishes token w (SwiGLU, H out).
template <int NT, bool Q8>
__device__ __forceinline__ void gateup_chunk(const uint4 *G, const uint4 *U, int kb0, int kb1,
                                             const Limbs &X, const SlotArgs &sa, int p0, int n,
                                             int c, int F, int f, const HOut &out,
                                             float (*s_red)[2][kMaxNT][64]) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    int row[NT];
#pragma unroll
    for (int t = 0; t < NT; t++)
        row[t] = __builtin_amdgcn_readfirstlane(slot_token(sa, p0, min(c + t, n - 1)));
    float ag[NT], au[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) ag[t] = au[t] = 0.0f;
    if constexpr (Q8)
        pass2_q8<NT>(G, U, kb0, kb1, X, row, ag, au);
    else
        pass2<NT>(G, U, kb0, kb1, X, row, ag, au);
#pragma unroll
    for (int t = 0; t < NT; t++) {
        s_red[wave][0][t][lane] = ag[t];
        s_red[wave][1][t][lane] = au[t];
    }
    __syncthreads();
    for (int t = wave; t < NT && c + t < n; t += kWaves) {
        float g = s_red[0][0][t][lane], u = s_red[0][1][t][lane];
#pragma unroll
        for (int w = 1; w < kWaves; w++) {
            g = g + s_red[w][0][t][lane];
            u = u + s_red[w][1][t][lane];
        }
        const float h = silu(g) * u;
        const int64_t p = p0 + c + t;
        if (out.f) out.f[p * F + f] = h;
        if (out.h) {
            int hi, lo;
            float s, sum;
            quant2_half(h, hi, lo, s, sum);
            out.h[p * F + f] = (int8_t)hi;
            out.l[p * F + f] = (int8_t)lo;
            if ((lane & 31) == 0) {
                out.s[p * (F >> 5) + (f >> 5)] = s;
                out.m[p * (F >> 5) + (f >> 5)] = sum;
            }
        }
        if (out.h16) {  // rows of ceil(F / 256) pieces, 8 sums per piece
            const int nkb = (F + 255) >> 8;
            const _Float16 hi = (_Float16)h, lo = (_Float16)(h - (float)hi);
            float part = (float)hi + (float)lo;
#pragma unroll
            for (int off = 1; off < 32; off <<= 1) part += __shfl_xor(part, off, 64);
            _Float16 *piece = out.h16 + (p * nkb + (f >> 8)) * 512 + act16_pos(f & 255);
            piece[0] = hi;
            piece[256] = lo;
            if ((lane & 31) == 0) {
                const _Float16 shi = (_Float16)part, slo = (_Float16)(part - (float)shi);
                out.hs16[(p * nkb * 8 + (f >> 5)) * 2] = shi;
                out.hs16[(p * nkb * 8 + (f >> 5)) * 2 + 1] = slo;
            }
        }
    }
    __syncthreads();
}

// Chain tiles of one wave (wave 0 of each chain block): one-token tiles run
// two chunks of loads ahead, the shortest chains (T = 1) being the ones that
// must finish inside the shortest gate/up launch.
__device__ __forceinline__ void run_chains(const ChainArgs &ch, float *lds) {
    static_assert(chain_lds_floats(9, 256) >= chain_lds_floats(16, 128), "chain LDS");
    for (int tile = blockIdx.x; tile < ch.tiles; tile += gridDim.x) {
        if (ch.nt == 1)
            chain_tile<1, 256, 1>(ch, tile, lds);
        else
            chain_tile<8, 128, 1>(ch, tile, lds);
    }
}

// grid (F/64 row tiles, [chain row +] slots); Q8: RPL64 Q8_0 weights
template <bool Q8>
__global__ __launch_bounds__(256) void k_rpl_gateup(
    const uint8_t *__restrict__ gate, const uint8_t *__restrict__ up, int64_t estride,
    const int8_t *__restrict__ xh, const int8_t *__restrict__ xl, const float *__restrict__ xs,
    const float *__restrict__ xm, SlotArgs sa, int d, int F, float *__restrict__ hf,
    int8_t *__restrict__ hh, int8_t *__restrict__ hl, float *__restrict__ hs,
    float *__restrict__ hm, _Float16 *__restrict__ h16, _Float16 *__restrict__ hs16,
    ChainArgs ch) {
    int slot = blockIdx.y;
    if (ch.tiles) {  // row y = 0: exact router chains, one wave per block
        if (slot == 0) {
            __shared__ __attribute__((aligned(16))) float s_chain[chain_lds_floats(9, 256)];
            if (threadIdx.x < 64) run_chains(ch, s_chain);
            return;
        }
        slot -= 1;
    }
    const Limbs X{xh, xl, xs, xm, d};
    const HOut out{hf, hh, hl, hs, hm, h16, hs16};
    int e, p0, n;
    if (!slot_info(sa, slot, e, p0, n)) return;
    e = __builtin_amdgcn_readfirstlane(e);
    p0 = __builtin_amdgcn_readfirstlane(p0);
    n = __builtin_amdgcn_readfirstlane(n);
    __shared__ float s_red[kWaves][2][kMaxNT][64];
    // wave index made provably uniform so block indices and x addresses stay scalar
    const int NB = d >> 8, rt = blockIdx.x, lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int kb0 = NB * wave / kWaves, kb1 = NB * (wave + 1) / kWaves;
    const int64_t tile = (int64_t)rt * NB * (Q8 ? kQ8Chunks : 9) * 64 + lane;
    const uint4 *G = reinterpret_cast<const uint4 *>(gate + (int64_t)e * estride) + tile;
    const uint4 *U = reinterpret_cast<const uint4 *>(up + (int64_t)e * estride) + tile;
    const int f = rt * 64 + lane;
    for (int c = 0; c < n; c += kMaxNT) {
        const int left = n - c;
        if (left > 2)
            gateup_chunk<4, Q8>(G, U, kb0, kb1, X, sa, p0, n, c, F, f, out, s_red);
        else if (left == 2)
            gateup_chunk<2, Q8>(G, U, kb0, kb1, X, sa, p0, n, c, F, f, out, s_red);
        else
            gateup_chunk<1, Q8>(G, U, kb0, kb1, X, sa, p0, n, c, F, f, out, s_red);
    }
}

// weight format: 0 Q4_K, 1 Q6_K (D: the rows' d), 2 Q8_0
template <int NT, int FMT>
__device__ __forceinline__ void down_chunk(const uint4 *W, const uint16_t *D, int kb0, int kb1,
                                           const Limbs &X, int p0, int n, int c, int d, int r,
                                           float *Y, float (*s_red)[kMaxNT][64]) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    int row[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) row[t] = __builtin_amdgcn_readfirstlane(p0 + min(c + t, n - 1));
    float acc[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) acc[t] = 0.0f;
    if constexpr (FMT == 1)
        pass1_q6<NT>(W, D, kb0, kb1, X, row, acc);
    else if constexpr (FMT == 2)
        pass1_q8<NT>(W, kb0, kb1, X, row, acc);
    else if constexpr (FMT == 3)
        pass1_split<NT>(W, kb0, kb1, (X.len + 255) >> 8, (X.len & 255) != 0, X, row, acc);
    else
        pass1<NT>(W, kb0, kb1, X, row, acc);
#pragma unroll
    for (int t = 0; t < NT; t++) s_red[wave][t][lane] = acc[t];
    __syncthreads();
    for (int t = wave; t < NT && c + t < n; t += kWaves) {
        float v = s_red[0][t][lane];
#pragma unroll
        for (int w = 1; w < kWaves; w++) v = v + s_red[w][t][lane];
        Y[(int64_t)(p0 + c + t) * d + r] = v;
    }
    __syncthreads();
}

// grid (d/64 tiles, slots, ksplit): block z covers super-block slices
// 4z .. 4z+3 of the 4*ksplit slices of the F dimension; its partial row sums
// go to Y + z * split_stride and the combine adds the splits in order.
// FMT: RPL64 Q4_K (576 uint4 per tile and super-block), Q6_K (840), Q8_0
// (1,088) or split Q4_K (592 per tile and virtual super-block)
template <int FMT>
__global__ __launch_bounds__(256) void k_rpl_down(
    const uint8_t *__restrict__ down, int64_t estride, const int8_t *__restrict__ xh,
    const int8_t *__restrict__ xl, const float *__restrict__ xs, const float *__restrict__ xm,
    SlotArgs sa, int d, int F, float *__restrict__ Y, int64_t split_stride) {
    const Limbs X{xh, xl, xs, xm, F};
    int e, p0, n;
    if (!slot_info(sa, blockIdx.y, e, p0, n)) return;
    e = __builtin_amdgcn_readfirstlane(e);
    p0 = __builtin_amdgcn_readfirstlane(p0);
    n = __builtin_amdgcn_readfirstlane(n);
    __shared__ float s_red[kWaves][kMaxNT][64];
    const int NB = FMT == 3 ? (F + 255) >> 8 : F >> 8, rt = blockIdx.x, lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int slices = kWaves * gridDim.z, s = blockIdx.z * kWaves + wave;
    const int kb0 = (int)((int64_t)NB * s / slices), kb1 = (int)((int64_t)NB * (s + 1) / slices);
    const int tsb = FMT == 1 ? kQ6Uint4 : FMT == 2 ? kQ8Chunks * 64 : FMT == 3 ? kSplitUint4 : 9 * 64;
    const uint4 *T = reinterpret_cast<const uint4 *>(down + (int64_t)e * estride) +
                     (int64_t)rt * NB * tsb;
    const uint4 *W = T + lane;
    const uint16_t *D = reinterpret_cast<const uint16_t *>(T + 13 * 64) + lane;
    float *Yz = Y + (int64_t)blockIdx.z * split_stride;
    const int r = rt * 64 + lane;
    for (int c = 0; c < n; c += kMaxNT) {
        const int left = n - c;
        if (left > 2)
            down_chunk<4, FMT>(W, D, kb0, kb1, X, p0, n, c, d, r, Yz, s_red);
        else if (left == 2)
            down_chunk<2, FMT>(W, D, kb0, kb1, X, p0, n, c, d, r, Yz, s_red);
        else
            down_chunk<1, FMT>(W, D, kb0, kb1, X, p0, n, c, d, r, Yz, s_red);
    }
}

}  // namespace

hipError_t launch_rpl_gateup(const uint8_t *gate, const uint8_t *up, int64_t estride,
                             const int8_t *xh, const int8_t *xl, const float *xs, const float *xm,
                             const SlotArgsHost &sa, int slots, int d, int F, float *Hf, int8_t *hh,
                             int8_t *hl, float *hs, float *hm, _Float16 *h16, _Float16 *hs16,
                             const ChainArgs &ch, hipStream_t st, bool q8) {
    SlotArgs s{sa.perm, sa.counts, sa.offsets, sa.touched, sa.E, sa.K, sa.T, sa.shared, sa.nr, sa.S, sa.sbase, sa.ns, sa.sl, sa.pslots};
    ChainArgs c = ch;
    if (c.tiles) {
        if (c.k0 % 256 || c.k1 % 256) return hipErrorInvalidValue;
        c = with_nt(ch, ch.T == 1 ? 1 : 8);
    }
    const dim3 grid(F / 64, slots + (c.tiles ? 1 : 0));
    if (q8)
        hipLaunchKernelGGL(k_rpl_gateup<true>, grid, dim3(256), 0, st, gate, up, estride, xh, xl,
                           xs, xm, s, d, F, Hf, hh, hl, hs, hm, h16, hs16, c);
    else
        hipLaunchKernelGGL(k_rpl_gateup<false>, grid, dim3(256), 0, st, gate, up, estride, xh, xl,
                           xs, xm, s, d, F, Hf, hh, hl, hs, hm, h16, hs16, c);
    return hipGetLastError();
}

hipError_t launch_rpl_down(const uint8_t *down, int64_t estride, const int8_t *hh,
                           const int8_t *hl, const float *hs, const float *hm,
                           const SlotArgsHost &sa, int slots, int d, int F, int ksplit, float *Y,
                           int64_t split_stride, hipStream_t st, int fmt) {
    SlotArgs s{sa.perm, sa.counts, sa.offsets, sa.touched, sa.E, sa.K, sa.T, sa.shared, sa.nr, sa.S, sa.sbase, sa.ns, sa.sl, sa.pslots};
    const dim3 grid(d / 64, slots, ksplit);
    if (fmt == 1)
        hipLaunchKernelGGL(k_rpl_down<1>, grid, dim3(256), 0, st, down, estride, hh, hl, hs, hm, s,
                           d, F, Y, split_stride);
    else if (fmt == 2)
        hipLaunchKernelGGL(k_rpl_down<2>, grid, dim3(256), 0, st, down, estride, hh, hl, hs, hm, s,
                           d, F, Y, split_stride);
    else if (fmt == 3)
        hipLaunchKernelGGL(k_rpl_down<3>, grid, dim3(256), 0, st, down, estride, hh, hl, hs, hm, s,
                           d, F, Y, split_stride);
    else
        hipLaunchKernelGGL(k_rpl_down<0>, grid, dim3(256), 0, st, down, estride, hh, hl, hs, hm, s,
                           d, F, Y, split_stride);
    return hipGetLastError();
}

}  // namespace lcmoe
