// Decoder-layer kernels around the MoE FFN for the end-to-end engine
// (lcmoe_model_*): the parts of rust/src/inference/engine.rs:78-132 that are
// not the FFN.  None of them is the hot path; each is a plain, bounds-checked
// HIP kernel in f32 with the reference's formulas:
//   k_embed        embed_lookup (engine.rs:134-144) over the GGUF table
//   k_linear       x W for GGUF weights [N rows, K cols] (Tensor::matmul of
//                  the dequantised, transposed weight, tensor.rs:107-135),
//                  optional residual add (Tensor::add, engine.rs:106)
//   k_rope_kv      apply_rotary_emb (attention.rs:13-34) on q and k, and the
//                  f16 KV cache append (cache/mod.rs:33-63)
//   k_attn_part /  masked softmax attention (attention.rs:56-115), split
//   k_attn_combine over 128-position chunks of the context, then merged
//   k_argmax       greedy sample_top_p (sampler.rs:8-10): max_by(total_cmp),
//                  the last of equal maxima
//   k_advance      the cache length after a forward
// Cache lengths and the token buffers live in device memory, so a decode
// step is the same launch sequence every time (it is captured once into a
// HIP graph and replayed).

#include <algorithm>

#include "device_common.h"
#include "kernels.h"

namespace lcmoe {
namespace {

constexpr int kAttnChunk = 128;  // context positions per attention partial

template <int QT>
__device__ __forceinline__ void dec8(const uint8_t *row, int64_t k, float (&w)[8]) {
    Dec<QT>::run(row, k, w);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// rows [nq] of x [.., d]: row q = token tok[q] of the table, zeros for an id
// outside [0, vocab)
template <int QT>
__global__ __launch_bounds__(256) void k_embed(const uint8_t *__restrict__ table,
                                               int64_t row_bytes, int vocab, int d,
                                               const int32_t *__restrict__ tok, int nq,
                                               float *__restrict__ x) {
    const int q = blockIdx.x;
    if (q >= nq) return;
    const int t = tok[q];
    float *xr = x + (int64_t)q * d;
    for (int c = 8 * threadIdx.x; c < d; c += 8 * blockDim.x) {
        float w[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        if (t >= 0 && t < vocab) dec8<QT>(table + (int64_t)t * row_bytes, c, w);
#pragma unroll
        for (int i = 0; i < 8; i++) xr[c + i] = w[i];
    }
}

// Y[t, n] = (R ? R[t, n] : 0) + sum_k X[t, k] W[n, k] for t < T, n < N.
// One wave per output row (four per block), lanes over K in steps of 8
// decoded elements; TC tokens per block (grid.y).  Y may be R (in place).
template <int QT, int TC>
__global__ __launch_bounds__(256) void k_linear(const uint8_t *__restrict__ W, int64_t row_bytes,
                                                int N, int K, const float *__restrict__ X,
                                                int64_t ldx, int T, const float *R, float *Y,
                                                int64_t ldy) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int n = blockIdx.x * 4 + wave;
    if (n >= N) return;
    const int t0 = blockIdx.y * TC, nt = min(TC, T - t0);
    const uint8_t *wr = W + (int64_t)n * row_bytes;
    float acc[TC];
#pragma unroll
    for (int t = 0; t < TC; t++) acc[t] = 0.0f;
    for (int k = 8 * lane; k < K; k += 512) {
        float w[8];
        dec8<QT>(wr, k, w);
#pragma unroll
        for (int t = 0; t < TC; t++) {
            if (t < nt) {
                const float4 *xp = reinterpret_cast<const float4 *>(X + (int64_t)(t0 + t) * ldx + k);
                const float4 a = xp[0], b = xp[1];
                float s = acc[t];
                s = __builtin_fmaf(a.x, w[0], s);
                s = __builtin_fmaf(a.y, w[1], s);
                s = __builtin_fmaf(a.z, w[2], s);
                s = __builtin_fmaf(a.w, w[3], s);
                s = __builtin_fmaf(b.x, w[4], s);
                s = __builtin_fmaf(b.y, w[5], s);
                s = __builtin_fmaf(b.z, w[6], s);
                s = __builtin_fmaf(b.w, w[7], s);
                acc[t] = s;
            }
        }
    }
#pragma unroll
    for (int t = 0; t < TC; t++) {
        const float s = wave_sum(acc[t]);
        if (lane == 0 && t < nt) {
            const int64_t o = (int64_t)(t0 + t) * ldy + n;
            Y[o] = R ? R[o] + s : s;
        }
    }
}

// Q4_K weights (K a multiple of 256), one token (decode at batch 1): a wave
// takes RW consecutive rows; lane l takes sub-block l % 8 of super-blocks
// l / 8, l / 8 + 8, ...; per sub-block and row it loads the super-block
// header and its pair's 32 quant bytes (three 16-byte loads) and adds
// (d sc) sum_k x q - (dmin m) sum_k x, the decoder's two terms
// (rust/src/kernels/mod.rs:66-98) factored out of the sum.  The lane's 32
// columns of x are loaded once per super-block for all RW rows, and their
// sum once.  Measured on the config-5 decoder at batch 1: RW = 2 513.8
// decode tokens/s, RW = 1 490, RW = 4 503, RW = 8 479 (fewer waves than
// the chip holds).
template <int RW>
__global__ __launch_bounds__(256) void k_linear_q4k_rows(const uint8_t *__restrict__ W,
                                                         int64_t row_bytes, int N, int K,
                                                         const float *__restrict__ X,
                                                         const float *R, float *Y) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int n0 = (blockIdx.x * 4 + wave) * RW;
    if (n0 >= N) return;
    const int j = lane & 7, nsb = K >> 8, sh = 4 * (j & 1), jb = 8 * (j & 3);
    float acc[RW];
#pragma unroll
    for (int r = 0; r < RW; r++) acc[r] = 0.0f;
    for (int sb = lane >> 3; sb < nsb; sb += 8) {
        const float4 *xp = reinterpret_cast<const float4 *>(X + (int64_t)sb * 256 + 32 * j);
        float4 xa[8];
#pragma unroll
        for (int u = 0; u < 8; u++) xa[u] = xp[u];
        uint4 hdr[RW], qa[RW], qb[RW];
#pragma unroll
        for (int r = 0; r < RW; r++) {
            if (n0 + r < N) {
                const uint8_t *blk = W + (int64_t)(n0 + r) * row_bytes + (int64_t)sb * 144;
                hdr[r] = *reinterpret_cast<const uint4 *>(blk);
                const uint4 *qp = reinterpret_cast<const uint4 *>(blk + 16 + 32 * (j >> 1));
                qa[r] = qp[0];
                qb[r] = qp[1];
            }
        }
        float sx = 0.0f;
#pragma unroll
        for (int u = 0; u < 8; u++) sx = sx + xa[u].x + xa[u].y + xa[u].z + xa[u].w;
#pragma unroll
        for (int r = 0; r < RW; r++) {
            if (n0 + r < N) {
                // get_scale_min_k4 (kernels/mod.rs:54-63) from the header words
                const uint32_t by = (hdr[r].y >> jb) & 0xff, bz = (hdr[r].z >> jb) & 0xff;
                const uint32_t bw = (hdr[r].w >> jb) & 0xff;
                const int sc = j < 4 ? (int)(by & 63) : (int)((bw & 15) | ((by >> 6) << 4));
                const int mn = j < 4 ? (int)(bz & 63) : (int)((bw >> 4) | ((bz >> 6) << 4));
                const float dl = dh2f(hdr[r].x & 0xffff) * (float)sc;
                const float ml = dh2f(hdr[r].x >> 16) * (float)mn;
                const uint32_t qw[8] = {qa[r].x, qa[r].y, qa[r].z, qa[r].w,
                                        qb[r].x, qb[r].y, qb[r].z, qb[r].w};
                float sq = 0.0f;
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    const uint32_t w = qw[u] >> sh;
                    sq = __builtin_fmaf(xa[u].x, (float)(w & 15), sq);
                    sq = __builtin_fmaf(xa[u].y, (float)((w >> 8) & 15), sq);
                    sq = __builtin_fmaf(xa[u].z, (float)((w >> 16) & 15), sq);
                    sq = __builtin_fmaf(xa[u].w, (float)((w >> 24) & 15), sq);
                }
                acc[r] = __builtin_fmaf(dl, sq, __builtin_fmaf(-ml, sx, acc[r]));
            }
        }
    }
#pragma unroll
    for (int r = 0; r < RW; r++) {
        const float s = wave_sum(acc[r]);
        if (lane == 0 && n0 + r < N) Y[n0 + r] = R ? R[n0 + r] + s : s;
    }
}

// q rows [nq][H*hd] (rotated) and the cache rows of this call's tokens from
// the projections qkv [nq][(H + 2 KVH) hd] (q, then k, then v).  Query q is
// token i = q % T of sequence b = seq0 + q / T; it lands at cache position
// lens[b] + i and rotates by position i (per-call positions, as the
// reference) or lens[b] + i (absolute).  freq[d] = 1 / theta^(2d/hd) comes
// from the host.  Block (q, head): heads [0, H) rotate q, [H, H + KVH)
// rotate k into the cache, [H + KVH, H + 2 KVH) copy v into it.
__global__ __launch_bounds__(128) void k_rope_kv(const float *__restrict__ qkv, int ks,
                                                 int64_t stride, int nq, int T, int seq0,
                                                 const int32_t *__restrict__ lens, int H, int KVH,
                                                 int hd, const float *__restrict__ freq,
                                                 int absolute, float *__restrict__ qo,
                                                 _Float16 *__restrict__ kc,
                                                 _Float16 *__restrict__ vc, int ctx) {
    const int q = blockIdx.x, hh = blockIdx.y;
    if (q >= nq) return;
    const int b = seq0 + q / T, i = q % T;
    const int pos = lens[b] + i;
    const int half = hd / 2, ldq = (H + 2 * KVH) * hd;
    const float *src = qkv + (int64_t)q * ldq + (int64_t)hh * hd;
    // the projection value: its K-slice partials added in slice order
    auto val = [&](int e) {
        float v = src[e];
        for (int z = 1; z < ks; z++) v = v + src[z * stride + e];
        return v;
    };
    const int64_t crow = ((int64_t)b * ctx + pos) * KVH * hd;
    if (hh >= H + KVH) {  // v
        _Float16 *dst = vc + crow + (int64_t)(hh - H - KVH) * hd;
        for (int e = threadIdx.x; e < hd; e += blockDim.x) dst[e] = (_Float16)val(e);
        return;
    }
    const float fp = (float)(absolute ? pos : i);
    for (int d = threadIdx.x; d < half; d += blockDim.x) {
        const float angle = fp * freq[d];
        const float c = cosf(angle), s = sinf(angle);
        const float x1 = val(d), x2 = val(d + half);
        const float y1 = x1 * c - x2 * s, y2 = x1 * s + x2 * c;
        if (hh < H) {
            float *dst = qo + (int64_t)q * H * hd + (int64_t)hh * hd;
            dst[d] = y1;
            dst[d + half] = y2;
        } else {
            _Float16 *dst = kc + crow + (int64_t)(hh - H) * hd;
            dst[d] = (_Float16)y1;
            dst[d + half] = (_Float16)y2;
        }
    }
}

// One 128-position chunk c of the context of query q, head h: the chunk's
// max score m, sum of exp(score - m) l, and sum of exp(score - m) v (hd
// values).  Query q (token i of sequence b) sees positions [0, lens[b] + i].
// 256 threads: scores by two threads per position (half the dims each),
// then the weighted sum of v by 256 / hd groups of hd threads over
// interleaved positions, added in LDS.
template <int NK>  // 16-byte K loads per thread: hd / 2 <= 8 NK
__global__ __launch_bounds__(256) void k_attn_part(const float *__restrict__ qr, int nq, int T,
                                                   int seq0, const int32_t *__restrict__ lens,
                                                   int H, int KVH, int hd,
                                                   const _Float16 *__restrict__ kc,
                                                   const _Float16 *__restrict__ vc, int ctx,
                                                   int chunks, float *__restrict__ part) {
    typedef _Float16 h8 __attribute__((ext_vector_type(8)));
    const int q = blockIdx.x, h = blockIdx.y, c = blockIdx.z, t = threadIdx.x;
    if (q >= nq) return;
    const int b = seq0 + q / T, i = q % T;
    const int L = lens[b] + i + 1;  // visible positions
    const int kvh = h / (H / KVH);
    float *out = part + (((int64_t)q * H + h) * chunks + c) * (hd + 2);
    const int p0 = c * kAttnChunk;
    if (p0 >= L) {
        for (int d = t; d < hd; d += blockDim.x) out[d] = 0.0f;
        if (t == 0) {
            out[hd] = -INFINITY;
            out[hd + 1] = 0.0f;
        }
        return;
    }
    const int np = min(kAttnChunk, L - p0);
    __shared__ float s_q[256];
    __shared__ float s_half[kAttnChunk];
    __shared__ float s_p[kAttnChunk];
    __shared__ float s_red[8];
    __shared__ float s_acc[2048];
    // One memory round trip for the block: the query element, the chunk's
    // K rows and the first group of V rows all go out before anything
    // waits; positions past np (and K offsets past hd / 2) re-read the last
    // one, never used, so no load sits under a branch.
    const float qv = qr[(int64_t)q * H * hd + h * hd + min(t, hd - 1)];
    const int64_t pstride = (int64_t)KVH * hd;  // elements between positions
    // scores: position p0 + (t % 128), dims [half * hd/2, half * hd/2 + hd/2)
    const int key = t & (kAttnChunk - 1), hf = t >> 7, hd2 = hd / 2;
    h8 kv[NK];
    {
        const _Float16 *kr = kc + ((int64_t)b * ctx + p0 + min(key, np - 1)) * pstride +
                             kvh * hd + hf * hd2;
#pragma unroll
        for (int u = 0; u < NK; u++) kv[u] = *reinterpret_cast<const h8 *>(kr + min(8 * u, hd2 - 8));
    }
    // weighted sum of v: thread (position group kg, dims 8 dg .. 8 dg + 7)
    // over positions kg, kg + KG, ... (one 16-byte load each), then the KG
    // groups added in LDS
    const int DG = hd / 8, KG = 256 / DG, dg = t % DG, kg = t / DG;
    const _Float16 *vr = vc + ((int64_t)b * ctx + p0) * pstride + kvh * hd + 8 * dg;
    h8 vv[8];
#pragma unroll
    for (int u = 0; u < 8; u++)
        vv[u] = *reinterpret_cast<const h8 *>(vr + min(min(kg, KG - 1) + u * KG, np - 1) * pstride);
    if (t < hd) s_q[t] = qv;
    __syncthreads();
    float dot = 0.0f;
    if (key < np) {
#pragma unroll
        for (int u = 0; u < NK; u++)
            if (8 * u < hd2) {
#pragma unroll
                for (int e = 0; e < 8; e++)
                    dot = __builtin_fmaf(s_q[hf * hd2 + 8 * u + e], (float)kv[u][e], dot);
            }
    }
    if (hf) s_half[key] = dot;
    __syncthreads();
    float sc = -INFINITY;
    if (!hf && key < np) sc = (dot + s_half[key]) / sqrtf((float)hd);
    // block max and sum over the chunk's positions (threads 0-127)
    float m = wave_max(sc);
    if ((t & 63) == 0) s_red[t >> 6] = m;
    __syncthreads();
    m = fmaxf(s_red[0], s_red[1]);
    const float p = (!hf && key < np) ? expf(sc - m) : 0.0f;
    if (!hf) s_p[key] = p;
    float l = wave_sum(p);
    __syncthreads();
    if ((t & 63) == 0) s_red[4 + (t >> 6)] = l;
    __syncthreads();
    l = s_red[4] + s_red[5];
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if (kg < KG) {
        for (int k0 = kg; k0 < np; k0 += 8 * KG) {
            if (k0 != kg) {  // groups past the first (hd > 128)
#pragma unroll
                for (int u = 0; u < 8; u++)
                    if (k0 + u * KG < np)
                        vv[u] = *reinterpret_cast<const h8 *>(vr + (k0 + u * KG) * pstride);
            }
#pragma unroll
            for (int u = 0; u < 8; u++)
                if (k0 + u * KG < np) {
                    const float pk = s_p[k0 + u * KG];
#pragma unroll
                    for (int e = 0; e < 8; e++) acc[e] = __builtin_fmaf(pk, (float)vv[u][e], acc[e]);
                }
        }
    }
    float *s_o = s_acc;  // [KG][hd] partial sums, KG * hd <= 2048
    if (kg < KG) {
#pragma unroll
        for (int e = 0; e < 8; e++) s_o[kg * hd + 8 * dg + e] = acc[e];
    }
    __syncthreads();
    if (t < hd) {
        float o = 0.0f;
        for (int j = 0; j < KG; j++) o += s_o[j * hd + t];
        out[t] = o;
    }
    if (t == 0) {
        out[hd] = m;
        out[hd + 1] = l;
    }
}

// out[q][h*hd + d] = sum_c e^(m_c - M) o_c[d] / sum_c e^(m_c - M) l_c
// With x16, the block's hd outputs also go to the matrix-core activation
// format (act16_subblock over the row of H * hd, staged through LDS).
__global__ __launch_bounds__(256) void k_attn_combine(const float *__restrict__ part, int nq,
                                                      int H, int hd, int chunks,
                                                      float *__restrict__ out,
                                                      _Float16 *__restrict__ x16,
                                                      _Float16 *__restrict__ xs) {
    __shared__ __attribute__((aligned(16))) float s_o[256];
    const int q = blockIdx.x, h = blockIdx.y;
    if (q >= nq) return;
    const float *pp = part + ((int64_t)q * H + h) * chunks * (hd + 2);
    float M = -INFINITY;
    for (int c = 0; c < chunks; c++) M = fmaxf(M, pp[c * (hd + 2) + hd]);
    float den = 0.0f;
    for (int c = 0; c < chunks; c++) {
        const float mc = pp[c * (hd + 2) + hd];
        if (mc != -INFINITY) den += expf(mc - M) * pp[c * (hd + 2) + hd + 1];
    }
    for (int d = threadIdx.x; d < hd; d += blockDim.x) {
        float acc = 0.0f;
        for (int c = 0; c < chunks; c++) {
            const float mc = pp[c * (hd + 2) + hd];
            if (mc != -INFINITY) acc += expf(mc - M) * pp[c * (hd + 2) + d];
        }
        out[(int64_t)q * H * hd + h * hd + d] = acc / den;
        s_o[d] = acc / den;
    }
    if (!x16) return;
    __syncthreads();
    const int sb = threadIdx.x;  // this head's 32-column sub-blocks
    if (sb < hd / 32) act16_subblock(s_o + 32 * sb, q, H * hd, h * (hd / 32) + sb, x16, xs);
}

// f32::total_cmp order as a signed integer key
__device__ __forceinline__ int32_t total_key(float v) {
    int32_t b = __float_as_int(v);
    return b ^ (int32_t)(((uint32_t)(b >> 31)) >> 1);
}

// greedy token of row r of logits [nseq][V] (last maximum under total_cmp);
// written to next[seq0 + r] and out[(seq0 + r) * out_ld + *step]
__global__ __launch_bounds__(1024) void k_argmax(const float *__restrict__ logits, int V,
                                                 int seq0, int32_t *__restrict__ next,
                                                 int32_t *__restrict__ out, int out_ld,
                                                 const int32_t *__restrict__ step) {
    const int r = blockIdx.x;
    const float *lr = logits + (int64_t)r * V;
    int32_t bk = INT32_MIN;
    int bi = -1;
    for (int i = threadIdx.x; i < V; i += blockDim.x) {
        const int32_t k = total_key(lr[i]);
        if (bi < 0 || k >= bk) {
            bk = k;
            bi = i;
        }
    }
    __shared__ int32_t s_k[1024];
    __shared__ int32_t s_i[1024];
    s_k[threadIdx.x] = bk;
    s_i[threadIdx.x] = bi;
    __syncthreads();
    for (int o = blockDim.x / 2; o > 0; o >>= 1) {
        if (threadIdx.x < o) {
            const int32_t k2 = s_k[threadIdx.x + o];
            const int i2 = s_i[threadIdx.x + o];
            // larger key wins; on equal keys the larger index (the last maximum)
            if (i2 >= 0 && (s_i[threadIdx.x] < 0 || k2 > s_k[threadIdx.x] ||
                            (k2 == s_k[threadIdx.x] && i2 > s_i[threadIdx.x]))) {
                s_k[threadIdx.x] = k2;
                s_i[threadIdx.x] = i2;
            }
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const int tok = s_i[0] < 0 ? 0 : s_i[0];
        next[seq0 + r] = tok;
        if (out) out[(int64_t)(seq0 + r) * out_ld + *step] = tok;
    }
}

// Y[t, :N] = (R[t] +) sum over slices z in order of part[z][t, :N]; one
// float4 of columns per thread, grid (column blocks of 1024, T)
__global__ __launch_bounds__(256) void k_linear_reduce(const float *__restrict__ part, int ks,
                                                       int64_t stride, int N, const float *R,
                                                       float *Y, int64_t ldy) {
    const int t = blockIdx.y, c4 = blockIdx.x * 256 + threadIdx.x;
    if (4 * c4 >= N) return;
    const float4 *p = reinterpret_cast<const float4 *>(part + (int64_t)t * N) + c4;
    float4 s = p[0];
    for (int z = 1; z < ks; z++) {
        const float4 u = p[z * stride / 4];
        s.x = s.x + u.x; s.y = s.y + u.y; s.z = s.z + u.z; s.w = s.w + u.w;
    }
    if (R) {  // hidden + attn W_o (Tensor::add, engine.rs:106); R may be Y
        const float4 r = reinterpret_cast<const float4 *>(R + (int64_t)t * ldy)[c4];
        s.x = r.x + s.x; s.y = r.y + s.y; s.z = r.z + s.z; s.w = r.w + s.w;
    }
    reinterpret_cast<float4 *>(Y + (int64_t)t * ldy)[c4] = s;
}

// lens[seq0 .. seq0 + nseq) += T; *step += dstep
__global__ void k_advance(int32_t *lens, int seq0, int nseq, int T, int32_t *step, int dstep) {
    const int b = threadIdx.x;
    if (b < nseq) lens[seq0 + b] += T;
    if (b == 0 && step) *step += dstep;
}

}  // namespace

hipError_t launch_embed(int qt, const uint8_t *table, int vocab, int d, const int32_t *tok, int nq,
                        float *x, hipStream_t st) {
    const int64_t rb = (int64_t)lcmoe_tensor_size(qt, d);
    if (nq <= 0) return hipSuccess;
    switch (qt) {
    case LCMOE_TYPE_Q4_K:
        hipLaunchKernelGGL(k_embed<LCMOE_TYPE_Q4_K>, dim3(nq), dim3(256), 0, st, table, rb, vocab,
                           d, tok, nq, x);
        break;
    case LCMOE_TYPE_Q8_0:
        hipLaunchKernelGGL(k_embed<LCMOE_TYPE_Q8_0>, dim3(nq), dim3(256), 0, st, table, rb, vocab,
                           d, tok, nq, x);
        break;
    default:
        hipLaunchKernelGGL(k_embed<LCMOE_TYPE_F32>, dim3(nq), dim3(256), 0, st, table, rb, vocab,
                           d, tok, nq, x);
    }
    return hipGetLastError();
}

template <int QT>
static void linear_tc(const uint8_t *W, int64_t rb, int N, int K, const float *X, int64_t ldx,
                      int T, const float *R, float *Y, int64_t ldy, hipStream_t st) {
    if (T <= 1)
        hipLaunchKernelGGL((k_linear<QT, 1>), dim3((N + 3) / 4, 1), dim3(256), 0, st, W, rb, N, K,
                           X, ldx, T, R, Y, ldy);
    else
        hipLaunchKernelGGL((k_linear<QT, 4>), dim3((N + 3) / 4, (T + 3) / 4), dim3(256), 0, st, W,
                           rb, N, K, X, ldx, T, R, Y, ldy);
}

hipError_t launch_linear(int qt, const uint8_t *W, int N, int K, const float *X, int64_t ldx, int T,
                         const float *R, float *Y, int64_t ldy, hipStream_t st) {
    if (T <= 0 || N <= 0) return hipSuccess;
    const int64_t rb = (int64_t)lcmoe_tensor_size(qt, K);
    switch (qt) {
    case LCMOE_TYPE_Q4_K:
        // one token: the Q4_K sub-block kernel; batches: the generic kernel,
        // whose x reads span fewer cache lines per load (measured faster)
        if (T <= 1)
            hipLaunchKernelGGL(k_linear_q4k_rows<2>, dim3((N + 7) / 8), dim3(256), 0, st, W, rb,
                               N, K, X, R, Y);
        else
            linear_tc<LCMOE_TYPE_Q4_K>(W, rb, N, K, X, ldx, T, R, Y, ldy, st);
        break;
    case LCMOE_TYPE_Q8_0: linear_tc<LCMOE_TYPE_Q8_0>(W, rb, N, K, X, ldx, T, R, Y, ldy, st); break;
    default: linear_tc<LCMOE_TYPE_F32>(W, rb, N, K, X, ldx, T, R, Y, ldy, st);
    }
    return hipGetLastError();
}

// One 32-token pass per block (pass groups of the down kernel); K split
// while the grid holds fewer than 256 blocks (one CU each), at least one
// super-block per slice.
static void linear_mfma_plan(int N, int K, int T, int &chunks, int &ks) {
    chunks = std::min(64, std::max(1, (T + 31) / 32));
    const int base = (N / 64 + 3) / 4 * chunks, NB = K / 256;
    ks = 1;
    while (ks * 2 <= NB && base * ks < 256) ks *= 2;
}

// the largest partials buffer any batch of up to T rows needs
int64_t linear_mfma_part_floats(int N, int K, int T) {
    int64_t most = 0;
    for (int t = 2; t <= T; t++) {
        int chunks, ks;
        linear_mfma_plan(N, K, t, chunks, ks);
        most = std::max(most, (int64_t)ks * t * N);
    }
    return most;
}

hipError_t launch_linear_mfma(const uint8_t *Wr, int N, int K, const float *X, int T,
                              const float *R, float *Y, int64_t ldy, _Float16 *x16, _Float16 *xs,
                              float *part, hipStream_t st, bool act_ready, int *slices) {
    if (T <= 0 || N <= 0) return hipSuccess;
    if (!linear_mfma_ok(N, K) || ldy % 4 || (slices && (R || ldy != N))) return hipErrorInvalidValue;
    int chunks, ks;
    linear_mfma_plan(N, K, T, chunks, ks);
    hipError_t e = act_ready ? hipSuccess : launch_act16(X, T, K, x16, xs, st);
    if (e != hipSuccess) return e;
    // one slot of T tokens (the shared-expert form of the slot arguments)
    const SlotArgsHost sa{nullptr, nullptr, nullptr, nullptr, 1, 1, T, 1, 1, 0, INT32_MAX, 1, 32};
    const bool direct = ks == 1 && !R && ldy == N;
    const int64_t stride = (int64_t)T * N;
    e = launch_mfma_down(Wr, 0, x16, xs, sa, 1, chunks, N, K, ks, direct ? Y : part, stride, st);
    if (slices) {  // the caller adds the slices as it reads them
        *slices = ks;
        return e;
    }
    if (e != hipSuccess || direct) return e;
    hipLaunchKernelGGL(k_linear_reduce, dim3((N / 4 + 255) / 256, T), dim3(256), 0, st, part, ks,
                       stride, N, R, Y, ldy);
    return hipGetLastError();
}

hipError_t launch_rope_kv(const float *qkv, int nq, int T, int seq0, const int32_t *lens, int H,
                          int KVH, int hd, const float *freq, int absolute, float *qo,
                          _Float16 *kc, _Float16 *vc, int ctx, hipStream_t st, int ks,
                          int64_t stride) {
    if (nq <= 0) return hipSuccess;
    if (ks < 1) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_rope_kv, dim3(nq, H + 2 * KVH), dim3(128), 0, st, qkv, ks, stride, nq, T,
                       seq0, lens, H, KVH, hd, freq, absolute, qo, kc, vc, ctx);
    return hipGetLastError();
}

hipError_t launch_attention(const float *qr, int nq, int T, int seq0, const int32_t *lens, int H,
                            int KVH, int hd, const _Float16 *kc, const _Float16 *vc, int ctx,
                            float *part, float *out, hipStream_t st, _Float16 *x16,
                            _Float16 *xs) {
    if (nq <= 0) return hipSuccess;
    if (x16 && ((H * hd) % 256 || hd % 32 || hd > 256)) return hipErrorInvalidValue;
    const int chunks = (ctx + kAttnChunk - 1) / kAttnChunk;
    const dim3 grid(nq, H, chunks);
    if (hd <= 64)
        hipLaunchKernelGGL(k_attn_part<4>, grid, dim3(256), 0, st, qr, nq, T, seq0, lens, H, KVH,
                           hd, kc, vc, ctx, chunks, part);
    else if (hd <= 128)
        hipLaunchKernelGGL(k_attn_part<8>, grid, dim3(256), 0, st, qr, nq, T, seq0, lens, H, KVH,
                           hd, kc, vc, ctx, chunks, part);
    else
        hipLaunchKernelGGL(k_attn_part<16>, grid, dim3(256), 0, st, qr, nq, T, seq0, lens, H, KVH,
                           hd, kc, vc, ctx, chunks, part);
    hipLaunchKernelGGL(k_attn_combine, dim3(nq, H), dim3(128), 0, st, part, nq, H, hd, chunks, out,
                       x16, xs);
    return hipGetLastError();
}

hipError_t launch_argmax(const float *logits, int nseq, int V, int seq0, int32_t *next,
                         int32_t *out, int out_ld, const int32_t *step, hipStream_t st) {
    if (nseq <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_argmax, dim3(nseq), dim3(1024), 0, st, logits, V, seq0, next, out, out_ld,
                       step);
    return hipGetLastError();
}

hipError_t launch_advance(int32_t *lens, int seq0, int nseq, int T, int32_t *step, int dstep,
                          hipStream_t st) {
    hipLaunchKernelGGL(k_advance, dim3(1), dim3(1024), 0, st, lens, seq0, nseq, T, step, dstep);
    return hipGetLastError();
}

int64_t attention_part_floats(int nq, int H, int hd, int ctx) {
    return (int64_t)nq * H * ((ctx + kAttnChunk - 1) / kAttnChunk) * (hd + 2);
}

}  // namespace lcmoe
