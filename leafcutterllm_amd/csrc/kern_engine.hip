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

#include "device_common.h"
#include "kernels.h"

namespace lcmoe {
namespace {

constexpr int kAttnChunk = 128;  // context positions per attention partial

template <int QT>
__device__ __forceinline__ void dec8(const uint8_t *row, int64_t k, float (&w)[8]) {
    Dec<QT>::run(row, k, w);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
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

// q rows [nq][H*hd] (rotated) and the cache rows of this call's tokens from
// the projections qkv [nq][(H + 2 KVH) hd] (q, then k, then v).  Query q is
// token i = q % T of sequence b = seq0 + q / T; it lands at cache position
// lens[b] + i and rotates by position i (per-call positions, as the
// reference) or lens[b] + i (absolute).  freq[d] = 1 / theta^(2d/hd) comes
// from the host.
__global__ __launch_bounds__(256) void k_rope_kv(const float *__restrict__ qkv, int nq, int T,
                                                 int seq0, const int32_t *__restrict__ lens, int H,
                                                 int KVH, int hd, const float *__restrict__ freq,
                                                 int absolute, float *__restrict__ qo,
                                                 _Float16 *__restrict__ kc,
                                                 _Float16 *__restrict__ vc, int ctx) {
    const int q = blockIdx.x;
    if (q >= nq) return;
    const int b = seq0 + q / T, i = q % T;
    const int pos = lens[b] + i;
    const float fp = (float)(absolute ? pos : i);
    const int half = hd / 2, ldq = (H + 2 * KVH) * hd;
    const float *src = qkv + (int64_t)q * ldq;
    const int64_t crow = ((int64_t)b * ctx + pos) * KVH * hd;
    // q heads then k heads: one (head, d < hd/2) pair per thread step
    for (int p = threadIdx.x; p < (H + KVH) * half; p += blockDim.x) {
        const int hh = p / half, d = p % half;
        const float angle = fp * freq[d];
        const float c = cosf(angle), s = sinf(angle);
        const float x1 = src[hh * hd + d], x2 = src[hh * hd + d + half];
        const float y1 = x1 * c - x2 * s, y2 = x1 * s + x2 * c;
        if (hh < H) {
            qo[(int64_t)q * H * hd + hh * hd + d] = y1;
            qo[(int64_t)q * H * hd + hh * hd + d + half] = y2;
        } else {
            const int kh = hh - H;
            kc[crow + kh * hd + d] = (_Float16)y1;
            kc[crow + kh * hd + d + half] = (_Float16)y2;
        }
    }
    for (int e = threadIdx.x; e < KVH * hd; e += blockDim.x)
        vc[crow + e] = (_Float16)src[(H + KVH) * hd + e];
}

// One 128-position chunk c of the context of query q, head h: the chunk's
// max score m, sum of exp(score - m) l, and sum of exp(score - m) v (hd
// values).  Query q (token i of sequence b) sees positions [0, lens[b] + i].
// One wave; lane j owns positions c*128 + j and c*128 + 64 + j.
__global__ __launch_bounds__(64) void k_attn_part(const float *__restrict__ qr, int nq, int T,
                                                  int seq0, const int32_t *__restrict__ lens,
                                                  int H, int KVH, int hd,
                                                  const _Float16 *__restrict__ kc,
                                                  const _Float16 *__restrict__ vc, int ctx,
                                                  int chunks, float *__restrict__ part) {
    const int q = blockIdx.x, h = blockIdx.y, c = blockIdx.z, lane = threadIdx.x;
    if (q >= nq) return;
    const int b = seq0 + q / T, i = q % T;
    const int L = lens[b] + i + 1;  // visible positions
    const int kvh = h / (H / KVH);
    float *out = part + (((int64_t)q * H + h) * chunks + c) * (hd + 2);
    const int p0 = c * kAttnChunk;
    if (p0 >= L) {
        for (int d = lane; d < hd; d += 64) out[d] = 0.0f;
        if (lane == 0) {
            out[hd] = -INFINITY;
            out[hd + 1] = 0.0f;
        }
        return;
    }
    __shared__ float s_q[256];
    __shared__ float s_p[kAttnChunk];
    for (int d = lane; d < hd; d += 64) s_q[d] = qr[(int64_t)q * H * hd + h * hd + d];
    __syncthreads();
    const float sq = sqrtf((float)hd);
    float sc[2];
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const int pos = p0 + 64 * u + lane;
        sc[u] = -INFINITY;
        if (pos < L) {
            const _Float16 *kr = kc + (((int64_t)b * ctx + pos) * KVH + kvh) * hd;
            float dot = 0.0f;
            for (int d = 0; d < hd; d += 8) {
                typedef _Float16 h8 __attribute__((ext_vector_type(8)));
                const h8 kv = *reinterpret_cast<const h8 *>(kr + d);
#pragma unroll
                for (int e = 0; e < 8; e++) dot = __builtin_fmaf(s_q[d + e], (float)kv[e], dot);
            }
            sc[u] = dot / sq;
        }
    }
    const float m = wave_max(fmaxf(sc[0], sc[1]));
    float p[2];
#pragma unroll
    for (int u = 0; u < 2; u++) {
        p[u] = sc[u] == -INFINITY ? 0.0f : expf(sc[u] - m);
        s_p[64 * u + lane] = p[u];
    }
    const float l = wave_sum(p[0] + p[1]);
    __syncthreads();
    const int np = min(kAttnChunk, L - p0);
    for (int d = lane; d < hd; d += 64) {
        float acc = 0.0f;
        const _Float16 *vr = vc + (((int64_t)b * ctx + p0) * KVH + kvh) * hd + d;
        for (int t = 0; t < np; t++)
            acc = __builtin_fmaf(s_p[t], (float)vr[(int64_t)t * KVH * hd], acc);
        out[d] = acc;
    }
    if (lane == 0) {
        out[hd] = m;
        out[hd + 1] = l;
    }
}

// out[q][h*hd + d] = sum_c e^(m_c - M) o_c[d] / sum_c e^(m_c - M) l_c
__global__ __launch_bounds__(256) void k_attn_combine(const float *__restrict__ part, int nq,
                                                      int H, int hd, int chunks,
                                                      float *__restrict__ out) {
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
    }
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
    case LCMOE_TYPE_Q4_K: linear_tc<LCMOE_TYPE_Q4_K>(W, rb, N, K, X, ldx, T, R, Y, ldy, st); break;
    case LCMOE_TYPE_Q8_0: linear_tc<LCMOE_TYPE_Q8_0>(W, rb, N, K, X, ldx, T, R, Y, ldy, st); break;
    default: linear_tc<LCMOE_TYPE_F32>(W, rb, N, K, X, ldx, T, R, Y, ldy, st);
    }
    return hipGetLastError();
}

hipError_t launch_rope_kv(const float *qkv, int nq, int T, int seq0, const int32_t *lens, int H,
                          int KVH, int hd, const float *freq, int absolute, float *qo,
                          _Float16 *kc, _Float16 *vc, int ctx, hipStream_t st) {
    if (nq <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_rope_kv, dim3(nq), dim3(256), 0, st, qkv, nq, T, seq0, lens, H, KVH, hd,
                       freq, absolute, qo, kc, vc, ctx);
    return hipGetLastError();
}

hipError_t launch_attention(const float *qr, int nq, int T, int seq0, const int32_t *lens, int H,
                            int KVH, int hd, const _Float16 *kc, const _Float16 *vc, int ctx,
                            float *part, float *out, hipStream_t st) {
    if (nq <= 0) return hipSuccess;
    const int chunks = (ctx + kAttnChunk - 1) / kAttnChunk;
    hipLaunchKernelGGL(k_attn_part, dim3(nq, H, chunks), dim3(64), 0, st, qr, nq, T, seq0, lens, H,
                       KVH, hd, kc, vc, ctx, chunks, part);
    hipLaunchKernelGGL(k_attn_combine, dim3(nq, H), dim3(128), 0, st, part, nq, H, hd, chunks, out);
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
