// Host-side launchers of the device kernels (one declaration per kernel
// family).  Internal to the library; not part of the ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../include/lcmoe.h"
#include "chains.h"

namespace lcmoe {

struct RouteParams {
    int kind, n_group, topk_group, has_bias;
    float scale;
};

// Router + x limb quantisation + top-k + dispatch, one launch.
struct RouterArgs {
    const float *x;    // [T, d]
    const float *wrt;  // router transposed on the device: [E, d]
    const float *wlc;  // the same in the fast router's lane-chunk order, or null
    const float *bias; // [E] or null
    int T, d, E, K;
    RouteParams rp;
    float *logits;        // [T, E] workspace
    int32_t *topk_idx;    // [T, K]
    float *topk_w;        // [T, K]
    int8_t *xh, *xl;      // [T, d] limbs, or null
    float *xs, *xm;       // [T, d/32] scale and quantised-sum
    _Float16 *x16, *x16s; // f16 hi/lo pieces and sums for the matrix-core path, or null
    bool x16_lo = true;   // sums of hi + lo (the products take both halves), else of hi
    int32_t *counts, *offsets, *perm, *inv, *touched;
    // pass slots, or null: [0] = their number P, then per slot v < P the
    // entry pass * 256 + e, the 32-token passes of every touched expert in
    // expert order (written by the batch dispatch)
    int32_t *pass_slots = nullptr;
    uint32_t *sync;       // [n_token_groups + 1] zero-initialised counters
    // Fused post-attention RMSNorm (certified fast router only): with xin
    // set, each token block first writes x[t] = rms_norm(xin[t]) * norm_w
    // (CpuBackend::rms_norm bit for bit) to xn (== x) and routes from it.
    const float *xin = nullptr, *norm_w = nullptr;
    float norm_eps = 0.0f;
    float *xn = nullptr;
    // Certified sigmoid-group router: float64 logit and bound per (t, e),
    // per-token block counters, and per-token fallback marks (1: the exact
    // chains decide this token); the chain and select launches that follow
    // it serve only the marked tokens when `flag` is set.
    uint64_t *bnd = nullptr;    // [T, E, 2]: keys (klo, khi), (km, finite) as float pairs
    uint32_t *tsync = nullptr;  // [T] zero-initialised
    int32_t *flag = nullptr;    // [T]
};
// The exact router: logits, limbs, top-k, dispatch.
hipError_t launch_router(const RouterArgs &a, hipStream_t st);
// The exact router as chain tiles over the whole chip, then selection and
// dispatch (two launches; d % 128 == 0).  Also writes the limbs (a.xh) and
// the f16 pieces (a.x16) when those are set.
bool route_chains_ok(const RouterArgs &a);
hipError_t launch_route_chains(const RouterArgs &a, hipStream_t st);
// Certified fast router for the softmax kinds: selection, dispatch, limbs
// and f16 pieces.  The weights come from the exact logits: their chains run
// in extra blocks of this launch (columns [0, ch.k1), none if ch.tiles == 0)
// and of the routed gate/up launch (the rest).
bool route_fast_ok(const RouterArgs &a);
hipError_t launch_route_fast(const RouterArgs &a, const ChainArgs &ch, hipStream_t st);
// Certified router with parallel float64 logit bounds (E <= 256, E % 4 == 0,
// d / 256 in {1, 2, 4, 8, 16, 28, 32}; the sigmoid-group kind with
// n_group <= 64, or a softmax kind): E / 4 blocks per token bound the
// logits, the last certifies the (group and) expert selection; a.bnd,
// a.tsync and a.flag set.  Writes topk_idx and the activations.  One token:
// the certifying block also runs the exact fallback and the dispatch.  More:
// the exact chains (launch_route_chains with a.flag) and selection then
// serve only tokens the bounds could not certify, and dispatch every token.
// ch: a first column range of the exact chains, run in blocks beside them.
bool route_sig_ok(const RouterArgs &a);
hipError_t launch_route_sig(const RouterArgs &a, const ChainArgs &ch, hipStream_t st);
int router_token_groups(int T, int d, int E);

// See SlotArgs (device_common.h): nr routed slots, then S fused shared
// experts (stored as experts E .. E+S-1) in ns slots of sl tokens each, at
// positions from sbase.
struct SlotArgsHost {
    const int32_t *perm, *counts, *offsets, *touched;
    int E, K, T, shared;
    int nr, S, sbase, ns, sl;
    // routed slot v < nr is pass slot v (one 32-token pass of one expert)
    // when set (RouterArgs::pass_slots)
    const int32_t *pslots = nullptr;
};

// Generic decode path on GGUF-layout tensors (any supported type, any
// shape): f32 activations in, f32 H / Y out.
// Every gate/up launch also runs the exact router chains `ch` (ch.tiles > 0)
// in blocks that precede the expert blocks: grid row y = 0 holds them and
// expert slot s is row s + 1.
hipError_t launch_generic_gateup(int qt, const uint8_t *gate, const uint8_t *up, int64_t estride,
                                 const float *x, const SlotArgsHost &sa, int slots, int d, int F,
                                 float *Hf, int8_t *hh, int8_t *hl, float *hs, float *hm,
                                 const ChainArgs &ch, hipStream_t st);
hipError_t launch_generic_down(int qt, const uint8_t *down, int64_t estride, const float *Hf,
                               const SlotArgsHost &sa, int slots, int d, int F, float *Y,
                               hipStream_t st);

// Row-per-lane Q4_K decode path on the RPL64 layout: int8-limb activations,
// exact integer dot products.
// H goes out as f32 (Hf), int8 limbs (hh, hl, hs, hm) and/or f16 pieces
// with 32-row sums (h16, hs16) for the matrix-core down; null skips a form.
hipError_t launch_rpl_gateup(const uint8_t *gate, const uint8_t *up, int64_t estride,
                             const int8_t *xh, const int8_t *xl, const float *xs, const float *xm,
                             const SlotArgsHost &sa, int slots, int d, int F, float *Hf, int8_t *hh,
                             int8_t *hl, float *hs, float *hm, _Float16 *h16, _Float16 *hs16,
                             const ChainArgs &ch, hipStream_t st, bool q8 = false);
// fmt: the down matrices are RPL64 Q4_K (0), Q6_K (1), Q8_0 (2) or the split
// Q4_K layout (3, F an odd multiple of 128)
hipError_t launch_rpl_down(const uint8_t *down, int64_t estride, const int8_t *hh,
                           const int8_t *hl, const float *hs, const float *hm,
                           const SlotArgsHost &sa, int slots, int d, int F, int ksplit, float *Y,
                           int64_t split_stride, hipStream_t st, int fmt = 0);

// Matrix-core path on the RPL64 layout: activations as f16 hi/lo pieces
// (per token and super-block: hi[256] then lo[256]) plus per-sub-block sums,
// H out in the same format (and/or f32).
hipError_t launch_act16(const float *x, int T, int d, _Float16 *x16, _Float16 *xs, hipStream_t st,
                        bool lo = true);
// `chunks` blocks share each slot's 32-token passes (block z takes passes
// z, z + chunks, ...), so experts with many tokens spread over the chip.
hipError_t launch_mfma_gateup(const uint8_t *gate, const uint8_t *up, int64_t estride,
                              const _Float16 *x16, const _Float16 *xs, const SlotArgsHost &sa,
                              int slots, int chunks, int d, int F, _Float16 *h16, _Float16 *hs,
                              float *hf, const ChainArgs &ch, hipStream_t st, bool x_lo);
// Q8_0 (RPL64 Q8_0 layout) on the matrix cores, one f16 per activation: a
// one-wave block per 16-token pass and 32 gate/up or 16 down rows.  Gate/up: grid (F / 32,
// slots [+ chain row], groups), SwiGLU into H as f16 pieces (the format of
// launch_mfma_gateup, no sub-block sums) scaled by 2^-e per token and
// 32-column block, e in hexp (one byte per position and block); down: grid
// (d / 16, slots, groups * ksplit) from those, partial sums into Y.  Token
// group z of `groups` takes the slot's 16-token passes z, z + groups, ...
hipError_t launch_mfma_gateup_q8(const uint8_t *gate, const uint8_t *up, int64_t estride,
                                 const _Float16 *x16, const SlotArgsHost &sa, int slots,
                                 int groups, int d, int F, _Float16 *h16, uint8_t *hexp,
                                 const ChainArgs &ch, hipStream_t st);
hipError_t launch_mfma_down_q8(const uint8_t *down, int64_t estride, const _Float16 *h16,
                               const uint8_t *hexp, const SlotArgsHost &sa, int slots, int groups,
                               int d, int F, int ksplit, float *Y, int64_t split_stride,
                               hipStream_t st);
hipError_t launch_mfma_down(const uint8_t *down, int64_t estride, const _Float16 *h16,
                            const _Float16 *hs, const SlotArgsHost &sa, int slots, int chunks,
                            int d, int F, int ksplit, float *Y, int64_t split_stride,
                            hipStream_t st, bool h_lo = true);
// The same down product for Q6_K weights in the RPL64 Q6_K layout (H as f16
// pieces, no sums needed).  h_lo: H enters as two f16 (hi + lo), in passes
// of 16 tokens (p16) or 32; without it as its hi halves, each slot in passes
// of 32 tokens and a last one of at most 16.
hipError_t launch_mfma_down_q6(const uint8_t *down, int64_t estride, const _Float16 *h16,
                               const SlotArgsHost &sa, int slots, int chunks, int d, int F,
                               int ksplit, float *Y, int64_t split_stride, hipStream_t st,
                               bool h_lo, bool p16);

// Routing weights computed by the combine from exact logits (fast-router
// path); logits == null: the weights are already in topk_w.
struct CombineRoute {
    const float *logits;     // [T, E] exact router logits, or null
    const int32_t *topk_idx; // [T, K]
    const float *bias;       // [E] or null
    int kind, E;
    float scale;
};

// y[t] = sum_k w[t,k] * sum_s Yr[s][inv[t,k]] + sum_j sum_s Ys[s][j*T + t].
// With cr.logits, w[t,k] is computed here (and stored to topk_w).
hipError_t launch_combine(const float *Yr, int ks_r, int64_t stride_r, const float *Ys, int ks_s,
                          int64_t stride_s, const int32_t *inv, float *topk_w, int T, int K,
                          int S, int d, const CombineRoute &cr, float *y, hipStream_t st,
                          const float *resid = nullptr);
// C[m,n] = A[m,k] B[k,n], B in the shard engine's Q8_0 / Q4_0 block layout
// (qt LCMOE_TYPE_Q8_0 or LCMOE_TYPE_Q4_0); n % 32 == 0, m <= 65535 * 8.
// S > 1: k in S slices (ceil(k / S) rows each) into ws [S, m, n], then
// added in slice order into C.
hipError_t launch_shard_matmul(int qt, const float *a, const uint8_t *b, float *c, int m, int k,
                               int n, hipStream_t st, int S = 1, float *ws = nullptr);
// The current device's address of the static k-slice scratch
// (kShardScratchFloats floats, one copy per GPU, kern_shard.hip), looked up
// once per device; it stands in for ws in launch_shard_matmul.
constexpr int64_t kShardScratchFloats = LCMOE_SHARD_SCRATCH_FLOATS;
hipError_t shard_scratch(float **out);
// out[t] = rms_norm(x[t]) * w, bit-exact with the reference CPU backend
// (rust/src/backend/cpu.rs:49-60); x, w, out 16-byte aligned, d % 4 == 0.
// With x16 (d % 256 == 0) the normed rows also go to the matrix-core
// activation format in x16 / xs (act16_subblock).
hipError_t launch_rmsnorm(const float *x, const float *w, float eps, int T, int d, float *out,
                          hipStream_t st, _Float16 *x16 = nullptr, _Float16 *xs = nullptr);

// C[m,n] = A[m,k] B[k,n] in f32, bit-identical to the CPU backend's
// avx2_matmul order (kern_matmul.hip); m <= 65535 * 8.
hipError_t launch_matmul_f32(const float *A, const float *B, float *C, int m, int k, int n,
                             hipStream_t st);

// ---- decoder-layer kernels of the end-to-end engine (kern_engine.hip) ----
hipError_t launch_embed(int qt, const uint8_t *table, int vocab, int d, const int32_t *tok, int nq,
                        float *x, hipStream_t st);
// Y[t, :N] (+= R) = X[t, :K] W^T, W GGUF [N, K] of type qt with K whole blocks
hipError_t launch_linear(int qt, const uint8_t *W, int N, int K, const float *X, int64_t ldx, int T,
                         const float *R, float *Y, int64_t ldy, hipStream_t st);
// Matrix-core linear for batches: Y[t, :N] (= or R[t] +) X[t, :K] W^T for
// Q4_K W [N, K] in the RPL64 layout (linear_mfma_ok), X rows contiguous
// (ld K).  X goes to f16 hi/lo pieces in x16 / xs (T * K * 2 and
// T * K / 16 halves), the product runs on the matrix-core down kernel (one
// slot holding all T tokens), K split into ks slices when that fills the
// GPU better; part (linear_mfma_part_floats(N, K, most rows)) takes the slices' partials,
// which a reduce adds in slice order (then R) into Y (row stride ldy).
inline bool linear_mfma_ok(int64_t N, int64_t K) { return N % 64 == 0 && K % 256 == 0; }
int64_t linear_mfma_part_floats(int N, int K, int T);
// act_ready: x16 / xs already hold X's pieces (X is not read).  slices !=
// null (R null): no reduce; the K-slice partials stay in part (several) or
// in Y (one, ldy == N), and *slices receives their number (the slices of
// row t at part + z * T * N + t * N, z in order).
hipError_t launch_linear_mfma(const uint8_t *Wr, int N, int K, const float *X, int T,
                              const float *R, float *Y, int64_t ldy, _Float16 *x16, _Float16 *xs,
                              float *part, hipStream_t st, bool act_ready = false,
                              int *slices = nullptr);
// qkv: ks K-slice partials of the projection, `stride` floats apart, added
// in slice order as they are read (ks = 1: the projection itself)
hipError_t launch_rope_kv(const float *qkv, int nq, int T, int seq0, const int32_t *lens, int H,
                          int KVH, int hd, const float *freq, int absolute, float *qo,
                          _Float16 *kc, _Float16 *vc, int ctx, hipStream_t st, int ks = 1,
                          int64_t stride = 0);
// With x16 (H * hd % 256 == 0), the output rows also go to the matrix-core
// activation format (act16_subblock) for the output projection.
hipError_t launch_attention(const float *qr, int nq, int T, int seq0, const int32_t *lens, int H,
                            int KVH, int hd, const _Float16 *kc, const _Float16 *vc, int ctx,
                            float *part, float *out, hipStream_t st, _Float16 *x16 = nullptr,
                            _Float16 *xs = nullptr);
hipError_t launch_argmax(const float *logits, int nseq, int V, int seq0, int32_t *next,
                         int32_t *out, int out_ld, const int32_t *step, hipStream_t st);
hipError_t launch_advance(int32_t *lens, int seq0, int nseq, int T, int32_t *step, int dstep,
                          hipStream_t st);
int64_t attention_part_floats(int nq, int H, int hd, int ctx);

hipError_t launch_debug_dequant(int qt, const uint8_t *src, int64_t count, float *out,
                                hipStream_t st);
hipError_t launch_debug_sigmoid(const float *x, int64_t n, float *out, hipStream_t st);
// Streaming-read probe over `bytes` (a multiple of 16) at p; sink: `blocks`
// words, written only on an impossible match.
hipError_t launch_stream_read(const void *p, int64_t bytes, int blocks, uint32_t *sink,
                              hipStream_t st);

// RPL64 eligibility: Q4_K, rows tile by 64, columns are whole super-blocks.
inline bool rpl64_ok(int qt, int64_t rows, int64_t cols) {
    return qt == 12 && rows % 64 == 0 && cols % 256 == 0;
}
// Q8_0 matrices the row-per-lane kernels serve (RPL64 Q8_0 layout)
inline bool rpl64_q8_ok(int qt, int64_t rows, int64_t cols) {
    return qt == 8 && rows % 64 == 0 && cols % 256 == 0;
}
// Q6_K matrices the matrix-core down serves (RPL64 Q6_K layout)
inline bool rpl64_q6_ok(int qt, int64_t rows, int64_t cols) {
    return qt == 14 && rows % 64 == 0 && cols % 256 == 0;
}

}  // namespace lcmoe
