/*
 * lcoracle.h -- CPU oracle for the MoE feed-forward hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker: it may be loaded by
 * tests/, by __graft_entry__.smoke() and by bench.py's cpu_baseline leg, and by
 * nothing else.  The product library (leafcutterllm_amd/liblcmoe.so) never
 * links, loads or calls it.
 *
 * It restates, in plain C, the arithmetic of the reference Rust CPU path that
 * the GPU path replaces (every function cites the reference file:line it
 * follows; paths are relative to the reference repository root), plus the MoE
 * routing / dispatch / combine semantics that the reference does not have and
 * that this project fixes in writing (router kinds, tie rules, slot order).
 *
 * Pinning status per function (what checks it besides itself):
 *   f16 <-> f32          : exhaustive vs numpy float16 (tests/test_oracle_core.py)
 *   dequant Q8_0         : reference KAT q8_0.rs:128-149, round trip q8_0.rs:151-166
 *   dequant Q4_K / Q6_K  : reference zero KATs kernels/mod.rs:235-251, block
 *                          geometry quant.rs:314-335 + gguf.rs:338-346, hand-built
 *                          layout KATs packed by an independent packer in the test
 *   quantize Q8_0        : reference round trip q8_0.rs:151-166, KATs
 *   quantize Q4_K / Q6_K : round-trip error <= half a quantisation step
 *   matmul (AVX2 order)  : reference KATs simd.rs:430-455 (exact), error bound vs
 *                          float64, FMA-lane vs mul+add-tail bit behaviour
 *   silu / softmax       : closed form in float64, tensor.rs:211-217 KAT
 *   lc_expf / sigmoid    : <= 2 ulp vs float64 exp over a dense sweep
 *   shard_matmul         : reference test matrices int8_gemm.rs:378-511 against
 *                          dequantise-then-matmul (1e-3), float64 bound, exact
 *                          small-integer KATs that fix operand order and nibbles
 *   rms_norm             : reference test tensor.rs:204-209, float64 closed form,
 *                          exact constant rows, scale-then-weight rounding order;
 *                          the four-lane sum-of-squares order (simd.rs:390-401)
 *                          bit for bit against an independent numpy float32
 *                          restatement, on rows where a sequential sum differs
 *   sanitize             : tests/test_oracle_core.py -- the closed form of
 *                          loader.rs:241-249 at its cut-off (+-100 kept, the
 *                          next float above 100 zeroed, NaN and +-inf zeroed)
 *                          and through the ingest of every type (hand-built
 *                          blocks whose outlier positions are known); the
 *                          layer forward sanitises router and bias as well
 *   route (all kinds)    : tests/test_oracle_route.py -- brute force over the
 *                          full sort of (-z, e) with ties, +-0, +-inf and NaN
 *                          for the softmax, renormalised-softmax and
 *                          sigmoid-group routers (group scores, kept groups),
 *                          weights in float64; hand-checked tie rows
 *   dispatch             : tests/test_oracle_route.py -- numpy stable argsort,
 *                          bincount / cumsum, permutation and inverse invariants
 *   layer forward        : tests/test_oracle_route.py -- float64 recomputation
 *                          from dequantised weights (selection, weights, experts,
 *                          shared experts, combine); E=1,K=1 equals the dense
 *                          ffn_forward (engine.rs:146-164) bit for bit;
 *                          all-zero experts -> 0; duplicated experts additive;
 *                          routed_scale exact; shared expert adds its FFN
 *   rope / attention /   : tests/test_oracle_engine.py -- position 0 is the
 *   argmax                 identity, pair norms kept, angles vs float64,
 *                          the reference's per-call positions; attention vs a
 *                          float64 restatement, one key -> its value, causal
 *                          mask; argmax KAT sampler.rs:57-61, last of ties,
 *                          total order over +-0 / NaN
 *   golden fixtures      : tests/golden/moe_*.npz (written by
 *                          tests/golden/make_golden.py) reproduced bit for bit
 *                          and checked against the float64 recomputation
 *                          (tests/test_golden.py)
 */
#ifndef LCORACLE_H
#define LCORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF ggml_type codes (rust/src/model/quant.rs:45-73). */
enum { LCO_F32 = 0, LCO_F16 = 1, LCO_Q8_0 = 8, LCO_Q4_K = 12, LCO_Q6_K = 14 };
/* The shard engine's Q4_0 (interleaved nibbles; GGML's Q4_0 code 2). */
enum { LCO_Q4_0_SHARD = 2 };

/* Router kinds. */
enum {
    LCO_ROUTE_SOFTMAX_RENORM = 0, /* softmax over the K selected logits      */
    LCO_ROUTE_SOFTMAX = 1,        /* full-E softmax probs of the selected    */
    LCO_ROUTE_SIGMOID_GROUP = 2   /* sigmoid + bias, group-limited, scaled   */
};

/* Layer descriptor; same field order and types as lcmoe_desc. */
typedef struct {
    int32_t d_model, d_ff, n_expert, n_expert_used;
    int32_t n_shared, d_ff_shared;
    int32_t route_kind, n_group, topk_group;
    float routed_scale;
    int32_t has_bias;
    int32_t type_gate, type_up, type_down;
    int32_t type_gate_sh, type_up_sh, type_down_sh;
    int32_t max_tokens;
} lco_desc;

/* Layer weights; same field order as lcmoe_weights.  Expert tensors are the
 * GGUF stacked layout: expert e's [rows, cols] matrix is the e-th contiguous
 * slice of tensor_size(rows*cols) bytes; blocks run along cols (the input
 * dimension).  gate/up: [d_ff rows, d_model cols]; down: [d_model, d_ff]. */
typedef struct {
    const float *router; /* [d_model, n_expert] f32, the post-load [in,out] form */
    const float *bias;   /* [n_expert] or NULL                                    */
    const uint8_t *gate, *up, *down;
    const uint8_t *gate_sh, *up_sh, *down_sh;
} lco_weights;

/* ---- formats ---------------------------------------------------------- */
float lco_f16_to_f32(uint16_t h);
uint16_t lco_f32_to_f16(float f);
void lco_f16_to_f32_n(const uint16_t *h, float *f, size_t n);
void lco_f32_to_f16_n(const float *f, uint16_t *h, size_t n);

size_t lco_block_size(int type);
size_t lco_block_bytes(int type);
size_t lco_tensor_size(int type, size_t count);

void lco_dequant_q8_0(const uint8_t *src, float *dst, size_t count);
void lco_dequant_q4_k(const uint8_t *src, float *dst, size_t count);
void lco_dequant_q6_k(const uint8_t *src, float *dst, size_t count);
int lco_dequant(int type, const uint8_t *src, float *dst, size_t count);
void lco_scale_min_k4(int j, const uint8_t *q, uint8_t *sc, uint8_t *m);

void lco_quantize_q8_0(const float *src, uint8_t *dst, size_t count);
void lco_quantize_q4_k(const float *src, uint8_t *dst, size_t count);
void lco_quantize_q6_k(const float *src, uint8_t *dst, size_t count);
int lco_quantize(int type, const float *src, uint8_t *dst, size_t count);

void lco_sanitize(float *v, size_t n);
/* scan_for_corruption: number of blocks with a non-finite or |scale|>1e4. */
size_t lco_scan_blocks(int type, const uint8_t *src, size_t count);

/* ---- synthetic data --------------------------------------------------- */
void lco_synth_normal(uint64_t seed, uint64_t stream, float stddev, float *out, size_t n);

/* ---- arithmetic --------------------------------------------------------- */
void lco_matmul(const float *a, const float *b, float *c, int m, int k, int n, int threads);
void lco_transpose(const float *a, float *b, int rows, int cols);
float lco_silu(float v);
void lco_rms_norm(const float *x, const float *w, float eps, int T, int d, float *out);
int lco_shard_matmul(int type, const float *a, const uint8_t *b, float *c, int m, int k, int n);
void lco_softmax(const float *x, float *y, int n);
float lco_expf_cw(float x);
float lco_sigmoid_cw(float x);
/* largest dip of lco_sigmoid_cw below its running maximum over all non-NaN
 * floats, in ulps (exhaustive; `threads` OpenMP threads) */
int64_t lco_sigmoid_max_dip(int threads);

/* ---- routing ---------------------------------------------------------- */
void lco_router_logits(const float *x, const float *w, float *l, int T, int d, int E);
int lco_route(const lco_desc *desc, const float *logits, const float *bias, int T,
              int32_t *topk_idx, float *topk_w);
int lco_dispatch(const int32_t *topk_idx, int T, int K, int E, int32_t *counts,
                 int32_t *offsets, int32_t *perm, int32_t *inv);

/* ---- whole layer -------------------------------------------------------- */
/* y[T, d] = MoE FFN of x[T, d].  Optional outputs may be NULL.  Weights are
 * dequantised one expert at a time (dequant -> transpose -> sanitize, as
 * loader.rs:145-168 does per tensor); the router and the bias are sanitised
 * too (loader.rs:161).  threads<=0 -> reference row split. */
int lco_moe_forward(const lco_desc *desc, const lco_weights *w, const float *x, int T,
                    float *y, int32_t *topk_idx, float *topk_w, int32_t *counts,
                    int32_t *offsets, int32_t *perm, int32_t *inv, int threads);

/* Dense SwiGLU FFN on f32 weights in the post-load [in,out] layout:
 * y = (silu(x Wg) * (x Wu)) Wd, engine.rs:146-164. */
void lco_ffn_dense(const float *x, int m, int d, int F, const float *wg_t,
                   const float *wu_t, const float *wd_t, float *y, int threads);

/* CPU baseline: experts pre-dequantised to f32 (post-load layout) once,
 * then timed forwards.  Returns an opaque handle. */
void *lco_resident_create(const lco_desc *desc, const lco_weights *w, int threads);
int lco_resident_forward(void *h, const float *x, int T, float *y, int threads);
void lco_resident_destroy(void *h);

/* ---- decoder-layer pieces (end-to-end engine, engine.rs:78-132) --------- */
/* apply_rotary_emb (attention.rs:13-34) with positions pos0 + i (the
 * reference: pos0 = 0 on every call). */
void lco_rope(float *x, int seq, int heads, int hd, float theta, int pos0);
/* attention_forward's core (attention.rs:56-115) over a cache of `total`
 * positions whose last `seq` are this call's tokens. */
void lco_attention_core(const float *q, const float *k, const float *v, int seq, int total,
                        int heads, int kv_heads, int hd, float *out);
/* greedy sample_top_p (sampler.rs:8-10): max_by(total_cmp), last maximum */
int lco_argmax_last(const float *x, int n);

#ifdef __cplusplus
}
#endif
#endif
