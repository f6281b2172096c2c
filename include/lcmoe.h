/*
 * lcmoe.h -- C ABI of the MI355X (gfx950) MoE feed-forward layer.
 *
 * Drop-in boundary for the reference engine's FFN call:
 *   Engine::ffn_forward(&self, x: &Tensor, weights) -> Tensor
 *     rust/src/inference/engine.rs:146-164 (called at engine.rs:114), and its
 *     twin ShardEngine::ffn_forward, rust/src/inference/shard_engine.rs:181-198
 *     (called at shard_engine.rs:146).
 * The arithmetic under it replaces Tensor::matmul's dispatch
 * (rust/src/model/tensor.rs:107-135) into Backend::matmul
 * (rust/src/backend/mod.rs:18-46, CpuBackend at rust/src/backend/cpu.rs:13-23)
 * and the quantised GEMMs (rust/src/kernels/int8_gemm.rs:172-194), with the
 * GGUF block decoders (rust/src/kernels/mod.rs:37-180) running on the GPU.
 *
 * Plain C: pointers, sizes, integer status codes.  No C++ or HIP types cross
 * the boundary (a stream is passed as void*).
 *
 * Threading: one handle = one HIP stream + one workspace; a handle serves one
 * caller at a time (the reference already serialises through
 * Arc<Mutex<Engine>>, rust/src/main.rs:41).  Distinct handles may be used
 * concurrently.  lcmoe_last_error() is per thread.
 */
#ifndef LCMOE_H
#define LCMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LCMOE_ABI_VERSION 1

typedef enum {
    LCMOE_OK = 0,
    LCMOE_ERR_INVALID_ARG = 1,    /* null pointer, bad shape or size         */
    LCMOE_ERR_UNSUPPORTED = 2,    /* quant type / router kind not supported  */
    LCMOE_ERR_CORRUPT = 3,        /* non-finite or absurd block scale,
                                     malformed or truncated GGUF file        */
    LCMOE_ERR_HIP = 4,            /* HIP runtime error (incl. no device)     */
    LCMOE_ERR_OUT_OF_MEMORY = 5,  /* device allocation failed                */
    LCMOE_ERR_STATE = 6,          /* e.g. query before any forward           */
    LCMOE_ERR_NOT_FOUND = 7,      /* GGUF tensor or metadata key absent      */
    LCMOE_ERR_IO = 8              /* file cannot be opened or mapped         */
} lcmoe_status;

/* GGUF ggml_type codes, QuantType::code, rust/src/model/quant.rs:45-73. */
enum {
    LCMOE_TYPE_F32 = 0,
    LCMOE_TYPE_Q4_0 = 2, /* lcmoe_shard_matmul only: the shard engine's Q4_0 */
    LCMOE_TYPE_Q8_0 = 8,
    LCMOE_TYPE_Q4_K = 12,
    LCMOE_TYPE_Q6_K = 14
};

/* Router kinds.  The reference has no router; these are the written
 * semantics this library implements (selection ties -> lower expert index,
 * NaN ranks as -inf). */
enum {
    /* z = l (+bias); top-K of z; w = softmax over the K selected z (Mixtral) */
    LCMOE_ROUTE_SOFTMAX_RENORM = 0,
    /* z = l (+bias); top-K of z; w = full-E softmax(z) at the selected      */
    LCMOE_ROUTE_SOFTMAX = 1,
    /* s = sigmoid(l); z = s (+bias); groups of E/n_group experts scored by
     * their top-2 z; top topk_group groups kept; top-K z inside them;
     * w = routed_scale * s / sum(s over the K)      (DeepSeek-V3 noaux_tc)  */
    LCMOE_ROUTE_SIGMOID_GROUP = 2
};

/* Layer descriptor.  Limits (checked by lcmoe_create): d_model % 32 == 0
 * and d_model <= 16384, d_ff % 32 == 0, n_expert <= 256, n_expert_used <= 16,
 * n_shared <= 8, max_tokens <= 65536.  The fast kernels need more: Q4_K /
 * Q6_K / Q8_0 experts take the row-tiled layouts when the matrix rows are a
 * multiple of 64 and d_model % 256 == 0, and the certified softmax router
 * needs d_model / 256 in {1, 2, 4, 8, 16} and n_expert <= 64; every other
 * valid shape runs the generic kernels and the exact router (same results,
 * lower speed).  K-quant blocks of 256 run over the flattened matrix, so a
 * K-quant matrix whose columns are not a multiple of 256 has blocks that
 * straddle rows, as the reference decoder allows (kernels/mod.rs:66-70). */
typedef struct {
    int32_t d_model;       /* d                                           */
    int32_t d_ff;          /* F, routed expert hidden size                */
    int32_t n_expert;      /* E                                           */
    int32_t n_expert_used; /* K                                           */
    int32_t n_shared;      /* S, always-on shared experts (weight 1.0)   */
    int32_t d_ff_shared;   /* hidden size of each shared expert           */
    int32_t route_kind;    /* LCMOE_ROUTE_*                               */
    int32_t n_group;       /* sigmoid-group router only                   */
    int32_t topk_group;    /* sigmoid-group router only                   */
    float routed_scale;    /* multiplies every routed weight (1.0 = none) */
    int32_t has_bias;      /* bias[E] added to the selection score        */
    int32_t type_gate, type_up, type_down;          /* LCMOE_TYPE_*     */
    int32_t type_gate_sh, type_up_sh, type_down_sh; /* shared experts   */
    int32_t max_tokens;    /* largest T a forward call may pass           */
} lcmoe_desc;

/* Host weight pointers, copied to the device by lcmoe_create (the caller
 * keeps ownership).  Expert tensors use the GGUF stacked layout
 * (ffn_{gate,up,down}_exps): expert e's [rows, cols] matrix is the e-th
 * contiguous slice of tensor_size(type, rows*cols) bytes, quant blocks along
 * cols (the input dimension) over the flattened matrix, exactly what
 * GGUFile::get_tensor_raw (rust/src/model/gguf.rs:121-127) returns.
 *   gate, up : E x [d_ff rows, d_model cols]
 *   down     : E x [d_model rows, d_ff cols]
 *   *_sh     : the same for the S shared experts with d_ff_shared.
 * router is f32 [d_model, n_expert] row-major, the post-load [in,out] form
 * produced by load_layer (rust/src/model/loader.rs:155-160). */
typedef struct {
    const float *router;
    const float *bias; /* [n_expert] f32, or NULL when has_bias == 0 */
    const uint8_t *gate, *up, *down;
    const uint8_t *gate_sh, *up_sh, *down_sh;
} lcmoe_weights;

typedef struct lcmoe_handle lcmoe_handle;

/* Validates desc, scans every block scale on the host (the per-block test of
 * scan_for_corruption, rust/src/model/loader.rs:301-422), uploads all
 * weights once to the current HIP device and keeps them resident.
 * Replaces the per-forward GGUFModel::load_layer ingest
 * (rust/src/model/loader.rs:145-168, called from engine.rs:96), including
 * its sanitize_weights step (loader.rs:161, :241-249): every router, bias and
 * expert weight whose dequantised value is NaN, +-Inf or |v| > 100 is used
 * as 0 (see lcmoe_sanitize_blocks; a Q4_K matrix kind with an outlier that
 * Q4_K cannot hold as zero is stored as f32 and runs the generic kernels).
 * Divergence: a block whose scale is non-finite or above 1e4 is refused
 * with LCMOE_ERR_CORRUPT, where the reference's Engine::load reports it and
 * runs on with the zeroed values (rust/src/inference/engine.rs:22-25); a
 * caller that wants that behaviour applies lcmoe_sanitize_blocks to the
 * bytes first, which zeroes non-finite-scale blocks. */
lcmoe_status lcmoe_create(const lcmoe_desc *desc, const lcmoe_weights *w, lcmoe_handle **out);
void lcmoe_destroy(lcmoe_handle *h);

/* y[T, d] = MoE FFN of x[T, d] (f32, host memory, row-major).  Synchronous:
 * returns after y is written, like ffn_forward (engine.rs:146-164).  The
 * residual add of engine.rs:115 stays with the caller.  topk_idx [T, K] and
 * topk_w [T, K] are optional (NULL to skip).  T may be 0. */
lcmoe_status lcmoe_forward(lcmoe_handle *h, const float *x, int32_t T, float *y,
                           int32_t *topk_idx, float *topk_w);

/* Same on device pointers, enqueued on `stream` (a hipStream_t, NULL = the
 * handle's own stream); returns without waiting.  x_dev / y_dev must stay
 * valid until the stream reaches this work. */
lcmoe_status lcmoe_forward_dev(lcmoe_handle *h, const float *x_dev, int32_t T, float *y_dev,
                               void *stream);

/* Activation operands of the matrix-core expert products (batches where
 * the experts see more tokens than there are experts, T*K > E, or T >= 4;
 * prefill).
 * The weights are always exact (sc*q in f16, scales in f32) and the sums
 * f32; the mode sets how x enters the gate/up products and H the down
 * products:
 *   LCMOE_ACT_F16   (default) one f16 per element: layer output within about
 *                   3.7e-4 relative L2 of the reference CPU path at every
 *                   benchmark shape (the bar is 1e-3), half the matrix-core
 *                   work and activation traffic of F16X2;
 *   LCMOE_ACT_F16X2 two f16 (hi + lo = x to about 22 bits): about 3e-6, for
 *                   deep stacks where per-layer error compounds (lcmoe_model
 *                   selects it for every layer).
 * The row-per-lane (decode) kernels always use exact integer products on
 * 15-bit activations.
 * No counterpart in the reference (its CPU path is f32 throughout). */
enum { LCMOE_ACT_F16 = 0, LCMOE_ACT_F16X2 = 1 };
lcmoe_status lcmoe_set_act_precision(lcmoe_handle *h, int32_t mode);

/* Post-attention RMSNorm weight [d_model] f32 and epsilon used by the
 * lcmoe_forward_norm_residual* calls below (the reference passes 1e-5,
 * engine.rs:111).  Copied to the device, sanitised as load_layer sanitises
 * every layer tensor (rust/src/model/loader.rs:161, :241-249: NaN, +-Inf and
 * |v| > 100 become 0); may be called again to replace it. */
lcmoe_status lcmoe_set_norm(lcmoe_handle *h, const float *weight, float eps);

/* The FFN half of a decoder layer with its norm and residual fused:
 *   out = hidden + ffn_forward(rms_norm(hidden, weight, eps))
 * replacing rust/src/inference/engine.rs:110-115 (rms_norm is
 * CpuBackend::rms_norm, rust/src/backend/cpu.rs:49-60, reproduced bit for
 * bit; the add is Tensor::add).  Host buffers, synchronous, as
 * lcmoe_forward; out may be hidden itself.  LCMOE_ERR_STATE before
 * lcmoe_set_norm. */
lcmoe_status lcmoe_forward_norm_residual(lcmoe_handle *h, const float *hidden, int32_t T,
                                         float *out, int32_t *topk_idx, float *topk_w);
/* Device-buffer, stream-ordered form (as lcmoe_forward_dev); out_dev is
 * hidden_dev itself (in place) or does not overlap it. */
lcmoe_status lcmoe_forward_norm_residual_dev(lcmoe_handle *h, const float *hidden_dev, int32_t T,
                                             float *out_dev, void *stream);

/* Routing and dispatch of the most recent forward (waits for it):
 * topk_idx/topk_w [T, K]; counts [E]; offsets [E+1] (exclusive scan, offsets[E]
 * = T*K); perm [T*K]: position -> assignment a = t*K + k (stable by a within
 * an expert); inv [T*K]: assignment -> position.  Any pointer may be NULL. */
lcmoe_status lcmoe_get_dispatch(lcmoe_handle *h, int32_t *T_out, int32_t *topk_idx,
                                float *topk_w, int32_t *counts, int32_t *offsets,
                                int32_t *perm, int32_t *inv);

/* Kernel timing.  When enabled, each forward records HIP events around each
 * of its kernels on the stream it runs on; lcmoe_get_timing returns, per
 * kernel slot, the accumulated milliseconds and launch count since the last
 * reset (waits for the stream).  Slot names come from lcmoe_timing_name. */
lcmoe_status lcmoe_set_timing(lcmoe_handle *h, int32_t enable);
lcmoe_status lcmoe_get_timing(lcmoe_handle *h, int32_t n_slots, double *ms, int64_t *launches);
const char *lcmoe_timing_name(int32_t slot);
int32_t lcmoe_timing_slots(void);

/* Per-thread message for the last non-OK status ("" if none). */
const char *lcmoe_last_error(void);

/* ---- host utilities (no GPU needed) ------------------------------------ */

/* QuantType::tensor_size, rust/src/model/quant.rs:256-261 (0 if unknown). */
size_t lcmoe_tensor_size(int32_t type, int64_t count);

/* Number of blocks whose scale(s) are non-finite or |.| > 1e4
 * (scan_for_corruption's test, rust/src/model/loader.rs:389-398). */
int64_t lcmoe_scan_blocks(int32_t type, const uint8_t *data, int64_t count);

/* GGUF bytes -> f32 on the host: GGUFModel::dequantize for F32, Q8_0, Q4_K
 * and Q6_K (rust/src/model/loader.rs:205-235, decoders
 * rust/src/kernels/mod.rs:37-180: whole blocks only, a partial tail stays 0),
 * then, when `sanitize` is nonzero, sanitize_weights (loader.rs:241-249:
 * NaN, +-Inf and |v| > 100 become 0).  Returns the number of values the
 * sanitising zeroed, or -1 for a NULL pointer, count < 0 or another type. */
int64_t lcmoe_dequantize(int32_t type, const uint8_t *data, int64_t count, float *out,
                         int32_t sanitize);

/* sanitize_weights (loader.rs:241-249) applied to GGUF bytes in place, as
 * lcmoe_create and lcmoe_model_create apply it to every weight they upload:
 * an element whose decoded value is NaN, +-Inf or |v| > 100 gets the code of
 * an exact zero (Q8_0: q = 0; Q6_K: 6-bit code 32; Q4_K: q = 0 where
 * dmin * m is zero; F32: 0.0f), and a block whose scale is not finite gets
 * zero scales.  Returns the number of elements zeroed, or -1 as above.
 * *unzeroable (optional) receives the number of Q4_K outliers left as they
 * are because their sub-block cannot encode zero; lcmoe_create stores such
 * a tensor as its sanitised f32 dequantisation instead. */
int64_t lcmoe_sanitize_blocks(int32_t type, uint8_t *data, int64_t count, int64_t *unzeroable);

/* Quantise f32 to GGUF blocks.  Q8_0 is quantize_f32_to_q8_0
 * (rust/src/kernels/q8_0.rs:90-122); Q4_K and Q6_K are this project's own
 * encoders (the reference has none).  count % block size must be 0.
 * Multithreaded; the bytes do not depend on the thread count. */
lcmoe_status lcmoe_quantize(int32_t type, const float *src, uint8_t *dst, int64_t count);

/* Synthetic N(0, stddev^2) data: counter-based splitmix64 + Box-Muller in
 * float64; element i depends only on (seed, stream, i). */
void lcmoe_synth_normal(uint64_t seed, uint64_t stream, float stddev, float *out, int64_t n);

/* ---- GGUF ingest (host only, no GPU needed) --------------------------- */

/* A GGUF v3 file, memory-mapped read-only and parsed, as GGUFile::open does
 * (rust/src/model/gguf.rs:76-119): header, metadata, tensor infos, data
 * section at general.alignment (default 32).  Unlike the reference, every
 * tensor of known type is checked to lie inside the file at open
 * (LCMOE_ERR_CORRUPT otherwise); version != 3 is LCMOE_ERR_UNSUPPORTED, as
 * GGUError::UnsupportedVersion.  One caller at a time per handle. */
typedef struct lcmoe_gguf lcmoe_gguf;

lcmoe_status lcmoe_gguf_open(const char *path, lcmoe_gguf **out);
/* Unmaps the file; every pointer obtained from the handle dies with it. */
void lcmoe_gguf_close(lcmoe_gguf *g);

/* GGUFile::get_metadata_int (gguf.rs:133-157): any integer or float value
 * (floats truncated), or a one-element U32/I32/U64/I64 array.
 * LCMOE_ERR_NOT_FOUND if absent, LCMOE_ERR_INVALID_ARG if of another type. */
lcmoe_status lcmoe_gguf_meta_int(const lcmoe_gguf *g, const char *key, int64_t *out);
/* A string value (bytes as stored, NUL-terminated), NULL if absent or not a
 * string.  Valid until lcmoe_gguf_close. */
const char *lcmoe_gguf_meta_str(const lcmoe_gguf *g, const char *key);

/* GGUFile::get_tensor_info + get_tensor_raw (gguf.rs:121-131): the first
 * tensor of that name.  dims[4] lists ne0 (fastest) first, 1-padded; data /
 * bytes are NULL / 0 for a GGUF type whose block size this library does not
 * know.  Any output pointer may be NULL. */
lcmoe_status lcmoe_gguf_tensor(const lcmoe_gguf *g, const char *name, int32_t *type,
                               int32_t *n_dims, int64_t *dims, const uint8_t **data,
                               uint64_t *bytes);

/* <general.architecture>.block_count, else 1 + the largest N of the blk.N.*
 * tensor names (0 if none); -1 for g == NULL. */
int32_t lcmoe_gguf_block_count(const lcmoe_gguf *g);
/* 1 if blk.<layer>.ffn_gate_inp.weight exists, else 0. */
int32_t lcmoe_gguf_is_moe_layer(const lcmoe_gguf *g, int32_t layer);

/* Descriptor and weights of MoE layer `layer`, ready for lcmoe_create: the
 * MoE counterpart of load_layer (rust/src/model/loader.rs:145-168), whose
 * architecture table maps dense FFN tensors only
 * (rust/src/model/arch.rs:83-96).  Reads blk.<layer>.ffn_gate_inp.weight
 * (router, F32/F16/BF16, transposed into the [d, E] form lcmoe_weights
 * takes), the stacked ffn_{gate,up,down}_exps.weight tensors (or per-expert
 * ffn_{gate,up,down}.<e>.weight), optional ffn_{gate,up,down}_shexp.weight
 * (2D: one shared expert; 3D: dims[2] of them), optional exp_probs_b.bias
 * (sigmoid gating) or ffn_gate_inp.bias (softmax gating), and the metadata
 * <arch>.expert_used_count (required), expert_gating_func,
 * expert_weights_norm, expert_weights_scale, expert_group_count and
 * expert_group_used_count; shapes are cross-checked against expert_count,
 * embedding_length and expert_feed_forward_length where present.  The
 * descriptor is validated as lcmoe_create would.  Expert pointers point into
 * the mapping (stacked form) or into copies the handle owns; router and bias
 * are handle-owned f32 copies.  They stay valid until lcmoe_gguf_close or
 * the next call for the same layer.  Unsupported layouts (a gated shared
 * expert, ffn_gate_inp_shexp) return LCMOE_ERR_UNSUPPORTED. */
lcmoe_status lcmoe_gguf_moe_layer(lcmoe_gguf *g, int32_t layer, int32_t max_tokens,
                                  lcmoe_desc *desc, lcmoe_weights *w);

/* ---- end-to-end decoder model (the MoE FFN's caller) ------------------ */

/* The reference engine's decode path around the MoE FFN, on the GPU:
 * Engine::forward / generate (rust/src/inference/engine.rs:51-132) with the
 * dense ffn_forward call (engine.rs:114) replaced by this library's MoE
 * layer.  Per layer: rms_norm (cpu.rs:49-60) -> attention_forward
 * (attention.rs:37-118: x W_q / W_k / W_v, RoPE, f16 KV cache
 * (cache/mod.rs:33-78), causal softmax attention, x W_o) -> residual ->
 * lcmoe_forward_norm_residual_dev (norm, MoE FFN, residual); then the final
 * rms_norm, the lm_head product of each sequence's last token and greedy
 * sampling (sample_top_p with temperature 0, sampler.rs:8-10: the LAST of
 * equal maxima under f32::total_cmp).  Several sequences (a batch) each keep
 * their own cache. */

/* RoPE positions: the reference rotates token i of each forward call by
 * position i, restarting at 0 on every call (attention.rs:13-17, called with
 * the call's seq_len: a decode token is rotated by 0).  ABSOLUTE rotates by
 * the token's position in its sequence instead. */
enum { LCMOE_ROPE_PER_CALL = 0, LCMOE_ROPE_ABSOLUTE = 1 };

typedef struct {
    int32_t n_layer, d_model, n_head, n_kv_head, head_dim, vocab;
    float rope_theta;      /* rope.freq_base (loader.rs:124-125)          */
    float norm_eps;        /* 1e-5 in the reference (engine.rs:100, :111) */
    int32_t rope_positions;/* LCMOE_ROPE_*                                */
    int32_t attn_type;     /* GGUF type of attn_q/k/v/o, token_embd and
                              output: LCMOE_TYPE_Q4_K, _Q8_0 or _F32      */
    int32_t max_batch;     /* sequences decoded together (<= 1024)        */
    int32_t max_prompt;    /* longest prompt (prefilled one sequence per
                              call)                                       */
    int32_t max_ctx;       /* KV cache positions per sequence             */
    lcmoe_desc moe;        /* every layer's MoE FFN; d_model must match;
                              max_tokens is set by the model              */
} lcmoe_model_desc;

/* One decoder layer, GGUF tensors blk.N.* (arch.rs:83-96 names them
 * input_layernorm / self_attn.* / post_attention_layernorm): matrices are
 * [out rows, in cols] with blocks along the input, exactly the GGUF bytes;
 * the norms are f32. */
typedef struct {
    const float *attn_norm;                /* [d]                         */
    const uint8_t *attn_q;                 /* [n_head * head_dim, d]      */
    const uint8_t *attn_k, *attn_v;        /* [n_kv_head * head_dim, d]   */
    const uint8_t *attn_o;                 /* [d, n_head * head_dim]      */
    const float *ffn_norm;                 /* [d]                         */
    lcmoe_weights moe;                     /* as lcmoe_create takes       */
} lcmoe_layer_weights;

typedef struct {
    const uint8_t *token_embd;             /* [vocab, d]                  */
    const float *output_norm;              /* [d]                         */
    const uint8_t *output;                 /* lm_head [vocab, d]; NULL =
                                              tied to token_embd, as
                                              load_special does without
                                              output.weight (loader.rs:
                                              193-199)                    */
    const lcmoe_layer_weights *layers;     /* n_layer of them             */
} lcmoe_model_weights;

typedef struct lcmoe_model lcmoe_model;

/* Engine::load's resident counterpart: validates, uploads every tensor once
 * (each layer's MoE through lcmoe_create) and allocates the KV caches of
 * max_batch sequences.  The caller keeps ownership of the host bytes.  Every
 * tensor is sanitised as load_layer / load_special do (loader.rs:161, :188,
 * :241-249; see lcmoe_sanitize_blocks); a Q4_K tensor with an outlier that
 * Q4_K cannot hold as zero is stored as its sanitised f32 dequantisation. */
lcmoe_status lcmoe_model_create(const lcmoe_model_desc *desc, const lcmoe_model_weights *w,
                                lcmoe_model **out);
void lcmoe_model_destroy(lcmoe_model *m);
/* KVCache::clear (cache/mod.rs:27-31) for every sequence. */
lcmoe_status lcmoe_model_reset(lcmoe_model *m);
/* Engine::forward (engine.rs:78-132) for sequences 0 .. B-1, each taking
 * its T tokens tokens[b * T .. b * T + T) after what its cache holds;
 * logits [B, vocab] of each sequence's last token.  Host buffers,
 * synchronous.  T == 1 runs the batch together; T > 1 one sequence at a
 * time (T <= max_prompt).  An id outside [0, vocab) embeds as zeros
 * (engine.rs:138). */
lcmoe_status lcmoe_model_forward(lcmoe_model *m, const int32_t *tokens, int32_t B, int32_t T,
                                 float *logits);
/* A forward or generate that fails after enqueueing device work leaves the
 * model refusing lcmoe_model_forward with LCMOE_ERR_STATE until
 * lcmoe_model_reset (the cache lengths on the device may have advanced);
 * lcmoe_model_generate resets by itself. */
/* Engine::generate (engine.rs:51-76) with greedy sampling for B sequences
 * of P prompt tokens each (prompt [B, P]): reset, prefill each sequence,
 * then n_new - 1 batched decode steps (one captured HIP graph, replayed).
 * out [B, n_new] receives the generated ids; n_out[b] (optional) the count
 * up to and including the first `eos` (the reference stops at id 2; pass -1
 * to never stop).  P + n_new - 1 <= max_ctx. */
lcmoe_status lcmoe_model_generate(lcmoe_model *m, const int32_t *prompt, int32_t B, int32_t P,
                                  int32_t n_new, int32_t eos, int32_t *out, int32_t *n_out);
/* Decode steps of lcmoe_model_generate as one captured HIP graph (enable =
 * 1, the default) or as eager launches (0: for callers that capture the
 * call into a graph of their own, and for tools that cannot trace
 * graph-launched kernels).  Results are identical either way. */
lcmoe_status lcmoe_model_set_decode_graph(lcmoe_model *m, int32_t enable);
/* Device time of the last lcmoe_model_generate: prefill (all sequences)
 * and decode (all steps), milliseconds, from HIP events on its stream. */
lcmoe_status lcmoe_model_last_timing(lcmoe_model *m, double *prefill_ms, double *decode_ms);

/* ---- shard-layout quantised GEMM -------------------------------------- */

/* C[m,n] = A[m,k] B[k,n] for the shard engine's quantised matrices: the
 * Q8_0 / Q4_0 arms of Tensor::matmul (rust/src/model/tensor.rs:118-128),
 * which call q8_0_matmul / q4_0_matmul (rust/src/kernels/int8_gemm.rs
 * :172-194, :336-358).  B is k rows of n/32 blocks along n, row-major: type
 * LCMOE_TYPE_Q8_0 = 34-byte blocks (f16 scale, 32 int8; q8_0.rs:24-32),
 * LCMOE_TYPE_Q4_0 = the shard engine's 18-byte blocks (f16 scale, 16 bytes,
 * element 2t the low nibble of byte t and 2t+1 the high one, minus 8;
 * q4_0.rs:27-46 -- not GGUF's Q4_0 order).  A and C are row-major f32.
 * Results are bit-identical to the reference's x86 path
 * (q8_0_matmul_avx2_inner :47-98 and its Q4_0 twin :240-290): per output,
 * c = fma(a[i,l], q * scale, c) for l = 0 .. k-1 from 0.  n % 32 == 0,
 * 0 <= m <= 524280, k >= 0.  Host buffers, synchronous (B is copied to
 * the device on every call). */
lcmoe_status lcmoe_shard_matmul(int32_t type, const float *a, const uint8_t *b, float *c,
                                int32_t m, int32_t k, int32_t n);
/* Device buffers, enqueued on `stream` (NULL: the null stream); B resident. */
lcmoe_status lcmoe_shard_matmul_dev(int32_t type, const float *a_dev, const uint8_t *b_dev,
                                    float *c_dev, int32_t m, int32_t k, int32_t n, void *stream);

/* lcmoe_shard_matmul_dev with k split into k_split slices (1..64, at most
 * k) run in parallel: each slice an in-order fma chain over its ceil(k /
 * k_split) rows into `workspace` (k_split * m * n floats, device, 4-byte
 * aligned), then the slices added in slice order.  Deterministic and within
 * float rounding of the exact product, but not bit-identical to the
 * reference (k_split = 1 is, and then needs no workspace).  No counterpart
 * in the reference: it is this library's faster variant of
 * q8_0_matmul / q4_0_matmul (int8_gemm.rs:172-194, :336-358) for callers
 * that accept reassociation. */
lcmoe_status lcmoe_shard_matmul_split_dev(int32_t type, const float *a_dev, const uint8_t *b_dev,
                                          float *c_dev, int32_t m, int32_t k, int32_t n,
                                          int32_t k_split, float *workspace, void *stream);

/* lcmoe_shard_matmul_split_dev without the workspace argument, for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  No counterpart in the
 * reference.  The k-slice planes live in a static device array of
 * LCMOE_SHARD_SCRATCH_FLOATS floats (16 MiB) that each GPU holds until the
 * process ends; a call whose slices need more (S * m * n floats, S the slice
 * count the k_split rule below gives, S > 1) returns LCMOE_ERR_INVALID_ARG.
 * The call allocates nothing.  All calls on one GPU share its array: calls
 * that overlap in time on one GPU (two streams, two threads) race and must
 * be ordered by the caller.  Same results as lcmoe_shard_matmul_split_dev
 * with the same k_split. */
#define LCMOE_SHARD_SCRATCH_FLOATS (4 * 1024 * 1024)
lcmoe_status lcmoe_shard_matmul_split_noalloc_dev(int32_t type, const float *a_dev,
                                                  const uint8_t *b_dev, float *c_dev, int32_t m,
                                                  int32_t k, int32_t n, int32_t k_split,
                                                  void *stream);

/* ---- f32 matrix product: the Backend::matmul operator ----------------- */

/* C[m,n] = A[m,k] B[k,n], f32 row-major: Backend::matmul
 * (rust/src/backend/mod.rs:18-46) for a HIP backend in place of WgpuBackend
 * (rust/src/backend/wgpu.rs:152-237, whose WGSL shader rounds in its own
 * order and falls back to the CPU below 256^3).  Bit-identical to
 * CpuBackend::matmul on x86 (rust/src/backend/cpu.rs:13-23 ->
 * avx2_matmul, rust/src/kernels/simd.rs:226-249): for the first
 * 8 * floor(n / 8) columns each output is an in-order fma chain over k from
 * 0, the n % 8 tail columns add rounded products.  m, k, n >= 0,
 * m <= 524280.  Host buffers, synchronous (the operands are copied to the
 * device and C back on every call, as the trait's slice-in / Vec-out
 * interface has it). */
lcmoe_status lcmoe_matmul_f32(const float *a, const float *b, float *c, int32_t m, int32_t k,
                              int32_t n);
/* Device buffers (4-byte aligned), enqueued on `stream` (NULL: the null
 * stream); returns without waiting. */
lcmoe_status lcmoe_matmul_f32_dev(const float *a_dev, const float *b_dev, float *c_dev, int32_t m,
                                  int32_t k, int32_t n, void *stream);

/* ---- device self-tests (need a GPU; used by the parity tests) ---------- */

/* Decode `count` elements of a GGUF tensor with the device decoders and
 * return them as f32 (bit-exact with dequantize_* in kernels/mod.rs). */
lcmoe_status lcmoe_debug_dequant(int32_t type, const uint8_t *data, int64_t count, float *out);
/* The device RMSNorm (rows of x [T, d], d % 4 == 0), for bit parity with
 * CpuBackend::rms_norm (rust/src/backend/cpu.rs:49-60). */
lcmoe_status lcmoe_debug_rmsnorm(const float *x, const float *w, float eps, int32_t T, int32_t d,
                                 float *out);
/* The router's sigmoid evaluated on the device, for host/device bit parity. */
lcmoe_status lcmoe_debug_sigmoid(const float *x, int64_t n, float *out);
/* HBM streaming-read rate: reads `slice_bytes` (a multiple of 16 MiB, at
 * most 1 GiB) of a 4 GiB device buffer per launch with a plain 16-byte-load
 * kernel, each launch a different slice (past the 256 MB MALL), `reps`
 * launches after two unmeasured ones; *gbps = bytes / mean launch time by
 * HIP events.  The practical ceiling the expert kernels are compared with.
 * No counterpart in the reference. */
lcmoe_status lcmoe_debug_read_bandwidth(int64_t slice_bytes, int32_t reps, double *gbps);
/* Tokens of the handle's last forward whose expert selection the certified
 * router with parallel float64 bounds (the sigmoid-group kind's, and the
 * softmax kinds' at one token with 32 or more experts) left to the exact
 * chain logits (their bounds could not order the decision); -1 when that
 * forward did not use it.  Waits for the forward.  No counterpart in the
 * reference: it observes which of two bit-identical routes ran. */
lcmoe_status lcmoe_debug_route_fallbacks(lcmoe_handle *h, int32_t *count);

/* Testing of the error path only (no counterpart in the reference): the
 * model's n-th internal forward from now on (0-based; one per prefilled
 * sequence, one per decode step or graph capture) fails before enqueueing
 * anything; n < 0 cancels. */
lcmoe_status lcmoe_model_debug_fail_forward(lcmoe_model *m, int32_t n);

/* Observation only (no counterpart in the reference): layer `layer`'s MoE
 * handle, owned by the model, for lcmoe_get_dispatch (the routing of that
 * layer's most recent forward).  Not to be destroyed or run by the caller. */
lcmoe_status lcmoe_model_debug_layer_moe(lcmoe_model *m, int32_t layer, lcmoe_handle **out);

#ifdef __cplusplus
}
#endif
#endif
