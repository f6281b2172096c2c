// The end-to-end decoder model (lcmoe_model_*, include/lcmoe.h): the
// reference engine's forward and greedy generation
// (rust/src/inference/engine.rs:51-132) on one GPU, with every layer's FFN
// through the MoE layer (lcmoe_forward_norm_residual_dev).  Weights are
// resident from lcmoe_model_create; each sequence of a batch keeps its own
// f16 KV cache.  A decode step reads the cache lengths and the previous
// tokens from device memory, so its launch sequence never changes: it is
// captured once into a HIP graph and replayed for every step.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <new>
#include <vector>

#include "kernels.h"
#include "lcmoe_internal.h"

using namespace lcmoe;

#define HIP_TRY(expr)                                                                    \
    do {                                                                                 \
        hipError_t e_ = (expr);                                                          \
        if (e_ != hipSuccess)                                                            \
            return fail(LCMOE_ERR_HIP, "%s: %s", #expr, hipGetErrorString(e_));          \
    } while (0)

struct lcmoe_model {
    lcmoe_model_desc desc{};
    int device = 0;
    hipStream_t stream = nullptr;
    std::vector<void *> allocs;
    struct Layer {
        uint8_t *wqkv = nullptr, *wo = nullptr;  // q, k, v rows stacked; o
        int qt_qkv = 0, qt_o = 0;                // stored types (f32 after a sanitising conversion)
        // the same Q4_K matrices in the RPL64 layout for the matrix-core
        // linears of batches (null where the shapes do not fit)
        uint8_t *wqkv_r = nullptr, *wo_r = nullptr;
        float *attn_norm = nullptr;
        lcmoe_handle *moe = nullptr;
    };
    std::vector<Layer> layers;
    uint8_t *embd = nullptr, *out_w = nullptr, *out_r = nullptr;
    int qt_embd = 0, qt_out = 0;  // stored types of token_embd and output
    _Float16 *x16 = nullptr, *xs16 = nullptr;  // activations of the matrix-core linears
    float *lpart = nullptr;                    // their K-slice partials
    float *out_norm = nullptr, *freq = nullptr;
    _Float16 *kc = nullptr, *vc = nullptr;  // [layer][seq][ctx][kv head][head_dim]
    int32_t *lens = nullptr, *step = nullptr, *tok = nullptr, *next = nullptr, *out_tok = nullptr;
    float *hidden = nullptr, *xn = nullptr, *qkv = nullptr, *qr = nullptr, *attn = nullptr,
          *part = nullptr, *logits = nullptr;
    int tmax = 0;                  // tokens per internal forward
    std::vector<int32_t> lens_h;   // host mirror of lens (every update goes through here)
    // set when a forward failed after enqueueing work: the device lengths
    // may have advanced past lens_h, so every call but reset is refused
    bool needs_reset = false;
    int fail_at = -1;  // testing: internal forward number that fails (lcmoe_model_debug_fail_forward)
    hipGraphExec_t graph = nullptr;
    int graph_B = 0;
    bool use_graph = true;
    hipEvent_t ev[4] = {nullptr, nullptr, nullptr, nullptr};  // start, prefilled, decode, end
    double prefill_ms = 0, decode_ms = 0;
};

namespace {

template <class T>
lcmoe_status alloc_n(lcmoe_model *m, T **p, size_t n) {
    void *v = nullptr;
    hipError_t e = hipMalloc(&v, std::max<size_t>(n * sizeof(T), 256));
    if (e != hipSuccess) {
        (void)hipGetLastError();
        *p = nullptr;
        return fail(e == hipErrorOutOfMemory ? LCMOE_ERR_OUT_OF_MEMORY : LCMOE_ERR_HIP,
                    "hipMalloc(%zu): %s", n * sizeof(T), hipGetErrorString(e));
    }
    m->allocs.push_back(v);
    *p = static_cast<T *>(v);
    return LCMOE_OK;
}

template <class T>
lcmoe_status upload(lcmoe_model *m, T **dst, const void *src, size_t bytes) {
    lcmoe_status st = alloc_n(m, reinterpret_cast<uint8_t **>(dst), bytes);
    if (st) return st;
    HIP_TRY(hipMemcpy(*dst, src, bytes, hipMemcpyHostToDevice));
    return LCMOE_OK;
}

void free_model(lcmoe_model *m) {
    if (!m) return;
    (void)hipSetDevice(m->device);
    if (m->stream) (void)hipStreamSynchronize(m->stream);
    if (m->graph) (void)hipGraphExecDestroy(m->graph);
    for (auto &L : m->layers)
        if (L.moe) lcmoe_destroy(L.moe);
    for (void *p : m->allocs) (void)hipFree(p);
    for (hipEvent_t e : m->ev)
        if (e) (void)hipEventDestroy(e);
    if (m->stream) (void)hipStreamDestroy(m->stream);
    delete m;
}

bool attn_type_ok(int t) {
    return t == LCMOE_TYPE_Q4_K || t == LCMOE_TYPE_Q8_0 || t == LCMOE_TYPE_F32;
}

// One GGUF tensor of `qt`, the concatenation of `parts` (whole blocks each),
// sanitised as load_layer / load_special sanitise every tensor
// (rust/src/model/loader.rs:161, :188, :241-249): outliers zero-coded in
// place where the type holds a zero (lcmoe_sanitize_blocks), otherwise the
// whole tensor becomes its sanitised f32 dequantisation.  `out` receives
// the bytes to upload; returns their type.
int sanitized_tensor(int qt, std::initializer_list<std::pair<const void *, int64_t>> parts,
                     std::vector<uint8_t> &out) {
    int64_t count = 0;
    out.clear();
    for (const auto &p : parts) {
        const size_t bytes = lcmoe_tensor_size(qt, p.second);
        const uint8_t *b = static_cast<const uint8_t *>(p.first);
        out.insert(out.end(), b, b + bytes);
        count += p.second;
    }
    int64_t unz = 0;
    if (count_outliers(qt, out.data(), count, &unz) == 0) return qt;
    if (unz == 0) {
        lcmoe_sanitize_blocks(qt, out.data(), count, nullptr);
        return qt;
    }
    std::vector<uint8_t> f((size_t)count * 4);
    lcmoe_dequantize(qt, out.data(), count, reinterpret_cast<float *>(f.data()), 1);
    out.swap(f);
    return LCMOE_TYPE_F32;
}

lcmoe_status validate(const lcmoe_model_desc *d, const lcmoe_model_weights *w) {
    if (!d || !w || !w->token_embd || !w->output_norm || !w->layers)
        return fail(LCMOE_ERR_INVALID_ARG, "desc, weights or a model tensor is NULL");
    if (d->n_layer < 1 || d->n_layer > 4096)
        return fail(LCMOE_ERR_INVALID_ARG, "n_layer=%d outside [1, 4096]", d->n_layer);
    if (d->d_model != d->moe.d_model)
        return fail(LCMOE_ERR_INVALID_ARG, "d_model=%d differs from moe.d_model=%d", d->d_model,
                    d->moe.d_model);
    if (d->n_head < 1 || d->n_kv_head < 1 || d->n_head % d->n_kv_head)
        return fail(LCMOE_ERR_INVALID_ARG, "n_head=%d must be a positive multiple of n_kv_head=%d",
                    d->n_head, d->n_kv_head);
    if (d->head_dim < 16 || d->head_dim > 256 || d->head_dim % 16)
        return fail(LCMOE_ERR_INVALID_ARG, "head_dim=%d must be a multiple of 16 in [16, 256]",
                    d->head_dim);
    if (d->vocab < 1) return fail(LCMOE_ERR_INVALID_ARG, "vocab=%d", d->vocab);
    if (!attn_type_ok(d->attn_type))
        return fail(LCMOE_ERR_UNSUPPORTED, "attn_type=%d (Q4_K, Q8_0 or F32)", d->attn_type);
    const int64_t bs = block_size(d->attn_type);
    const int64_t qd = (int64_t)d->n_head * d->head_dim;
    if (d->d_model % bs || qd % bs || qd % 8 || d->d_model % 8)
        return fail(LCMOE_ERR_INVALID_ARG,
                    "d_model=%d and n_head*head_dim=%lld must be whole blocks of %lld", d->d_model,
                    (long long)qd, (long long)bs);
    if (!(d->rope_theta > 0.0f) || !std::isfinite(d->rope_theta))
        return fail(LCMOE_ERR_INVALID_ARG, "rope_theta must be finite and > 0");
    if (!(d->norm_eps >= 0.0f) || !std::isfinite(d->norm_eps))
        return fail(LCMOE_ERR_INVALID_ARG, "norm_eps must be finite and >= 0");
    if (d->rope_positions != LCMOE_ROPE_PER_CALL && d->rope_positions != LCMOE_ROPE_ABSOLUTE)
        return fail(LCMOE_ERR_INVALID_ARG, "rope_positions=%d", d->rope_positions);
    if (d->max_batch < 1 || d->max_batch > 1024)
        return fail(LCMOE_ERR_INVALID_ARG, "max_batch=%d outside [1, 1024]", d->max_batch);
    if (d->max_ctx < 1 || d->max_prompt < 1 || d->max_prompt > d->max_ctx)
        return fail(LCMOE_ERR_INVALID_ARG, "need 1 <= max_prompt=%d <= max_ctx=%d", d->max_prompt,
                    d->max_ctx);
    if (std::max(d->max_prompt, d->max_batch) > 65536)
        return fail(LCMOE_ERR_INVALID_ARG, "max_prompt and max_batch must be <= 65536");
    for (int l = 0; l < d->n_layer; l++) {
        const lcmoe_layer_weights &L = w->layers[l];
        if (!L.attn_norm || !L.ffn_norm || !L.attn_q || !L.attn_k || !L.attn_v || !L.attn_o)
            return fail(LCMOE_ERR_INVALID_ARG, "layer %d: an attention tensor or norm is NULL", l);
    }
    return LCMOE_OK;
}

// Rows [q0, q0 + nq) of the batch forward.  nseq sequences starting at seq0
// take T tokens each from tok (nseq == 1 or T == 1); their last tokens'
// logits land in m->logits rows 0 .. nseq-1, the greedy ids in m->next
// (and, with rec, in m->out_tok at column *m->step); the cache lengths
// advance by T and *m->step by dstep.
lcmoe_status forward_dev(lcmoe_model *m, int seq0, int nseq, int T, const int32_t *tok, bool rec,
                         int dstep) {
    if (m->fail_at >= 0 && m->fail_at-- == 0)
        return fail(LCMOE_ERR_STATE, "forward failure requested by lcmoe_model_debug_fail_forward");
    const lcmoe_model_desc &D = m->desc;
    const int d = D.d_model, H = D.n_head, KVH = D.n_kv_head, hd = D.head_dim, V = D.vocab;
    const int nq = nseq * T, nqkv = (H + 2 * KVH) * hd;
    const int64_t cache_layer = (int64_t)D.max_batch * D.max_ctx * KVH * hd;
    hipStream_t st = m->stream;
    // Y (= or R +) X W^T over `rows` rows of X (ld K): the matrix-core linear
    // for batches of rows when W has its RPL64 copy, else launch_linear
    auto linear = [&](int wt, const uint8_t *W, const uint8_t *Wr, int N, int K, const float *X,
                      int rows, const float *R, float *Y, int64_t ldy) {
        if (Wr && rows >= 2)
            return launch_linear_mfma(Wr, N, K, X, rows, R, Y, ldy, m->x16, m->xs16, m->lpart, st);
        return launch_linear(wt, W, N, K, X, K, rows, R, Y, ldy, st);
    };
    HIP_TRY(launch_embed(m->qt_embd, m->embd, V, d, tok, nq, m->hidden, st));
    for (int l = 0; l < D.n_layer; l++) {
        const auto &L = m->layers[l];
        _Float16 *kc = m->kc + l * cache_layer, *vc = m->vc + l * cache_layer;
        // Batches on the matrix-core linears: the attention norm also writes
        // the QKV projection's f16 pieces, RoPE adds the projection's K
        // slices as it reads them, and the attention's combine writes the
        // output projection's pieces (no launches of their own).
        const bool mq = L.wqkv_r && nq >= 2;
        const bool mo = L.wo_r && nq >= 2 && hd % 32 == 0 && hd <= 256;  // whole sub-blocks per head
        HIP_TRY(launch_rmsnorm(m->hidden, L.attn_norm, D.norm_eps, nq, d, m->xn, st,
                               mq ? m->x16 : nullptr, m->xs16));
        int ks = 1;
        if (mq)
            HIP_TRY(launch_linear_mfma(L.wqkv_r, nqkv, d, nullptr, nq, nullptr, m->qkv, nqkv,
                                       m->x16, m->xs16, m->lpart, st, true, &ks));
        else
            HIP_TRY(linear(L.qt_qkv, L.wqkv, nullptr, nqkv, d, m->xn, nq, nullptr, m->qkv, nqkv));
        HIP_TRY(launch_rope_kv(ks > 1 ? m->lpart : m->qkv, nq, T, seq0, m->lens, H, KVH, hd,
                               m->freq, D.rope_positions == LCMOE_ROPE_ABSOLUTE, m->qr, kc, vc,
                               D.max_ctx, st, ks, (int64_t)nq * nqkv));
        HIP_TRY(launch_attention(m->qr, nq, T, seq0, m->lens, H, KVH, hd, kc, vc, D.max_ctx,
                                 m->part, m->attn, st, mo ? m->x16 : nullptr, m->xs16));
        // hidden += attn W_o (Tensor::add, engine.rs:106)
        if (mo)
            HIP_TRY(launch_linear_mfma(L.wo_r, d, H * hd, nullptr, nq, m->hidden, m->hidden, d,
                                       m->x16, m->xs16, m->lpart, st, true));
        else
            HIP_TRY(linear(L.qt_o, L.wo, L.wo_r, d, H * hd, m->attn, nq, m->hidden, m->hidden, d));
        // hidden += ffn(rms_norm(hidden)) (engine.rs:109-115)
        lcmoe_status s = lcmoe_forward_norm_residual_dev(L.moe, m->hidden, nq, m->hidden, st);
        if (s) return s;
    }
    // the final norm and lm_head of each sequence's last token
    const float *last = m->hidden + (int64_t)(T - 1) * d;  // nseq == 1, or T == 1
    HIP_TRY(launch_rmsnorm(last, m->out_norm, D.norm_eps, nseq, d, m->xn, st));
    HIP_TRY(linear(m->qt_out, m->out_w, m->out_r, V, d, m->xn, nseq, nullptr, m->logits, V));
    HIP_TRY(launch_argmax(m->logits, nseq, V, seq0, m->next, rec ? m->out_tok : nullptr,
                          D.max_ctx, m->step, st));
    HIP_TRY(launch_advance(m->lens, seq0, nseq, T, m->step, dstep, st));
    return LCMOE_OK;
}

lcmoe_status set_step(lcmoe_model *m, int32_t v) {
    HIP_TRY(hipMemcpyAsync(m->step, &v, 4, hipMemcpyHostToDevice, m->stream));
    HIP_TRY(hipStreamSynchronize(m->stream));
    return LCMOE_OK;
}

lcmoe_status reset(lcmoe_model *m) {
    // drain whatever a failed call left queued before rewriting the lengths
    HIP_TRY(hipStreamSynchronize(m->stream));
    std::fill(m->lens_h.begin(), m->lens_h.end(), 0);
    HIP_TRY(hipMemcpyAsync(m->lens, m->lens_h.data(), 4 * m->lens_h.size(), hipMemcpyHostToDevice,
                           m->stream));
    lcmoe_status st = set_step(m, 0);
    if (!st) m->needs_reset = false;
    return st;
}

// A call that fails after enqueueing device work may leave the device cache
// lengths ahead of lens_h (the host check of capacity): the model then
// refuses every call but lcmoe_model_reset.
lcmoe_status failed_after_enqueue(lcmoe_model *m, lcmoe_status st) {
    m->needs_reset = true;
    return st;
}

// Engine::generate's device work after the reset: prefill each sequence,
// the batched decode steps (captured once per batch size and replayed),
// the ids copied to `out`; returns after everything finished.
lcmoe_status generate_dev(lcmoe_model *m, const int32_t *prompt, int B, int P, int n_new,
                          int32_t *out) {
    const lcmoe_model_desc &D = m->desc;
    lcmoe_status st;
    hipStream_t s = m->stream;
    HIP_TRY(hipEventRecord(m->ev[0], s));
    for (int b = 0; b < B; b++) {  // Engine::generate's prefill, one sequence per call
        HIP_TRY(hipMemcpyAsync(m->tok, prompt + (size_t)b * P, 4 * (size_t)P,
                               hipMemcpyHostToDevice, s));
        if ((st = forward_dev(m, b, 1, P, m->tok, true, 0))) return st;
    }
    HIP_TRY(hipEventRecord(m->ev[1], s));
    if (n_new > 1) {
        int32_t one = 1;
        HIP_TRY(hipMemcpyAsync(m->step, &one, 4, hipMemcpyHostToDevice, s));
        if (m->use_graph && (!m->graph || m->graph_B != B)) {
            if (m->graph) {
                HIP_TRY(hipGraphExecDestroy(m->graph));
                m->graph = nullptr;
            }
            HIP_TRY(hipStreamSynchronize(s));
            hipGraph_t g = nullptr;
            HIP_TRY(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
            st = forward_dev(m, 0, B, 1, m->next, true, 1);
            hipError_t ec = hipStreamEndCapture(s, &g);
            if (st) {
                if (g) (void)hipGraphDestroy(g);
                return st;
            }
            if (ec != hipSuccess) return fail(LCMOE_ERR_HIP, "graph capture: %s", hipGetErrorString(ec));
            ec = hipGraphInstantiate(&m->graph, g, nullptr, nullptr, 0);
            (void)hipGraphDestroy(g);
            if (ec != hipSuccess) {
                m->graph = nullptr;
                return fail(LCMOE_ERR_HIP, "graph instantiate: %s", hipGetErrorString(ec));
            }
            m->graph_B = B;
        }
    }
    HIP_TRY(hipEventRecord(m->ev[2], s));
    for (int i = 1; i < n_new; i++) {
        if (m->use_graph) {
            HIP_TRY(hipGraphLaunch(m->graph, s));
        } else if ((st = forward_dev(m, 0, B, 1, m->next, true, 1))) {
            return st;
        }
    }
    HIP_TRY(hipEventRecord(m->ev[3], s));
    for (int b = 0; b < B; b++)
        HIP_TRY(hipMemcpyAsync(out + (size_t)b * n_new, m->out_tok + (size_t)b * D.max_ctx,
                               4 * (size_t)n_new, hipMemcpyDeviceToHost, s));
    HIP_TRY(hipStreamSynchronize(s));
    float a = 0, c = 0;
    HIP_TRY(hipEventElapsedTime(&a, m->ev[0], m->ev[1]));
    HIP_TRY(hipEventElapsedTime(&c, m->ev[2], m->ev[3]));
    m->prefill_ms = a;
    m->decode_ms = c;
    return LCMOE_OK;
}

// lcmoe_model_forward's device work: T == 1 as one batch, longer inputs one
// sequence at a time; returns after the logits are on the host.
lcmoe_status forward_tokens(lcmoe_model *m, const int32_t *tokens, int B, int T, float *logits) {
    const int V = m->desc.vocab;
    lcmoe_status st;
    if (T == 1) {
        HIP_TRY(hipMemcpyAsync(m->tok, tokens, 4 * (size_t)B, hipMemcpyHostToDevice, m->stream));
        if ((st = forward_dev(m, 0, B, 1, m->tok, false, 0))) return st;
        HIP_TRY(hipMemcpyAsync(logits, m->logits, 4 * (size_t)B * V, hipMemcpyDeviceToHost,
                               m->stream));
    } else {
        for (int b = 0; b < B; b++) {
            HIP_TRY(hipMemcpyAsync(m->tok, tokens + (size_t)b * T, 4 * (size_t)T,
                                   hipMemcpyHostToDevice, m->stream));
            if ((st = forward_dev(m, b, 1, T, m->tok, false, 0))) return st;
            HIP_TRY(hipMemcpyAsync(logits + (size_t)b * V, m->logits, 4 * (size_t)V,
                                   hipMemcpyDeviceToHost, m->stream));
        }
    }
    HIP_TRY(hipStreamSynchronize(m->stream));
    return LCMOE_OK;
}

}  // namespace

extern "C" lcmoe_status lcmoe_model_create(const lcmoe_model_desc *desc,
                                           const lcmoe_model_weights *w, lcmoe_model **out) {
    clear_error();
    if (!out) return fail(LCMOE_ERR_INVALID_ARG, "out is NULL");
    *out = nullptr;
    lcmoe_status st = validate(desc, w);
    if (st) return st;
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev < 1) {
        (void)hipGetLastError();
        return fail(LCMOE_ERR_HIP, "no HIP device available");
    }
    lcmoe_model *m = new (std::nothrow) lcmoe_model();
    if (!m) return fail(LCMOE_ERR_OUT_OF_MEMORY, "host allocation failed");
    auto bail = [&](lcmoe_status s) {
        free_model(m);
        return s;
    };
    m->desc = *desc;
    const lcmoe_model_desc &D = m->desc;
    if (hipGetDevice(&m->device) != hipSuccess) return bail(fail(LCMOE_ERR_HIP, "hipGetDevice"));
    if (hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking) != hipSuccess)
        return bail(fail(LCMOE_ERR_HIP, "hipStreamCreate failed"));
    for (hipEvent_t &e : m->ev)
        if (hipEventCreate(&e) != hipSuccess) return bail(fail(LCMOE_ERR_HIP, "hipEventCreate"));
    const int d = D.d_model, H = D.n_head, KVH = D.n_kv_head, hd = D.head_dim, V = D.vocab;
    const int qt = D.attn_type;
    m->tmax = std::max(D.max_prompt, D.max_batch);
    // per-pair RoPE frequencies, computed as the reference does (f32 powf)
    std::vector<float> freq(hd / 2);
    for (int i = 0; i < hd / 2; i++)
        freq[i] = 1.0f / std::pow(D.rope_theta, 2.0f * (float)i / (float)hd);
    if ((st = upload(m, &m->freq, freq.data(), 4 * freq.size()))) return bail(st);
    // Every tensor is sanitised on the way up (sanitized_tensor); the tied
    // LM head of load_special (loader.rs:193-199: no output.weight -> the
    // embedding, transposed) is output == NULL: the same [vocab, d] bytes.
    std::vector<uint8_t> host, rpl;
    const void *out_src = w->output ? w->output : w->token_embd;
    m->qt_embd = sanitized_tensor(qt, {{w->token_embd, (int64_t)V * d}}, host);
    if ((st = upload(m, &m->embd, host.data(), host.size()))) return bail(st);
    m->qt_out = sanitized_tensor(qt, {{out_src, (int64_t)V * d}}, host);
    if ((st = upload(m, &m->out_w, host.data(), host.size()))) return bail(st);
    std::vector<float> nw;
    auto upload_norm = [&](float **dst, const float *src) {
        nw.assign(src, src + d);
        lcmoe_sanitize_blocks(LCMOE_TYPE_F32, reinterpret_cast<uint8_t *>(nw.data()), d, nullptr);
        return upload(m, dst, nw.data(), 4 * (size_t)d);
    };
    if ((st = upload_norm(&m->out_norm, w->output_norm))) return bail(st);
    // RPL64 copies of the Q4_K linears for the matrix-core path of batches
    // (of the sanitised bytes; none for a tensor stored as f32)
    const int nqkv = (H + 2 * KVH) * hd;
    auto upload_rpl = [&](uint8_t **dst, const uint8_t *src, int64_t rows, int64_t cols) {
        const size_t bytes = lcmoe_tensor_size(LCMOE_TYPE_Q4_K, cols) * rows;
        rpl.resize(bytes);
        repack_rpl64_q4k(src, rpl.data(), rows, cols);
        return upload(m, dst, rpl.data(), bytes);
    };
    bool any_rpl = false, r_qkv_any = false, r_o_any = false;
    if (m->qt_out == LCMOE_TYPE_Q4_K && linear_mfma_ok(V, d)) {
        if ((st = upload_rpl(&m->out_r, host.data(), V, d))) return bail(st);
        any_rpl = true;
    }
    lcmoe_desc md = D.moe;
    md.max_tokens = m->tmax;
    m->layers.resize(D.n_layer);
    for (int l = 0; l < D.n_layer; l++) {
        const lcmoe_layer_weights &L = w->layers[l];
        auto &ML = m->layers[l];
        ML.qt_qkv = sanitized_tensor(qt, {{L.attn_q, (int64_t)H * hd * d},
                                          {L.attn_k, (int64_t)KVH * hd * d},
                                          {L.attn_v, (int64_t)KVH * hd * d}}, host);
        if ((st = upload(m, &ML.wqkv, host.data(), host.size()))) return bail(st);
        if (ML.qt_qkv == LCMOE_TYPE_Q4_K && linear_mfma_ok(nqkv, d)) {
            if ((st = upload_rpl(&ML.wqkv_r, host.data(), nqkv, d))) return bail(st);
            any_rpl = r_qkv_any = true;
        }
        ML.qt_o = sanitized_tensor(qt, {{L.attn_o, (int64_t)d * H * hd}}, host);
        if ((st = upload(m, &ML.wo, host.data(), host.size()))) return bail(st);
        if (ML.qt_o == LCMOE_TYPE_Q4_K && linear_mfma_ok(d, H * hd)) {
            if ((st = upload_rpl(&ML.wo_r, host.data(), d, H * hd))) return bail(st);
            any_rpl = r_o_any = true;
        }
        if ((st = upload_norm(&ML.attn_norm, L.attn_norm))) return bail(st);
        if ((st = lcmoe_create(&md, &L.moe, &ML.moe))) return bail(st);
        // 24 layers compound each layer's error (and near-tie routing flips
        // follow it): the decoder takes the two-f16 activations
        if ((st = lcmoe_set_act_precision(ML.moe, LCMOE_ACT_F16X2))) return bail(st);
        if ((st = lcmoe_set_norm(ML.moe, L.ffn_norm, D.norm_eps))) return bail(st);
    }
    const int64_t cache = (int64_t)D.n_layer * D.max_batch * D.max_ctx * KVH * hd;
    const int64_t T = m->tmax;
    if ((st = alloc_n(m, &m->kc, cache)) || (st = alloc_n(m, &m->vc, cache)) ||
        (st = alloc_n(m, &m->lens, D.max_batch)) || (st = alloc_n(m, &m->step, 1)) ||
        (st = alloc_n(m, &m->tok, T)) || (st = alloc_n(m, &m->next, D.max_batch)) ||
        (st = alloc_n(m, &m->out_tok, (size_t)D.max_batch * D.max_ctx)) ||
        (st = alloc_n(m, &m->hidden, T * d)) || (st = alloc_n(m, &m->xn, T * d)) ||
        (st = alloc_n(m, &m->qkv, T * (H + 2 * KVH) * hd)) || (st = alloc_n(m, &m->qr, T * H * hd)) ||
        (st = alloc_n(m, &m->attn, T * H * hd)) ||
        (st = alloc_n(m, &m->part, attention_part_floats((int)T, H, hd, D.max_ctx))) ||
        (st = alloc_n(m, &m->logits, (size_t)D.max_batch * V)))
        return bail(st);
    if (any_rpl) {
        const int64_t kmax = std::max<int64_t>(d, (int64_t)H * hd);
        int64_t part = 0;
        if (r_qkv_any) part = std::max(part, linear_mfma_part_floats(nqkv, d, (int)T));
        if (r_o_any) part = std::max(part, linear_mfma_part_floats(d, H * hd, (int)T));
        if (m->out_r) part = std::max(part, linear_mfma_part_floats(V, d, D.max_batch));
        if ((st = alloc_n(m, &m->x16, 2 * T * kmax)) || (st = alloc_n(m, &m->xs16, T * kmax / 16)) ||
            (st = alloc_n(m, &m->lpart, part)))
            return bail(st);
    }
    m->lens_h.assign(D.max_batch, 0);
    if ((st = reset(m))) return bail(st);
    *out = m;
    return LCMOE_OK;
}

extern "C" void lcmoe_model_destroy(lcmoe_model *m) { free_model(m); }

extern "C" lcmoe_status lcmoe_model_reset(lcmoe_model *m) {
    clear_error();
    if (!m) return fail(LCMOE_ERR_INVALID_ARG, "model is NULL");
    HIP_TRY(hipSetDevice(m->device));
    return reset(m);
}

extern "C" lcmoe_status lcmoe_model_forward(lcmoe_model *m, const int32_t *tokens, int32_t B,
                                            int32_t T, float *logits) {
    clear_error();
    if (!m || !tokens || !logits) return fail(LCMOE_ERR_INVALID_ARG, "model, tokens or logits is NULL");
    const lcmoe_model_desc &D = m->desc;
    if (B < 1 || B > D.max_batch) return fail(LCMOE_ERR_INVALID_ARG, "B=%d outside [1, %d]", B, D.max_batch);
    if (T < 1 || T > D.max_prompt) return fail(LCMOE_ERR_INVALID_ARG, "T=%d outside [1, %d]", T, D.max_prompt);
    if (m->needs_reset)
        return fail(LCMOE_ERR_STATE, "an earlier call failed after enqueueing work: lcmoe_model_reset first");
    for (int b = 0; b < B; b++)
        if (m->lens_h[b] + T > D.max_ctx)
            return fail(LCMOE_ERR_INVALID_ARG, "sequence %d: %d cached + %d new > max_ctx=%d", b,
                        m->lens_h[b], T, D.max_ctx);
    HIP_TRY(hipSetDevice(m->device));
    lcmoe_status st = forward_tokens(m, tokens, B, T, logits);
    if (st) return failed_after_enqueue(m, st);
    for (int b = 0; b < B; b++) m->lens_h[b] += T;
    return LCMOE_OK;
}

extern "C" lcmoe_status lcmoe_model_generate(lcmoe_model *m, const int32_t *prompt, int32_t B,
                                             int32_t P, int32_t n_new, int32_t eos, int32_t *out,
                                             int32_t *n_out) {
    clear_error();
    if (!m || !prompt || !out) return fail(LCMOE_ERR_INVALID_ARG, "model, prompt or out is NULL");
    const lcmoe_model_desc &D = m->desc;
    if (B < 1 || B > D.max_batch) return fail(LCMOE_ERR_INVALID_ARG, "B=%d outside [1, %d]", B, D.max_batch);
    if (P < 1 || P > D.max_prompt) return fail(LCMOE_ERR_INVALID_ARG, "P=%d outside [1, %d]", P, D.max_prompt);
    if (n_new < 1 || P + n_new - 1 > D.max_ctx)
        return fail(LCMOE_ERR_INVALID_ARG, "n_new=%d: need 1 <= n_new and P + n_new - 1 <= max_ctx=%d",
                    n_new, D.max_ctx);
    HIP_TRY(hipSetDevice(m->device));
    // generate starts from a cleared cache, so it runs after a failed call
    lcmoe_status st;
    if ((st = reset(m))) return failed_after_enqueue(m, st);
    if ((st = generate_dev(m, prompt, B, P, n_new, out))) return failed_after_enqueue(m, st);
    for (int b = 0; b < B; b++) {
        m->lens_h[b] = P + n_new - 1;
        if (n_out) {
            int n = n_new;
            for (int i = 0; i < n_new; i++)
                if (out[(size_t)b * n_new + i] == eos) {
                    n = i + 1;
                    break;
                }
            n_out[b] = n;
        }
    }
    return LCMOE_OK;
}

extern "C" lcmoe_status lcmoe_model_set_decode_graph(lcmoe_model *m, int32_t enable) {
    clear_error();
    if (!m) return fail(LCMOE_ERR_INVALID_ARG, "model is NULL");
    m->use_graph = enable != 0;
    return LCMOE_OK;
}

extern "C" lcmoe_status lcmoe_model_last_timing(lcmoe_model *m, double *prefill_ms,
                                                double *decode_ms) {
    clear_error();
    if (!m) return fail(LCMOE_ERR_INVALID_ARG, "model is NULL");
    if (prefill_ms) *prefill_ms = m->prefill_ms;
    if (decode_ms) *decode_ms = m->decode_ms;
    return LCMOE_OK;
}

extern "C" lcmoe_status lcmoe_model_debug_fail_forward(lcmoe_model *m, int32_t n) {
    clear_error();
    if (!m) return fail(LCMOE_ERR_INVALID_ARG, "model is NULL");
    m->fail_at = n < 0 ? -1 : n;
    return LCMOE_OK;
}

extern "C" lcmoe_status lcmoe_model_debug_layer_moe(lcmoe_model *m, int32_t layer,
                                                    lcmoe_handle **out) {
    clear_error();
    if (!m || !out) return fail(LCMOE_ERR_INVALID_ARG, "model or out is NULL");
    if (layer < 0 || layer >= m->desc.n_layer)
        return fail(LCMOE_ERR_INVALID_ARG, "layer=%d outside [0, %d)", layer, m->desc.n_layer);
    *out = m->layers[layer].moe;
    return LCMOE_OK;
}
