// C ABI entry points (include/lcmoe.h): resident weights, workspace, and the
// per-forward launch sequence on one stream:
//   router (logits, x limbs, top-k, dispatch) -> gate/up (+SwiGLU) -> down
//   -> combine.
// Layout decisions are made once at lcmoe_create: Q4_K matrices whose rows
// tile by 64 and whose columns are whole super-blocks are repacked to RPL64
// and served by the integer row-per-lane kernels; everything else keeps the
// GGUF layout and the generic kernels.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <new>
#include <thread>
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

namespace {

enum Slot { kSlotRouter, kSlotPrep, kSlotGateUp, kSlotGateUpSh, kSlotDown, kSlotDownSh,
            kSlotCombine, kSlotNorm, kNumSlots };
const char *kSlotNames[kNumSlots] = {"router", "act16", "gateup", "gateup_shared", "down",
                                     "down_shared", "combine", "rmsnorm"};
constexpr int kMaxKSplit = 4;
// largest T * E * d served by the certified per-token router
constexpr int64_t kFastRouterElems = (int64_t)1 << 24;
// largest T * E * d served by the certified sigmoid-group router.  It
// re-reads the router matrix per token, and a token its bounds cannot settle
// (about 2% at DeepSeek-V3 shapes) makes the forward wait for the exact
// chains: past about 24 tokens at those shapes the chain router alone is
// the faster one.
constexpr int64_t kSigRouterElems = (int64_t)1 << 25;
// Softmax routers this wide take the parallel-bounds certified router at one
// token (config 5, E = 60: the fast router's one block reads 491 KB of
// router weights alone).
constexpr int kParallelBoundsMinE = 32;

struct ExpertSet {  // one family of experts (routed or shared)
    int n = 0, F = 0, qt_gu = 0, qt_dn = 0;
    // RPL64 Q4_K gate/up; RPL64 Q4_K down (row-per-lane and matrix-core);
    // RPL64 Q6_K down and split-layout Q4_K down (F an odd multiple of 128),
    // both matrix-core only
    bool rpl_gu = false, rpl_dn = false, q6_dn = false, split_dn = false;
    bool q8 = false;  // RPL64 Q8_0 gate, up and down (row-per-lane only)
    uint8_t *gate = nullptr, *up = nullptr, *down = nullptr;
    int64_t sz_gu = 0, sz_dn = 0;
    // H between the two products: f32 (generic down), int8 limbs (row-per-lane
    // down), f16 hi/lo halves + sub-block sums (matrix-core down)
    float *Hf = nullptr;
    int8_t *hh = nullptr, *hl = nullptr;
    float *hs = nullptr, *hm = nullptr;
    _Float16 *h16 = nullptr, *h16s = nullptr;  // [positions][F/256][hi 256 | lo 256], sums
    uint8_t *hexp = nullptr;  // Q8_0 matrix-core H: [positions][F/32] block exponents
    // down output partials [kmax][positions][d]
    float *Y = nullptr;
    int kmax = 1;
    int64_t positions = 0;
};

}  // namespace

struct lcmoe_handle {
    lcmoe_desc desc{};
    int device = 0;
    hipStream_t stream = nullptr;
    std::vector<void *> allocs;
    float *wrt = nullptr, *bias = nullptr;
    // router in the fast router's lane-chunk order (null when d is not
    // 64 * a power-of-two multiple of 4): element (e, lane*C + 4i + j) at
    // ((e * C/4 + i) * 64 + lane) * 4 + j, C = d / 64
    float *wlc = nullptr;
    ExpertSet routed, shared;
    bool fused = false;  // shared experts stored and launched with the routed ones
    float *x_dev = nullptr, *y_dev = nullptr, *logits = nullptr;
    float *chain_part = nullptr;  // [max_tokens, E] router chain running sums
    float *norm_w = nullptr, *xn = nullptr;  // post-attention RMSNorm weight, normed rows
    float norm_eps = 1e-5f;
    int8_t *xh = nullptr, *xl = nullptr;
    float *xs = nullptr, *xm = nullptr;
    _Float16 *x16 = nullptr, *x16s = nullptr;
    int32_t *topk_idx = nullptr, *counts = nullptr, *offsets = nullptr, *perm = nullptr,
            *inv = nullptr, *touched = nullptr;
    int32_t *pass_slots = nullptr;  // RouterArgs::pass_slots
    float *topk_w = nullptr;
    uint32_t *sync = nullptr;
    // certified sigmoid-group router: bounds, per-token counters and marks
    uint64_t *sig_bnd = nullptr;
    uint32_t *sig_sync = nullptr;
    int32_t *sig_flag = nullptr;
    int last_T = -1;
    bool last_sig = false;  // the last forward used the parallel-bounds certified router
    hipStream_t last_stream = nullptr;
    bool timing = false;
    // matrix-core gate/up products take x as two f16 (hi + lo) instead of
    // one (lcmoe_set_act_precision)
    bool x_lo = false;
    struct Pending { int slot; hipEvent_t a, b; };
    std::vector<Pending> pending;
    std::vector<hipEvent_t> event_pool;
    double t_ms[kNumSlots] = {};
    int64_t t_n[kNumSlots] = {};
};

// Pass slots a forward of T tokens can need: sum over the touched experts of
// ceil(count / 32) < T K / 32 + touched.
static int64_t max_pass_slots(const lcmoe_desc &D, int64_t T) {
    const int64_t A = T * D.n_expert_used;
    return (A + 31) / 32 + std::min<int64_t>(D.n_expert, A);
}

namespace {

lcmoe_status dev_alloc(lcmoe_handle *h, void **p, size_t bytes) {
    *p = nullptr;
    if (bytes == 0) bytes = 256;
    hipError_t e = hipMalloc(p, bytes);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return fail(e == hipErrorOutOfMemory ? LCMOE_ERR_OUT_OF_MEMORY : LCMOE_ERR_HIP,
                    "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
    }
    h->allocs.push_back(*p);
    return LCMOE_OK;
}

template <class T>
lcmoe_status alloc_n(lcmoe_handle *h, T **dst, size_t n) {
    void *p;
    lcmoe_status st = dev_alloc(h, &p, n * sizeof(T));
    *dst = static_cast<T *>(p);
    return st;
}

// Uploads the stacked expert matrices of `src` (sanitised, as stored: see
// SanitizedStack), repacking each to RPL64 (Q4_K, Q6_K or Q8_0, by the stored
// type) when `rpl`, or to the split Q4_K layout when `split` (one expert at a
// time through a host staging buffer).  *sz_out: device bytes per expert.
lcmoe_status upload_stack(lcmoe_handle *h, uint8_t **dst, const SanitizedStack &src, bool rpl,
                          int64_t *sz_out, bool split = false) {
    const int qt = src.qt, n = src.na + src.nb;
    const int64_t rows = src.rows, cols = src.cols;
    const int64_t sz = src.stored_bytes();
    const int64_t dsz = split ? rows / 64 * ((cols + 255) / 256) * (9 * 1024 + 256) : sz;
    *sz_out = dsz;
    lcmoe_status st = alloc_n(h, dst, (size_t)dsz * n);
    if (st) return st;
    const bool as_given =
        qt == src.qt_in && std::none_of(src.fix.begin(), src.fix.end(), [](uint8_t f) { return f; });
    if (!rpl && !split && as_given) {
        HIP_TRY(hipMemcpy(*dst, src.a, (size_t)sz * src.na, hipMemcpyHostToDevice));
        if (src.nb)
            HIP_TRY(hipMemcpy(*dst + (size_t)sz * src.na, src.b, (size_t)sz * src.nb,
                              hipMemcpyHostToDevice));
        return LCMOE_OK;
    }
    std::vector<uint8_t> buf(rpl || split ? (size_t)dsz : 0), sbuf;
    for (int e = 0; e < n; e++) {
        const uint8_t *s = src.get(e, sbuf);
        if (!rpl && !split) {
            HIP_TRY(hipMemcpy(*dst + (size_t)e * sz, s, (size_t)sz, hipMemcpyHostToDevice));
            continue;
        }
        if (split) {  // straddling blocks: one thread (the layout reads across rows)
            repack_rpl64_q4k_split(s, buf.data(), rows, cols);
            HIP_TRY(hipMemcpy(*dst + (size_t)e * dsz, buf.data(), (size_t)dsz,
                              hipMemcpyHostToDevice));
            continue;
        }
        // repack 64-row tiles in parallel
        const int64_t tiles = rows / 64;
        unsigned nth = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
        std::vector<std::thread> th;
        for (unsigned t = 0; t < nth; t++)
            th.emplace_back([&, t] {
                const int64_t NB = cols / 256;
                const bool q6 = qt == LCMOE_TYPE_Q6_K, q8 = qt == LCMOE_TYPE_Q8_0;
                const int64_t tb = NB * (q6 ? 13 * 1024 + 128 : q8 ? 17 * 1024 : 9 * 1024);
                const int64_t bb = q6 ? 210 : q8 ? 272 : 144;  // bytes per row and 256 columns
                for (int64_t rt = t; rt < tiles; rt += nth) {
                    if (q6)
                        repack_rpl64_q6k(s + rt * 64 * NB * bb, buf.data() + rt * tb, 64, cols);
                    else if (q8)
                        repack_rpl64_q8(s + rt * 64 * NB * bb, buf.data() + rt * tb, 64, cols);
                    else
                        repack_rpl64_q4k(s + rt * 64 * NB * bb, buf.data() + rt * tb, 64, cols);
                }
            });
        for (auto &x : th) x.join();
        HIP_TRY(hipMemcpy(*dst + (size_t)e * sz, buf.data(), (size_t)sz, hipMemcpyHostToDevice));
    }
    return LCMOE_OK;
}

void free_handle(lcmoe_handle *h) {
    if (!h) return;
    if (h->stream) (void)hipStreamSynchronize(h->stream);
    for (auto &p : h->pending) {
        (void)hipEventDestroy(p.a);
        (void)hipEventDestroy(p.b);
    }
    for (auto ev : h->event_pool) (void)hipEventDestroy(ev);
    for (void *p : h->allocs) (void)hipFree(p);
    if (h->stream) (void)hipStreamDestroy(h->stream);
    delete h;
}

hipEvent_t take_event(lcmoe_handle *h) {
    if (!h->event_pool.empty()) {
        hipEvent_t e = h->event_pool.back();
        h->event_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

template <class Fn>
hipError_t timed(lcmoe_handle *h, hipStream_t st, int slot, Fn fn) {
    if (!h->timing) return fn();
    hipEvent_t a = take_event(h), b = take_event(h);
    if (!a || !b) return fn();
    (void)hipEventRecord(a, st);
    hipError_t e = fn();
    (void)hipEventRecord(b, st);
    h->pending.push_back({slot, a, b});
    return e;
}

// Column splits of the row-per-lane down product so that small batches
// launch about four blocks per CU (measured: T = 2-3 on config 2 run the down
// launch 10% faster at 4 splits than at 2); each wave keeps >= 2 super-blocks
// (it loads the next while computing the current one).  Config 1 (Q8_0,
// F = 2816: 11 super-blocks) then splits in two: down 10.8 -> 8.4 us at T = 1,
// 25.3 -> 20.1 us at T = 8; configs 2 and 5 are unchanged.
int choose_ksplit(const ExpertSet &s, int d, int active) {
    if (!s.rpl_dn && !s.q6_dn && !s.q8 && !s.split_dn) return 1;
    const int NB = (s.F + 255) / 256, tiles = (d / 64) * std::max(1, active);
    int ks = 1;
    while (ks < s.kmax && tiles * ks < 1024 && NB >= 4 * ks * 2) ks *= 2;
    return ks;
}

// Matrix-core down: 256-row blocks, two resident per CU; split K until
// about two blocks per CU exist, keeping >= 4 super-blocks per split.
int choose_ksplit_mfma(const ExpertSet &s, int d, int active) {
    if (!s.rpl_dn && !s.q6_dn && !s.split_dn) return 1;
    const int NB = (s.F + 255) / 256, blocks = ((d / 64 + 3) / 4) * std::max(1, active);
    int ks = 1;
    while (ks < s.kmax && blocks * ks < 512 && NB >= 4 * ks * 2) ks *= 2;
    return ks;
}

// Q8_0 matrix-core down: one-wave blocks of 16 rows and 16 tokens; split K
// until about eight blocks per CU exist, keeping >= 2 groups of 256 columns
// per split.
int choose_ksplit_q8(const ExpertSet &s, int d, int active) {
    const int NG = s.F / 256, blocks = (d / 16) * std::max(1, active);
    int ks = 1;
    while (ks < s.kmax && blocks * ks < 2048 && NG >= 2 * ks * 2) ks *= 2;
    return ks;
}

// An expert family from its sanitised gate, up and down stacks (experts
// [0, na) routed or shared; fused shared experts as [na, na + nb), stored
// after them).  The layouts follow the stored types.
lcmoe_status setup_set(lcmoe_handle *h, ExpertSet &s, int F, const SanitizedStack &g,
                       const SanitizedStack &u, const SanitizedStack &dn, int64_t positions) {
    const int64_t d = h->desc.d_model;
    const int qgu = g.qt, qdn = dn.qt;
    s.n = g.na;
    s.F = F;
    s.qt_gu = qgu;
    s.qt_dn = qdn;
    s.positions = positions;
    s.rpl_gu = rpl64_ok(qgu, F, d);
    s.rpl_dn = s.rpl_gu && rpl64_ok(qdn, d, F);
    s.q6_dn = s.rpl_gu && rpl64_q6_ok(qdn, d, F);
    s.split_dn = s.rpl_gu && qdn == LCMOE_TYPE_Q4_K && d % 64 == 0 && F % 256 == 128;
    s.q8 = rpl64_q8_ok(qgu, F, d) && rpl64_q8_ok(qdn, d, F);
    s.kmax = s.rpl_dn || s.q6_dn || s.split_dn || s.q8 ? kMaxKSplit : 1;
    int64_t szu = 0;
    lcmoe_status st;
    const bool rgu = s.rpl_gu || s.q8;
    if ((st = upload_stack(h, &s.gate, g, rgu, &s.sz_gu))) return st;
    if ((st = upload_stack(h, &s.up, u, rgu, &szu))) return st;
    if ((st = upload_stack(h, &s.down, dn, s.rpl_dn || s.q6_dn || s.q8, &s.sz_dn, s.split_dn)))
        return st;
    if (s.rpl_dn || s.q6_dn || s.q8 || s.split_dn) {  // limbs for the row-per-lane down
        if ((st = alloc_n(h, &s.hh, positions * F))) return st;
        if ((st = alloc_n(h, &s.hl, positions * F))) return st;
        if ((st = alloc_n(h, &s.hs, positions * F / 32))) return st;
        if ((st = alloc_n(h, &s.hm, positions * F / 32))) return st;
    } else {
        if ((st = alloc_n(h, &s.Hf, positions * F))) return st;
    }
    if (s.q8) {  // H of the Q8_0 matrix-core products: block exponents
        if ((st = alloc_n(h, &s.hexp, positions * F / 32))) return st;
    }
    if (s.rpl_gu || s.q8) {
        // ceil(F / 256) pieces of 512 halves and 8 sum pairs per piece per
        // position; the part past F is never written and stays zero
        const int64_t nkb = (F + 255) / 256;
        if ((st = alloc_n(h, &s.h16, positions * nkb * 512))) return st;
        if ((st = alloc_n(h, &s.h16s, positions * nkb * 16))) return st;
        HIP_TRY(hipMemset(s.h16, 0, sizeof(_Float16) * positions * nkb * 512));
        HIP_TRY(hipMemset(s.h16s, 0, sizeof(_Float16) * positions * nkb * 16));
    }
    return alloc_n(h, &s.Y, (size_t)s.kmax * positions * d);
}

}  // namespace

extern "C" lcmoe_status lcmoe_create(const lcmoe_desc *desc, const lcmoe_weights *w,
                                     lcmoe_handle **out) {
    clear_error();
    if (!out) return fail(LCMOE_ERR_INVALID_ARG, "out is NULL");
    *out = nullptr;
    lcmoe_status st = validate_desc(desc);
    if (st) return st;
    if (desc->type_gate != desc->type_up || (desc->n_shared && desc->type_gate_sh != desc->type_up_sh))
        return fail(LCMOE_ERR_UNSUPPORTED, "gate and up must share a quant type");
    if ((st = scan_weights(desc, w))) return st;

    int ndev = 0;
    hipError_t he = hipGetDeviceCount(&ndev);
    if (he != hipSuccess || ndev < 1) {
        (void)hipGetLastError();
        return fail(LCMOE_ERR_HIP, "no HIP device available (%s)", hipGetErrorString(he));
    }
    lcmoe_handle *h = new (std::nothrow) lcmoe_handle();
    if (!h) return fail(LCMOE_ERR_OUT_OF_MEMORY, "host allocation failed");
    h->desc = *desc;
    const lcmoe_desc &D = h->desc;
    auto bail = [&](lcmoe_status s) {
        free_handle(h);
        return s;
    };
    if (hipGetDevice(&h->device) != hipSuccess) return bail(fail(LCMOE_ERR_HIP, "hipGetDevice failed"));
    if (hipStreamCreateWithFlags(&h->stream, hipStreamNonBlocking) != hipSuccess)
        return bail(fail(LCMOE_ERR_HIP, "hipStreamCreate failed"));

    const int64_t d = D.d_model, E = D.n_expert, K = D.n_expert_used, S = D.n_shared,
                  Tm = D.max_tokens, A = Tm * K;
    // router, transposed to [E, d] so each expert's row is contiguous, and
    // sanitised as load_layer does (loader.rs:161, :241-249)
    {
        std::vector<float> wt((size_t)E * d);
        for (int64_t k = 0; k < d; k++)
            for (int64_t e = 0; e < E; e++) wt[e * d + k] = w->router[k * E + e];
        lcmoe_sanitize_blocks(LCMOE_TYPE_F32, reinterpret_cast<uint8_t *>(wt.data()), E * d, nullptr);
        if ((st = alloc_n(h, &h->wrt, wt.size()))) return bail(st);
        if (hipMemcpy(h->wrt, wt.data(), wt.size() * 4, hipMemcpyHostToDevice) != hipSuccess)
            return bail(fail(LCMOE_ERR_HIP, "router upload failed"));
        if (d % 256 == 0) {
            const int64_t C = d / 64, nc4 = C / 4;
            std::vector<float> wl((size_t)E * d);
            for (int64_t e = 0; e < E; e++)
                for (int64_t l = 0; l < 64; l++)
                    for (int64_t i = 0; i < nc4; i++)
                        for (int64_t j = 0; j < 4; j++)
                            wl[(((e * nc4 + i) * 64 + l) * 4) + j] = wt[e * d + l * C + 4 * i + j];
            if ((st = alloc_n(h, &h->wlc, wl.size()))) return bail(st);
            if (hipMemcpy(h->wlc, wl.data(), wl.size() * 4, hipMemcpyHostToDevice) != hipSuccess)
                return bail(fail(LCMOE_ERR_HIP, "router upload failed"));
        }
    }
    if (D.has_bias) {  // the selection bias is a layer tensor too: sanitised
        std::vector<float> b(w->bias, w->bias + E);
        lcmoe_sanitize_blocks(LCMOE_TYPE_F32, reinterpret_cast<uint8_t *>(b.data()), E, nullptr);
        if ((st = alloc_n(h, &h->bias, E))) return bail(st);
        if (hipMemcpy(h->bias, b.data(), E * 4, hipMemcpyHostToDevice) != hipSuccess)
            return bail(fail(LCMOE_ERR_HIP, "bias upload failed"));
    }
    // Expert matrices, sanitised (sanitize_weights, loader.rs:241-249):
    // outliers zero-coded in place where the type can hold a zero; a family
    // whose Q4_K gate or up (or down) has an outlier that cannot be is
    // stored as f32 for that matrix kind (gate and up share one type).
    auto stack = [](const uint8_t *a, int na, int qt, int64_t rows, int64_t cols) {
        SanitizedStack t;
        t.a = a;
        t.na = na;
        t.qt_in = t.qt = qt;
        t.rows = rows;
        t.cols = cols;
        return t;
    };
    const int64_t F = D.d_ff, FS = D.d_ff_shared;
    SanitizedStack rg = stack(w->gate, (int)E, D.type_gate, F, d),
                   ru = stack(w->up, (int)E, D.type_up, F, d),
                   rd = stack(w->down, (int)E, D.type_down, d, F), sg, su, sd;
    const bool rg_f32 = rg.analyse(), ru_f32 = ru.analyse();  // both scanned: each fills its fix list
    const bool rgu_f32 = rg_f32 || ru_f32;
    if (rgu_f32) rg.qt = ru.qt = LCMOE_TYPE_F32;
    if (rd.analyse()) rd.qt = LCMOE_TYPE_F32;
    if (S > 0) {
        sg = stack(w->gate_sh, (int)S, D.type_gate_sh, FS, d);
        su = stack(w->up_sh, (int)S, D.type_up_sh, FS, d);
        sd = stack(w->down_sh, (int)S, D.type_down_sh, d, FS);
        const bool sg_f32 = sg.analyse(), su_f32 = su.analyse();
        const bool sgu_f32 = sg_f32 || su_f32;
        if (sgu_f32) sg.qt = su.qt = LCMOE_TYPE_F32;
        if (sd.analyse()) sd.qt = LCMOE_TYPE_F32;
    }
    // shared experts of the routed experts' shape and stored types run as
    // extra slots of the routed launches (their positions follow the A
    // routed ones)
    h->fused = S > 0 && FS == F && sg.qt == rg.qt && sd.qt == rd.qt;
    if (h->fused) {
        for (SanitizedStack *p : {&rg, &ru, &rd}) {
            const SanitizedStack &q = p == &rg ? sg : p == &ru ? su : sd;
            p->b = q.a;
            p->nb = q.na;
            p->fix.insert(p->fix.end(), q.fix.begin(), q.fix.end());
        }
        if ((st = setup_set(h, h->routed, (int)F, rg, ru, rd, A + S * Tm))) return bail(st);
    } else {
        if ((st = setup_set(h, h->routed, (int)F, rg, ru, rd, A))) return bail(st);
        if (S > 0 && (st = setup_set(h, h->shared, (int)FS, sg, su, sd, S * Tm))) return bail(st);
    }
    const bool limbs = h->routed.rpl_gu || h->routed.q8 ||
                       (S > 0 && !h->fused && (h->shared.rpl_gu || h->shared.q8));
    if ((st = alloc_n(h, &h->x_dev, Tm * d))) return bail(st);
    if ((st = alloc_n(h, &h->y_dev, Tm * d))) return bail(st);
    if ((st = alloc_n(h, &h->logits, Tm * E))) return bail(st);
    if ((st = alloc_n(h, &h->chain_part, Tm * E))) return bail(st);
    if (limbs) {
        if ((st = alloc_n(h, &h->xh, Tm * d))) return bail(st);
        if ((st = alloc_n(h, &h->xl, Tm * d))) return bail(st);
        if ((st = alloc_n(h, &h->xs, Tm * d / 32))) return bail(st);
        if ((st = alloc_n(h, &h->xm, Tm * d / 32))) return bail(st);
        if ((st = alloc_n(h, &h->x16, 2 * Tm * d))) return bail(st);
        if ((st = alloc_n(h, &h->x16s, Tm * d / 16))) return bail(st);
    }
    if ((st = alloc_n(h, &h->topk_idx, A))) return bail(st);
    if ((st = alloc_n(h, &h->topk_w, A))) return bail(st);
    if ((st = alloc_n(h, &h->counts, E))) return bail(st);
    if ((st = alloc_n(h, &h->offsets, E + 1))) return bail(st);
    if ((st = alloc_n(h, &h->perm, A))) return bail(st);
    if ((st = alloc_n(h, &h->inv, A))) return bail(st);
    if ((st = alloc_n(h, &h->touched, E + 1))) return bail(st);
    if ((st = alloc_n(h, &h->pass_slots, 1 + max_pass_slots(D, Tm)))) return bail(st);
    const int nsync = router_token_groups((int)Tm, (int)d, (int)E) + 1;
    if ((st = alloc_n(h, &h->sync, nsync))) return bail(st);
    if (hipMemset(h->sync, 0, sizeof(uint32_t) * nsync) != hipSuccess)
        return bail(fail(LCMOE_ERR_HIP, "workspace clear failed"));
    if (D.route_kind == LCMOE_ROUTE_SIGMOID_GROUP || E >= kParallelBoundsMinE) {
        if ((st = alloc_n(h, &h->sig_bnd, 2 * Tm * E))) return bail(st);
        if ((st = alloc_n(h, &h->sig_sync, Tm))) return bail(st);
        if ((st = alloc_n(h, &h->sig_flag, Tm))) return bail(st);
        if (hipMemset(h->sig_sync, 0, sizeof(uint32_t) * Tm) != hipSuccess ||
            hipMemset(h->sig_flag, 0, sizeof(int32_t) * Tm) != hipSuccess)
            return bail(fail(LCMOE_ERR_HIP, "workspace clear failed"));
    }
    *out = h;
    return LCMOE_OK;
}

extern "C" void lcmoe_destroy(lcmoe_handle *h) { free_handle(h); }

// Which product kernels serve an expert family this forward.
struct Plan {
    bool mfma;
    bool passes;  // routed slots are pass slots (one 32-token pass each)
    int slots, ks;
    int chunks;  // blocks sharing one matrix-core slot's 32-token passes
    int sl, ns;  // fused shared experts: tokens per slot, slots per expert
    int per_slot;  // average tokens per slot
};


// fused: the routed plan also carries the fused shared experts (slots
// p.slots .. p.slots + n_shared - 1, all T tokens each)
// fused_only: a launch of the fused shared experts alone (no routed slots)
static Plan plan_set(lcmoe_handle *h, const ExpertSet &s, bool shared, int T, int fused = 0,
                     bool fused_only = false) {
    const lcmoe_desc &D = h->desc;
    Plan p;
    if (fused_only) shared = true;
    p.slots = fused_only ? 0 : shared ? s.n : std::min(D.n_expert, T * D.n_expert_used);
    // the matrix-core kernels decode each weight once for up to 32 tokens,
    // the row-per-lane ones once per pass of up to 4 tokens: matrix cores
    // when there are more assignments than experts (T K > E; a shared expert
    // sees every token, so T > 1), and from 4 tokens on.  Measured with one
    // f16 per activation (tokens/s, row-per-lane against matrix cores):
    // config 4 T = 2 / 4 / 16 / 32: 12.0k / 16.1k / 26.8k / 32.5k against
    // 11.5k / 19.0k / 34.1k / 53.1k; config 2 T = 3 / 4: 25.7k / 28.5k
    // against 22.2k / 28.4k; config 5's layer T = 4: 54.0k against 60.2k.
    const int64_t assign = shared ? T : (int64_t)T * D.n_expert_used;
    // Q8_0 sets: the matrix-core kernels take one f16 per activation only,
    // and pay from T K > E on (config 1, row-per-lane against matrix cores:
    // T = 4 / 8 / 12: 39.5 / 53.1 / 61.3 us against 44.8 / 46.8 / 47.0 us)
    const bool mma_ok = s.rpl_gu || (s.q8 && !h->x_lo);
    p.mfma = mma_ok && (shared ? assign > 1
                               : (assign > (int64_t)D.n_expert || (T >= 4 && !s.q8)));
    // passes per slot: all T tokens for a shared expert, the average over
    // the touched experts for the routed ones (busier experts run several
    // passes per block)
    const int64_t per_slot =
        shared ? T : ((int64_t)T * D.n_expert_used + p.slots - 1) / std::max(1, p.slots);
    p.chunks = p.mfma ? (int)std::min<int64_t>(64, std::max<int64_t>(1, (per_slot + 31) / 32)) : 1;
    p.per_slot = (int)std::min<int64_t>(per_slot, INT32_MAX);
    // Routed experts averaging more than one pass, and any batch past 32
    // tokens (an expert can then need several passes although the average
    // is under one: config 4 T = 256, 21 of 137 touched experts hold 33-85
    // tokens): one block per 32-token pass of each touched expert (pass
    // slots from the dispatch), so busy experts spread over the grid instead
    // of leaving their passes to one block after another (config 4 T = 256:
    // gate/up 570 -> 500 us, down 470 -> 447 us).
    p.passes = p.mfma && !shared && (p.chunks > 1 || T > 32) && h->pass_slots;
    if (p.passes) {
        p.slots = (int)max_pass_slots(D, T);
        p.chunks = 1;
    }
    // fused shared experts: slices of the tokens one slot takes (the passes
    // of its chunk blocks, or one row-per-lane pass)
    p.sl = p.mfma ? 32 * p.chunks : 4;
    p.ns = fused ? (T + p.sl - 1) / p.sl : 0;
    const int all = p.slots + fused * p.ns;
    p.ks = p.mfma && s.q8     ? choose_ksplit_q8(s, D.d_model, all * 2 * p.chunks)
           : p.mfma && (s.rpl_dn || s.q6_dn || s.split_dn)
               ? choose_ksplit_mfma(s, D.d_model, all * p.chunks)
               : choose_ksplit(s, D.d_model, all);
    return p;
}

// fused: number of shared experts run as extra slots of this (routed) set;
// fused_only: no routed slots (pl from plan_set(..., fused_only))
static lcmoe_status run_set(lcmoe_handle *h, ExpertSet &s, bool shared, const float *x, int T,
                            const Plan &pl, const ChainArgs &ch, hipStream_t st, int fused = 0,
                            bool fused_only = false) {
    const lcmoe_desc &D = h->desc;
    const int d = D.d_model, K = D.n_expert_used, E = D.n_expert;
    const int A = D.max_tokens * K;  // routed positions; fused shared ones follow
    SlotArgsHost sa{h->perm, h->counts, h->offsets, h->touched, E, K, T, shared ? 1 : 0,
                    pl.slots, fused, fused ? A : INT32_MAX, std::max(1, pl.ns), pl.sl,
                    pl.passes ? h->pass_slots : nullptr};
    const int slots = pl.slots + fused * pl.ns;
    // H between the products in the form the down kernel reads: f16 pieces
    // for the matrix-core downs, int8 limbs for the row-per-lane ones (Q4_K,
    // split Q4_K and Q6_K below one token per expert), f32 for the generic one
    const bool h16_out = pl.mfma && (s.rpl_dn || s.q6_dn || s.split_dn);
    const bool limb_out = !pl.mfma && (s.rpl_dn || s.q6_dn || s.q8 || s.split_dn);
    HIP_TRY(timed(h, st, shared || fused_only ? kSlotGateUpSh : kSlotGateUp, [&] {
        if (pl.mfma && s.q8)
            return launch_mfma_gateup_q8(s.gate, s.up, s.sz_gu, h->x16, sa, slots,
                                         2 * pl.chunks, d, s.F, s.h16, s.hexp, ch, st);
        if (pl.mfma)
            return launch_mfma_gateup(s.gate, s.up, s.sz_gu, h->x16, h->x16s, sa, slots,
                                      pl.chunks, d, s.F, h16_out ? s.h16 : nullptr, s.h16s,
                                      h16_out ? nullptr : s.Hf, ch, st, h->x_lo);
        if (s.rpl_gu || s.q8)
            return launch_rpl_gateup(s.gate, s.up, s.sz_gu, h->xh, h->xl, h->xs, h->xm, sa,
                                     slots, d, s.F, s.Hf, limb_out ? s.hh : nullptr, s.hl,
                                     s.hs, s.hm, h16_out ? s.h16 : nullptr, s.h16s, ch, st, s.q8);
        return launch_generic_gateup(s.qt_gu, s.gate, s.up, s.sz_gu, x, sa, slots, d, s.F,
                                     s.Hf, nullptr, nullptr, nullptr, nullptr, ch, st);
    }));
    HIP_TRY(timed(h, st, shared || fused_only ? kSlotDownSh : kSlotDown, [&] {
        // Q6_K: each expert's passes sized by its own token count (32-token
        // passes decode each weight once for up to 32 tokens, a 16-token one
        // does half the matrix-core work; config 4 T = 256, where the 136
        // touched experts hold 15 tokens on average and the busiest dozens:
        // down 876 us with 16-token passes, 717 with 32-token passes); with
        // two f16 per activation one pass size per launch, by the average
        if (s.q8 && pl.mfma)
            return launch_mfma_down_q8(s.down, s.sz_dn, s.h16, s.hexp, sa, slots, 2 * pl.chunks, d, s.F,
                                       pl.ks, s.Y, s.positions * d, st);
        if (s.q6_dn && pl.mfma)
            return launch_mfma_down_q6(s.down, s.sz_dn, s.h16, sa, slots, pl.chunks, d, s.F,
                                       pl.ks, s.Y, s.positions * d, st, h->x_lo,
                                       pl.per_slot <= 16);
        if (s.q6_dn || s.q8 || (s.split_dn && !pl.mfma))
            return launch_rpl_down(s.down, s.sz_dn, s.hh, s.hl, s.hs, s.hm, sa, slots, d, s.F,
                                   pl.ks, s.Y, s.positions * d, st, s.q8 ? 2 : s.split_dn ? 3 : 1);
        if (s.split_dn || (s.rpl_dn && pl.mfma))
            return launch_mfma_down(s.down, s.sz_dn, s.h16, s.h16s, sa, slots, pl.chunks, d,
                                    s.F, pl.ks, s.Y, s.positions * d, st, h->x_lo);
        if (s.rpl_dn)
            return launch_rpl_down(s.down, s.sz_dn, s.hh, s.hl, s.hs, s.hm, sa, slots, d, s.F,
                                   pl.ks, s.Y, s.positions * d, st);
        return launch_generic_down(s.qt_dn, s.down, s.sz_dn, s.Hf, sa, slots, d, s.F, s.Y, st);
    }));
    return LCMOE_OK;
}

// y = ffn(x), or y = resid + ffn(x) when resid is given (y may be resid).
// With norm_in, x is the handle's norm buffer and receives
// rms_norm(norm_in) first: inside the certified router's entry (each token
// block normalises its own row) for matrix-core batches, otherwise as a
// launch of its own.
static lcmoe_status enqueue_forward(lcmoe_handle *h, const float *x, int32_t T, float *y,
                                    hipStream_t st, const float *resid = nullptr,
                                    const float *norm_in = nullptr) {
    const lcmoe_desc &D = h->desc;
    const int d = D.d_model, E = D.n_expert, K = D.n_expert_used, S = D.n_shared;
    // Fused shared experts ride in the routed launches while every routed
    // slot is one matrix-core block (or a row-per-lane one); past that
    // (prefill) they get launches of their own, which schedule better.
    const int Sf = h->fused ? S : 0;
    const Plan pr0 = plan_set(h, h->routed, false, T);
    const bool together = Sf > 0 && pr0.chunks == 1;
    const int fused = together ? Sf : 0;
    const Plan pr = together ? plan_set(h, h->routed, false, T, Sf) : pr0;
    const Plan off{false, false, 0, 1, 1, 4, 0, 0};
    const Plan pf = Sf > 0 && !together ? plan_set(h, h->routed, false, T, Sf, true) : off;
    const Plan ps = S > 0 && !h->fused ? plan_set(h, h->shared, true, T) : off;
    const bool sep_f = Sf > 0 && !together;
    const bool mfma = pr.mfma || ps.mfma || pf.mfma;
    // int8 limbs only feed the row-per-lane kernels
    const bool limbs = ((h->routed.rpl_gu || h->routed.q8) && (!pr.mfma || (sep_f && !pf.mfma))) ||
                       (S > 0 && !h->fused && (h->shared.rpl_gu || h->shared.q8) && !ps.mfma);
    RouterArgs ra{};
    ra.x = x;
    ra.wrt = h->wrt;
    ra.wlc = h->wlc;
    ra.bias = h->bias;
    ra.T = T;
    ra.d = d;
    ra.E = E;
    ra.K = K;
    ra.rp = RouteParams{D.route_kind, D.n_group, D.topk_group, D.has_bias, D.routed_scale};
    ra.logits = h->logits;
    ra.topk_idx = h->topk_idx;
    ra.topk_w = h->topk_w;
    ra.xh = limbs ? h->xh : nullptr;
    ra.xl = h->xl;
    ra.xs = h->xs;
    ra.xm = h->xm;
    ra.x16 = nullptr;
    ra.x16s = h->x16s;
    ra.x16_lo = h->x_lo;
    ra.counts = h->counts;
    ra.offsets = h->offsets;
    ra.perm = h->perm;
    ra.inv = h->inv;
    ra.touched = h->touched;
    ra.pass_slots = pr.passes ? h->pass_slots : nullptr;
    ra.sync = h->sync;
    // the fast router reads the whole router matrix once per token: past
    // kFastRouterElems multiply-adds per forward the chain router, which
    // reads each router row once per 8 tokens, is the faster one
    // the certified router with parallel float64 bounds (E / 4 blocks per
    // token, the last one certifying): the sigmoid-group kind's, and at one
    // token the softmax kinds' when E >= kParallelBoundsMinE (the fast
    // router's single block would read the whole router matrix alone).  Its
    // weights, like the fast router's, come from the chains and the combine.
    RouterArgs rs = ra;
    rs.bnd = h->sig_bnd;
    rs.tsync = h->sig_sync;
    rs.flag = h->sig_flag;
    const bool par = T == 1 && E >= kParallelBoundsMinE &&
                     D.route_kind != LCMOE_ROUTE_SIGMOID_GROUP && route_sig_ok(rs);
    const bool fast = !par && route_fast_ok(ra) && (int64_t)T * E * d <= kFastRouterElems;
    const bool sig = !fast && route_sig_ok(rs) && (int64_t)T * E * d <= kSigRouterElems;
    // With the certified fast router, selection, dispatch and activations
    // come from it; the exact chains of the routing weights run in extra
    // blocks beside them, and the combine turns the chains into weights.  The
    // chains are sequential: columns [0, kA) run in the router launch, the
    // rest in the routed gate/up launch, which outlasts them.  The
    // row-per-lane and generic gate/up launches of small batches are short,
    // so the router launch takes a share of the chains; the matrix-core one
    // takes them all.
    ChainArgs ch_r{}, ch_g{};
    // The norm fuses into the certified router's entry when the exact chains
    // run wholly in the gate/up launch anyway (matrix-core batches).  For
    // row-per-lane batches the router launch hosts a share of the chains,
    // which read x while a fused norm would still be writing it; there the
    // separate norm launch measured faster (config 2, T = 1: 73 against
    // 78 us per call).
    if (norm_in && fast && pr.mfma) {
        ra.xin = norm_in;
        ra.norm_w = h->norm_w;
        ra.norm_eps = h->norm_eps;
        ra.xn = h->xn;
    } else if (norm_in) {
        HIP_TRY(timed(h, st, kSlotNorm, [&] {
            return launch_rmsnorm(norm_in, h->norm_w, h->norm_eps, T, d, h->xn, st);
        }));
    }
    if (fast) {
        // the router launch's share of the exact chains reads x, which the
        // fused norm is still writing there: all chains go to gate/up then
        const int kA = pr.mfma || ra.xin ? 0 : (d / 4) & ~255;
        if (kA > 0) ch_r = make_chains(x, h->wrt, h->logits, h->chain_part, T, d, E, 0, kA, 8);
        ch_g = make_chains(x, h->wrt, h->logits, h->chain_part, T, d, E, kA, d, 8);
        ra.x16 = mfma ? h->x16 : nullptr;
        HIP_TRY(timed(h, st, kSlotRouter, [&] { return launch_route_fast(ra, ch_r, st); }));
    } else if (sig) {
        // One token: its gate/up launch is short next to the d-long
        // sequential chains (config 4: 37 us of expert streaming against
        // ~57 us of chains), so the router launch runs the first half of the
        // columns beside the bounds; larger batches leave them all to gate/up.
        const int kA = T == 1 ? (d / 2) & ~255 : 0;
        if (kA > 0) ch_r = make_chains(x, h->wrt, h->logits, h->chain_part, T, d, E, 0, kA, 8);
        ch_g = make_chains(x, h->wrt, h->logits, h->chain_part, T, d, E, kA, d, 8);
        rs.x16 = mfma ? h->x16 : nullptr;
        HIP_TRY(timed(h, st, kSlotRouter, [&] { return launch_route_sig(rs, ch_r, st); }));
    } else if (route_chains_ok(ra)) {
        ra.x16 = mfma ? h->x16 : nullptr;
        HIP_TRY(timed(h, st, kSlotRouter, [&] { return launch_route_chains(ra, st); }));
    } else {
        HIP_TRY(timed(h, st, kSlotRouter, [&] { return launch_router(ra, st); }));
        if (mfma)
            HIP_TRY(timed(h, st, kSlotPrep, [&] {
                return launch_act16(x, T, d, h->x16, h->x16s, st, h->x_lo);
            }));
    }
    lcmoe_status s;
    if ((s = run_set(h, h->routed, false, x, T, pr, ch_g, st, fused))) return s;
    if (sep_f && (s = run_set(h, h->routed, false, x, T, pf, ChainArgs{}, st, Sf, true))) return s;
    if (S > 0 && !h->fused && (s = run_set(h, h->shared, true, x, T, ps, ChainArgs{}, st)))
        return s;
    const int ks_r = pr.ks, ks_s = ps.ks;
    CombineRoute cr{};
    if (fast || sig)
        cr = CombineRoute{h->logits, h->topk_idx, D.has_bias ? h->bias : nullptr, D.route_kind,
                          E, D.routed_scale};
    HIP_TRY(timed(h, st, kSlotCombine, [&] {
        // fused shared experts' partials follow the routed positions
        const float *Ys = Sf ? h->routed.Y + (int64_t)D.max_tokens * K * d : h->shared.Y;
        const int64_t ss = Sf ? h->routed.positions * d : h->shared.positions * d;
        const int kss = !Sf ? ks_s : together ? ks_r : pf.ks;
        return launch_combine(h->routed.Y, ks_r, h->routed.positions * d, Ys, kss, ss, h->inv,
                              h->topk_w, T, K, S, d, cr, y, st, resid);
    }));
    h->last_T = T;
    h->last_stream = st;
    h->last_sig = sig;
    return LCMOE_OK;
}

extern "C" lcmoe_status lcmoe_forward_dev(lcmoe_handle *h, const float *x_dev, int32_t T,
                                          float *y_dev, void *stream) {
    clear_error();
    if (!h) return fail(LCMOE_ERR_INVALID_ARG, "handle is NULL");
    if (T < 0 || T > h->desc.max_tokens)
        return fail(LCMOE_ERR_INVALID_ARG, "T=%d outside [0, max_tokens=%d]", T, h->desc.max_tokens);
    if (T > 0 && (!x_dev || !y_dev)) return fail(LCMOE_ERR_INVALID_ARG, "x or y is NULL");
    if (((uintptr_t)x_dev | (uintptr_t)y_dev) & 15)
        return fail(LCMOE_ERR_INVALID_ARG, "x and y must be 16-byte aligned");
    HIP_TRY(hipSetDevice(h->device));
    hipStream_t st = stream ? (hipStream_t)stream : h->stream;
    if (T == 0) {
        h->last_T = 0;
        h->last_stream = st;
        return LCMOE_OK;
    }
    return enqueue_forward(h, x_dev, T, y_dev, st);
}

extern "C" lcmoe_status lcmoe_forward(lcmoe_handle *h, const float *x, int32_t T, float *y,
                                      int32_t *topk_idx, float *topk_w) {
    clear_error();
    if (!h) return fail(LCMOE_ERR_INVALID_ARG, "handle is NULL");
    if (T < 0 || T > h->desc.max_tokens)
        return fail(LCMOE_ERR_INVALID_ARG, "T=%d outside [0, max_tokens=%d]", T, h->desc.max_tokens);
    HIP_TRY(hipSetDevice(h->device));
    if (T == 0) {
        h->last_T = 0;
        h->last_stream = h->stream;
        return LCMOE_OK;
    }
    if (!x || !y) return fail(LCMOE_ERR_INVALID_ARG, "x or y is NULL");
    const size_t xb = sizeof(float) * (size_t)T * h->desc.d_model;
    const size_t kb = (size_t)T * h->desc.n_expert_used;
    HIP_TRY(hipMemcpyAsync(h->x_dev, x, xb, hipMemcpyHostToDevice, h->stream));
    lcmoe_status st = enqueue_forward(h, h->x_dev, T, h->y_dev, h->stream);
    if (st) return st;
    HIP_TRY(hipMemcpyAsync(y, h->y_dev, xb, hipMemcpyDeviceToHost, h->stream));
    if (topk_idx)
        HIP_TRY(hipMemcpyAsync(topk_idx, h->topk_idx, kb * 4, hipMemcpyDeviceToHost, h->stream));
    if (topk_w) HIP_TRY(hipMemcpyAsync(topk_w, h->topk_w, kb * 4, hipMemcpyDeviceToHost, h->stream));
    HIP_TRY(hipStreamSynchronize(h->stream));
    return LCMOE_OK;
}

extern "C" lcmoe_status lcmoe_set_act_precision(lcmoe_handle *h, int32_t mode) {
    clear_error();
    if (!h) return fail(LCMOE_ERR_INVALID_ARG, "handle is NULL");
    if (mode != LCMOE_ACT_F16 && mode != LCMOE_ACT_F16X2)
        return fail(LCMOE_ERR_INVALID_ARG, "mode=%d (LCMOE_ACT_F16 or LCMOE_ACT_F16X2)", mode);
    // a forward may still be reading the activations in the other format
    HIP_TRY(hipSetDevice(h->device));
    HIP_TRY(hipStreamSynchronize(h->stream));
    if (h->last_stream) HIP_TRY(hipStreamSynchronize(h->last_stream));
    h->x_lo = mode == LCMOE_ACT_F16X2;
    return LCMOE_OK;
}

extern "C" lcmoe_status lcmoe_set_norm(lcmoe_handle *h, const float *weight, float eps) {
    clear_error();
    if (!h || !weight) return fail(LCMOE_ERR_INVALID_ARG, "handle or weight is NULL");
    if (!(eps >= 0.0f) || !std::isfinite(eps))
        return fail(LCMOE_ERR_INVALID_ARG, "eps must be finite and >= 0");
    HIP_TRY(hipSetDevice(h->device));
    const int d = h->desc.d_model;
    lcmoe_status st;
    if (!h->norm_w || !h->xn) {
        // both buffers or neither: the handle keeps them only when both allocations succeed
        float *w = nullptr, *xn = nullptr;
        if ((st = alloc_n(h, &xn, (size_t)h->desc.max_tokens * d))) return st;
        if ((st = alloc_n(h, &w, d))) return st;
        h->xn = xn;
        h->norm_w = w;
    }
    // the stream may still be reading the previous weight
    HIP_TRY(hipStreamSynchronize(h->stream));
    if (h->last_stream) HIP_TRY(hipStreamSynchronize(h->last_stream));
    // the norm weight is sanitised as load_layer sanitises it (loader.rs:161)
    std::vector<float> wn(weight, weight + d);
    lcmoe_sanitize_blocks(LCMOE_TYPE_F32, reinterpret_cast<uint8_t *>(wn.data()), d, nullptr);
    HIP_TRY(hipMemcpy(h->norm_w, wn.data(), sizeof(float) * d, hipMemcpyHostToDevice));
    h->norm_eps = eps;
    return LCMOE_OK;
}

static lcmoe_status enqueue_norm_residual(lcmoe_handle *h, const float *hidden, int32_t T,
                                          float *out, hipStream_t st) {
    return enqueue_forward(h, h->xn, T, out, st, hidden, hidden);
}

extern "C" lcmoe_status lcmoe_forward_norm_residual_dev(lcmoe_handle *h, const float *hidden_dev,
                                                        int32_t T, float *out_dev, void *stream) {
    clear_error();
    if (!h) return fail(LCMOE_ERR_INVALID_ARG, "handle is NULL");
    if (!h->norm_w || !h->xn) return fail(LCMOE_ERR_STATE, "lcmoe_set_norm has not been called");
    if (T < 0 || T > h->desc.max_tokens)
        return fail(LCMOE_ERR_INVALID_ARG, "T=%d outside [0, max_tokens=%d]", T, h->desc.max_tokens);
    if (T > 0 && (!hidden_dev || !out_dev))
        return fail(LCMOE_ERR_INVALID_ARG, "hidden or out is NULL");
    if (((uintptr_t)hidden_dev | (uintptr_t)out_dev) & 15)
        return fail(LCMOE_ERR_INVALID_ARG, "hidden and out must be 16-byte aligned");
    if (out_dev != hidden_dev && T > 0) {
        const size_t rb = sizeof(float) * (size_t)T * h->desc.d_model;
        const uintptr_t a = (uintptr_t)hidden_dev, b = (uintptr_t)out_dev;
        if (a < b + rb && b < a + rb)
            return fail(LCMOE_ERR_INVALID_ARG, "out must be hidden itself or not overlap it");
    }
    HIP_TRY(hipSetDevice(h->device));
    hipStream_t st = stream ? (hipStream_t)stream : h->stream;
    if (T == 0) {
        h->last_T = 0;
        h->last_stream = st;
        return LCMOE_OK;
    }
    return enqueue_norm_residual(h, hidden_dev, T, out_dev, st);
}

extern "C" lcmoe_status lcmoe_forward_norm_residual(lcmoe_handle *h, const float *hidden,
                                                    int32_t T, float *out, int32_t *topk_idx,
                                                    float *topk_w) {
    clear_error();
    if (!h) return fail(LCMOE_ERR_INVALID_ARG, "handle is NULL");
    if (!h->norm_w || !h->xn) return fail(LCMOE_ERR_STATE, "lcmoe_set_norm has not been called");
    if (T < 0 || T > h->desc.max_tokens)
        return fail(LCMOE_ERR_INVALID_ARG, "T=%d outside [0, max_tokens=%d]", T, h->desc.max_tokens);
    HIP_TRY(hipSetDevice(h->device));
    if (T == 0) {
        h->last_T = 0;
        h->last_stream = h->stream;
        return LCMOE_OK;
    }
    if (!hidden || !out) return fail(LCMOE_ERR_INVALID_ARG, "hidden or out is NULL");
    const size_t xb = sizeof(float) * (size_t)T * h->desc.d_model;
    const size_t kb = (size_t)T * h->desc.n_expert_used;
    HIP_TRY(hipMemcpyAsync(h->x_dev, hidden, xb, hipMemcpyHostToDevice, h->stream));
    lcmoe_status st = enqueue_norm_residual(h, h->x_dev, T, h->y_dev, h->stream);
    if (st) return st;
    HIP_TRY(hipMemcpyAsync(out, h->y_dev, xb, hipMemcpyDeviceToHost, h->stream));
    if (topk_idx)
        HIP_TRY(hipMemcpyAsync(topk_idx, h->topk_idx, kb * 4, hipMemcpyDeviceToHost, h->stream));
    if (topk_w) HIP_TRY(hipMemcpyAsync(topk_w, h->topk_w, kb * 4, hipMemcpyDeviceToHost, h->stream));
    HIP_TRY(hipStreamSynchronize(h->stream));
    return LCMOE_OK;
}

extern "C" lcmoe_status lcmoe_get_dispatch(lcmoe_handle *h, int32_t *T_out, int32_t *topk_idx,
                                           float *topk_w, int32_t *counts, int32_t *offsets,
                                           int32_t *perm, int32_t *inv) {
    clear_error();
    if (!h) return fail(LCMOE_ERR_INVALID_ARG, "handle is NULL");
    if (h->last_T < 0) return fail(LCMOE_ERR_STATE, "no forward has run on this handle");
    HIP_TRY(hipSetDevice(h->device));
    HIP_TRY(hipStreamSynchronize(h->last_stream));
    const int T = h->last_T, K = h->desc.n_expert_used, E = h->desc.n_expert;
    if (T_out) *T_out = T;
    const size_t A = (size_t)T * K;
    if (T == 0) {
        if (counts) std::memset(counts, 0, sizeof(int32_t) * E);
        if (offsets) std::memset(offsets, 0, sizeof(int32_t) * (E + 1));
        return LCMOE_OK;
    }
    if (topk_idx) HIP_TRY(hipMemcpy(topk_idx, h->topk_idx, A * 4, hipMemcpyDeviceToHost));
    if (topk_w) HIP_TRY(hipMemcpy(topk_w, h->topk_w, A * 4, hipMemcpyDeviceToHost));
    if (counts) HIP_TRY(hipMemcpy(counts, h->counts, (size_t)E * 4, hipMemcpyDeviceToHost));
    if (offsets) HIP_TRY(hipMemcpy(offsets, h->offsets, (size_t)(E + 1) * 4, hipMemcpyDeviceToHost));
    if (perm) HIP_TRY(hipMemcpy(perm, h->perm, A * 4, hipMemcpyDeviceToHost));
    if (inv) HIP_TRY(hipMemcpy(inv, h->inv, A * 4, hipMemcpyDeviceToHost));
    return LCMOE_OK;
}

extern "C" lcmoe_status lcmoe_set_timing(lcmoe_handle *h, int32_t enable) {
    clear_error();
    if (!h) return fail(LCMOE_ERR_INVALID_ARG, "handle is NULL");
    h->timing = enable != 0;
    return LCMOE_OK;
}

extern "C" lcmoe_status lcmoe_get_timing(lcmoe_handle *h, int32_t n_slots, double *ms,
                                         int64_t *launches) {
    clear_error();
    if (!h) return fail(LCMOE_ERR_INVALID_ARG, "handle is NULL");
    HIP_TRY(hipSetDevice(h->device));
    for (auto &p : h->pending) {
        HIP_TRY(hipEventSynchronize(p.b));
        float t = 0.0f;
        HIP_TRY(hipEventElapsedTime(&t, p.a, p.b));
        h->t_ms[p.slot] += t;
        h->t_n[p.slot] += 1;
        h->event_pool.push_back(p.a);
        h->event_pool.push_back(p.b);
    }
    h->pending.clear();
    for (int i = 0; i < n_slots && i < kNumSlots; i++) {
        if (ms) ms[i] = h->t_ms[i];
        if (launches) launches[i] = h->t_n[i];
    }
    for (int i = 0; i < kNumSlots; i++) {
        h->t_ms[i] = 0.0;
        h->t_n[i] = 0;
    }
    return LCMOE_OK;
}

extern "C" const char *lcmoe_timing_name(int32_t slot) {
    return (slot >= 0 && slot < kNumSlots) ? kSlotNames[slot] : "";
}

extern "C" int32_t lcmoe_timing_slots(void) { return kNumSlots; }

extern "C" lcmoe_status lcmoe_debug_dequant(int32_t type, const uint8_t *data, int64_t count,
                                            float *out) {
    clear_error();
    if (!data || !out || count <= 0 || count % 8)
        return fail(LCMOE_ERR_INVALID_ARG, "bad arguments");
    int64_t bs = block_size(type);
    if (!bs) return fail(LCMOE_ERR_UNSUPPORTED, "type %d", type);
    if (count % bs) return fail(LCMOE_ERR_INVALID_ARG, "count not a whole number of blocks");
    size_t nbytes = lcmoe_tensor_size(type, count);
    void *src = nullptr, *dst = nullptr;
    HIP_TRY(hipMalloc(&src, nbytes + 16));
    hipError_t e = hipMalloc(&dst, sizeof(float) * count);
    if (e == hipSuccess) e = hipMemcpy(src, data, nbytes, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = launch_debug_dequant(type, (const uint8_t *)src, count, (float *)dst, nullptr);
    if (e == hipSuccess) e = hipMemcpy(out, dst, sizeof(float) * count, hipMemcpyDeviceToHost);
    (void)hipFree(src);
    if (dst) (void)hipFree(dst);
    if (e != hipSuccess) return fail(LCMOE_ERR_HIP, "debug_dequant: %s", hipGetErrorString(e));
    return LCMOE_OK;
}

static lcmoe_status shard_args(int32_t type, int32_t m, int32_t k, int32_t n, size_t *b_bytes) {
    if (type != LCMOE_TYPE_Q8_0 && type != LCMOE_TYPE_Q4_0)
        return fail(LCMOE_ERR_UNSUPPORTED, "shard matmul type %d (Q8_0 = 8 or Q4_0 = 2)", type);
    if (m < 0 || k < 0 || n < 0 || n % 32 || m > 65535 * 8)
        return fail(LCMOE_ERR_INVALID_ARG, "shard matmul shape m=%d k=%d n=%d (n %% 32 == 0)", m,
                    k, n);
    *b_bytes = (size_t)k * (n / 32) * (type == LCMOE_TYPE_Q8_0 ? 34 : 18);
    return LCMOE_OK;
}

extern "C" lcmoe_status lcmoe_shard_matmul_dev(int32_t type, const float *a_dev,
                                               const uint8_t *b_dev, float *c_dev, int32_t m,
                                               int32_t k, int32_t n, void *stream) {
    clear_error();
    size_t bb;
    if (lcmoe_status s = shard_args(type, m, k, n, &bb)) return s;
    if ((size_t)m * n == 0) return LCMOE_OK;
    if (!c_dev || (k > 0 && (!a_dev || !b_dev)))
        return fail(LCMOE_ERR_INVALID_ARG, "a, b or c is NULL");
    if ((uintptr_t)b_dev & 1) return fail(LCMOE_ERR_INVALID_ARG, "b must be 2-byte aligned");
    HIP_TRY(launch_shard_matmul(type, a_dev, b_dev, c_dev, m, k, n, (hipStream_t)stream));
    return LCMOE_OK;
}

extern "C" lcmoe_status lcmoe_shard_matmul_split_dev(int32_t type, const float *a_dev,
                                                     const uint8_t *b_dev, float *c_dev,
                                                     int32_t m, int32_t k, int32_t n,
                                                     int32_t k_split, float *workspace,
                                                     void *stream) {
    clear_error();
    size_t bb;
    if (lcmoe_status s = shard_args(type, m, k, n, &bb)) return s;
    if (k_split < 1 || k_split > 64)
        return fail(LCMOE_ERR_INVALID_ARG, "k_split=%d outside [1, 64]", k_split);
    if ((size_t)m * n == 0) return LCMOE_OK;
    if (!c_dev || (k > 0 && (!a_dev || !b_dev)))
        return fail(LCMOE_ERR_INVALID_ARG, "a, b or c is NULL");
    if ((uintptr_t)b_dev & 1) return fail(LCMOE_ERR_INVALID_ARG, "b must be 2-byte aligned");
    // slices of ks = ceil(k / k_split) rows, and only as many as it takes to
    // cover k: every slice holds at least one row (S <= k_split)
    const int ks = k > 0 ? (k + k_split - 1) / k_split : 1;
    const int S = k > 0 ? (k + ks - 1) / ks : 1;
    if (S > 1 && (!workspace || ((uintptr_t)workspace & 3)))
        return fail(LCMOE_ERR_INVALID_ARG, "k_split > 1 needs a 4-byte aligned workspace");
    HIP_TRY(launch_shard_matmul(type, a_dev, b_dev, c_dev, m, k, n, (hipStream_t)stream, S,
                                workspace));
    return LCMOE_OK;
}

extern "C" lcmoe_status lcmoe_shard_matmul_split_noalloc_dev(int32_t type, const float *a_dev,
                                                             const uint8_t *b_dev, float *c_dev,
                                                             int32_t m, int32_t k, int32_t n,
                                                             int32_t k_split, void *stream) {
    clear_error();
    size_t bb;
    if (lcmoe_status s = shard_args(type, m, k, n, &bb)) return s;
    if (k_split < 1 || k_split > 64)
        return fail(LCMOE_ERR_INVALID_ARG, "k_split=%d outside [1, 64]", k_split);
    if ((size_t)m * n == 0) return LCMOE_OK;
    if (!c_dev || (k > 0 && (!a_dev || !b_dev)))
        return fail(LCMOE_ERR_INVALID_ARG, "a, b or c is NULL");
    if ((uintptr_t)b_dev & 1) return fail(LCMOE_ERR_INVALID_ARG, "b must be 2-byte aligned");
    const int ks = k > 0 ? (k + k_split - 1) / k_split : 1;
    const int S = k > 0 ? (k + ks - 1) / ks : 1;
    float *ws = nullptr;
    if (S > 1) {
        if ((int64_t)S * m * n > kShardScratchFloats)
            return fail(LCMOE_ERR_INVALID_ARG,
                        "%d slices of %d x %d need %lld floats of scratch, more than the %lld "
                        "of the static array (lower k_split)",
                        S, m, n, (long long)S * m * n, (long long)kShardScratchFloats);
        HIP_TRY(shard_scratch(&ws));
    }
    HIP_TRY(launch_shard_matmul(type, a_dev, b_dev, c_dev, m, k, n, (hipStream_t)stream, S, ws));
    return LCMOE_OK;
}

extern "C" lcmoe_status lcmoe_shard_matmul(int32_t type, const float *a, const uint8_t *b,
                                           float *c, int32_t m, int32_t k, int32_t n) {
    clear_error();
    size_t bb;
    if (lcmoe_status s = shard_args(type, m, k, n, &bb)) return s;
    if ((size_t)m * n == 0) return LCMOE_OK;
    if (!c || (k > 0 && (!a || !b))) return fail(LCMOE_ERR_INVALID_ARG, "a, b or c is NULL");
    const size_t ab = sizeof(float) * (size_t)m * k, cb = sizeof(float) * (size_t)m * n;
    void *da = nullptr, *db = nullptr, *dc = nullptr;
    hipError_t e = hipMalloc(&da, ab ? ab : 4);
    if (e == hipSuccess) e = hipMalloc(&db, bb ? bb : 4);
    if (e == hipSuccess) e = hipMalloc(&dc, cb);
    if (e == hipSuccess && ab) e = hipMemcpy(da, a, ab, hipMemcpyHostToDevice);
    if (e == hipSuccess && bb) e = hipMemcpy(db, b, bb, hipMemcpyHostToDevice);
    if (e == hipSuccess)
        e = launch_shard_matmul(type, (const float *)da, (const uint8_t *)db, (float *)dc, m, k,
                                n, nullptr);
    if (e == hipSuccess) e = hipMemcpy(c, dc, cb, hipMemcpyDeviceToHost);
    for (void *p : {da, db, dc})
        if (p) (void)hipFree(p);
    if (e != hipSuccess) return fail(LCMOE_ERR_HIP, "shard_matmul: %s", hipGetErrorString(e));
    return LCMOE_OK;
}

static lcmoe_status matmul_args(int32_t m, int32_t k, int32_t n) {
    if (m < 0 || k < 0 || n < 0) return fail(LCMOE_ERR_INVALID_ARG, "m=%d k=%d n=%d", m, k, n);
    if (m > 524280) return fail(LCMOE_ERR_INVALID_ARG, "m=%d exceeds 524280", m);
    return LCMOE_OK;
}

extern "C" lcmoe_status lcmoe_matmul_f32_dev(const float *a_dev, const float *b_dev, float *c_dev,
                                             int32_t m, int32_t k, int32_t n, void *stream) {
    clear_error();
    if (lcmoe_status s = matmul_args(m, k, n)) return s;
    if ((size_t)m * n == 0) return LCMOE_OK;
    if (!c_dev || (k > 0 && (!a_dev || !b_dev)))
        return fail(LCMOE_ERR_INVALID_ARG, "a, b or c is NULL");
    if (((uintptr_t)a_dev | (uintptr_t)b_dev | (uintptr_t)c_dev) & 3)
        return fail(LCMOE_ERR_INVALID_ARG, "a, b and c must be 4-byte aligned");
    HIP_TRY(launch_matmul_f32(a_dev, b_dev, c_dev, m, k, n, (hipStream_t)stream));
    return LCMOE_OK;
}

extern "C" lcmoe_status lcmoe_matmul_f32(const float *a, const float *b, float *c, int32_t m,
                                         int32_t k, int32_t n) {
    clear_error();
    if (lcmoe_status s = matmul_args(m, k, n)) return s;
    if ((size_t)m * n == 0) return LCMOE_OK;
    if (!c || (k > 0 && (!a || !b))) return fail(LCMOE_ERR_INVALID_ARG, "a, b or c is NULL");
    const size_t ab = sizeof(float) * (size_t)m * k, bb = sizeof(float) * (size_t)k * n,
                 cb = sizeof(float) * (size_t)m * n;
    void *da = nullptr, *db = nullptr, *dc = nullptr;
    hipError_t e = hipMalloc(&da, ab ? ab : 4);
    if (e == hipSuccess) e = hipMalloc(&db, bb ? bb : 4);
    if (e == hipSuccess) e = hipMalloc(&dc, cb);
    if (e == hipSuccess && ab) e = hipMemcpy(da, a, ab, hipMemcpyHostToDevice);
    if (e == hipSuccess && bb) e = hipMemcpy(db, b, bb, hipMemcpyHostToDevice);
    if (e == hipSuccess)
        e = launch_matmul_f32((const float *)da, (const float *)db, (float *)dc, m, k, n, nullptr);
    if (e == hipSuccess) e = hipMemcpy(c, dc, cb, hipMemcpyDeviceToHost);
    for (void *p : {da, db, dc})
        if (p) (void)hipFree(p);
    if (e != hipSuccess) return fail(LCMOE_ERR_HIP, "matmul_f32: %s", hipGetErrorString(e));
    return LCMOE_OK;
}

extern "C" lcmoe_status lcmoe_debug_rmsnorm(const float *x, const float *w, float eps, int32_t T,
                                            int32_t d, float *out) {
    clear_error();
    if (!x || !w || !out || T <= 0 || d <= 0 || d % 4)
        return fail(LCMOE_ERR_INVALID_ARG, "bad arguments (T > 0, d > 0 and d %% 4 == 0)");
    const size_t n = (size_t)T * d;
    void *a = nullptr, *b = nullptr, *c = nullptr;
    hipError_t e = hipMalloc(&a, sizeof(float) * n);
    if (e == hipSuccess) e = hipMalloc(&b, sizeof(float) * d);
    if (e == hipSuccess) e = hipMalloc(&c, sizeof(float) * n);
    if (e == hipSuccess) e = hipMemcpy(a, x, sizeof(float) * n, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(b, w, sizeof(float) * d, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = launch_rmsnorm((const float *)a, (const float *)b, eps, T, d, (float *)c, nullptr);
    if (e == hipSuccess) e = hipMemcpy(out, c, sizeof(float) * n, hipMemcpyDeviceToHost);
    for (void *p : {a, b, c})
        if (p) (void)hipFree(p);
    if (e != hipSuccess) return fail(LCMOE_ERR_HIP, "debug_rmsnorm: %s", hipGetErrorString(e));
    return LCMOE_OK;
}

extern "C" lcmoe_status lcmoe_debug_read_bandwidth(int64_t slice_bytes, int32_t reps,
                                                   double *gbps) {
    clear_error();
    const int64_t total = (int64_t)4 << 30, mib16 = (int64_t)16 << 20;
    if (!gbps || reps < 1 || slice_bytes < mib16 || slice_bytes % mib16 ||
        slice_bytes > ((int64_t)1 << 30))
        return fail(LCMOE_ERR_INVALID_ARG, "slice of 16 MiB multiples up to 1 GiB, reps >= 1");
    int dev = 0, cus = 0;
    HIP_TRY(hipGetDevice(&dev));
    HIP_TRY(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    const int blocks = 4 * std::max(cus, 1);
    void *buf = nullptr, *sink = nullptr;
    hipEvent_t a = nullptr, b = nullptr;
    hipError_t e = hipMalloc(&buf, total);
    if (e == hipSuccess) e = hipMalloc(&sink, sizeof(uint32_t) * blocks);
    if (e == hipSuccess) e = hipMemset(buf, 1, total);
    if (e == hipSuccess) e = hipEventCreate(&a);
    if (e == hipSuccess) e = hipEventCreate(&b);
    const int64_t nslice = total / slice_bytes;
    float ms = 0.0f;
    for (int r = 0; e == hipSuccess && r < reps + 2; r++) {
        if (r == 2) e = hipEventRecord(a, nullptr);
        if (e == hipSuccess)
            e = launch_stream_read((const char *)buf + (r % nslice) * slice_bytes, slice_bytes,
                                   blocks, (uint32_t *)sink, nullptr);
    }
    if (e == hipSuccess) e = hipEventRecord(b, nullptr);
    if (e == hipSuccess) e = hipEventSynchronize(b);
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, a, b);
    if (a) (void)hipEventDestroy(a);
    if (b) (void)hipEventDestroy(b);
    if (buf) (void)hipFree(buf);
    if (sink) (void)hipFree(sink);
    if (e != hipSuccess) return fail(LCMOE_ERR_HIP, "read probe: %s", hipGetErrorString(e));
    *gbps = (double)slice_bytes * reps / (ms * 1e-3) / 1e9;
    return LCMOE_OK;
}

extern "C" lcmoe_status lcmoe_debug_route_fallbacks(lcmoe_handle *h, int32_t *count) {
    clear_error();
    if (!h || !count) return fail(LCMOE_ERR_INVALID_ARG, "handle or count is NULL");
    *count = -1;
    if (!h->last_sig || h->last_T <= 0) return LCMOE_OK;
    HIP_TRY(hipSetDevice(h->device));
    HIP_TRY(hipStreamSynchronize(h->last_stream));
    std::vector<int32_t> f((size_t)h->last_T);
    HIP_TRY(hipMemcpy(f.data(), h->sig_flag, sizeof(int32_t) * f.size(), hipMemcpyDeviceToHost));
    int32_t n = 0;
    for (int32_t v : f) n += v != 0;
    *count = n;
    return LCMOE_OK;
}

extern "C" lcmoe_status lcmoe_debug_sigmoid(const float *x, int64_t n, float *out) {
    clear_error();
    if (!x || !out || n <= 0) return fail(LCMOE_ERR_INVALID_ARG, "bad arguments");
    void *a = nullptr, *b = nullptr;
    HIP_TRY(hipMalloc(&a, sizeof(float) * n));
    hipError_t e = hipMalloc(&b, sizeof(float) * n);
    if (e == hipSuccess) e = hipMemcpy(a, x, sizeof(float) * n, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = launch_debug_sigmoid((const float *)a, n, (float *)b, nullptr);
    if (e == hipSuccess) e = hipMemcpy(out, b, sizeof(float) * n, hipMemcpyDeviceToHost);
    (void)hipFree(a);
    if (b) (void)hipFree(b);
    if (e != hipSuccess) return fail(LCMOE_ERR_HIP, "debug_sigmoid: %s", hipGetErrorString(e));
    return LCMOE_OK;
}
