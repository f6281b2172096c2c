"""Pins the oracle's MoE semantics (no GPU): routing, dispatch and the whole
layer, each against an independent numpy restatement.

The reference has no router, dispatch or combine, so these functions of
oracle/lcoracle.c (lco_route, lco_dispatch, lco_moe_forward) are fixed by the
written semantics alone: top-k by a full sort of (-z, e) with NaN ranked as
-inf; DeepSeek-V3 group-limited selection; a stable counting sort; the
slot-ordered combine.  Every check below is computed without the oracle's
code path (brute-force sorts, numpy argsort, float64 arithmetic over the
dequantised weights), and is chosen so that a plausible slip -- ties to the
higher index, NaN ranked high, a group scored by its top-1 only, weights
renormalised over the wrong set, an unstable dispatch, a dropped shared
expert or a wrong slot weight -- fails it.  The building blocks it relies on
(dequantisation, lco_sigmoid_cw, f32 GEMM order) are pinned in
test_oracle_core.py.
"""
import numpy as np
import pytest

import lcoracle as O

RENORM, SOFTMAX, SIGMOID = O.ROUTE_SOFTMAX_RENORM, O.ROUTE_SOFTMAX, O.ROUTE_SIGMOID_GROUP


def desc(E, K, kind, n_group=0, topk_group=0, scale=1.0, has_bias=0, d=256, F=256,
         qt=O.Q4_K, qd=None, S=0, FS=0, max_tokens=64):
    qd = qt if qd is None else qd
    o = O.Desc()
    o.d_model, o.d_ff, o.n_expert, o.n_expert_used = d, F, E, K
    o.n_shared, o.d_ff_shared = S, FS
    o.route_kind, o.n_group, o.topk_group = kind, n_group, topk_group
    o.routed_scale, o.has_bias = scale, has_bias
    o.type_gate = o.type_up = qt
    o.type_down = qd
    o.type_gate_sh = o.type_up_sh = qt if S else 0
    o.type_down_sh = qd if S else 0
    o.max_tokens = max_tokens
    return o


# ------------------------------------------------------- brute force ------

def rank_key(v):
    """Selection key: NaN ranks as -inf."""
    v = float(v)
    return -np.inf if np.isnan(v) else v


def brute_topk(z, K, allowed=None):
    """The K best of z by a full sort of (-z, e): larger z first, ties to
    the lower index."""
    cand = [e for e in range(len(z)) if allowed is None or allowed[e]]
    order = sorted(cand, key=lambda e: (-rank_key(z[e]), e))
    return order[:K]


def brute_route(kind, logits, K, bias=None, n_group=0, topk_group=0, scale=1.0):
    """Independent restatement of the three router kinds (selection on the
    float32 values, weights in float64)."""
    T, E = logits.shape
    idx = np.empty((T, K), np.int64)
    w = np.empty((T, K), np.float64)
    for t in range(T):
        lt = logits[t].astype(np.float32)
        if kind == SIGMOID:
            s = O.sigmoid_cw(lt)  # the shared sigmoid, pinned in test_oracle_core
            z = (s + bias).astype(np.float32) if bias is not None else s
            gs = E // n_group
            gscore = np.empty(n_group, np.float32)
            for g in range(n_group):
                zg = z[g * gs:(g + 1) * gs]
                top = brute_topk(zg, min(2, gs))
                gscore[g] = np.float32(zg[top[0]]) + np.float32(zg[top[1]]) if gs >= 2 else zg[top[0]]
            keep = brute_topk(gscore, topk_group)
            allowed = np.zeros(E, bool)
            for g in keep:
                allowed[g * gs:(g + 1) * gs] = True
            sel = brute_topk(z, K, allowed)
            ss = s[sel].astype(np.float64)
            idx[t] = sel
            with np.errstate(all="ignore"):
                w[t] = ss / ss.sum() * scale
        else:
            z = (lt + bias).astype(np.float32) if bias is not None else lt
            sel = brute_topk(z, K)
            idx[t] = sel
            z64 = z.astype(np.float64)
            with np.errstate(all="ignore"):
                if kind == RENORM:
                    zs = z64[sel]
                    e = np.exp(zs - zs.max())
                    w[t] = e / e.sum() * scale
                else:
                    e = np.exp(z64 - z64.max())
                    w[t] = (e / e.sum())[sel] * scale
    return idx, w


def adversarial_logits(rng, T, E):
    """Heavy ties, +-0, +-inf and NaN."""
    pool = np.array([0.0, -0.0, 1.0, -1.0, 0.5, 2.0, np.inf, -np.inf, np.nan, 1e-30, -1e-30,
                     3.0, 0.25], np.float32)
    kind = rng.integers(0, 4, size=T)
    out = np.empty((T, E), np.float32)
    for t in range(T):
        if kind[t] == 0:    # few distinct values: ties everywhere
            out[t] = rng.choice(pool[:6], size=E)
        elif kind[t] == 1:  # every special value
            out[t] = rng.choice(pool, size=E)
        elif kind[t] == 2:  # all equal
            out[t] = pool[rng.integers(0, len(pool))]
        else:               # continuous with a few exact duplicates
            v = rng.standard_normal(E).astype(np.float32)
            v[rng.integers(0, E, size=E // 4)] = v[0]
            out[t] = v
    return out


def check_weights(w_oracle, w_ref, tol=2e-6):
    w_oracle = w_oracle.astype(np.float64)
    fin = np.isfinite(w_ref)
    assert np.all(np.abs(w_oracle[fin] - w_ref[fin]) <= tol * np.abs(w_ref[fin]) + 1e-30)
    assert np.all(~np.isfinite(w_oracle[~fin]))


@pytest.mark.parametrize("kind,E,K", [(RENORM, 8, 2), (RENORM, 16, 4), (SOFTMAX, 60, 4),
                                      (SOFTMAX, 12, 3), (RENORM, 5, 5), (SOFTMAX, 1, 1)])
@pytest.mark.parametrize("adversarial", [False, True])
def test_softmax_route_brute_force(kind, E, K, adversarial):
    rng = np.random.default_rng(1000 * E + K + adversarial)
    T = 300
    logits = (adversarial_logits(rng, T, E) if adversarial
              else rng.standard_normal((T, E)).astype(np.float32))
    for bias in (None, np.where(np.arange(E) < min(8, E), 2.0, 0.0).astype(np.float32)):
        d = desc(E, K, kind, has_bias=int(bias is not None))
        with np.errstate(all="ignore"):
            idx, w = O.route(d, logits, bias)
        ref_idx, ref_w = brute_route(kind, logits, K, bias)
        assert np.array_equal(idx, ref_idx)
        if not adversarial:
            check_weights(w, ref_w)
        else:
            fin = np.all(np.isfinite(logits), axis=1)
            check_weights(w[fin], ref_w[fin])


@pytest.mark.parametrize("E,K,G,TG", [(32, 4, 4, 2), (256, 8, 8, 4), (16, 3, 8, 3), (8, 2, 8, 8),
                                      (12, 4, 3, 1)])
@pytest.mark.parametrize("adversarial", [False, True])
def test_sigmoid_group_route_brute_force(E, K, G, TG, adversarial):
    rng = np.random.default_rng(7 * E + G + adversarial)
    T = 200 if E == 256 else 300
    logits = (adversarial_logits(rng, T, E) if adversarial
              else rng.standard_normal((T, E)).astype(np.float32))
    for bias in (None, (0.1 * rng.standard_normal(E)).astype(np.float32)):
        d = desc(E, K, SIGMOID, n_group=G, topk_group=TG, scale=2.5,
                 has_bias=int(bias is not None))
        with np.errstate(all="ignore"):
            idx, w = O.route(d, logits, bias)
        ref_idx, ref_w = brute_route(SIGMOID, logits, K, bias, G, TG, 2.5)
        assert np.array_equal(idx, ref_idx)
        fin = np.all(np.isfinite(logits), axis=1)
        check_weights(w[fin], ref_w[fin])


def test_route_tie_and_nan_rules_by_hand():
    """Hand-checked rows: ties go to the lower index, NaN ranks as -inf, -0
    ties +0, and a group is scored by its two best members."""
    d = desc(6, 3, RENORM)
    logits = np.array([[1, 1, 1, 1, 1, 1],
                       [np.nan, 0, -0.0, 5, np.nan, 5],
                       [-np.inf, np.nan, -np.inf, -np.inf, np.nan, -np.inf],
                       [0.0, -0.0, 0.0, 1, 2, 3]], np.float32)
    with np.errstate(all="ignore"):
        idx, _ = O.route(d, logits)
    assert idx.tolist() == [[0, 1, 2], [3, 5, 1], [0, 1, 2], [5, 4, 3]]
    # groups of 4: group 0 = {0.9, 0.1, 0.1, 0.1} (top-1 best, top-2 sum 1.0),
    # group 1 = {0.6, 0.6, 0, 0} (top-2 sum 1.2): the pair wins
    g = desc(8, 2, SIGMOID, n_group=2, topk_group=1, has_bias=1)
    bias = np.array([0.9, 0.1, 0.1, 0.1, 0.6, 0.6, 0.0, 0.0], np.float32)
    lg = np.full((1, 8), -np.inf, np.float32)  # sigmoid = 0: z = bias exactly
    idx, w = O.route(g, lg, bias)
    assert idx.tolist() == [[4, 5]]


# ---------------------------------------------------------- dispatch ------

@pytest.mark.parametrize("T,K,E", [(0, 2, 8), (1, 1, 1), (7, 2, 8), (300, 4, 60), (256, 8, 256),
                                   (64, 3, 5), (33, 16, 16)])
def test_dispatch_is_a_stable_sort(T, K, E):
    rng = np.random.default_rng(T * 131 + K * 7 + E)
    # skewed: a few experts take most assignments, some take none
    p = rng.dirichlet(np.full(E, 0.3))
    idx = rng.choice(E, size=(T, K), p=p).astype(np.int32)
    counts, offsets, perm, inv = O.dispatch(idx, E)
    flat = idx.ravel()
    assert np.array_equal(counts, np.bincount(flat, minlength=E))
    assert offsets[0] == 0 and np.array_equal(np.diff(offsets), counts)
    assert offsets[-1] == T * K and np.all(np.diff(offsets) >= 0)
    assert np.array_equal(perm, np.argsort(flat, kind="stable"))
    assert np.array_equal(np.sort(perm), np.arange(T * K))          # a permutation
    assert np.array_equal(inv[perm], np.arange(T * K))              # inv is its inverse
    for e in range(E):                                              # runs ascend in a
        run = perm[offsets[e]:offsets[e + 1]]
        assert np.all(flat[run] == e) and np.all(np.diff(run) > 0)


def test_dispatch_rejects_out_of_range():
    with pytest.raises(ValueError):
        O.dispatch(np.array([[0, 8]], np.int32), 8)
    with pytest.raises(ValueError):
        O.dispatch(np.array([[-1, 0]], np.int32), 8)


# ---------------------------------------------------- float64 layer -------

def synth_layer(d, F, E, qt, qd, S=0, FS=0, seed=0, bias=None, zero=False):
    rng = np.random.default_rng(seed)

    def stack(rows, cols, n, q):
        if n == 0:
            return None
        w = (0.02 * rng.standard_normal((n, rows * cols))).astype(np.float32)
        if zero:
            w[:] = 0
        return np.concatenate([O.quantize(q, w[i]) for i in range(n)])

    lay = {"router": (0.02 * rng.standard_normal((d, E))).astype(np.float32),
           "bias": bias, "gate": stack(F, d, E, qt), "up": stack(F, d, E, qt),
           "down": stack(d, F, E, qd)}
    if S:
        lay.update(gate_sh=stack(FS, d, S, qt), up_sh=stack(FS, d, S, qt),
                   down_sh=stack(d, FS, S, qd))
    return lay


def deq(q, data, n, rows, cols):
    """Expert n of a stacked tensor as float64 [rows, cols] (GGUF orientation)."""
    sz = O.tensor_size(q, rows * cols)
    return O.dequant(q, data[n * sz:(n + 1) * sz], rows * cols).astype(np.float64).reshape(rows, cols)


def ffn64(x, wg, wu, wd):
    g = x @ wg.T
    u = x @ wu.T
    return ((g / (1.0 + np.exp(-g))) * u) @ wd.T


def layer64(d_, lay, x):
    """The MoE layer in float64: logits, selection (on the float64 scores),
    weights, experts and combine, none of it through the oracle."""
    d, F, E, K = d_.d_model, d_.d_ff, d_.n_expert, d_.n_expert_used
    x64 = x.astype(np.float64)
    logits = x64 @ lay["router"].astype(np.float64)
    b = None if lay.get("bias") is None else lay["bias"].astype(np.float64)
    T = x.shape[0]
    idx = np.empty((T, K), np.int64)
    w = np.empty((T, K))
    for t in range(T):
        lt = logits[t]
        if d_.route_kind == SIGMOID:
            s = 1.0 / (1.0 + np.exp(-lt))
            z = s + b if b is not None else s
            gs = E // d_.n_group
            gsc = [np.sort(z[g * gs:(g + 1) * gs])[::-1][:2].sum() for g in range(d_.n_group)]
            keep = np.argsort(-np.array(gsc), kind="stable")[:d_.topk_group]
            allowed = np.zeros(E, bool)
            for g in keep:
                allowed[g * gs:(g + 1) * gs] = True
            zz = np.where(allowed, z, -np.inf)
            sel = np.argsort(-zz, kind="stable")[:K]
            idx[t] = sel
            w[t] = s[sel] / s[sel].sum() * d_.routed_scale
        else:
            z = lt + b if b is not None else lt
            sel = np.argsort(-z, kind="stable")[:K]
            idx[t] = sel
            if d_.route_kind == RENORM:
                e = np.exp(z[sel] - z[sel].max())
                w[t] = e / e.sum()
            else:
                e = np.exp(z - z.max())
                w[t] = (e / e.sum())[sel]
            w[t] *= d_.routed_scale
    y = np.zeros((T, d))
    for e in np.unique(idx):
        wg = deq(d_.type_gate, lay["gate"], e, F, d)
        wu = deq(d_.type_up, lay["up"], e, F, d)
        wd = deq(d_.type_down, lay["down"], e, d, F)
        ye = ffn64(x64, wg, wu, wd)
        y += np.where(idx == e, w, 0.0).sum(axis=1)[:, None] * ye
    for s in range(d_.n_shared):
        FS = d_.d_ff_shared
        y += ffn64(x64, deq(d_.type_gate_sh, lay["gate_sh"], s, FS, d),
                   deq(d_.type_up_sh, lay["up_sh"], s, FS, d),
                   deq(d_.type_down_sh, lay["down_sh"], s, d, FS))
    return y, idx, w, logits


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


LAYERS = {
    # name: (desc kwargs, layer kwargs)
    "q4k-renorm": (dict(E=8, K=2, kind=RENORM, d=256, F=512, qt=O.Q4_K), {}),
    "q8-softmax-shared-bias": (dict(E=12, K=3, kind=SOFTMAX, d=256, F=256, qt=O.Q8_0, S=2, FS=384,
                                    has_bias=1), dict(bias="plus2")),
    "sigmoid-q6k-shared": (dict(E=32, K=4, kind=SIGMOID, n_group=4, topk_group=2, scale=2.5,
                                d=512, F=256, qt=O.Q4_K, qd=O.Q6_K, S=1, FS=256, has_bias=1),
                           dict(bias="normal")),
    "q4k-straddle": (dict(E=8, K=2, kind=SOFTMAX, d=256, F=384, qt=O.Q4_K), {}),
    "f32": (dict(E=4, K=2, kind=RENORM, d=128, F=256, qt=O.F32), {}),
}


@pytest.mark.parametrize("name", sorted(LAYERS))
def test_layer_forward_vs_float64(name):
    dk, lk = LAYERS[name]
    d_ = desc(**dk)
    E = d_.n_expert
    rng = np.random.default_rng(len(name))
    bias = None
    if lk.get("bias") == "plus2":
        bias = np.where(np.arange(E) < 8, 2.0, 0.0).astype(np.float32)
    elif lk.get("bias") == "normal":
        bias = (0.1 * rng.standard_normal(E)).astype(np.float32)
    lay = synth_layer(d_.d_model, d_.d_ff, E, d_.type_gate, d_.type_down, d_.n_shared,
                      d_.d_ff_shared, seed=len(name) + 1, bias=bias)
    x = rng.standard_normal((24, d_.d_model)).astype(np.float32)
    out = O.moe_forward(d_, lay, x, threads=4)
    y64, idx64, w64, logits64 = layer64(d_, lay, x)
    # selection: the float32 chain and the float64 sums rank alike wherever
    # the float64 scores are not within rounding of a tie
    assert np.array_equal(out["topk_idx"], idx64)
    assert np.all(np.abs(out["topk_w"] - w64) <= 1e-5 * np.abs(w64) + 1e-7)
    assert rel_l2(out["y"], y64) < 2e-5, rel_l2(out["y"], y64)


# --------------------------------------------------------- invariants -----

def test_e1_k1_is_the_dense_ffn_bit_for_bit():
    d_ = desc(1, 1, RENORM, d=256, F=512, qt=O.Q4_K)
    lay = synth_layer(256, 512, 1, O.Q4_K, O.Q4_K, seed=3)
    x = np.random.default_rng(3).standard_normal((5, 256)).astype(np.float32)
    out = O.moe_forward(d_, lay, x)
    assert np.all(out["topk_idx"] == 0) and np.all(out["topk_w"] == 1.0)
    wg = O.dequant(O.Q4_K, lay["gate"], 512 * 256).reshape(512, 256).T
    wu = O.dequant(O.Q4_K, lay["up"], 512 * 256).reshape(512, 256).T
    wd = O.dequant(O.Q4_K, lay["down"], 256 * 512).reshape(256, 512).T
    ref = O.ffn_dense(x, wg, wu, wd)
    assert np.array_equal(out["y"].view(np.uint32), ref.view(np.uint32))


def test_all_zero_experts_give_zero():
    d_ = desc(8, 2, SOFTMAX, d=256, F=256, qt=O.Q8_0, S=1, FS=256)
    lay = synth_layer(256, 256, 8, O.Q8_0, O.Q8_0, S=1, FS=256, seed=4, zero=True)
    x = np.random.default_rng(4).standard_normal((6, 256)).astype(np.float32)
    out = O.moe_forward(d_, lay, x)
    assert np.all(out["y"] == 0.0)
    assert np.all(np.isfinite(out["topk_w"])) and out["counts"].sum() == 12


@pytest.mark.parametrize("kind", [RENORM, SOFTMAX])
def test_duplicated_experts_are_additive(kind):
    """Every expert identical: y = (sum of the token's slot weights) times the
    one expert's FFN -- 1 for the renormalised router."""
    E, d, F = 4, 256, 256
    one = synth_layer(d, F, 1, O.Q4_K, O.Q4_K, seed=5)
    lay = dict(one, gate=np.tile(one["gate"], E), up=np.tile(one["up"], E),
               down=np.tile(one["down"], E),
               router=np.random.default_rng(5).standard_normal((d, E)).astype(np.float32) * 0.02)
    x = np.random.default_rng(6).standard_normal((7, d)).astype(np.float32)
    out = O.moe_forward(desc(E, 3, kind, d=d, F=F), lay, x)
    dense = O.moe_forward(desc(1, 1, RENORM, d=d, F=F), one, x)["y"].astype(np.float64)
    wsum = out["topk_w"].astype(np.float64).sum(axis=1)
    if kind == RENORM:
        assert np.allclose(wsum, 1.0, atol=1e-6)
    assert rel_l2(out["y"], wsum[:, None] * dense) < 1e-6


def test_routed_scale_and_shared_expert_add():
    """routed_scale multiplies the routed sum exactly (a power of two); a
    shared expert adds its dense FFN."""
    d, F, E = 256, 256, 8
    lay = synth_layer(d, F, E, O.Q4_K, O.Q4_K, S=1, FS=256, seed=9)
    x = np.random.default_rng(9).standard_normal((5, d)).astype(np.float32)
    y1 = O.moe_forward(desc(E, 2, SOFTMAX, d=d, F=F), lay, x)["y"]
    y2 = O.moe_forward(desc(E, 2, SOFTMAX, d=d, F=F, scale=2.0), lay, x)["y"]
    assert np.array_equal(y2, 2.0 * y1)
    ysh = O.moe_forward(desc(E, 2, SOFTMAX, d=d, F=F, S=1, FS=256), lay, x)["y"]
    shared = O.moe_forward(desc(1, 1, RENORM, d=d, F=256),
                           {"router": np.ones((d, 1), np.float32), "bias": None,
                            "gate": lay["gate_sh"], "up": lay["up_sh"], "down": lay["down_sh"]},
                           x)["y"]
    assert rel_l2(ysh, y1.astype(np.float64) + shared) < 1e-6


def test_sigmoid_cw_dips_at_most_one_ulp():
    """The certified sigmoid-group router treats sigmoid_cw as monotone up to
    one ulp: its scores bound s(c) for c in [zlo, zhi] by one ulp below
    s(zlo) and above s(zhi).  Exhaustively, over every non-NaN float32 input
    in increasing order, the function never falls more than one ulp below
    its running maximum; and it does dip (so the widening is needed): the two
    adjacent inputs below step down by exactly one ulp."""
    lo = np.float32(0.0614658967)
    hi = np.nextafter(lo, np.float32(1.0))
    s = O.sigmoid_cw(np.array([lo, hi], np.float32))
    assert s.view(np.uint32)[0] - s.view(np.uint32)[1] == 1
    assert O.sigmoid_max_dip(8) == 1
