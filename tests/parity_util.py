"""Shared helpers for the GPU parity tests: build a layer, run the HIP path
through the C ABI, run the oracle on the same bytes, compare."""
import os

import numpy as np

import lcoracle as O
import leafcutterllm_amd as L

Y_REL_L2_TOL = 1e-3      # layer output, relative L2 over [T, d]
W_REL_TOL = 1e-5         # routed weights (device exp vs glibc exp)


def oracle_desc(d: L.Desc) -> O.Desc:
    od = O.Desc()
    for name, _ in d._fields_:
        setattr(od, name, getattr(d, name))
    return od


def rel_l2(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    nb = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (nb if nb > 0 else 1.0))


def check_routing(gpu: dict, ref: dict, T: int, K: int):
    assert np.array_equal(gpu["topk_idx"].reshape(T, K), ref["topk_idx"].reshape(T, K)), \
        "topk_idx differs"
    for k in ("counts", "offsets", "perm", "inv"):
        assert np.array_equal(gpu[k], ref[k]), f"{k} differs"
    w_g = gpu["topk_w"].reshape(T, K).astype(np.float64)
    w_r = ref["topk_w"].reshape(T, K).astype(np.float64)
    assert np.all(np.abs(w_g - w_r) <= W_REL_TOL * np.abs(w_r) + 1e-30), \
        f"topk_w max rel err {np.max(np.abs(w_g - w_r) / np.maximum(np.abs(w_r), 1e-30))}"


def run_and_check(cfg: L.LayerConfig, layer: dict, x: np.ndarray, moe: L.MoeFfn = None,
                  y_subset=None, threads: int = min(16, os.cpu_count() or 1)) -> dict:
    """Runs the HIP layer on x and checks it against the oracle.  Routing and
    dispatch are compared on the whole batch; y on all tokens, or only on the
    token rows in `y_subset` (each token's output depends on that token alone,
    so the oracle recomputes just those rows)."""
    T = x.shape[0]
    own = moe is None
    if own:
        moe = L.MoeFfn(cfg.desc(max(T, 1)), layer)
    try:
        y, idx, w = moe.forward(x)
        disp = moe.dispatch()
        assert np.array_equal(disp["topk_idx"], idx)
        od = oracle_desc(cfg.desc(max(T, 1)))
        # the router and bias as the reference ingests them (sanitised,
        # loader.rs:161), which is what lco_moe_forward routes with
        bias = layer.get("bias")
        logits = O.router_logits(x, O.sanitize(layer["router"]))
        r_idx, r_w = O.route(od, logits, None if bias is None else O.sanitize(bias))
        counts, offsets, perm, inv = O.dispatch(r_idx, cfg.n_expert)
        check_routing(disp, {"topk_idx": r_idx, "topk_w": r_w, "counts": counts,
                             "offsets": offsets, "perm": perm, "inv": inv}, T, cfg.n_expert_used)
        rows = np.arange(T) if y_subset is None else np.asarray(y_subset)
        ref = O.moe_forward(od, layer, x[rows], threads=threads)
        err = rel_l2(y[rows], ref["y"])
        assert np.all(np.isfinite(y)), "non-finite output"
        assert err <= Y_REL_L2_TOL, f"y rel-L2 {err:.3e} > {Y_REL_L2_TOL}"
        return {"rel_l2": err, "y": y, "topk_idx": idx, "counts": counts}
    finally:
        if own:
            moe.close()
