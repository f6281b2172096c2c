"""Writes the MoE-layer golden fixtures tests/golden/moe_*.npz.

Each fixture is a small seeded layer (T <= 4, d <= 256, E <= 8, F <= 128):
the inputs (x, the f32 router and bias, the GGUF expert bytes) and the
oracle's outputs on them (topk_idx, topk_w, counts, offsets, perm, inv, y).
The oracle (oracle/lcoracle.c) is the writer; its routing, dispatch and layer
semantics are pinned independently by tests/test_oracle_route.py.  Rerun
with `python tests/golden/make_golden.py` only when the written semantics
change on purpose; tests/test_golden.py then shows what moved.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

import lcoracle as O  # noqa: E402

DESC_FIELDS = [f for f, _ in O.Desc._fields_]

# name: (d, F, E, K, kind, qt gate/up, qt down, S, FS, extra desc, bias, T, router)
FIXTURES = {
    "q4k_renorm": (256, 64, 4, 2, O.ROUTE_SOFTMAX_RENORM, O.Q4_K, O.Q4_K, 0, 0, {}, None, 4,
                   "normal"),
    "q8_softmax_shared_bias": (256, 32, 4, 2, O.ROUTE_SOFTMAX, O.Q8_0, O.Q8_0, 1, 32, {},
                               "plus2_first", 3, "normal"),
    "sigmoid_group_q6k": (256, 32, 8, 2, O.ROUTE_SIGMOID_GROUP, O.Q4_K, O.Q6_K, 1, 32,
                          {"n_group": 4, "topk_group": 2, "routed_scale": 2.5}, "normal0.1", 4,
                          "normal"),
    # d = 128: K-quant blocks of 256 straddle rows of every matrix
    "q4k_straddle_d128": (128, 128, 4, 2, O.ROUTE_SOFTMAX, O.Q4_K, O.Q4_K, 0, 0, {}, None, 4,
                          "normal"),
    # tied router columns: selection decided by the lower-index rule
    "ties_renorm": (256, 32, 8, 4, O.ROUTE_SOFTMAX_RENORM, O.Q4_K, O.Q4_K, 0, 0, {}, None, 4,
                    "ties"),
}


def make(name, spec, seed):
    d, F, E, K, kind, qg, qd, S, FS, extra, bias_kind, T, router_kind = spec
    desc = O.Desc()
    desc.d_model, desc.d_ff, desc.n_expert, desc.n_expert_used = d, F, E, K
    desc.n_shared, desc.d_ff_shared, desc.route_kind = S, FS, kind
    desc.n_group = extra.get("n_group", 0)
    desc.topk_group = extra.get("topk_group", 0)
    desc.routed_scale = extra.get("routed_scale", 1.0)
    desc.has_bias = int(bias_kind is not None)
    desc.type_gate = desc.type_up = qg
    desc.type_down = qd
    desc.type_gate_sh = desc.type_up_sh = qg if S else 0
    desc.type_down_sh = qd if S else 0
    desc.max_tokens = T

    def stack(rows, cols, n, q, stream):
        return np.concatenate([O.quantize(q, O.synth_normal(seed, stream + i, 0.02, rows * cols))
                               for i in range(n)])

    lay = {"gate": stack(F, d, E, qg, 100), "up": stack(F, d, E, qg, 200),
           "down": stack(d, F, E, qd, 300)}
    if S:
        lay.update(gate_sh=stack(FS, d, S, qg, 400), up_sh=stack(FS, d, S, qg, 500),
                   down_sh=stack(d, FS, S, qd, 600))
    router = O.synth_normal(seed, 1, 0.02, d * E).reshape(d, E)
    x = O.synth_normal(seed, 0, 1.0, T * d).reshape(T, d)
    if router_kind == "ties":
        router[:, 1] = router[:, 0]           # experts 0 and 1 tie on every token
        router[:, 5] = router[:, 2]           # 2 and 5 tie
        router[:, 7] = 0.0                    # expert 7 scores exactly 0
        x[3] = 0.0                            # every expert ties: 0, 1, 2, 3
    lay["router"] = np.ascontiguousarray(router)
    bias = None
    if bias_kind == "plus2_first":
        bias = np.zeros(E, np.float32)
        bias[0] = 2.0
    elif bias_kind == "normal0.1":
        bias = O.synth_normal(seed, 2, 0.1, E)
    lay["bias"] = bias
    out = O.moe_forward(desc, lay, x, threads=1)
    rec = {"desc_i32": np.array([getattr(desc, f) if f != "routed_scale" else 0
                                 for f in DESC_FIELDS], np.int32),
           "routed_scale": np.float32(desc.routed_scale), "x": x, "router": lay["router"],
           "bias": np.zeros(0, np.float32) if bias is None else bias}
    for k in ("gate", "up", "down", "gate_sh", "up_sh", "down_sh"):
        rec[k] = lay.get(k, np.zeros(0, np.uint8))
    for k in ("topk_idx", "topk_w", "counts", "offsets", "perm", "inv", "y"):
        rec[k] = out[k]
    np.savez_compressed(os.path.join(HERE, f"moe_{name}.npz"), **rec)
    return rec


def load(path):
    """(desc, layer dict, x, expected outputs) of one fixture."""
    z = np.load(path, allow_pickle=False)
    desc = O.Desc()
    for f, v in zip(DESC_FIELDS, z["desc_i32"]):
        if f != "routed_scale":
            setattr(desc, f, int(v))
    desc.routed_scale = float(z["routed_scale"])
    lay = {"router": z["router"], "bias": z["bias"] if z["bias"].size else None}
    for k in ("gate", "up", "down", "gate_sh", "up_sh", "down_sh"):
        lay[k] = z[k] if z[k].size else None
    exp = {k: z[k] for k in ("topk_idx", "topk_w", "counts", "offsets", "perm", "inv", "y")}
    return desc, lay, z["x"], exp


if __name__ == "__main__":
    O.build()
    for i, (name, spec) in enumerate(sorted(FIXTURES.items())):
        r = make(name, spec, seed=77 + i)
        print(f"moe_{name}.npz: T={r['x'].shape[0]} idx={r['topk_idx'].tolist()}")
