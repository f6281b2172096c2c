"""The HIP layer through the C ABI against the committed golden fixtures
(tests/golden/moe_*.npz): routing and dispatch bit-identical, routed weights
within 1e-5 relative, y within 1e-3 relative L2."""
import glob
import os
import sys

import numpy as np
import pytest

import leafcutterllm_amd as L
from parity_util import W_REL_TOL, Y_REL_L2_TOL, rel_l2

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, GOLDEN)
from make_golden import load  # noqa: E402

FILES = sorted(glob.glob(os.path.join(GOLDEN, "moe_*.npz")))


def product_desc(od) -> L.Desc:
    d = L.Desc()
    for name, _ in d._fields_:
        setattr(d, name, getattr(od, name))
    return d


@pytest.mark.parametrize("path", FILES, ids=[os.path.basename(f) for f in FILES])
def test_golden_fixture(path):
    od, lay, x, exp = load(path)
    T, K = x.shape[0], od.n_expert_used
    print(f"golden {os.path.basename(path)}: T={T} d={od.d_model} E={od.n_expert}", flush=True)
    with L.MoeFfn(product_desc(od), lay) as moe:
        y, idx, w = moe.forward(x)
        disp = moe.dispatch()
    assert np.array_equal(idx, exp["topk_idx"])
    for k in ("counts", "offsets", "perm", "inv"):
        assert np.array_equal(disp[k], exp[k]), k
    assert np.all(np.abs(w - exp["topk_w"]) <= W_REL_TOL * np.abs(exp["topk_w"]) + 1e-30)
    assert np.all(np.isfinite(y))
    assert rel_l2(y, exp["y"]) <= Y_REL_L2_TOL
