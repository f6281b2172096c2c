"""The committed golden fixtures (tests/golden/moe_*.npz, written by
tests/golden/make_golden.py) on the CPU: the oracle reproduces every stored
output bit for bit, the stored dispatch is the stable sort of the stored
selection, and the stored layer output agrees with an independent float64
recomputation (tests/test_oracle_route.py: layer64)."""
import glob
import os
import sys

import numpy as np
import pytest

import lcoracle as O
from test_oracle_route import layer64, rel_l2

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, GOLDEN)
from make_golden import load  # noqa: E402

FILES = sorted(glob.glob(os.path.join(GOLDEN, "moe_*.npz")))


def test_fixtures_present():
    assert len(FILES) >= 5


@pytest.mark.parametrize("path", FILES, ids=[os.path.basename(f) for f in FILES])
def test_oracle_reproduces_fixture(path):
    desc, lay, x, exp = load(path)
    out = O.moe_forward(desc, lay, x, threads=2)
    for k in ("topk_idx", "counts", "offsets", "perm", "inv"):
        assert np.array_equal(out[k], exp[k]), k
    for k in ("topk_w", "y"):
        assert np.array_equal(out[k].view(np.uint32), exp[k].view(np.uint32)), k


@pytest.mark.parametrize("path", FILES, ids=[os.path.basename(f) for f in FILES])
def test_fixture_consistency(path):
    desc, lay, x, exp = load(path)
    T, K, E = x.shape[0], desc.n_expert_used, desc.n_expert
    flat = exp["topk_idx"].ravel()
    assert exp["topk_idx"].shape == (T, K)
    assert np.array_equal(exp["counts"], np.bincount(flat, minlength=E))
    assert np.array_equal(exp["offsets"], np.concatenate([[0], np.cumsum(exp["counts"])]))
    assert np.array_equal(exp["perm"], np.argsort(flat, kind="stable"))
    assert np.array_equal(exp["inv"][exp["perm"]], np.arange(T * K))
    y64, idx64, w64, _ = layer64(desc, lay, x)
    assert np.array_equal(exp["topk_idx"], idx64)
    assert np.all(np.abs(exp["topk_w"] - w64) <= 1e-5 * np.abs(w64) + 1e-7)
    assert rel_l2(exp["y"], y64) < 2e-5
