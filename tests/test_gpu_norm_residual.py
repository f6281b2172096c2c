"""GPU: the fused FFN half of a decoder layer (engine.rs:110-115),
out = hidden + ffn_forward(rms_norm(hidden)).

Bar: the device RMSNorm bit-identical to the oracle's CpuBackend::rms_norm;
routing on the normed rows exact; out bit-identical to hidden + the plain
forward of the oracle-normed rows (the residual add is one f32 add per
element); the layer output within the parity tolerance of the oracle.
"""

import numpy as np
import pytest

import lcoracle as O
import leafcutterllm_amd as L
from leafcutterllm_amd import hip
from leafcutterllm_amd.configs import small_config, synth_x
from parity_util import run_and_check

pytestmark = pytest.mark.gpu

Q4, Q6, Q8 = L.TYPE_Q4_K, L.TYPE_Q6_K, L.TYPE_Q8_0


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("d", [4, 32, 100, 256, 260, 4096, 4100, 6144, 8192, 8196, 16384])
def test_device_rmsnorm_bit_exact(d):
    rng = np.random.default_rng(d)
    T = 7
    x = (rng.standard_normal((T, d)) * np.logspace(-3, 3, T)[:, None]).astype(np.float32)
    x[1] = 0.0                              # all-zero row: scale = 1/sqrt(eps)
    x[2, ::3] = 0.0
    x[3] = np.float32(1e-20) * (1 + np.arange(d, dtype=np.float32) % 5)  # squares underflow
    w = rng.standard_normal(d).astype(np.float32)
    for eps in (1e-5, 1e-6):
        dev = L.debug_rmsnorm(x, w, eps)
        ref = O.rms_norm(x, w, eps)
        assert np.array_equal(_bits(dev), _bits(ref)), (d, eps)
    # eps = 0 on the rows without zeros (a zero row would give 0 * inf = NaN,
    # whose bit pattern is not specified)
    rows = [0, 3, 4, 5, 6]
    dev = L.debug_rmsnorm(x[rows], w, 0.0)
    assert np.array_equal(_bits(dev), _bits(O.rms_norm(x[rows], w, 0.0))), d


def test_device_rmsnorm_rejects_bad_shape():
    with pytest.raises(L.LcmoeError):
        L.debug_rmsnorm(np.ones((2, 6), np.float32), np.ones(6, np.float32))


NORM_CASES = {
    "q4k-renorm": small_config("q4k-renorm", 256, 512, 8, 2, L.ROUTE_SOFTMAX_RENORM, Q4, Q4),
    "q8-shared": small_config("q8-shared", 256, 512, 8, 2, L.ROUTE_SOFTMAX, Q8, Q8,
                              n_shared=1, d_ff_shared=512),
    "sigmoid-group-q6k": small_config("sigmoid-group", 512, 1024, 16, 4,
                                      L.ROUTE_SIGMOID_GROUP, Q4, Q6, n_shared=1,
                                      d_ff_shared=512, n_group=4, topk_group=2,
                                      bias="plus2_first8"),
    # the norm fused into the certified router's entry, several norm chunks
    "d2048-e60-fused": small_config("d2048", 2048, 256, 60, 4, L.ROUTE_SOFTMAX, Q4, Q4,
                                    n_shared=1, d_ff_shared=256),
    "d4096-fused": small_config("d4096", 4096, 256, 8, 2, L.ROUTE_SOFTMAX_RENORM, Q4, Q4),
    # the exact router (d % 128 != 0): the norm as a launch of its own
    "d288-separate": small_config("d288", 288, 512, 8, 2, L.ROUTE_SOFTMAX_RENORM, Q4, Q4),
}


def _hidden(cfg, T, seed):
    # residual-stream rows: larger and less uniform than the FFN's input
    rng = np.random.default_rng(seed)
    return (synth_x(cfg, T, seed=seed) * rng.uniform(0.5, 20.0, (T, 1))).astype(np.float32)


@pytest.mark.parametrize("name", sorted(NORM_CASES))
@pytest.mark.parametrize("T", [1, 6, 64])
def test_norm_residual_matches_composition_and_oracle(name, T):
    cfg = NORM_CASES[name]
    lay = L.synth_layer(cfg, seed=4)
    hidden = _hidden(cfg, T, 100 + T)
    w_norm = (1.0 + 0.1 * np.random.default_rng(9).standard_normal(cfg.d_model)).astype(np.float32)
    xn = O.rms_norm(hidden, w_norm, 1e-5)
    with L.MoeFfn(cfg.desc(T), lay) as moe:
        with pytest.raises(L.LcmoeError):   # no norm weight yet
            moe.forward_norm_residual(hidden)
        moe.set_norm(w_norm, 1e-5)
        out, idx, tw = moe.forward_norm_residual(hidden)
        y, idx2, tw2 = moe.forward(xn)
        assert np.array_equal(idx, idx2)
        assert np.array_equal(_bits(tw), _bits(tw2))
        assert np.array_equal(_bits(out), _bits(hidden + y))
        run_and_check(cfg, lay, xn, moe=moe)


def test_norm_residual_dev_in_place_and_separate():
    cfg = NORM_CASES["q4k-renorm"]
    lay = L.synth_layer(cfg, seed=5)
    T, d = 40, cfg.d_model
    hidden = _hidden(cfg, T, 7)
    w_norm = np.random.default_rng(2).uniform(0.5, 1.5, d).astype(np.float32)
    with L.MoeFfn(cfg.desc(T), lay) as moe:
        moe.set_norm(w_norm, 1e-6)
        ref, _, _ = moe.forward_norm_residual(hidden)
        a = hip.DeviceBuffer(hidden.nbytes).upload(hidden)
        b = hip.DeviceBuffer(hidden.nbytes)
        st = hip.Stream()   # the calls are stream-ordered: wait before reading
        try:
            moe.forward_norm_residual_dev(a.ptr, T, b.ptr, st.ptr)      # separate buffers
            st.synchronize()
            sep = b.download(np.empty_like(hidden))
            moe.forward_norm_residual_dev(a.ptr, T, a.ptr, st.ptr)      # in place
            st.synchronize()
            inp = a.download(np.empty_like(hidden))
            with pytest.raises(L.LcmoeError):                           # partial overlap
                moe.forward_norm_residual_dev(a.ptr, T, a.ptr + 4 * d, st.ptr)
        finally:
            a.free()
            b.free()
        assert np.array_equal(_bits(sep), _bits(ref))
        assert np.array_equal(_bits(inp), _bits(ref))
        # replacing the weight takes effect on the next call
        moe.set_norm(2 * w_norm, 1e-6)
        out2, _, _ = moe.forward_norm_residual(hidden)
        y2, _, _ = moe.forward(O.rms_norm(hidden, 2 * w_norm, 1e-6))
        assert np.array_equal(_bits(out2), _bits(hidden + y2))
