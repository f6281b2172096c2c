"""C-ABI checks that need no GPU: the library loads, exports every symbol
include/lcmoe.h declares, rejects bad descriptors and corrupt weights before
touching a device, and its host encoders / generator reproduce the oracle's
bytes."""
import ctypes as C
import os
import re

import numpy as np
import pytest

import lcoracle as O
import leafcutterllm_amd as L
from leafcutterllm_amd import _lib
from leafcutterllm_amd.configs import quantize, synth_normal

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_symbols():
    txt = open(os.path.join(ROOT, "include", "lcmoe.h")).read()
    return sorted(set(re.findall(r"\b(lcmoe_[a-z0-9_]+)\s*\(", txt)))


def test_exports_every_declared_symbol():
    syms = header_symbols()
    assert len(syms) >= 16
    lib = C.CDLL(_lib.LIB_PATH)
    for s in syms:
        assert hasattr(lib, s), s
    assert sorted(_lib.EXPORTS) == syms


def test_desc_layout_matches_oracle():
    assert C.sizeof(L.Desc) == C.sizeof(O.Desc) == 18 * 4
    assert [f[0] for f in L.Desc._fields_] == [f[0] for f in O.Desc._fields_]


def test_tensor_size_and_scan_match_oracle():
    for qt in (L.TYPE_Q8_0, L.TYPE_Q4_K, L.TYPE_Q6_K, L.TYPE_F32):
        for n in (256, 512, 2048 * 1408, 4096 * 14336):
            assert L.lib().lcmoe_tensor_size(qt, n) == O.tensor_size(qt, n)
    x = synth_normal(1, 2, 0.02, 256 * 8)
    for qt in (L.TYPE_Q8_0, L.TYPE_Q4_K, L.TYPE_Q6_K):
        b = quantize(qt, x)
        bb = b.copy()
        off = 208 if qt == L.TYPE_Q6_K else 0
        bb[off:off + 2] = np.frombuffer(np.array([np.inf], np.float16).tobytes(), np.uint8)
        for data in (b, bb):
            assert L.lib().lcmoe_scan_blocks(qt, data.ctypes.data, x.size) == \
                O.scan_blocks(qt, data, x.size)
        assert L.lib().lcmoe_scan_blocks(qt, bb.ctypes.data, x.size) == 1


@pytest.mark.parametrize("qt", [L.TYPE_Q8_0, L.TYPE_Q4_K, L.TYPE_Q6_K])
def test_product_encoder_bytes_equal_oracle(qt):
    x = synth_normal(7, 3, 0.02, 256 * 200)
    x[:256] *= 1e-6
    x[256:512] = 0.0
    x[512:768] = np.abs(x[512:768])
    assert np.array_equal(quantize(qt, x), O.quantize(qt, x))


def test_product_generator_equals_oracle():
    n = 100_003
    assert np.array_equal(synth_normal(42, 7 << 32, 0.02, n), O.synth_normal(42, 7 << 32, 0.02, n))


def _layer(cfg):
    return L.synth_layer(cfg, seed=1)


def _create(desc, layer):
    w = L.Weights()
    keep = []
    for k in ("router", "bias", "gate", "up", "down", "gate_sh", "up_sh", "down_sh"):
        a = layer.get(k)
        if a is not None:
            keep.append(a)
        setattr(w, k, None if a is None else a.ctypes.data)
    h = C.c_void_p()
    st = L.lib().lcmoe_create(C.byref(desc), C.byref(w), C.byref(h))
    if st == 0:
        L.lib().lcmoe_destroy(h)
    return st, L.lib().lcmoe_last_error().decode()


SMALL = L.configs.small_config("abi", 256, 256, 8, 2, L.ROUTE_SOFTMAX_RENORM, L.TYPE_Q4_K,
                               L.TYPE_Q4_K)


@pytest.mark.parametrize("field,value,status", [
    ("d_model", 100, 1), ("d_model", 0, 1), ("d_ff", 33, 1), ("n_expert", 0, 1),
    ("n_expert", 257, 1), ("n_expert_used", 0, 1), ("n_expert_used", 9, 1),
    ("route_kind", 7, 2), ("type_gate", 2, 2), ("type_down", 99, 2), ("max_tokens", 0, 1),
    ("n_shared", 9, 1), ("routed_scale", float("nan"), 1),
])
def test_create_rejects_bad_desc(field, value, status):
    layer = _layer(SMALL)
    d = SMALL.desc(4)
    setattr(d, field, value)
    st, msg = _create(d, layer)
    assert st == status and msg


def test_create_rejects_bad_group_router():
    cfg = L.configs.small_config("g", 256, 256, 32, 8, L.ROUTE_SIGMOID_GROUP, L.TYPE_Q4_K,
                                 L.TYPE_Q4_K, n_group=5, topk_group=2)
    st, msg = _create(cfg.desc(4), _layer(L.configs.small_config(
        "g2", 256, 256, 32, 8, L.ROUTE_SOFTMAX, L.TYPE_Q4_K, L.TYPE_Q4_K)))
    assert st == 1 and "n_group" in msg


def test_create_rejects_corrupt_block_and_null():
    layer = _layer(SMALL)
    bad = dict(layer)
    bad["down"] = layer["down"].copy()
    sz = L.configs.tensor_size(L.TYPE_Q4_K, 256 * 256)
    bad["down"][3 * sz + 144 * 5 + 2: 3 * sz + 144 * 5 + 4] = np.frombuffer(
        np.array([np.nan], np.float16).tobytes(), np.uint8)
    st, msg = _create(SMALL.desc(4), bad)
    assert st == 3 and "down[3]" in msg
    bad = dict(layer)
    bad["gate"] = None
    st, msg = _create(SMALL.desc(4), bad)
    assert st == 1 and "gate" in msg
    d = SMALL.desc(4)
    d.has_bias = 1
    st, msg = _create(d, layer)
    assert st == 1 and "bias" in msg


def test_create_without_gpu_fails_cleanly_or_succeeds():
    st, msg = _create(SMALL.desc(4), _layer(SMALL))
    assert st in (0, 4)
    if st == 4:
        assert "device" in msg


def test_quantize_errors():
    x = np.zeros(33, np.float32)
    out = np.zeros(64, np.uint8)
    assert L.lib().lcmoe_quantize(L.TYPE_Q8_0, x.ctypes.data, out.ctypes.data, 33) == 1
    assert L.lib().lcmoe_quantize(3, x.ctypes.data, out.ctypes.data, 32) == 2


def test_norm_residual_argument_errors():
    """Checked before any device work, so they need no GPU."""
    lib = L.lib()
    w = np.ones(8, np.float32)
    x = np.ones((2, 8), np.float32)
    assert lib.lcmoe_set_norm(None, w.ctypes.data, 1e-5) == 1
    assert lib.lcmoe_forward_norm_residual(None, x.ctypes.data, 2, x.ctypes.data,
                                           None, None) == 1
    assert lib.lcmoe_forward_norm_residual_dev(None, None, 0, None, None) == 1
    x6 = np.ones((2, 6), np.float32)
    assert lib.lcmoe_debug_rmsnorm(x6.ctypes.data, w.ctypes.data, 1e-5, 2, 6,
                                   x6.ctypes.data) == 1
    assert lib.lcmoe_debug_rmsnorm(x.ctypes.data, w.ctypes.data, 1e-5, 0, 8,
                                   x.ctypes.data) == 1


def test_shard_matmul_argument_errors():
    lib = L.lib()
    a = np.ones((2, 4), np.float32)
    b = np.zeros(4 * 34, np.uint8)
    c = np.zeros((2, 32), np.float32)
    args = (a.ctypes.data, b.ctypes.data, c.ctypes.data)
    assert lib.lcmoe_shard_matmul(12, *args, 2, 4, 32) == 2      # Q4_K: not a shard type
    assert lib.lcmoe_shard_matmul(8, *args, 2, 4, 40) == 1       # n % 32
    assert lib.lcmoe_shard_matmul(8, *args, -1, 4, 32) == 1
    assert lib.lcmoe_shard_matmul(8, None, None, None, 2, 4, 32) == 1
    assert lib.lcmoe_shard_matmul_dev(8, None, None, None, 0, 4, 32, None) == 0  # empty


def test_shard_matmul_split_argument_errors():
    lib = L.lib()
    a = np.ones((2, 8), np.float32)
    b = np.zeros(8 * 34, np.uint8)
    c = np.zeros((2, 32), np.float32)
    args = (a.ctypes.data, b.ctypes.data, c.ctypes.data, 2, 8, 32)
    assert lib.lcmoe_shard_matmul_split_dev(8, *args, 0, None, None) == 1    # k_split < 1
    assert lib.lcmoe_shard_matmul_split_dev(8, *args, 65, None, None) == 1   # k_split > 64
    assert lib.lcmoe_shard_matmul_split_dev(8, *args, 4, None, None) == 1    # no workspace


def test_model_create_rejects_bad_desc_before_device_work():
    """lcmoe_model_create validates the descriptor and the tensor pointers
    first: each case fails the same way with or without a GPU."""
    from leafcutterllm_amd.configs import ModelConfig, small_config, synth_model
    from leafcutterllm_amd.model import Model

    mc = ModelConfig("tiny", 1, 4, 2, 64, 32, 10000.0,
                     small_config("m", 256, 256, 8, 2, L.ROUTE_SOFTMAX, L.TYPE_Q4_K, L.TYPE_Q4_K))
    w = synth_model(mc, seed=1)
    cases = [("n_kv_head", 3, "LCMOE_ERR_INVALID_ARG"), ("head_dim", 12, "LCMOE_ERR_INVALID_ARG"),
             ("attn_type", L.TYPE_Q6_K, "LCMOE_ERR_UNSUPPORTED"), ("d_model", 512, "LCMOE_ERR_INVALID_ARG"),
             ("max_prompt", 100, "LCMOE_ERR_INVALID_ARG"), ("rope_positions", 2, "LCMOE_ERR_INVALID_ARG"),
             ("max_batch", 0, "LCMOE_ERR_INVALID_ARG")]
    for field, value, status in cases:
        d = mc.desc(2, 16, 32)
        setattr(d, field, value)
        with pytest.raises(L.LcmoeError) as e:
            Model(d, w)
        assert _lib.STATUS[e.value.status] == status, field
    w2 = dict(w, layers=[dict(w["layers"][0], attn_v=None)])
    with pytest.raises(L.LcmoeError) as e:
        Model(mc.desc(2, 16, 32), w2)
    assert _lib.STATUS[e.value.status] == "LCMOE_ERR_INVALID_ARG"


def test_matmul_f32_argument_errors():
    """lcmoe_matmul_f32 validates before any device work."""
    lib = L.lib()
    a = np.zeros(4, np.float32)
    for m, k, n in [(-1, 2, 2), (2, -1, 2), (2, 2, -1), (524281, 1, 1)]:
        st = lib.lcmoe_matmul_f32(a.ctypes.data, a.ctypes.data, a.ctypes.data, m, k, n)
        assert _lib.STATUS[st] == "LCMOE_ERR_INVALID_ARG", (m, k, n)
    assert _lib.STATUS[lib.lcmoe_matmul_f32(None, None, a.ctypes.data, 2, 2, 2)] == \
        "LCMOE_ERR_INVALID_ARG"
    assert lib.lcmoe_matmul_f32(None, None, None, 0, 5, 3) == 0   # empty: nothing to do
    st = lib.lcmoe_matmul_f32_dev(6, 4, 4, 1, 1, 1, None)        # misaligned a
    assert _lib.STATUS[st] == "LCMOE_ERR_INVALID_ARG"


def test_read_bandwidth_argument_errors():
    """lcmoe_debug_read_bandwidth validates its slice and repeat count before
    touching a device."""
    lib = L.lib()
    out = np.zeros(1, np.float64)
    mib = 1 << 20
    for slice_bytes, reps in [(8 * mib, 4), (24 * mib, 4), (2048 * mib, 4), (64 * mib, 0)]:
        st = lib.lcmoe_debug_read_bandwidth(slice_bytes, reps, out.ctypes.data)
        assert _lib.STATUS[st] == "LCMOE_ERR_INVALID_ARG", (slice_bytes, reps)
    assert _lib.STATUS[lib.lcmoe_debug_read_bandwidth(64 * mib, 4, None)] == "LCMOE_ERR_INVALID_ARG"
