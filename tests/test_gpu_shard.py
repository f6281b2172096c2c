"""GPU: the shard-layout GEMM (lcmoe_shard_matmul) bit-identical to the
oracle's restatement of int8_gemm.rs's x86 path, over row tiles, partial
column blocks, odd k, signed and subnormal f16 scales, and m = 0 / k = 0."""
import numpy as np
import pytest

import lcoracle as O
import leafcutterllm_amd as L
from leafcutterllm_amd import hip
from leafcutterllm_amd._lib import check
from shard_pack import pack_q4, pack_q8, reference_test_matrices

pytestmark = pytest.mark.gpu

Q8, Q4 = L.TYPE_Q8_0, L.TYPE_Q4_0


def _case(qtype, m, k, n, seed):
    rng = np.random.default_rng(seed)
    a = (rng.standard_normal((m, k)) * rng.uniform(0.1, 10, (m, 1))).astype(np.float32)
    scales = rng.uniform(-0.05, 0.05, (k, n // 32)).astype(np.float32)
    scales.flat[::7] = 3e-6          # f16 subnormal
    if qtype == Q8:
        codes = rng.integers(-128, 128, (k, n))
        b = pack_q8(scales, codes)
    else:
        codes = rng.integers(0, 16, (k, n))
        b = pack_q4(scales, codes)
    return a, b


def _bits(x):
    return np.ascontiguousarray(x, np.float32).view(np.uint32)


@pytest.mark.parametrize("qtype", [Q8, Q4])
@pytest.mark.parametrize("m,k,n", [(1, 64, 32), (1, 1, 4096), (3, 101, 96), (8, 16, 64),
                                   (9, 250, 288), (17, 33, 1056), (64, 512, 512),
                                   (1, 2048, 2048), (1, 777, 1056), (2, 1000, 96),
                                   (4, 700, 160), (16, 300, 64)])
def test_shard_matmul_bit_exact(qtype, m, k, n):
    a, b = _case(qtype, m, k, n, seed=m * 1000 + k + n)
    dev = L.shard_matmul(qtype, a, b, k, n)
    ref = O.shard_matmul(qtype, a, b, k, n)
    assert np.array_equal(_bits(dev), _bits(ref))


@pytest.mark.parametrize("qtype", [Q8, Q4])
def test_shard_matmul_reference_matrices(qtype):
    m, k, n = 8, 16, 64
    a = (np.arange(m * k, dtype=np.float32) * np.float32(0.01) - np.float32(0.5)).reshape(m, k)
    scales, codes = reference_test_matrices(qtype, k, n)
    b = pack_q8(scales, codes) if qtype == Q8 else pack_q4(scales, codes)
    assert np.array_equal(_bits(L.shard_matmul(qtype, a, b, k, n)),
                          _bits(O.shard_matmul(qtype, a, b, k, n)))


def test_shard_matmul_empty_and_k0():
    assert L.shard_matmul(Q8, np.zeros((0, 8), np.float32), np.zeros(8 * 34, np.uint8),
                          8, 32).shape == (0, 32)
    c = L.shard_matmul(Q4, np.zeros((2, 0), np.float32), np.zeros(0, np.uint8), 0, 64)
    assert np.array_equal(c, np.zeros((2, 64), np.float32))


def test_shard_matmul_dev_matches_host():
    m, k, n = 5, 300, 640
    a, b = _case(Q8, m, k, n, seed=3)
    ref = L.shard_matmul(Q8, a, b, k, n)
    da, db = hip.DeviceBuffer(a.nbytes).upload(a), hip.DeviceBuffer(b.nbytes).upload(b)
    dc = hip.DeviceBuffer(4 * m * n)
    st = hip.Stream()
    try:
        check(L.lib().lcmoe_shard_matmul_dev(Q8, da.ptr, db.ptr, dc.ptr, m, k, n, st.ptr),
                "lcmoe_shard_matmul_dev")
        st.synchronize()
        out = dc.download(np.empty((m, n), np.float32))
    finally:
        for x in (da, db, dc):
            x.free()
    assert np.array_equal(_bits(out), _bits(ref))


@pytest.mark.parametrize("qtype", [Q8, Q4])
@pytest.mark.parametrize("m,k,n,S", [(1, 4096, 512, 16), (3, 101, 96, 4), (9, 250, 288, 64),
                                     (1, 5, 64, 8), (2, 300, 64, 1)])
def test_shard_matmul_split(qtype, m, k, n, S):
    """k split into slices: deterministic, within the float64 error bound of
    the exact product; one slice is bit-identical to the exact path."""
    a, b = _case(qtype, m, k, n, seed=7 * k + S)
    ref = O.shard_matmul(qtype, a, b, k, n)
    da, db = hip.DeviceBuffer(a.nbytes).upload(a), hip.DeviceBuffer(b.nbytes).upload(b)
    dc, ws = hip.DeviceBuffer(4 * m * n), hip.DeviceBuffer(4 * S * m * n)
    st = hip.Stream()
    outs = []
    try:
        for _ in range(2):
            check(L.lib().lcmoe_shard_matmul_split_dev(qtype, da.ptr, db.ptr, dc.ptr, m, k, n, S,
                                                       ws.ptr, st.ptr),
                  "lcmoe_shard_matmul_split_dev")
            st.synchronize()
            outs.append(dc.download(np.empty((m, n), np.float32)))
    finally:
        for x in (da, db, dc, ws):
            x.free()
    assert np.array_equal(_bits(outs[0]), _bits(outs[1]))
    if S == 1:
        assert np.array_equal(_bits(outs[0]), _bits(ref))
    # float64 product of the same dequantised weights, with a k-step bound
    w = O.shard_matmul(qtype, np.eye(k, dtype=np.float32), b, k, n).astype(np.float64)
    exact = a.astype(np.float64) @ w
    bound = (k + S + 2) * 2.0 ** -24 * (np.abs(a.astype(np.float64)) @ np.abs(w))
    assert np.all(np.abs(outs[0] - exact) <= bound + 1e-30)
