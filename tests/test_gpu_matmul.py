"""GPU: Backend::matmul (lcmoe_matmul_f32) bit-identical to the oracle's
restatement of the x86 CPU backend's avx2_matmul order (fma chains in k for
the first 8 * floor(n / 8) columns, rounded products added for the tail;
oracle pinned in test_oracle_core.py)."""
import numpy as np
import pytest

import lcoracle as O
import leafcutterllm_amd as L
from leafcutterllm_amd import hip
from leafcutterllm_amd._lib import check

pytestmark = pytest.mark.gpu


def _bits(x):
    return np.ascontiguousarray(x, np.float32).view(np.uint32)


# Shapes for both kernels: n % 4 != 0 (one wave per 64 columns) and
# n % 4 == 0 (streaming: 16-column blocks for m <= 16, 64-column blocks
# above; k % 4 == 0 loads A as float4), with ragged column blocks, the
# n % 8 tail columns, k below, at and past one 128- or 64-step window
@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (1, 5, 7), (3, 17, 13), (8, 256, 512), (9, 300, 77),
                                   (2, 1000, 9), (5, 64, 8), (64, 512, 515), (1, 2048, 4096),
                                   (512, 512, 512), (17, 3000, 100), (1, 333, 100),
                                   (4, 4096, 4096), (16, 777, 260), (5, 1, 12), (1, 4096, 16),
                                   (3, 130, 48), (20, 64, 68), (33, 200, 4), (7, 128, 1028),
                                   (100, 65, 36)])
def test_matmul_bit_exact(m, k, n):
    rng = np.random.default_rng(m * 7919 + k * 31 + n)
    a = (rng.standard_normal((m, k)) * rng.uniform(0.01, 100, (m, 1))).astype(np.float32)
    b = (0.02 * rng.standard_normal((k, n))).astype(np.float32)
    b[rng.random((k, n)) < 0.01] = 3e-39   # subnormals stay exact (no flush)
    print(f"matmul m={m} k={k} n={n}", flush=True)
    assert np.array_equal(_bits(L.matmul(a, b)), _bits(O.matmul(a, b, threads=8)))


def test_matmul_reference_kat_and_empty():
    # simd.rs:430-455: identity and a known 2x3 @ 3x2 product
    a = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    b = np.array([[7, 8], [9, 10], [11, 12]], np.float32)
    assert np.array_equal(L.matmul(a, b), [[58, 64], [139, 154]])
    eye = np.eye(9, dtype=np.float32)
    x = np.arange(81, dtype=np.float32).reshape(9, 9)
    assert np.array_equal(L.matmul(x, eye), x)
    assert L.matmul(np.zeros((0, 4), np.float32), np.zeros((4, 3), np.float32)).shape == (0, 3)
    z = L.matmul(np.zeros((2, 0), np.float32), np.zeros((0, 9), np.float32))
    assert np.array_equal(_bits(z), np.zeros((2, 9), np.uint32))   # +0, as setzero / 0.0


@pytest.mark.parametrize("a_off,b_off", [(1, 0), (0, 1), (3, 2)])
def test_matmul_dev_unaligned_operands(a_off, b_off):
    """Device operands 4-byte aligned only (the entry point's contract): A
    off 16 bytes loads it per element, B off 16 bytes takes the per-column
    kernel; same bits either way."""
    m, k, n = 5, 256, 64
    rng = np.random.default_rng(a_off * 10 + b_off)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    ref = O.matmul(a, b, threads=4)
    def padded(x, off):   # x at float offset `off` of a device buffer
        h = np.zeros(x.size + 16, np.float32)
        h[off:off + x.size] = x.ravel()
        return hip.DeviceBuffer(h.nbytes).upload(h)

    da, db = padded(a, a_off), padded(b, b_off)
    dc = hip.DeviceBuffer(4 * m * n)
    st = hip.Stream()
    try:
        check(L.lib().lcmoe_matmul_f32_dev(da.ptr + 4 * a_off, db.ptr + 4 * b_off, dc.ptr, m, k,
                                           n, st.ptr), "lcmoe_matmul_f32_dev")
        st.synchronize()
        out = dc.download(np.empty((m, n), np.float32))
    finally:
        for x in (da, db, dc):
            x.free()
    assert np.array_equal(_bits(out), _bits(ref))


def test_matmul_dev_matches_host():
    m, k, n = 6, 333, 200
    rng = np.random.default_rng(4)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    ref = L.matmul(a, b)
    da, db = hip.DeviceBuffer(a.nbytes).upload(a), hip.DeviceBuffer(b.nbytes).upload(b)
    dc = hip.DeviceBuffer(4 * m * n)
    st = hip.Stream()
    try:
        check(L.lib().lcmoe_matmul_f32_dev(da.ptr, db.ptr, dc.ptr, m, k, n, st.ptr),
              "lcmoe_matmul_f32_dev")
        st.synchronize()
        out = dc.download(np.empty((m, n), np.float32))
    finally:
        for x in (da, db, dc):
            x.free()
    assert np.array_equal(_bits(out), _bits(ref))
