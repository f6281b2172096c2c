"""The allocation-free shard GEMM entry point
(lcmoe_shard_matmul_split_noalloc_dev: k-slice planes in a static device
array instead of a caller workspace) against lcmoe_shard_matmul_split_dev
with the same k_split: bit-identical on two calls in a row, the second with
a smaller input, and the size limit refused before any device work."""
import numpy as np
import pytest

import leafcutterllm_amd as L
from leafcutterllm_amd import _lib, hip
from leafcutterllm_amd._lib import check
from test_gpu_shard import _bits, _case

Q8, Q4 = L.TYPE_Q8_0, L.TYPE_Q4_0
SCRATCH = 4 * 1024 * 1024  # LCMOE_SHARD_SCRATCH_FLOATS


def test_noalloc_refuses_oversize_before_device_work():
    # 64 slices of 16 x 8192 = 8M floats > the static array; the pointers are
    # never dereferenced (the size check comes first)
    fake = 4096
    st = L.lib().lcmoe_shard_matmul_split_noalloc_dev(Q8, fake, fake, fake, 16, 4096, 8192, 64,
                                                      None)
    assert _lib.STATUS[st] == "LCMOE_ERR_INVALID_ARG"
    assert b"scratch" in L.lib().lcmoe_last_error()
    st = L.lib().lcmoe_shard_matmul_split_noalloc_dev(Q8, fake, fake, fake, 1, 64, 32, 0, None)
    assert _lib.STATUS[st] == "LCMOE_ERR_INVALID_ARG"


def _run(fn, qtype, a, b, m, k, n, S, with_ws):
    da, db = hip.DeviceBuffer(a.nbytes).upload(a), hip.DeviceBuffer(b.nbytes).upload(b)
    dc = hip.DeviceBuffer(4 * m * n)
    ws = hip.DeviceBuffer(4 * S * m * n) if with_ws else None
    st = hip.Stream()
    try:
        args = (qtype, da.ptr, db.ptr, dc.ptr, m, k, n, S) + ((ws.ptr,) if with_ws else ())
        check(fn(*args, st.ptr), fn.__name__)
        st.synchronize()
        return dc.download(np.empty((m, n), np.float32))
    finally:
        for x in (da, db, dc) + ((ws,) if with_ws else ()):
            x.free()


@pytest.mark.gpu
@pytest.mark.parametrize("qtype", [Q8, Q4])
def test_noalloc_matches_workspace_variant(qtype):
    lib = L.lib()
    # the first call fills most of the static array (16 * 4096 * 32 = 2M
    # floats); the second, smaller one must not see its leftovers
    for m, k, n, S in [(16, 4096, 4096, 32), (3, 250, 288, 64), (1, 5, 64, 8), (2, 300, 64, 1)]:
        print(f"noalloc qtype={qtype} m={m} k={k} n={n} k_split={S}", flush=True)
        assert S * m * n <= SCRATCH
        a, b = _case(qtype, m, k, n, seed=m + k + n + S)
        ref = _run(lib.lcmoe_shard_matmul_split_dev, qtype, a, b, m, k, n, S, True)
        out = _run(lib.lcmoe_shard_matmul_split_noalloc_dev, qtype, a, b, m, k, n, S, False)
        assert np.array_equal(_bits(out), _bits(ref))
