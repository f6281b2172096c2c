"""ctypes binding of the CPU oracle (oracle/liblcoracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() and by
bench.py's cpu_baseline leg, as the checker.  The product package
(leafcutterllm_amd) never imports it.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liblcoracle.so")

F32, F16, Q8_0, Q4_K, Q6_K = 0, 1, 8, 12, 14
ROUTE_SOFTMAX_RENORM, ROUTE_SOFTMAX, ROUTE_SIGMOID_GROUP = 0, 1, 2


class Desc(C.Structure):
    """Same field order and types as lco_desc / lcmoe_desc."""

    _fields_ = [
        ("d_model", C.c_int32), ("d_ff", C.c_int32), ("n_expert", C.c_int32),
        ("n_expert_used", C.c_int32), ("n_shared", C.c_int32), ("d_ff_shared", C.c_int32),
        ("route_kind", C.c_int32), ("n_group", C.c_int32), ("topk_group", C.c_int32),
        ("routed_scale", C.c_float), ("has_bias", C.c_int32),
        ("type_gate", C.c_int32), ("type_up", C.c_int32), ("type_down", C.c_int32),
        ("type_gate_sh", C.c_int32), ("type_up_sh", C.c_int32), ("type_down_sh", C.c_int32),
        ("max_tokens", C.c_int32),
    ]


class Weights(C.Structure):
    _fields_ = [
        ("router", C.c_void_p), ("bias", C.c_void_p),
        ("gate", C.c_void_p), ("up", C.c_void_p), ("down", C.c_void_p),
        ("gate_sh", C.c_void_p), ("up_sh", C.c_void_p), ("down_sh", C.c_void_p),
    ]


def build() -> None:
    """Compile the oracle with its own Makefile (gcc only)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = C.CDLL(_LIB_PATH)
        vp, i32, sz, f32 = C.c_void_p, C.c_int, C.c_size_t, C.c_float
        sigs = {
            "lco_f16_to_f32": (f32, [C.c_uint16]),
            "lco_f32_to_f16": (C.c_uint16, [f32]),
            "lco_f16_to_f32_n": (None, [vp, vp, sz]),
            "lco_f32_to_f16_n": (None, [vp, vp, sz]),
            "lco_block_size": (sz, [i32]),
            "lco_block_bytes": (sz, [i32]),
            "lco_tensor_size": (sz, [i32, sz]),
            "lco_dequant": (i32, [i32, vp, vp, sz]),
            "lco_quantize": (i32, [i32, vp, vp, sz]),
            "lco_scale_min_k4": (None, [i32, vp, vp, vp]),
            "lco_sanitize": (None, [vp, sz]),
            "lco_scan_blocks": (sz, [i32, vp, sz]),
            "lco_synth_normal": (None, [C.c_uint64, C.c_uint64, f32, vp, sz]),
            "lco_matmul": (None, [vp, vp, vp, i32, i32, i32, i32]),
            "lco_transpose": (None, [vp, vp, i32, i32]),
            "lco_silu": (f32, [f32]),
            "lco_rms_norm": (None, [vp, vp, f32, i32, i32, vp]),
            "lco_shard_matmul": (i32, [i32, vp, vp, vp, i32, i32, i32]),
            "lco_softmax": (None, [vp, vp, i32]),
            "lco_expf_cw": (f32, [f32]),
            "lco_sigmoid_cw": (f32, [f32]),
            "lco_sigmoid_max_dip": (C.c_int64, [i32]),
            "lco_router_logits": (None, [vp, vp, vp, i32, i32, i32]),
            "lco_route": (i32, [C.POINTER(Desc), vp, vp, i32, vp, vp]),
            "lco_dispatch": (i32, [vp, i32, i32, i32, vp, vp, vp, vp]),
            "lco_moe_forward": (i32, [C.POINTER(Desc), C.POINTER(Weights), vp, i32, vp, vp, vp,
                                      vp, vp, vp, vp, i32]),
            "lco_ffn_dense": (None, [vp, i32, i32, i32, vp, vp, vp, vp, i32]),
            "lco_resident_create": (vp, [C.POINTER(Desc), C.POINTER(Weights), i32]),
            "lco_resident_forward": (i32, [vp, vp, i32, vp, i32]),
            "lco_resident_destroy": (None, [vp]),
            "lco_rope": (None, [vp, i32, i32, i32, f32, i32]),
            "lco_attention_core": (None, [vp, vp, vp, i32, i32, i32, i32, i32, vp]),
            "lco_argmax_last": (i32, [vp, i32]),
        }
        for name, (res, args) in sigs.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data


# ---- formats ---------------------------------------------------------------

def tensor_size(qtype: int, count: int) -> int:
    return int(lib().lco_tensor_size(qtype, count))


def dequant(qtype: int, data: np.ndarray, count: int) -> np.ndarray:
    data = np.ascontiguousarray(data, dtype=np.uint8)
    assert data.size >= tensor_size(qtype, count)
    out = np.empty(count, np.float32)
    assert lib().lco_dequant(qtype, _p(data), _p(out), count) == 0
    return out


def sanitize(v: np.ndarray) -> np.ndarray:
    """sanitize_weights (loader.rs:241-249) on a copy: lco_sanitize."""
    out = np.array(v, np.float32, copy=True)
    flat = out.reshape(-1)
    lib().lco_sanitize(_p(flat), flat.size)
    return out


def ingest(qtype: int, data: np.ndarray, count: int) -> np.ndarray:
    """A tensor's values as the reference's loader leaves them: dequantised
    (loader.rs:205-235), then sanitised (loader.rs:241-249)."""
    return sanitize(dequant(qtype, data, count))


def quantize(qtype: int, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    out = np.zeros(tensor_size(qtype, x.size), np.uint8)
    assert lib().lco_quantize(qtype, _p(x), _p(out), x.size) == 0
    return out


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().lco_f32_to_f16_n(_p(x), _p(out), x.size)
    return out


def f16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().lco_f16_to_f32_n(_p(h), _p(out), h.size)
    return out


def scale_min_k4(j: int, scales12: bytes):
    q = np.frombuffer(bytes(scales12), np.uint8).copy()
    sc = (C.c_uint8 * 1)()
    m = (C.c_uint8 * 1)()
    lib().lco_scale_min_k4(j, _p(q), sc, m)
    return int(sc[0]), int(m[0])


def scan_blocks(qtype: int, data: np.ndarray, count: int) -> int:
    data = np.ascontiguousarray(data, dtype=np.uint8)
    return int(lib().lco_scan_blocks(qtype, _p(data), count))


def synth_normal(seed: int, stream: int, std: float, n: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().lco_synth_normal(seed, stream, std, _p(out), n)
    return out


# ---- arithmetic --------------------------------------------------------------

def matmul(a: np.ndarray, b: np.ndarray, threads: int = 1) -> np.ndarray:
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    m, k = a.shape
    k2, n = b.shape
    assert k == k2
    c = np.empty((m, n), np.float32)
    lib().lco_matmul(_p(a), _p(b), _p(c), m, k, n, threads)
    return c


def silu(v: float) -> float:
    return float(lib().lco_silu(v))


def rms_norm(x: np.ndarray, w: np.ndarray, eps: float = 1e-5) -> np.ndarray:
    """CpuBackend::rms_norm over the rows of x [T, d] (lco_rms_norm)."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    T, d = x.shape
    out = np.empty_like(x)
    lib().lco_rms_norm(_p(x), _p(w), eps, T, d, _p(out))
    return out


def softmax(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32).ravel()
    y = np.empty_like(x)
    lib().lco_softmax(_p(x), _p(y), x.size)
    return y


def expf_cw(x: np.ndarray) -> np.ndarray:
    f = lib().lco_expf_cw
    return np.array([f(float(v)) for v in np.asarray(x, np.float32).ravel()], np.float32)


def sigmoid_cw(x: np.ndarray) -> np.ndarray:
    f = lib().lco_sigmoid_cw
    return np.array([f(float(v)) for v in np.asarray(x, np.float32).ravel()], np.float32)


def sigmoid_max_dip(threads: int = 8) -> int:
    """Exhaustive: the largest dip of sigmoid_cw below its running maximum
    over every non-NaN float, in ulps (lco_sigmoid_max_dip)."""
    return int(lib().lco_sigmoid_max_dip(threads))


def router_logits(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    T, d = x.shape
    d2, E = w.shape
    assert d == d2
    out = np.empty((T, E), np.float32)
    lib().lco_router_logits(_p(x), _p(w), _p(out), T, d, E)
    return out


def route(desc: Desc, logits: np.ndarray, bias=None):
    logits = np.ascontiguousarray(logits, np.float32)
    T = logits.shape[0]
    K = desc.n_expert_used
    idx = np.empty((T, K), np.int32)
    w = np.empty((T, K), np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    rc = lib().lco_route(C.byref(desc), _p(logits), _p(b), T, _p(idx), _p(w))
    assert rc == 0
    return idx, w


def dispatch(topk_idx: np.ndarray, E: int):
    topk_idx = np.ascontiguousarray(topk_idx, np.int32)
    T, K = topk_idx.shape
    counts = np.empty(E, np.int32)
    offsets = np.empty(E + 1, np.int32)
    perm = np.empty(T * K, np.int32)
    inv = np.empty(T * K, np.int32)
    rc = lib().lco_dispatch(_p(topk_idx), T, K, E, _p(counts), _p(offsets), _p(perm), _p(inv))
    if rc != 0:
        raise ValueError("expert index out of range")
    return counts, offsets, perm, inv


def ffn_dense(x, wg_t, wu_t, wd_t, threads: int = 1):
    x = np.ascontiguousarray(x, np.float32)
    m, d = x.shape
    F = wg_t.shape[1]
    # keep the contiguous copies alive across the call
    wg_c = np.ascontiguousarray(wg_t, np.float32)
    wu_c = np.ascontiguousarray(wu_t, np.float32)
    wd_c = np.ascontiguousarray(wd_t, np.float32)
    y = np.empty((m, d), np.float32)
    lib().lco_ffn_dense(_p(x), m, d, F, _p(wg_c), _p(wu_c), _p(wd_c), _p(y), threads)
    return y


def _weights_struct(layer) -> Weights:
    """Pointers into `layer`; the arrays must be C-contiguous (float32 router
    and bias, uint8 tensors) and stay alive while the struct is used."""
    w = Weights()
    for k in ("router", "bias", "gate", "up", "down", "gate_sh", "up_sh", "down_sh"):
        a = layer.get(k)
        if a is not None:
            assert a.flags["C_CONTIGUOUS"], k
            assert a.dtype == (np.float32 if k in ("router", "bias") else np.uint8), k
        setattr(w, k, _p(a))
    return w


def moe_forward(desc: Desc, layer: dict, x: np.ndarray, threads: int = 1) -> dict:
    """Whole MoE layer.  `layer` holds numpy arrays: router [d,E] f32, bias
    [E] f32 or None, gate/up/down (uint8, E stacked GGUF tensors), and the
    shared-expert tensors when desc.n_shared > 0."""
    x = np.ascontiguousarray(x, np.float32)
    T = x.shape[0]
    K, E, D = desc.n_expert_used, desc.n_expert, desc.d_model
    out = {
        "y": np.empty((T, D), np.float32),
        "topk_idx": np.empty((T, K), np.int32),
        "topk_w": np.empty((T, K), np.float32),
        "counts": np.empty(E, np.int32),
        "offsets": np.empty(E + 1, np.int32),
        "perm": np.empty(T * K, np.int32),
        "inv": np.empty(T * K, np.int32),
    }
    w = _weights_struct(layer)
    rc = lib().lco_moe_forward(C.byref(desc), C.byref(w), _p(x), T, _p(out["y"]),
                               _p(out["topk_idx"]), _p(out["topk_w"]), _p(out["counts"]),
                               _p(out["offsets"]), _p(out["perm"]), _p(out["inv"]), threads)
    if rc != 0:
        raise ValueError("oracle rejected the descriptor")
    return out


class Resident:
    """CPU baseline: experts dequantised to f32 once, then forward calls."""

    def __init__(self, desc: Desc, layer: dict, threads: int = 0):
        self._desc = desc
        self._layer = layer  # keep host arrays alive
        self._w = _weights_struct(layer)
        self._h = lib().lco_resident_create(C.byref(desc), C.byref(self._w), threads)
        if not self._h:
            raise ValueError("oracle rejected the descriptor")

    def forward(self, x: np.ndarray, threads: int = 0) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty_like(x)
        lib().lco_resident_forward(self._h, _p(x), x.shape[0], _p(y), threads)
        return y

    def close(self):
        if self._h:
            lib().lco_resident_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


Q4_0_SHARD = 2


def shard_matmul(qtype: int, a: np.ndarray, b: np.ndarray, k: int, n: int) -> np.ndarray:
    """int8_gemm.rs q8_0_matmul / q4_0_matmul on x86 (lco_shard_matmul):
    a [m, k] f32, b the shard blocks as bytes."""
    a = np.ascontiguousarray(a, np.float32)
    if a.ndim != 2:
        a = a.reshape(-1, k)
    b = np.ascontiguousarray(b, np.uint8)
    m = a.shape[0]
    out = np.zeros((m, n), np.float32)
    if lib().lco_shard_matmul(qtype, _p(a), _p(b), _p(out), m, k, n) != 0:
        raise ValueError("lco_shard_matmul: bad type or shape")
    return out


# ---- decoder-layer pieces ------------------------------------------------------

def rope(x: np.ndarray, heads: int, hd: int, theta: float, pos0: int = 0) -> np.ndarray:
    """apply_rotary_emb (attention.rs:13-34) on x [seq, heads * hd]; returns a copy."""
    y = np.ascontiguousarray(x, np.float32).copy()
    lib().lco_rope(_p(y), y.shape[0], heads, hd, theta, pos0)
    return y


def attention_core(q, k, v, heads: int, kv_heads: int, hd: int) -> np.ndarray:
    """attention_forward's core (attention.rs:56-115): q [seq, heads*hd] after
    RoPE, k / v [total, kv_heads*hd] the decompressed cache."""
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    seq, total = q.shape[0], k.shape[0]
    out = np.empty((seq, heads * hd), np.float32)
    lib().lco_attention_core(_p(q), _p(k), _p(v), seq, total, heads, kv_heads, hd, _p(out))
    return out


def argmax_last(x: np.ndarray) -> int:
    """Greedy sample_top_p (sampler.rs:8-10): the last maximum under total_cmp."""
    x = np.ascontiguousarray(x, np.float32).ravel()
    return int(lib().lco_argmax_last(_p(x), x.size))
