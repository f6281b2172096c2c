"""Host-side mirror of the reference layer API over the C ABI.

`MoeFfn.ffn_forward(x) -> y` has the contract of the reference's
Engine::ffn_forward (rust/src/inference/engine.rs:146-164): x [T, d_model]
f32 in, y [T, d_model] f32 out, synchronous, residual add left to the caller
(engine.rs:115).  Errors raise LcmoeError carrying the ABI status (the
reference panics; a caller that wants that can let the exception propagate).
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import Desc, LcmoeError, Weights, check, lib


def _ptr(a):
    return None if a is None else a.ctypes.data


class MoeFfn:
    """One resident MoE layer on the current HIP device."""

    def __init__(self, desc: Desc, layer: dict):
        self.desc = desc
        w = Weights()
        router = np.ascontiguousarray(layer["router"], np.float32)
        keep = [router]  # the arrays must outlive lcmoe_create, which copies them
        w.router = _ptr(router)
        bias = layer.get("bias")
        if bias is not None:
            bias = np.ascontiguousarray(bias, np.float32)
            keep.append(bias)
        w.bias = _ptr(bias)
        for k in ("gate", "up", "down", "gate_sh", "up_sh", "down_sh"):
            a = layer.get(k)
            if a is not None:
                a = np.ascontiguousarray(a, np.uint8)
                keep.append(a)
            setattr(w, k, _ptr(a))
        self._create(desc, w)

    def _create(self, desc: Desc, w: Weights) -> None:
        h = C.c_void_p()
        check(lib().lcmoe_create(C.byref(desc), C.byref(w), C.byref(h)), "lcmoe_create")
        self._h = h

    @classmethod
    def from_gguf(cls, source, layer: int, max_tokens: int) -> "MoeFfn":
        """MoE layer `layer` of a GGUF file (a path or an open GgufFile),
        uploaded resident: GgufFile.moe_layer then lcmoe_create, which copies
        the weights, so the file may be closed afterwards."""
        from .gguf import GgufFile

        f = source if isinstance(source, GgufFile) else GgufFile(source)
        try:
            desc, w = f.moe_layer(layer, max_tokens)
            self = cls.__new__(cls)
            self.desc = desc
            self._create(desc, w)
            return self
        finally:
            if f is not source:
                f.close()

    @property
    def handle(self) -> int:
        return self._h.value

    def ffn_forward(self, x: np.ndarray) -> np.ndarray:
        return self.forward(x)[0]

    def forward(self, x: np.ndarray):
        """Returns (y, topk_idx, topk_w)."""
        x = np.ascontiguousarray(x, np.float32)
        if x.ndim != 2 or x.shape[1] != self.desc.d_model:
            raise LcmoeError(1, "ffn_forward", f"x must be [T, {self.desc.d_model}]")
        T, K = x.shape[0], self.desc.n_expert_used
        y = np.empty_like(x)
        idx = np.empty((T, K), np.int32)
        w = np.empty((T, K), np.float32)
        check(lib().lcmoe_forward(self._h, _ptr(x), T, _ptr(y), _ptr(idx), _ptr(w)),
              "lcmoe_forward")
        return y, idx, w

    def forward_dev(self, x_dev: int, T: int, y_dev: int, stream: int | None = None) -> None:
        check(lib().lcmoe_forward_dev(self._h, x_dev, T, y_dev, stream), "lcmoe_forward_dev")

    def set_act_precision(self, mode: int) -> None:
        """ACT_F16 (default) or ACT_F16X2: how x enters the matrix-core
        gate/up products (lcmoe_set_act_precision)."""
        check(lib().lcmoe_set_act_precision(self._h, int(mode)), "lcmoe_set_act_precision")

    def set_norm(self, weight: np.ndarray, eps: float = 1e-5) -> None:
        """Post-attention RMSNorm weight [d_model] for forward_norm_residual."""
        weight = np.ascontiguousarray(weight, np.float32)
        if weight.shape != (self.desc.d_model,):
            raise LcmoeError(1, "set_norm", f"weight must be [{self.desc.d_model}]")
        check(lib().lcmoe_set_norm(self._h, _ptr(weight), eps), "lcmoe_set_norm")

    def forward_norm_residual(self, hidden: np.ndarray):
        """hidden + ffn_forward(rms_norm(hidden)) (engine.rs:110-115);
        returns (out, topk_idx, topk_w)."""
        hidden = np.ascontiguousarray(hidden, np.float32)
        if hidden.ndim != 2 or hidden.shape[1] != self.desc.d_model:
            raise LcmoeError(1, "forward_norm_residual", f"hidden must be [T, {self.desc.d_model}]")
        T, K = hidden.shape[0], self.desc.n_expert_used
        out = np.empty_like(hidden)
        idx = np.empty((T, K), np.int32)
        w = np.empty((T, K), np.float32)
        check(lib().lcmoe_forward_norm_residual(self._h, _ptr(hidden), T, _ptr(out), _ptr(idx),
                                                _ptr(w)), "lcmoe_forward_norm_residual")
        return out, idx, w

    def forward_norm_residual_dev(self, hidden_dev: int, T: int, out_dev: int,
                                  stream: int | None = None) -> None:
        check(lib().lcmoe_forward_norm_residual_dev(self._h, hidden_dev, T, out_dev, stream),
              "lcmoe_forward_norm_residual_dev")

    def dispatch(self) -> dict:
        E, K = self.desc.n_expert, self.desc.n_expert_used
        T = C.c_int32()
        check(lib().lcmoe_get_dispatch(self._h, C.byref(T), None, None, None, None, None, None),
              "lcmoe_get_dispatch")
        T = T.value
        out = {
            "topk_idx": np.empty((T, K), np.int32), "topk_w": np.empty((T, K), np.float32),
            "counts": np.empty(E, np.int32), "offsets": np.empty(E + 1, np.int32),
            "perm": np.empty(T * K, np.int32), "inv": np.empty(T * K, np.int32),
        }
        check(lib().lcmoe_get_dispatch(self._h, None, *(_ptr(out[k]) for k in (
            "topk_idx", "topk_w", "counts", "offsets", "perm", "inv"))), "lcmoe_get_dispatch")
        return out

    def route_fallbacks(self) -> int:
        """Tokens of the last forward that the parallel-bounds certified
        router (sigmoid-group kind; softmax kinds at one token with E >= 32)
        left to the exact chain logits; -1 when that forward did not use it."""
        n = np.zeros(1, np.int32)
        check(lib().lcmoe_debug_route_fallbacks(self._h, _ptr(n)), "lcmoe_debug_route_fallbacks")
        return int(n[0])

    def set_timing(self, on: bool) -> None:
        check(lib().lcmoe_set_timing(self._h, 1 if on else 0), "lcmoe_set_timing")

    def get_timing(self) -> dict:
        n = lib().lcmoe_timing_slots()
        ms = np.zeros(n, np.float64)
        cnt = np.zeros(n, np.int64)
        check(lib().lcmoe_get_timing(self._h, n, _ptr(ms), _ptr(cnt)), "lcmoe_get_timing")
        return {lib().lcmoe_timing_name(i).decode(): (float(ms[i]), int(cnt[i])) for i in range(n)}

    def close(self) -> None:
        if getattr(self, "_h", None) is not None and self._h.value:
            lib().lcmoe_destroy(self._h)
            self._h = C.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def dequantize(qtype: int, data: np.ndarray, count: int, sanitize: bool = True) -> np.ndarray:
    """GGUFModel::dequantize (+ sanitize_weights) on the host:
    lcmoe_dequantize."""
    data = np.ascontiguousarray(data, np.uint8)
    out = np.empty(count, np.float32)
    n = lib().lcmoe_dequantize(qtype, data.ctypes.data, count, out.ctypes.data, int(sanitize))
    if n < 0:
        raise ValueError(f"lcmoe_dequantize: bad type {qtype} or count {count}")
    return out


def sanitize_blocks(qtype: int, data: np.ndarray, count: int):
    """sanitize_weights on GGUF bytes, on a copy (lcmoe_sanitize_blocks):
    (bytes, elements zeroed, outliers Q4_K could not zero in place)."""
    out = np.array(data, np.uint8, copy=True)
    unz = C.c_int64()
    n = lib().lcmoe_sanitize_blocks(qtype, out.ctypes.data, count, C.byref(unz))
    if n < 0:
        raise ValueError(f"lcmoe_sanitize_blocks: bad type {qtype} or count {count}")
    return out, int(n), int(unz.value)


def debug_dequant(qtype: int, data: np.ndarray, count: int) -> np.ndarray:
    data = np.ascontiguousarray(data, np.uint8)
    out = np.empty(count, np.float32)
    check(lib().lcmoe_debug_dequant(qtype, _ptr(data), count, _ptr(out)), "lcmoe_debug_dequant")
    return out


def debug_sigmoid(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32).ravel()
    out = np.empty_like(x)
    check(lib().lcmoe_debug_sigmoid(_ptr(x), x.size, _ptr(out)), "lcmoe_debug_sigmoid")
    return out


def debug_rmsnorm(x: np.ndarray, w: np.ndarray, eps: float = 1e-5) -> np.ndarray:
    """The device RMSNorm over the rows of x [T, d]."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    out = np.empty_like(x)
    check(lib().lcmoe_debug_rmsnorm(_ptr(x), _ptr(w), eps, x.shape[0], x.shape[1], _ptr(out)),
          "lcmoe_debug_rmsnorm")
    return out


def shard_matmul(qtype: int, a: np.ndarray, b: np.ndarray, k: int, n: int) -> np.ndarray:
    """C = A B for the shard engine's Q8_0 / Q4_0 matrices (Tensor::matmul's
    quantised arms, tensor.rs:118-128) on the GPU: a [m, k] f32, b the block
    bytes (k rows of n/32 blocks along n)."""
    a = np.ascontiguousarray(a, np.float32)
    if a.ndim != 2:
        a = a.reshape(-1, k)
    b = np.ascontiguousarray(b, np.uint8)
    out = np.empty((a.shape[0], n), np.float32)
    check(lib().lcmoe_shard_matmul(qtype, _ptr(a), _ptr(b), _ptr(out), a.shape[0], k, n),
          "lcmoe_shard_matmul")
    return out


def read_bandwidth(slice_mib: int, reps: int = 8) -> float:
    """HBM streaming-read rate in GB/s over distinct `slice_mib` MiB slices
    (lcmoe_debug_read_bandwidth)."""
    out = np.zeros(1, np.float64)
    check(lib().lcmoe_debug_read_bandwidth(slice_mib << 20, reps, _ptr(out)),
          "lcmoe_debug_read_bandwidth")
    return float(out[0])


def matmul(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Backend::matmul (rust/src/backend/mod.rs:18-46) on the GPU:
    a [m, k] @ b [k, n] in f32, bit-identical to the x86 CPU backend
    (lcmoe_matmul_f32)."""
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    if a.ndim != 2 or b.ndim != 2 or a.shape[1] != b.shape[0]:
        raise LcmoeError(1, "matmul", f"shapes {a.shape} @ {b.shape}")
    m, k = a.shape
    n = b.shape[1]
    c = np.empty((m, n), np.float32)
    check(lib().lcmoe_matmul_f32(_ptr(a), _ptr(b), c.ctypes.data, m, k, n), "lcmoe_matmul_f32")
    return c
