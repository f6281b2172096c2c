"""Packs the shard engine's quantised matrices (rust/src/kernels/q8_0.rs,
q4_0.rs) from integer codes and scales, written from the block layout alone
(f16 scale then the codes; Q4_0 element 2t in the low nibble of byte t).
B is [k, n]: k rows of n/32 blocks along n."""
import numpy as np


def pack_q8(scales: np.ndarray, q: np.ndarray) -> np.ndarray:
    """scales [k, n/32] (rounded to f16), q [k, n] int8 codes."""
    k, n = q.shape
    out = np.zeros((k, n // 32, 34), np.uint8)
    out[:, :, :2] = np.asarray(scales, np.float16).reshape(k, n // 32, 1).view(np.uint8)
    out[:, :, 2:] = np.asarray(q, np.int8).reshape(k, n // 32, 32).view(np.uint8)
    return out.reshape(-1)


def pack_q4(scales: np.ndarray, nib: np.ndarray) -> np.ndarray:
    """scales [k, n/32], nib [k, n] codes 0..15 (value = code - 8)."""
    k, n = nib.shape
    nb = np.asarray(nib, np.uint8).reshape(k, n // 32, 16, 2)
    out = np.zeros((k, n // 32, 18), np.uint8)
    out[:, :, :2] = np.asarray(scales, np.float16).reshape(k, n // 32, 1).view(np.uint8)
    out[:, :, 2:] = nb[..., 0] | (nb[..., 1] << 4)
    return out.reshape(-1)


def dequant(qtype: int, scales: np.ndarray, codes: np.ndarray) -> np.ndarray:
    """[k, n] f32 weights: code (minus 8 for Q4_0) times the f16 scale."""
    k, n = codes.shape
    s = np.repeat(np.asarray(scales, np.float16).astype(np.float32), 32, axis=1)
    v = codes.astype(np.float32) - (8.0 if qtype == 2 else 0.0)
    return (v * s).astype(np.float32)


def reference_test_matrices(qtype: int, rows: int, cols: int):
    """make_test_matrix / make_q4_test_matrix (int8_gemm.rs:377-393,
    :447-463): scale 0.01 (row + 1); Q8 codes (b*32 + jj) as i8 - 16
    (wrapping), Q4 codes min(8 + c % 8, 15) for column c."""
    scales = np.array([[0.01 * (r + 1)] * (cols // 32) for r in range(rows)], np.float32)
    c = np.arange(cols)
    if qtype == 8:
        codes = np.tile(((c.astype(np.int64) - 16 + 128) % 256 - 128).astype(np.int8), (rows, 1))
    else:
        codes = np.tile(np.minimum(8 + c % 8, 15).astype(np.uint8), (rows, 1))
    return scales, codes
