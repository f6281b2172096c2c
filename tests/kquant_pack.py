"""Independent block packers used to pin the decoders.

These build GGUF blocks from *logical* contents (scales, mins, integer quants)
by writing bit fields, i.e. in the encoding direction, from the block layouts
that rust/src/kernels/mod.rs decodes:

Q4_K (144 B, kernels/mod.rs:66-98): f16 d @0, f16 dmin @2, 12 scale bytes @4,
  128 qs bytes @16.  Element 64*j + l (l < 32) is the low nibble of qs[32*j+l]
  and uses sub-block 2*j; element 64*j + 32 + l is the high nibble of the same
  byte and uses sub-block 2*j+1.  6-bit (sc, m) pairs for sub-blocks 0..3 sit in
  the low 6 bits of scale bytes 0..3 / 4..7; for sub-blocks 4..7 the low 4 bits
  of sc / m are the low / high nibble of scale bytes 8..11 and the top 2 bits
  are the top 2 bits of bytes 0..3 (sc) / 4..7 (m)  (get_scale_min_k4,
  kernels/mod.rs:54-63).
Q6_K (210 B, kernels/mod.rs:145-180): ql[128] @0, qh[64] @128, int8 scales[16]
  @192, f16 d @208.  Element e = 128*n + 32*s + l (n < 2, s < 4, l < 32) has a
  6-bit code c = q + 32: its low 4 bits are the low (s < 2) or high (s >= 2)
  nibble of ql[64*n + 32*(s & 1) + l], its top 2 bits are bits 2s..2s+1 of
  qh[32*n + l]; it uses scale e // 16.
Q8_0 (34 B, kernels/mod.rs:37-51): f16 d @0 then 32 int8.
"""
import numpy as np


def f16_bytes(v: float) -> bytes:
    return np.array([v], np.float16).tobytes()


def pack_q4_k(d: float, dmin: float, sc, m, q) -> bytes:
    sc = [int(v) for v in sc]
    m = [int(v) for v in m]
    q = np.asarray(q, np.int64)
    assert len(sc) == 8 and len(m) == 8 and q.shape == (256,)
    assert all(0 <= v < 64 for v in sc + m) and q.min() >= 0 and q.max() < 16
    scales = bytearray(12)
    for j in range(8):
        if j < 4:
            scales[j] |= sc[j] & 0x3F
            scales[j + 4] |= m[j] & 0x3F
        else:
            scales[j + 4] |= (sc[j] & 0x0F) | ((m[j] & 0x0F) << 4)
            scales[j - 4] |= (sc[j] >> 4) << 6
            scales[j] |= (m[j] >> 4) << 6
    qs = bytearray(128)
    for e in range(256):
        j, r = divmod(e, 64)
        hi, l = divmod(r, 32)
        qs[32 * j + l] |= int(q[e]) << (4 * hi)
    return f16_bytes(d) + f16_bytes(dmin) + bytes(scales) + bytes(qs)


def pack_q6_k(d: float, sc, q) -> bytes:
    sc = [int(v) for v in sc]
    q = np.asarray(q, np.int64)
    assert len(sc) == 16 and q.shape == (256,) and q.min() >= -32 and q.max() < 32
    ql = bytearray(128)
    qh = bytearray(64)
    for e in range(256):
        n, w = divmod(e, 128)
        s, l = divmod(w, 32)
        c = int(q[e]) + 32
        ql[64 * n + 32 * (s & 1) + l] |= (c & 15) << (0 if s < 2 else 4)
        qh[32 * n + l] |= (c >> 4) << (2 * s)
    return bytes(ql) + bytes(qh) + np.array(sc, np.int8).tobytes() + f16_bytes(d)


def pack_q8_0(d: float, q) -> bytes:
    q = np.asarray(q, np.int64)
    assert q.shape == (32,)
    return f16_bytes(d) + q.astype(np.int8).tobytes()


def expected_q4_k(d, dmin, sc, m, q):
    """Element values from logical contents, float32, two roundings."""
    d32, m32 = np.float32(np.float16(d)), np.float32(np.float16(dmin))
    out = np.empty(256, np.float32)
    for e in range(256):
        j = e // 32
        out[e] = np.float32(d32 * np.float32(sc[j])) * np.float32(q[e]) - np.float32(m32 * np.float32(m[j]))
    return out


def expected_q6_k(d, sc, q):
    d32 = np.float32(np.float16(d))
    out = np.empty(256, np.float32)
    for e in range(256):
        out[e] = np.float32(d32 * np.float32(sc[e // 16])) * np.float32(q[e])
    return out
