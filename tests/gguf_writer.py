"""Minimal GGUF v3 writer for the GGUF ingest tests.

Written from the file layout (header, typed metadata, tensor infos, data
section aligned to general.alignment, each tensor's offset aligned too), not
from any reader in this repository, so a round trip through it checks the
readers independently.  Metadata values are given as (type code, value):
0 U8, 1 I8, 2 U16, 3 I16, 4 U32, 5 I32, 6 F32, 7 BOOL, 8 STRING, 9 ARRAY
(value = (element type, [element values])), 10 U64, 11 I64, 12 F64.
"""
from __future__ import annotations

import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f",
        BOOL: "<?", U64: "<Q", I64: "<q", F64: "<d"}

T_F32, T_F16, T_Q8_0, T_Q4_K, T_Q6_K, T_BF16 = 0, 1, 8, 12, 14, 30


def _str(s) -> bytes:
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _value(typ: int, v) -> bytes:
    if typ == STRING:
        return _str(v)
    if typ == ARRAY:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(_value(et, x) for x in items)
    return struct.pack(_FMT[typ], v)


def gguf_header(metadata, infos, alignment: int = 32, version: int = 3,
                magic: int = 0x46554747) -> bytes:
    """Header, metadata and tensor infos (name, dims ne0-first, ggml type,
    data-relative offset), zero-padded to `alignment`."""
    head = struct.pack("<IIQQ", magic, version, len(infos), len(metadata))
    for key, typ, v in metadata:
        head += _str(key) + struct.pack("<I", typ) + _value(typ, v)
    for name, dims, typ, off in infos:
        head += _str(name) + struct.pack("<I", len(dims))
        head += b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", typ, off)
    return head + b"\0" * ((alignment - len(head) % alignment) % alignment)


def gguf_bytes(metadata, tensors, alignment: int = 32, version: int = 3,
               magic: int = 0x46554747) -> bytes:
    """metadata: list of (key, type, value); tensors: list of
    (name, dims ne0-first, ggml type, payload bytes), packed in order with
    each offset rounded up to `alignment`.  `alignment` lays out the file; it
    is written as general.alignment only if metadata has it."""
    infos, body = [], bytearray()
    for name, dims, typ, payload in tensors:
        body += b"\0" * ((alignment - len(body) % alignment) % alignment)
        infos.append((name, dims, typ, len(body)))
        body += bytes(payload)
    return gguf_header(metadata, infos, alignment, version, magic) + bytes(body)


def write(path, metadata, tensors, **kw) -> None:
    with open(path, "wb") as f:
        f.write(gguf_bytes(metadata, tensors, **kw))


def f32(a) -> bytes:
    return np.ascontiguousarray(a, "<f4").tobytes()


def moe_tensors(layer: int, lay: dict, d: int, F: int, E: int, types, *,
                per_expert: bool = False, shared=None, bias_name=None,
                router_type: int = T_F32) -> list:
    """GGUF tensors of one MoE layer from the arrays the library's direct
    API takes: router [d, E] f32 (written as dims [d, E], i.e. E rows of d),
    stacked expert bytes, optional shared (S, Fs, types) and bias."""
    pre = f"blk.{layer}."
    r = np.ascontiguousarray(np.asarray(lay["router"], np.float32).T)  # [E, d]
    if router_type == T_F32:
        rb = f32(r)
    elif router_type == T_F16:
        rb = r.astype("<f2").tobytes()
    else:  # BF16: keep the high half of each f32 (exact when the low half is 0)
        rb = (r.view(np.uint32) >> 16).astype("<u2").tobytes()
    out = [(pre + "ffn_gate_inp.weight", [d, E], router_type, rb)]
    kinds = (("gate", [d, F]), ("up", [d, F]), ("down", [F, d]))
    for (k, dims), t in zip(kinds, types):
        blob = np.asarray(lay[k], np.uint8).tobytes()
        if per_expert:
            n = len(blob) // E
            for e in range(E):
                out.append((pre + f"ffn_{k}.{e}.weight", dims, t, blob[e * n:(e + 1) * n]))
        else:
            out.append((pre + f"ffn_{k}_exps.weight", dims + [E], t, blob))
    if shared is not None:
        S, Fs, st = shared
        kinds = (("gate", [d, Fs]), ("up", [d, Fs]), ("down", [Fs, d]))
        for (k, dims), t in zip(kinds, st):
            blob = np.asarray(lay[k + "_sh"], np.uint8).tobytes()
            out.append((pre + f"ffn_{k}_shexp.weight", dims + ([S] if S > 1 else []), t, blob))
    if bias_name is not None:
        out.append((pre + bias_name, [E], T_F32, f32(lay["bias"])))
    return out
