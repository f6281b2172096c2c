"""Pure-Python restatement of the reference GGUF reader and of the MoE layer
mapping the product's GGUF ingest implements.

TEST INFRASTRUCTURE ONLY: imported by tests/ as the checker of the product's
GGUF reader (leafcutterllm_amd/csrc/lcmoe_gguf.cpp).  The product package never
imports it.

Reader, following rust/src/model/gguf.rs:
  header            read_header        :169-176  magic u32, version u32,
                                                  tensor_count u64, metadata_count u64
  magic / version   GGUFile::open      :82-87    0x46554747, version 3 only
  metadata KV       read_metadata_kv   :178-183  string key, u32 type, value
  values            read_value         :185-210  types 0..12, 9 = array
                                                  (u32 elem type, u64 len, elems)
  tensor info       read_tensor_info   :212-227  string name, u32 n_dims,
                                                  u64 dims, u32 type, u64 offset
  strings           read_string        :296-304  u64 length + bytes
  data offset       GGUFile::open      :100-110  general.alignment (U32/U64,
                                                  default 32), pad to it
  tensor bytes      get_tensor_raw     :121-127  data_offset + offset,
                                                  calculate_tensor_size long
  tensor size       calculate_tensor_size :307-313 with
                    QuantType::tensor_size (rust/src/model/quant.rs:256-261,
                    block geometry :170-239; unknown types: count bytes)
  integer metadata  get_metadata_int   :133-157
  2D load           GGUFModel::load_layer (rust/src/model/loader.rs:145-168):
                    dims reversed into the shape, 2D tensors transposed

Parity pins (tests/test_gguf_cpu.py): the reference's own known answers for
calculate_tensor_size (gguf.rs:338-346) and the tensor sizes and contiguous
offsets a real file showed (rust/TEST_REPORT.md:158-167, a Qwen2.5-3B file),
plus round trips through an independently written GGUF writer
(tests/gguf_writer.py).  The MoE mapping (moe_layer) has no counterpart in
the reference (arch.rs:83-96 maps dense tensors only): it restates the
product's written mapping, and is pinned by those round trips alone.
"""
from __future__ import annotations

import struct

import numpy as np

GGUF_MAGIC = 0x46554747
GGUF_VERSION = 3

# QuantType::block_size / block_bytes (quant.rs:170-239) for the codes shared
# with ggml; F16 = 1, BF16 = 30
_GEOM = {0: (1, 4), 1: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24),
         8: (32, 34), 9: (32, 36), 10: (256, 84), 11: (256, 110), 12: (256, 144),
         13: (256, 176), 14: (256, 210), 15: (256, 292), 16: (256, 66), 17: (256, 74),
         18: (256, 98), 30: (1, 2)}

_SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 10: "<Q",
           11: "<q", 12: "<d"}


class GgufError(Exception):
    """kind: 'magic', 'version', 'truncated', 'value_type' (the GGUError
    variants, gguf.rs:17-31)."""

    def __init__(self, kind: str, msg: str = ""):
        self.kind = kind
        super().__init__(f"{kind}: {msg}")


def tensor_size(dims, typ: int) -> int:
    """calculate_tensor_size, gguf.rs:307-313 (ceil blocks; unknown: count)."""
    count = 1
    for d in dims:
        count *= int(d)
    if typ in _GEOM:
        bs, bb = _GEOM[typ]
        return (count + bs - 1) // bs * bb
    return count


class _Reader:
    def __init__(self, data):
        self.data = data
        self.pos = 0

    def take(self, n: int) -> bytes:
        if self.pos + n > len(self.data):
            raise GgufError("truncated", f"need {n} bytes at {self.pos}")
        b = bytes(self.data[self.pos:self.pos + n])
        self.pos += n
        return b

    def scalar(self, fmt: str):
        return struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]

    def string(self) -> bytes:
        n = self.scalar("<Q")
        return self.take(n)

    def value(self, typ: int):
        """(type, python value); arrays are ('arr', elem type, [values])."""
        if typ in _SCALAR:
            return typ, self.scalar(_SCALAR[typ])
        if typ == 7:
            return typ, self.scalar("<B") != 0
        if typ == 8:
            return typ, self.string()
        if typ == 9:
            et = self.scalar("<I")
            n = self.scalar("<Q")
            return typ, (et, [self.value(et) for _ in range(n)])
        raise GgufError("value_type", str(typ))


class GgufRef:
    """GGUFile (gguf.rs:33-127) over a bytes-like object."""

    def __init__(self, data):
        r = _Reader(data)
        magic, version = r.scalar("<I"), r.scalar("<I")
        n_tensors, n_kv = r.scalar("<Q"), r.scalar("<Q")
        if magic != GGUF_MAGIC:
            raise GgufError("magic", hex(magic))
        if version != GGUF_VERSION:
            raise GgufError("version", str(version))
        self.metadata = {}
        for _ in range(n_kv):
            key = r.string().decode("utf-8", "replace")
            typ = r.scalar("<I")
            self.metadata[key] = r.value(typ)
        self.tensors = []
        for _ in range(n_tensors):
            name = r.string().decode("utf-8", "replace")
            nd = r.scalar("<I")
            dims = [r.scalar("<Q") for _ in range(nd)]
            typ = r.scalar("<I")
            off = r.scalar("<Q")
            self.tensors.append({"name": name, "dims": dims, "type": typ, "offset": off})
        align = 32
        a = self.metadata.get("general.alignment")
        if a is not None and a[0] in (4, 10):
            align = a[1]
        pos = r.pos
        self.data_offset = pos + (align - pos % align) % align
        self.data = data

    def info(self, name: str):
        for t in self.tensors:
            if t["name"] == name:
                return t
        return None

    def raw(self, name: str):
        t = self.info(name)
        if t is None:
            return None
        start = self.data_offset + t["offset"]
        end = start + tensor_size(t["dims"], t["type"])
        if end > len(self.data):
            raise GgufError("truncated", f"{name} ends at {end} > {len(self.data)}")
        return np.frombuffer(self.data, np.uint8, end - start, start)

    def meta_int(self, key: str):
        """get_metadata_int, gguf.rs:133-157 (None where the reference gives None)."""
        v = self.metadata.get(key)
        if v is None:
            return None
        typ, val = v
        if typ in (0, 1, 2, 3, 4, 5, 10, 11):
            return _wrap_i64(val)
        if typ in (6, 12):
            return _f_as_i64(val)
        if typ == 9:
            et, arr = val
            if len(arr) == 1 and et in (4, 5, 10, 11):
                return _wrap_i64(arr[0][1])
        return None

    def meta_str(self, key: str):
        v = self.metadata.get(key)
        return v[1] if v is not None and v[0] == 8 else None

    def floats(self, name: str) -> np.ndarray:
        """F32 / F16 / BF16 tensor as f32, in file order."""
        t = self.info(name)
        raw = self.raw(name)
        if t["type"] == 0:
            return raw.view("<f4").astype(np.float32)
        if t["type"] == 1:
            return raw.view("<f2").astype(np.float32)
        if t["type"] == 30:
            return (raw.view("<u2").astype(np.uint32) << 16).view(np.float32)
        raise ValueError(f"{name}: type {t['type']} is not a float type")

    def load_2d(self, name: str) -> np.ndarray:
        """load_layer's treatment of a 2D float tensor (loader.rs:155-160):
        shape = reversed dims, then transposed -> [dims[0], dims[1]]."""
        t = self.info(name)
        ne0, ne1 = t["dims"]
        m = self.floats(name).reshape(ne1, ne0)  # shape reversed
        return np.ascontiguousarray(m.T)          # transposed


def _wrap_i64(v: int) -> int:
    v &= (1 << 64) - 1
    return v - (1 << 64) if v >= 1 << 63 else v


def _f_as_i64(f: float) -> int:
    if f != f:
        return 0
    if f >= 2.0 ** 63:
        return (1 << 63) - 1
    if f <= -(2.0 ** 63):
        return -(1 << 63)
    return int(f)


# ---- MoE layer mapping (no reference counterpart; the product's spec) -----

_NORM_DEFAULT = {"llama": True, "mixtral": True, "qwen3moe": True,
                 "qwen2moe": False, "olmoe": False, "deepseek2": False}


class MappingError(Exception):
    """status: the lcmoe_status name the product returns for this case."""

    def __init__(self, status: str, msg: str = ""):
        self.status = status
        super().__init__(f"{status}: {msg}")


def moe_layer(g: GgufRef, layer: int):
    """(desc dict without max_tokens, layer dict of numpy arrays) of MoE
    layer `layer`; raises MappingError with the product's status name."""
    pre = f"blk.{layer}."
    arch = g.meta_str("general.architecture")
    arch = arch.decode("utf-8", "replace") if arch is not None else ""
    rt = g.info(pre + "ffn_gate_inp.weight")
    if rt is None:
        raise MappingError("LCMOE_ERR_NOT_FOUND", "no router")
    if len(rt["dims"]) != 2:
        raise MappingError("LCMOE_ERR_CORRUPT", "router dims")
    if rt["type"] not in (0, 1, 30):
        raise MappingError("LCMOE_ERR_UNSUPPORTED", "router type")
    d, E = rt["dims"]
    if g.info(pre + "ffn_gate_inp_shexp.weight") is not None:
        raise MappingError("LCMOE_ERR_UNSUPPORTED", "gated shared expert")
    out = {"router": g.load_2d(pre + "ffn_gate_inp.weight")}
    desc = {"d_model": d, "n_expert": E}

    def stacked(suffix):
        names = [pre + f"ffn_{k}{suffix}.weight" for k in ("gate", "up", "down")]
        infos = [g.info(n) for n in names]
        if all(i is None for i in infos):
            return None
        if any(i is None for i in infos):
            raise MappingError("LCMOE_ERR_NOT_FOUND", suffix)
        gd, ud, dd = (i["dims"] for i in infos)
        if len(gd) not in (2, 3):
            raise MappingError("LCMOE_ERR_CORRUPT", "expert dims")
        F = gd[1]
        n = gd[2] if len(gd) == 3 else 1
        want_gu = [d, F] + ([n] if len(gd) == 3 else [])
        want_d = [F, d] + ([n] if len(gd) == 3 else [])
        if gd != want_gu or ud != want_gu or dd != want_d:
            raise MappingError("LCMOE_ERR_CORRUPT", "expert dims disagree")
        return F, n, [i["type"] for i in infos], [g.raw(nm) for nm in names]

    r = stacked("_exps")
    if r is None:
        if g.info(pre + "ffn_gate.0.weight") is None:
            raise MappingError("LCMOE_ERR_NOT_FOUND", "no experts")
        F = g.info(pre + "ffn_gate.0.weight")["dims"][1]
        types, blobs = [], []
        for k in ("gate", "up", "down"):
            parts = []
            for e in range(E):
                t = g.info(pre + f"ffn_{k}.{e}.weight")
                if t is None:
                    raise MappingError("LCMOE_ERR_NOT_FOUND", f"{k}.{e}")
                parts.append(g.raw(t["name"]))
                if e == 0:
                    types.append(t["type"])
            blobs.append(np.concatenate(parts))
        r = (F, E, types, blobs)
    F, n, types, blobs = r
    if n != E:
        raise MappingError("LCMOE_ERR_CORRUPT", "expert count")
    desc.update(d_ff=F, type_gate=types[0], type_up=types[1], type_down=types[2])
    out.update(gate=blobs[0], up=blobs[1], down=blobs[2])
    s = stacked("_shexp")
    if s is not None:
        Fs, S, ts, bs = s
        desc.update(n_shared=S, d_ff_shared=Fs, type_gate_sh=ts[0], type_up_sh=ts[1],
                    type_down_sh=ts[2])
        out.update(gate_sh=bs[0], up_sh=bs[1], down_sh=bs[2])
    else:
        desc.update(n_shared=0, d_ff_shared=0, type_gate_sh=0, type_up_sh=0, type_down_sh=0)

    ak = arch + "."
    K = g.meta_int(ak + "expert_used_count")
    if K is None:
        raise MappingError("LCMOE_ERR_NOT_FOUND", "expert_used_count")
    for key, val in (("expert_count", E), ("embedding_length", d),
                     ("expert_feed_forward_length", F)):
        v = g.meta_int(ak + key)
        if v is not None and v != val:
            raise MappingError("LCMOE_ERR_CORRUPT", key)
    gating = g.meta_int(ak + "expert_gating_func")
    gating = 1 if gating is None else gating
    nv = g.metadata.get(ak + "expert_weights_norm")
    norm = None
    if nv is not None and nv[0] == 7:
        norm = bool(nv[1])
    elif g.meta_int(ak + "expert_weights_norm") is not None:
        norm = g.meta_int(ak + "expert_weights_norm") != 0
    sv = g.metadata.get(ak + "expert_weights_scale")
    scale = 1.0
    if sv is not None and sv[0] in (6, 12):
        scale = float(sv[1])
    elif g.meta_int(ak + "expert_weights_scale") is not None:
        scale = float(g.meta_int(ak + "expert_weights_scale"))
    n_group = g.meta_int(ak + "expert_group_count")
    n_group = 1 if n_group is None else n_group
    topk_group = g.meta_int(ak + "expert_group_used_count")
    topk_group = n_group if topk_group is None else topk_group
    sel_b = g.info(pre + "exp_probs_b.bias")
    logit_b = g.info(pre + "ffn_gate_inp.bias")
    if sel_b is not None and logit_b is not None:
        raise MappingError("LCMOE_ERR_UNSUPPORTED", "two biases")
    bt = sel_b if sel_b is not None else logit_b
    if bt is not None and (bt["dims"] != [E] or bt["type"] not in (0, 1, 30)):
        raise MappingError("LCMOE_ERR_CORRUPT", "bias shape")
    if gating in (0, 1):
        if norm is None:
            if arch not in _NORM_DEFAULT:
                raise MappingError("LCMOE_ERR_NOT_FOUND", "expert_weights_norm")
            norm = _NORM_DEFAULT[arch]
        kind = 0 if norm else 1
    elif gating == 3:
        kind = 0
    elif gating == 2:
        if norm is False:
            raise MappingError("LCMOE_ERR_UNSUPPORTED", "sigmoid without norm")
        kind = 2
    else:
        raise MappingError("LCMOE_ERR_UNSUPPORTED", "gating")
    if kind == 2:
        if logit_b is not None:
            raise MappingError("LCMOE_ERR_UNSUPPORTED", "logit bias with sigmoid")
    else:
        if sel_b is not None:
            raise MappingError("LCMOE_ERR_UNSUPPORTED", "selection bias with softmax")
        if n_group > 1:
            raise MappingError("LCMOE_ERR_UNSUPPORTED", "groups with softmax")
    desc.update(n_expert_used=K, route_kind=kind,
                n_group=n_group if kind == 2 else 1, topk_group=topk_group if kind == 2 else 1,
                routed_scale=float(np.float32(scale)), has_bias=int(bt is not None))
    if bt is not None:
        out["bias"] = g.floats(bt["name"])
    return desc, out
