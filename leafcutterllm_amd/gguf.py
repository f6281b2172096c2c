"""GGUF ingest over the C ABI (lcmoe_gguf_*, include/lcmoe.h).

`GgufFile` mirrors the reference reader's surface, GGUFile
(rust/src/model/gguf.rs:33-157): open, get_metadata_int, get_tensor_info +
get_tensor_raw; `moe_layer` is the MoE counterpart of GGUFModel::load_layer
(rust/src/model/loader.rs:145-168).  Parsing and mapping run in the native
library; nothing here reads the file itself.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from ._lib import Desc, Weights, check, lib


class GgufFile:
    """A memory-mapped GGUF v3 file (the library's lcmoe_gguf handle)."""

    def __init__(self, path):
        h = C.c_void_p()
        check(lib().lcmoe_gguf_open(os.fsencode(path), C.byref(h)), "lcmoe_gguf_open")
        self._h = h

    @property
    def handle(self) -> int:
        return self._h.value

    def get_metadata_int(self, key: str):
        """Integer metadata as GGUFile::get_metadata_int; None if absent or
        not an integer."""
        v = C.c_int64()
        st = lib().lcmoe_gguf_meta_int(self._h, key.encode(), C.byref(v))
        if st in (1, 7):  # INVALID_ARG (another type), NOT_FOUND
            return None
        check(st, "lcmoe_gguf_meta_int")
        return v.value

    def get_metadata_str(self, key: str):
        s = lib().lcmoe_gguf_meta_str(self._h, key.encode())
        return None if s is None else s.decode("utf-8", "replace")

    def get_tensor_info(self, name: str):
        """{'type', 'dims'} or None."""
        t, nd = C.c_int32(), C.c_int32()
        dims = (C.c_int64 * 4)()
        st = lib().lcmoe_gguf_tensor(self._h, name.encode(), C.byref(t), C.byref(nd), dims,
                                     None, None)
        if st == 7:
            return None
        check(st, "lcmoe_gguf_tensor")
        return {"type": t.value, "dims": [dims[i] for i in range(nd.value)]}

    def get_tensor_raw(self, name: str):
        """The tensor's bytes as a read-only uint8 view of the mapping (valid
        while this file is open), or None."""
        p, n = C.c_void_p(), C.c_uint64()
        st = lib().lcmoe_gguf_tensor(self._h, name.encode(), None, None, None, C.byref(p),
                                     C.byref(n))
        if st == 7:
            return None
        check(st, "lcmoe_gguf_tensor")
        if not p.value:
            return None
        buf = (C.c_uint8 * n.value).from_address(p.value)
        a = np.frombuffer(buf, np.uint8)
        a.flags.writeable = False
        return a

    def block_count(self) -> int:
        return lib().lcmoe_gguf_block_count(self._h)

    def is_moe_layer(self, layer: int) -> bool:
        return bool(lib().lcmoe_gguf_is_moe_layer(self._h, layer))

    def moe_layer(self, layer: int, max_tokens: int):
        """(Desc, Weights) of MoE layer `layer`; the Weights pointers stay
        valid until close() or the next moe_layer call for that layer."""
        d, w = Desc(), Weights()
        check(lib().lcmoe_gguf_moe_layer(self._h, layer, max_tokens, C.byref(d), C.byref(w)),
              "lcmoe_gguf_moe_layer")
        return d, w

    def close(self) -> None:
        if getattr(self, "_h", None) is not None and self._h.value:
            lib().lcmoe_gguf_close(self._h)
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
