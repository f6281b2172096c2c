"""GGUF ingest on the CPU: the product reader (lcmoe_gguf_*, through the C
ABI) against the oracle restatement of the reference reader
(oracle/lcgguf.py, rust/src/model/gguf.rs) and the reference's known answers,
on files written by tests/gguf_writer.py.  Nothing here touches a GPU."""
import ctypes as C
import os
import random

import numpy as np
import pytest

import gguf_writer as W
import lcgguf as G
import leafcutterllm_amd as L
from leafcutterllm_amd import _lib
from leafcutterllm_amd.configs import small_config, synth_layer, tensor_size

Q4, Q6, Q8 = L.TYPE_Q4_K, L.TYPE_Q6_K, L.TYPE_Q8_0
STATUS = {v: k for k, v in _lib.STATUS.items()}


def open_status(path):
    h = C.c_void_p()
    st = L.lib().lcmoe_gguf_open(os.fsencode(path), C.byref(h))
    if st == 0:
        L.lib().lcmoe_gguf_close(h)
    return _lib.STATUS[st]


def layer_status(path, layer=0, max_tokens=64):
    with L.GgufFile(path) as f:
        d, w = L.Desc(), L.Weights()
        return _lib.STATUS[L.lib().lcmoe_gguf_moe_layer(f.handle, layer, max_tokens, C.byref(d),
                                                        C.byref(w))]


def read_ptr(p, n, dtype=np.uint8):
    return np.frombuffer((C.c_uint8 * n).from_address(p), np.uint8).view(dtype).copy()


# ------------------------------------------------ reference known answers --

def test_tensor_size_reference_vectors(tmp_path):
    """calculate_tensor_size's own test, rust/src/model/gguf.rs:338-346."""
    cases = [(12, 144), (13, 176), (14, 210), (15, 292), (2, 144), (8, 272)]
    for typ, want in cases:
        assert G.tensor_size([256], typ) == want
    p = tmp_path / "sizes.gguf"
    W.write(p, [], [(f"t{typ}", [256], typ, bytes(want)) for typ, want in cases])
    with L.GgufFile(p) as f:
        for typ, want in cases:
            assert f.get_tensor_info(f"t{typ}") == {"type": typ, "dims": [256]}
            assert f.get_tensor_raw(f"t{typ}").size == want


# A Qwen2.5-3B file's first tensors (rust/TEST_REPORT.md:158-167): sizes and
# data-relative offsets, contiguous with 32-byte alignment.
REPORT = [("token_embd.weight", [2048, 151936], 14, 0, 255_252_480),
          ("blk.0.attn_norm.weight", [2048], 0, 255_252_480, 8_192),
          ("blk.0.ffn_down.weight", [11008, 2048], 14, 255_260_672, 18_493_440),
          ("blk.0.ffn_gate.weight", [2048, 11008], 12, 273_754_112, 12_681_216)]


def test_real_file_sizes_and_offsets(tmp_path):
    for (_, dims, typ, off, size), nxt in zip(REPORT, REPORT[1:] + [None]):
        assert G.tensor_size(dims, typ) == size
        assert off % 32 == 0
        if nxt is not None:
            assert nxt[3] == off + size  # the report's "verified contiguous"
    head = W.gguf_header([("general.architecture", W.STRING, "qwen2")],
                         [(n, dims, typ, off) for n, dims, typ, off, _ in REPORT])
    end = len(head) + REPORT[-1][3] + REPORT[-1][4]
    p = tmp_path / "report.gguf"
    with open(p, "wb") as fh:  # sparse: only the header is written
        fh.write(head)
        fh.truncate(end)
    with L.GgufFile(p) as f:
        base = None
        for name, dims, typ, off, size in REPORT:
            n, t = C.c_uint64(), C.c_void_p()
            _lib.check(L.lib().lcmoe_gguf_tensor(f.handle, name.encode(), None, None, None,
                                                 C.byref(t), C.byref(n)), "tensor")
            assert n.value == size
            base = t.value - off if base is None else base
            assert t.value - base == off
        assert f.block_count() == 1 and not f.is_moe_layer(0)
    with open(p, "r+b") as fh:
        fh.truncate(end - 1)
    assert open_status(p) == "LCMOE_ERR_CORRUPT"


# ------------------------------------------------ MoE layer round trips ----

ROUND_TRIP = {
    # name: (config, arch, extra metadata, writer options, shared (S, 2D/3D))
    "mixtral-llama": (small_config("q4k", 256, 512, 8, 2, L.ROUTE_SOFTMAX_RENORM, Q4, Q4),
                      "llama", [], {}),
    "mixtral-per-expert": (small_config("q4k", 256, 512, 8, 2, L.ROUTE_SOFTMAX_RENORM, Q4, Q4),
                           "llama", [], {"per_expert": True}),
    "q8-norm-key": (small_config("q8", 256, 384, 8, 2, L.ROUTE_SOFTMAX_RENORM, Q8, Q8),
                    "custommoe", [("custommoe.expert_weights_norm", W.BOOL, True)], {}),
    "qwen2moe-shared3d-logit-bias": (
        small_config("straddle", 256, 352, 12, 3, L.ROUTE_SOFTMAX, Q4, Q4, n_shared=2,
                     d_ff_shared=352, bias="plus2_first8"),
        "qwen2moe", [], {"bias_name": "ffn_gate_inp.bias"}),
    "deepseek-sigmoid-group": (
        small_config("sig", 512, 256, 32, 4, L.ROUTE_SIGMOID_GROUP, Q4, Q6, n_shared=1,
                     d_ff_shared=256, n_group=4, topk_group=2, routed_scale=2.5,
                     bias="normal0.1"),
        "deepseek2", [("deepseek2.expert_gating_func", W.U32, 2),
                      ("deepseek2.expert_weights_norm", W.BOOL, True),
                      ("deepseek2.expert_weights_scale", W.F32, 2.5),
                      ("deepseek2.expert_group_count", W.U32, 4),
                      ("deepseek2.expert_group_used_count", W.U32, 2)],
        {"bias_name": "exp_probs_b.bias"}),
    "olmoe-e60": (small_config("e60", 256, 256, 60, 4, L.ROUTE_SOFTMAX, Q4, Q4), "olmoe", [], {}),
    "f32-f16-router": (small_config("f32", 128, 256, 4, 2, L.ROUTE_SOFTMAX_RENORM, L.TYPE_F32,
                                    L.TYPE_F32), "llama", [], {"router_type": W.T_F16}),
    "bf16-router-gating3": (small_config("q4k", 256, 256, 8, 2, L.ROUTE_SOFTMAX_RENORM, Q4, Q6),
                            "custommoe", [("custommoe.expert_gating_func", W.I32, 3)],
                            {"router_type": W.T_BF16}),
}


def make_layer_file(path, cfg, arch, extra, opts, layer=0, seed=3, extra_layers=()):
    lay = synth_layer(cfg, seed)
    rt = opts.get("router_type", W.T_F32)
    if rt == W.T_F16:
        lay["router"] = lay["router"].astype(np.float16).astype(np.float32)
    elif rt == W.T_BF16:
        lay["router"] = (lay["router"].view(np.uint32) & 0xFFFF0000).view(np.float32)
    meta = [("general.architecture", W.STRING, arch),
            (f"{arch}.block_count", W.U32, max((layer,) + tuple(extra_layers)) + 1),
            (f"{arch}.expert_count", W.U32, cfg.n_expert),
            (f"{arch}.expert_used_count", W.U32, cfg.n_expert_used),
            (f"{arch}.embedding_length", W.U32, cfg.d_model),
            (f"{arch}.expert_feed_forward_length", W.U32, cfg.d_ff)] + list(extra)
    shared = None
    if cfg.n_shared:
        qs = (cfg.qtype_gate, cfg.qtype_gate, cfg.qtype_down)
        shared = (cfg.n_shared, cfg.d_ff_shared, qs)
    types = (cfg.qtype_gate, cfg.qtype_gate, cfg.qtype_down)
    tensors = [("token_embd.weight", [cfg.d_model, 4], W.T_F32, W.f32(np.ones((4, cfg.d_model))))]
    for extra_layer in extra_layers:  # dense layers around the MoE one
        tensors.append((f"blk.{extra_layer}.ffn_gate.weight", [cfg.d_model, 32], W.T_F32,
                        W.f32(np.zeros((32, cfg.d_model)))))
    tensors += W.moe_tensors(layer, lay, cfg.d_model, cfg.d_ff, cfg.n_expert, types,
                             per_expert=opts.get("per_expert", False), shared=shared,
                             bias_name=opts.get("bias_name"), router_type=rt)
    W.write(path, meta, tensors)
    return lay


def product_layer(f, layer, cfg, max_tokens=64):
    d, w = f.moe_layer(layer, max_tokens)
    E, dm, F = d.n_expert, d.d_model, d.d_ff
    out = {"router": read_ptr(w.router, 4 * dm * E, np.float32).reshape(dm, E)}
    out["bias"] = read_ptr(w.bias, 4 * E, np.float32) if w.bias else None
    out["gate"] = read_ptr(w.gate, E * tensor_size(d.type_gate, F * dm))
    out["up"] = read_ptr(w.up, E * tensor_size(d.type_up, F * dm))
    out["down"] = read_ptr(w.down, E * tensor_size(d.type_down, F * dm))
    if d.n_shared:
        S, Fs = d.n_shared, d.d_ff_shared
        out["gate_sh"] = read_ptr(w.gate_sh, S * tensor_size(d.type_gate_sh, Fs * dm))
        out["up_sh"] = read_ptr(w.up_sh, S * tensor_size(d.type_up_sh, Fs * dm))
        out["down_sh"] = read_ptr(w.down_sh, S * tensor_size(d.type_down_sh, Fs * dm))
    else:
        assert not (w.gate_sh or w.up_sh or w.down_sh)
    return d, out


@pytest.mark.parametrize("name", list(ROUND_TRIP))
def test_moe_layer_round_trip(tmp_path, name):
    cfg, arch, extra, opts = ROUND_TRIP[name]
    p = tmp_path / f"{name}.gguf"
    lay = make_layer_file(p, cfg, arch, extra, opts)
    want = cfg.desc(64).as_dict()
    if cfg.route_kind != L.ROUTE_SIGMOID_GROUP:
        want["n_group"] = want["topk_group"] = 1
    with L.GgufFile(p) as f:
        assert f.block_count() == 1 and f.is_moe_layer(0) and not f.is_moe_layer(1)
        d, got = product_layer(f, 0, cfg)
        assert d.as_dict() == want
        for k in ("router", "gate", "up", "down", "gate_sh", "up_sh", "down_sh", "bias"):
            if lay.get(k) is None:
                assert got.get(k) is None, k
            else:
                np.testing.assert_array_equal(got[k], np.asarray(lay[k]).reshape(got[k].shape),
                                              err_msg=k)
    # the oracle restatement maps the same file to the same layer
    od, ol = G.moe_layer(G.GgufRef(p.read_bytes()), 0)
    for k, v in od.items():
        assert want[k] == v, k
    for k, v in ol.items():
        np.testing.assert_array_equal(v, np.asarray(got[k]).reshape(v.shape), err_msg=k)


def test_layer_buffers_survive_other_layers(tmp_path):
    """Two MoE layers in one file (with dense layers between); each call
    keeps its own copies; a repeated call for a layer gives equal contents."""
    cfg = small_config("q4k", 256, 256, 8, 2, L.ROUTE_SOFTMAX_RENORM, Q4, Q4)
    lay0 = synth_layer(cfg, 1)
    lay2 = synth_layer(cfg, 2)
    types = (Q4, Q4, Q4)
    tensors = (W.moe_tensors(0, lay0, 256, 256, 8, types, per_expert=True)
               + [("blk.1.ffn_gate.weight", [256, 32], W.T_F32, W.f32(np.zeros((32, 256))))]
               + W.moe_tensors(2, lay2, 256, 256, 8, types))
    p = tmp_path / "two.gguf"
    W.write(p, [("general.architecture", W.STRING, "llama"),
                ("llama.expert_used_count", W.U32, 2)], tensors)
    with L.GgufFile(p) as f:
        assert f.block_count() == 3  # no block_count key: from the blk.N names
        assert [f.is_moe_layer(i) for i in range(4)] == [True, False, True, False]
        _, a = product_layer(f, 0, cfg)
        d0, w0 = f.moe_layer(0, 8)
        _, b = product_layer(f, 2, cfg)
        for k in ("router", "gate", "up", "down"):
            np.testing.assert_array_equal(a[k], np.asarray(lay0[k]).reshape(a[k].shape))
            np.testing.assert_array_equal(b[k], np.asarray(lay2[k]).reshape(b[k].shape))
        # layer 0's newest copies stay valid after layer 2 was mapped
        np.testing.assert_array_equal(read_ptr(w0.gate, a["gate"].size), a["gate"])
        assert d0.max_tokens == 8
        assert layer_status(p, 1) == "LCMOE_ERR_NOT_FOUND"  # dense layer


# ------------------------------------------------ metadata and layout ------

def test_metadata_int_matches_reference_rules(tmp_path):
    meta = [("u8", W.U8, 200), ("i8", W.I8, -7), ("u16", W.U16, 65000), ("i16", W.I16, -300),
            ("u32", W.U32, 4_000_000_000), ("i32", W.I32, -5), ("u64", W.U64, 2**64 - 3),
            ("i64", W.I64, -2**62), ("f32", W.F32, -5.75), ("f64", W.F64, 1e30),
            ("f64nan", W.F64, float("nan")), ("f32inf", W.F32, float("-inf")),
            ("bool", W.BOOL, True), ("str", W.STRING, "mixtral"),
            ("arr1u32", W.ARRAY, (W.U32, [77])), ("arr1i64", W.ARRAY, (W.I64, [-9])),
            ("arr1u8", W.ARRAY, (W.U8, [5])), ("arr2", W.ARRAY, (W.U32, [1, 2])),
            ("arrstr", W.ARRAY, (W.STRING, ["a", "bc", ""])),
            ("nested", W.ARRAY, (W.ARRAY, [(W.U32, [1]), (W.STRING, ["x"])])),
            ("arr0", W.ARRAY, (W.F32, [])),
            ("dup", W.U32, 1), ("dup", W.U32, 2)]
    p = tmp_path / "meta.gguf"
    W.write(p, meta, [("t", [4], W.T_F32, W.f32([1, 2, 3, 4]))])
    ref = G.GgufRef(p.read_bytes())
    with L.GgufFile(p) as f:
        for key in sorted({k for k, _, _ in meta}):
            assert f.get_metadata_int(key) == ref.meta_int(key), key
        assert f.get_metadata_int("absent") is None
        assert f.get_metadata_str("str") == "mixtral" and f.get_metadata_str("u8") is None
        assert f.get_metadata_int("dup") == 2  # last value wins, as the reference's map
        np.testing.assert_array_equal(f.get_tensor_raw("t").view("<f4"), [1, 2, 3, 4])
    assert ref.meta_int("u64") == -3 and ref.meta_int("f32") == -5
    assert ref.meta_int("f64nan") == 0 and ref.meta_int("f32inf") == -2**63
    assert ref.meta_int("bool") is None and ref.meta_int("arr1u8") is None


@pytest.mark.parametrize("align_kv,layout", [(None, 32), ((W.U32, 64), 64), ((W.U64, 256), 256),
                                             ((W.I32, 64), 32), ((W.U32, 1), 1)])
def test_alignment(tmp_path, align_kv, layout):
    rng = np.random.default_rng(5)
    payloads = [rng.integers(0, 256, n, dtype=np.uint8).tobytes() for n in (7 * 4, 33 * 4, 4)]
    meta = [("pad", W.STRING, "x" * 13)]
    if align_kv is not None:
        meta.append(("general.alignment", *align_kv))
    tensors = [(f"t{i}", [len(b) // 4], W.T_F32, b) for i, b in enumerate(payloads)]
    p = tmp_path / "align.gguf"
    W.write(p, meta, tensors, alignment=layout)
    ref = G.GgufRef(p.read_bytes())
    assert ref.data_offset % layout == 0
    with L.GgufFile(p) as f:
        for i, b in enumerate(payloads):
            assert f.get_tensor_raw(f"t{i}").tobytes() == b == ref.raw(f"t{i}").tobytes()


# ------------------------------------------------ errors -------------------

def base_file(tmp_path, name="base.gguf", **kw):
    cfg, arch, extra, opts = ROUND_TRIP["mixtral-llama"]
    p = tmp_path / name
    make_layer_file(p, cfg, arch, extra, opts, **kw)
    return p


def test_open_errors(tmp_path):
    good = base_file(tmp_path).read_bytes()
    assert open_status(tmp_path / "missing.gguf") == "LCMOE_ERR_IO"
    assert open_status(tmp_path) == "LCMOE_ERR_IO"  # a directory
    cases = {
        "magic": (b"GGUG" + good[4:], "LCMOE_ERR_CORRUPT", "magic"),
        "version2": (good[:4] + (2).to_bytes(4, "little") + good[8:], "LCMOE_ERR_UNSUPPORTED",
                     "version"),
        "short": (good[:20], "LCMOE_ERR_CORRUPT", "truncated"),
    }
    for name, (data, status, kind) in cases.items():
        p = tmp_path / f"{name}.gguf"
        p.write_bytes(data)
        assert open_status(p) == status, name
        with pytest.raises(G.GgufError) as e:
            G.GgufRef(data)
        assert e.value.kind == kind
    # unknown metadata value type: the reference's InvalidTensorType
    p = tmp_path / "kvtype.gguf"
    data = W.gguf_bytes([("general.architecture", W.STRING, "llama"), ("k", W.U32, 1)], [])
    key_at = data.index(b"\x01\x00\x00\x00\x00\x00\x00\x00k") + 9  # the type after key "k"
    p.write_bytes(data[:key_at] + (13).to_bytes(4, "little") + data[key_at + 4:])
    assert open_status(p) == "LCMOE_ERR_UNSUPPORTED"
    with pytest.raises(G.GgufError, match="value_type"):
        G.GgufRef(p.read_bytes())
    # alignment 0, five dims
    p = tmp_path / "align0.gguf"
    W.write(p, [("general.alignment", W.U32, 0)], [])
    assert open_status(p) == "LCMOE_ERR_CORRUPT"
    p = tmp_path / "dims5.gguf"
    W.write(p, [], [("t", [1, 1, 1, 1, 2], W.T_F32, bytes(8))])
    assert open_status(p) == "LCMOE_ERR_CORRUPT"


@pytest.mark.parametrize("dims", [[0, 4], [4, 0, 2], [0], [3, 5, 0, 7]])
def test_zero_dimension_tensor(tmp_path, dims):
    """A zero dimension makes an empty tensor (count 0, 0 bytes, as
    calculate_tensor_size gives, gguf.rs:307-313): the file opens and the
    tensor reads back with its dims and no data."""
    p = tmp_path / "zero.gguf"
    W.write(p, [], [("z", dims, W.T_F32, b""), ("t", [2], W.T_F32, W.f32([1.0, 2.0]))])
    assert open_status(p) == "LCMOE_OK"
    ref = G.GgufRef(p.read_bytes())
    assert len(ref.raw("z")) == 0
    with L.GgufFile(p) as f:
        assert f.get_tensor_info("z")["dims"] == dims
        assert np.array_equal(np.frombuffer(f.get_tensor_raw("t"), np.float32), [1.0, 2.0])


def test_truncation_sweep(tmp_path):
    """Every prefix of a small file: the product reader returns an error
    (never faults) exactly when the reference would fail to read the file
    or one of its tensors."""
    cfg = small_config("f32", 128, 256, 4, 2, L.ROUTE_SOFTMAX_RENORM, L.TYPE_F32, L.TYPE_F32)
    p = tmp_path / "full.gguf"
    make_layer_file(p, cfg, "llama", [], {})
    data = p.read_bytes()
    q = tmp_path / "cut.gguf"
    cuts = sorted(set(list(range(0, 700)) + list(range(len(data) - 300, len(data) + 1))
                      + random.Random(1).sample(range(len(data)), 200)))
    for n in cuts:
        q.write_bytes(data[:n])
        try:
            ref = G.GgufRef(data[:n])
            for t in ref.tensors:
                ref.raw(t["name"])
            ref_ok = True
        except G.GgufError:
            ref_ok = False
        st = open_status(q)
        assert (st == "LCMOE_OK") == ref_ok, (n, st)


def test_corruption_fuzz(tmp_path):
    """Random byte changes in the header: the product never faults, fails
    whenever the reference fails, and when both read the file they see the
    same tensors."""
    p = base_file(tmp_path)
    data = p.read_bytes()
    ref0 = G.GgufRef(data)
    head = ref0.data_offset
    rng = random.Random(7)
    q = tmp_path / "fuzz.gguf"
    for it in range(400):
        b = bytearray(data)
        for _ in range(rng.choice((1, 1, 2, 4))):
            b[rng.randrange(head)] = rng.randrange(256)
        q.write_bytes(bytes(b))
        try:
            ref = G.GgufRef(bytes(b))
            for t in ref.tensors:
                if t["type"] in G._GEOM:
                    ref.raw(t["name"])
        except (G.GgufError, ZeroDivisionError, MemoryError, OverflowError):
            ref = None
        h = C.c_void_p()
        st = L.lib().lcmoe_gguf_open(os.fsencode(q), C.byref(h))
        if ref is None:
            assert st != 0, it
            continue
        if st != 0:
            continue  # the product also rejects some files the reference reads
        try:
            for t in ref.tensors:
                if t["type"] not in G._GEOM or len(t["dims"]) > 4:
                    continue
                typ, nd, n = C.c_int32(), C.c_int32(), C.c_uint64()
                dims = (C.c_int64 * 4)()
                s2 = L.lib().lcmoe_gguf_tensor(h, t["name"].encode("utf-8", "surrogateescape"),
                                               C.byref(typ), C.byref(nd), dims, None, C.byref(n))
                if s2 != 0 or "�" in t["name"]:
                    continue  # names the oracle decoded lossily
                first = ref.info(t["name"])
                assert (typ.value, nd.value) == (first["type"], len(first["dims"])), it
                assert n.value == G.tensor_size(first["dims"], first["type"]), it
            # the layer mapping never faults either
            d, w = L.Desc(), L.Weights()
            L.lib().lcmoe_gguf_moe_layer(h, 0, 16, C.byref(d), C.byref(w))
        finally:
            L.lib().lcmoe_gguf_close(h)


def test_layer_errors(tmp_path):
    cfg, arch, extra, opts = ROUND_TRIP["mixtral-llama"]
    lay = synth_layer(cfg, 3)
    types = (Q4, Q4, Q4)

    def status(meta, tensors, arch_name="llama"):
        p = tmp_path / "e.gguf"
        W.write(p, [("general.architecture", W.STRING, arch_name)] + meta, tensors)
        return layer_status(p)

    K = [("llama.expert_used_count", W.U32, 2)]
    t = W.moe_tensors(0, lay, 256, 512, 8, types)
    assert status(K, t) == "LCMOE_OK"
    assert status([], t) == "LCMOE_ERR_NOT_FOUND"                          # no K
    assert status(K + [("llama.expert_count", W.U32, 9)], t) == "LCMOE_ERR_CORRUPT"
    assert status(K + [("llama.embedding_length", W.U32, 512)], t) == "LCMOE_ERR_CORRUPT"
    assert status(K + [("llama.expert_gating_func", W.U32, 7)], t) == "LCMOE_ERR_UNSUPPORTED"
    assert status(K + [("llama.expert_used_count", W.U32, 9)], t) == "LCMOE_ERR_INVALID_ARG"
    assert status([("other.expert_used_count", W.U32, 2)], t, "other") == "LCMOE_ERR_NOT_FOUND"
    assert status(K, t[1:]) == "LCMOE_ERR_NOT_FOUND"                       # no router
    assert status(K, [x for x in t if "ffn_up" not in x[0]]) == "LCMOE_ERR_NOT_FOUND"
    assert status(K, [t[0]]) == "LCMOE_ERR_NOT_FOUND"                     # no experts
    bad = [(n, dims[:2] + [4] if "exps" in n else dims, ty, b[: len(b) // 2] if "exps" in n else b)
           for n, dims, ty, b in t]
    assert status(K, bad) == "LCMOE_ERR_CORRUPT"                           # 4 experts, E = 8
    q_router = [(t[0][0], [256, 8], Q8, bytes(tensor_size(Q8, 256 * 8)))] + t[1:]
    assert status(K, q_router) == "LCMOE_ERR_UNSUPPORTED"
    f16_exp = [(n, dims, W.T_F16 if "exps" in n else ty,
                bytes(2 * int(np.prod(dims))) if "exps" in n else b) for n, dims, ty, b in t]
    assert status(K, f16_exp) == "LCMOE_ERR_UNSUPPORTED"
    gated = t + [("blk.0.ffn_gate_inp_shexp.weight", [256], W.T_F32, W.f32(np.zeros(256)))]
    assert status(K, gated) == "LCMOE_ERR_UNSUPPORTED"
    sel_b = t + [("blk.0.exp_probs_b.bias", [8], W.T_F32, W.f32(np.zeros(8)))]
    assert status(K, sel_b) == "LCMOE_ERR_UNSUPPORTED"                     # softmax gating
    both = sel_b + [("blk.0.ffn_gate_inp.bias", [8], W.T_F32, W.f32(np.zeros(8)))]
    sig = K + [("llama.expert_gating_func", W.U32, 2)]
    assert status(sig, both) == "LCMOE_ERR_UNSUPPORTED"
    assert status(sig, sel_b) == "LCMOE_OK"
    assert status(sig + [("llama.expert_weights_norm", W.BOOL, False)], sel_b) == \
        "LCMOE_ERR_UNSUPPORTED"
    logit_b = t + [("blk.0.ffn_gate_inp.bias", [8], W.T_F32, W.f32(np.zeros(8)))]
    assert status(sig, logit_b) == "LCMOE_ERR_UNSUPPORTED"
    assert status(K, logit_b) == "LCMOE_OK"
    assert status(K + [("llama.expert_group_count", W.U32, 2)], t) == "LCMOE_ERR_UNSUPPORTED"
    wrong_b = t + [("blk.0.ffn_gate_inp.bias", [7], W.T_F32, W.f32(np.zeros(7)))]
    assert status(K, wrong_b) == "LCMOE_ERR_CORRUPT"
    # oracle agrees on every status above that it models
    for meta, tensors, want in ((K, gated, "LCMOE_ERR_UNSUPPORTED"),
                                (K, sel_b, "LCMOE_ERR_UNSUPPORTED"),
                                ([], t, "LCMOE_ERR_NOT_FOUND")):
        data = W.gguf_bytes([("general.architecture", W.STRING, "llama")] + meta, tensors)
        with pytest.raises(G.MappingError) as e:
            G.moe_layer(G.GgufRef(data), 0)
        assert e.value.status == want
    with L.GgufFile(tmp_path / "e.gguf") as f:
        with pytest.raises(L.LcmoeError):
            f.moe_layer(-1, 16)
