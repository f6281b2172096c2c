"""Benchmark: Mixtral-8x7B-shaped Q4_K MoE layer on one MI355X.

A step is one MoE-layer forward (router, dispatch, expert products, combine)
over one batch of T synthetic tokens whose activations already sit in HBM.
The headline line is T=64; the JSON also carries T=1 and T=8.  Layer
replicas (separate device copies of the same bytes) are cycled from step to
step so that re-reads cannot be served from the 256 MB Infinity Cache.

Prints ONE JSON line (rank 0, N=1).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense f16 matrix peak
FP32_PEAK_TFLOPS = 157.3  # MI355X fp32 (vector) peak
MALL_BYTES = 256 << 20


def algorithmic_bytes(cfg, counts, T):
    """Per-call bytes: quant blocks of every touched and every shared expert
    (gate, up, down), the f32 router, x in and y out (intermediates
    excluded); the routed gate/up launch's bytes (touched experts' gate and
    up, x, H); and the shared experts' gate/up bytes, which that launch also
    reads when they ride in it."""
    from leafcutterllm_amd.configs import tensor_size
    touched = int(sum(1 for c in counts if c > 0))
    gu = 2 * tensor_size(cfg.qtype_gate, cfg.d_ff * cfg.d_model)
    dn = tensor_size(cfg.qtype_down, cfg.d_model * cfg.d_ff)
    S, FS = cfg.n_shared, cfg.d_ff_shared
    gu_sh = S * 2 * tensor_size(cfg.qtype_gate, FS * cfg.d_model) if S else 0
    dn_sh = S * tensor_size(cfg.qtype_down, cfg.d_model * FS) if S else 0
    layer = (touched * (gu + dn) + gu_sh + dn_sh + 4 * cfg.d_model * cfg.n_expert
             + 8 * T * cfg.d_model)
    gateup = touched * gu + 4 * T * cfg.d_model + 4 * T * cfg.n_expert_used * cfg.d_ff
    shared_gateup = gu_sh + 4 * T * S * FS
    return layer, gateup, shared_gateup, touched


def cpu_baseline(cfg, layer, sweep, head_T, budget_s=5.0):
    """The oracle's restatement of the reference CPU path (rust/src/kernels/
    simd.rs f32 GEMM order, engine.rs:146-164 SwiGLU), timed on this host at
    every batch of the sweep, three ways:
      faithful   : experts dequantised to f32 once, then the reference's
                   rayon row split (simd.rs:298-311, MIN_ROWS_PER_TASK = 4:
                   an expert with <= 4 rows runs on one core);
      all_cores  : the same arithmetic split over column blocks on every
                   thread of the pool;
      as_shipped : the engine as it ships, re-dequantising and transposing
                   every touched expert on every forward (engine.rs:96,
                   loader.rs:145-168) before the row-split GEMMs.
    Each figure is the median of up to 5 forwards within about `budget_s`
    (one forward at least; as_shipped, the slowest, one forward)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import lcoracle as O

    import leafcutterllm_amd as L

    host = os.cpu_count() or 1
    pool = max(1, min(host, int(os.environ.get("OMP_NUM_THREADS", host))))
    od = O.Desc()
    for name, _ in od._fields_:
        setattr(od, name, getattr(cfg.desc(max(sweep)), name))
    t0 = time.perf_counter()
    res = O.Resident(od, layer, pool)
    t_load = time.perf_counter() - t0

    def med(fn, T, budget=budget_s):
        times = []
        while len(times) < 5 and (not times or sum(times) < budget):
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
        times.sort()
        m = times[len(times) // 2]
        return {"tokens_per_s": round(T / m, 3), "ms": round(m * 1e3, 2), "runs": len(times)}

    per = {}
    for T in sweep:
        x = L.synth_x(cfg, T, seed=0, index=T)
        per[str(T)] = {
            "faithful": med(lambda: res.forward(x, 0), T),
            "all_cores": med(lambda: res.forward(x, pool), T),
            "as_shipped": med(lambda: O.moe_forward(od, layer, x, threads=0), T, 0.0),
        }
    res.close()
    head = per[str(head_T)]["faithful"]
    return {
        "value": head["tokens_per_s"], "unit": "tokens/s", "cores": pool, "host_cores": host,
        "kind": "port",
        "sample": (f"T={head_T}: median of {head['runs']} forward(s) of the same layer, experts "
                   f"dequantised to f32 once ({t_load:.1f} s), reference f32 GEMM order with the "
                   f"reference's rayon row split (>= 4 rows per task) on a pool of {pool} threads "
                   f"of the host's {host}"),
        "per_batch": per,
    }


def layer_flops(cfg, T):
    """Algorithmic flops of one layer call: 2 per multiply-add over gate, up
    and down of every routed assignment and every shared expert token."""
    return (6 * cfg.d_model * cfg.d_ff * T * cfg.n_expert_used
            + 6 * cfg.d_model * cfg.d_ff_shared * T * cfg.n_shared)


# sources of the matrix-core expert kernels: a traffic figure measured on
# other sources is stale
TRAFFIC_SOURCES = ("leafcutterllm_amd/csrc/kern_mfma.hip", "leafcutterllm_amd/csrc/device_common.h",
                   "leafcutterllm_amd/csrc/chains.h", "leafcutterllm_amd/csrc/lcmoe_api.hip")


def _code_tokens(text: str) -> str:
    """The source without comments and whitespace: edits to comments leave
    the stamp unchanged, any change to the code changes it."""
    import re
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    text = re.sub(r"//[^\n]*", " ", text)
    return "".join(text.split())


def kernel_source_stamp() -> str:
    import hashlib
    h = hashlib.sha256()
    for rel in TRAFFIC_SOURCES:
        with open(os.path.join(ROOT, rel), encoding="utf-8") as f:
            h.update(_code_tokens(f.read()).encode())
    return h.hexdigest()[:16]


def measured_traffic(config: int, tokens: int):
    """HBM bytes per gate/up launch from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE passes (profiles/traffic.json, calibrated by a plain copy), when
    they were taken on this workload and on the kernel sources of this tree
    (their stamp); None otherwise."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    if t.get("workload") != f"config {config}, T={tokens}":
        return None
    if t.get("source_stamp") != kernel_source_stamp():
        return None
    return int(t["bytes"])


def copy_probe(mib: int):
    """Three plain device-to-device copies of `mib` MiB: a known byte count to
    scale rocprofv3's FETCH_SIZE / WRITE_SIZE counters by."""
    from leafcutterllm_amd import hip
    n = mib << 20
    a, b = hip.DeviceBuffer(n), hip.DeviceBuffer(n)
    rt = hip.rt()
    rt.hipMemset(a.ptr, 1, n)
    for _ in range(3):
        rt.hipMemcpy(b.ptr, a.ptr, n, 3)  # hipMemcpyDeviceToDevice
    rt.hipDeviceSynchronize()
    print(json.dumps({"copy_probe_bytes": n, "copies": 3}), flush=True)


def shard_matmul_bench(args) -> None:
    """Times the shard-layout GEMM (Tensor::matmul's Q8_0 / Q4_0 arms) on
    resident device buffers: HIP events around `steps` launches."""
    import numpy as np

    import leafcutterllm_amd as L
    from leafcutterllm_amd import hip
    from leafcutterllm_amd._lib import check

    name, m, k, n = args.shard_matmul.split(",")
    m, k, n = int(m), int(k), int(n)
    qt = {"q8": L.TYPE_Q8_0, "q4": L.TYPE_Q4_0}[name]
    bb = k * (n // 32) * (34 if qt == L.TYPE_Q8_0 else 18)
    rng = np.random.default_rng(0)
    b = rng.integers(0, 256, bb, dtype=np.uint8)
    b.reshape(-1, 34 if qt == L.TYPE_Q8_0 else 18)[:, :2] = \
        np.full(1, 0.01, np.float16).view(np.uint8)  # finite scales
    a = rng.standard_normal((m, k)).astype(np.float32)
    # weight replicas cycled so that re-reads cannot come from the MALL
    R = max(2, -(-2 * MALL_BYTES // bb) + 1)
    dbs = [hip.DeviceBuffer(bb).upload(b) for _ in range(R)]
    da, dc = hip.DeviceBuffer(a.nbytes).upload(a), hip.DeviceBuffer(4 * m * n)
    S = args.shard_split
    ws = hip.DeviceBuffer(4 * S * m * n) if S > 1 else None
    st = hip.Stream()

    def launch(i):
        if S > 1:
            check(L.lib().lcmoe_shard_matmul_split_dev(qt, da.ptr, dbs[i % R].ptr, dc.ptr, m, k,
                                                        n, S, ws.ptr, st.ptr),
                  "lcmoe_shard_matmul_split_dev")
        else:
            check(L.lib().lcmoe_shard_matmul_dev(qt, da.ptr, dbs[i % R].ptr, dc.ptr, m, k, n,
                                                  st.ptr), "lcmoe_shard_matmul_dev")

    for i in range(args.warmup):
        launch(i)
    st.synchronize()
    e0, e1 = hip.Event(), hip.Event()
    e0.record(st)
    for i in range(args.steps):
        launch(i)
    e1.record(st)
    ms = e0.elapsed_ms(e1) / args.steps
    alg = bb + a.nbytes + 4 * m * n
    print(json.dumps({
        "metric": "shard-layout quantised GEMM time", "value": round(ms * 1e3, 3), "unit": "us",
        "higher_is_better": False, "steps": args.steps, "warmup": args.warmup,
        "config": {"workload": f"lcmoe_shard_matmul{'_split' if S > 1 else ''}_dev {name} "
                               f"m={m} k={k} n={n}" + (f" k_split={S}" if S > 1 else ""),
                   "replicas": R},
        "roofline": {"bound": "hbm", "achieved": round(alg / (ms * 1e-3) / 1e9, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(alg / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                     "algorithmic_bytes": alg},
    }))


def matmul_f32_bench(args) -> None:
    """Times Backend::matmul's HIP replacement (lcmoe_matmul_f32_dev, the x86
    CpuBackend's per-output order, bit for bit) on resident device buffers:
    HIP events around `steps` launches, B cycled through replicas past the
    MALL.  Each output is one k-long chain of dependent fused multiply-adds
    in k order, so besides HBM bytes and fp32 flops the bound is that chain:
    k steps of the dependent-FMA latency, measured at about 2.7 ns per step
    (a one-wave clock64 probe, 4096 steps in ~11 us)."""
    import numpy as np

    from leafcutterllm_amd import hip
    from leafcutterllm_amd._lib import check
    import leafcutterllm_amd as L

    m, k, n = (int(v) for v in args.matmul_f32.split(","))
    rng = np.random.default_rng(0)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    R = max(2, -(-2 * MALL_BYTES // b.nbytes) + 1)
    dbs = [hip.DeviceBuffer(b.nbytes).upload(b) for _ in range(R)]
    da, dc = hip.DeviceBuffer(a.nbytes).upload(a), hip.DeviceBuffer(4 * m * n)
    st = hip.Stream()

    def launch(i):
        check(L.lib().lcmoe_matmul_f32_dev(da.ptr, dbs[i % R].ptr, dc.ptr, m, k, n, st.ptr),
              "lcmoe_matmul_f32_dev")

    for i in range(args.warmup):
        launch(i)
    st.synchronize()
    e0, e1 = hip.Event(), hip.Event()
    e0.record(st)
    for i in range(args.steps):
        launch(i)
    e1.record(st)
    ms = e0.elapsed_ms(e1) / args.steps
    alg = a.nbytes + b.nbytes + 4 * m * n
    tflops = 2.0 * m * n * k / (ms * 1e-3) / 1e12
    chain_us = k * 2.7e-3
    gbs = alg / (ms * 1e-3) / 1e9
    print(json.dumps({
        "metric": "Backend::matmul (f32, CPU-backend order) time", "value": round(ms * 1e3, 3),
        "unit": "us", "higher_is_better": False, "steps": args.steps, "warmup": args.warmup,
        "dtype": "f32 (fused multiply-add chains in k order, bit-identical to the x86 CpuBackend)",
        "config": {"workload": f"lcmoe_matmul_f32_dev m={m} k={k} n={n}", "replicas": R},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "algorithmic_bytes": alg},
        "fp32_TFLOPs": round(tflops, 3), "fp32_frac": round(tflops / FP32_PEAK_TFLOPS, 4),
        "chain_floor_us": round(chain_us, 2), "frac_of_chain_floor": round(chain_us / (ms * 1e3), 4),
    }))


def e2e_bench(args) -> None:
    """Config 5: the 24-layer synthetic MoE decoder end to end
    (lcmoe_model_generate): a 512-token random-id prompt per sequence, then
    256 greedy tokens, at B = 1 and B = 16.  Prefill runs one sequence per
    forward (the reference's one-call prompt, engine.rs:54); the 255 decode
    steps replay one captured HIP graph.  Times come from HIP events on the
    model's stream; the first generate of each batch size (8 tokens) is the
    warm-up that also captures its graph."""
    import numpy as np

    import leafcutterllm_amd as L
    from leafcutterllm_amd.configs import tensor_size

    mc = L.MODEL_CONFIGS[5]
    P, n_new = 512, 256
    batches = [int(b) for b in args.e2e_batches.split(",")]
    t0 = time.perf_counter()
    w = L.synth_model(mc, seed=0)
    t_synth = time.perf_counter() - t0
    rng = np.random.default_rng(0)
    per = {}
    with L.Model(mc.desc(max(batches), P, P + n_new), w) as m:
        del w
        if args.no_graph:
            m.set_decode_graph(False)
        for B in batches:
            prompts = rng.integers(0, mc.vocab, (B, P)).astype(np.int32)
            m.generate(prompts, 8)
            t0 = time.perf_counter()
            out, _ = m.generate(prompts, n_new)
            wall = time.perf_counter() - t0
            pre, dec = m.last_timing()
            per[str(B)] = {
                "prefill_ms": round(pre, 3), "decode_ms": round(dec, 3),
                "decode_tokens_per_s": round(B * (n_new - 1) / (dec * 1e-3), 2),
                "ms_per_decode_step": round(dec / (n_new - 1), 4),
                "e2e_tokens_per_s": round(B * n_new / ((pre + dec) * 1e-3), 2),
                "prefill_tokens_per_s": round(B * P / (pre * 1e-3), 1),
                "wall_s": round(wall, 3),
                "distinct_ids": int(len(np.unique(out))),
            }
    # B = 1 decode step: every weight byte a token touches (one token uses
    # exactly K routed + S shared experts per layer) plus the KV cache it
    # reads at the mean context
    lc = mc.layer
    d, qd = mc.d_model, mc.n_head * mc.head_dim
    attn = tensor_size(mc.attn_type, (qd + 2 * mc.n_kv_head * mc.head_dim) * d) \
        + tensor_size(mc.attn_type, d * qd)
    moe = (lc.n_expert_used * lc.expert_bytes() + lc.n_shared * lc.shared_bytes()
           + 4 * d * lc.n_expert)
    kv = 2 * 2 * mc.n_kv_head * mc.head_dim * (P + n_new / 2)
    step_bytes = mc.n_layer * (attn + moe + kv) + tensor_size(mc.attn_type, mc.vocab * d)
    head = per[str(max(batches))]
    b1 = per.get("1")
    out = {
        "metric": "end-to-end greedy decode tokens/s, config 5 (24-layer MoE decoder, Q4_K)",
        "value": head["decode_tokens_per_s"], "unit": "tokens/s", "n_gpus": 1,
        "steps": n_new - 1, "warmup": 1, "ms_per_step": head["ms_per_decode_step"],
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": ("f32 (Q4_K weights; MoE products exact int8 dot4 on 15-bit activation limbs "
                  "when T*K <= E, f16 hi+lo activations on MFMA above; f16 KV cache)"),
        "data": "synthetic (seeded N(0,0.02) weights quantised to Q4_K, random prompt ids)",
        "config": {"workload": f"config 5: {mc.note}, prompt {P}, {n_new} greedy tokens, "
                               f"B={max(batches)}", "entry": "lcmoe_model_generate",
                   "n_layer": mc.n_layer, "d_model": d, "n_head": mc.n_head,
                   "head_dim": mc.head_dim, "vocab": mc.vocab, "batches": batches},
        "per_batch": per,
        "synth_s": round(t_synth, 1),
    }
    if b1:
        gbs = step_bytes / (b1["ms_per_decode_step"] * 1e-3) / 1e9
        out["roofline"] = {"bound": "hbm", "kernel": "whole B=1 decode step (all launches)",
                           "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                           "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                           "algorithmic_bytes": int(step_bytes)}
    print(json.dumps(out), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", type=int, default=2)
    ap.add_argument("--tokens", type=int, default=64, help="headline batch")
    ap.add_argument("--sweep", default="1,8,64")
    ap.add_argument("--device-warmup", type=float, default=0.5, metavar="S",
                    help="seconds of untimed forwards at the headline batch before the sweep")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--norm-residual", action="store_true",
                    help="time lcmoe_forward_norm_residual_dev (post-attention RMSNorm, "
                         "the layer and the residual add) instead of lcmoe_forward_dev")
    ap.add_argument("--kernel-events", type=int, default=1,
                    help="time each kernel with HIP events in a second timed region")
    ap.add_argument("--read-probe", action="store_true",
                    help="only measure the HBM streaming-read rate over 64 MiB - 1 GiB slices")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only run device-to-device copies of this size (FETCH_SIZE calibration)")
    ap.add_argument("--shard-matmul", default="", metavar="TYPE,M,K,N",
                    help="only time lcmoe_shard_matmul_dev (TYPE q8 or q4) on one shape")
    ap.add_argument("--matmul-f32", default="", metavar="M,K,N",
                    help="only time lcmoe_matmul_f32_dev (Backend::matmul) on one shape")
    ap.add_argument("--shard-split", type=int, default=1, metavar="S",
                    help="with --shard-matmul: time lcmoe_shard_matmul_split_dev with S k-slices")
    ap.add_argument("--e2e-batches", default="1,16",
                    help="with --config 5: batch sizes of the end-to-end decode")
    ap.add_argument("--layer", action="store_true",
                    help="with --config 5: time the MoE layer alone instead of the whole decoder")
    ap.add_argument("--no-graph", action="store_true",
                    help="with --config 5: eager decode launches instead of the captured graph "
                         "(for profilers that cannot trace graph launches)")
    args = ap.parse_args()

    if args.read_probe:
        import leafcutterllm_amd as LP
        print(json.dumps({"stream_read_GBps": {str(m): round(LP.read_bandwidth(m, reps=16), 1)
                                               for m in (64, 128, 256, 512, 1024)},
                          "peak_GBps": HBM_PEAK_GBS}), flush=True)
        return
    if args.copy_probe:
        copy_probe(args.copy_probe)
        return
    if args.shard_matmul:
        shard_matmul_bench(args)
        return
    if args.matmul_f32:
        matmul_f32_bench(args)
        return

    if args.config == 5 and args.gpus == 1 and not args.layer:
        e2e_bench(args)
        return

    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only; --gpus {args.gpus} is not supported "
              "(the MoE layer would shard by expert across GPUs, see DESIGN.md)", file=sys.stderr)
        sys.exit(2)

    import numpy as np

    import leafcutterllm_amd as L
    from leafcutterllm_amd import hip

    cfg = L.CONFIGS[args.config]
    sweep = sorted({int(t) for t in args.sweep.split(",") if t} | {args.tokens})
    Tmax = max(sweep)
    t0 = time.perf_counter()
    layer = L.synth_layer(cfg, seed=0)
    t_synth = time.perf_counter() - t0

    # replicas: reuse distance of the smallest touched set >= 2x the MALL
    min_touched = min(cfg.n_expert, cfg.n_expert_used) * cfg.expert_bytes()
    R = max(2, math.ceil(2 * MALL_BYTES / min_touched) + 1)
    moes = [L.MoeFfn(cfg.desc(Tmax), layer) for _ in range(R)]
    if args.norm_residual:
        w_norm = 1.0 + 0.1 * L.configs.synth_normal(0, 77, 1.0, cfg.d_model)
        for m in moes:
            m.set_norm(w_norm, 1e-5)

    def step(r: int, T: int) -> None:
        if args.norm_residual:
            moes[r].forward_norm_residual_dev(xbufs[(r, T)].ptr, T, ybufs[r].ptr, stream.ptr)
        else:
            moes[r].forward_dev(xbufs[(r, T)].ptr, T, ybufs[r].ptr, stream.ptr)
    stream = hip.Stream()
    xbufs = {}
    ybufs = [hip.DeviceBuffer(4 * Tmax * cfg.d_model) for _ in range(R)]
    for T in sweep:
        for r in range(R):
            x = L.synth_x(cfg, T, seed=0, index=1000 * r + T)
            xbufs[(r, T)] = hip.DeviceBuffer(x.nbytes).upload(x)

    # Device warm-up: the headline batch runs untimed for `device_warmup`
    # seconds before the sweep, so that every batch size is timed at the
    # clocks a busy GPU holds.  From idle, the first tenths of a second of
    # forwards run slower (config 2: T=8 ~177-185 us against ~168 us warm,
    # T=64 ~203-220 against ~198 us; T=1 unchanged).
    t_w = time.perf_counter()
    n_w = 0
    while time.perf_counter() - t_w < args.device_warmup:
        for _ in range(16):
            step(n_w % R, args.tokens)
            n_w += 1
        stream.synchronize()

    per_batch = {}
    for T in sweep:
        # realised routing of every replica's input -> algorithmic bytes
        call_bytes, gu_bytes, touched = [], [], []
        sh_bytes = 0
        for r in range(R):
            step(r, T)
            stream.synchronize()
            counts = moes[r].dispatch()["counts"]
            b, g, sh_bytes, n = algorithmic_bytes(cfg, counts, T)
            call_bytes.append(b)
            gu_bytes.append(g)
            touched.append(n)
        for i in range(args.warmup):
            step(i % R, T)
        stream.synchronize()

        def timed_region(events: bool):
            """K steps bracketed by HIP events on the launch stream; with
            `events`, every launch is also bracketed (per-kernel times)."""
            for m in moes:
                m.set_timing(events)
                m.get_timing()  # reset
            ev0, ev1 = hip.Event(), hip.Event()
            stream.synchronize()
            ev0.record(stream)
            for i in range(args.steps):
                step(i % R, T)
            ev1.record(stream)
            stream.synchronize()
            kern = {}
            for m in moes:
                for name, (kms, n) in m.get_timing().items():
                    a, b = kern.get(name, (0.0, 0))
                    kern[name] = (a + kms, b + n)
                m.set_timing(False)
            return ev0.elapsed_ms(ev1) / args.steps, kern

        # the step time comes from a region without per-launch events (they
        # add host and queue overhead); a second region times each kernel
        ms, _ = timed_region(False)
        kern = timed_region(True)[1] if args.kernel_events else {}
        bytes_per_step = sum(call_bytes[i % R] for i in range(args.steps)) / args.steps
        gu_per_launch = sum(gu_bytes[i % R] for i in range(args.steps)) / args.steps
        # shared experts timed without a launch of their own ride in the
        # routed gate/up launch
        shared_in_routed = (cfg.n_shared > 0 and bool(kern)
                            and kern.get("gateup_shared", (0.0, 0))[1] == 0)
        if shared_in_routed:
            gu_per_launch += sh_bytes
        gu = kern.get("gateup", (0.0, 0))
        gu_ms = gu[0] / gu[1] if gu[1] else float("nan")
        per_batch[T] = {
            "tokens_per_s": T / (ms * 1e-3),
            "ms_per_step": ms,
            "layer_GBps": bytes_per_step / (ms * 1e-3) / 1e9,
            "layer_bytes": bytes_per_step,
            "touched_experts": sum(touched) / len(touched),
            "gateup_ms": gu_ms,
            "gateup_bytes": gu_per_launch,
            "gateup_GBps": gu_per_launch / (gu_ms * 1e-3) / 1e9 if gu_ms == gu_ms else float("nan"),
            "shared_in_routed_launch": shared_in_routed,
            "kernel_ms": {k: v[0] / max(1, v[1]) for k, v in kern.items()},
        }

    head = per_batch[args.tokens]
    T = args.tokens
    qname = {L.TYPE_Q8_0: "Q8_0", L.TYPE_Q4_K: "Q4_K", L.TYPE_Q6_K: "Q6_K", L.TYPE_F32: "F32"}
    gq = qname[cfg.qtype_gate]
    gu_flops = 4 * cfg.d_model * cfg.d_ff * T * cfg.n_expert_used
    if head["shared_in_routed_launch"]:
        gu_flops += 4 * cfg.d_model * cfg.d_ff_shared * T * cfg.n_shared
    gu_weight_bytes = (head["gateup_bytes"] - 4 * T * cfg.d_model
                       - 4 * T * cfg.n_expert_used * cfg.d_ff
                       - (4 * T * cfg.n_shared * cfg.d_ff_shared
                          if head["shared_in_routed_launch"] else 0))
    if gu_flops / (MFMA_F16_PEAK_TFLOPS * 1e12) > gu_weight_bytes / (HBM_PEAK_GBS * 1e9):
        # past the ridge point (prefill-sized batches): the gate/up products
        # are bound by the f16 dense MFMA peak, not by streaming the weights
        roof = {
            "bound": "mfma",
            "kernel": (f"routed{' + shared' if head['shared_in_routed_launch'] else ''} gate/up "
                       f"launch (k_mfma_gateup: {gq} dequant + gate/up + SwiGLU)"),
            "achieved": round(gu_flops / (head["gateup_ms"] * 1e-3) / 1e12, 2),
            "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(gu_flops / (head["gateup_ms"] * 1e-3) / 1e12 / MFMA_F16_PEAK_TFLOPS, 4),
            "traffic": None,
            "algorithmic_flops": gu_flops,
        }
        lf = layer_flops(cfg, T)
        head["layer_TFLOPs"] = lf / (head["ms_per_step"] * 1e-3) / 1e12
        head["layer_mfma_frac"] = head["layer_TFLOPs"] / MFMA_F16_PEAK_TFLOPS
    else:
        roof = {
            "bound": "hbm",
            "kernel": f"gate/up launch (fused {gq} dequant + gate/up products + SwiGLU)",
            "achieved": round(head["gateup_GBps"], 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(head["gateup_GBps"] / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(args.config, args.tokens),
            "traffic_unit": "bytes per launch (rocprofv3 FETCH_SIZE + WRITE_SIZE, copy-calibrated, "
                            "profiles/traffic.json; null when measured on other kernel sources)",
            "kernel_source_stamp": kernel_source_stamp(),
            "algorithmic_bytes": round(head["gateup_bytes"]),
        }
    qdesc = qname[cfg.qtype_gate] + ("" if cfg.qtype_down == cfg.qtype_gate
                                     else f" gate/up, {qname[cfg.qtype_down]} down")
    metric = ("MoE-layer tokens/s + % HBM roofline, Mixtral-shape Q4_K, batch 1-64"
              if args.config == 2 else
              f"MoE-layer tokens/s + % {roof['bound'].upper()} roofline, config {args.config} "
              f"({qdesc})")
    out = {
        "metric": metric,
        "value": round(head["tokens_per_s"], 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": (("f32 in/out; expert products exact int8 dot4 of the Q8_0 weights with "
                   "15-bit two-limb activations at every T; f32 accumulate")
                  if cfg.qtype_gate == L.TYPE_Q8_0 else
                  ("f32 in/out; expert products on exact weights (f16 sc*q, f32 scales) with "
                   "one f16 per activation (x and H) on MFMA when T >= 4 or T*K > E "
                   "(LCMOE_ACT_F16, the default: layer rel-L2 3.6e-4 vs the reference CPU path), "
                   "exact int8 dot4 on 15-bit two-limb activations below; f32 accumulate")),
        "data": ("synthetic (seeded splitmix64 N(0,1) activations, N(0,0.02) weights quantised "
                 f"to {qdesc})"),
        "config": {
            "workload": f"config {args.config}: {cfg.note}, d_model={cfg.d_model}, d_ff={cfg.d_ff}, "
                        f"E={cfg.n_expert}, top-{cfg.n_expert_used}, T={args.tokens} tokens/step"
                        + (", with RMSNorm + residual" if args.norm_residual else ""),
            "entry": "lcmoe_forward_norm_residual_dev" if args.norm_residual else "lcmoe_forward_dev",
            "batch": args.tokens, "d_model": cfg.d_model, "d_ff": cfg.d_ff,
            "n_expert": cfg.n_expert, "top_k": cfg.n_expert_used, "replicas": R,
            "device_warmup_s": args.device_warmup,
        },
        "roofline": roof,
        "layer_roofline_frac": round(head["layer_GBps"] / HBM_PEAK_GBS, 4),
        "per_batch": {str(T): {k: (round(v, 4) if isinstance(v, float) else v)
                               for k, v in d.items() if k != "kernel_ms"} |
                      {"kernel_ms": {k: round(v, 5) for k, v in d["kernel_ms"].items()},
                       "layer_frac": round(d["layer_GBps"] / HBM_PEAK_GBS, 4)}
                      for T, d in per_batch.items()},
        "synth_s": round(t_synth, 2),
    }
    for m in moes:
        m.close()
    if roof["bound"] == "hbm":
        # the practical ceiling beside the 8 TB/s peak: a plain streaming read
        # of slices the size of the dominant launch's bytes (past the MALL)
        sl = max(16, min(1024, int(round(roof["algorithmic_bytes"] / 2 ** 24)) * 16))
        bw = L.read_bandwidth(sl, reps=8)
        roof["stream_read_GBps"] = round(bw, 1)
        roof["stream_read_slice_MiB"] = sl
        roof["frac_of_stream"] = round(roof["achieved"] / bw, 4)
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(cfg, layer, sweep, args.tokens)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
