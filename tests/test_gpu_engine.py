"""GPU: the end-to-end decoder model (lcmoe_model_*) against the oracle's
composition of the reference engine (oracle/lcengine.py, pinned in
tests/test_oracle_engine.py).

Bar: last-token logits within 1e-3 relative L2 of the oracle at every
forward (prefill and decode, teacher-forced on the same ids); greedy ids
identical to the oracle's except from a step whose top-2 logits are within
rounding of each other (none occur in these cases; the check says so)."""
import numpy as np
import pytest

import lcengine as E
import lcoracle as O
import leafcutterllm_amd as L
from leafcutterllm_amd.configs import MODEL_CONFIGS, ModelConfig, small_config, synth_model
from test_oracle_engine import TINY, rel, spec

pytestmark = pytest.mark.gpu

LOGIT_TOL = 1e-3


def assert_same_greedy(got, ref, trace):
    for i, (g, r) in enumerate(zip(got, ref)):
        if g != r:
            lg = trace[i]
            gap = abs(float(lg[r]) - float(lg[g])) / float(np.sqrt(np.mean(lg.astype(np.float64) ** 2)))
            assert gap < 1e-4, f"step {i}: {g} != {r} with a clear margin ({gap:.2e})"
            return
    assert len(got) == len(ref)


def model(mc, w, mode, n_layer=0, B=4, P=16, ctx=64):
    return L.Model(mc.desc(B, P, ctx, mode, n_layer=n_layer), w)


@pytest.mark.parametrize("mode", [E.ROPE_PER_CALL, E.ROPE_ABSOLUTE])
def test_tiny_forward_matches_oracle(mode):
    w = synth_model(TINY, seed=7)
    ref = E.RefEngine(spec(TINY, mode), w, threads=8)
    calls = [[5, 17, 3, 95, 0, 60, 200], [11], [42], [7], [1, 2]]
    print(f"tiny model mode={mode}", flush=True)
    with model(TINY, w, mode) as m:
        for c in calls:
            g = m.forward(np.array([c]))[0]
            r = ref.forward(c)
            assert rel(g, r.astype(np.float64)) < LOGIT_TOL, rel(g, r.astype(np.float64))
        m.reset()
        ref.clear()
        assert rel(m.forward(np.array([[9, 8, 7]]))[0], ref.forward([9, 8, 7])) < LOGIT_TOL


def test_tiny_batch_rows_are_independent():
    """Three sequences prefilled separately, then decoded together: each row
    equals its own single-sequence run."""
    w = synth_model(TINY, seed=8)
    prompts = [[1, 2, 3, 4], [50, 60, 70, 80], [9, 9, 9, 9]]
    steps = [[10, 20, 30], [11, 21, 31], [12, 22, 32]]
    with model(TINY, w, E.ROPE_PER_CALL) as m:
        m.forward(np.array(prompts))                    # T > 1: one sequence per call
        batch = [m.forward(np.array([[s[i]] for s in steps])) for i in range(3)]
    for b in range(3):
        ref = E.RefEngine(spec(TINY, E.ROPE_PER_CALL), w, threads=8)
        ref.forward(prompts[b])
        for i in range(3):
            r = ref.forward([steps[b][i]])
            assert rel(batch[i][b], r.astype(np.float64)) < LOGIT_TOL


@pytest.mark.parametrize("mode", [E.ROPE_PER_CALL, E.ROPE_ABSOLUTE])
def test_tiny_generate_matches_oracle(mode):
    """Greedy generation through the captured decode graph, three sequences
    at once, twice in a row (graph reuse), then with two (a new graph)."""
    w = synth_model(TINY, seed=9)
    prompts = np.array([[3, 1, 4, 1, 5, 9], [2, 7, 1, 8, 2, 8], [90, 91, 92, 93, 94, 95]])
    n_new = 12
    refs = []
    for p in prompts:
        ref = E.RefEngine(spec(TINY, mode), w, threads=8)
        refs.append(ref.generate(list(p), n_new))
    with model(TINY, w, mode) as m:
        for B in (3, 3, 2):
            out, n = m.generate(prompts[:B], n_new)
            assert np.all(n == n_new)
            for b in range(B):
                assert_same_greedy(list(out[b]), refs[b][0], refs[b][1])
        eos = refs[0][0][3]
        out, n = m.generate(prompts[:1], n_new, eos=eos)
        assert n[0] == refs[0][0].index(eos) + 1
        pre, dec = m.last_timing()
        assert pre > 0 and dec > 0


@pytest.mark.parametrize("qt", [L.TYPE_Q8_0, L.TYPE_F32])
def test_tiny_other_weight_types(qt):
    mc = ModelConfig("tiny-q", 2, 4, 4, 64, 64, 500.0,
                     small_config("tiny-q8", 256, 256, 8, 2, L.ROUTE_SOFTMAX, L.TYPE_Q8_0,
                                  L.TYPE_Q8_0), attn_type=qt)
    w = synth_model(mc, seed=10)
    ref = E.RefEngine(spec(mc, E.ROPE_ABSOLUTE), w, threads=8)
    with model(mc, w, E.ROPE_ABSOLUTE) as m:
        for c in ([4, 5, 6, 7, 8], [1], [63]):
            assert rel(m.forward(np.array([c]))[0], ref.forward(c).astype(np.float64)) < LOGIT_TOL


@pytest.mark.parametrize("hd,H,KVH", [(160, 2, 1), (256, 2, 2)])
def test_tiny_wide_heads(hd, H, KVH):
    """head_dim above 128 (the attention's widest K-load form, a head_dim
    that is not a power of two, grouped KV heads) over a prompt longer than
    one 128-position attention chunk, then single-token steps."""
    mc = ModelConfig("tiny-wide", 2, H, KVH, hd, 64, 10000.0,
                     small_config("tiny-wide", 256, 256, 8, 2, L.ROUTE_SOFTMAX_RENORM,
                                  L.TYPE_Q8_0, L.TYPE_Q8_0), attn_type=L.TYPE_Q8_0)
    w = synth_model(mc, seed=12)
    ref = E.RefEngine(spec(mc, E.ROPE_ABSOLUTE), w, threads=8)
    with model(mc, w, E.ROPE_ABSOLUTE, B=1, P=160, ctx=192) as m:
        for c in ([(7 * i + 3) % 64 for i in range(150)], [1], [2]):
            assert rel(m.forward(np.array([c]))[0], ref.forward(c).astype(np.float64)) < LOGIT_TOL


def test_config5_two_layer_cut():
    """The config-5 model's shapes (d 2048, 16 heads x 128, vocab 32000, the
    60+4-expert Q4_K MoE) cut to two layers: per-step logits and greedy ids
    for two sequences."""
    mc = MODEL_CONFIGS[5]
    w = synth_model(mc, seed=11, n_layer=2)
    s = spec(mc, E.ROPE_PER_CALL, n_layer=2)
    prompts = np.array([[(37 * i + 11) % mc.vocab for i in range(12)],
                        [(101 * i + 5) % mc.vocab for i in range(12)]])
    n_new = 5
    refs = []
    for p in prompts:
        refs.append(E.RefEngine(s, w, threads=16).generate(list(p), n_new))
    print("config-5 cut: oracle done", flush=True)
    with L.Model(mc.desc(2, 16, 32, E.ROPE_PER_CALL, n_layer=2), w) as m:
        out, n = m.generate(prompts, n_new)
        for b in range(2):
            assert_same_greedy(list(out[b]), refs[b][0], refs[b][1])
        # teacher-forced logits at every step, both sequences in one batch
        m.reset()
        first = m.forward(prompts)
        for b in range(2):
            assert rel(first[b], refs[b][1][0].astype(np.float64)) < LOGIT_TOL
        for i in range(1, n_new):
            lg = m.forward(np.array([[refs[0][0][i - 1]], [refs[1][0][i - 1]]]))
            for b in range(2):
                e = rel(lg[b], refs[b][1][i].astype(np.float64))
                print(f"config-5 cut step {i} seq {b}: logits rel-L2 {e:.2e}", flush=True)
                assert e < LOGIT_TOL


def test_eager_decode_equals_graph():
    w = synth_model(TINY, seed=12)
    prompts = np.array([[4, 8, 15, 16, 23, 42], [1, 1, 2, 3, 5, 8]])
    with model(TINY, w, E.ROPE_ABSOLUTE) as m:
        g, _ = m.generate(prompts, 10)
        m.set_decode_graph(False)
        e, _ = m.generate(prompts, 10)
        m.set_decode_graph(True)
        g2, _ = m.generate(prompts, 10)
    assert np.array_equal(g, e) and np.array_equal(g, g2)


def test_tiny_long_context_batch16_vs_oracle():
    """Sixteen sequences with 640-token prompts decoded together for 128
    steps (767 cache positions: six 128-position attention chunks; the
    batched matrix-core linears), each row against the oracle's engine
    teacher-forced on the same ids.  Logits agree within 1e-3 relative L2 at
    every step up to the first token that some layer routes to different
    experts than the oracle does (the two compute the router's input in
    different orders); that token must be a near-tie: the swapped experts'
    weights agree within 1e-3."""
    from test_gpu_config5_full import assert_near_tie, first_swap
    w = synth_model(TINY, seed=13)
    B, P, N = 16, 640, 128
    pr = np.array([[(17 * i + 31 * b + 5) % TINY.vocab for i in range(P)] for b in range(B)])
    with model(TINY, w, E.ROPE_PER_CALL, B=B, P=P, ctx=P + N) as m:
        ids, _ = m.generate(pr, N)
        m.reset()
        lg = [m.forward(pr)]
        rt = [None]
        for i in range(1, N):
            lg.append(m.forward(ids[:, i - 1:i]))
            rt.append([m.layer_routing(l) for l in range(TINY.n_layer)])
    reach, worst = [], 0.0
    for b in range(B):
        ref = E.RefEngine(spec(TINY, E.ROPE_PER_CALL), w, threads=8)
        e = rel(lg[0][b], ref.forward(list(pr[b])).astype(np.float64))
        assert e < LOGIT_TOL, (b, 0, e)
        worst = max(worst, e)
        ref.record_routing = True
        i = 1
        while i < N:
            ref.routing = []
            r = ref.forward([int(ids[b, i - 1])]).astype(np.float64)
            sw = first_swap(rt[i], ref.routing, row_a=b)
            if sw is not None:
                assert_near_tie(sw, (b, i))
                break
            e = rel(lg[i][b], r)
            worst = max(worst, e)
            assert e < LOGIT_TOL, (b, i, e)
            i += 1
        reach.append(i)
    print(f"tiny long context: worst rel-L2 {worst:.2e}, steps compared per row {reach}", flush=True)
    assert sum(reach) >= B * N // 2   # most of the decode is compared
