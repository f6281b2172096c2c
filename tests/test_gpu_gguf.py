"""GPU: layers ingested from GGUF files (MoeFfn.from_gguf over lcmoe_gguf_*)
run bit-identically to the same layers created from arrays, and pass the
oracle parity bar (routing exact, y within 1e-3 relative L2)."""
import numpy as np
import pytest

import leafcutterllm_amd as L
from leafcutterllm_amd.configs import synth_x
from parity_util import run_and_check
from test_gguf_cpu import ROUND_TRIP, make_layer_file

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", ["mixtral-per-expert", "qwen2moe-shared3d-logit-bias",
                                  "deepseek-sigmoid-group", "bf16-router-gating3"])
@pytest.mark.parametrize("T", [1, 5, 40])
def test_gguf_layer_matches_direct_and_oracle(tmp_path, name, T):
    cfg, arch, extra, opts = ROUND_TRIP[name]
    p = tmp_path / f"{name}.gguf"
    lay = make_layer_file(p, cfg, arch, extra, opts)
    x = synth_x(cfg, T, seed=11)
    # the file is closed by from_gguf before the first forward
    with L.MoeFfn.from_gguf(str(p), 0, T) as moe_g, L.MoeFfn(cfg.desc(T), lay) as moe_d:
        yg, ig, wg = moe_g.forward(x)
        yd, id_, wd = moe_d.forward(x)
        assert np.array_equal(ig, id_)
        assert np.array_equal(wg.view(np.uint32), wd.view(np.uint32))
        assert np.array_equal(yg.view(np.uint32), yd.view(np.uint32))
        run_and_check(cfg, lay, x, moe=moe_g)


def test_gguf_two_layers_one_file(tmp_path):
    """Two resident layers created from one open GgufFile."""
    cfg, arch, extra, opts = ROUND_TRIP["mixtral-llama"]
    p0 = tmp_path / "a.gguf"
    lay = make_layer_file(p0, cfg, arch, extra, opts, layer=1, extra_layers=(0,))
    x = synth_x(cfg, 9, seed=2)
    with L.GgufFile(p0) as f:
        assert f.block_count() == 2 and f.is_moe_layer(1) and not f.is_moe_layer(0)
        moe_a = L.MoeFfn.from_gguf(f, 1, 16)
        moe_b = L.MoeFfn.from_gguf(f, 1, 16)
    with moe_a, moe_b:
        ya = moe_a.ffn_forward(x)
        yb = moe_b.ffn_forward(x)
        assert np.array_equal(ya.view(np.uint32), yb.view(np.uint32))
        run_and_check(cfg, lay, x, moe=moe_a)
