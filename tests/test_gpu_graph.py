"""The correction pass recorded into a HIP graph: every replay equals an eager pass bit for bit.

Replays are interleaved with eager passes and host synchronisations, and each is checked (graph
replays have produced wrong results after the first on this hardware when memset nodes were
recorded, so one replay proves nothing). The running statistics keep accumulating over replays as
they do over eager passes. Two graphs, each owning its scratch memory (split-K partials), replay at
the same time on two streams and both equal their eager passes.
"""

import numpy as np
import pytest
import torch

from appcorr_amd import kernels as K
from tests.test_gpu_packed_run import _clone_context, _executor
from tests.util import assert_bits_equal

pytestmark = pytest.mark.gpu

STATS = ("_token_pscore_kept_mass_total", "_partial_token_kept_patch_total")


def _restore(ctx, pristine):
    """Inputs and caches back to their recorded-time values (in place); running statistics untouched."""
    for k, v in pristine["cache_feature"].items():
        if torch.is_tensor(v) and not k.startswith("_"):
            ctx["cache_feature"][k].copy_(v)


def _eager_one_pass(ex, params, config, pristine):
    e = _clone_context(pristine)
    for k in list(e["cache_feature"]):
        if k.endswith("_total"):
            del e["cache_feature"][k]
    with torch.no_grad():
        ex.correct_forward(params, e, config)
    torch.cuda.synchronize()
    return e


@pytest.mark.parametrize("bb,B,keep,layers", [("vits16", 2, 0.25, (0, 4)), ("vitl16", 16, 0.25, (0, 3))])
def test_graph_replays_equal_eager(dev, bb, B, keep, layers):
    ex, config, ctx = _executor(dev, bb, B, keep, 0.0, layers)
    params = {"layers": layers, "group_id": 1}
    pristine = _clone_context(ctx)
    g = _clone_context(ctx)
    base = {k: float(g["cache_feature"][k]) if torch.is_tensor(g["cache_feature"].get(k)) else 0.0 for k in STATS}
    keys = [f"layer{i}_{s}" for i in range(*layers) for s in ("kv", "blocks_out_sum")]
    replay = ex.capture_correct_forward(params, g, config)
    running = {k: np.float32(base[k]) for k in STATS}
    for it in range(3):
        print(f"case {bb} replay {it}", flush=True)
        _restore(g, pristine)
        replay()
        torch.cuda.synchronize()
        e = _eager_one_pass(ex, params, config, pristine)
        assert_bits_equal(g["current_feature"], e["current_feature"].cpu(), f"x_out, replay {it}")
        for k in keys:
            assert_bits_equal(g["cache_feature"][k], e["cache_feature"][k].cpu(), f"{k}, replay {it}")
        for k in STATS:  # running totals: one pass's value added per replay, in fp32
            running[k] = np.float32(running[k] + np.float32(float(e["cache_feature"][k])))
            assert float(g["cache_feature"][k]) == float(running[k]), (k, it)


def test_two_graphs_replay_concurrently(dev):
    """ViT-S at B = 2 splits fc2's K (the partials live in the stream scratch): two recorded passes own
    different scratch buffers, so replaying them at the same time on two streams is safe."""
    ex, config, ctx = _executor(dev, "vits16", 2, 0.25, 0.0, (0, 4))
    params = {"layers": (0, 4), "group_id": 1}
    pristine = _clone_context(ctx)
    ga, gb = _clone_context(ctx), _clone_context(ctx)
    gb["input_tokens"] = (gb["input_tokens"].float() * 0.5).to(torch.bfloat16)   # a different pass
    ra = ex.capture_correct_forward(params, ga, config)
    rb = ex.capture_correct_forward(params, gb, config)
    pa = {t.data_ptr() for t in ra.replay.scratch}
    pb = {t.data_ptr() for t in rb.replay.scratch}
    assert pa and pb and not (pa & pb), "each graph owns its scratch"
    pristine_b = _clone_context(pristine)
    pristine_b["input_tokens"] = gb["input_tokens"].clone()
    sa, sb = torch.cuda.Stream(device=dev), torch.cuda.Stream(device=dev)
    for it in range(3):
        print(f"concurrent replay {it}", flush=True)
        _restore(ga, pristine)
        _restore(gb, pristine)
        torch.cuda.synchronize()
        with torch.cuda.stream(sa):
            ra()
        with torch.cuda.stream(sb):
            rb()
        torch.cuda.synchronize()
        ea = _eager_one_pass(ex, params, config, pristine)
        eb = _eager_one_pass(ex, params, config, pristine_b)
        assert_bits_equal(ga["current_feature"], ea["current_feature"].cpu(), f"graph a, replay {it}")
        assert_bits_equal(gb["current_feature"], eb["current_feature"].cpu(), f"graph b, replay {it}")
    assert K.linear_splits_k(2 * (5 + 64), 384, 1536), "the case must exercise split-K scratch"
