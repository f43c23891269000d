"""The correction pass recorded into a HIP graph: every replay equals an eager pass bit for bit.

Replays are interleaved with eager passes and host synchronisations, and each is checked (graph
replays have produced wrong results after the first on this hardware when memset nodes were
recorded, so one replay proves nothing).
"""

import pytest
import torch

from tests.test_gpu_packed_run import _clone_context, _executor
from tests.util import assert_bits_equal

pytestmark = pytest.mark.gpu


def _restore(ctx, pristine):
    for k, v in pristine["cache_feature"].items():
        if torch.is_tensor(v):
            ctx["cache_feature"][k].copy_(v)


@pytest.mark.parametrize("bb,B,keep,layers", [("vits16", 2, 0.25, (0, 4)), ("vitl16", 16, 0.25, (0, 3))])
def test_graph_replays_equal_eager(dev, bb, B, keep, layers):
    ex, config, ctx = _executor(dev, bb, B, keep, 0.0, layers)
    params = {"layers": layers, "group_id": 1}
    pristine = _clone_context(ctx)
    g = _clone_context(ctx)
    keys = [f"layer{i}_{s}" for i in range(*layers) for s in ("kv", "blocks_out_sum")]
    replay = ex.capture_correct_forward(params, g, config)
    for it in range(3):
        print(f"case {bb} replay {it}", flush=True)
        _restore(g, pristine)
        replay()
        torch.cuda.synchronize()
        e = _clone_context(pristine)
        with torch.no_grad():
            ex.correct_forward(params, e, config)
        torch.cuda.synchronize()
        assert_bits_equal(g["current_feature"], e["current_feature"].cpu(), f"x_out, replay {it}")
        for k in keys:
            assert_bits_equal(g["cache_feature"][k], e["cache_feature"][k].cpu(), f"{k}, replay {it}")
        for k in ("_token_pscore_kept_mass_total", "_partial_token_kept_patch_total"):
            assert float(g["cache_feature"][k]) == float(e["cache_feature"][k]), (k, it)
