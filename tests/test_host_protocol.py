"""Host-side logic of the drop-in (CPU only): option normalisation, the executor registry, group plans,
the block's parameter names, the product path's refusal of CPU tensors, and bench.py's one-GPU rule.

Semantics follow offload/common/protocol.py:6-181 and offload/server/model/__init__.py:4-40.
"""

import os
import subprocess
import sys

import pytest
import torch

from appcorr_amd import kernels as K
from appcorr_amd.dinov3 import SelfAttentionBlock
from appcorr_amd.server import default_appcorr_kwargs, get_model_executor, normalize_appcorr_kwargs
from appcorr_amd.server.dinov3_classifier import make_group_plan

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_defaults_match_reference_values():
    d = default_appcorr_kwargs()
    assert d["token_keep_ratio"] == 0.2 and d["token_keep_thres"] is None
    assert d["server_pscore"] == "cls_attn_prob" and d["server_pscore_weight"] == 1.0
    assert d["mobile_pscore"] == "none" and d["mobile_pscore_weight"] == 0.0
    assert d["pscore_fusion"] == "add" and d["method"] == "partial_token" and d["num_groups"] == 1
    # empty kwargs -> disabled; any explicit option enables unless "enabled" says otherwise
    assert normalize_appcorr_kwargs({})["enabled"] is False
    assert normalize_appcorr_kwargs({"token_keep_ratio": 0.5})["enabled"] is True
    assert normalize_appcorr_kwargs({"token_keep_ratio": 0.5, "enabled": False})["enabled"] is False


def test_aliases_and_coercions():
    o = normalize_appcorr_kwargs({"mobile_pscore": "patch_residual_l2", "pscore_fusion": "mul",
                                  "server_pscore": "pseudo_patch_attn_prob", "token_keep_thres": "None",
                                  "num_groups": 0, "sdpa_query_bucket_size": -3, "token_prune_min_keep": 0})
    assert o["mobile_pscore"] == "residual_energy"
    assert o["pscore_fusion"] == "multiply"
    assert o["server_pscore"] == "patch_pseudo_attn_prob"
    assert o["token_keep_thres"] is None
    assert o["num_groups"] == 1 and o["sdpa_query_bucket_size"] == 0 and o["token_prune_min_keep"] == 1
    assert normalize_appcorr_kwargs({"cls_alive_ratio": 0.3})["token_keep_ratio"] == 0.3
    assert normalize_appcorr_kwargs({"token_prune_score": "patch_attn_prob"})["server_pscore"] == "patch_attn_prob"
    o = normalize_appcorr_kwargs({"server_pscore": "cls_attn_prob", "server_pscore_layer_fusion": "mean"})
    assert o["server_pscore"] == "cls_attn_prob_layermean"
    assert normalize_appcorr_kwargs({"pscore_fusion": "bogus"})["pscore_fusion"] == "add"


def test_validation_errors():
    with pytest.raises(ValueError, match="Unknown server_pscore"):
        normalize_appcorr_kwargs({"server_pscore": "nope"})
    with pytest.raises(ValueError, match="persist_correction_residual"):
        normalize_appcorr_kwargs({"persist_correction_residual": True})
    with pytest.raises(ValueError, match="num_groups must match"):
        normalize_appcorr_kwargs({"num_groups": 2}, {"num_groups": 4})
    with pytest.raises(ValueError, match="pyramid_levels must match"):
        normalize_appcorr_kwargs({"pyramid_levels": [0]}, {"pyramid_levels": [0, 1]})
    assert normalize_appcorr_kwargs({"token_keep_ratio": 0.1}, {"num_groups": 4})["num_groups"] == 4


def test_executor_registry():
    ex = get_model_executor("dinov3_vitl16_classifier", torch.device("cpu"))
    assert type(ex).__name__ == "DINOv3ClassifierExecutor"
    for name in ("sam3", "dinov3_vitl16_detector", "gemma3"):
        with pytest.raises(ValueError):
            get_model_executor(name, torch.device("cpu"))


def test_group_plan_fields():
    dind = torch.arange(10).unsqueeze(0).expand(3, -1).contiguous()
    gp = make_group_plan(dind, 5)
    assert gp.prefix_dindice.shape == (3, 5) and gp.group_patch_dindice.shape == (3, 5)
    assert torch.equal(gp.group_patch_keep_local_idx[1], torch.arange(5))
    assert gp.full_patch_count.tolist() == [5, 5, 5]


def test_block_parameter_names_match_reference_tree():
    names = set(SelfAttentionBlock(64, 4, qkv_bias=True, mask_k_bias=True, init_values=1e-5).state_dict())
    want = {"norm1.weight", "norm1.bias", "attn.qkv.weight", "attn.qkv.bias", "attn.qkv.bias_mask",
            "attn.proj.weight", "attn.proj.bias", "ls1.gamma", "norm2.weight", "norm2.bias", "mlp.fc1.weight",
            "mlp.fc1.bias", "mlp.fc2.weight", "mlp.fc2.bias", "ls2.gamma"}
    assert names == want
    sw = set(SelfAttentionBlock(128, 4, ffn_layer="swiglu64", ffn_ratio=3.0).state_dict())
    assert {"mlp.w1.weight", "mlp.w2.weight", "mlp.w3.weight"} <= sw


def test_product_path_refuses_cpu_tensors():
    x = torch.zeros(4, 8, 16, dtype=torch.bfloat16)
    idx = torch.zeros(2, dtype=torch.long)
    with pytest.raises(Exception):
        K.gather_rows(x, idx, idx)
    with pytest.raises(Exception):
        K.layer_norm(x.view(-1, 16), torch.ones(16, dtype=torch.bfloat16), torch.zeros(16, dtype=torch.bfloat16))


@pytest.mark.parametrize("cap", [0, 4])
def test_threshold_selection_has_no_cpu_fallback(cap):
    """Both threshold builders reach the HIP plan kernels, which refuse CPU tensors."""
    blk = SelfAttentionBlock(64, 4).to(torch.bfloat16)
    kv = torch.zeros(1, 9, 2, 4, 16, dtype=torch.bfloat16)
    cache = {"layer0_kv": kv, "layer0_blocks_out_sum": torch.zeros(1, 9, 64, dtype=torch.bfloat16)}
    with pytest.raises(ValueError, match="GPU only"):
        blk.correct(torch.zeros(1, 9, 64, dtype=torch.bfloat16), torch.arange(9)[None], None, cache, "layer0",
                    token_keep_thres="0.5", token_keep_cap=cap, num_pretokens=1, server_pscore_weight=0.0,
                    appcorr_method="partial_token")


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 2 and "one MI355X" in r.stderr


def test_explicit_low_precision_request_raises_when_unavailable():
    """dinov3_precision.py:723-731: an explicit fp8 request the build cannot serve is an error, not a
    silent bf16 run; bf16 and auto construct normally."""
    from torch import nn

    from appcorr_amd.server.precision import DINOv3CorrectPrecisionController

    blocks = nn.ModuleList()
    for p in ("bf16", "auto"):
        c = DINOv3CorrectPrecisionController(blocks, precision=p)
        assert c.event_metadata()["correct_precision_requested"] == p
    with pytest.raises(RuntimeError, match="fp8"):
        DINOv3CorrectPrecisionController(blocks, precision="fp8")
    with pytest.raises(ValueError):
        DINOv3CorrectPrecisionController(blocks, precision="int3")


def test_device_pointer_array_lives_with_its_holder():
    """The fold kernel's pointer array is cached in the dict that owns the pointed-to tensors and is
    dropped only once that dict no longer holds all of them (a graph over them could not replay)."""
    holder = {"layer0_blocks_out_sum": torch.zeros(4), "layer1_blocks_out_sum": torch.zeros(4)}
    ptrs = [holder["layer0_blocks_out_sum"].data_ptr(), holder["layer1_blocks_out_sum"].data_ptr()]
    a = K.device_pointer_array(ptrs, "cpu", holder)
    assert a.tolist() == ptrs
    assert K.device_pointer_array(ptrs, "cpu", holder) is a          # cached: no new host copy
    one = K.device_pointer_array(ptrs[:1], "cpu", holder)             # another list over live tensors
    store = holder[K.POINTER_ARRAYS_KEY]
    assert len(store) == 2
    holder["layer1_blocks_out_sum"] = torch.ones(4)                   # a new approx pass replaces a tensor
    new_ptrs = [ptrs[0], holder["layer1_blocks_out_sum"].data_ptr()]
    b = K.device_pointer_array(new_ptrs, "cpu", holder)
    assert b.tolist() == new_ptrs
    keys = {k[1] for k in store}
    assert tuple(ptrs) not in keys, "array over a tensor the holder dropped must be evicted"
    assert tuple(ptrs[:1]) in keys and store[("cpu", tuple(ptrs[:1]))] is one
    assert K.device_pointer_array(ptrs, "cpu", None) is not a         # no holder: a fresh array each call


def test_stream_workspace_keeps_outgrown_buffers(monkeypatch):
    """The per-stream fp32 scratch is reused while it is large enough; when it grows, the old buffer
    stays allocated under its stream (a graph recorded on that stream keeps its address) and the new
    one at least doubles, so only a few buffers are ever retired."""
    from appcorr_amd import _lib
    monkeypatch.setattr(_lib, "stream_of", lambda t: 12345)
    monkeypatch.setattr(K, "_STREAM_WS", {})
    monkeypatch.setattr(K, "_RETIRED_WS", {})
    x = torch.zeros(1)
    key = (x.device, 12345)
    a = K._stream_workspace(x, 100)
    assert a.numel() == 100 and K._stream_workspace(x, 60) is a
    b = K._stream_workspace(x, 150)
    assert b is not a and b.numel() == 200 and K._RETIRED_WS == {key: [a]}
    c = K._stream_workspace(x, 1000)
    assert c.numel() == 1000 and K._RETIRED_WS[key][-1] is b
    assert K._stream_workspace(x, 1000) is c and len(K._RETIRED_WS[key]) == 2


def test_stream_workspaces_are_per_stream_and_taken_by_a_graph(monkeypatch):
    """Launch sequences on different streams get different scratch buffers; taking a stream's buffers
    (what graphs.capture does after recording on its own stream) hands over the current one and the
    ones it outgrew, leaves the other streams' untouched, and the next launch on that stream gets a
    fresh buffer instead of the one the graph now owns."""
    from appcorr_amd import _lib
    cur = {"s": 1}
    monkeypatch.setattr(_lib, "stream_of", lambda t: cur["s"])
    monkeypatch.setattr(K, "_STREAM_WS", {})
    monkeypatch.setattr(K, "_RETIRED_WS", {})
    x = torch.zeros(1)
    a1 = K._stream_workspace(x, 10)
    cur["s"] = 2
    b1 = K._stream_workspace(x, 10)
    b2 = K._stream_workspace(x, 50)
    assert a1 is not b1 and b2 is not b1
    owned = K.take_stream_workspaces(x.device, 2)
    assert len(owned) == 2 and owned[0] is b1 and owned[1] is b2
    assert (x.device, 2) not in K._STREAM_WS and (x.device, 2) not in K._RETIRED_WS
    assert K._STREAM_WS[(x.device, 1)] is a1
    b3 = K._stream_workspace(x, 10)
    assert b3 is not b1 and b3 is not b2 and b3.numel() == 10
    assert K.take_stream_workspaces(x.device, 99) == []


def test_trace_ranges_nest_and_survive_exceptions():
    """roctx ranges (the reference's NVTX annotations) are balanced even when the body raises."""
    from appcorr_amd import tracing

    @tracing.annotate("outer")
    def f(fail):
        with tracing.trace_range("inner"):
            if fail:
                raise KeyError("x")
        return 3

    assert f(False) == 3
    with pytest.raises(KeyError):
        f(True)
    with tracing.trace_range("after"):
        pass
