"""The HIP library against the committed golden fixtures (tests/golden/*.npz), through the C ABI.

Bit-exact for the plan, row movement and NVFP4; the ViT-S correction block within the propagated
bf16 tolerance (fp32 MFMA accumulation vs the oracle's fp64), unselected rows bit-exact.
"""

import os
import sys

import numpy as np
import pytest
import torch

from appcorr_amd import kernels as K
from appcorr_amd.dinov3 import SelfAttentionBlock
from oracle import model as OM
from oracle.bf16 import bits_to_torch_bf16
from tests.util import assert_bits_equal, assert_propagated_close, bf16_ulp

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, GOLDEN)
import make_golden  # noqa: E402


def load(name):
    return np.load(os.path.join(GOLDEN, name))


def bf(a, dev):
    return bits_to_torch_bf16(a).to(dev)


def test_topk_plan_golden(dev):
    z = load("topk_plan.npz")
    for name in sorted({k.split("/")[0] for k in z.files}):
        pre, N, k = z[f"{name}/meta"].tolist()
        print(f"case {name}", flush=True)
        p = K.topk_plan(torch.from_numpy(z[f"{name}/scores"]).to(dev), k, torch.from_numpy(z[f"{name}/dindice"]).to(dev),
                        pre, N)
        for f in ("update_indice", "active_batch_idx", "active_pos_idx", "active_token_idx", "active_patch_mask",
                  "active_rope_idx", "keep_mask", "row_slot"):
            assert_bits_equal(getattr(p, f), z[f"{name}/{f}"], f"{name}/{f}")


def test_rows_golden(dev):
    z = load("rows.npz")
    b, t = torch.from_numpy(z["b"]).to(dev), torch.from_numpy(z["t"]).to(dev)
    x, bos = bf(z["x"], dev), bf(z["bos"], dev)
    x_act = K.gather_rows(x, b, t)
    assert_bits_equal(x_act, z["x_act"], "gather")
    out = K.reconstruct_scatter_persist(x, bos, torch.from_numpy(z["row_slot"]).to(dev), x_act, bf(z["x_attn"], dev),
                                        bf(z["mlp"], dev))
    assert_bits_equal(out, z["x_out"], "x_out")
    assert_bits_equal(bos, z["bos_new"], "blocks_out_sum (in place)")
    kv = bf(z["kv"], dev)
    K.scatter_rows(kv, b, t, bf(z["kv_rows"], dev))
    assert_bits_equal(kv, z["kv_new"], "K/V scatter")


def test_nvfp4_golden(dev):
    z = load("nvfp4.npz")
    x = bf(z["x"], dev)
    ts = torch.from_numpy(z["ts"]).to(dev)
    q, s = K.quantize_nvfp4_swizzled(x, ts)
    assert_bits_equal(q, z["qdata"], "qdata")
    assert_bits_equal(s.view(torch.uint8), z["scales"], "scales")
    assert_bits_equal(K.dequantize_nvfp4(q, s, ts), z["deq"], "dequantized")


def test_vits_block_golden(dev):
    z = load("vits_block.npz")
    cfg, weights = make_golden.vits_block_weights()
    blk = SelfAttentionBlock(cfg.dim, cfg.heads, ffn_ratio=cfg.ffn_hidden / cfg.dim, qkv_bias=True,
                             init_values=1.0, mask_k_bias=True)
    blk.load_state_dict(weights[0], strict=True)
    blk = blk.to(device=dev, dtype=torch.bfloat16)
    sin, cos = OM.rope_tables(cfg)
    cache = {"layer0_kv": bf(z["kv_in"], dev), "layer0_blocks_out_sum": bf(z["bos_in"], dev)}
    dind = OM.full_dindice(cfg, 1).to(dev)
    with torch.no_grad():
        x_out, cache = blk.correct(bf(z["x_in"], dev), dind, (sin.to(dev), cos.to(dev)), cache, "layer0",
                                   token_keep_ratio=0.5, mobile_pscore="residual_energy", mobile_pscore_weight=1.0,
                                   mobile_pscore_hint=torch.from_numpy(z["importance"]).to(dev),
                                   server_pscore_weight=0.0)
    plan = next(iter(cache["_partial_token_query_plan_cache"].values()))
    assert_bits_equal(plan.update_indice, z["update_indice"], "update_indice")
    sel = np.zeros(x_out.shape[:2], dtype=bool)
    sel[0, z["update_indice"][0]] = True
    ref = bits_to_torch_bf16(z["x_out"])
    assert_bits_equal(x_out.cpu()[torch.from_numpy(~sel)], ref[torch.from_numpy(~sel)], "unselected rows")
    assert_propagated_close(x_out, ref, what="x_out")
    assert_propagated_close(cache["layer0_kv"], bits_to_torch_bf16(z["kv_out"]), max_ulps=2, mean_rel=2.0 ** -12,
                            what="K/V")
    bos_ref = bits_to_torch_bf16(z["bos_out"])
    floor = 4 * bf16_ulp(ref.float().abs().numpy() + bos_ref.float().abs().numpy())
    assert_propagated_close(cache["layer0_blocks_out_sum"], bos_ref, floor_abs=floor, what="blocks_out_sum")
