"""Selected rows kept packed across a run of correction blocks: bit-identical to the block-by-block path.

The per-block path (gather -> block -> reconstruct_scatter_persist, block.py:1111-1179, for each layer
of the executor loop dinov3_classifier.py:591-663) is itself checked against the oracle elsewhere;
here the packed run (packed_residual_persist per block, one fold_residual_rows at the end) must give
the same bits for the output tokens, every layer's K/V cache and every layer's blocks_out_sum.
"""

import numpy as np
import pytest
import torch

from appcorr_amd import kernels as K
from appcorr_amd.dinov3.layers import SelfAttentionBlock, correct_blocks_packed
from appcorr_amd.server.dinov3_classifier import DINOv3ClassifierExecutor, make_group_plan
from appcorr_amd.server.protocol import ExperimentConfig
from tests.util import assert_bits_equal

pytestmark = pytest.mark.gpu


def _rand_bf16(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(torch.bfloat16)


@pytest.mark.parametrize("B,N,C,M,L", [(16, 261, 1024, 1104, 24), (2, 9, 8, 5, 0), (3, 7, 16, 7, 1),
                                       (2, 33, 24, 20, 5), (1, 201, 384, 0, 3)])
def test_fold_equals_blockwise_reconstruct(dev, B, N, C, M, L):
    """L blocks of random corrections: per block reconstruct_scatter_persist over the full tensor vs
    packed_residual_persist on the packed rows and one fold at the end (bit-exact, both the
    outputs and every blocks_out_sum)."""
    rng = np.random.default_rng(B * 1000 + N + L)
    flat = np.sort(rng.choice(B * N, M, replace=False))
    bi = torch.from_numpy(flat // N).to(dev)
    ti = torch.from_numpy(flat % N).to(dev)
    row_slot = torch.full((B * N,), -1, dtype=torch.int32)
    row_slot[torch.from_numpy(flat)] = torch.arange(M, dtype=torch.int32)
    row_slot = row_slot.view(B, N).to(dev)
    x = _rand_bf16((B, N, C), 1).to(dev)
    bos0 = [_rand_bf16((B, N, C), 10 + i, 0.1).to(dev) for i in range(L)]
    upd = [(_rand_bf16((M, C), 100 + i, 0.5).to(dev), _rand_bf16((M, C), 200 + i, 0.2).to(dev)) for i in range(L)]

    # block by block over the full tensor
    xr, bos_r = x.clone(), [b.clone() for b in bos0]
    for i in range(L):
        x_act = K.gather_rows(xr, bi, ti) if M else xr.new_empty((0, C))
        x_attn = (x_act.float() + upd[i][0].float()).to(torch.bfloat16)
        xr = K.reconstruct_scatter_persist(xr, bos_r[i], row_slot, x_act, x_attn, upd[i][1])

    # packed
    bos_p = [b.clone() for b in bos0]
    xp = K.gather_rows(x, bi, ti) if M else x.new_empty((0, C))
    for i in range(L):
        x_attn = (xp.float() + upd[i][0].float()).to(torch.bfloat16)
        if M:
            xp = K.packed_residual_persist(xp, x_attn, upd[i][1], bi, ti, bos_p[i])
    out = K.fold_residual_rows(x, row_slot, xp, bos_p)
    assert_bits_equal(out, xr.cpu(), "x_out")
    for i in range(L):
        assert_bits_equal(bos_p[i], bos_r[i].cpu(), f"blocks_out_sum[{i}]")
    # in place (out aliases x)
    x2 = x.clone()
    assert K.fold_residual_rows(x2, row_slot, xp, bos_p, out=x2).data_ptr() == x2.data_ptr()
    assert_bits_equal(x2, xr.cpu(), "x_out in place")


def _executor(dev, bb, B, keep, server_w, layers):
    img = 256
    grid = img // 16
    P = grid * grid
    N = 5 + P
    config = ExperimentConfig(model_name=f"dinov3_classifier_{bb}", batch_size=B, image_shape=(img, img, 3),
                              backbone=bb, appcorr_kwargs={
                                  "method": "partial_token", "token_keep_ratio": keep,
                                  "mobile_pscore": "residual_energy", "mobile_pscore_weight": 1.0,
                                  "server_pscore_weight": server_w, "pscore_fusion": "add"})
    torch.manual_seed(0)
    ex = DINOv3ClassifierExecutor(dev)
    ex.load_model(config.model_name, config)
    C = ex.model.embed_dim
    g = torch.Generator(device=dev).manual_seed(3)
    x_base = torch.randn(B, N, C, generator=g, device=dev)
    delta = torch.randn(B, P, C, generator=g, device=dev)
    x_full = x_base.clone()
    x_full[:, 5:] += delta
    context = {"input_tokens": x_base.to(torch.bfloat16).contiguous(), "rope_sincos": ex.model.rope_embed(H=grid, W=grid)}
    dind = torch.arange(N, device=dev).unsqueeze(0).expand(B, -1).contiguous()
    context["group_plans"] = {1: make_group_plan(dind, 5)}
    with torch.no_grad():
        ex.approx_forward({"layers": layers}, context, config)
    context["input_tokens"] = x_full.to(torch.bfloat16).contiguous()
    context["mobile_pscore_hint_map"] = K.patch_importance(delta)
    return ex, config, context


def _clone_context(ctx):
    out = dict(ctx)
    out["cache_feature"] = {k: (v.clone() if torch.is_tensor(v) else v) for k, v in ctx["cache_feature"].items()}
    SelfAttentionBlock._invalidate_partial_token_derived_caches(out["cache_feature"])
    return out


@pytest.mark.parametrize("bb,B,keep,layers", [("vitl16", 16, 0.25, (0, 4)), ("vits16", 3, 0.1, (0, 12)),
                                              ("vitb16", 2, 0.0, (2, 5))])
def test_executor_packed_run_bit_identical(dev, bb, B, keep, layers):
    ex, config, ctx = _executor(dev, bb, B, keep, 0.0, layers)
    params = {"layers": layers, "group_id": 1}
    ca, cb = _clone_context(ctx), _clone_context(ctx)
    print(f"case {bb} B={B} keep={keep} layers={layers}", flush=True)
    with torch.no_grad():
        ex.packed_correction = True
        meta_a = ex.correct_forward(params, ca, config)
        ex.packed_correction = False
        meta_b = ex.correct_forward(params, cb, config)
    assert meta_a == meta_b
    assert_bits_equal(ca["current_feature"], cb["current_feature"].cpu(), "x_out")
    for i in range(*layers):
        for key in (f"layer{i}_kv", f"layer{i}_blocks_out_sum", f"layer{i}_combined_pscore"):
            assert_bits_equal(ca["cache_feature"][key], cb["cache_feature"][key].cpu(), key)
    sa = {k: float(v) for k, v in ca["cache_feature"].items() if k.startswith("_token_prune")}
    sb = {k: float(v) for k, v in cb["cache_feature"].items() if k.startswith("_token_prune")}
    assert sa == sb


def test_packed_run_declines_per_layer_plans(dev):
    """A layer-dependent server score (cls_attn_prob, weight 1) gives each block its own plan: the
    packed run declines before computing or caching anything, and the executor runs block by block."""
    ex, config, ctx = _executor(dev, "vits16", 2, 0.25, 1.0, (0, 3))
    c = _clone_context(ctx)
    before = dict(c["cache_feature"])
    res = correct_blocks_packed(list(ex.model.blocks[:3]), c["input_tokens"], ctx["group_plans"][1].pruned_dindice,
                                c["rope_sincos"], c["cache_feature"], ["layer0", "layer1", "layer2"],
                                server_pscore_weight=1.0, server_pscore="cls_attn_prob", token_keep_ratio=0.25)
    assert res is None
    assert c["cache_feature"].keys() == before.keys()
    assert all(c["cache_feature"][k] is before[k] for k in before)
    ca, cb = _clone_context(ctx), _clone_context(ctx)
    with torch.no_grad():
        ex.packed_correction = True
        ex.correct_forward({"layers": (0, 3), "group_id": 1}, ca, config)
        ex.packed_correction = False
        ex.correct_forward({"layers": (0, 3), "group_id": 1}, cb, config)
    assert_bits_equal(ca["current_feature"], cb["current_feature"].cpu(), "x_out")


def test_packed_run_in_place(dev):
    ex, config, ctx = _executor(dev, "vits16", 2, 0.25, 0.0, (0, 2))
    ca, cb = _clone_context(ctx), _clone_context(ctx)
    blocks = list(ex.model.blocks[:2])
    dind = ctx["group_plans"][1].pruned_dindice
    kw = dict(token_keep_ratio=0.25, mobile_pscore="residual_energy", mobile_pscore_weight=1.0,
              mobile_pscore_hint=ctx["mobile_pscore_hint_map"], server_pscore_weight=0.0)
    xa = ca["input_tokens"].clone()
    with torch.no_grad():
        out_a, _ = correct_blocks_packed(blocks, xa, dind, ca["rope_sincos"], ca["cache_feature"],
                                         ["layer0", "layer1"], inplace_residual_add=True, **kw)
        xb = cb["input_tokens"].clone()
        for i, blk in enumerate(blocks):
            xb, _ = blk.correct(xb, dind, cb["rope_sincos"], cb["cache_feature"], f"layer{i}", **kw)
    assert out_a.data_ptr() == xa.data_ptr()
    assert_bits_equal(out_a, xb.cpu(), "x_out")


@pytest.mark.parametrize("B,N,C,M", [(16, 261, 1024, 4176), (2, 40, 384, 30), (1, 9, 8, 3), (3, 20, 1536, 17),
                                     (2, 30, 2048, 5), (4, 414, 4096, 1656), (2, 9, 4096, 7), (1, 9, 1032, 5)])
def test_packed_residual_ln_equals_unfused(dev, B, N, C, M):
    """The residual step fused with the next block's LayerNorm equals packed_residual_persist followed by
    layer_norm, bit for bit (x_new, blocks_out_sum rows and the LayerNorm output)."""
    rng = np.random.default_rng(C + M)
    flat = np.sort(rng.choice(B * N, M, replace=False))
    bi = torch.from_numpy(flat // N).to(dev)
    ti = torch.from_numpy(flat % N).to(dev)
    x_act = _rand_bf16((M, C), 1).to(dev)
    x_attn = (x_act.float() + _rand_bf16((M, C), 2, 0.5).float().to(dev)).to(torch.bfloat16)
    mlp = _rand_bf16((M, C), 3, 0.3).to(dev)
    bos0 = _rand_bf16((B, N, C), 4, 0.1).to(dev)
    w = (1.0 + _rand_bf16((C,), 5, 0.2).float()).to(torch.bfloat16).to(dev)
    b = _rand_bf16((C,), 6, 0.1).to(dev)
    bos_u, bos_f = bos0.clone(), bos0.clone()
    x_u = K.packed_residual_persist(x_act, x_attn, mlp, bi, ti, bos_u)
    ln_u = K.layer_norm(x_u, w, b, 1e-6)
    x_f, ln_f = K.packed_residual_persist_ln(x_act, x_attn, mlp, bi, ti, bos_f, w, b, 1e-6)
    assert_bits_equal(x_f, x_u.cpu(), "x_new")
    assert_bits_equal(bos_f, bos_u.cpu(), "blocks_out_sum")
    assert_bits_equal(ln_f, ln_u.cpu(), "LayerNorm(x_new)")


@pytest.mark.parametrize("B,N,C,hid,M,with_ln", [(1, 201, 384, 1536, 103, True), (16, 1029, 1024, 4096, 1712, True),
                                                 (3, 40, 384, 1536, 72, False), (4, 700, 4096, 8192, 1656, True)])
def test_splitk_ls_residual_equals_unfused(dev, B, N, C, hid, M, with_ln):
    """The last MLP product split K with its reduce fused into the residual step (ViT-S fc2 in 12
    slices, ViT-L keep-10 % fc2 and ViT-7B w3 in 2, with and without the next block's LayerNorm)
    equals linear(EPI_BIAS_LS) followed by packed_residual_persist(_ln), bit for bit."""
    from appcorr_amd import _lib
    assert K.linear_splits_k(M, C, hid)
    rng = np.random.default_rng(C + M)
    flat = np.sort(rng.choice(B * N, M, replace=False))
    bi = torch.from_numpy(flat // N).to(dev)
    ti = torch.from_numpy(flat % N).to(dev)
    h = _rand_bf16((M, hid), 11).to(dev)
    w = _rand_bf16((C, hid), 12, 0.02).to(dev)
    fb = _rand_bf16((C,), 13, 0.1).to(dev)
    g = _rand_bf16((C,), 14, 0.5).to(dev)
    x_act = _rand_bf16((M, C), 15).to(dev)
    x_attn = (x_act.float() + _rand_bf16((M, C), 16, 0.5).float().to(dev)).to(torch.bfloat16)
    bos0 = _rand_bf16((B, N, C), 17, 0.1).to(dev)
    lw = (1.0 + _rand_bf16((C,), 18, 0.2).float()).to(torch.bfloat16).to(dev)
    lb = _rand_bf16((C,), 19, 0.1).to(dev)
    ln = (lw, lb, 1e-6) if with_ln else None
    bos_u, bos_f = bos0.clone(), bos0.clone()
    mlp = K.linear(h, w, fb, epilogue=_lib.EPI_BIAS_LS, gamma=g)
    if with_ln:
        x_u, ln_u = K.packed_residual_persist_ln(x_act, x_attn, mlp, bi, ti, bos_u, lw, lb, 1e-6)
    else:
        x_u, ln_u = K.packed_residual_persist(x_act, x_attn, mlp, bi, ti, bos_u), None
    out = K.linear_ls_packed_residual(h, w, fb, g, x_act, x_attn, bi, ti, bos_f, ln)
    assert out is not None
    x_f, ln_f = out
    assert_bits_equal(x_f, x_u.cpu(), "x_new")
    assert_bits_equal(bos_f, bos_u.cpu(), "blocks_out_sum")
    if with_ln:
        assert_bits_equal(ln_f, ln_u.cpu(), "LayerNorm(x_new)")
    else:
        assert ln_f is None
