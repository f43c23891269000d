"""GPU parity of the approximate pass's server scores (attention.py:241-273) against oracle/pscore.py.

  * the query-score kernel (cls_attn_prob, and the pseudo score) is bit-exact against the oracle on the
    same q and K cache, at the ViT-S / ViT-L / ViT-7B shapes, strided exactly as the approx pass
    hands them over (the cls row of the packed queries, the K half of the {tag}_kv cache);
  * the pseudo query is bit-exact;
  * the top-k plan built from those scores is bit-exact (ties -- frequent among bf16 scores -- go to
    the lower candidate index), so the default per-layer plan selects the oracle's tokens;
  * inside the approx block the cached {tag}_server_pscore equals the oracle applied to the block's own
    q and K, for cls_attn_prob (fp32), the pseudo score (bf16) and "random" (the reference computes the
    cls score for it and draws the random control at plan time, attention.py:266-271);
  * the attention's row log-sum-exp (what cuDNN's SDPA hands the reference's fused score) against the
    float64 row log-sum-exp, with the attention output unchanged, and the fused score computed from it
    against the oracle, alone and inside an approx block of 32 heads of 128.
"""

import numpy as np
import pytest
import torch

from appcorr_amd import kernels as K
from appcorr_amd.dinov3 import SelfAttentionBlock
from oracle import model as OM
from oracle import plan as OP
from oracle import pscore as PS
from tests.util import assert_bits_equal

pytestmark = pytest.mark.gpu

SHAPES = [(1, 6, 201, 64), (16, 16, 1029, 64), (2, 32, 4101, 128)]


def _qkv(B, H, N, D, seed, dev):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(B, N, H, D, generator=g) * 2.0).to(torch.bfloat16)
    kv = torch.randn(B, N, 2, H, D, generator=g).to(torch.bfloat16)
    return q, kv, q.to(dev), kv.to(dev)


@pytest.mark.parametrize("B,H,N,D", SHAPES)
def test_cls_attn_prob_bit_exact(dev, B, H, N, D):
    print(f"cls_attn_prob B={B} H={H} N={N} D={D}", flush=True)
    q, kv, qd, kvd = _qkv(B, H, N, D, N, dev)
    scale = D ** -0.5
    got = K.query_attention_prob(qd[:, 0], kvd, scale)
    torch.cuda.synchronize()
    ref = PS.query_attention_prob(q[:, 0].float().numpy(), kv[:, :, 0].float().numpy(), scale)
    assert got.dtype == torch.float32
    np.testing.assert_array_equal(got.cpu().numpy(), ref)
    got16 = K.query_attention_prob(qd[:, 0], kvd, scale, out_dtype=torch.bfloat16)
    assert_bits_equal(got16, torch.from_numpy(ref).to(torch.bfloat16), "bf16 output")


@pytest.mark.parametrize("B,H,N,D", SHAPES)
def test_pseudo_query_bit_exact(dev, B, H, N, D):
    print(f"pseudo_query B={B} H={H} N={N} D={D}", flush=True)
    q, kv, qd, kvd = _qkv(B, H, N, D, N + 1, dev)
    q = (q.float() + 0.25).to(torch.bfloat16)
    qd = q.to(dev)
    P = N - 5
    got = K.pseudo_query(qd[:, 5:])
    torch.cuda.synchronize()
    ref = PS.pseudo_query(np.ascontiguousarray(q[:, 5:].float().numpy().transpose(0, 2, 1, 3)))
    assert P > 0
    assert_bits_equal(got, torch.from_numpy(ref).to(torch.bfloat16), "pseudo query")
    # and the score from it
    s = K.query_attention_prob(got, kvd, D ** -0.5, out_dtype=torch.bfloat16)
    s_ref = PS.query_attention_prob(ref, kv[:, :, 0].float().numpy(), D ** -0.5)
    assert_bits_equal(s, torch.from_numpy(s_ref).to(torch.bfloat16), "pseudo score")


@pytest.mark.parametrize("ratio", [0.1, 0.25, 0.5])
def test_plan_from_cls_scores_bit_exact(dev, ratio):
    B, H, N, D = 16, 16, 1029, 64
    q, kv, qd, kvd = _qkv(B, H, N, D, 77, dev)
    s = K.query_attention_prob(qd[:, 0], kvd, D ** -0.5)
    P = N - 5
    k = OP.keep_count(P, ratio)
    dind = torch.arange(N, device=dev).unsqueeze(0).expand(B, -1).contiguous()
    scores = s[:, 5:].contiguous()   # server.gather(1, dindice_patches) with dindice = arange
    tp = K.topk_plan(scores, k, dind, 5, N)
    torch.cuda.synchronize()
    sc = scores.cpu().numpy()
    assert len(np.unique(sc[0])) < P // 2, "bf16-valued scores should carry many ties"
    ref = OP.build_plan(sc, k, dind.cpu().numpy(), 5, N)
    assert_bits_equal(tp.update_indice, ref.update_indice, "update_indice")
    assert_bits_equal(tp.keep_mask, ref.keep_mask, "keep_mask")


def _block(cfg, w, dev):
    blk = SelfAttentionBlock(cfg.dim, cfg.heads, ffn_ratio=cfg.ffn_hidden / cfg.dim, qkv_bias=cfg.qkv_bias,
                             init_values=1.0, mask_k_bias=True)
    blk.load_state_dict(w)
    return blk.to(device=dev, dtype=torch.bfloat16)


@pytest.mark.parametrize("kind", ["cls_attn_prob", "patch_pseudo_attn_prob", "random", "cls_attn_prob_layermean"])
def test_approx_block_caches_the_reference_score(dev, kind):
    cfg = OM.CONFIGS["vitb16_512"]
    B = 2
    w = OM.make_block_weights(cfg, 0, gamma=1.0, bias_std=0.05, ln_std=0.1, depth=1)[0]
    x_base, _, _, _ = OM.make_inputs(cfg, B, 1)
    rope = OM.rope_tables(cfg)
    r = (rope[0].to(dev), rope[1].to(dev))
    blk = _block(cfg, w, dev)
    x = x_base.to(dev)
    with torch.no_grad():
        _, cache = blk.approx(x, r, {}, "layer0", server_pscore=kind, server_pscore_weight=1.0)
        # the block's own queries, recomputed by the same (deterministic) kernels
        N, C = cfg.num_tokens, cfg.dim
        xn = K.layer_norm(x.reshape(B * N, C), blk.norm1.weight, blk.norm1.bias, blk.norm1.eps)
        kv2 = torch.empty_like(cache["layer0_kv"])
        from appcorr_amd.dinov3.layers import PackedQueryState
        tok = torch.arange(N, device=dev)
        qs = PackedQueryState(torch.arange(B, device=dev).repeat_interleave(N), tok.repeat(B), tok.repeat(B),
                              None, None, None, True, (tok >= 5).repeat(B), (tok - 5).clamp_min(0).repeat(B))
        q, _ = blk.attn._qkv_attention(xn, r, kv2, qs)
    torch.cuda.synchronize()
    assert_bits_equal(kv2, cache["layer0_kv"], "recomputed K/V")
    got = cache["layer0_server_pscore"]
    qn = q.view(B, N, cfg.heads, cfg.head_dim).cpu()
    ref = OM.server_score(kind, qn, cache["layer0_kv"][:, :, 0].cpu(), cfg.num_patches, cfg.head_dim ** -0.5)
    assert got.dtype == ref.dtype, (got.dtype, ref.dtype)
    assert_bits_equal(got, ref, f"{kind} score")


def test_per_layer_plan_uses_the_cached_score(dev):
    """Default kwargs (server_pscore cls_attn_prob, weight 1): the correction's plan is the top-k of the
    cached score of that layer, bit for bit."""
    cfg = OM.CONFIGS["vitb16_512"]
    B, ratio = 2, 0.25
    w = OM.make_block_weights(cfg, 0, gamma=1.0, bias_std=0.05, ln_std=0.1, depth=1)[0]
    x_base, x_full, _, _ = OM.make_inputs(cfg, B, 1)
    rope = OM.rope_tables(cfg)
    r = (rope[0].to(dev), rope[1].to(dev))
    blk = _block(cfg, w, dev)
    dind = OM.full_dindice(cfg, B).to(dev)
    with torch.no_grad():
        _, cache = blk.approx(x_base.to(dev), r, {}, "layer0")
        _, cache = blk.correct(x_full.to(dev), dind, r, cache, "layer0", token_keep_ratio=ratio, debug=True)
    torch.cuda.synchronize()
    score = cache["layer0_server_pscore"].cpu().numpy()
    k = OP.keep_count(cfg.num_patches, ratio)
    ref = OP.build_plan(score[:, 5:], k, dind.cpu().numpy(), 5, cfg.num_tokens)
    assert_bits_equal(cache["layer0_update_indice"], ref.update_indice, "update_indice")


def _bf16_ulps(got: torch.Tensor, ref: torch.Tensor) -> np.ndarray:
    g = got.float().cpu().numpy().astype(np.float64)
    r = ref.float().cpu().numpy().astype(np.float64)
    e = np.floor(np.log2(np.maximum(np.abs(r), 2.0 ** -126)))
    return np.abs(g - r) / 2.0 ** (e - 7)


@pytest.mark.parametrize("B,H,N,D,mode", [(1, 6, 201, 64, K.PATTN_DENSE), (2, 16, 1029, 64, K.PATTN_DENSE),
                                          (1, 32, 301, 128, K.PATTN_DENSE), (1, 32, 1029, 128, K.PATTN_LSE),
                                          (2, 4, 77, 64, K.PATTN_LSE)])
def test_patch_attention_prob_vs_oracle(dev, B, H, N, D, mode):
    """The dense score (and the fused key-side score) against the exact evaluation: the kernel's fp32
    MFMA accumulation, fp32 exponential and fp32 sums over heads and queries move a value by at most one
    bf16 step, and only where it sits next to a rounding boundary."""
    print(f"patch_attention_prob B={B} H={H} N={N} D={D} mode={mode}", flush=True)
    q, kv, qd, kvd = _qkv(B, H, N, D, 11 + N, dev)
    got = K.patch_attention_prob(qd.reshape(B * N, H, D), kvd, D ** -0.5, mode)
    qh = np.ascontiguousarray(q.float().numpy().transpose(0, 2, 1, 3))
    kn = kv[:, :, 0].float().numpy()
    fn = PS.patch_attn_prob if mode == K.PATTN_DENSE else PS.patch_attn_prob_fused
    ref = torch.from_numpy(fn(qh, kn, D ** -0.5)).to(torch.bfloat16)
    u = _bf16_ulps(got, ref)
    print(f"  ulps: max {u.max():.3g}, differing {float((u > 0).mean()):.4%}", flush=True)
    assert u.max() <= 1.0 and float((u > 0).mean()) <= 0.02


def test_patch_attention_prob_vit7b_mass(dev):
    """ViT-7B at 1024 px (N = 4101 > 4096: the dense path even for the layer-mean kind): every query's
    probabilities sum to one, so the key scores of an image sum to one up to the bf16 roundings."""
    B, H, N, D = 1, 32, 4101, 128
    q, kv, qd, kvd = _qkv(B, H, N, D, 3, dev)
    got = K.patch_attention_prob(qd.reshape(B * N, H, D), kvd, D ** -0.5, K.PATTN_DENSE).float()
    assert bool((got >= 0).all())
    tot = float(got.sum())
    assert abs(tot - 1.0) < 2e-2, tot


@pytest.mark.parametrize("kind", ["patch_attn_prob", "patch_attn_prob_layermean"])
def test_approx_block_caches_the_dense_score(dev, kind):
    cfg = OM.CONFIGS["vits16_224"]
    B = 2
    w = OM.make_block_weights(cfg, 0, gamma=1.0, bias_std=0.05, ln_std=0.1, depth=1)[0]
    x_base, _, _, _ = OM.make_inputs(cfg, B, 1)
    rope = OM.rope_tables(cfg)
    r = (rope[0].to(dev), rope[1].to(dev))
    blk = _block(cfg, w, dev)
    x = x_base.to(dev)
    with torch.no_grad():
        _, cache = blk.approx(x, r, {}, "layer0", server_pscore=kind, server_pscore_weight=1.0)
        N, C = cfg.num_tokens, cfg.dim
        xn = K.layer_norm(x.reshape(B * N, C), blk.norm1.weight, blk.norm1.bias, blk.norm1.eps)
        kv2 = torch.empty_like(cache["layer0_kv"])
        from appcorr_amd.dinov3.layers import PackedQueryState
        tok = torch.arange(N, device=dev)
        qs = PackedQueryState(torch.arange(B, device=dev).repeat_interleave(N), tok.repeat(B), tok.repeat(B),
                              None, None, None, True, (tok >= 5).repeat(B), (tok - 5).clamp_min(0).repeat(B))
        q, _ = blk.attn._qkv_attention(xn, r, kv2, qs)
    torch.cuda.synchronize()
    got = cache["layer0_server_pscore"]
    qn = q.view(B, N, cfg.heads, cfg.head_dim).cpu()
    ref = OM.server_score(kind, qn, cache["layer0_kv"][:, :, 0].cpu(), cfg.num_patches, cfg.head_dim ** -0.5)
    assert got.dtype == ref.dtype == torch.bfloat16
    u = _bf16_ulps(got, ref)
    assert u.max() <= 1.0 and float((u > 0).mean()) <= 0.02, (u.max(), float((u > 0).mean()))


@pytest.mark.parametrize("B,H,N,D", [(1, 32, 1029, 128), (2, 4, 77, 64), (1, 8, 300, 64)])
def test_attention_row_lse_and_fused_score(dev, B, H, N, D):
    """sparse_query_attention(..., lse=) over all N queries of an image: the output equals the call
    without lse (bit for bit at Dh = 128, where both run the register-staged kernel), lse is the float64
    row log-sum-exp of the same bf16 q and K within 2e-4 (fp32 score accumulation, fp32 exponentials and
    an fp32 sum of up to N probabilities; a wrong log base or a dropped max is off by > 0.1), and the
    key-side score computed from it is within the fused score's bound of the oracle."""
    print(f"attention lse B={B} H={H} N={N} D={D}", flush=True)
    q, kv, qd, kvd = _qkv(B, H, N, D, 5 + N, dev)
    qp = qd.reshape(B * N, H, D)
    scale = D ** -0.5
    lse = torch.full((B, H, N), float("nan"), device=dev)
    out = K.sparse_query_attention(qp, kvd, N, scale, lse=lse)
    if D == 128:
        assert_bits_equal(out, K.sparse_query_attention(qp, kvd, N, scale).cpu(), "attention output with lse")
    qh = np.ascontiguousarray(q.float().numpy().transpose(0, 2, 1, 3))
    kn = kv[:, :, 0].float().numpy()
    ref = PS.row_logsumexp(qh, kn, scale)
    err = np.abs(lse.cpu().numpy().astype(np.float64) - ref)
    print(f"  lse max err {err.max():.3g}", flush=True)
    assert np.isfinite(err).all() and err.max() <= 2e-4
    got = K.patch_attention_prob_from_lse(qp, kvd, scale, lse)
    want = torch.from_numpy(PS.patch_attn_prob_fused(qh, kn, scale)).to(torch.bfloat16)
    u = _bf16_ulps(got, want)
    print(f"  score ulps: max {u.max():.3g}, differing {float((u > 0).mean()):.4%}", flush=True)
    assert u.max() <= 1.0 and float((u > 0).mean()) <= 0.02


def test_approx_block_fused_score_from_the_attention_lse(dev):
    """An approx block of 32 heads of 128 (the ViT-7B width at 224 px, N = 201) caching
    patch_attn_prob_layermean: the fused score now comes from the attention's own log-sum-exp and
    still equals the oracle's fused score of the block's q and K within its bound."""
    cfg = OM.with_overrides(OM.CONFIGS["vit7b16_1024"], img_size=224, name="vit7b16_224")
    B = 1
    w = OM.make_block_weights(cfg, 0, gamma=1.0, bias_std=0.05, ln_std=0.1, depth=1)[0]
    x_base, _, _, _ = OM.make_inputs(cfg, B, 1)
    rope = OM.rope_tables(cfg)
    r = (rope[0].to(dev), rope[1].to(dev))
    blk = SelfAttentionBlock(cfg.dim, cfg.heads, ffn_ratio=3.0, qkv_bias=cfg.qkv_bias, init_values=1.0,
                             ffn_layer="swiglu64", mask_k_bias=True)
    blk.load_state_dict(w)
    blk = blk.to(device=dev, dtype=torch.bfloat16)
    x = x_base.to(dev)
    kind = "patch_attn_prob_layermean"
    assert blk._fused_patch_score(kind, cfg.heads, cfg.head_dim, cfg.num_tokens)
    with torch.no_grad():
        _, cache = blk.approx(x, r, {}, "layer0", server_pscore=kind, server_pscore_weight=1.0)
        N, C = cfg.num_tokens, cfg.dim
        xn = K.layer_norm(x.reshape(B * N, C), blk.norm1.weight, blk.norm1.bias, blk.norm1.eps)
        kv2 = torch.empty_like(cache["layer0_kv"])
        from appcorr_amd.dinov3.layers import PackedQueryState
        tok = torch.arange(N, device=dev)
        qs = PackedQueryState(torch.arange(B, device=dev).repeat_interleave(N), tok.repeat(B), tok.repeat(B),
                              None, None, None, True, (tok >= 5).repeat(B), (tok - 5).clamp_min(0).repeat(B))
        q, _ = blk.attn._qkv_attention(xn, r, kv2, qs)
        # the score the stats-based LSE mode gives on the same q and K (no attention log-sum-exp)
        stats_score = K.patch_attention_prob(q.view(B * N, cfg.heads, cfg.head_dim), cache["layer0_kv"],
                                             cfg.head_dim ** -0.5, K.PATTN_LSE)
    torch.cuda.synchronize()
    assert_bits_equal(kv2, cache["layer0_kv"], "recomputed K/V")
    got = cache["layer0_server_pscore"]
    qn = q.view(B, N, cfg.heads, cfg.head_dim).cpu()
    ref = OM.server_score(kind, qn, cache["layer0_kv"][:, :, 0].cpu(), cfg.num_patches, cfg.head_dim ** -0.5)
    assert got.dtype == ref.dtype == torch.bfloat16
    u = _bf16_ulps(got, ref)
    print(f"block score ulps: max {u.max():.3g}, differing {float((u > 0).mean()):.4%}", flush=True)
    assert u.max() <= 1.0 and float((u > 0).mean()) <= 0.02
    v = _bf16_ulps(got, stats_score)
    assert v.max() <= 1.0 and float((v > 0).mean()) <= 0.02
