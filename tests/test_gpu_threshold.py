"""GPU parity of threshold token selection (token_keep_thres, with and without token_keep_cap).

  1. the plan kernels against oracle.plan.threshold_plan, bit for bit: kept mask and counts,
     update_indice, query_valid, every packed-row array and row_slot, for both builders, with NaN,
     -inf (padded candidates), signed zeros, images keeping nothing or everything, the largest P, a
     threshold that rounds to fp32, candidate subsets;
  2. one block with identical inputs against the fp64 oracle run on the reference's form of the plan
     (the padded builder's compacted rows scattered into a padded query buffer): unselected rows
     bit-exact, selected rows within the propagated bound -- which shows that the repeated packed
     rows of this build compute and write exactly what the reference's rows do;
  3. two blocks run packed equal two blocks run one by one, bit for bit, with repeated rows.
"""

import numpy as np
import pytest
import torch

from appcorr_amd import kernels as K
from appcorr_amd.dinov3.layers import correct_blocks_packed
from oracle import model as OM
from oracle import plan as OP
from tests.test_gpu_block import KW, _gpu_blocks, _gpu_cache, _setup
from tests.util import assert_bits_equal, assert_propagated_close, bf16_ulp

pytestmark = pytest.mark.gpu


def _scores(B, P, seed, special=True):
    g = np.random.default_rng(seed)
    s = g.standard_normal((B, P)).astype(np.float32)
    if special and P >= 8:
        s[0, 1::7] = np.nan
        s[0, 2::11] = -np.inf
        s[-1, 3::5] = -0.0
        s[-1, 4::5] = 0.0
    if B >= 3:
        s[1] = -10.0          # keeps nothing
        s[2] = 10.0           # keeps everything
    return s


def _dind(B, P, pre, N, seed):
    g = np.random.default_rng(seed + 100)
    rows = [np.concatenate([np.arange(pre), pre + g.permutation(N - pre)[:P]]) for _ in range(B)]
    return np.stack(rows).astype(np.int64)


CASES = [  # B, P, pre, N, thres, cap
    (16, 1024, 5, 1029, 0.67, 0),
    (16, 1024, 5, 1029, 0.67, 256),
    (16, 1024, 5, 1029, 0.0, 0),
    (16, 1024, 5, 1029, -0.0, 100),
    (4, 4096, 5, 4101, 1.2815, 0),
    (4, 4096, 5, 4101, 1.2815, 409),
    (3, 196, 5, 201, 0.1, 0),
    (3, 196, 5, 201, 1.0000000001, 7),
    (2, 16384, 5, 16389, 2.0, 0),
    (5, 1000, 5, 1100, 0.3, 1000),
    (2, 37, 0, 50, -0.5, 40),
    (3, 37, 0, 50, float("-inf"), 0),
    (2, 0, 5, 5, 0.0, 3),
]


@pytest.mark.parametrize("B,P,pre,N,thres,cap", CASES)
def test_threshold_plan_bit_exact(dev, B, P, pre, N, thres, cap):
    print(f"threshold plan B={B} P={P} pre={pre} thres={thres} cap={cap}", flush=True)
    s = _scores(B, P, B * 31 + P)
    d = _dind(B, P, pre, N, P)
    ref = OP.threshold_plan(s, thres, d, pre, N, keep_cap=cap)
    st, dt = torch.from_numpy(s).to(dev), torch.from_numpy(d).to(dev)
    keep, cnt = K.threshold_keep(st, thres)
    assert_bits_equal(keep, ref.keep_mask, "threshold_keep mask")
    assert_bits_equal(cnt.long(), ref.kept_count, "threshold_keep count")
    padded = cap == 0
    width = int(ref.kept_count.max()) if padded else min(cap, P)
    if padded and pre == 0 and width > 0 and int(ref.kept_count.min()) == 0:
        pytest.skip("padded plan with no pretokens and an empty image is rejected by the block")
    tp = K.threshold_plan(st, thres, dt, pre, width, padded=padded, num_tokens=N)
    assert_bits_equal(tp.update_indice, ref.update_indice, "update_indice")
    assert_bits_equal(tp.query_valid, ref.query_valid_mask, "query_valid")
    assert_bits_equal(tp.keep_mask, ref.keep_mask, "keep_mask")
    assert_bits_equal(tp.kept_count.long(), ref.kept_count, "kept_count")
    rows = ref.rows
    for f in ("active_batch_idx", "active_pos_idx", "active_token_idx", "active_patch_mask", "active_rope_idx",
              "row_slot"):
        assert_bits_equal(getattr(tp, f), getattr(rows, f), f)
    # the reference's compacted rows are the packed rows at query_valid
    v = tp.query_valid.reshape(-1)
    assert_bits_equal(tp.active_token_idx[v], ref.active_token_idx, "compacted active_token_idx")
    assert_bits_equal(tp.active_pos_idx[v], ref.active_pos_idx, "compacted active_pos_idx")


def _thres_kw(thres, cap):
    kw = dict(KW)
    kw.update(token_keep_thres=thres, token_keep_cap=cap)
    return kw


@pytest.mark.parametrize("cap", [0, 200, 64])
def test_single_block_threshold_identical_inputs(dev, cap):
    """ViT-B, B=3, one block; the threshold keeps a different number of patches per image (image 1
    keeps none), so the padded builder pads two images and cap=64 truncates."""
    print(f"vitb block threshold cap={cap}", flush=True)
    cfg = OM.CONFIGS["vitb16_512"]
    B = 3
    weights, x_base, x_full, imp, rope = _setup(cfg, B, 1, dev, gamma=1.0, bias_std=0.05, ln_std=0.1)
    imp = imp.clone()
    thres = float(np.quantile(imp[2].numpy(), 0.8))
    imp[0] = imp[0] * (thres / float(np.quantile(imp[0].numpy(), 0.93)))
    imp[1] = -1.0
    _, cache = OM.approx_pass(cfg, weights, x_base, rope)
    dind = OM.full_dindice(cfg, B)
    plan = OP.threshold_plan(imp.numpy(), thres, dind.numpy(), cfg.num_pretokens, cfg.num_tokens, keep_cap=cap)
    counts = plan.kept_count.tolist()
    assert len(set(counts)) == 3, counts
    x_ref, cache_ref = OM.correct_block(cfg, weights[0], x_full, plan, rope,
                                        {k_: v.clone() for k_, v in cache.items()}, "layer0")
    blk = _gpu_blocks(cfg, weights, dev)[0]
    gcache = _gpu_cache(cache, dev)
    with torch.no_grad():
        x_got, gcache = blk.correct(x_full.to(dev), dind.to(dev), (rope[0].to(dev), rope[1].to(dev)), gcache,
                                    "layer0", mobile_pscore_hint=imp.to(dev), **_thres_kw(thres, cap))
    gplan = next(iter(gcache["_partial_token_query_plan_cache"].values()))
    assert_bits_equal(gplan.update_indice, plan.update_indice, "update_indice")
    assert_bits_equal(gplan.fixed_query_state.query_valid_mask, plan.query_valid_mask, "query_valid_mask")
    assert gplan.fixed_query_state.all_valid == plan.all_valid
    sel = np.zeros((B, cfg.num_tokens), dtype=bool)
    sel[plan.active_batch_idx, plan.active_token_idx] = True
    st = torch.from_numpy(sel)
    assert_bits_equal(x_got.cpu()[~st], x_ref[~st], "unselected rows")
    assert_bits_equal(gcache["layer0_kv"].cpu()[~st], cache["layer0_kv"][~st], "unselected K/V rows")
    assert_propagated_close(x_got, x_ref, what="x_out")
    assert_propagated_close(gcache["layer0_kv"], cache_ref["layer0_kv"], max_ulps=2, mean_rel=2.0 ** -12,
                            what="kv cache")
    bos_ref = cache_ref["layer0_blocks_out_sum"]
    summand = (x_ref.float().abs() + bos_ref.float().abs()).numpy()
    assert_propagated_close(gcache["layer0_blocks_out_sum"], bos_ref, floor_abs=4 * bf16_ulp(summand),
                            what="blocks_out_sum")


@pytest.mark.parametrize("cap", [0, 300])
def test_packed_run_equals_blockwise_threshold(dev, cap):
    """ViT-L width, B=4, 3 blocks, threshold keeping ~25 % with per-image counts that differ: the packed
    run (repeated rows carried through the blocks) equals block-by-block correction bit for bit."""
    print(f"vitl packed threshold cap={cap}", flush=True)
    cfg = OM.CONFIGS["vitl16_512"]
    B = 4
    weights = OM.make_block_weights(cfg, 0, gamma=1.0, bias_std=0.05, ln_std=0.1, depth=3)
    blocks = _gpu_blocks(cfg, weights, dev)
    g = torch.Generator().manual_seed(9)
    N, C, H, D, P = cfg.num_tokens, cfg.dim, cfg.heads, cfg.head_dim, cfg.num_patches
    x = torch.randn(B, N, C, generator=g).to(torch.bfloat16)
    cache = {}
    for i in range(3):
        cache[f"layer{i}_kv"] = torch.randn(B, N, 2, H, D, generator=g).to(torch.bfloat16)
        cache[f"layer{i}_blocks_out_sum"] = (torch.randn(B, N, C, generator=g) * 0.1).to(torch.bfloat16)
    imp = torch.rand(B, P, generator=g) * torch.tensor([1.0, 0.9, 0.8, 1.1])[:, None]
    rope = OM.rope_tables(cfg)
    r = (rope[0].to(dev), rope[1].to(dev))
    dd = OM.full_dindice(cfg, B).to(dev)
    kw = dict(mobile_pscore_hint=imp.to(dev), **_thres_kw(0.75, cap))
    ca, cb = _gpu_cache(cache, dev), _gpu_cache(cache, dev)
    tags = [f"layer{i}" for i in range(3)]
    with torch.no_grad():
        xa, ca = correct_blocks_packed(blocks, x.to(dev), dd, r, ca, tags, **kw)
        xb = x.to(dev)
        for i, blk in enumerate(blocks):
            xb, cb = blk.correct(xb, dd, r, cb, tags[i], **kw)
    plan = next(iter(ca["_partial_token_query_plan_cache"].values()))
    qs = plan.fixed_query_state
    if cap == 0:
        assert not bool(qs.query_valid_mask.all())       # padded rows present
    else:
        assert int(torch.unique(qs.active_token_idx.view(B, -1)[0]).numel()) < qs.active_token_idx.numel() // B
    assert_bits_equal(xa, xb.cpu(), "packed x_out")
    for t in tags:
        for key in (f"{t}_kv", f"{t}_blocks_out_sum"):
            assert_bits_equal(ca[key], cb[key].cpu(), f"packed {key}")
