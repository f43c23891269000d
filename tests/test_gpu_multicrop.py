"""Batched multi-crop correction (appcorr_amd/server/multicrop.py) on the GPU.

Two crops of one request carry different candidate lists (600 and 424 patch tokens) and their own
caches. Batched, their candidate lists are padded to 600 with invalid slots, their caches are
concatenated, the blocks run once over both, and the caches are split back. Checks, per crop:
  * the kept set equals the crop's own threshold selection (oracle.plan.threshold_plan), bit for bit
    -- padded slots are never selected;
  * x_out and the returned caches match the fp64 oracle run on that crop alone within the propagated
    bound, and the rows the plan does not touch are bit-exact (x + blocks_out_sum; K/V unchanged);
  * the batch's plan statistics reach the first crop's cache.
"""

import numpy as np
import pytest
import torch

from appcorr_amd.server.multicrop import CropItem, correct_crops_batched, union_dindices
from oracle import model as OM
from oracle import plan as OP
from tests.test_gpu_block import KW, _gpu_blocks
from tests.util import assert_bits_equal, assert_propagated_close

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("cap", [0, 150])
def test_two_crops_batched_equal_each_crop_alone(dev, cap):
    print(f"multicrop vitb two crops cap={cap}", flush=True)
    cfg = OM.CONFIGS["vitb16_512"]
    N, C, H, D, P, pre = cfg.num_tokens, cfg.dim, cfg.heads, cfg.head_dim, cfg.num_patches, cfg.num_pretokens
    L = 2
    weights = OM.make_block_weights(cfg, 0, gamma=1.0, bias_std=0.05, ln_std=0.1, depth=L)
    blocks = _gpu_blocks(cfg, weights, dev)
    rope = OM.rope_tables(cfg)
    rg = (rope[0].to(dev), rope[1].to(dev))
    g = torch.Generator().manual_seed(21)
    rng = np.random.default_rng(21)
    crops = []
    for n_cand in (600, 424):
        cand = np.sort(rng.permutation(P)[:n_cand]) + pre
        dind = torch.from_numpy(np.concatenate([np.arange(pre), cand])[None].astype(np.int64))
        x = torch.randn(1, N, C, generator=g).to(torch.bfloat16)
        cache = {}
        for l in range(L):
            cache[f"layer{l}_kv"] = torch.randn(1, N, 2, H, D, generator=g).to(torch.bfloat16)
            cache[f"layer{l}_blocks_out_sum"] = (torch.randn(1, N, C, generator=g) * 0.1).to(torch.bfloat16)
        hint = torch.rand(1, P, generator=g)
        crops.append((dind, x, cache, hint))
    thres = 0.8
    kw = dict(KW)
    kw.update(token_keep_thres=thres, token_keep_cap=cap)

    items = [CropItem(input_tokens=x.to(dev), dindice=d.to(dev), num_pre=pre,
                      cache={k: v.to(dev).clone() for k, v in c.items()}, rope=rg, mobile_pscore_hint=h.to(dev))
             for d, x, c, h in crops]

    def run_block(l, x, d, r, cache, tag, source_key=None, **k):
        return blocks[l].correct(x, d, r, cache, tag, **k)

    with torch.no_grad():
        outs = correct_crops_batched(run_block, items, 0, L, **kw)
    assert items[1].dindice.shape[1] == pre + 600 and not bool(items[1].cand_valid.all())
    assert "_partial_token_kept_patch_total" in items[0].cache

    for (dind, x, cache, hint), it, out in zip(crops, items, outs):
        d = dind.numpy()
        scores = hint.numpy()[:, d[0, pre:] - pre]
        plan = OP.threshold_plan(scores, thres, d, pre, N, keep_cap=cap)
        x_ref, c_ref = OM.correct_pass(cfg, weights, x, plan, rope, {k: v.clone() for k, v in cache.items()})
        sel = np.zeros((1, N), dtype=bool)
        sel[plan.active_batch_idx, plan.active_token_idx] = True
        st = torch.from_numpy(sel)
        # x + bos_0 + bos_1 on the rows no block touches
        ref_un = x
        for l in range(L):
            ref_un = (ref_un.float() + cache[f"layer{l}_blocks_out_sum"].float()).to(torch.bfloat16)
        assert_bits_equal(out.cpu()[~st], ref_un[~st], "untouched rows")
        for l in range(L):
            assert_bits_equal(it.cache[f"layer{l}_kv"].cpu()[~st], cache[f"layer{l}_kv"][~st], "untouched K/V")
            assert_propagated_close(it.cache[f"layer{l}_kv"], c_ref[f"layer{l}_kv"], what=f"layer{l} K/V")
        assert_propagated_close(out, x_ref, what="x_out")


def test_union_dindices():
    a = torch.tensor([[0, 5, 9], [1, 2, 3]])
    b = torch.tensor([[5, 7, 0], [3, 4, 1]])
    assert union_dindices([a, b]).tolist() == [[0, 5, 7, 9], [1, 2, 3, 4]]
