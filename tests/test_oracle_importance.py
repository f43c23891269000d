"""Pins of the pixel-residual importance oracle (oracle/importance.py), on the CPU.

  * patch_residual_score against the reference's own op sequences, evaluated by torch and numpy: the
    server's view / permute / square / mean / sqrt (dinov3_classifier.py:112-122) and the mobile crop
    scores (progressive.py:14-22) -- within the few ulp their fp32 reductions may differ by;
  * closed forms: a constant residual c gives RMS |c|, ENERGY n c^2, L2 sqrt(n) |c|;
  * residual_prune: hand-derived plans (threshold, the top-min_keep rescue, ties, the
    "some image keeps everything -> nothing pruned" rule of :166-174) and mass totals.
"""

import numpy as np
import pytest
import torch

from oracle import importance as OI


def _ulps(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    return np.abs(a.astype(np.float64) - b.astype(np.float64)) / np.spacing(np.maximum(np.abs(a), np.abs(b)))


@pytest.mark.parametrize("dtype", [np.uint8, np.float32])
def test_rms_matches_reference_torch_sequence(dtype):
    rng = np.random.default_rng(1)
    B, H, W, C, ph, pw = 3, 64, 48, 3, 16, 16
    if dtype == np.uint8:
        curr, prev = (rng.integers(0, 256, (B, H, W, C), dtype=np.uint8) for _ in range(2))
    else:
        curr, prev = (rng.standard_normal((B, H, W, C)).astype(np.float32) for _ in range(2))
    got = OI.patch_residual_score(curr, prev, ph, pw, OI.RMS, image_idx=np.array([2, 0]))
    c = torch.from_numpy(curr).float()[[2, 0]]
    p = torch.from_numpy(prev).float()[[2, 0]]
    res = (c - p).view(2, H // ph, ph, W // pw, pw, C).permute(0, 1, 3, 2, 4, 5).contiguous()
    ref = torch.sqrt(res.square().mean(dim=(3, 4, 5)).view(2, -1)).numpy()
    assert _ulps(got, ref).max() <= 2


@pytest.mark.parametrize("mode", [OI.RMS, OI.ENERGY])
def test_crop_scores_match_mobile_numpy(mode):
    rng = np.random.default_rng(2)
    resid = rng.integers(-300, 300, (1, 32, 32, 3)).astype(np.int16)
    got = OI.patch_residual_score(resid, None, 16, 16, mode)[0]
    want = []
    for i in range(4):
        y, x = divmod(i, 2)
        crop = resid[0, 16 * y:16 * y + 16, 16 * x:16 * x + 16].astype(np.float32, copy=False)
        sq = np.square(crop, dtype=np.float32)
        want.append(np.sqrt(sq.mean(dtype=np.float32)) if mode == OI.RMS else sq.sum(dtype=np.float32))
    assert _ulps(got, np.array(want, np.float32)).max() <= 4


def test_closed_forms():
    c = np.full((1, 16, 32, 3), 7, np.int16)
    n = 16 * 16 * 3
    np.testing.assert_array_equal(OI.patch_residual_score(c, None, 16, 16, OI.RMS), [[7.0, 7.0]])
    np.testing.assert_array_equal(OI.patch_residual_score(c, None, 16, 16, OI.ENERGY), [[49.0 * n] * 2])
    np.testing.assert_array_equal(OI.patch_residual_score(c, None, 16, 16, OI.L2),
                                  np.float32(np.sqrt(np.float32(49.0 * n))) * np.ones((1, 2), np.float32))
    z = np.zeros((2, 16, 16, 3), np.uint8)
    np.testing.assert_array_equal(OI.patch_residual_score(z, z, 16, 16), [[0.0], [0.0]])


def test_prune_hand_derived():
    # 2 pretokens; 6 candidate patches per image; G = 8 patches in the residual map
    rms = np.array([[0.1, 0.9, 0.2, 0.8, 0.5, 0.5, 0.0, 0.3],
                    [0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0]], np.float32)
    spatial = np.array([[1, 2, 3, 4, 5, 7], [0, 2, 4, 6, 1, 3]])
    dind = np.concatenate([np.tile([0, 1], (2, 1)), spatial + 2], axis=1)
    p = OI.residual_prune(dind, spatial, rms, threshold=0.5, min_keep=1)
    # image 0: r = [.9, .2, .8, .5, .5, .3] -> keeps candidates 0, 2, 3, 4 (spatial 1, 3, 4, 5)
    # image 1: all zero -> threshold keeps none; min_keep=1 rescues the first of the tie (candidate 0)
    np.testing.assert_array_equal(p.kept_patch_count, [4, 1])
    np.testing.assert_array_equal(p.pruned_dindice, [[0, 1, 3, 5, 6, 7], [0, 1, 2, 2, 2, 2]])
    np.testing.assert_array_equal(p.kept_local_idx, [[0, 2, 3, 4], [0, 0, 0, 0]])
    np.testing.assert_allclose(p.full_residual_mass, [3.2, 0.0], rtol=1e-6)
    np.testing.assert_allclose(p.kept_residual_mass, [2.7, 0.0], rtol=1e-6)
    # min_keep rescues the largest below the threshold
    p2 = OI.residual_prune(dind, spatial, rms, threshold=0.95, min_keep=2)
    np.testing.assert_array_equal(p2.pruned_dindice[0], [0, 1, 3, 5])
    # an image keeping every candidate: nothing is pruned for any image
    p3 = OI.residual_prune(dind, spatial, rms, threshold=0.0, min_keep=1)
    np.testing.assert_array_equal(p3.pruned_dindice, dind)
    np.testing.assert_array_equal(p3.kept_local_idx, np.tile(np.arange(6), (2, 1)))
    np.testing.assert_array_equal(p3.kept_patch_count, [6, 6])
    # no residual map: unpruned
    p4 = OI.residual_prune(dind, spatial, None, 0.5, 1)
    np.testing.assert_array_equal(p4.pruned_dindice, dind)
