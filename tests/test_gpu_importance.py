"""GPU parity of the importance producer (next-rank row f4) against oracle/importance.py.

  * patch_residual_score, bit for bit: uint8 frames of the BASELINE image sizes with an active-image
    subset (dinov3_classifier.py:91-122), int16 Laplacian residual crops scored as RMS / energy / L2
    (progressive.py:14-22), fp32 frames with values on a 2^-8 grid (exact float64 sums), an image
    index outside the batch (NaN row);
  * image-residual pruning (dinov3_classifier.py:124-197): kept mask, counts, masses (exact on a
    2^-10 grid), the compacted pruned dindice and local indices, the min_keep rescue, ties, NaN;
  * the executor: preprocess builds the hint map of the finest transmitted level, row-normalised, and
    per-group plans pruned by the residual RMS of input_hr_np against prev_input_hr_np, equal to the
    oracle's plan on the same frames.
"""

import numpy as np
import pytest
import torch

from appcorr_amd import _lib
from appcorr_amd import kernels as K
from appcorr_amd.server.dinov3_classifier import DINOv3ClassifierExecutor
from appcorr_amd.server.protocol import ExperimentConfig, Patch, Task
from oracle import importance as OI
from tests.util import assert_bits_equal

pytestmark = pytest.mark.gpu

MODES = {OI.RMS: _lib.IMPORTANCE_RMS, OI.ENERGY: _lib.IMPORTANCE_ENERGY, OI.L2: _lib.IMPORTANCE_L2}


@pytest.mark.parametrize("B,H,W,idx", [(16, 512, 512, None), (4, 512, 512, [3, 1]), (1, 1024, 1024, None),
                                       (3, 224, 224, [2, 2, 0])])
def test_residual_rms_uint8_frames(dev, B, H, W, idx):
    print(f"residual rms u8 B={B} {H}x{W} idx={idx}", flush=True)
    rng = np.random.default_rng(B + H)
    curr = rng.integers(0, 256, (B, H, W, 3), dtype=np.uint8)
    prev = rng.integers(0, 256, (B, H, W, 3), dtype=np.uint8)
    prev[0, :32] = curr[0, :32]        # some zero-residual patches
    ii = None if idx is None else np.array(idx)
    want = OI.patch_residual_score(curr, prev, 16, 16, OI.RMS, image_idx=ii)
    got = K.patch_residual_score(torch.from_numpy(curr).to(dev), torch.from_numpy(prev).to(dev), (16, 16),
                                 _lib.IMPORTANCE_RMS, None if ii is None else torch.from_numpy(ii).to(dev))
    assert_bits_equal(got, want, "rms")


@pytest.mark.parametrize("mode", [OI.RMS, OI.ENERGY, OI.L2])
def test_residual_crop_scores_int16(dev, mode):
    rng = np.random.default_rng(mode)
    resid = rng.integers(-510, 511, (2, 256, 192, 3)).astype(np.int16)
    want = OI.patch_residual_score(resid, None, 16, 16, mode)
    got = K.patch_residual_score(torch.from_numpy(resid).to(dev), None, (16, 16), MODES[mode])
    assert_bits_equal(got, want, f"mode {mode}")


def test_residual_score_fp32_and_bad_index(dev):
    rng = np.random.default_rng(9)
    curr = (rng.integers(-2048, 2048, (3, 64, 80, 3)) / 256.0).astype(np.float32)
    prev = (rng.integers(-2048, 2048, (3, 64, 80, 3)) / 256.0).astype(np.float32)
    for pw in (16, 8):
        want = OI.patch_residual_score(curr, prev, 16, pw, OI.RMS)
        got = K.patch_residual_score(torch.from_numpy(curr).to(dev), torch.from_numpy(prev).to(dev), (16, pw))
        assert_bits_equal(got, want, f"fp32 pw={pw}")
    got = K.patch_residual_score(torch.from_numpy(curr).to(dev), torch.from_numpy(prev).to(dev), (16, 16),
                                 image_idx=torch.tensor([1, 7], device=dev))
    assert torch.isnan(got[1]).all() and not torch.isnan(got[0]).any()


@pytest.mark.parametrize("B,G,P,thr,min_keep", [(16, 1024, 1024, 0.6, 1), (4, 1024, 256, 0.8, 40), (3, 196, 49, 0.5, 0),
                                                (2, 4096, 4096, 0.95, 300), (3, 64, 64, 0.0, 1)])
def test_residual_prune_bit_exact(dev, B, G, P, thr, min_keep):
    print(f"residual prune B={B} G={G} P={P} thr={thr} min_keep={min_keep}", flush=True)
    rng = np.random.default_rng(G + P)
    rms = (rng.integers(0, 1024, (B, G)) / 1024.0).astype(np.float32)
    if B >= 3:
        rms[1] = 0.25                      # ties everywhere: the rescue takes the lowest candidates
        rms[2, ::17] = np.nan
    spatial = np.stack([np.sort(rng.permutation(G)[:P]) for _ in range(B)]).astype(np.int64)
    dind = np.concatenate([np.tile(np.arange(5), (B, 1)), spatial + 5], axis=1)
    want = OI.residual_prune(dind, spatial, rms, thr, min_keep)
    rt, st, dt = (torch.from_numpy(a).to(dev) for a in (rms, spatial, dind))
    pk = K.residual_prune_keep(rt, st, thr, min_keep)
    assert_bits_equal(pk.keep, want.keep, "keep")
    assert_bits_equal(pk.kept_count.long(), want.kept_patch_count, "count")
    # exact float64 sums on the 2^-10 grid: equal values, NaN where a NaN residual enters the sum
    np.testing.assert_array_equal(pk.full_mass.cpu().numpy(), want.full_residual_mass)
    np.testing.assert_array_equal(pk.kept_mass.cpu().numpy(), want.kept_residual_mass)
    width = int(want.kept_patch_count.max())
    if width < P:
        pruned, local = K.residual_prune_compact(pk.keep, st, dt, 5, width)
        assert_bits_equal(pruned, want.pruned_dindice, "pruned dindice")
        assert_bits_equal(local, want.kept_local_idx, "kept local idx")


def test_executor_hint_map_and_residual_pruning(dev):
    """ViT-S 224 (14 x 14 patches), B=2, one group over every patch, token pruning on."""
    B, H = 2, 224
    config = ExperimentConfig(model_name="dinov3_classifier_vits16", batch_size=B, image_shape=(H, H, 3),
                              backbone="vits16",
                              appcorr_kwargs={"method": "partial_token", "token_prune_enabled": True,
                                              "token_prune_threshold": 60.0, "token_prune_min_keep": 3,
                                              "mobile_pscore": "residual_energy", "mobile_pscore_weight": 1.0},
                              transmission_kwargs={"pyramid_levels": [1, 0]})
    ex = DINOv3ClassifierExecutor(dev)
    ex.load_model(config.model_name, config)
    rng = np.random.default_rng(4)
    curr = rng.integers(0, 256, (B, H, H, 3), dtype=np.uint8)
    prev = curr.copy()
    noisy = rng.random((B, 14, 14)) < 0.3                 # patches that changed
    for b, i, j in zip(*np.nonzero(noisy)):
        prev[b, 16 * i:16 * i + 16, 16 * j:16 * j + 16] = rng.integers(0, 256, (16, 16, 3), dtype=np.uint8)
    payload = []
    hints = rng.random((B, 196)).astype(np.float32)
    for b in range(B):
        for s in range(196):
            payload.append(Patch(image_idx=b, spatial_idx=s, res_level=0, group_id=1, pscore_hint=float(hints[b, s])))
            payload.append(Patch(image_idx=b, spatial_idx=s, res_level=1, group_id=1, pscore_hint=99.0))
    task = Task(task_id=0, request_id=0, payload=[p for p in payload if p.res_level == 0], instructions=[])
    task_all = Task(task_id=0, request_id=0, payload=payload, instructions=[])
    ctx = {"input_hr_np": curr, "prev_input_hr_np": prev}
    with torch.no_grad():
        ex.preprocess(torch.from_numpy(curr), task, ctx, config)
    hint = ctx["mobile_pscore_hint_map"].cpu().numpy()
    want_hint = hints / np.maximum(hints.sum(axis=1, keepdims=True), np.finfo(np.float32).eps)
    np.testing.assert_allclose(hint, want_hint, rtol=1e-6, atol=0)
    # only the finest level's hints enter the map
    m2 = ex._build_mobile_pscore_hint_map(task_all, ctx, config, B, 196).cpu().numpy()
    np.testing.assert_allclose(m2, want_hint, rtol=1e-6, atol=0)
    plan = ctx["group_plans"][1]
    rms = OI.patch_residual_score(curr, prev, 16, 16, OI.RMS)
    spatial = np.tile(np.arange(196), (B, 1))
    dind = np.concatenate([np.tile(np.arange(5), (B, 1)), spatial + 5], axis=1)
    want = OI.residual_prune(dind, spatial, rms, 60.0, 3)
    assert int(want.kept_patch_count.max()) < 196
    assert_bits_equal(plan.pruned_dindice, want.pruned_dindice, "pruned dindice")
    assert_bits_equal(plan.kept_patch_count.long(), want.kept_patch_count, "kept count")
    assert_bits_equal(plan.group_patch_keep_local_idx, want.kept_local_idx, "local idx")
    np.testing.assert_allclose(plan.kept_residual_mass.cpu().numpy(), want.kept_residual_mass, rtol=1e-6)
    qs = plan.query_state
    assert int(qs.active_token_idx.numel()) == B * 5 + int(want.kept_patch_count.sum())
