"""GPU parity of the top-k plan kernel against the numpy oracle: bit-exact indices and masks."""

import numpy as np
import pytest
import torch

from appcorr_amd import kernels as K
from oracle import plan as OP
from tests.util import assert_bits_equal

pytestmark = pytest.mark.gpu


def _check(dev, scores: np.ndarray, k: int, npre: int, ntok: int | None = None, dindice: np.ndarray | None = None):
    B, P = scores.shape
    if dindice is None:
        dindice = np.broadcast_to(np.arange(npre + P, dtype=np.int64), (B, npre + P)).copy()
    N = int(dindice.max()) + 1 if ntok is None else ntok
    got = K.topk_plan(torch.from_numpy(scores).to(dev), k, torch.from_numpy(dindice).to(dev), npre, N)
    ref = OP.build_plan(scores, k, dindice, npre, N)
    assert_bits_equal(got.update_indice, ref.update_indice, "update_indice")
    assert_bits_equal(got.active_batch_idx, ref.active_batch_idx, "active_batch_idx")
    assert_bits_equal(got.active_pos_idx, ref.active_pos_idx, "active_pos_idx")
    assert_bits_equal(got.active_token_idx, ref.active_token_idx, "active_token_idx")
    assert_bits_equal(got.active_patch_mask, ref.active_patch_mask.astype(np.uint8), "patch_mask")
    assert_bits_equal(got.active_rope_idx, ref.active_rope_idx, "rope_idx")
    assert_bits_equal(got.keep_mask, ref.keep_mask.astype(np.uint8), "keep_mask")
    assert_bits_equal(got.row_slot, ref.row_slot, "row_slot")


@pytest.mark.parametrize("B,P,ratio", [(16, 1024, 0.25), (16, 1024, 0.10), (16, 1024, 0.50), (8, 1024, 0.25),
                                       (1, 196, 0.5), (4, 4096, 0.10), (3, 100, 0.33), (2, 16384, 0.05)])
def test_topk_laplace_importance(dev, B, P, ratio):
    rng = np.random.default_rng(P + B)
    delta = rng.laplace(size=(B, P, 32)).astype(np.float32)
    scores = np.linalg.norm(delta, axis=-1).astype(np.float32)
    _check(dev, scores, OP.keep_count(P, ratio), 5)


@pytest.mark.parametrize("k", [0, 1, 7, 63, 64, 65, 127, 128])
def test_topk_edge_k(dev, k):
    rng = np.random.default_rng(k)
    scores = rng.standard_normal((3, 128)).astype(np.float32)
    _check(dev, scores, k, 5)


def test_topk_all_keep(dev):
    scores = np.random.default_rng(0).standard_normal((2, 196)).astype(np.float32)
    _check(dev, scores, 196, 5)


def test_topk_ties_lowest_index_wins(dev):
    scores = np.zeros((4, 300), dtype=np.float32)
    scores[1, ::3] = 1.0
    scores[2] = np.repeat(np.arange(30, dtype=np.float32), 10)
    scores[3, 5] = -0.0
    _check(dev, scores, 77, 5)


def test_topk_negative_inf_candidates_and_nan(dev):
    rng = np.random.default_rng(5)
    scores = rng.standard_normal((2, 200)).astype(np.float32)
    scores[0, 10:150] = -np.inf
    scores[1, [3, 17]] = np.nan
    scores[1, [4, 18]] = np.inf
    _check(dev, scores, 100, 5)


def test_topk_candidate_subset_dindice(dev):
    # Candidates are a strided group of patches (a correction group), not all patches.
    rng = np.random.default_rng(6)
    B, N, npre = 4, 1029, 5
    grp = np.arange(npre, N)[::4]
    dind = np.stack([np.concatenate([np.arange(npre), grp])] * B).astype(np.int64)
    scores = rng.standard_normal((B, grp.size)).astype(np.float32)
    _check(dev, scores, 64, npre, ntok=N, dindice=dind)



def _check_stats(dev, scores: np.ndarray, keep: np.ndarray):
    got = K.plan_stats(torch.from_numpy(scores).to(dev), torch.from_numpy(keep).to(dev)).cpu().numpy().astype(np.float64)
    ref = OP.plan_stats(scores, keep)
    # fp32 sums in a fixed order against the float64 oracle: |error| <= n * 2^-24 * sum|s|.
    bound = scores.size * 2.0 ** -24 * float(np.abs(scores[np.isfinite(scores)]).sum()) + 1e-30
    for i in range(2):
        if np.isnan(ref[i]) or np.isinf(ref[i]):
            assert (np.isnan(got[i]) and np.isnan(ref[i])) or got[i] == ref[i], (i, got[i], ref[i])
        else:
            assert abs(got[i] - ref[i]) <= bound, (i, got[i], ref[i], bound)
    np.testing.assert_array_equal(got[2:], ref[2:])


@pytest.mark.parametrize("B,P,ratio", [(16, 1024, 0.25), (1, 196, 0.5), (3, 100, 0.33), (2, 16384, 0.05)])
def test_plan_stats_against_oracle(dev, B, P, ratio):
    rng = np.random.default_rng(B * 7 + P)
    scores = np.abs(rng.laplace(size=(B, P))).astype(np.float32)
    k = OP.keep_count(P, ratio)
    got = K.topk_plan(torch.from_numpy(scores).to(dev), k,
                      torch.from_numpy(np.broadcast_to(np.arange(5 + P, dtype=np.int64), (B, 5 + P)).copy()).to(dev), 5)
    _check_stats(dev, scores, got.keep_mask.cpu().numpy().astype(bool))


def test_plan_stats_masked_and_special_values(dev):
    rng = np.random.default_rng(11)
    scores = rng.standard_normal((3, 300)).astype(np.float32)
    keep = rng.random((3, 300)) < 0.3
    _check_stats(dev, scores, keep)
    s2 = scores.copy()
    s2[0, ~keep[0]] = -np.inf           # masked candidates (candidate_valid_mask): NaN kept mass
    _check_stats(dev, s2, keep)
    s3 = scores.copy()
    s3[1, np.flatnonzero(keep[1])[:2]] = -np.inf  # only kept -inf: kept mass -inf
    _check_stats(dev, s3, keep)
    _check_stats(dev, np.zeros((2, 0), dtype=np.float32), np.zeros((2, 0), dtype=bool))
