"""Pins of the threshold-selection oracle (oracle.plan.threshold_keep / threshold_plan).

Facts fixed independently of the oracle's code:
  * the kept mask is torch's own `fp32 tensor >= python float` (block.py:374-376), evaluated by torch
    on inputs where fp32 and float64 comparison disagree (a threshold that rounds down to a score),
    and on NaN, +-inf, -0.0;
  * hand-derived plans for both builders (block.py:492-560 fixed width; 562-621 padded): truncation
    in candidate order, the last-kept fill, candidate 0 for an image that keeps nothing, token 0
    padding, the compacted active rows, all_valid;
  * with distinct scores and the threshold at each image's k-th largest score, the threshold plan
    keeps exactly the top-k set (oracle.topk_keep, itself pinned by brute force), and its packed
    rows equal the top-k plan's;
  * properties: the fixed-width builder with a cap at or above every count has the padded builder's
    queries; every non-query row repeats a query row of its image; row_slot points at the first slot
    of each query token.
"""

import numpy as np
import pytest
import torch

from oracle import plan as OP


def test_keep_mask_is_torchs_fp32_comparison():
    s = np.array([1.0, np.nan, -np.inf, np.inf, -0.0, 0.0, np.float32(0.1), 1.0000001, 0.99999994], np.float32)
    for thres in (1.0000000001, 0.0, -0.0, float("-inf"), float("inf"), 0.1, 1.0, -1.5):
        want = (torch.from_numpy(s) >= thres).numpy()
        np.testing.assert_array_equal(OP.threshold_keep(s[None], thres)[0], want, err_msg=str(thres))
    # the case that separates fp32 from float64 comparison: 1.0 >= 1.0000000001 only in fp32
    assert OP.threshold_keep(np.array([[1.0]], np.float32), 1.0000000001)[0, 0]


def _dind():
    # 2 pretokens, 5 candidates; image 1 uses a candidate subset with other token ids
    return np.array([[0, 1, 2, 3, 4, 5, 6], [0, 1, 10, 11, 12, 13, 14]], dtype=np.int64)


SC = np.array([[0.5, 0.1, 0.9, 0.3, 0.7],
               [0.0, 0.0, 0.0, 0.0, 0.0]], dtype=np.float32)


def test_padded_builder_hand_derived():
    p = OP.threshold_plan(SC, 0.4, _dind(), 2, 15)
    # image 0 keeps candidates 0, 2, 4 -> tokens 2, 4, 6; image 1 keeps none
    np.testing.assert_array_equal(p.update_indice, [[0, 1, 2, 4, 6], [0, 1, 0, 0, 0]])
    np.testing.assert_array_equal(p.query_valid_mask, [[1, 1, 1, 1, 1], [1, 1, 0, 0, 0]])
    np.testing.assert_array_equal(p.kept_count, [3, 0])
    np.testing.assert_array_equal(p.active_batch_idx, [0, 0, 0, 0, 0, 1, 1])
    np.testing.assert_array_equal(p.active_pos_idx, [0, 1, 2, 3, 4, 0, 1])
    np.testing.assert_array_equal(p.active_token_idx, [0, 1, 2, 4, 6, 0, 1])
    np.testing.assert_array_equal(p.active_rope_idx, [0, 0, 0, 2, 4, 0, 0])
    assert p.all_valid is False
    # packed rows: image 1's non-query slots repeat its last pretoken (token 1)
    np.testing.assert_array_equal(p.rows.update_indice, [[0, 1, 2, 4, 6], [0, 1, 1, 1, 1]])
    rs = p.rows.row_slot
    assert rs[0, 2] == 2 and rs[0, 4] == 3 and rs[0, 6] == 4 and rs[0, 3] == -1
    assert rs[1, 0] == 5 and rs[1, 1] == 6 and (rs[1, 2:] == -1).all()


def test_fixed_width_builder_hand_derived():
    p = OP.threshold_plan(SC, 0.4, _dind(), 2, 15, keep_cap=2)
    # image 0 keeps 3 > cap: the first two in candidate order; image 1 keeps none: candidate 0 twice
    np.testing.assert_array_equal(p.update_indice, [[0, 1, 2, 4], [0, 1, 10, 10]])
    assert p.query_valid_mask.all() and p.all_valid
    np.testing.assert_array_equal(p.active_token_idx, [0, 1, 2, 4, 0, 1, 10, 10])
    np.testing.assert_array_equal(p.kept_count, [3, 0])
    p5 = OP.threshold_plan(SC, 0.4, _dind(), 2, 15, keep_cap=9)   # cap clamps to P = 5
    np.testing.assert_array_equal(p5.update_indice, [[0, 1, 2, 4, 6, 6, 6], [0, 1, 10, 10, 10, 10, 10]])
    assert p5.row_slot[0, 6] == 4 and p5.row_slot[1, 10] == 9


def test_empty_and_full_selection():
    d = _dind()
    none = OP.threshold_plan(SC, 5.0, d, 2, 15)
    assert none.update_indice.shape == (2, 2) and none.active_token_idx.tolist() == [0, 1, 0, 1] and none.all_valid
    full = OP.threshold_plan(SC, -1.0, d, 2, 15)
    np.testing.assert_array_equal(full.update_indice, d)
    assert full.all_valid


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_threshold_at_kth_score_is_topk(seed):
    rng = np.random.default_rng(seed)
    B, P, pre, k = 1, 300, 5, 77
    s = rng.permutation(np.arange(P, dtype=np.float32) * 0.01 - 1.0)[None]
    d = np.concatenate([np.arange(pre), pre + np.arange(P)])[None].astype(np.int64)
    thres = float(np.sort(s[0])[::-1][k - 1])
    tp = OP.threshold_plan(s, thres, d, pre, pre + P)
    ref = OP.build_plan(s, k, d, pre, pre + P)
    np.testing.assert_array_equal(tp.keep_mask, ref.keep_mask)
    for f in ("update_indice", "active_token_idx", "active_pos_idx", "active_rope_idx", "row_slot"):
        np.testing.assert_array_equal(getattr(tp, f), getattr(ref, f), err_msg=f)
        np.testing.assert_array_equal(getattr(tp.rows, f), getattr(ref, f), err_msg=f)


def test_builder_properties_random():
    rng = np.random.default_rng(7)
    B, P, pre, N = 6, 97, 5, 5 + 97 + 3
    s = rng.standard_normal((B, P)).astype(np.float32)
    s[1] = -5.0                       # keeps nothing
    s[2, ::3] = np.nan
    d = np.concatenate([np.tile(np.arange(pre), (B, 1)),
                        np.stack([pre + rng.permutation(P + 3)[:P] for _ in range(B)])], axis=1).astype(np.int64)
    padded = OP.threshold_plan(s, 0.3, d, pre, N)
    capped = OP.threshold_plan(s, 0.3, d, pre, N, keep_cap=int(padded.kept_count.max()))
    T = padded.update_indice.shape[1]
    assert capped.update_indice.shape[1] == T
    v = padded.query_valid_mask
    np.testing.assert_array_equal(capped.update_indice[v], padded.update_indice[v])
    assert (padded.update_indice[~v] == 0).all()
    assert padded.active_token_idx.size == B * pre + int(padded.kept_count.sum())
    rows = padded.rows.update_indice
    for b in range(B):
        qset = set(padded.update_indice[b][v[b]].tolist())
        assert set(rows[b].tolist()) <= qset
        for t in qset:
            first = int(np.flatnonzero(rows[b] == t)[0])
            assert padded.row_slot[b, t] == b * T + first
