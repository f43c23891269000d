"""Pins of the top-k / packed-plan oracle (oracle/plan.py) and the row oracle (oracle/rows.py).

Facts fixed independently of the oracle's code:
  * keep_count: hand-computed values of min(int(P * ratio), P) (block.py:378), including the
    truncations a rounding mistake would change;
  * topk_keep: a brute-force pairwise ranking (i is kept iff fewer than k candidates beat it), a
    different formulation from the oracle's lexsort; torch.topk on distinct scores; hand-derived
    known answers for ties, -0/+0, -inf and NaN;
  * build_plan: a hand-derived plan for a candidate subset with pretokens, and the inverse relation
    between row_slot and update_indice;
  * rows: layerscale_add against torch's fp32 evaluation (the product of two bf16 values is exact
    in fp32, so two fp32 ops equal one fused rounding).
"""

import itertools

import numpy as np
import pytest
import torch

from oracle import plan as OP
from oracle import rows as OR
from oracle.bf16 import bits_to_torch_bf16, torch_bf16_to_bits


@pytest.mark.parametrize("P,ratio,k", [
    (1024, 0.25, 256), (1024, 1.0, 1024), (1024, 1.5, 1024), (1024, 0.0, 0), (196, 0.5, 98),
    (196, 0.3, 58), (196, 0.1, 19), (4096, 0.25, 1024), (3, 0.999, 2), (1, 0.5, 0),
])
def test_keep_count_known_values(P, ratio, k):
    assert OP.keep_count(P, ratio) == k


def _beats(sj, si, j, i):
    nj, ni = np.isnan(sj), np.isnan(si)
    if nj != ni:
        return bool(nj)
    if nj and ni:
        return j < i
    return bool(sj > si or (sj == si and j < i))


def _brute_keep(row, k):
    P = row.shape[0]
    kept = [i for i in range(P) if sum(_beats(row[j], row[i], j, i) for j in range(P) if j != i) < k]
    return np.array(sorted(kept), dtype=np.int64)


def test_topk_brute_force_small():
    rng = np.random.default_rng(0)
    for trial in range(300):
        P = int(rng.integers(1, 12))
        pool = np.array([0.0, -0.0, 1.0, -1.0, 2.5, np.inf, -np.inf, np.nan], dtype=np.float32)
        row = rng.choice(pool, P) if trial % 2 else rng.standard_normal(P).astype(np.float32)
        for k in range(0, P + 1):
            got = OP.topk_keep(row[None], k)[0]
            np.testing.assert_array_equal(got, _brute_keep(row, k), err_msg=f"{row} k={k}")


def test_topk_matches_torch_on_distinct_scores():
    g = torch.Generator().manual_seed(1)
    for B, P, k in [(4, 1024, 256), (2, 196, 98), (3, 4096, 1024), (1, 64, 1)]:
        s = torch.randperm(B * P, generator=g).reshape(B, P).to(torch.float32) / (B * P)
        ref = torch.topk(s, k, dim=-1).indices.sort(dim=-1).values.numpy()
        np.testing.assert_array_equal(OP.topk_keep(s.numpy(), k), ref)


def test_topk_known_answers():
    nan, inf = np.float32(np.nan), np.float32(np.inf)
    cases = [
        ([0.1, 0.5, 0.5, 0.3], 2, [1, 2]),
        ([0.1, 0.5, 0.5, 0.3], 1, [1]),          # tie: lowest index wins
        ([0.5, 0.5, 0.5, 0.5], 2, [0, 1]),
        ([-0.0, 0.0], 1, [0]),                   # -0 == +0: lowest index
        ([0.0, -0.0], 1, [0]),
        ([-inf, -inf, 1.0], 2, [0, 2]),          # -inf candidates still fill the quota in index order
        ([1.0, nan, 2.0], 1, [1]),               # NaN ranks above everything
        ([inf, nan, inf], 2, [0, 1]),
        ([3.0, 1.0, 2.0], 3, [0, 1, 2]),
        ([3.0, 1.0, 2.0], 0, []),
    ]
    for row, k, want in cases:
        got = OP.topk_keep(np.array([row], dtype=np.float32), k)[0]
        assert got.tolist() == want, (row, k, got)


def test_build_plan_hand_derived():
    # 2 images, 2 pretokens, 6 patch tokens (N = 8); the group covers patch tokens {3, 5, 6, 7}
    dind = np.array([[0, 1, 3, 5, 6, 7], [0, 1, 3, 5, 6, 7]], dtype=np.int64)
    scores = np.array([[0.9, 0.1, 0.8, 0.2], [0.0, 0.5, 0.5, 0.7]], dtype=np.float32)
    p = OP.build_plan(scores, 2, dind, num_pretokens=2, num_tokens=8)
    # image 0 keeps candidates {0, 2} -> tokens {3, 6}; image 1 keeps {3, 1} -> tokens {5, 7}
    np.testing.assert_array_equal(p.update_indice, [[0, 1, 3, 6], [0, 1, 5, 7]])
    np.testing.assert_array_equal(p.active_batch_idx, [0, 0, 0, 0, 1, 1, 1, 1])
    np.testing.assert_array_equal(p.active_pos_idx, [0, 1, 2, 3, 0, 1, 2, 3])
    np.testing.assert_array_equal(p.active_token_idx, [0, 1, 3, 6, 0, 1, 5, 7])
    np.testing.assert_array_equal(p.active_patch_mask, [0, 0, 1, 1, 0, 0, 1, 1])
    np.testing.assert_array_equal(p.active_rope_idx, [0, 0, 1, 4, 0, 0, 3, 5])
    np.testing.assert_array_equal(p.keep_mask, [[True, False, True, False], [False, True, False, True]])
    np.testing.assert_array_equal(p.row_slot, [[0, 1, -1, 2, -1, -1, 3, -1], [4, 5, -1, -1, -1, 6, -1, 7]])


def test_row_slot_inverts_update_indice():
    rng = np.random.default_rng(2)
    for B, P, k, pre in [(3, 64, 16, 5), (2, 196, 98, 5), (1, 10, 0, 5), (2, 10, 10, 1)]:
        N = pre + P
        dind = np.tile(np.arange(N), (B, 1))
        p = OP.build_plan(rng.standard_normal((B, P)).astype(np.float32), k, dind, pre, N)
        T = pre + k
        for b, s in itertools.product(range(B), range(T)):
            assert p.row_slot[b, p.update_indice[b, s]] == b * T + s
        assert (p.row_slot >= 0).sum() == B * T
        assert p.keep_mask.sum() == B * k


def test_layerscale_add_single_rounding_matches_torch_fp32():
    g = torch.Generator().manual_seed(3)
    x = (torch.randn(64, 512, generator=g) * 4).to(torch.bfloat16)
    a = torch.randn(64, 512, generator=g).to(torch.bfloat16)
    gam = (torch.rand(512, generator=g) * 2 - 1).to(torch.bfloat16)
    ref = (x.float() + a.float() * gam.float()).to(torch.bfloat16)  # a*g exact in fp32
    got = OR.layerscale_add(torch_bf16_to_bits(x), torch_bf16_to_bits(a), torch_bf16_to_bits(gam)[None])
    np.testing.assert_array_equal(got, torch_bf16_to_bits(ref))


def test_reconstruct_matches_torch_eager_sequence():
    """block.py:1143-1179 as torch bf16 eager ops (each op rounds once): x + bos on every row, then
    x_attn + mlp on selected rows, and bos rows = (x_attn - x_act) + mlp."""
    g = torch.Generator().manual_seed(4)
    B, N, C, T = 2, 12, 64, 5
    x = torch.randn(B, N, C, generator=g).to(torch.bfloat16)
    bos = (torch.randn(B, N, C, generator=g) * 0.1).to(torch.bfloat16)
    b = np.repeat(np.arange(B), T)
    t = np.concatenate([np.sort(np.random.default_rng(b_).choice(N, T, replace=False)) for b_ in range(B)])
    x_act = x[torch.from_numpy(b), torch.from_numpy(t)]
    x_attn = (x_act.float() + torch.randn(B * T, C, generator=g) * 0.3).to(torch.bfloat16)
    mlp = (torch.randn(B * T, C, generator=g) * 0.2).to(torch.bfloat16)
    x_out = x + bos
    x_out[torch.from_numpy(b), torch.from_numpy(t)] = x_attn + mlp
    bos_ref = bos.clone()
    bos_ref[torch.from_numpy(b), torch.from_numpy(t)] = (x_attn - x_act) + mlp
    xo, nb = OR.reconstruct_scatter_persist(torch_bf16_to_bits(x), torch_bf16_to_bits(bos), b, t,
                                            torch_bf16_to_bits(x_act), torch_bf16_to_bits(x_attn),
                                            torch_bf16_to_bits(mlp))
    np.testing.assert_array_equal(xo, torch_bf16_to_bits(x_out))
    np.testing.assert_array_equal(nb, torch_bf16_to_bits(bos_ref))
    assert bits_to_torch_bf16(xo).shape == x.shape


def test_plan_stats_known_answers():
    # Hand-derived: masses are sums of the kept / all scores, counts are plain counts.
    s = np.array([[1.0, 2.0, 3.0, 4.0], [0.5, -1.5, 2.5, 0.0]], dtype=np.float32)
    keep = np.array([[0, 1, 0, 1], [1, 0, 1, 0]], dtype=bool)
    got = OP.plan_stats(s, keep)
    np.testing.assert_array_equal(got, [2.0 + 4.0 + 0.5 + 2.5, 1 + 2 + 3 + 4 + 0.5 - 1.5 + 2.5 + 0.0, 4.0, 8.0, 2.0])
    # An unkept -inf score: -inf * 0 is NaN in the kept mass; the full mass is -inf.
    s2 = s.copy()
    s2[0, 0] = -np.inf
    got = OP.plan_stats(s2, keep)
    assert np.isnan(got[0]) and got[1] == -np.inf and got[2] == 4.0
    # Kept -inf alone: the kept mass is -inf, not NaN.
    keep2 = keep.copy()
    keep2[0, 0] = True
    got = OP.plan_stats(s2, keep2)
    assert got[0] == -np.inf and got[2] == 5.0


def test_plan_stats_matches_torch_formula():
    import torch
    rng = np.random.default_rng(3)
    s = rng.standard_normal((16, 1024)).astype(np.float32)
    keep = rng.random((16, 1024)) < 0.25
    st, kt = torch.from_numpy(s), torch.from_numpy(keep)
    ref = [float((st * kt.to(st.dtype)).sum(dtype=torch.float32)), float(st.sum(dtype=torch.float32)),
           float(kt.sum(dtype=torch.float32))]
    got = OP.plan_stats(s, keep)
    np.testing.assert_allclose(got[:3], ref, rtol=1e-5, atol=1e-3)
    assert got[3] == 16 * 1024 and got[4] == 16
