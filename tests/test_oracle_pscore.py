"""Pins of the server-score oracle (oracle/pscore.py), on the CPU.

  * each score against torch's own CPU evaluation of the reference's expression on bf16 tensors
    (attention.py:251-271): the same rounding points, fp32 accumulation in torch's order. Equal on
    almost every element and never more than 1 bf16 ulp apart (the only freedom is where an fp32
    value falls within an fp32 ulp of a bf16 rounding boundary);
  * closed forms: identical keys give p = bf16(1/N) everywhere; a dominant key takes all the mass;
    the scores of one image sum to 1 within the bf16 rounding of its N entries;
  * the fused (log-sum-exp) score against float64 softmax column means;
  * the row log-sum-exp against torch.logsumexp of the float64 scores, and its closed form for
    identical keys (s + ln N).
"""

import math

import numpy as np
import pytest
import torch

from oracle import pscore as PS
from oracle.bf16 import round_bf16


def _bf(t):
    return t.to(torch.bfloat16)


def _ulps(a, b):
    """|a - b| in units of the bf16 ulp of max(|a|, |b|) (both bf16 values)."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    m = np.maximum(np.abs(a), np.abs(b))
    ulp = np.where(m > 0, 2.0 ** (np.floor(np.log2(np.where(m > 0, m, 1.0))) - 7), 2.0 ** -133)
    return np.abs(a - b) / ulp


def _qk(B, H, N, D, seed, qscale=1.0):
    g = torch.Generator().manual_seed(seed)
    q = _bf(torch.randn(B, H, N, D, generator=g) * qscale)
    k = _bf(torch.randn(B, N, H, D, generator=g))
    return q, k


@pytest.mark.parametrize("B,H,N,D", [(2, 6, 201, 64), (2, 16, 1029, 64), (1, 32, 300, 128)])
def test_cls_attn_prob_matches_torch_bf16(B, H, N, D):
    q, k = _qk(B, H, N, D, seed=N, qscale=2.0)
    scale = D ** -0.5
    kt = k.permute(0, 2, 1, 3)                                            # [B, H, N, D] view, as in the reference
    ref = (q[:, :, 0:1, :] @ kt.transpose(-2, -1).contiguous() * scale).softmax(-1).mean(dim=1).squeeze(1).float()
    got = PS.query_attention_prob(q[:, :, 0].float().numpy(), k.float().numpy(), scale)
    u = _ulps(got, ref.numpy())
    assert float(u.max()) <= 1.0
    assert float((u == 0).mean()) >= 0.995


def test_query_attention_prob_identical_keys():
    B, H, N, D = 2, 6, 201, 64
    g = torch.Generator().manual_seed(3)
    q = _bf(torch.randn(B, H, D, generator=g)).float().numpy()
    k = np.broadcast_to(_bf(torch.randn(1, 1, H, D, generator=g)).float().numpy(), (B, N, H, D))
    got = PS.query_attention_prob(q, np.ascontiguousarray(k), D ** -0.5)
    want = round_bf16(np.float32(1.0) / np.float32(N))
    np.testing.assert_array_equal(got, np.full((B, N), want, dtype=np.float32))


def test_query_attention_prob_dominant_key_and_mass():
    B, H, N, D = 2, 16, 1029, 64
    q, k = _qk(B, H, N, D, seed=5)
    qn = q[:, :, 0].float().numpy()
    kn = k.float().numpy().copy()
    kn[:, 17] = qn * 8.0                                                  # key 17 aligned with the query in every head
    kn = round_bf16(kn)
    got = PS.query_attention_prob(qn, kn, D ** -0.5)
    assert np.all(got.argmax(axis=1) == 17) and np.all(got[:, 17] > 0.99)
    q2, k2 = _qk(B, H, N, D, seed=6)
    p = PS.query_attention_prob(q2[:, :, 0].float().numpy(), k2.float().numpy(), D ** -0.5)
    assert np.all(np.abs(p.astype(np.float64).sum(axis=1) - 1.0) <= N * 2.0 ** -9 * p.max())


def test_pseudo_query_matches_torch_bf16():
    B, H, P, D = 2, 6, 196, 64
    g = torch.Generator().manual_seed(9)
    q_patch = _bf(torch.randn(B, H, P, D, generator=g) + 0.3)
    # attention.py:254-259 on bf16 tensors
    q_mean = q_patch.mean(dim=2, keepdim=True)
    q_mean_norm = q_mean.norm(dim=-1, keepdim=True).clamp_min(torch.finfo(q_mean.dtype).eps)
    target_norm = q_patch.norm(dim=-1, keepdim=True).mean(dim=2, keepdim=True)
    ref = (q_mean * (target_norm / q_mean_norm))[:, :, 0].float().numpy()
    got = PS.pseudo_query(q_patch.float().numpy())
    u = _ulps(got, ref)
    assert float(u.max()) <= 1.0 and float((u == 0).mean()) >= 0.98


def test_pseudo_query_clamps_a_zero_mean():
    """q_mean = 0 (every patch query paired with its negative): the norm is clamped to bf16 eps, so
    the pseudo query is 0 * target / eps = 0 rather than 0 / 0."""
    B, H, P, D = 1, 2, 8, 64
    g = torch.Generator().manual_seed(2)
    half = _bf(torch.randn(B, H, P // 2, D, generator=g)).float().numpy()
    q = np.concatenate([half, -half], axis=2)
    got = PS.pseudo_query(q)
    assert np.all(got == 0) and np.all(np.isfinite(got))


@pytest.mark.parametrize("B,H,N,D", [(1, 6, 201, 64), (1, 4, 300, 64)])
def test_patch_attn_prob_matches_torch_bf16(B, H, N, D):
    q, k = _qk(B, H, N, D, seed=11, qscale=1.5)
    scale = D ** -0.5
    kt = k.permute(0, 2, 1, 3).contiguous()
    ref = (q @ kt.transpose(-2, -1).contiguous() * scale).softmax(dim=-1).mean(dim=1).mean(dim=1).float().numpy()
    got = PS.patch_attn_prob(q.float().numpy(), k.float().numpy(), scale)
    u = _ulps(got, ref)
    assert float(u.max()) <= 1.0 and float((u == 0).mean()) >= 0.98


def test_patch_attn_prob_fused_matches_float64_softmax():
    B, H, N, D = 1, 4, 257, 128
    q, k = _qk(B, H, N, D, seed=13)
    scale = D ** -0.5
    qd = q.double()
    kd = k.double().permute(0, 2, 1, 3)
    p = torch.softmax(qd @ kd.transpose(-2, -1) * scale, dim=-1)          # [B, H, N, N]
    want = round_bf16((p.sum(dim=(1, 2)) / (H * N)).float().numpy())
    got = PS.patch_attn_prob_fused(q.float().numpy(), k.float().numpy(), scale)
    u = _ulps(got, want)
    assert float(u.max()) <= 1.0 and float((u == 0).mean()) >= 0.99
    assert math.isclose(float(got.astype(np.float64).sum()), 1.0, rel_tol=N * 2.0 ** -8)


def test_row_logsumexp_matches_torch_and_closed_form():
    B, H, N, D = 2, 3, 97, 64
    q, k = _qk(B, H, N, D, seed=21, qscale=3.0)
    scale = D ** -0.5
    s = q.double() @ k.double().permute(0, 2, 3, 1) * scale                  # [B, H, N, N]
    want = torch.logsumexp(s, dim=-1).numpy()
    got = PS.row_logsumexp(q.float().numpy(), k.float().numpy(), scale)
    assert got.shape == (B, H, N)
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-12)
    assert bool((got >= s.max(dim=-1).values.numpy() - 1e-12).all())
    # identical keys: every score of a query is the same s, so lse = s + ln N
    k1 = k[:, :1].expand(B, N, H, D).contiguous()
    s1 = (q.double() @ k1.double().permute(0, 2, 3, 1) * scale)[..., 0]
    got1 = PS.row_logsumexp(q.float().numpy(), k1.float().numpy(), scale)
    np.testing.assert_allclose(got1, s1.numpy() + math.log(N), rtol=0, atol=1e-11)
