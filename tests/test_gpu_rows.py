"""GPU parity of the row-movement kernels against the numpy oracle: bit-exact."""

import numpy as np
import pytest
import torch

from appcorr_amd import kernels as K
from oracle import rows as R
from oracle.bf16 import bits_to_torch_bf16
from tests.util import assert_bits_equal, bits

pytestmark = pytest.mark.gpu


def _rand_bf16(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g).to(torch.bfloat16)


def _sel(B, N, T, seed):
    rng = np.random.default_rng(seed)
    toks = np.stack([np.sort(rng.choice(N, T, replace=False)) for _ in range(B)])
    b = np.repeat(np.arange(B), T)
    return torch.from_numpy(b.astype(np.int64)), torch.from_numpy(toks.reshape(-1).astype(np.int64))


@pytest.mark.parametrize("B,N,C,T", [(16, 1029, 1024, 261), (4, 1029, 4096, 414), (1, 201, 384, 103), (3, 7, 8, 5),
                                     (2, 9, 12, 3)])
def test_gather_rows(dev, B, N, C, T):
    x = _rand_bf16((B, N, C), 0)
    bi, ti = _sel(B, N, T, 1)
    got = K.gather_rows(x.to(dev), bi.to(dev), ti.to(dev))
    ref = R.gather_rows(bits(x), bi.numpy(), ti.numpy())
    assert_bits_equal(got, ref, "gather_rows")


@pytest.mark.parametrize("B,N,C,T,fp4", [(16, 1029, 1024, 261, False), (4, 1029, 4096, 414, False),
                                         (1, 201, 384, 103, False), (3, 7, 8, 5, False), (4, 1029, 4096, 414, True),
                                         (2, 40, 384, 17, True)])
def test_gather_rows_ln_equals_gather_then_layernorm(dev, B, N, C, T, fp4):
    """The packed run's first step (gather + block 0's norm1, optionally as the NVFP4 qkv operand) in one
    launch: the gathered rows equal the oracle's gather and the LayerNorm equals the standalone kernel's
    on them, bit for bit (the standalone kernel is pinned against the oracle elsewhere)."""
    x = _rand_bf16((B, N, C), 2)
    bi, ti = _sel(B, N, T, 3)
    w = (1.0 + 0.1 * _rand_bf16((C,), 4).float()).to(torch.bfloat16).to(dev)
    b = (0.1 * _rand_bf16((C,), 5).float()).to(torch.bfloat16).to(dev)
    ts = torch.tensor([0.37], device=dev) if fp4 else None
    xd = x.to(dev)
    xp, xn = K.gather_rows_ln(xd, bi.to(dev), ti.to(dev), w, b, 1e-6, nvfp4_scale=ts)
    assert_bits_equal(xp, R.gather_rows(bits(x), bi.numpy(), ti.numpy()), "gathered rows")
    assert_bits_equal(xn, K.layer_norm(xp, w, b, 1e-6, nvfp4_scale=ts).cpu(), "LayerNorm of the gathered rows")


@pytest.mark.parametrize("rows,C", [(16 * 1029, 1024), (4 * 4101, 4096), (201, 384), (3, 8)])
def test_residual_pair(dev, rows, C):
    """The approximate block's blocks_out_sum and output in one launch equal the two LayerScale adds
    with a gamma of ones (bf16(a + b) each; the add kernel is pinned against the oracle)."""
    inc, xa, mlp = (_rand_bf16((rows, C), s).to(dev) for s in (6, 7, 8))
    ones = torch.ones(C, dtype=torch.bfloat16, device=dev)
    bos, out = K.residual_pair(inc, xa, mlp)
    assert_bits_equal(bos, K.fused_layerscale_add(inc, mlp, ones).cpu(), "blocks_out_sum")
    assert_bits_equal(out, K.fused_layerscale_add(xa, mlp, ones).cpu(), "block output")


def test_gather_rows_empty(dev):
    x = _rand_bf16((2, 5, 64), 0).to(dev)
    e = torch.empty(0, dtype=torch.long, device=dev)
    assert K.gather_rows(x, e, e).shape == (0, 64)


@pytest.mark.parametrize("B,N,H,D,T", [(16, 1029, 16, 64, 261), (4, 4101, 32, 128, 414), (1, 201, 6, 64, 103)])
def test_kv_rewrite_from_strided_qkv_view(dev, B, N, H, D, T):
    """The K/V rewrite source is qkv_new[:, 1:] (row stride 3C, row 2C), attention.py:444-454."""
    kv = _rand_bf16((B, N, 2, H, D), 2)
    qkv = _rand_bf16((B * T, 3, H, D), 3)
    bi, ti = _sel(B, N, T, 4)
    kv_d = kv.to(dev)
    src = qkv.to(dev)[:, 1:]
    assert not src.is_contiguous()
    K.scatter_rows(kv_d, bi.to(dev), ti.to(dev), src)
    ref = R.scatter_rows(bits(kv), bi.numpy(), ti.numpy(), bits(qkv)[:, 1:])
    assert_bits_equal(kv_d, ref, "kv rewrite")


def test_scatter_rows_odd_width(dev):
    # 6-byte rows exercise the narrow-vector path
    dst = _rand_bf16((3, 11, 3), 5)
    src = _rand_bf16((4, 3), 6)
    bi = torch.tensor([0, 1, 2, 2])
    ti = torch.tensor([10, 0, 3, 4])
    d = dst.to(dev)
    K.scatter_rows(d, bi.to(dev), ti.to(dev), src.to(dev))
    assert_bits_equal(d, R.scatter_rows(bits(dst), bi.numpy(), ti.numpy(), bits(src)), "scatter odd")


@pytest.mark.parametrize("B,N,C,T", [(16, 1029, 1024, 261), (2, 201, 384, 50)])
def test_active_token_update(dev, B, N, C, T):
    x = _rand_bf16((B, N, C), 7)
    a = _rand_bf16((B * T, C), 8)
    d = _rand_bf16((B * T, C), 9)
    bi, ti = _sel(B, N, T, 10)
    got = K.active_token_update(x.to(dev), bi.to(dev), ti.to(dev), a.to(dev), d.to(dev))
    ref = R.active_token_update(bits(x), bi.numpy(), ti.numpy(), bits(a), bits(d))
    assert_bits_equal(got, ref, "active_token_update")


@pytest.mark.parametrize("B,N,C,T", [(16, 1029, 1024, 261), (1, 201, 384, 103), (2, 9, 64, 0), (2, 9, 64, 9)])
@pytest.mark.parametrize("inplace", [False, True])
def test_reconstruct_scatter_persist(dev, B, N, C, T, inplace):
    x = _rand_bf16((B, N, C), 11)
    bos = (_rand_bf16((B, N, C), 12).float() * 0.1).to(torch.bfloat16)
    xa = _rand_bf16((B * T, C), 13)
    xt = _rand_bf16((B * T, C), 14)
    ml = _rand_bf16((B * T, C), 15)
    bi, ti = _sel(B, N, T, 16)
    slot = np.full((B, N), -1, dtype=np.int32)
    slot[bi.numpy(), ti.numpy()] = np.arange(B * T, dtype=np.int32)
    xd, bd = x.to(dev), bos.to(dev)
    out = K.reconstruct_scatter_persist(xd, bd, torch.from_numpy(slot).to(dev), xa.to(dev), xt.to(dev), ml.to(dev),
                                        out=xd if inplace else None)
    ref_x, ref_b = R.reconstruct_scatter_persist(bits(x), bits(bos), bi.numpy(), ti.numpy(), bits(xa), bits(xt),
                                                 bits(ml))
    assert_bits_equal(out, ref_x, "x_out")
    assert_bits_equal(bd, ref_b, "blocks_out_sum")
    if inplace:
        assert out.data_ptr() == xd.data_ptr()


def test_fused_layerscale_add(dev):
    x = _rand_bf16((4176, 1024), 17)
    a = _rand_bf16((4176, 1024), 18)
    g = _rand_bf16((1024,), 19)
    got = K.fused_layerscale_add(x.to(dev), a.to(dev), g.to(dev))
    assert_bits_equal(got, R.layerscale_add(bits(x), bits(a), bits(g)), "layerscale_add")


def test_patch_importance(dev):
    g = torch.Generator().manual_seed(20)
    d = torch.randn(16, 1024, 1024, generator=g)
    for mode, ref in ((0, d.double().norm(dim=-1)), (1, (d.double() ** 2).sum(-1)),
                      (2, (d.double() ** 2).mean(-1).sqrt())):
        got = K.patch_importance(d.to(dev), mode).cpu().double()
        torch.testing.assert_close(got, ref, rtol=2e-6, atol=0)
