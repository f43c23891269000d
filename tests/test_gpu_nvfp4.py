"""GPU parity of NVFP4 quantize / dequantize against the numpy oracle: bit-exact bytes.

Shapes: the standalone BASELINE config ([16*1029, 1024] and [16*1029, 4096], N(0,1) with 1% x50
outliers), the reference test's M x K grid (tests/test_nvfp4_fused_quantize.py:14-15) and masked
tails (M % 128 != 0, K % 64 != 0)."""

import numpy as np
import pytest
import torch

from appcorr_amd import kernels as K
from oracle import nvfp4 as Q
from oracle.bf16 import bits_to_torch_bf16, f32_to_bf16_bits, bf16_bits_to_f32
from tests.util import assert_bits_equal, bits

pytestmark = pytest.mark.gpu


def _activations(M, K_, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((M, K_), dtype=np.float32)
    out = rng.random((M, K_)) < 0.01
    x[out] *= 50.0
    b = f32_to_bf16_bits(x)
    return b, bf16_bits_to_f32(b)


def _run(dev, M, K_, seed):
    xb, xf = _activations(M, K_, seed)
    ts = Q.per_tensor_amax_to_scale(np.abs(xf).max())
    x = bits_to_torch_bf16(xb).to(dev)
    tsd = torch.tensor([ts], dtype=torch.float32, device=dev)
    qd, sc = K.quantize_nvfp4_swizzled(x, tsd)
    rq, rs = Q.quantize(xf, ts)
    assert_bits_equal(qd, rq, f"qdata M={M} K={K_}")
    assert_bits_equal(sc.view(torch.uint8), rs, f"scales M={M} K={K_}")
    xh = K.dequantize_nvfp4(qd, sc, tsd)
    assert_bits_equal(xh, f32_to_bf16_bits(Q.dequantize(rq, rs, ts, M, K_)), f"dequant M={M} K={K_}")
    return x, xh


@pytest.mark.parametrize("M,K_", [(16464, 1024), (16464, 4096)])
def test_standalone_config_bit_exact(dev, M, K_):
    _run(dev, M, K_, M + K_)


@pytest.mark.parametrize("M", [1027, 1280, 2068, 5120])
@pytest.mark.parametrize("K_", [4096, 8192])
def test_reference_test_grid(dev, M, K_):
    x, xh = _run(dev, M, K_, 7 * M + K_)
    rel = ((x.float() - xh.float()).norm() / x.float().norm()).item()
    assert rel < 0.25  # tests/test_nvfp4_fused_quantize.py:107-109


@pytest.mark.parametrize("M,K_", [(1, 16), (5, 48), (130, 80), (129, 1040), (300, 16)])
def test_masked_tails(dev, M, K_):
    _run(dev, M, K_, M * 31 + K_)


def test_strided_rows(dev):
    xb, xf = _activations(256, 128, 3)
    big = torch.zeros(256, 256, dtype=torch.bfloat16)
    big[:, :128] = bits_to_torch_bf16(xb)
    ts = Q.per_tensor_amax_to_scale(np.abs(xf).max())
    qd, sc = K.quantize_nvfp4_swizzled(big.to(dev)[:, :128], torch.tensor([ts], device=dev))
    rq, rs = Q.quantize(xf, ts)
    assert_bits_equal(qd, rq, "qdata strided")
    assert_bits_equal(sc.view(torch.uint8), rs, "scales strided")


def test_signed_zeros_tiny_values_and_rounding_boundaries(dev):
    """-0.0 must encode as 0x8 (x / tot keeps the sign of x), tiny values as signed zero codes, and
    quotients that land exactly on or one ulp around an e2m1 rounding boundary (0.25, 0.75, 1.25,
    1.75, 2.5, 3.5, 5.0) must round as IEEE division does. Each 16-element block holds its maximum
    6 * tot at element 0, so the block's divisor is known, and boundary quotients are built by
    scaling that divisor."""
    M, K_ = 128, 256
    rng = np.random.default_rng(11)
    xf = rng.standard_normal((M, K_)).astype(np.float32)
    xb = f32_to_bf16_bits(xf)
    xf = bf16_bits_to_f32(xb)
    blocks = xf.reshape(M, K_ // 16, 16)
    blocks[:, :, 1] = -0.0
    blocks[:, :, 2] = 0.0
    blocks[:, ::3, 3] = -1e-30
    bounds = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0], np.float32)
    amax = np.abs(blocks).max(axis=2, keepdims=True)
    for e in range(4, 16):
        t = bounds[(e - 4) % 7] * (1.0 if e % 2 else -1.0)
        # a multiple of the block maximum, nudged by -1/0/+1 bf16 ulp; its quotient by the block's
        # divisor lands on or next to the boundary t (exactly on it when the scale is exact)
        v = bf16_bits_to_f32(f32_to_bf16_bits((amax[..., 0] * np.float32(t / 6.0)).astype(np.float32)))
        vb = f32_to_bf16_bits(v).astype(np.int32) + ((e % 3) - 1)
        blocks[:, :, e] = bf16_bits_to_f32(vb.astype(np.uint16))
    xb = f32_to_bf16_bits(blocks.reshape(M, K_))  # -1e-30 rounds to a bf16 value; the rest is bf16 already
    xf = bf16_bits_to_f32(xb)
    assert (np.signbit(xf.reshape(M, K_ // 16, 16)[:, :, 1]) & (xf.reshape(M, K_ // 16, 16)[:, :, 1] == 0)).all()
    ts = Q.per_tensor_amax_to_scale(np.abs(xf).max())
    x = bits_to_torch_bf16(xb).to(dev)
    tsd = torch.tensor([ts], dtype=torch.float32, device=dev)
    qd, sc = K.quantize_nvfp4_swizzled(x, tsd)
    rq, rs = Q.quantize(xf, ts)
    assert_bits_equal(qd, rq, "qdata signed zeros / boundaries")
    assert_bits_equal(sc.view(torch.uint8), rs, "scales signed zeros / boundaries")
    codes = np.stack([rq & 15, rq >> 4], axis=-1).reshape(M, K_)
    assert (codes.reshape(M, K_ // 16, 16)[:, :, 1] == 8).all()  # -0.0 -> 0x8 in the oracle too
