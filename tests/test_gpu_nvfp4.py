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
