"""Pins of the low-precision linear oracle (oracle/lowp.py), on the CPU.

  * FP8 activation quantizer: known answers from the OCP e4m3 definition (ties to even at the
    midpoints, the subnormal range, saturation by the clamp), with the fp32 product x * inv;
  * FP8 weight quantizer: the quotient is rounded to bf16 before the e4m3 rounding (eager bf16 ops) --
    a case where that double rounding gives another e4m3 value than rounding the fp32 quotient once;
  * NVFP4 operand: every x_hat is an e2m1 grid value times its block's e4m3 scale, within half an e2m1
    step of x / ts, and equal to the packed tensor's dequantized value divided by the tensor scale;
  * the exact GEMMs against float64 matmuls of the quantized operands, the FP8 scales on the
    accumulator, the NVFP4 out_scale rounded to bf16;
  * the SwiGLU epilogue at closed-form points (silu(0) = 0, silu(a) -> a for large a).
"""

import numpy as np
import torch

from oracle import lowp as LPO
from oracle import nvfp4 as Q
from oracle.bf16 import round_bf16

GRID = np.array([0, 0.5, 1, 1.5, 2, 3, 4, 6], dtype=np.float32)


def test_fp8_activation_known_answers():
    inv = 1.0
    x = np.array([1.0625, 1.1875, 1.0626, 500.0, -500.0, 2 ** -10, 3 * 2 ** -10, 0.0, -0.0, 17.0, 240.0, 232.0],
                 dtype=np.float32)
    want = np.array([1.0, 1.25, 1.125, 448.0, -448.0, 0.0, 2 * 2 ** -9, 0.0, -0.0, 16.0, 240.0, 224.0],
                    dtype=np.float32)
    got = LPO.fp8_act(x, inv)
    np.testing.assert_array_equal(got, want)
    assert np.signbit(got[8])
    # the product is an fp32 product: x * inv with inv = bf16(1 / 3)
    inv3 = float(round_bf16(np.float32(1.0) / np.float32(3.0)))
    x3 = np.array([3.0, 6.0, 300.0], dtype=np.float32)
    np.testing.assert_array_equal(LPO.fp8_act(x3, inv3), LPO.e4m3(np.clip(x3 * np.float32(inv3), -448, 448)))


def test_fp8_weight_rounds_the_quotient_to_bf16_first():
    # w / s = 1.0660 (fp32): bf16 -> 1.0625, an e4m3 tie -> 1.0 (even); rounded once it would be 1.125
    w = np.array([1.0660], dtype=np.float32)
    assert float(round_bf16(w)[0]) == 1.0625
    assert float(LPO.e4m3(w)[0]) == 1.125
    assert float(LPO.fp8_weight(w, 1.0)[0]) == 1.0
    # the scale itself is held in bf16: s = 3 exactly, s = 0.3 as bf16(0.3)
    w2 = np.array([0.9, -2.5, 1000.0], dtype=np.float32)
    s = float(round_bf16(np.float32(0.3)))
    want = LPO.e4m3(np.clip(round_bf16((w2.astype(np.float64) / s).astype(np.float32)), -448, 448))
    np.testing.assert_array_equal(LPO.fp8_weight(w2, 0.3), want)


def test_nvfp4_operand_is_grid_times_block_scale():
    rng = np.random.default_rng(3)
    x = round_bf16((rng.standard_normal((130, 96)) * np.exp(rng.uniform(-2, 2, (130, 1)))).astype(np.float32))
    ts = Q.per_tensor_amax_to_scale(float(np.abs(x).max()))
    xh = LPO.nvfp4_xhat(x, ts)
    q, s = Q.quantize(x, ts)
    s8 = Q.e4m3_decode(Q.unswizzle_scales(s, 130, 96)).astype(np.float64)       # [M, K/16]
    ratio = np.abs(xh.astype(np.float64)).reshape(130, 6, 16) / s8[:, :, None]
    assert np.all(np.isin(ratio, GRID.astype(np.float64)))
    # within half an e2m1 step (<= 1 at the top of the grid) of x / (ts s8)
    err = np.abs(x.astype(np.float64).reshape(130, 6, 16) / (ts * s8[:, :, None]) - ratio * np.sign(xh.reshape(130, 6, 16)))
    assert float(err.max()) <= 1.0 + 1e-6
    # the packed tensor dequantized with ts = x_hat * ts
    deq = Q.dequantize(q, s, ts, 130, 96)
    np.testing.assert_array_equal(deq, round_bf16((xh * np.float32(ts)).astype(np.float32)))


def test_fp4_raw_and_out_scale():
    rng = np.random.default_rng(4)
    x = round_bf16(rng.standard_normal((40, 64)).astype(np.float32))
    w = round_bf16((rng.standard_normal((48, 64)) * 0.02).astype(np.float32))
    sa, ws = Q.per_tensor_amax_to_scale(float(np.abs(x).max())), LPO.fp4_weight_scale(w)
    raw = LPO.fp4_raw(x, sa, w, ws)
    ref = torch.from_numpy(LPO.nvfp4_xhat(x, sa)).double() @ torch.from_numpy(LPO.nvfp4_xhat(w, ws)).double().T
    np.testing.assert_array_equal(raw, round_bf16(ref.float().numpy()))
    os_ = LPO.fp4_out_scale(sa, ws)
    assert os_ == float(torch.tensor(np.float32(sa) * np.float32(ws)).to(torch.bfloat16))


def test_fp8_linear_applies_both_scales_to_the_accumulator():
    rng = np.random.default_rng(5)
    x = round_bf16(rng.standard_normal((30, 64)).astype(np.float32))
    w = round_bf16((rng.standard_normal((32, 64)) * 0.02).astype(np.float32))
    b = round_bf16((rng.standard_normal(32) * 0.1).astype(np.float32))
    sa = LPO.fp8_act_scale(float(np.abs(x).max()))
    ws = LPO.fp8_weight_scale(w)
    got = LPO.fp8_linear(x, sa, w, ws, b)
    inv = round_bf16(np.float32(1.0) / sa)
    acc = LPO.fp8_act(x, inv).astype(np.float64) @ LPO.fp8_weight(w, ws).astype(np.float64).T
    want = round_bf16((acc * np.float64(np.float32(sa * ws)) + b).astype(np.float32))
    np.testing.assert_array_equal(got, want)
    # and it approximates the bf16 linear to FP8 precision
    full = x.astype(np.float64) @ w.astype(np.float64).T + b
    assert np.sqrt(((got - full) ** 2).mean() / (full ** 2).mean()) < 0.08


def test_scale_bias_single_rounding_and_layerscale():
    raw = np.array([1.0, -3.0, 0.5], dtype=np.float32)
    s = np.float32(0.1)
    b = np.array([0.25, 0.0, -0.05], dtype=np.float32)
    want = round_bf16((raw.astype(np.float64) * np.float64(s) + b).astype(np.float32))
    np.testing.assert_array_equal(LPO.scale_bias(raw, s, b), want)
    g = np.array([2.0, 0.5, -1.0], dtype=np.float32)
    np.testing.assert_array_equal(LPO.scale_bias(raw, s, b, g), round_bf16(want * g))


def test_swiglu_scaled_closed_forms():
    raw1 = np.array([0.0, 40.0, -40.0], dtype=np.float32)
    raw2 = np.array([3.0, 2.0, 5.0], dtype=np.float32)
    got = LPO.swiglu_scaled(raw1, 1.0, None, raw2, 1.0, None)
    assert got[0] == 0.0 and got[1] == 80.0 and abs(got[2]) < 1e-15
