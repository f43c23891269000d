"""Row gather / scatter and the residual reconstruct step, restated in numpy. Test infrastructure only.

Follows appcorr/models/dinov3/layers/triton_kernels/token_update.py:
  _gather_rows_kernel / gather_rows_triton     :371-387, 455-473   out[i] = src[b_i, t_i]
  _scatter_rows_kernel / scatter_rows_triton   :352-368, 417-452   dst[b_i, t_i] = src[i]
  _active_token_update_kernel                  :257-294            x_out[b_i, t_i] = a_i + d_i
  _fused_layerscale_add_kernel                 :10-41              x + attn * gamma
and the residual step of appcorr/models/dinov3/layers/block.py:1140-1179.

bf16 tensors are handled as uint16 bit arrays; arithmetic is done in fp32 and rounded to bf16
(round to nearest even) exactly where the reference materialises a bf16 tensor.
"""

from __future__ import annotations

import numpy as np

from .bf16 import bf16_bits_to_f32, f32_to_bf16_bits


def gather_rows(src: np.ndarray, b: np.ndarray, t: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(src[b, t])


def scatter_rows(dst: np.ndarray, b: np.ndarray, t: np.ndarray, src: np.ndarray) -> np.ndarray:
    out = dst.copy()
    out[b, t] = src
    return out


def active_token_update(x_base: np.ndarray, b, t, a: np.ndarray, d: np.ndarray) -> np.ndarray:
    out = x_base.copy()
    out[b, t] = f32_to_bf16_bits(bf16_bits_to_f32(a) + bf16_bits_to_f32(d))
    return out


def layerscale_add(x: np.ndarray, a: np.ndarray, g: np.ndarray) -> np.ndarray:
    """bf16(x + a * g) with one rounding (the product of two bf16 values is exact in fp64)."""
    xf = bf16_bits_to_f32(x).astype(np.float64)
    v = xf + bf16_bits_to_f32(a).astype(np.float64) * bf16_bits_to_f32(g).astype(np.float64)
    return f32_to_bf16_bits(v.astype(np.float32))


def reconstruct_scatter_persist(x, bos, b, t, x_act, x_attn, mlp):
    """block.py:1140-1179 on bit arrays: returns (x_out, new_blocks_out_sum)."""
    xo = f32_to_bf16_bits(bf16_bits_to_f32(x) + bf16_bits_to_f32(bos))
    a = bf16_bits_to_f32(x_attn)
    m = bf16_bits_to_f32(mlp)
    xo[b, t] = f32_to_bf16_bits(a + m)
    new_bos = bos.copy()
    inc = bf16_bits_to_f32(f32_to_bf16_bits(a - bf16_bits_to_f32(x_act)))
    new_bos[b, t] = f32_to_bf16_bits(inc + m)
    return xo, new_bos
