"""NVFP4 quantize / dequantize, restated in numpy. Test infrastructure only.

Follows appcorr/models/dinov3/layers/triton_kernels/nvfp4_fused.py:
  constants                      :48-50
  per-tile body (128 x 64)        :53-116
  buffer shapes and grid          :119-145
with the per-tensor scale convention of tests/test_nvfp4_fused_quantize.py:48
(ts = amax / (448 * 6), torchao's per_tensor_amax_to_scale).

Rounding choices where the reference delegates to code that cannot run here:
  * block scale: IEEE round-to-nearest division for amax/6 and for the division by ts
    (nvfp4_fused.py:88-89 use Triton's default '/', whose rounding is not pinned -- "parity
    unpinned"), then e4m3 round-to-nearest-even (:90).
  * data: IEEE division (tl.div_rn, :92), then e2m1 round-to-nearest-even with saturation to +-6,
    sign kept (torchao convert_fp32_to_fp4_packed, :109; nibble order: even element in the low
    nibble -- torchao's convention, "parity unpinned" here).
  * all-zero blocks divide 0 by 0; the result is NaN and its code is not pinned -- fixtures avoid it.

Both format conversions are done by nearest-value search over the enumerated code grid, an
arithmetic route independent of the bit manipulation the HIP kernel uses.
"""

from __future__ import annotations

import numpy as np

F4_E2M1_MAX = np.float32(6.0)
F8E4M3_MAX = np.float32(448.0)
E4M3_EPS = np.float32(1.5258789e-05)

# Positive e4m3fn values indexed by code 0..126 (0x7f is NaN).
E4M3_POS = np.array(
    [(m / 8.0) * 2.0**-6 if e == 0 else (1.0 + m / 8.0) * 2.0 ** (e - 7) for e in range(16) for m in range(8)][:127],
    dtype=np.float64,
)
# e2m1 magnitudes indexed by code 0..7.
E2M1_POS = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], dtype=np.float64)


def _nearest_even_code(a: np.ndarray, grid: np.ndarray) -> np.ndarray:
    """Code of the grid value nearest to a >= 0; ties go to the even code; above the top -> top."""
    a = np.asarray(a, dtype=np.float64)
    hi = np.searchsorted(grid, a, side="left")
    hi = np.clip(hi, 0, len(grid) - 1)
    lo = np.clip(hi - 1, 0, len(grid) - 1)
    d_lo = np.abs(a - grid[lo])
    d_hi = np.abs(grid[hi] - a)
    pick_hi = (d_hi < d_lo) | ((d_hi == d_lo) & (hi % 2 == 0))
    code = np.where(pick_hi, hi, lo)
    code = np.where(a >= grid[-1], len(grid) - 1, code)
    return code.astype(np.uint8)


def e4m3_encode(v: np.ndarray) -> np.ndarray:
    """Finite non-negative fp32 values (<= 448) -> e4m3fn codes, round to nearest even."""
    return _nearest_even_code(v, E4M3_POS)


def e4m3_decode(c: np.ndarray) -> np.ndarray:
    c = np.asarray(c, dtype=np.uint8)
    mag = E4M3_POS[np.minimum(c & 0x7F, 126)].astype(np.float32)
    return np.where(c & 0x80, -mag, mag).astype(np.float32)


def e2m1_encode(q: np.ndarray) -> np.ndarray:
    """fp32 values -> e2m1 codes (bit 3 = sign, kept for -0 and negatives rounding to 0)."""
    q = np.asarray(q, dtype=np.float32)
    mag = np.abs(q).astype(np.float64)
    code = _nearest_even_code(np.where(np.isnan(mag), np.inf, mag), E2M1_POS)
    sign = (q.view(np.uint32) >> 31).astype(np.uint8)
    return (code | (sign << 3)).astype(np.uint8)


def e2m1_decode(c: np.ndarray) -> np.ndarray:
    c = np.asarray(c, dtype=np.uint8)
    mag = E2M1_POS[c & 7].astype(np.float32)
    return np.where(c & 8, -mag, mag).astype(np.float32)


def per_tensor_amax_to_scale(amax: float) -> np.float32:
    return np.float32(np.float32(amax) / np.float32(F8E4M3_MAX * F4_E2M1_MAX))


def scale_numel(M: int, K: int) -> int:
    return -(-M // 128) * -(-K // 64) * 512


def quantize(x_f32: np.ndarray, ts: float):
    """x [M, K] (fp32 values of bf16 inputs) -> (qdata uint8 [M, K/2], scales uint8 [tiles * 512])."""
    x = np.asarray(x_f32, dtype=np.float32)
    M, K = x.shape
    assert K % 16 == 0
    ts = np.float32(ts)
    gm, gn = -(-M // 128), -(-K // 64)
    # Pad to whole tiles with zeros (the reference's masked load, nvfp4_fused.py:74-82).
    xp = np.zeros((gm * 128, gn * 64), dtype=np.float32)
    xp[:M, :K] = x
    blocks = xp.reshape(gm * 128, gn * 4, 16)
    amax = np.abs(blocks).max(axis=2)                                   # [rows, blocks]
    with np.errstate(divide="ignore", invalid="ignore"):
        bs = (amax / F4_E2M1_MAX).astype(np.float32)
        scaled = np.clip((bs / ts).astype(np.float32), E4M3_EPS, F8E4M3_MAX)
        s8 = e4m3_encode(scaled)
        total = (ts * e4m3_decode(s8)).astype(np.float32)
        qv = (blocks / total[:, :, None]).astype(np.float32)
    codes = e2m1_encode(qv).reshape(gm * 128, gn * 64)
    packed = (codes[:, 0::2] | (codes[:, 1::2] << 4)).astype(np.uint8)
    qdata = np.ascontiguousarray(packed[:M, : K // 2])
    # Scales of padding rows / blocks are stored as 0 (:94-96).
    rows = np.arange(gm * 128)[:, None]
    blk = np.arange(gn * 4)[None, :]
    s8 = np.where((rows < M) & (blk < K // 16), s8, 0).astype(np.uint8)
    # Tile (pm, pn) holds its [128, 4] scales as reshape(4, 32, 4).permute(1, 0, 2) -> [32, 16] (:98-107).
    tiles = s8.reshape(gm, 128, gn, 4).transpose(0, 2, 1, 3)            # [gm, gn, 128, 4]
    sw = tiles.reshape(gm, gn, 4, 32, 4).transpose(0, 1, 3, 2, 4).reshape(gm * gn * 512)
    return qdata, np.ascontiguousarray(sw)


def unswizzle_scales(scales: np.ndarray, M: int, K: int) -> np.ndarray:
    """Swizzled scale buffer -> [M, K/16] e4m3 codes (inverse of the tile permutation)."""
    gm, gn = -(-M // 128), -(-K // 64)
    t = np.asarray(scales, dtype=np.uint8).reshape(gm, gn, 32, 4, 4).transpose(0, 1, 3, 2, 4).reshape(gm, gn, 128, 4)
    full = t.transpose(0, 2, 1, 3).reshape(gm * 128, gn * 4)
    return full[:M, : K // 16]


def dequantize(qdata: np.ndarray, scales: np.ndarray, ts: float, M: int, K: int) -> np.ndarray:
    """fp32 values of bf16(fp32(e2m1 * e4m3) * ts), [M, K]."""
    q = np.asarray(qdata, dtype=np.uint8)
    codes = np.empty((M, K), dtype=np.uint8)
    codes[:, 0::2] = q & 0xF
    codes[:, 1::2] = q >> 4
    s = e4m3_decode(unswizzle_scales(scales, M, K))                     # [M, K/16]
    vals = (e2m1_decode(codes).reshape(M, K // 16, 16) * s[:, :, None]).astype(np.float32)
    vals = (vals * np.float32(ts)).astype(np.float32).reshape(M, K)
    from .bf16 import round_bf16

    return round_bf16(vals)
