"""Pins of the NVFP4 oracle (oracle/nvfp4.py) against facts fixed independently of it.

The reference's only test for this path (tests/test_nvfp4_fused_quantize.py) compares against
torchao on sm100 GPUs and cannot run here, so the oracle is pinned by:
  * e4m3 rounding vs torch's CPU float8_e4m3fn cast (an independent implementation);
  * e2m1 rounding at every grid point and midpoint, derived by hand from the OCP MX definition;
  * known-answer blocks whose bytes are derived by hand below;
  * a swizzle-placement check with one distinct scale per (row, block);
  * the dequantize round trip: per-element error within half a grid step, and the reference test's
    rel-L2 < 0.25 criterion (test_nvfp4_fused_quantize.py:107-109).
"""

import numpy as np
import pytest
import torch

from oracle import nvfp4 as Q
from oracle.bf16 import round_bf16


def test_e4m3_grid_matches_torch_float8():
    codes = np.arange(127, dtype=np.uint8)
    vals = torch.from_numpy(codes).view(torch.float8_e4m3fn).to(torch.float32).numpy()
    np.testing.assert_array_equal(Q.E4M3_POS.astype(np.float32), vals)


def test_e4m3_rounding_matches_torch_cast():
    rng = np.random.default_rng(0)
    v = np.concatenate([
        rng.uniform(2.0**-16, 448.0, 200000),
        np.exp(rng.uniform(np.log(2.0**-16), np.log(448.0), 200000)),
        # exact midpoints between neighbouring codes (ties -> even code)
        ((Q.E4M3_POS[1:] + Q.E4M3_POS[:-1]) / 2.0),
        Q.E4M3_POS[1:],
        [2.0**-10, 1.5 * 2.0**-9, 2.0**-16, 448.0],
    ]).astype(np.float32)
    v = np.clip(v, np.float32(2.0**-16), np.float32(448.0))
    ours = Q.e4m3_encode(v)
    ref = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(ours, ref)


@pytest.mark.parametrize("value,code", [
    (0.0, 0), (0.25, 0), (0.2500001, 1), (0.5, 1), (0.75, 2), (0.7499999, 1), (1.0, 2), (1.25, 2),
    (1.2500001, 3), (1.5, 3), (1.75, 4), (2.0, 4), (2.5, 4), (2.5000002, 5), (3.0, 5), (3.5, 6), (4.0, 6),
    (5.0, 6), (5.0000005, 7), (6.0, 7), (7.0, 7), (1e30, 7), (float("inf"), 7),
])
def test_e2m1_grid_and_midpoints(value, code):
    assert int(Q.e2m1_encode(np.float32(value))) == code
    assert int(Q.e2m1_encode(np.float32(-value))) == code | 8  # sign kept, -0 -> 0x8


def test_e2m1_negative_small_keeps_sign():
    assert int(Q.e2m1_encode(np.float32(-0.1))) == 0x8
    assert int(Q.e2m1_encode(np.float32(-0.0))) == 0x8


def test_known_answer_block_unit_scale():
    # ts = 1/6 and a block with amax 6: amax/6 = 1, 1/ts = 6 -> e4m3(6) = 6 exactly, total scale 1.
    # Then every grid value encodes to its own code.
    grid = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]
    row = np.array(grid + [-v for v in grid], dtype=np.float32)
    x = np.tile(row, (1, 4))                        # 1 row x 64 cols (4 blocks)
    ts = np.float32(1.0) / np.float32(6.0)
    qd, sc = Q.quantize(x, ts)
    # scale: (6/6) / (1/6) = 6.0000005 in fp32 -> e4m3 nearest is 6.0 = code 0x4C (e=9, m=4)
    assert Q.e4m3_encode(np.float32(6.0)) == 0x4C
    s = Q.unswizzle_scales(sc, 1, 64)
    assert s.shape == (1, 4) and (s == 0x4C).all()
    codes = [0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15]
    expected = bytes((codes[2 * i] | (codes[2 * i + 1] << 4)) for i in range(8))
    assert qd[0, :8].tobytes() == expected        # low nibble = even element
    assert (qd[0].reshape(4, 8) == qd[0, :8]).all()


def test_known_answer_scale_and_rounding():
    # Block amax 3.0, ts = 0.25: bs = 0.5, sc = 2.0 (e4m3 exact) -> total 0.5; x = 0.6 -> 1.2 -> 1.0 (code 2);
    # x = 0.65 -> 1.3 -> 1.5 (code 3); x = 3 -> 6 (code 7); x = -1.25 -> -2.5 -> tie -> 2 (code 0xC).
    x = np.zeros((1, 16), dtype=np.float32)
    x[0, :4] = [0.6, 0.65, 3.0, -1.25]
    x = round_bf16(x)  # inputs are bf16 values
    qd, sc = Q.quantize(x, np.float32(0.25))
    assert Q.unswizzle_scales(sc, 1, 16)[0, 0] == Q.e4m3_encode(np.float32(2.0))
    codes = np.concatenate([qd[0] & 0xF, qd[0] >> 4])  # even elements then odd
    even, odd = qd[0] & 0xF, qd[0] >> 4
    assert even[0] == Q.e2m1_encode(round_bf16(np.float32(0.6)) / np.float32(0.5))
    assert (even[0], odd[0], even[1], odd[1]) == (2, 3, 7, 0xC)
    assert codes is not None


def test_swizzle_placement_unique_scales():
    # One row-block pair per distinct amax so every scale byte is distinct; check the tile layout
    # byte (r % 32) * 16 + (r // 32) * 4 + j of tile (pm, pn) holds the scale of row pm*128+r, block pn*4+j.
    M, K = 130, 128
    x = np.zeros((M, K), dtype=np.float32)
    rng = np.random.default_rng(1)
    amax = rng.permutation(M * (K // 16)).reshape(M, K // 16).astype(np.float32)
    x[:, ::16] = (amax * 0.01 + 0.5)
    ts = np.float32(0.01)
    qd, sc = Q.quantize(round_bf16(x), ts)
    full = Q.unswizzle_scales(sc, M, K)
    gn = K // 64
    for r in range(M):
        for jb in range(K // 16):
            pm, pn, rr, j = r // 128, jb // 4, r % 128, jb % 4
            byte = sc[(pm * gn + pn) * 512 + (rr % 32) * 16 + (rr // 32) * 4 + j]
            assert byte == full[r, jb]
    # padding rows of the last row-tile have scale 0
    tile = sc[1 * gn * 512:].reshape(gn, 32, 4, 4)      # [pn, r%32, r//32, j]
    rows_pad = [(rr % 32, rr // 32) for rr in range(2, 128)]
    assert all((tile[:, a, b, :] == 0).all() for a, b in rows_pad)


def test_roundtrip_error_bounds():
    rng = np.random.default_rng(2)
    M, K = 256, 256
    x = rng.standard_normal((M, K)).astype(np.float32)
    out_idx = rng.random((M, K)) < 0.01
    x[out_idx] *= 50.0
    x = round_bf16(x)
    ts = Q.per_tensor_amax_to_scale(np.abs(x).max())
    qd, sc = Q.quantize(x, ts)
    xh = Q.dequantize(qd, sc, ts, M, K)
    s = Q.e4m3_decode(Q.unswizzle_scales(sc, M, K)).repeat(16, axis=1) * ts
    # |x - xhat| <= half the largest grid gap (1.0 between 4 and 6) * block scale, plus bf16 rounding
    assert (np.abs(x - xh) <= 1.0 * s + np.abs(xh) * 2.0**-8 + 1e-30).all()
    rel = np.linalg.norm(x - xh) / np.linalg.norm(x)
    assert rel < 0.25


def test_masked_tail_shapes():
    x = round_bf16(np.random.default_rng(3).standard_normal((5, 48)).astype(np.float32))
    qd, sc = Q.quantize(x, Q.per_tensor_amax_to_scale(np.abs(x).max()))
    assert qd.shape == (5, 24)
    assert sc.shape == (Q.scale_numel(5, 48),) == (512,)
    full = Q.unswizzle_scales(sc, 5, 48)
    assert full.shape == (5, 3)
    # block 3 of each row is padding (K/16 = 3) -> 0; rows >= 5 -> 0
    t = sc.reshape(32, 4, 4)
    assert (t[:, :, 3] == 0).all()
    assert (t[5:, 0, :] == 0).all() and (t[:, 1:, :] == 0).all()
