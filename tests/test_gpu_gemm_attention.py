"""GPU numerics of the MFMA GEMM (every epilogue), LayerNorm, RoPE, the fused post-QKV step and the
sparse-query attention, against float64 references of the same ops rounded to bf16 at the
reference's points (oracle/model.py primitives).

Tolerance: results may differ from the fp64 oracle only through fp32 accumulation order, so every
element must be within 1 bf16 ulp of the oracle and only a small fraction may differ at all
(attention additionally rounds P to bf16 before P.V, as flash attention does: 2 ulps)."""

import math

import numpy as np
import pytest
import torch

from appcorr_amd import _lib
from appcorr_amd import kernels as K
from oracle import model as OM
from tests.util import assert_bf16_close, assert_bits_equal, bf16_ulp

pytestmark = pytest.mark.gpu

F64 = OM._F64


def _ref_linear(dev, x, w, b):
    """fp64 oracle linear evaluated on the device (fp64 GEMM), rounded to bf16 via fp32 on the host."""
    return F64.linear(x.to(dev), w.to(dev), None if b is None else b.to(dev)).cpu()


def _rand(shape, seed, std=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * std).to(torch.bfloat16)


U32 = 2.0 ** -24


def _check_gemm(dev, got, x, w, b, what):
    """|got - oracle| <= ulp(oracle) + 2 sqrt(K) u (|x| . |w|^T): the final bf16 rounding plus an fp32
    accumulation-order bound (u = 2^-24); at most 2% of elements may differ at all."""
    ref = _ref_linear(dev, x, w, b).double()
    mag = (x.to(dev).float().abs() @ w.to(dev).float().abs().T).double().cpu()
    bound = torch.from_numpy(bf16_ulp(ref.numpy())) + 2.0 * math.sqrt(x.shape[-1]) * U32 * mag
    diff = (got.detach().cpu().double() - ref).abs()
    bad = diff > bound
    assert not bad.any(), f"{what}: {int(bad.sum())} elements beyond bound, worst excess {float((diff - bound).max())}"
    frac = float((diff > 0).double().mean())
    assert frac <= 0.02, f"{what}: {frac:.3%} differ"


@pytest.mark.parametrize("M,N,Kd", [(4176, 3072, 1024), (4176, 1024, 1024), (4176, 4096, 1024), (4176, 1024, 4096),
                                    (103, 1152, 384), (1, 64, 64), (130, 192, 128), (1656, 8192, 4096),
                                    (1712, 3072, 1024), (1712, 4096, 1024), (8272, 3072, 1024), (8272, 4096, 1024),
                                    (1656, 12288, 4096), (1656, 4096, 4096), (1656, 4096, 8192),
                                    (414, 12288, 4096), (414, 4096, 4096), (414, 8192, 4096), (414, 4096, 8192),
                                    (1712, 1024, 1024), (2088, 768, 768), (8272, 1024, 1024), (8272, 1024, 4096),
                                    # approximate-pass grids (M = B N), several rounds of 288 x 256 tiles
                                    (16464, 4096, 1024), (16404, 8192, 4096), (16404, 4096, 4096)])
def test_linear_bias(dev, M, N, Kd):
    x, w, b = _rand((M, Kd), 1), _rand((N, Kd), 2, 0.02), _rand((N,), 3, 0.1)
    got = K.linear(x.to(dev), w.to(dev), b.to(dev))
    _check_gemm(dev, got, x, w, b, f"linear {M}x{N}x{Kd}")


@pytest.mark.parametrize("M", [1712, 4176, 8272])
def test_linear_repeatable_at_keep_ratios(dev, M):
    """The N = C projections (proj K = C, fc2 K = 4C) at the ViT-L row counts of keep 10 / 25 / 50 %
    (M = 16 (5 + k)): within the accumulation bound of the fp64 oracle, and repeated launches are
    bit-identical (fixed summation order, no atomics)."""
    for Kd in (1024, 4096):
        x, w, b = _rand((M, Kd), 30), _rand((1024, Kd), 31, 0.02), _rand((1024,), 32, 0.1)
        xd, wd, bd = x.to(dev), w.to(dev), b.to(dev)
        outs = [K.linear(xd, wd, bd) for _ in range(3)]
        _check_gemm(dev, outs[0], x, w, b, f"N=C GEMM {M}x1024x{Kd}")
        for o in outs[1:]:
            assert_bits_equal(o, outs[0], "repeat")


def test_linear_no_bias_and_strided_input(dev):
    x, w = _rand((300, 256), 4), _rand((128, 192), 5, 0.02)
    got = K.linear(x.to(dev)[:, 32:224], w.to(dev), None)
    _check_gemm(dev, got, x[:, 32:224].contiguous(), w, None, "strided")


# Epilogues: the plain GEMM (EPI_BIAS) is checked against the fp64 oracle above; each fused epilogue
# must then equal the oracle's epilogue applied to that same bf16(acc + bias), because it reads the
# identical fp32 accumulators. LayerScale and residual forms are exact in fp32 -> bit-exact; GELU and
# SiLU use fp32 transcendentals -> at most 1 ulp on at most 0.1% of elements.


def _epi_case(dev, M, N, Kd, seed):
    x, w, b = _rand((M, Kd), seed), _rand((N, Kd), seed + 1, 0.02), _rand((N,), seed + 2, 0.1)
    xd, wd, bd = x.to(dev), w.to(dev), b.to(dev)
    base = K.linear(xd, wd, bd)
    _check_gemm(dev, base, x, w, b, "epilogue base")
    return xd, wd, bd, base.cpu()


def test_linear_gelu(dev):
    xd, wd, bd, base = _epi_case(dev, 4176, 4096, 1024, 6)
    got = K.linear(xd, wd, bd, epilogue=_lib.EPI_BIAS_GELU)
    assert_bf16_close(got, F64.gelu(base), max_ulps=1, max_frac_off=1e-3, what="fc1+gelu")


def test_linear_layerscale_residual(dev):
    xd, wd, bd, base = _epi_case(dev, 4176, 1024, 1024, 9)
    g, r = _rand((1024,), 12), _rand((4176, 1024), 13)
    got = K.linear(xd, wd, bd, epilogue=_lib.EPI_BIAS_LS_RESID, gamma=g.to(dev), resid=r.to(dev))
    assert_bits_equal(got, F64.fma_add(r, base, g), "proj+ls+resid")


def test_linear_layerscale(dev):
    xd, wd, bd, base = _epi_case(dev, 4176, 1024, 4096, 14)
    g = _rand((1024,), 17)
    got = K.linear(xd, wd, bd, epilogue=_lib.EPI_BIAS_LS, gamma=g.to(dev))
    assert_bits_equal(got, F64.mul(base, g), "fc2+ls")


def test_linear_layerscale_residual_7b_proj(dev):
    """The ViT-7B proj (1656 x 4096 x 4096, 16-row-block 128 x 256 tiles): LayerScale + residual on the
    same accumulators as the plain GEMM, bit-exact."""
    assert "gemm_bf16_r16_kernel<128, 256, 2, 4, 1, 64, 3" in K.linear_kernel_name(1656, 4096, 4096,
                                                                                 _lib.EPI_BIAS_LS_RESID)
    xd, wd, bd, base = _epi_case(dev, 1656, 4096, 4096, 70)
    g, r = _rand((4096,), 73), _rand((1656, 4096), 74)
    got = K.linear(xd, wd, bd, epilogue=_lib.EPI_BIAS_LS_RESID, gamma=g.to(dev), resid=r.to(dev))
    assert_bits_equal(got, F64.fma_add(r, base, g), "7B proj + ls + resid")


@pytest.mark.parametrize("M,N,Kd", [(600, 1024, 512), (414, 8192, 4096), (1656, 8192, 4096)])
def test_linear_silu_mul(dev, M, N, Kd):
    xd, wd, bd, base = _epi_case(dev, M, N, Kd, 18)
    x2 = _rand((M, N), 21)
    got = K.linear(xd, wd, bd, epilogue=_lib.EPI_BIAS_SILU_MUL, resid=x2.to(dev))
    assert_bf16_close(got, F64.silu_mul(base, x2), max_ulps=1, max_frac_off=1e-3, what="swiglu")


# Split K: shapes whose tiles leave most CUs idle -- 144 x 128 tiles in two slices (ViT-L keep 10 %
# fc2, M = 1712; ViT-B fc2), 288 x 256 ping-pong tiles in two slices (ViT-7B w3, K = 8192) and a
# ViT-S-width product of 103 rows with a long K (16 slices). The
# partial tiles and the in-order fp32 sum of the slices stay within the accumulation bound; the
# epilogues read the same sums, so each equals the oracle's epilogue applied to the split GEMM's own
# bf16(acc + bias) (exactly, or to 1 ulp for GELU and SiLU).
SPLIT_SHAPES = [(1712, 1024, 4096), (2088, 768, 3072), (1656, 4096, 8192), (103, 384, 4096)]


@pytest.mark.parametrize("M,N,Kd", SPLIT_SHAPES)
def test_linear_split_k(dev, M, N, Kd):
    print(f"split-K GEMM {M}x{N}x{Kd}", flush=True)
    for epi in (_lib.EPI_BIAS, _lib.EPI_BIAS_LS, _lib.EPI_BIAS_LS_RESID, _lib.EPI_BIAS_GELU, _lib.EPI_BIAS_SILU_MUL):
        assert _lib.load().oudjat_linear_workspace_elems(M, N, Kd, epi) >= 2 * M * N
    xd, wd, bd, base = _epi_case(dev, M, N, Kd, 40)
    again = K.linear(xd, wd, bd)
    assert_bits_equal(again, base, "split-K repeat")
    g, r = _rand((N,), 44), _rand((M, N), 45)
    got = K.linear(xd, wd, bd, epilogue=_lib.EPI_BIAS_LS, gamma=g.to(dev))
    assert_bits_equal(got, F64.mul(base, g), "split-K + ls")
    got = K.linear(xd, wd, bd, epilogue=_lib.EPI_BIAS_LS_RESID, gamma=g.to(dev), resid=r.to(dev))
    assert_bits_equal(got, F64.fma_add(r, base, g), "split-K + ls + resid")
    got = K.linear(xd, wd, bd, epilogue=_lib.EPI_BIAS_GELU)
    assert_bf16_close(got, F64.gelu(base), max_ulps=1, max_frac_off=1e-3, what="split-K + gelu")
    got = K.linear(xd, wd, bd, epilogue=_lib.EPI_BIAS_SILU_MUL, resid=r.to(dev))
    assert_bf16_close(got, F64.silu_mul(base, r), max_ulps=1, max_frac_off=1e-3, what="split-K + swiglu")


@pytest.mark.parametrize("M,N,Kd", [(103, 384, 384), (103, 1536, 384), (103, 384, 768), (1, 64, 64), (300, 192, 192)])
def test_linear_tiny_grid(dev, M, N, Kd):
    """Grids of at most 32 tiles of 128 x 128 with K < 1024 (the ViT-S B = 1 proj and fc1; one row;
    three tile rows) run on 128 x 32 tiles: within the accumulation bound of the oracle, and every
    epilogue equals the oracle's epilogue applied to the same bf16(acc + bias). (With K >= 1024 and
    a workspace they split K instead: test_linear_split_k.)"""
    lib = _lib.load()
    for epi in (_lib.EPI_BIAS, _lib.EPI_BIAS_LS, _lib.EPI_BIAS_LS_RESID, _lib.EPI_BIAS_GELU, _lib.EPI_BIAS_SILU_MUL):
        assert lib.oudjat_linear_workspace_elems(M, N, Kd, epi) == 0
        assert "gemm_bf16_dma_kernel<128, 32, 4, 1" in K.linear_kernel_name(M, N, Kd, epi)
    xd, wd, bd, base = _epi_case(dev, M, N, Kd, 60)
    g, r = _rand((N,), 64), _rand((M, N), 65)
    got = K.linear(xd, wd, bd, epilogue=_lib.EPI_BIAS_LS, gamma=g.to(dev))
    assert_bits_equal(got, F64.mul(base, g), "tiny + ls")
    got = K.linear(xd, wd, bd, epilogue=_lib.EPI_BIAS_LS_RESID, gamma=g.to(dev), resid=r.to(dev))
    assert_bits_equal(got, F64.fma_add(r, base, g), "tiny + ls + resid")
    got = K.linear(xd, wd, bd, epilogue=_lib.EPI_BIAS_GELU)
    assert_bf16_close(got, F64.gelu(base), max_ulps=1, max_frac_off=1e-3, what="tiny + gelu")
    got = K.linear(xd, wd, bd, epilogue=_lib.EPI_BIAS_SILU_MUL, resid=r.to(dev))
    assert_bf16_close(got, F64.silu_mul(base, r), max_ulps=1, max_frac_off=1e-3, what="tiny + swiglu")


def test_linear_without_workspace_does_not_split(dev):
    """The C ABI without a workspace runs the one-launch kernel: same bound, and the workspace size
    query is 0 for a shape that fills the GPU."""
    M, N, Kd = 1712, 1024, 4096
    assert _lib.load().oudjat_linear_workspace_elems(4176, 4096, 1024, _lib.EPI_BIAS_GELU) == 0
    x, w, b = _rand((M, Kd), 50), _rand((N, Kd), 51, 0.02), _rand((N,), 52, 0.1)
    xd, wd, bd = x.to(dev), w.to(dev), b.to(dev)
    out = torch.empty(M, N, device=dev, dtype=torch.bfloat16)
    _lib.call("oudjat_linear_bf16", K._ptr(xd), M, Kd, Kd, K._ptr(wd), N, Kd, K._ptr(bd), _lib.EPI_BIAS, None, None, 0,
              K._ptr(out), N, 1.0, None, 0, K._stream(xd))
    _check_gemm(dev, out, x, w, b, "unsplit")


@pytest.mark.parametrize("rows,C", [(4176, 1024), (103, 384), (1656, 4096), (7, 8192), (5, 2048), (3, 1536),
                                    (9, 3072), (6, 1032)])
def test_layer_norm(dev, rows, C):
    """|got - oracle| <= ulp(oracle) + 64 u rstd |w| max|x_row| (fp32 statistics vs fp64). Rows wider than
    1024 run on 2 or 4 waves each (C = 1536, 2048: two; 3072, 4096, 8192: four; 1032 does not split
    evenly and stays on one), with row counts that leave rows past the end in the last workgroup."""
    x = (_rand((rows, C), 22).float() * 3 + 1).to(torch.bfloat16)
    w, b = _rand((C,), 23), _rand((C,), 24)
    got = K.layer_norm(x.to(dev), w.to(dev), b.to(dev), 1e-5).cpu().double()
    ref = F64.ln(x, w, b, 1e-5).double()
    xf = x.double()
    rstd = 1.0 / torch.sqrt(xf.var(-1, unbiased=False, keepdim=True) + 1e-5)
    bound = torch.from_numpy(bf16_ulp(ref.numpy())) + 64 * U32 * rstd * w.double().abs() * xf.abs().amax(-1, True)
    diff = (got - ref).abs()
    assert (diff <= bound).all(), float((diff - bound).max())
    assert float((diff > 0).double().mean()) <= 0.01


@pytest.mark.parametrize("rows,C,pf_elems,pf_dtype", [(4176, 1024, 4 << 20, torch.bfloat16),
                                                      (3, 1024, (1 << 20) + 7, torch.float32),
                                                      (103, 384, 31, torch.bfloat16),
                                                      (1656, 4096, 1 << 22, torch.bfloat16)])
def test_layer_norm_prefetch_is_the_same_layer_norm(dev, rows, C, pf_elems, pf_dtype):
    """Warming a region in the same launch leaves the output bits alone: regions of one line per lane,
    of many lines per lane (3 rows: a 4-wave grid), below one line, and of a ragged byte count."""
    x = (_rand((rows, C), 25).float() * 3 + 1).to(torch.bfloat16).to(dev)
    w, b = _rand((C,), 26).to(dev), _rand((C,), 27).to(dev)
    region = torch.ones(pf_elems, device=dev, dtype=pf_dtype)
    want = K.layer_norm(x, w, b, 1e-5)
    got = K.layer_norm(x, w, b, 1e-5, prefetch=region)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    assert bool((region == 1).all())  # read only


@pytest.mark.parametrize("M,N,Kd,epi,warm_elems", [(4176, 1024, 1024, _lib.EPI_BIAS_LS_RESID, 1 << 22),
                                                    (4176, 4096, 1024, _lib.EPI_BIAS_GELU, 3 << 20),
                                                    (4176, 1024, 4096, _lib.EPI_BIAS_LS, 1 << 20),
                                                    (1712, 4096, 1024, _lib.EPI_BIAS, 77),
                                                    (8272, 4096, 1024, _lib.EPI_BIAS_GELU, 1 << 22),
                                                    (414, 1024, 1024, _lib.EPI_BIAS, 1 << 20)])
def test_linear_warm_is_the_same_linear(dev, M, N, Kd, epi, warm_elems):
    """Warming workgroups (added to launches with fewer tiles than CUs: the headline's proj, fc1 and
    fc2 shapes) leave the product's bits alone; launches that fill the GPU or split K take none. The
    region (any size, here also below one line) is only read."""
    x = _rand((M, Kd), 50).to(dev)
    w = _rand((N, Kd), 51, 0.02).to(dev)
    b = _rand((N,), 52, 0.1).to(dev)
    g = _rand((N,), 53).to(dev)
    r = _rand((M, N), 54).to(dev)
    region = torch.ones(warm_elems, device=dev, dtype=torch.bfloat16)
    kw = dict(epilogue=epi, gamma=g if epi in (_lib.EPI_BIAS_LS, _lib.EPI_BIAS_LS_RESID) else None,
              resid=r if epi == _lib.EPI_BIAS_LS_RESID else None)
    want = K.linear(x, w, b, **kw)
    got = K.linear(x, w, b, warm=region, **kw)
    torch.cuda.synchronize()
    assert_bits_equal(got, want, "linear with warming workgroups")
    assert bool((region == 1).all())


def test_linear_qkv_rope_kv_warm_is_the_same(dev):
    """The fused QKV GEMM at the headline shape with a warm region: same q and K/V bits."""
    B, T, H, D, Kd, N = 16, 261, 16, 64, 1024, 1029
    M = B * T
    _, sin, cos, _, _, _ = _rope_inputs(1, H, D, 0)
    rng = np.random.default_rng(7)
    toks = np.stack([np.concatenate([np.arange(5), np.sort(rng.choice(np.arange(5, N), T - 5, replace=False))])
                     for _ in range(B)])
    tok = torch.from_numpy(toks.reshape(-1).astype(np.int64)).to(dev)
    bi = torch.arange(B).repeat_interleave(T).to(dev)
    pm, ri = tok >= 5, (tok - 5).clamp_min(0)
    x = _rand((M, Kd), 60).to(dev)
    w = _rand((3 * H * D, Kd), 61, 0.02).to(dev)
    b = _rand((3 * H * D,), 62, 0.1).to(dev)
    kv0 = _rand((B, N, 2, H, D), 63).to(dev)
    rope = (sin.to(dev), cos.to(dev))
    region = torch.ones(4 << 20, device=dev, dtype=torch.bfloat16)
    kv_a, q_a = kv0.clone(), torch.empty((M, H, D), dtype=torch.bfloat16, device=dev)
    K.linear_qkv_rope_kv(x, w, b, rope, pm, ri, bi, tok, kv_a, q_a)
    kv_b, q_b = kv0.clone(), torch.empty((M, H, D), dtype=torch.bfloat16, device=dev)
    K.linear_qkv_rope_kv(x, w, b, rope, pm, ri, bi, tok, kv_b, q_b, warm=region)
    torch.cuda.synchronize()
    assert_bits_equal(q_b, q_a, "q packed")
    assert_bits_equal(kv_b, kv_a, "kv cache")
    assert bool((region == 1).all())


def _rope_inputs(M, H, D, seed):
    cfg = OM.with_overrides(OM.CONFIGS["vitl16_512"], dim=H * D, heads=H)
    sin, cos = OM.rope_tables(cfg)
    rng = np.random.default_rng(seed)
    tok = torch.from_numpy(rng.integers(0, cfg.num_tokens, M).astype(np.int64))
    pm = tok >= 5
    ri = (tok - 5).clamp_min(0)
    return cfg, sin, cos, tok, pm, ri


def test_rope_active_inplace_bit_exact(dev):
    M, H, D = 4176, 16, 64
    cfg, sin, cos, tok, pm, ri = _rope_inputs(M, H, D, 0)
    qkv = _rand((M, 3, H, D), 25)
    qd = qkv.to(dev)
    K.apply_rope_active_inplace(qd[:, 0], qd[:, 1], (sin.to(dev), cos.to(dev)), pm.to(dev), ri.to(dev))
    s_sel, c_sel = sin[ri][:, None], cos[ri][:, None]
    ref = qkv.clone()
    ref[:, 0] = torch.where(pm[:, None, None], OM.rope_rotate(qkv[:, 0], s_sel, c_sel), qkv[:, 0])
    ref[:, 1] = torch.where(pm[:, None, None], OM.rope_rotate(qkv[:, 1], s_sel, c_sel), qkv[:, 1])
    assert_bits_equal(qd, ref, "rope in place (q, k rotated; v untouched)")


@pytest.mark.parametrize("B,T,H,D", [(16, 261, 16, 64), (2, 50, 32, 128)])
def test_qkv_rope_kv_scatter_bit_exact(dev, B, T, H, D):
    N = 1029
    M = B * T
    cfg, sin, cos, _, _, _ = _rope_inputs(1, H, D, 0)
    rng = np.random.default_rng(B)
    toks = np.stack([np.concatenate([np.arange(5), np.sort(rng.choice(np.arange(5, N), T - 5, replace=False))])
                     for _ in range(B)])
    tok = torch.from_numpy(toks.reshape(-1).astype(np.int64))
    bi = torch.arange(B).repeat_interleave(T)
    pm, ri = tok >= 5, (tok - 5).clamp_min(0)
    qkv = _rand((M, 3, H, D), 26)
    kv = _rand((B, N, 2, H, D), 27)
    kvd, qo = kv.to(dev), torch.empty((M, H, D), dtype=torch.bfloat16, device=dev)
    K.qkv_rope_kv_scatter(qkv.to(dev), (sin.to(dev), cos.to(dev)), pm.to(dev), ri.to(dev), bi.to(dev), tok.to(dev),
                          kvd, qo)
    s_sel, c_sel = sin[ri][:, None], cos[ri][:, None]
    q_ref = torch.where(pm[:, None, None], OM.rope_rotate(qkv[:, 0], s_sel, c_sel), qkv[:, 0])
    k_ref = torch.where(pm[:, None, None], OM.rope_rotate(qkv[:, 1], s_sel, c_sel), qkv[:, 1])
    kv_ref = kv.clone()
    kv_ref[bi, tok, 0] = k_ref
    kv_ref[bi, tok, 1] = qkv[:, 2]
    assert_bits_equal(qo, q_ref, "q packed")
    assert_bits_equal(kvd, kv_ref, "kv cache")


@pytest.mark.parametrize("B,T,H,D,Kd", [(16, 261, 16, 64, 1024), (1, 103, 6, 64, 384), (2, 50, 32, 128, 512),
                                        (16, 107, 16, 64, 1024), (16, 517, 16, 64, 1024), (4, 414, 32, 128, 4096),
                                        (1, 414, 32, 128, 4096), (16, 1029, 16, 64, 1024), (4, 1029, 32, 128, 4096)])
def test_linear_qkv_rope_kv_fused_equals_unfused(dev, B, T, H, D, Kd):
    """The fused QKV GEMM (qkv never materialised). Its raw bf16(acc + bias) values, taken from a run
    with no patch rows (no RoPE), are checked against the fp64 oracle like every GEMM; the pinned
    unfused RoPE kernel applied to those same values must then give the fused kernel's q and K/V
    bit-for-bit. (The fused launch may pick a different tile shape than `linear` for the same
    product, so the two GEMMs need not agree in the last bit.)"""
    N = 1029
    M = B * T
    _, sin, cos, _, _, _ = _rope_inputs(1, H, D, 0)
    rng = np.random.default_rng(B + H)
    toks = np.stack([np.concatenate([np.arange(5), np.sort(rng.choice(np.arange(5, N), T - 5, replace=False))])
                     for _ in range(B)])
    tok = torch.from_numpy(toks.reshape(-1).astype(np.int64)).to(dev)
    bi = torch.arange(B).repeat_interleave(T).to(dev)
    pm, ri = tok >= 5, (tok - 5).clamp_min(0)
    x = _rand((M, Kd), 40).to(dev)
    w = _rand((3 * H * D, Kd), 41, 0.02).to(dev)
    b = _rand((3 * H * D,), 42, 0.1).to(dev)
    kv0 = _rand((B, N, 2, H, D), 43).to(dev)
    rope = (sin.to(dev), cos.to(dev))
    assert K.qkv_fusable(H, D)
    kv_f, q_f = kv0.clone(), torch.empty((M, H, D), dtype=torch.bfloat16, device=dev)
    K.linear_qkv_rope_kv(x, w, b, rope, pm, ri, bi, tok, kv_f, q_f)
    kv_r, q_r = kv0.clone(), torch.empty((M, H, D), dtype=torch.bfloat16, device=dev)
    K.linear_qkv_rope_kv(x, w, b, rope, torch.zeros_like(pm), ri, bi, tok, kv_r, q_r)
    qkv_raw = torch.stack([q_r, kv_r[bi, tok, 0], kv_r[bi, tok, 1]], dim=1).contiguous()  # [M, 3, H, D]
    _check_gemm(dev, qkv_raw.view(M, 3 * H * D), x.cpu(), w.cpu(), b.cpu(), f"fused qkv GEMM {B}x{T}x{H}x{D}")
    kv_u, q_u = kv0.clone(), torch.empty((M, H, D), dtype=torch.bfloat16, device=dev)
    K.qkv_rope_kv_scatter(qkv_raw, rope, pm, ri, bi, tok, kv_u, q_u)
    assert_bits_equal(q_f, q_u, "q packed")
    assert_bits_equal(kv_f, kv_u, "kv cache")


def _check_attention(got, qb, kv, scale, ref, what):
    """P is rounded to bf16 before P.V (relative error <= 2^-9 per weight), so
    |got - oracle| <= 2 ulp(oracle) + 2^-8 * sum_j p_j |v_j|   (the second term from the oracle with |V|);
    and on average the error stays below 2^-10 of that magnitude (half of a bf16 P rounding)."""
    B, H, T, D = qb.shape
    mag = F64.sdpa(qb, kv[:, :, 0].transpose(1, 2), kv[:, :, 1].abs().transpose(1, 2), scale)
    mag = mag.transpose(1, 2).reshape(B * T, H * D).double()
    r = ref.double()
    bound = 2 * torch.from_numpy(bf16_ulp(r.numpy())) + 2.0 ** -8 * mag
    diff = (got.detach().cpu().double() - r).abs()
    assert (diff <= bound).all(), f"{what}: worst excess {float((diff - bound).max())}"
    rel = float(diff.mean() / mag.mean())
    assert rel <= 2.0 ** -10, f"{what}: mean error {rel:.3g} of mean sum p|v|"


@pytest.mark.parametrize("B,T,N,H,D", [(16, 261, 1029, 16, 64), (1, 103, 201, 6, 64), (2, 1029, 1029, 16, 64),
                                       (2, 7, 70, 4, 64), (1, 100, 4101, 32, 128), (3, 64, 64, 2, 64),
                                       (2, 269, 333, 4, 64), (1, 272, 1029, 3, 64), (1, 414, 4101, 32, 128),
                                       (4, 414, 4101, 32, 128)])
def test_sparse_query_attention(dev, B, T, N, H, D):
    q = _rand((B * T, H, D), 28)
    kv = _rand((B, N, 2, H, D), 29)
    scale = D ** -0.5
    got = K.sparse_query_attention(q.to(dev), kv.to(dev), T, scale)
    qb = q.reshape(B, T, H, D).transpose(1, 2)
    ref = F64.sdpa(qb, kv[:, :, 0].transpose(1, 2), kv[:, :, 1].transpose(1, 2), scale)
    ref = ref.transpose(1, 2).reshape(B * T, H * D)
    _check_attention(got, qb, kv, scale, ref, f"attention {B},{T},{N},{H},{D}")


@pytest.mark.parametrize("B,T,N,H,scale_up", [(16, 261, 1029, 16, 1.0), (2, 300, 777, 4, 1.0), (1, 256, 64, 3, 1.0),
                                               (2, 260, 65, 2, 1.0), (2, 261, 300, 2, 8.0), (16, 107, 1029, 16, 1.0),
                                               (16, 517, 1029, 16, 1.0), (2, 128, 1029, 4, 1.0), (2, 137, 1029, 4, 1.0),
                                               (2, 103, 201, 6, 8.0), (2, 261, 20, 2, 1.0), (1, 261, 40, 3, 8.0)])
def test_attention_buffer_load_kernel_shapes(dev, B, T, N, H, scale_up):
    """Dh = 64 with >= 8 waves runs the kernel that loads K/V tiles straight into LDS and reads V^T
    through LDS transpose reads, with the light last wave (T % 32 in 1..16: T = 261, 260, 300, 517)
    split over four waves by 16-key quarters of every tile (N = 20, 40: one tile whose last quarters
    hold no key, so those parts merge with nothing): one key tile, a ragged last tile of one key,
    10 waves, large logits, and
    the ViT-L keep-10 % / 50 % query counts (T = 107, 517); at few query waves (T = 103, 107, 128, 137)
    each full wave's key tiles are split over two waves and merged; all against the float64
    reference, and repeated launches are bit-identical."""
    D = 64
    q = (_rand((B * T, H, D), 40).float() * scale_up).to(torch.bfloat16)
    kv = (_rand((B, N, 2, H, D), 41).float() * scale_up).to(torch.bfloat16)
    got = K.sparse_query_attention(q.to(dev), kv.to(dev), T, D ** -0.5).cpu()
    qb = q.reshape(B, T, H, D).transpose(1, 2)
    o64 = F64.sdpa(qb, kv[:, :, 0].transpose(1, 2), kv[:, :, 1].transpose(1, 2), D ** -0.5)
    o64 = o64.transpose(1, 2).reshape(B * T, H * D)
    _check_attention(got, qb, kv, D ** -0.5, o64, f"attention {B},{T},{N},{H} x{scale_up}")
    again = K.sparse_query_attention(q.to(dev), kv.to(dev), T, D ** -0.5).cpu()
    assert_bits_equal(again, got, "repeat launch")


def _attention_call(entry, q, kv, B, T, H, N, out, *ws):
    lib = _lib.load()
    st = torch.cuda.current_stream().cuda_stream
    rc = getattr(lib, entry)(q.data_ptr(), q.stride(0), B, T, H, 64, kv.data_ptr(), kv.stride(0), kv.stride(1),
                             kv.stride(2), kv.stride(3), N, 64 ** -0.5, out.data_ptr(), out.stride(0), *ws, st)
    assert rc == 0, _lib.load().oudjat_last_error()


@pytest.mark.parametrize("B,T,N,H,scale_up", [(8, 261, 1029, 12, 1.0), (1, 103, 1029, 6, 1.0), (2, 300, 777, 4, 8.0),
                                               (1, 272, 577, 2, 1.0), (3, 107, 1029, 16, 1.0), (1, 5, 1029, 1, 1.0),
                                               (2, 32, 1100, 4, 1.0), (2, 256, 1029, 4, 1.0), (1, 33, 700, 3, 1.0),
                                               (2, 16, 900, 2, 1.0), (1, 261, 600, 2, 8.0)])
def test_attention_key_split(dev, B, T, N, H, scale_up):
    """Few (image, head) pairs with many key tiles (ViT-B at B = 8: 96 pairs of 17 tiles): the keys are
    dealt in contiguous tile ranges to several workgroups per pair, whose fp32 partials a second
    launch merges (with the light-wave split, the 16-query light wave, the two-wave split of few
    query waves, a ragged last tile of one key, and large logits inside the parts).
    Both the split and the unsplit kernel against the float64 reference with the same bound (each
    part rounds its probabilities to bf16 relative to its own running max, so the two differ by about
    a P rounding, which the bound covers); deterministic; and with a workspace one element short the
    entry runs the unsplit kernel bit for bit. Few key tiles (ViT-S: 197 keys) are not split."""
    D = 64
    lib = _lib.load()
    assert int(lib.oudjat_sparse_query_attention_workspace_elems(1, 103, 6, D, 197)) == 0
    elems = int(lib.oudjat_sparse_query_attention_workspace_elems(B, T, H, D, N))
    assert elems > 0, "this shape is expected to split its keys"
    q = (_rand((B * T, H, D), 44).float() * scale_up).to(torch.bfloat16).to(dev)
    kv = (_rand((B, N, 2, H, D), 45).float() * scale_up).to(torch.bfloat16).to(dev)
    got = K.sparse_query_attention(q, kv, T, D ** -0.5)
    qb = q.cpu().reshape(B, T, H, D).transpose(1, 2)
    kvc = kv.cpu()
    o64 = F64.sdpa(qb, kvc[:, :, 0].transpose(1, 2), kvc[:, :, 1].transpose(1, 2), D ** -0.5)
    o64 = o64.transpose(1, 2).reshape(B * T, H * D)
    _check_attention(got.cpu(), qb, kvc, D ** -0.5, o64, f"split attention {B},{T},{N},{H} x{scale_up}")
    plain = torch.empty_like(got)
    _attention_call("oudjat_sparse_query_attention", q, kv, B, T, H, N, plain)
    _check_attention(plain.cpu(), qb, kvc, D ** -0.5, o64, f"unsplit attention {B},{T},{N},{H} x{scale_up}")
    again = torch.empty_like(got)
    ws = torch.empty(elems, device=dev, dtype=torch.float32)
    _attention_call("oudjat_sparse_query_attention_ws", q, kv, B, T, H, N, again, ws.data_ptr(), elems)
    assert_bits_equal(again.cpu(), got.cpu(), "repeat launch")
    short = torch.empty_like(got)
    _attention_call("oudjat_sparse_query_attention_ws", q, kv, B, T, H, N, short, ws.data_ptr(), elems - 1)
    assert_bits_equal(short.cpu(), plain.cpu(), "workspace too small: unsplit kernel")


@pytest.mark.parametrize("B,T,N,H,scale_up", [(4, 414, 4101, 32, 1.0), (1, 7, 64, 2, 1.0), (2, 257, 65, 3, 1.0),
                                               (1, 300, 300, 4, 8.0), (2, 512, 1029, 2, 1.0), (1, 33, 129, 1, 1.0)])
def test_attention_dh128_shapes(dev, B, T, N, H, scale_up):
    """Dh = 128 (ViT-7B heads): the query waves spread over ceil(waves / 8) workgroups (T = 414: 7
    and 6 waves), one key tile, a ragged last tile of one key, one query wave, large logits; against
    the float64 reference, and repeated launches are bit-identical."""
    D = 128
    q = (_rand((B * T, H, D), 42).float() * scale_up).to(torch.bfloat16)
    kv = (_rand((B, N, 2, H, D), 43).float() * scale_up).to(torch.bfloat16)
    got = K.sparse_query_attention(q.to(dev), kv.to(dev), T, D ** -0.5).cpu()
    qb = q.reshape(B, T, H, D).transpose(1, 2)
    o64 = F64.sdpa(qb, kv[:, :, 0].transpose(1, 2), kv[:, :, 1].transpose(1, 2), D ** -0.5)
    o64 = o64.transpose(1, 2).reshape(B * T, H * D)
    _check_attention(got, qb, kv, D ** -0.5, o64, f"attention dh128 {B},{T},{N},{H} x{scale_up}")
    again = K.sparse_query_attention(q.to(dev), kv.to(dev), T, D ** -0.5).cpu()
    assert_bits_equal(again, got, "repeat launch")


def test_sparse_query_attention_peaked_softmax(dev):
    # Large logits: the online max rescaling must keep exp() in range.
    B, T, N, H, D = 2, 40, 300, 2, 64
    q = (_rand((B * T, H, D), 30).float() * 8).to(torch.bfloat16)
    kv = (_rand((B, N, 2, H, D), 31).float() * 8).to(torch.bfloat16)
    got = K.sparse_query_attention(q.to(dev), kv.to(dev), T, D ** -0.5)
    qb = q.reshape(B, T, H, D).transpose(1, 2)
    ref = F64.sdpa(qb, kv[:, :, 0].transpose(1, 2), kv[:, :, 1].transpose(1, 2), D ** -0.5)
    ref = ref.transpose(1, 2).reshape(B * T, H * D)
    _check_attention(got, qb, kv, D ** -0.5, ref, "peaked attention")
