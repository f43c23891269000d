"""GPU parity of the low-precision correction linears (appcorr_amd/dinov3/lowp.py) against oracle/lowp.py.

Kernels (identical inputs):
  * the NVFP4 operand x_hat and its packed bytes: bit-exact, and the bytes equal oudjat_nvfp4_quantize's;
  * the FP8 operand in both rounding modes: bit-exact;
  * the NVFP4 scale-and-bias (+ LayerScale) epilogue: bit-exact; the fused SwiGLU epilogue: at most one
    bf16 ulp on at most 0.1 % of elements (fp32 exp and division);
  * the calibration amax: exact, NaN propagating;
  * the FP8 GEMM (quantized operands, scales on the accumulator) and the NVFP4 GEMM: within the fp32
    accumulation bound of the exact oracle.
Block (a SwiGLU block driven through DINOv3CorrectPrecisionController): the calibration event runs the
exact bf16 block and observes every linear's input; after the freeze the block runs NVFP4 / FP8 and is
compared with the oracle block run with the controller's frozen activation scales. Upstream last-bit
differences can move an input across an e2m1 / e4m3 rounding boundary, so that comparison is
statistical: the GPU's distance from the oracle must be a small fraction (1/10) of the distance the
low-precision route itself puts between the oracle and the bf16 block.
"""

import math

import numpy as np
import pytest
import torch
from torch import nn

from appcorr_amd import _lib
from appcorr_amd import kernels as K
from appcorr_amd.dinov3 import SelfAttentionBlock
from appcorr_amd.dinov3 import lowp as LP
from appcorr_amd.server.precision import DINOv3CorrectPrecisionController
from oracle import lowp as LPO
from oracle import model as OM
from oracle import nvfp4 as Q
from oracle import plan as OP
from oracle.bf16 import round_bf16
from tests.util import assert_bf16_close, assert_bits_equal, bf16_ulp, close_stats

pytestmark = pytest.mark.gpu

U32 = 2.0 ** -24


def _x(shape, seed, outliers=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(shape, generator=g)
    if outliers:
        m = torch.rand(shape, generator=g) < 0.01
        x = torch.where(m, x * 50, x)
    return x.to(torch.bfloat16)


@pytest.mark.parametrize("M,Kd", [(1656, 4096), (414, 8192), (300, 64), (129, 1024)])
def test_nvfp4_operand_bit_exact(dev, M, Kd):
    x = _x((M, Kd), M)
    ts = torch.tensor(Q.per_tensor_amax_to_scale(float(x.float().abs().max())))
    xh, q, s = K.nvfp4_quantize_dequantize(x.to(dev), ts.to(dev), packed=True)
    torch.cuda.synchronize()
    ref = LPO.nvfp4_xhat(x.float().numpy(), float(ts))
    assert_bits_equal(xh, torch.from_numpy(ref).to(torch.bfloat16), "x_hat")
    q2, s2 = K.quantize_nvfp4_swizzled(x.to(dev), ts.to(dev))
    assert_bits_equal(q, q2, "qdata")
    assert torch.equal(s.view(torch.uint8).cpu(), s2.view(torch.uint8).cpu())
    assert_bits_equal(K.nvfp4_quantize_dequantize(x.to(dev), ts.to(dev)), xh, "x_hat without the packed outputs")


@pytest.mark.parametrize("M,Kd", [(1656, 4096), (37, 64)])
def test_fp8_operand_bit_exact(dev, M, Kd):
    x = _x((M, Kd), M + 1)
    sa = LPO.fp8_act_scale(float(x.float().abs().max()) * 0.5)    # part of the tensor saturates
    inv = float(round_bf16(np.float32(1.0) / sa))
    got = K.fp8_quantize_dequantize(x.to(dev), torch.tensor([inv], device=dev), K.FP8_ACTIVATION)
    ref = LPO.fp8_act(x.float().numpy(), inv)
    assert_bits_equal(got, torch.from_numpy(ref).to(torch.bfloat16), "fp8 activation")
    w = (x.float() * 0.02).to(torch.bfloat16)
    ws = LPO.fp8_weight_scale(w.float().numpy())
    got_w = K.fp8_quantize_dequantize(w.to(dev), torch.tensor([float(ws)], device=dev), K.FP8_WEIGHT)
    ref_w = LPO.fp8_weight(w.float().numpy(), ws)
    assert_bits_equal(got_w, torch.from_numpy(ref_w).to(torch.bfloat16), "fp8 weight")


def test_scale_bias_and_swiglu_epilogues(dev):
    M, N = 414, 8192
    r1, r2 = _x((M, N), 7, False), _x((M, N), 8, False)
    b1, b2, g = _x((N,), 9, False), _x((N,), 10, False), _x((N,), 11, False)
    s1, s2 = 0.0123, 3.7e-3
    for bias, gamma in ((None, None), (b1, None), (b1, g), (None, g)):
        got = K.scale_bias(r1.to(dev), s1, None if bias is None else bias.to(dev), None if gamma is None else gamma.to(dev))
        ref = LPO.scale_bias(r1.float().numpy(), s1, None if bias is None else bias.float().numpy(),
                             None if gamma is None else gamma.float().numpy())
        assert_bits_equal(got, torch.from_numpy(ref).to(torch.bfloat16), f"scale_bias bias={bias is not None}")
    x1 = r1.to(dev).clone()
    out = K.swiglu_scaled(x1, s1, b1.to(dev), r2.to(dev), s2, b2.to(dev))
    assert out.data_ptr() == x1.data_ptr()
    ref = LPO.swiglu_scaled(r1.float().numpy(), s1, b1.float().numpy(), r2.float().numpy(), s2, b2.float().numpy())
    assert_bf16_close(out, torch.from_numpy(ref), max_ulps=1, max_frac_off=1e-3, what="swiglu")


def test_amax_update(dev):
    x = _x((1000, 64), 12)
    a = torch.zeros((), device=dev)
    K.amax_update(x.to(dev), a)
    assert float(a) == float(x.float().abs().max())
    K.amax_update((x.float() * 0.5).to(torch.bfloat16).to(dev), a)   # smaller: unchanged
    assert float(a) == float(x.float().abs().max())
    y = x.clone()
    y[3, 5] = float("nan")
    K.amax_update(y.to(dev), a)
    assert math.isnan(float(a))


def test_scale_division_is_torchs(dev):
    """The reference's per-tensor scales divide a device tensor by a Python float (amax / 2688 in
    torchao's per_tensor_amax_to_scale, amax / 448 in FastFP8Linear): oracle.lowp.cuda_scalar_div (times
    the fp32 reciprocal) equals torch's own device division bit for bit; the IEEE quotient does not
    always (so the check tells the two apart)."""
    g = torch.Generator().manual_seed(21)
    n = 200000
    a = torch.rand(n, generator=g) * torch.exp2(torch.randint(-20, 10, (n,), generator=g).float())
    for b in (448.0 * 6.0, 448.0):
        got = (a.to(dev) / b).cpu().numpy()
        ref = LPO.cuda_scalar_div(a.numpy(), b)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), b
        assert (ref != (a.numpy() / np.float32(b)).astype(np.float32)).any(), b


def _gemm_bound(got, ref, mag, K_):
    d = (got.double() - ref.double()).abs()
    bound = torch.from_numpy(bf16_ulp(ref.double().numpy())) + 2.0 * math.sqrt(K_) * U32 * mag
    assert bool((d <= bound).all()), float((d - bound).max())


def test_fp8_and_fp4_gemms(dev):
    M, Kd, N = 414, 4096, 1024
    x = _x((M, Kd), 13, False)
    w = (_x((N, Kd), 14, False).float() * 0.02).to(torch.bfloat16)
    b = (_x((N,), 15, False).float() * 0.1).to(torch.bfloat16)
    # FP8: the GEMM's accumulator scale
    sa, ws = LPO.fp8_act_scale(float(x.float().abs().max())), LPO.fp8_weight_scale(w.float().numpy())
    inv = float(round_bf16(np.float32(1.0) / sa))
    xq = K.fp8_quantize_dequantize(x.to(dev), torch.tensor([inv], device=dev))
    wq = K.fp8_quantize_dequantize(w.to(dev), torch.tensor([float(ws)], device=dev), K.FP8_WEIGHT)
    alpha = float(np.float32(sa * ws))
    got = K.linear(xq, wq, b.to(dev), acc_scale=alpha).cpu()
    ref = torch.from_numpy(LPO.fp8_linear(x.float().numpy(), sa, w.float().numpy(), ws, b.float().numpy()))
    mag = (xq.float().abs() @ wq.float().abs().T).double().cpu() * alpha
    _gemm_bound(got, ref, mag, Kd)
    # NVFP4: raw GEMM of the exact operands
    sa4 = Q.per_tensor_amax_to_scale(float(x.float().abs().max()))
    ws4 = LPO.fp4_weight_scale(w.float().numpy())
    xh = K.nvfp4_quantize_dequantize(x.to(dev), torch.tensor([float(sa4)], device=dev))
    wh = K.nvfp4_quantize_dequantize(w.to(dev), torch.tensor([float(ws4)], device=dev))
    raw = K.linear(xh, wh, None).cpu()
    ref4 = torch.from_numpy(LPO.fp4_raw(x.float().numpy(), sa4, w.float().numpy(), ws4))
    _gemm_bound(raw, ref4, (xh.float().abs() @ wh.float().abs().T).double().cpu(), Kd)


def test_fp8_codes_are_the_operand_values(dev):
    """oudjat_fp8_quantize's bytes are the e4m3fn codes of exactly the values fp8_quantize_dequantize
    gives (both modes, saturation, signed zeros, NaN)."""
    x = _x((1656, 4096), 31)
    x[0, :4] = torch.tensor([0.0, -0.0, float("nan"), -1e9])
    inv = torch.tensor([float(round_bf16(np.float32(448.0) / np.float32(30.0)))], device=dev)
    for mode, scale in ((K.FP8_ACTIVATION, inv), (K.FP8_WEIGHT, torch.tensor([0.037], device=dev))):
        codes = K.fp8_quantize(x.to(dev), scale, mode)
        vals = K.fp8_quantize_dequantize(x.to(dev), scale, mode)
        dec = codes.view(torch.float8_e4m3fn).float()
        same = (dec == vals.float()) | (torch.isnan(dec) & torch.isnan(vals.float()))
        assert bool(same.all()), mode
        signs = (codes >> 7).bool() == torch.signbit(vals.float())
        assert bool((signs | torch.isnan(vals.float())).all()), mode


@pytest.mark.parametrize("B,T,H,N", [(4, 414, 32, 4101), (2, 50, 4, 300), (1, 7, 2, 70)])
def test_attention_fp8_codes_equal_quantize_after(dev, B, T, H, N):
    """The attention writing the FP8 proj's activation codes itself equals the bf16 attention followed
    by fp8_quantize (FastFP8Linear's activation mode), byte for byte; Dh = 128 (the ViT-7B heads)."""
    g = torch.Generator().manual_seed(B * T + N)
    D = 128
    q = (torch.randn(B * T, H, D, generator=g) * 2).to(torch.bfloat16).to(dev)
    kv = (torch.randn(B, N, 2, H, D, generator=g) * 2).to(torch.bfloat16).to(dev)
    inv = torch.tensor([float(round_bf16(np.float32(448.0) / np.float32(3.0)))], device=dev)
    want = K.fp8_quantize(K.sparse_query_attention(q, kv, T, D ** -0.5), inv, K.FP8_ACTIVATION)
    got = K.sparse_query_attention_fp8(q, kv, T, D ** -0.5, inv)
    torch.cuda.synchronize()
    assert got.dtype == torch.uint8 and got.shape == want.shape
    assert torch.equal(got, want)


@pytest.mark.parametrize("M,N,Kd,epi", [
    (1656, 12288, 4096, _lib.EPI_BIAS),          # the ViT-7B qkv shape (plain epilogue)
    (1656, 4096, 4096, _lib.EPI_BIAS_LS_RESID),  # proj
    (1656, 8192, 4096, _lib.EPI_BIAS_SILU_MUL),  # w1 with the w2 gate
    (1656, 4096, 8192, _lib.EPI_BIAS_LS),        # w3
    (37, 256, 128, _lib.EPI_BIAS),               # one ragged tile
    (300, 768, 384, _lib.EPI_BIAS_LS),
])
def test_native_fp8_gemm(dev, M, N, Kd, epi):
    """The FP8 MFMA GEMM on e4m3 codes against (a) the bf16 MFMA GEMM on the codes' exact bf16 values --
    the same exact products, fp32 sums in another order -- and (b) the exact oracle, both within the fp32
    accumulation bound; the kernel is the one linear_fp8_kernel_name names."""
    print(f"fp8 gemm M={M} N={N} K={Kd} epi={epi}: {K.linear_fp8_kernel_name(M, N, Kd, epi)}", flush=True)
    x = _x((M, Kd), 41, False)
    w = (_x((N, Kd), 42, False).float() * 0.02).to(torch.bfloat16)
    b = (_x((N,), 43, False).float() * 0.1).to(torch.bfloat16)
    gam = (_x((N,), 44, False).float() * 0.5).to(torch.bfloat16).to(dev)
    side = _x((M, N), 45, False).to(dev)
    sa, ws = LPO.fp8_act_scale(float(x.float().abs().max())), LPO.fp8_weight_scale(w.float().numpy())
    inv = torch.tensor([float(round_bf16(np.float32(1.0) / sa))], device=dev)
    wst = torch.tensor([float(ws)], device=dev)
    x8, w8 = K.fp8_quantize(x.to(dev), inv), K.fp8_quantize(w.to(dev), wst, K.FP8_WEIGHT)
    xq, wq = K.fp8_quantize_dequantize(x.to(dev), inv), K.fp8_quantize_dequantize(w.to(dev), wst, K.FP8_WEIGHT)
    alpha = float(np.float32(sa * ws))
    kw = {}
    if epi in (_lib.EPI_BIAS_LS, _lib.EPI_BIAS_LS_RESID):
        kw["gamma"] = gam
    if epi in (_lib.EPI_BIAS_LS_RESID, _lib.EPI_BIAS_SILU_MUL):
        kw["resid"] = side
    got = K.linear_fp8(x8, w8, b.to(dev), acc_scale=alpha, epilogue=epi, **kw).cpu()
    via_bf16 = K.linear(xq, wq, b.to(dev), acc_scale=alpha, epilogue=epi, **kw).cpu()
    torch.cuda.synchronize()
    mag = (xq.float().abs() @ wq.float().abs().T).double().cpu() * alpha
    if epi == _lib.EPI_BIAS:
        ref = torch.from_numpy(LPO.fp8_linear(x.float().numpy(), sa, w.float().numpy(), ws, b.float().numpy()))
        for name, t in (("fp8 mfma", got), ("bf16 mfma", via_bf16)):
            e = ((t.double() - ref.double()).abs() - torch.from_numpy(bf16_ulp(ref.double().numpy()))).clamp(min=0)
            print(f"  {name}: max accumulation error beyond one output ulp = {float((e / (U32 * mag)).max()):.2f} u*mag",
                  flush=True)
        # The worst case of fp32 accumulation in any order, K u mag (the MFMA's internal order of the
        # 128 products of one instruction is not specified), plus one rounding of the output.
        _gemm_bound(got, ref, mag * math.sqrt(Kd) / 2.0, Kd)
        _gemm_bound(via_bf16, ref, mag, Kd)
    # every epilogue: the two routes agree to the accumulation bound carried through the epilogue's
    # factor (gamma, the gate or 1) plus one rounding of the result
    fac = torch.ones(N, dtype=torch.float64)
    if "gamma" in kw:
        fac = kw["gamma"].double().abs().cpu()
    mult = fac.expand(M, N).clone()
    if epi == _lib.EPI_BIAS_SILU_MUL:
        mult = mult * side.double().abs().cpu() * 1.2
    d = (got.double() - via_bf16.double()).abs()
    bound = (torch.from_numpy(bf16_ulp(via_bf16.double().numpy())) * 2
             + mult * (2.0 * math.sqrt(Kd) * U32 * mag + torch.from_numpy(bf16_ulp(mag.numpy()))))
    assert bool((d <= bound).all()), float((d - bound).max())
    frac = float((got != via_bf16).float().mean())
    assert frac <= 0.05, frac


def _swiglu_cfg():
    # the ViT-7B block structure (SwiGLU, 128-wide heads, no qkv bias) at a width the oracle runs quickly
    return OM.with_overrides(OM.CONFIGS["vit7b16_1024"], dim=512, heads=4, ffn_hidden=1024, img_size=224, depth=1)


@pytest.mark.parametrize("precision", ["fp4", "fp8"])
def test_swiglu_block_through_the_controller(dev, precision):
    _controller_block(dev, precision, _swiglu_cfg(), 2, 0.25)


# The tiles the ViT-7B fp4 / fp8 passes launch at B = 4, keep 10 % (M = 1656 selected rows): the fused
# QKV on 192 x 256 ping-pong tiles (whole 128-wide heads), proj on 16-row-block 128 x 256 tiles, w1 / w2
# on 224 x 256 ping-pong tiles and w3 in two K slices of 288 x 256 ping-pong tiles (split K).
_VIT7B_TILES = {
    (1656, 12288, 4096, 5): "oudjat::gemm_bf16_pp_kernel<224, 384, 5>",  # 5: the fused QKV kernel
    (1656, 4096, 4096, _lib.EPI_BIAS_LS_RESID): "oudjat::gemm_bf16_r16_kernel<128, 256, 2, 4, 1, 64, 3, false, 2>",
    (1656, 8192, 4096, _lib.EPI_BIAS_SILU_MUL): "oudjat::gemm_bf16_pp_kernel<224, 256, 4>",
    (1656, 8192, 4096, _lib.EPI_BIAS): "oudjat::gemm_bf16_pp_kernel<224, 256, 0>",
    (1656, 4096, 8192, _lib.EPI_BIAS_LS): "oudjat::gemm_bf16_pp_kernel<288, 256, 6>",
    (1656, 4096, 8192, _lib.EPI_BIAS): "oudjat::gemm_bf16_pp_kernel<288, 256, 6>",
}


@pytest.mark.timeout(900)
@pytest.mark.parametrize("precision", ["fp4", "fp8"])
def test_vit7b_width_block_through_the_controller(dev, precision):
    """The controller block at the ViT-7B width and batch (C = 4096, 32 heads of 128, SwiGLU hidden 8192,
    1024 px: N = 4101, B = 4, keep 10 %): the FP8 accumulator scales and the NVFP4 operands run
    through the GEMM tile configurations the 7B passes use."""
    for (M, N_, K_, epi), name in _VIT7B_TILES.items():
        assert K.linear_kernel_name(M, N_, K_, epi) == name, (M, N_, K_, epi)
    cfg = OM.with_overrides(OM.CONFIGS["vit7b16_1024"], depth=1)
    _controller_block(dev, precision, cfg, 4, 0.1)


def _controller_block(dev, precision, cfg, B, ratio):
    N, C, H, D, P = cfg.num_tokens, cfg.dim, cfg.heads, cfg.head_dim, cfg.num_patches
    print(f"low-precision block {precision}: C={C} H={H}x{D} hidden={cfg.ffn_hidden} B={B} N={N}", flush=True)
    w = OM.make_block_weights(cfg, 0, gamma=1.0, bias_std=0.05, ln_std=0.1, depth=1)[0]
    blk = SelfAttentionBlock(C, H, ffn_ratio=cfg.ffn_hidden / C * 1.5, qkv_bias=False, init_values=1.0,
                             ffn_layer="swiglu64", mask_k_bias=True)
    blk.load_state_dict(w, strict=True)
    blk = blk.to(device=dev, dtype=torch.bfloat16)
    g = torch.Generator().manual_seed(6)
    x = torch.randn(B, N, C, generator=g).to(torch.bfloat16)
    cache = {"layer0_kv": torch.randn(B, N, 2, H, D, generator=g).to(torch.bfloat16),
             "layer0_blocks_out_sum": (torch.randn(B, N, C, generator=g) * 0.1).to(torch.bfloat16)}
    imp = torch.rand(B, P, generator=g)
    rope = OM.rope_tables(cfg)
    r = (rope[0].to(dev), rope[1].to(dev))
    dind = OM.full_dindice(cfg, B)
    kw = dict(token_keep_ratio=ratio, mobile_pscore="residual_energy", mobile_pscore_weight=1.0,
              mobile_pscore_hint=imp.to(dev), server_pscore_weight=0.0)
    ctrl = DINOv3CorrectPrecisionController(nn.ModuleList([blk]), precision=precision, device=dev)
    assert ctrl.calibrating

    def run():
        c = {k: v.to(dev).clone() for k, v in cache.items()}
        with torch.no_grad():
            out, c = ctrl.run_block(0, x.to(dev), dind.to(dev), r, c, "layer0", **kw)
        torch.cuda.synchronize()
        return out.cpu(), c

    ctrl.begin_event()                                   # calibration event: exact bf16 + observers
    x_cal, _ = run()
    with torch.no_grad():
        x_bf, _ = blk.correct(x.to(dev), dind.to(dev), r, {k: v.to(dev).clone() for k, v in cache.items()}, "layer0",
                              **kw)
    assert_bits_equal(x_cal, x_bf.cpu(), "calibration event = the bf16 block")
    assert ctrl.event_metadata()["correct_precision_effective"] == precision
    ctrl.begin_event()                                   # freeze, then the low-precision route
    assert not ctrl.calibrating
    x_lp, c_lp = run()
    mods = {n: m for n, m in ctrl.lowp_blocks[0].named_modules() if isinstance(m, LP._LowPrecisionLinear)}
    assert sorted(mods) == sorted(LP.LOW_PRECISION_LINEAR_SUFFIXES)
    routes = {n: (LP.low_precision_state(m), float(m.act_scale)) for n, m in mods.items()}
    want_kinds = {n: ("fp8" if precision == "fp8" or n == "attn.proj" else "fp4") for n in mods}
    assert {n: k for n, (k, _) in routes.items()} == want_kinds
    k = OP.keep_count(P, ratio)
    plan = OP.build_plan(imp.numpy(), k, dind.numpy(), cfg.num_pretokens, N)
    x_ref, c_ref = OM.correct_block(cfg, w, x, plan, rope, {kk: v.clone() for kk, v in cache.items()}, "layer0",
                                    lowp=routes)
    x_ref16, c16 = OM.correct_block(cfg, w, x, plan, rope, {kk: v.clone() for kk, v in cache.items()}, "layer0")
    sel = torch.zeros(B, N, dtype=torch.bool)
    sel[plan.active_batch_idx, plan.active_token_idx] = True
    assert_bits_equal(x_lp[~sel], x_ref[~sel], "unselected rows")
    # yardstick: the same algorithm with fp32-accumulating GEMMs and the reference's bf16 eager ops
    with LPO.fp32_accumulation():
        x_y, c_y = OM.correct_block(cfg, w, x, plan, rope, {kk: v.clone() for kk, v in cache.items()}, "layer0",
                                    mode="bf16", lowp=routes)

    def rms(a, b):
        return float(((a.double() - b.double()) ** 2).mean().sqrt())

    d_impl, d_yard, d_route = rms(x_lp[sel], x_ref[sel]), rms(x_y[sel], x_ref[sel]), rms(x_ref[sel], x_ref16[sel])
    mx, mean = close_stats(x_lp[sel], x_ref[sel])
    print(f"  rms to the exact oracle: gpu {d_impl:.4g}, fp32-accumulating evaluation {d_yard:.4g}; "
          f"the {precision} route itself moves the block by {d_route:.4g}; gpu max {mx:.4g} mean {mean:.4g}",
          flush=True)
    assert d_route > 0 and d_impl <= 2.0 * d_yard + 1e-3 * d_route, (d_impl, d_yard, d_route)
    # The rewritten K/V rows sit one quantizer (qkv's input) downstream of norm1: a last-bit difference
    # of the GPU's LayerNorm flips an e2m1 code now and then (more often the wider the rows), while
    # torch's CPU LayerNorm may match the exact one everywhere (yardstick zero). So everything after
    # norm1 -- the quantizer, the GEMM, scale-and-bias, RoPE -- is checked against the oracle fed the
    # GPU's own norm1 output, where only the GEMM's fp32 accumulation order separates the two; and the
    # whole K/V difference must be what the LayerNorm bits plus that account for.
    bi, ti = torch.from_numpy(plan.active_batch_idx), torch.from_numpy(plan.active_token_idx)
    with torch.no_grad():
        xn_gpu = K.layer_norm(x[bi, ti].to(dev), blk.norm1.weight, blk.norm1.bias, blk.norm1.eps).cpu()
    _, k_g, v_g = OM.qkv_rope_rows(cfg, w, xn_gpu, plan, rope, lowp=routes)
    kv_from_gpu_ln = torch.stack([k_g, v_g], dim=1).to(torch.bfloat16)
    kv_gpu = c_lp["layer0_kv"].cpu()[bi, ti]
    kv_impl = rms(kv_gpu, c_ref["layer0_kv"][bi, ti])
    kv_rest = rms(kv_gpu, kv_from_gpu_ln)
    kv_ln = rms(kv_from_gpu_ln, c_ref["layer0_kv"][bi, ti])
    kv_yard = rms(c_y["layer0_kv"][bi, ti], c_ref["layer0_kv"][bi, ti])
    kv_route = rms(c_ref["layer0_kv"][bi, ti], c16["layer0_kv"][bi, ti])
    print(f"  K/V rms to the exact oracle: gpu {kv_impl:.4g} (after the GPU's norm1: {kv_rest:.4g}; the norm1 "
          f"bits alone: {kv_ln:.4g}), yardstick {kv_yard:.4g}, route effect {kv_route:.4g}", flush=True)
    assert kv_rest <= max(2.0 * kv_yard, 1e-2 * kv_route), (kv_rest, kv_yard, kv_route)
    assert kv_impl <= kv_ln + kv_rest + 1e-6 * kv_route, (kv_impl, kv_ln, kv_rest)


@pytest.mark.parametrize("M,C", [(103, 384), (1656, 4096), (517, 3072), (64, 8192)])
def test_nvfp4_producers_equal_quantize_after(dev, M, C):
    """The producers that write the NVFP4 operand directly (LayerNorm, the fused residual + LayerNorm,
    the SwiGLU epilogue) give bit for bit nvfp4_quantize_dequantize of what they write otherwise, and
    the scaled post-QKV scatter equals scale_bias followed by the plain scatter."""
    g = torch.Generator().manual_seed(M + C)
    x = (torch.randn(M, C, generator=g) * 3).to(torch.bfloat16).to(dev)
    w = (1 + 0.1 * torch.randn(C, generator=g)).to(torch.bfloat16).to(dev)
    b = (0.1 * torch.randn(C, generator=g)).to(torch.bfloat16).to(dev)
    ts = torch.tensor(float(Q.per_tensor_amax_to_scale(4.0)), device=dev)
    ln = K.layer_norm(x, w, b, 1e-6)
    assert_bits_equal(K.layer_norm(x, w, b, 1e-6, nvfp4_scale=ts), K.nvfp4_quantize_dequantize(ln, ts).cpu(),
                      "layer_norm -> x_hat")
    # the packed residual step with the next block's norm1 as x_hat
    B, N = 4, (M + 3) // 4 + 7
    bi = torch.arange(M, device=dev) % B
    ti = torch.arange(M, device=dev) // B
    xa, mlp = (torch.randn(2, M, C, generator=g) * 0.5).to(torch.bfloat16).to(dev).unbind(0)
    bos1 = torch.zeros(B, N, C, device=dev, dtype=torch.bfloat16)
    bos2 = bos1.clone()
    xn1, l1 = K.packed_residual_persist_ln(xa, x, mlp, bi, ti, bos1, w, b, 1e-6)
    xn2, l2 = K.packed_residual_persist_ln(xa, x, mlp, bi, ti, bos2, w, b, 1e-6, nvfp4_scale=ts)
    assert_bits_equal(xn2, xn1.cpu(), "x_new")
    assert_bits_equal(bos2, bos1.cpu(), "blocks_out_sum rows")
    assert_bits_equal(l2, K.nvfp4_quantize_dequantize(l1, ts).cpu(), "residual LayerNorm -> x_hat")
    # the SwiGLU epilogue writing w3's operand
    r1, r2 = (torch.randn(2, M, C, generator=g) * 4).to(torch.bfloat16).to(dev).unbind(0)
    b1, b2 = (0.1 * torch.randn(2, C, generator=g)).to(torch.bfloat16).to(dev).unbind(0)
    h = K.swiglu_scaled(r1.clone(), 0.37, b1, r2, 0.11, b2)
    hx = K.swiglu_scaled(r1.clone(), 0.37, b1, r2, 0.11, b2, nvfp4_scale=ts)
    assert_bits_equal(hx, K.nvfp4_quantize_dequantize(h, ts).cpu(), "swiglu -> x_hat")
    if C % 3 == 0 and (C // 3) % 64 == 0:   # the scaled post-QKV scatter on a [M, 3, H, Dh] raw product
        H, D = C // 3 // 64, 64
        raw = x.view(M, 3, H, D)
        pm = (torch.arange(M, device=dev) % 3 != 0)
        ridx = torch.arange(M, device=dev) % 17
        tab = torch.randn(32, D, generator=g).to(dev)
        rope = (tab.sin().contiguous(), tab.cos().contiguous())
        bq = (0.1 * torch.randn(C, generator=g)).to(torch.bfloat16).to(dev)
        for bias in (None, bq):
            kv1 = torch.zeros(B, N, 2, H, D, device=dev, dtype=torch.bfloat16)
            kv2, q1, q2 = kv1.clone(), torch.empty(M, H, D, device=dev, dtype=torch.bfloat16), \
                torch.empty(M, H, D, device=dev, dtype=torch.bfloat16)
            K.qkv_rope_kv_scatter(K.scale_bias(x, 0.013, bias).view(M, 3, H, D), rope, pm, ridx, bi, ti, kv1, q1)
            K.qkv_rope_kv_scatter(raw, rope, pm, ridx, bi, ti, kv2, q2, scale=0.013, bias=bias)
            assert_bits_equal(kv2, kv1.cpu(), "scaled scatter K/V")
            assert_bits_equal(q2, q1.cpu(), "scaled scatter q")


@pytest.mark.parametrize("precision", ["fp4", "fp8"])
def test_packed_low_precision_run_equals_blockwise(dev, precision):
    """Three frozen SwiGLU blocks: the packed run (fused producers of the NVFP4 operands across block
    boundaries) equals the controller's block-by-block run bit for bit."""
    cfg = OM.with_overrides(_swiglu_cfg(), depth=3)
    B, ratio = 2, 0.25
    N, C, H, D, P = cfg.num_tokens, cfg.dim, cfg.heads, cfg.head_dim, cfg.num_patches
    ws = OM.make_block_weights(cfg, 0, gamma=1.0, bias_std=0.05, ln_std=0.1, depth=3)
    blocks = []
    for w in ws:
        blk = SelfAttentionBlock(C, H, ffn_ratio=3.0, qkv_bias=False, init_values=1.0, ffn_layer="swiglu64",
                                 mask_k_bias=True)
        blk.load_state_dict(w, strict=True)
        blocks.append(blk.to(device=dev, dtype=torch.bfloat16))
    g = torch.Generator().manual_seed(9)
    x = torch.randn(B, N, C, generator=g).to(torch.bfloat16).to(dev)
    cache = {}
    for i in range(3):
        cache[f"layer{i}_kv"] = torch.randn(B, N, 2, H, D, generator=g).to(torch.bfloat16).to(dev)
        cache[f"layer{i}_blocks_out_sum"] = (torch.randn(B, N, C, generator=g) * 0.1).to(torch.bfloat16).to(dev)
    imp = torch.rand(B, P, generator=g).to(dev)
    rope = OM.rope_tables(cfg)
    r = (rope[0].to(dev), rope[1].to(dev))
    dind = OM.full_dindice(cfg, B).to(dev)
    kw = dict(token_keep_ratio=ratio, mobile_pscore="residual_energy", mobile_pscore_weight=1.0,
              mobile_pscore_hint=imp, server_pscore_weight=0.0)
    ctrl = DINOv3CorrectPrecisionController(nn.ModuleList(blocks), precision=precision, device=dev)

    def blockwise():
        c = {k: v.clone() for k, v in cache.items()}
        y = x
        with torch.no_grad():
            for i in range(3):
                y, c = ctrl.run_block(i, y, dind, r, c, f"layer{i}", **kw)
        return y, c

    ctrl.begin_event()
    blockwise()                      # calibration
    ctrl.begin_event()               # freeze
    y_b, c_b = blockwise()
    c_p = {k: v.clone() for k, v in cache.items()}
    with torch.no_grad():
        y_p, c_p = ctrl.run_blocks_packed(range(3), x, dind, r, c_p, **kw)
    torch.cuda.synchronize()
    assert_bits_equal(y_p, y_b.cpu(), f"{precision} packed run")
    for i in range(3):
        for s_ in ("kv", "blocks_out_sum"):
            assert_bits_equal(c_p[f"layer{i}_{s_}"], c_b[f"layer{i}_{s_}"].cpu(), f"layer{i}_{s_}")


@pytest.mark.parametrize("M,N,Kd", [(1656, 4096, 8192), (1656, 4096, 4096), (414, 8192, 4096), (4176, 1024, 4096),
                                    (300, 384, 384)])
def test_raw_bf16_epilogues_equal_scale_bias_after(dev, M, N, Kd):
    """An NVFP4 linear's scale, bias and LayerScale (residual) folded into its GEMM (EPI_RAW_BF16: the
    accumulator rounded to bf16 first) equal the raw bf16 GEMM followed by the scale-bias kernel (and the
    LayerScale add) bit for bit -- the GEMM picks its tiles and K split independently of the epilogue, so
    both read the same accumulators. Includes the ViT-7B w3 shape, whose K splits in two slices."""
    print(f"raw_bf16 epilogues {M}x{N}x{Kd}", flush=True)
    x = (_x((M, Kd), 7, outliers=False).float() * 0.5).to(torch.bfloat16).to(dev)
    w = (_x((N, Kd), 8, outliers=False).float() * 0.02).to(torch.bfloat16).to(dev)
    b = (_x((N,), 9, outliers=False).float() * 0.1).to(torch.bfloat16).to(dev)
    g = (1.0 + 0.1 * _x((N,), 10, outliers=False).float()).to(torch.bfloat16).to(dev)
    r = _x((M, N), 11, outliers=False).to(dev)
    s = 0.37
    raw = K.linear(x, w, None)
    RAW = _lib.EPI_RAW_BF16
    for bias in (b, None):
        sb = K.scale_bias(raw, s, bias)
        got = K.linear(x, w, bias, epilogue=_lib.EPI_BIAS | RAW, acc_scale=s)
        assert_bits_equal(got, sb.cpu(), f"scale-bias (bias {bias is not None})")
        got = K.linear(x, w, bias, epilogue=_lib.EPI_BIAS_LS | RAW, gamma=g, acc_scale=s)
        assert_bits_equal(got, K.scale_bias(raw, s, bias, gamma=g).cpu(), "scale-bias + LayerScale")
        got = K.linear(x, w, bias, epilogue=_lib.EPI_BIAS_LS_RESID | RAW, gamma=g, resid=r, acc_scale=s)
        assert_bits_equal(got, K.fused_layerscale_add(r, sb, g).cpu(), "scale-bias + LayerScale + residual")


@pytest.mark.parametrize("B,T,H,D,Kd", [(4, 414, 32, 128, 4096), (2, 50, 4, 64, 256)])
def test_nvfp4_fused_qkv_equals_scaled_scatter(dev, B, T, H, D, Kd):
    """The NVFP4 qkv linear in the fused QKV kernel (bf16(bf16(acc) s + b), then RoPE and the K/V / q
    writes) equals the scaled post-QKV scatter applied to that kernel's own bf16 accumulator (taken from
    a run with scale 1, no bias and no patch rows), bit for bit."""
    N = 1029
    M = B * T
    rng = np.random.default_rng(B + H)
    toks = np.stack([np.concatenate([np.arange(5), np.sort(rng.choice(np.arange(5, N), T - 5, replace=False))])
                     for _ in range(B)])
    tok = torch.from_numpy(toks.reshape(-1).astype(np.int64)).to(dev)
    bi = torch.arange(B).repeat_interleave(T).to(dev)
    pm, ri = tok >= 5, (tok - 5).clamp_min(0)
    cfg = OM.with_overrides(OM.CONFIGS["vit7b16_1024"], dim=H * D, heads=H)
    sin, cos = (t.to(dev) for t in OM.rope_tables(cfg))
    x = _x((M, Kd), 12, outliers=False).to(dev)
    w = (_x((3 * H * D, Kd), 13, outliers=False).float() * 0.02).to(torch.bfloat16).to(dev)
    b = (_x((3 * H * D,), 14, outliers=False).float() * 0.1).to(torch.bfloat16).to(dev)
    kv0 = _x((B, N, 2, H, D), 15, outliers=False).to(dev)
    s = 0.37
    for bias in (b, None):
        kv_f, q_f = kv0.clone(), torch.empty((M, H, D), dtype=torch.bfloat16, device=dev)
        K.linear_qkv_rope_kv(x, w, bias, (sin, cos), pm, ri, bi, tok, kv_f, q_f, acc_scale=s, raw_bf16=True)
        kv_r, q_r = kv0.clone(), torch.empty((M, H, D), dtype=torch.bfloat16, device=dev)
        K.linear_qkv_rope_kv(x, w, None, (sin, cos), torch.zeros_like(pm), ri, bi, tok, kv_r, q_r, acc_scale=1.0,
                             raw_bf16=True)
        raw = torch.stack([q_r, kv_r[bi, tok, 0], kv_r[bi, tok, 1]], dim=1).contiguous()  # bf16(acc)
        kv_u, q_u = kv0.clone(), torch.empty((M, H, D), dtype=torch.bfloat16, device=dev)
        K.qkv_rope_kv_scatter(raw, (sin, cos), pm, ri, bi, tok, kv_u, q_u, scale=s, bias=bias)
        assert_bits_equal(q_f, q_u.cpu(), f"q (bias {bias is not None})")
        assert_bits_equal(kv_f, kv_u.cpu(), f"kv (bias {bias is not None})")


@pytest.mark.parametrize("M,N,Kd,same_tiles", [(1656, 8192, 4096, True), (4176, 4096, 1024, True),
                                               (600, 1024, 512, False)])
def test_swiglu_nvfp4_gemm_equals_gemm_then_swiglu(dev, M, N, Kd, same_tiles):
    """w2's NVFP4 GEMM with the SwiGLU and w3's quantizer in its epilogue equals the raw w2 GEMM followed
    by the SwiGLU kernel writing x_hat, bit for bit where both take the same tiles (the ViT-7B w2 shape);
    where the plain GEMM would take other tiles (the fused entry keeps ping-pong tiles) the accumulators
    differ in the last fp32 bit, and at least 99 % of the x_hat values must still agree."""
    print(f"swiglu nvfp4 gemm {M}x{N}x{Kd}", flush=True)
    xh = (_x((M, Kd), 16, outliers=False).float() * 0.5).to(torch.bfloat16).to(dev)
    w2 = (_x((N, Kd), 17, outliers=False).float() * 0.02).to(torch.bfloat16).to(dev)
    x1 = _x((M, N), 18, outliers=False).to(dev)
    b1 = (_x((N,), 19, outliers=False).float() * 0.1).to(torch.bfloat16).to(dev)
    b2 = (_x((N,), 20, outliers=False).float() * 0.1).to(torch.bfloat16).to(dev)
    ts = torch.tensor([0.013], device=dev)
    for bias in (True, False):
        bb1, bb2 = (b1, b2) if bias else (None, None)
        got = K.linear_swiglu_nvfp4(xh, w2, x1, 0.7, bb1, 1.3, bb2, ts)
        r2 = K.linear(xh, w2, None)
        ref = K.swiglu_scaled(x1.clone(), 0.7, bb1, r2, 1.3, bb2, nvfp4_scale=ts)
        if same_tiles:
            assert_bits_equal(got, ref.cpu(), f"x_hat (bias {bias})")
        else:
            same = float((got == ref).float().mean())
            assert same >= 0.99, same
