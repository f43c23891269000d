"""Low-precision correction linears (NVFP4 / FP8) restated on the CPU. Test infrastructure only.

Follows offload/server/model/fp4_fast_linear.py:103-283 (FastFP4Linear, SharedFP4Activation),
fp8_fast_linear.py:83-196 (FastFP8Linear), appcorr/models/dinov3/layers/triton_kernels/
token_update.py:571-669 (scale_bias_inplace, fused_swiglu_epilogue) and ffn_layers.py:84-115 (the
SwiGLU consumer), with the block flow of oracle.model.correct_block.

  NVFP4 linear  x_hat = e2m1(q) * e4m3(s) of x quantized with the activation scale (oracle.nvfp4,
                bit-exact restatement of the reference quantizer), W_hat likewise with the weight
                scale amax(|W|) / 2688; raw = bf16(x_hat . W_hat^T) (torch._scaled_mm, out_dtype bf16,
                fp32 accumulation -- evaluated exactly here, then rounded to fp32 and bf16);
                out = bf16(raw * out_scale + bias) with out_scale = bf16(act_scale * weight_scale)
                (one fp32 rounding: the fused multiply-add the reference's Triton epilogue compiles to
                when a bias is present; raw * out_scale without one).
  FP8 linear    x_q = e4m3(clamp(x * bf16(1 / act_scale), +-448)) (fp32 product, the compiled
                quantizer), W_q = e4m3(clamp(bf16(W / bf16(w_scale)), +-448)) (eager bf16 ops),
                out = bf16(acc * (act_scale * w_scale) + bias) (scales and bias inside _scaled_mm).
  SwiGLU        a = raw1 * s1 + b1, b = raw2 * s2 + b2 (fp32), out = bf16(silu(a) * b).
e4m3 conversions use torch's CPU float8_e4m3fn cast (round to nearest even, pinned in
tests/test_oracle_nvfp4.py).

Scales computed from a maximum divide as torch does on a GPU tensor (cuda_scalar_div: times the fp32
reciprocal). Parity unpinned: torch._scaled_mm's / cuBLASLt's fp32 accumulation order and where it
applies the two scales (taken here as the exact acc times the fp32 product of the scales); Triton's fp32 exp and
division inside sigmoid; whether the reference's scale-and-bias contracts to an FMA (taken: yes).
"""

from __future__ import annotations

import contextlib
import hashlib

import numpy as np
import torch

from . import nvfp4 as Q
from .bf16 import round_bf16

E4M3_MAX = 448.0


def _f32(a) -> np.ndarray:
    return np.asarray(a, dtype=np.float64).astype(np.float32)


def amax(x: torch.Tensor) -> np.float32:
    return np.float32(x.float().abs().max())


def nvfp4_xhat(x: np.ndarray, ts: float) -> np.ndarray:
    """e2m1(q) * e4m3(s) of x [M, K] (bf16 values) quantized with tensor scale ts: fp32 [M, K]."""
    x = np.asarray(x, dtype=np.float32)
    M, K = x.shape
    q, s = Q.quantize(x, ts)
    return Q.dequantize(q, s, 1.0, M, K)


def e4m3(v: np.ndarray) -> np.ndarray:
    """Nearest-even e4m3fn value of fp32 v (already clamped to +-448), as fp32."""
    return torch.from_numpy(np.asarray(v, dtype=np.float32)).to(torch.float8_e4m3fn).float().numpy()


def fp8_act(x: np.ndarray, inv_scale_bf16: float) -> np.ndarray:
    """The compiled activation quantizer (fp8_fast_linear.py:71-73): e4m3(clamp(x * inv, +-448))."""
    return e4m3(np.clip(np.asarray(x, dtype=np.float32) * np.float32(inv_scale_bf16), -E4M3_MAX, E4M3_MAX))


def fp8_weight(w: np.ndarray, w_scale: float) -> np.ndarray:
    """The eager weight quantizer (fp8_fast_linear.py:123-125): the bf16 quotient by the bf16 scale."""
    s = round_bf16(np.float32(w_scale))
    quot = round_bf16(_f32(np.asarray(w, dtype=np.float64) / np.float64(s)))
    return e4m3(np.clip(quot, -E4M3_MAX, E4M3_MAX))


_EXACT = [True]


@contextlib.contextmanager
def fp32_accumulation():
    """Within this context the GEMMs accumulate in fp32 (torch's CPU matmul) instead of exactly: an
    independent fp32-accumulating evaluation of the same algorithm, the way a GPU GEMM accumulates,
    used as the yardstick of how far last-bit differences carry through the quantizers."""
    _EXACT[0] = False
    try:
        yield
    finally:
        _EXACT[0] = True


def _matmul_exact(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """a [M, K] . b [N, K]^T in float64 (exact for products of bf16-representable operands), or in
    fp32 inside fp32_accumulation()."""
    if not _EXACT[0]:
        ta = torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32))
        tb = torch.from_numpy(np.ascontiguousarray(b, dtype=np.float32))
        return (ta @ tb.T).double().numpy()
    return np.asarray(a, dtype=np.float64) @ np.asarray(b, dtype=np.float64).T


_WEIGHT_MEMO: dict = {}


def _memo_weight(kind: str, w: np.ndarray, scale: float, fn):
    """fn(w, scale) for a weight, remembered by the content of w (blake2b) and the scale: a quantized
    weight is a pure function of both, and the repeated oracle evaluations of one test (exact,
    fp32-accumulating) then quantize each weight once."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    key = (kind, w.shape, float(np.float32(scale)), hashlib.blake2b(w, digest_size=16).digest())
    hit = _WEIGHT_MEMO.get(key)
    if hit is None:
        if len(_WEIGHT_MEMO) >= 16:
            _WEIGHT_MEMO.clear()
        hit = fn(w, scale)
        _WEIGHT_MEMO[key] = hit
    return hit


def cuda_scalar_div(a, b: float) -> np.float32:
    """fp32 a / Python float b as torch evaluates it on a GPU tensor -- the reference's scales are such
    divisions of device tensors (torchao's per_tensor_amax_to_scale, amax / (448 * 6); FastFP8Linear's
    amax / 448, fp8_fast_linear.py:122, 164-168): a times the reciprocal of b rounded to fp32 on the
    host (aten/src/ATen/native/cuda/BinaryDivTrueKernel.cu, the scalar-divisor case), which differs from
    the IEEE quotient by one ulp for some a. Pinned against torch's own device division
    (tests/test_gpu_lowp.py::test_scale_division_is_torchs)."""
    return np.float32(np.float32(a) * (np.float32(1.0) / np.float32(b)))


def fp4_weight_scale(w: np.ndarray) -> np.float32:
    """per_tensor_amax_to_scale(amax(|W|)) on the device: amax * fp32(1 / 2688) (fp4_fast_linear.py:129-133)."""
    return cuda_scalar_div(np.abs(np.asarray(w, dtype=np.float32)).max(), E4M3_MAX * 6.0)


def fp4_raw(x: np.ndarray, act_scale: float, w: np.ndarray, w_scale: float) -> np.ndarray:
    """bf16(x_hat . W_hat^T) as fp32 (torch._scaled_mm with NVFP4 operands, out_dtype bf16)."""
    return round_bf16(_f32(_matmul_exact(nvfp4_xhat(x, act_scale), _memo_weight("fp4", w, w_scale, nvfp4_xhat))))


def fp4_out_scale(act_scale: float, w_scale: float) -> np.float32:
    """out_scale = bf16(act_scale * weight_scale) (fp4_fast_linear.py:163-166)."""
    return np.float32(round_bf16(np.float32(np.float32(act_scale) * np.float32(w_scale))))


def scale_bias(raw: np.ndarray, s: float, bias: np.ndarray | None, gamma: np.ndarray | None = None) -> np.ndarray:
    """bf16(raw * s + bias) (one fp32 rounding; raw * s without a bias), then bf16(. * gamma)."""
    r = np.asarray(raw, dtype=np.float64) * np.float64(np.float32(s))
    if bias is not None:
        r = r + np.asarray(bias, dtype=np.float64)
    y = _f32(r)
    if gamma is not None:
        y = round_bf16(y) * np.asarray(gamma, dtype=np.float32)
    return round_bf16(y)


def swiglu_scaled(raw1, s1, b1, raw2, s2, b2) -> np.ndarray:
    """bf16(silu(raw1 * s1 + b1) * (raw2 * s2 + b2)), the fp32 pre-activations rounded once each."""
    def pre(r, s, b):
        v = np.asarray(r, dtype=np.float64) * np.float64(np.float32(s))
        if b is not None:
            v = v + np.asarray(b, dtype=np.float64)
        return _f32(v).astype(np.float64)
    a, b = pre(raw1, s1, b1), pre(raw2, s2, b2)
    return round_bf16(_f32(a / (1.0 + np.exp(-a)) * b))


def fp8_linear(x: np.ndarray, act_scale: float, w: np.ndarray, w_scale: float, bias: np.ndarray | None) -> np.ndarray:
    """bf16(acc * (act_scale * w_scale) + bias), acc the exact sum of the e4m3 products."""
    inv = round_bf16(np.float32(1.0) / np.float32(act_scale))
    acc = _matmul_exact(fp8_act(x, inv), _memo_weight("fp8", w, w_scale, fp8_weight))
    alpha = np.float64(np.float32(np.float32(act_scale) * np.float32(w_scale)))
    r = acc * alpha
    if bias is not None:
        r = r + np.asarray(bias, dtype=np.float64)
    return round_bf16(_f32(r))


def fp8_weight_scale(w: np.ndarray) -> np.float32:
    """max(amax(|W|) / 448, 1e-12) in fp32, the division as on the device (fp8_fast_linear.py:122)."""
    return np.float32(max(cuda_scalar_div(np.abs(np.asarray(w, dtype=np.float32)).max(), E4M3_MAX),
                          np.float32(1e-12)))


def fp8_act_scale(amax_: float) -> np.float32:
    """max(amax / 448, 1e-12), the division as on the device (fp8_fast_linear.py:164-168)."""
    return np.float32(max(cuda_scalar_div(amax_, E4M3_MAX), np.float32(1e-12)))


def linear_out(route, x: torch.Tensor, w: torch.Tensor, b: torch.Tensor | None) -> torch.Tensor:
    """The bf16 output of one correction linear on `route` = (kind, act_scale): kind "fp4" (NVFP4 GEMM
    and its scale-and-bias epilogue) or "fp8"; x [M, K], w [N, K], b [N] bf16 tensors."""
    kind, sa = route
    xn, wn = x.float().numpy(), w.float().numpy()
    bn = None if b is None else b.float().numpy()
    if kind == "fp4":
        ws = fp4_weight_scale(wn)
        y = scale_bias(fp4_raw(xn, sa, wn, ws), fp4_out_scale(sa, ws), bn)
    elif kind == "fp8":
        y = fp8_linear(xn, sa, wn, fp8_weight_scale(wn), bn)
    else:
        raise ValueError(kind)
    return torch.from_numpy(np.ascontiguousarray(y)).to(torch.bfloat16)


def swiglu_mlp(routes: dict, blk: dict, x: torch.Tensor, gamma: torch.Tensor) -> torch.Tensor:
    """gamma * w3(silu(w1 x) * w2 x) with NVFP4 w1 / w2 / w3 (ffn_layers.py:84-115): w2 reuses the
    activation w1 quantized (SharedFP4Activation keeps the first caller's quantization, so both use
    w1's activation scale), both epilogues fold into the SwiGLU kernel, w3 gets its scale-and-bias and
    the LayerScale."""
    (k1, sa1), (k2, _), (k3, sa3) = routes["mlp.w1"], routes["mlp.w2"], routes["mlp.w3"]
    assert k1 == k2 == k3 == "fp4"
    xn = x.float().numpy()
    w1, w2, w3 = (blk[f"mlp.{n}.weight"].float().numpy() for n in ("w1", "w2", "w3"))
    b1, b2, b3 = (None if blk.get(f"mlp.{n}.bias") is None else blk[f"mlp.{n}.bias"].float().numpy()
                  for n in ("w1", "w2", "w3"))
    xh = nvfp4_xhat(xn, sa1)
    ws1, ws2, ws3 = fp4_weight_scale(w1), fp4_weight_scale(w2), fp4_weight_scale(w3)
    raw1 = round_bf16(_f32(_matmul_exact(xh, _memo_weight("fp4", w1, ws1, nvfp4_xhat))))
    raw2 = round_bf16(_f32(_matmul_exact(xh, _memo_weight("fp4", w2, ws2, nvfp4_xhat))))
    sa2 = routes["mlp.w2"][1]
    h = swiglu_scaled(raw1, fp4_out_scale(sa1, ws1), b1, raw2, fp4_out_scale(sa2, ws2), b2)
    raw3 = fp4_raw(h, sa3, w3, ws3)
    y = scale_bias(raw3, fp4_out_scale(sa3, ws3), b3, gamma.float().numpy())
    return torch.from_numpy(np.ascontiguousarray(y)).to(torch.bfloat16)
