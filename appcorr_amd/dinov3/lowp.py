"""Low-precision correction linears: the NVFP4 and FP8 routes of the correction GEMMs.

Counterparts of FastFP4Linear / SharedFP4Activation (offload/server/model/fp4_fast_linear.py:71-283)
and FastFP8Linear (offload/server/model/fp8_fast_linear.py:83-196), with the same lifecycle: a
module starts *calibrating* (the block runs its exact bf16 GEMM while an observer keeps the running
max |x| of the module's input), and `freeze_activation_scale` bakes a static activation scale from that
maximum, after which the block runs the low-precision route.

gfx950 has no MFMA for NVFP4 (16-element blocks, e4m3 scales), and every value an NVFP4 GEMM multiplies
(e2m1 code x e4m3 block scale) is exact in bf16. So the NVFP4 operands are quantized with the
reference's rounding and kept as those exact bf16 values (`weight_hat`, once at construction; the
activation per call), and the bf16 MFMA GEMM with fp32 accumulation computes the scaled GEMM's
products and sum, up to the order of the fp32 additions. FP8 (OCP e4m3) is native on gfx950: the FP8
linears keep e4m3 codes and run the FP8 MFMA (exact products, fp32 accumulation). The per-tensor
factors follow the reference:
  NVFP4: raw = bf16(A_hat . W_hat^T) (torch._scaled_mm, out_dtype bf16), then raw * out_scale + bias in
         fp32 (scale_bias_inplace_triton), out_scale = bf16(act_scale * weight_scale);
  FP8:   bf16(acc * act_scale * weight_scale + bias) (torch._scaled_mm with scales and bias), applied
         by the GEMM's accumulator scale.
The block code (dinov3/layers.py) dispatches on these module types; only SwiGLU blocks (ViT-7B) have
the five eligible linears (dinov3_precision.py:17-73).
"""

from __future__ import annotations

import torch
from torch import nn

from .. import kernels as K

E4M3_MAX = 448.0
E2M1_MAX = 6.0
LOW_PRECISION_LINEAR_SUFFIXES = ("attn.qkv", "attn.proj", "mlp.w1", "mlp.w2", "mlp.w3")


def _amax(t: torch.Tensor) -> torch.Tensor:
    a = torch.zeros((), device=t.device, dtype=torch.float32)
    K.amax_update(t, a)
    return a


def per_tensor_amax_to_scale(amax: torch.Tensor) -> torch.Tensor:
    """NVFP4 per-tensor scale amax / (448 * 6) in fp32 (torchao's per_tensor_amax_to_scale, used by
    fp4_fast_linear.py:129-133, 159-160)."""
    return amax.to(torch.float32) / (E4M3_MAX * E2M1_MAX)


class SharedFP4Activation:
    """One quantized activation shared by sibling linears fed the same tensor (mlp.w1 / mlp.w2), keyed by
    (data_ptr, shape, dtype) with a strong reference to the input (fp4_fast_linear.py:71-100)."""

    __slots__ = ("_x", "_value")

    def __init__(self) -> None:
        self._x = None
        self._value = None

    def get(self, x: torch.Tensor):
        c = self._x
        if c is not None and c.data_ptr() == x.data_ptr() and c.shape == x.shape and c.dtype == x.dtype:
            return self._value
        return None

    def put(self, x: torch.Tensor, value) -> None:
        self._x = x
        self._value = value


class _LowPrecisionLinear(nn.Module):
    """Common state: the original bf16 weight and bias (used while calibrating), the observer."""

    def __init__(self, linear: nn.Linear) -> None:
        super().__init__()
        if linear.weight.dtype != torch.bfloat16 or not linear.weight.is_cuda:
            raise ValueError("low-precision linears take a bf16 nn.Linear on the GPU")
        self.in_features = linear.in_features
        self.out_features = linear.out_features
        self.weight = linear.weight            # shared with the bf16 block, not copied
        self.bias = linear.bias
        self.amax = torch.zeros((), device=linear.weight.device, dtype=torch.float32)
        self.calibrating = True

    def observe(self, x2d: torch.Tensor) -> None:
        """The calibrating forward's observer: amax = max(amax, max |x|) (fp4_fast_linear.py:256-259)."""
        K.amax_update(x2d, self.amax)


class FastFP4Linear(_LowPrecisionLinear):
    """nn.Linear in NVFP4 (fp4_fast_linear.py:103-283)."""

    def __init__(self, linear: nn.Linear, share: SharedFP4Activation | None = None, bucket_rows: int = 0) -> None:
        if linear.in_features % 32 or linear.out_features % 16:
            raise ValueError("Packed FP4 _scaled_mm needs in_features % 32 == 0 and out_features % 16 == 0, "
                             f"got {linear.in_features}x{linear.out_features}")
        super().__init__(linear)
        self.bucket_rows = max(0, int(bucket_rows))  # accepted for the interface; fixed shapes need no padding here
        self._share = share
        with torch.no_grad():
            self.weight_scale = per_tensor_amax_to_scale(_amax(self.weight))
            self.weight_hat = K.nvfp4_quantize_dequantize(self.weight, self.weight_scale)
        self.act_scale = torch.zeros((), device=self.weight.device, dtype=torch.float32)
        self.out_scale = torch.zeros((), device=self.weight.device, dtype=torch.bfloat16)
        self.out_scale_f = 0.0

    @torch.no_grad()
    def freeze_activation_scale(self) -> bool:
        """Bake the observed amax into the static activation scale (fp4_fast_linear.py:148-169).
        False while nothing has been observed (the linear then stays on the exact bf16 route)."""
        if not self.calibrating:
            return True
        if float(self.amax) <= 0.0:
            return False
        self.act_scale = per_tensor_amax_to_scale(self.amax)
        self.out_scale = (self.act_scale * self.weight_scale).to(torch.bfloat16)
        self.out_scale_f = float(self.out_scale)   # once, on the host: no sync per call
        self.calibrating = False
        return True

    def quantize(self, x2d: torch.Tensor) -> torch.Tensor:
        """The exact bf16 values of the NVFP4 activation (shared with a sibling fed the same tensor)."""
        if self._share is not None:
            cached = self._share.get(x2d)
            if cached is not None:
                return cached
        xq = K.nvfp4_quantize_dequantize(x2d, self.act_scale)
        if self._share is not None:
            self._share.put(x2d, xq)
        return xq

    def forward_raw(self, x2d: torch.Tensor, site: str = "linear") -> torch.Tensor:
        """bf16(x_hat . W_hat^T) -- torch._scaled_mm's output before the scale-and-bias epilogue
        (fp4_fast_linear.py:221-249)."""
        return K.linear(self.quantize(x2d), self.weight_hat, None, site=site)

    def extra_repr(self) -> str:
        return f"in={self.in_features}, out={self.out_features}, state={'calibrating' if self.calibrating else 'fp4'}"


class FastFP8Linear(_LowPrecisionLinear):
    """nn.Linear in FP8 e4m3 with per-tensor scales (fp8_fast_linear.py:83-196).

    Where the native FP8 GEMM takes the shape (K % 128 == 0, N % 256 == 0: every ViT-7B linear) the
    weight is kept as its e4m3 codes (`weight_q`) and the product runs on the FP8 MFMA with the
    activation quantized to codes per call; otherwise as the codes' exact bf16 values (`weight_hat`)
    on the bf16 MFMA. Both compute the same exact products with fp32 accumulation."""

    def __init__(self, linear: nn.Linear, bucket_rows: int = 0) -> None:
        if linear.in_features % 16 or linear.out_features % 16:
            raise ValueError("FP8 _scaled_mm requires both dimensions divisible by 16, got "
                             f"{linear.in_features}x{linear.out_features}")
        super().__init__(linear)
        self.bucket_rows = max(0, int(bucket_rows))
        self.native = K.fp8_gemm_supported(self.in_features, self.out_features)
        with torch.no_grad():
            self.weight_scale = (_amax(self.weight) / E4M3_MAX).clamp(min=1e-12)
            if self.native:
                self.weight_q = K.fp8_quantize(self.weight, self.weight_scale.reshape(1), K.FP8_WEIGHT)
                self.weight_hat = None
            else:
                self.weight_q = None
                self.weight_hat = K.fp8_quantize_dequantize(self.weight, self.weight_scale, K.FP8_WEIGHT)
        self.act_scale = torch.zeros((), device=self.weight.device, dtype=torch.float32)
        self.act_inv_scale = torch.zeros((), device=self.weight.device, dtype=torch.bfloat16)
        self._act_inv_f32 = torch.zeros(1, device=self.weight.device, dtype=torch.float32)
        self.acc_scale_f = 0.0

    @torch.no_grad()
    def freeze_activation_scale(self) -> bool:
        """fp8_fast_linear.py:149-172: scale = max(amax / 448, 1e-12), inverse held in bf16; the GEMM's
        accumulator factor scale_a * scale_b (fp32) is taken to the host once."""
        if not self.calibrating:
            return True
        if float(self.amax) <= 0.0:
            return False
        scale = (self.amax.float() / E4M3_MAX).clamp(min=1e-12)
        self.act_scale = scale
        self.act_inv_scale = (1.0 / scale).to(torch.bfloat16)
        self._act_inv_f32 = self.act_inv_scale.float().reshape(1)  # the quantizer's fp32 operand, once
        self.acc_scale_f = float(self.act_scale * self.weight_scale)
        self.calibrating = False
        return True

    def quantize(self, x2d: torch.Tensor) -> torch.Tensor:
        """The activation's e4m3 values as bf16 (the operand of the bf16-MFMA route)."""
        return K.fp8_quantize_dequantize(x2d, self._act_inv_f32, K.FP8_ACTIVATION)

    def quantize_codes(self, x2d: torch.Tensor) -> torch.Tensor:
        """The activation's e4m3fn codes, uint8 (the operand of the native FP8 GEMM)."""
        return K.fp8_quantize(x2d, self._act_inv_f32, K.FP8_ACTIVATION)

    @property
    def act_inv_f32(self) -> torch.Tensor:
        """The frozen activation quantizer's operand: the bf16 inverse scale as an fp32 device scalar."""
        return self._act_inv_f32

    def linear_codes(self, x8: torch.Tensor, bias: torch.Tensor | None, site: str, **kw) -> torch.Tensor:
        """`linear` of an activation already given as its e4m3fn codes (quantize_codes' output, written by
        the producer itself); native FP8 GEMM only."""
        return K.linear_fp8(x8, self.weight_q, bias, acc_scale=self.acc_scale_f, site=site, **kw)

    def linear(self, x: torch.Tensor, bias: torch.Tensor | None, site: str, **kw) -> torch.Tensor:
        """The frozen linear's output: bf16(acc * act_scale * weight_scale + bias) with the epilogue of
        `kw` (fp8_fast_linear.py:174-196)."""
        if self.native:
            return K.linear_fp8(self.quantize_codes(x), self.weight_q, bias, acc_scale=self.acc_scale_f, site=site,
                                **kw)
        return K.linear(self.quantize(x), self.weight_hat, bias, site=site, acc_scale=self.acc_scale_f, **kw)

    def extra_repr(self) -> str:
        return f"in={self.in_features}, out={self.out_features}, state={'calibrating' if self.calibrating else 'fp8'}"


def low_precision_state(mod) -> str:
    """'fp4' / 'fp8' for a frozen low-precision linear, 'bf16' otherwise (a plain nn.Linear or one still
    calibrating)."""
    if isinstance(mod, FastFP4Linear) and not mod.calibrating:
        return "fp4"
    if isinstance(mod, FastFP8Linear) and not mod.calibrating:
        return "fp8"
    return "bf16"


def eligible_linears(block: nn.Module, *, fp4: bool) -> list[tuple[str, nn.Linear]]:
    """The five correction linears of a block (dinov3_precision.py:36-73); raises RuntimeError when the
    block does not have exactly those (a GELU-MLP block) or their shapes do not fit."""
    eligible = [(n, m) for n, m in block.named_modules()
                if isinstance(m, nn.Linear) and n.endswith(LOW_PRECISION_LINEAR_SUFFIXES)]
    if len(eligible) != len(LOW_PRECISION_LINEAR_SUFFIXES):
        raise RuntimeError("Expected exactly five low-precision Linear layers per DINOv3 block, found "
                           f"{[n for n, _ in eligible]}")
    bad = [(n, tuple(m.weight.shape)) for n, m in eligible if m.in_features % 16 or m.out_features % 16]
    if bad:
        raise RuntimeError(f"Low-precision _scaled_mm requires dimensions divisible by 16: {bad}")
    if fp4:
        bad = [(n, tuple(m.weight.shape)) for n, m in eligible if m.in_features % 32]
        if bad:
            raise RuntimeError(f"Packed FP4 _scaled_mm requires in_features divisible by 32: {bad}")
    return eligible


def _rebuilt(module: nn.Module, children: dict) -> nn.Module:
    """A shallow copy of `module` whose child modules `children` are replaced (parameters shared)."""
    clone = module.__class__.__new__(module.__class__)
    clone.__dict__.update(module.__dict__)
    clone._modules = dict(module._modules)
    clone._modules.update(children)
    return clone


def convert_block(block: nn.Module, precision: str, *, proj_precision: str = "fp8", bucket_rows: int = 0):
    """A view of `block` whose five correction linears run in `precision` ("fp4": qkv, w1, w2, w3 in
    NVFP4 with w1 / w2 sharing one quantized activation, attn.proj in `proj_precision`; "fp8": all five
    in FP8), sharing every other parameter with `block` (convert_linears_to_fast_fp4,
    fp4_fast_linear.py:286-311; convert_linears_to_fast_fp8, fp8_fast_linear.py:199-210).
    Returns (converted block, number of FP4 linears, number of FP8 linears)."""
    eligible = dict(eligible_linears(block, fp4=precision == "fp4"))
    shared = SharedFP4Activation()
    made, n4, n8 = {}, 0, 0
    for name in sorted(eligible):
        lin = eligible[name]
        if precision == "fp8" or (name.endswith("attn.proj") and proj_precision == "fp8"):
            made[name] = FastFP8Linear(lin, bucket_rows=bucket_rows)
            n8 += 1
        else:
            share = shared if name.endswith(("mlp.w1", "mlp.w2")) else None
            made[name] = FastFP4Linear(lin, share=share, bucket_rows=bucket_rows)
            n4 += 1
    attn = _rebuilt(block.attn, {"qkv": made["attn.qkv"], "proj": made["attn.proj"]})
    attn._bias_key = None
    mlp = _rebuilt(block.mlp, {"w1": made["mlp.w1"], "w2": made["mlp.w2"], "w3": made["mlp.w3"]})
    return _rebuilt(block, {"attn": attn, "mlp": mlp}), n4, n8
