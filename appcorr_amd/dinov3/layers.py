"""DINOv3 transformer block whose approx / correct passes run on the gfx950 kernels.

Module tree and parameter names are those of the reference (appcorr/models/dinov3/layers/block.py,
attention.py, ffn_layers.py, layer_scale.py), so a reference state_dict loads unchanged:
    norm1.{weight,bias}  attn.qkv.{weight,bias,bias_mask}  attn.proj.{weight,bias}  ls1.gamma
    norm2.{weight,bias}  mlp.fc1/fc2.{weight,bias} | mlp.w1/w2/w3.{weight,bias}     ls2.gamma
The modules only hold parameters; their forward never runs a torch op on the hot path. Every step of
`SelfAttentionBlock.correct_partial_token` is a library call (appcorr_amd.kernels):

    topk_plan (once per plan) -> gather_rows -> layer_norm
    -> linear_qkv_rope_kv [qkv GEMM + bias + RoPE + K/V cache rows + packed q, one kernel]
    -> sparse_query_attention -> linear[proj, +LayerScale +residual] -> layer_norm
    -> linear[fc1, +GELU] -> linear[fc2, +LayerScale] -> reconstruct_scatter_persist

A run of blocks sharing one query plan (`correct_blocks_packed`, what the executor uses when the
plan does not depend on the layer) keeps the selected rows packed: gather_rows once, per block the
same kernels with packed_residual_persist_ln (residual + persist + the next block's layer_norm)
in place of reconstruct_scatter_persist, and one fold_residual_rows at the end.

Plan-level bookkeeping that the reference does with small torch ops on [B, P] score tensors (score
resolution and fusion, the plan cache, the pscore statistics) is kept as torch ops: it runs once per
plan, not per block.
"""

from __future__ import annotations

import math
import os
from dataclasses import dataclass
from typing import Dict, Tuple

import torch
from torch import Tensor, nn

from .. import _lib
from .. import kernels as K
from ..tracing import annotate, trace_range
from . import lowp as LP


def _linear_route(mod: nn.Module, x: Tensor, site: str, *, bias: Tensor | None = None, **kw) -> Tensor:
    """One correction linear on its route: FP8 (e4m3 operands on the FP8 MFMA, or their exact bf16
    values where the FP8 GEMM does not take the shape; the per-tensor scales on the fp32 accumulator;
    fp8_fast_linear.py:174-196) when `mod` is a frozen FastFP8Linear, else bf16 -- a plain nn.Linear,
    or a low-precision linear still calibrating, whose observer sees the input first
    (fp4_fast_linear.py:255-259). `bias` overrides mod.bias (the masked qkv bias)."""
    b = mod.bias if bias is None else bias
    if LP.low_precision_state(mod) == "fp8":
        return mod.linear(x, b, site, **kw)
    if isinstance(mod, LP._LowPrecisionLinear):
        mod.observe(x)
    return K.linear(x, mod.weight, b, site=site, **kw)


def _bf16_weight(mod: nn.Module | None) -> Tensor | None:
    """The weight a bf16 linear's GEMM reads (a cache-warming target), or None when `mod` is absent or
    runs in low precision."""
    if mod is None or LP.low_precision_state(mod) != "bf16":
        return None
    w = getattr(mod, "weight", None)
    return w if isinstance(w, Tensor) and w.dtype == torch.bfloat16 and w.is_contiguous() else None


_IDENTITY_PLANS: Dict[tuple, "PackedQueryState"] = {}


def _identity_query_state(B: int, N: int, prefix: int, dev: torch.device) -> "PackedQueryState":
    """The approximate pass's plan (every token of every image is a query, T = N), built once per
    (B, N, prefix, device) and shared by every block and pass: its tensors are only read."""
    key = (B, N, prefix, str(dev))
    qs = _IDENTITY_PLANS.get(key)
    if qs is None:
        tok = torch.arange(N, device=dev, dtype=torch.long)
        qs = PackedQueryState(
            active_batch_idx=torch.arange(B, device=dev, dtype=torch.long).repeat_interleave(N),
            active_pos_idx=tok.repeat(B), active_token_idx=tok.repeat(B),
            query_valid_mask=torch.ones((B, N), device=dev, dtype=torch.bool),
            active_query_pos_padded=tok.unsqueeze(0).expand(B, -1), active_query_mask=None, all_valid=True,
            active_patch_mask=(tok >= prefix).repeat(B), active_rope_idx=(tok - prefix).clamp_min(0).repeat(B))
        if len(_IDENTITY_PLANS) >= 16:
            _IDENTITY_PLANS.clear()
        _IDENTITY_PLANS[key] = qs
    return qs


def _fp4_scale(mod: nn.Module) -> Tensor | None:
    """The NVFP4 activation scale of a frozen FastFP4Linear (its input's producer then writes the NVFP4
    operand x_hat directly), else None."""
    return mod.act_scale if LP.low_precision_state(mod) == "fp4" else None


def _fp4_linear(mod: "LP.FastFP4Linear", x: Tensor, site: str, epilogue: int = _lib.EPI_BIAS, **kw) -> Tensor:
    """A frozen FastFP4Linear (fp4_fast_linear.py:221-283): torch._scaled_mm's bf16 output
    bf16(x_hat . W_hat^T), then bf16(. * out_scale + bias), then `epilogue`'s LayerScale / residual --
    one GEMM with the accumulator rounded to bf16 before the scale (EPI_RAW_BF16)."""
    return K.linear(mod.quantize(x), mod.weight_hat, mod.bias, epilogue=epilogue | _lib.EPI_RAW_BF16,
                    acc_scale=mod.out_scale_f, site=site, **kw)


# ------------------------------------------------------------------------------------------------
# Plan types (attention.py:52-74; block.py:33-44)
# ------------------------------------------------------------------------------------------------


@dataclass
class PackedQueryState:
    """The packed rows of one plan, B x T of them (T = pretokens + patch slots). For the padded
    threshold builder the reference keeps only the rows at query_valid_mask; here the other slots are
    packed rows too, each repeating its image's last valid row, so they compute and write back exactly
    what that row does, and the rows at query_valid_mask are the reference's active rows."""
    active_batch_idx: Tensor
    active_pos_idx: Tensor
    active_token_idx: Tensor
    query_valid_mask: Tensor
    active_query_pos_padded: Tensor
    active_query_mask: Tensor
    all_valid: bool
    active_patch_mask: Tensor | None = None
    active_rope_idx: Tensor | None = None
    # Token -> packed row map [B, N] int32 (-1 off the plan); consumed by the fused residual kernel.
    row_slot: Tensor | None = None


@dataclass
class PartialTokenQueryPlan:
    update_indice: Tensor
    fixed_query_state: PackedQueryState
    server_patch_scores: Tensor
    mobile_patch_scores: Tensor | None
    combined_patch_scores: Tensor
    kept_pscore_mass: Tensor
    full_pscore_mass: Tensor
    kept_patch_total: Tensor
    full_patch_total: Tensor
    sample_total: Tensor


# ------------------------------------------------------------------------------------------------
# Parameter-holding modules
# ------------------------------------------------------------------------------------------------


class LayerScale(nn.Module):
    """layer_scale.py:12-29 (parameter holder)."""

    def __init__(self, dim: int, init_values: float = 1e-5, device=None):
        super().__init__()
        self.gamma = nn.Parameter(torch.empty(dim, device=device))
        self.init_values = init_values

    def reset_parameters(self):
        nn.init.constant_(self.gamma, self.init_values)


class LinearKMaskedBias(nn.Linear):
    """attention.py:39-49: the K third of the qkv bias is multiplied by a 0/1 mask."""

    def __init__(self, *args, **kwargs):
        super().__init__(*args, **kwargs)
        if self.out_features % 3 != 0:
            raise ValueError("qkv out_features must be a multiple of 3")
        if self.bias is not None:
            self.register_buffer("bias_mask", torch.full_like(self.bias, fill_value=math.nan))

    def masked_bias(self) -> Tensor | None:
        if self.bias is None:
            return None
        return self.bias * self.bias_mask.to(self.bias.dtype)


class Mlp(nn.Module):
    """ffn_layers.py:24-49: fc1 -> exact GELU -> fc2."""

    def __init__(self, in_features: int, hidden_features: int, bias: bool = True, device=None):
        super().__init__()
        self.fc1 = nn.Linear(in_features, hidden_features, bias=bias, device=device)
        self.fc2 = nn.Linear(hidden_features, in_features, bias=bias, device=device)


class SwiGLUFFN(nn.Module):
    """ffn_layers.py:60-115: silu(w1 x) * (w2 x) -> w3; hidden = int(h * 2/3) rounded up to align_to."""

    def __init__(self, in_features: int, hidden_features: int, bias: bool = True, align_to: int = 64, device=None):
        super().__init__()
        d = int(hidden_features * 2 / 3)
        hidden = d + (-d % align_to)
        self.w1 = nn.Linear(in_features, hidden, bias=bias, device=device)
        self.w2 = nn.Linear(in_features, hidden, bias=bias, device=device)
        self.w3 = nn.Linear(hidden, in_features, bias=bias, device=device)


class SelfAttention(nn.Module):
    """attention.py:77-110 (parameters) and the attention half of the correction step (:393-534)."""

    def __init__(self, dim: int, num_heads: int, qkv_bias: bool = False, proj_bias: bool = True,
                 mask_k_bias: bool = False, device=None):
        super().__init__()
        self.num_heads = num_heads
        self.head_dim = dim // num_heads
        self.scale = self.head_dim ** -0.5
        linear_class = LinearKMaskedBias if mask_k_bias else nn.Linear
        self.qkv = linear_class(dim, dim * 3, bias=qkv_bias, device=device)
        self.proj = nn.Linear(dim, dim, bias=proj_bias, device=device)
        self._bias_key = None
        self._bias_val = None

    def qkv_bias(self) -> Tensor | None:
        """Masked qkv bias, recomputed only when the bias or its mask changes."""
        b = self.qkv.bias
        if b is None:
            return None
        mask = getattr(self.qkv, "bias_mask", None)
        key = (b.data_ptr(), b._version, None if mask is None else (mask.data_ptr(), mask._version))
        if key != self._bias_key:
            val = b.detach() if mask is None else (b.detach() * mask.to(b.dtype))
            self._bias_val = val.to(torch.bfloat16).contiguous()
            self._bias_key = key
        return self._bias_val

    def correct_partial_token(self, x_sel: Tensor, dindice: Tensor, rope, cache_feature: Dict, tag: str, *,
                              fixed_query_state: PackedQueryState, sdpa_query_bucket_size: int = 0,
                              **_) -> Tuple[Tensor, Dict]:
        """Attention half of the correction for pre-normalised selected rows x_sel [M, C]:
        qkv, RoPE, in-place K/V rewrite, sparse-query attention, proj. Returns (proj(attn), cache).

        `sdpa_query_bucket_size` only padded the reference's SDPA query length; the kernel here
        reads the packed queries directly, so it has no effect on the result.
        """
        kv = cache_feature[f"{tag}_kv"]
        q_packed, attn = self._qkv_attention(x_sel, rope, kv, fixed_query_state)
        if LP.low_precision_state(self.proj) == "fp4":
            out = _fp4_linear(self.proj, attn, "proj")
        else:
            out = _linear_route(self.proj, attn, "proj")
        return out, cache_feature

    def _qkv_attention(self, xn: Tensor, rope, kv: Tensor, qs: PackedQueryState, xn_is_xhat: bool = False,
                       lse: Tensor | None = None, fp8_out: Tensor | None = None, warm: Tensor | None = None):
        """q, K/V rows and the attention output of the packed rows from their norm1 output xn -- for a
        frozen NVFP4 qkv linear, xn may already be its NVFP4 operand x_hat (xn_is_xhat: the producer wrote
        it). lse (fp32 [B, H, T]) receives the attention's row log-sum-exp when given. fp8_out (the
        frozen FP8 proj's activation inverse scale): the output is instead its e4m3fn codes (uint8). warm:
        a later launch's weight, read into the caches by the bf16 QKV GEMM's idle CUs."""
        M, C = xn.shape
        H, D = self.num_heads, self.head_dim
        B = kv.shape[0]
        if M % B != 0:
            raise ValueError(f"packed rows {M} do not split evenly over {B} images")
        T = M // B
        q = torch.empty((M, H, D), device=xn.device, dtype=torch.bfloat16)
        mod = self.qkv
        state = LP.low_precision_state(mod)
        if state == "fp4":
            # NVFP4: the bf16 GEMM output (fp4_fast_linear.py:221-249), then its scale and bias
            # (fp4_fast_linear.py:251-283) and RoPE and the K/V write -- in the GEMM's epilogue when it
            # takes whole heads, else on the way into RoPE and the K/V write (one kernel)
            xh = xn if xn_is_xhat else mod.quantize(xn)
            if K.qkv_fusable(H, D):
                K.linear_qkv_rope_kv(xh, mod.weight_hat, mod.bias, rope, qs.active_patch_mask, qs.active_rope_idx,
                                     qs.active_batch_idx, qs.active_token_idx, kv, q, acc_scale=mod.out_scale_f,
                                     raw_bf16=True)
            else:
                raw = K.linear(xh, mod.weight_hat, None, site="qkv")
                K.qkv_rope_kv_scatter(raw.view(M, 3, H, D), rope, qs.active_patch_mask, qs.active_rope_idx,
                                      qs.active_batch_idx, qs.active_token_idx, kv, q, scale=mod.out_scale_f,
                                      bias=mod.bias)
            qkv = None
        elif state == "fp8" and mod.native and K.qkv_fusable(H, D):
            K.linear_qkv_rope_kv_fp8(mod.quantize_codes(xn), mod.weight_q, self.qkv_bias(), rope, qs.active_patch_mask,
                                     qs.active_rope_idx, qs.active_batch_idx, qs.active_token_idx, kv, q,
                                     acc_scale=mod.acc_scale_f)
            qkv = None
        elif K.qkv_fusable(H, D):
            if state == "fp8":
                a, w, s = mod.quantize(xn), mod.weight_hat, mod.acc_scale_f
            else:
                if isinstance(mod, LP._LowPrecisionLinear):
                    mod.observe(xn)
                a, w, s = xn, mod.weight, 1.0
            K.linear_qkv_rope_kv(a, w, self.qkv_bias(), rope, qs.active_patch_mask, qs.active_rope_idx,
                                 qs.active_batch_idx, qs.active_token_idx, kv, q, acc_scale=s, warm=warm)
            qkv = None
        else:
            qkv = _linear_route(mod, xn, "qkv", bias=self.qkv_bias())
        if qkv is not None:
            K.qkv_rope_kv_scatter(qkv.view(M, 3, H, D), rope, qs.active_patch_mask, qs.active_rope_idx,
                                  qs.active_batch_idx, qs.active_token_idx, kv, q)
        if fp8_out is not None:
            return q, K.sparse_query_attention_fp8(q, kv, T, self.scale, fp8_out)
        attn = K.sparse_query_attention(q, kv, T, self.scale, lse=lse)
        return q, attn


# ------------------------------------------------------------------------------------------------
# The block
# ------------------------------------------------------------------------------------------------


class SelfAttentionBlock(nn.Module):
    _MOBILE_HINT_PSCORE_ALIASES = frozenset({
        "residual_rms", "patch_residual_rms", "residual_l2", "residual_l2_energy", "residual_energy",
        "patch_residual_l2", "patch_residual_energy",
    })
    _VALID_SERVER_PSCORES = frozenset({
        "cls_attn_prob", "patch_attn_prob", "patch_attn_prob_layermean", "patch_pseudo_attn_prob",
        "patch_pseudo_attn_prob_layermean", "cls_attn_prob_layermean", "random",
    })
    _LAYERMEAN_SERVER_PSCORES = frozenset({
        "patch_attn_prob_layermean", "patch_pseudo_attn_prob_layermean", "cls_attn_prob_layermean",
    })
    _PARTIAL_TOKEN_PLAN_CACHE_KEY = "_partial_token_query_plan_cache"

    def __init__(self, dim: int, num_heads: int, ffn_ratio: float = 4.0, qkv_bias: bool = False,
                 proj_bias: bool = True, ffn_bias: bool = True, init_values: float | None = None,
                 norm_eps: float = 1e-5, ffn_layer: str = "mlp", mask_k_bias: bool = False, device=None):
        super().__init__()
        self.norm1 = nn.LayerNorm(dim, eps=norm_eps, device=device)
        self.attn = SelfAttention(dim, num_heads, qkv_bias=qkv_bias, proj_bias=proj_bias, mask_k_bias=mask_k_bias,
                                  device=device)
        self.ls1 = LayerScale(dim, init_values, device=device) if init_values else nn.Identity()
        self.norm2 = nn.LayerNorm(dim, eps=norm_eps, device=device)
        hidden = int(dim * ffn_ratio)
        if ffn_layer == "mlp":
            self.mlp = Mlp(dim, hidden, bias=ffn_bias, device=device)
        elif ffn_layer.startswith("swiglu"):
            align = int(ffn_layer[len("swiglu"):] or 8)
            self.mlp = SwiGLUFFN(dim, hidden, bias=ffn_bias, align_to=align, device=device)
        else:
            raise ValueError(f"unknown ffn_layer {ffn_layer!r}")
        self.ls2 = LayerScale(dim, init_values, device=device) if init_values else nn.Identity()
        self._ones = None

    # -- helpers ---------------------------------------------------------------------------------

    def _gamma(self, ls: nn.Module, like: Tensor) -> Tensor:
        g = getattr(ls, "gamma", None)
        if g is not None:
            return g if g.dtype == torch.bfloat16 else g.to(torch.bfloat16)
        if self._ones is None or self._ones.device != like.device or self._ones.numel() != like.shape[-1]:
            self._ones = torch.ones(like.shape[-1], device=like.device, dtype=torch.bfloat16)
        return self._ones

    def _mlp_scaled(self, xn: Tensor, xn_is_xhat: bool = False, warm=(None, None)) -> Tensor:
        """gamma2 * MLP(xn) with GELU / SwiGLU and LayerScale fused into the GEMM epilogues; the SwiGLU
        linears in their low-precision route when the block is a converted view (dinov3/lowp.py). With
        NVFP4 linears xn may already be w1's NVFP4 operand x_hat (xn_is_xhat), and the SwiGLU kernel
        writes w3's x_hat directly. warm: the weights (or None) that the bf16 fc1 and fc2 GEMMs read
        into the caches from their idle CUs."""
        g2 = self._gamma(self.ls2, xn)
        if isinstance(self.mlp, Mlp):
            h = K.linear(xn, self.mlp.fc1.weight, self.mlp.fc1.bias, epilogue=_lib.EPI_BIAS_GELU, site="fc1",
                         warm=warm[0])
            return K.linear(h, self.mlp.fc2.weight, self.mlp.fc2.bias, epilogue=_lib.EPI_BIAS_LS, gamma=g2, site="fc2",
                            warm=warm[1])
        w1, w2, w3 = self.mlp.w1, self.mlp.w2, self.mlp.w3
        states = {LP.low_precision_state(m) for m in (w1, w2, w3)}
        if "fp4" in states:
            if states != {"fp4"}:
                raise RuntimeError("SwiGLU linears partially calibrated: freeze all three NVFP4 linears together")
            # ffn_layers.py:84-115 with FastFP4Linear: both epilogues folded into the SwiGLU kernel
            # (token_update.py:620-669), then w3 with its scale-and-bias and the LayerScale.
            # (w2 takes the activation w1 quantized: SharedFP4Activation, fp4_fast_linear.py:71-100)
            xh = xn if xn_is_xhat else w1.quantize(xn)
            r1 = K.linear(xh, w1.weight_hat, None, site="w1")
            if w2.out_features % 256 == 0:  # w2's GEMM finishes the SwiGLU and writes w3's operand
                xh3 = K.linear_swiglu_nvfp4(xh, w2.weight_hat, r1, w1.out_scale_f, w1.bias, w2.out_scale_f, w2.bias,
                                            w3.act_scale, site="w2")
            else:
                r2 = K.linear(xh, w2.weight_hat, None, site="w2")
                xh3 = K.swiglu_scaled(r1, w1.out_scale_f, w1.bias, r2, w2.out_scale_f, w2.bias,
                                      nvfp4_scale=w3.act_scale)
            # w3's scale and bias, then the LayerScale, in its GEMM epilogue (bf16(bf16(acc) s + b) * gamma)
            return K.linear(xh3, w3.weight_hat, w3.bias, epilogue=_lib.EPI_BIAS_LS | _lib.EPI_RAW_BF16, gamma=g2,
                            acc_scale=w3.out_scale_f, site="w3")
        x2 = _linear_route(w2, xn, "w2")
        h = _linear_route(w1, xn, "w1", epilogue=_lib.EPI_BIAS_SILU_MUL, resid=x2)
        return _linear_route(w3, h, "w3", epilogue=_lib.EPI_BIAS_LS, gamma=g2)

    # -- dispatch (block.py:274-310) --------------------------------------------------------------

    @annotate("approx")
    def approx(self, x: Tensor, rope, cache_feature: Dict, tag: str, **kwargs):
        method = kwargs.get("appcorr_method", "partial_token")
        if method != "partial_token":
            raise NotImplementedError(f"appcorr_method {method!r} is not part of this build (partial_token only)")
        return self.approx_partial_token(x, rope, cache_feature, tag, **kwargs)

    @annotate("correct")
    def correct(self, x: Tensor, dindice: Tensor, rope, cache_feature: Dict, tag: str, **kwargs):
        method = kwargs.get("appcorr_method", "partial_token")
        if method != "partial_token":
            raise NotImplementedError(f"appcorr_method {method!r} is not part of this build (partial_token only)")
        return self.correct_partial_token(x, dindice, rope, cache_feature, tag, **kwargs)

    # -- approximate pass: the cache producer (block.py:312-349; attention.py:215-278) -------------

    def approx_partial_token(self, x: Tensor, rope, cache_feature: Dict, tag: str, **kwargs):
        """Full forward over all tokens that caches {tag}_kv (K after RoPE) and
        {tag}_blocks_out_sum, on the same kernels as the correction (identity plan, T = N)."""
        server_pscore = str(kwargs.get("server_pscore", "cls_attn_prob"))
        if float(kwargs.get("server_pscore_weight", 1.0)) == 0.0:
            server_pscore = "none"
        self._invalidate_partial_token_derived_caches(cache_feature)
        B, N, C = x.shape
        H, D = self.attn.num_heads, self.attn.head_dim
        prefix = N - rope[0].shape[0] if rope is not None else N
        dev = x.device
        qs = _identity_query_state(B, N, prefix, dev)
        x2 = x.reshape(B * N, C)
        kv = torch.empty((B, N, 2, H, D), device=dev, dtype=torch.bfloat16)
        cache_feature[f"{tag}_kv"] = kv
        xn = K.layer_norm(x2, self.norm1.weight, self.norm1.bias, self.norm1.eps)
        # The fused key-side score reads the attention's own row log-sum-exp (one more pass over the
        # scores), as the reference takes cuDNN's (attention_pscore.py:172-241).
        lse = (torch.empty((B, H, N), device=dev, dtype=torch.float32)
               if self._fused_patch_score(server_pscore, H, D, N) else None)
        q, attn = self.attn._qkv_attention(xn, rope, kv, qs, lse=lse)
        g1 = self._gamma(self.ls1, x2)
        inc = K.linear(attn, self.attn.proj.weight, self.attn.proj.bias, epilogue=_lib.EPI_BIAS_LS, gamma=g1,
                       site="proj")
        ones = self._gamma(nn.Identity(), x2)
        x_attn = K.fused_layerscale_add(x2, inc, ones)                       # x + ls1(attn)
        mlp = self._mlp_scaled(K.layer_norm(x_attn, self.norm2.weight, self.norm2.bias, self.norm2.eps,
                                            prefetch=self._mlp_prefetch()))
        bos, out = K.residual_pair(inc, x_attn, mlp)  # block.py:336-347: inc + mlp cached, x_attn + mlp out
        cache_feature[f"{tag}_blocks_out_sum"] = bos.view(B, N, C)
        out = out.view(B, N, C)
        if server_pscore not in ("none", "disabled"):
            cache_feature[f"{tag}_server_pscore"] = self._server_pscore(q.view(B, N, H, D), kv, server_pscore,
                                                                        N - prefix, lse=lse)
        return out, cache_feature

    _PATCH_ATTN_PSCORES = frozenset({"patch_attn_prob", "patch_attn_prob_layermean"})
    _PSEUDO_ATTN_PSCORES = frozenset({"patch_pseudo_attn_prob", "patch_pseudo_attn_prob_layermean"})

    @classmethod
    def _fused_patch_score(cls, kind: str, H: int, D: int, N: int) -> bool:
        """The reference's fused key-side score applies (attention.py:241-250; the shape limits of
        attention_pscore.py:100-131)."""
        return kind == "patch_attn_prob_layermean" and H == 32 and D == 128 and 0 < N <= 4096

    def _server_pscore(self, q: Tensor, kv: Tensor, kind: str, num_patches: int, lse: Tensor | None = None) -> Tensor:
        """The approx pass's server score (attention.py:241-273) from the queries q [B, N, H, Dh] and the
        cache kv [B, N, 2, H, Dh] (both after RoPE), with the reference's rounding points:
          patch_attn_prob(_layermean): mean over heads, then over all queries, of the full softmax
          (:251-253), bf16 [B, N]; patch_attn_prob_layermean on 32 heads of 128 with N <= 4096 takes the
          fused key-side sum from the row log-sum-exp instead (:241-250, attention_pscore.py:100-131) --
          the attention's own (lse [B, H, N]) when the caller has it, else computed here;
          patch_pseudo_attn_prob(_layermean): softmax of the pseudo query (:254-261), bf16 [B, N];
          any other kind (cls_attn_prob, cls_attn_prob_layermean, random: the reference's else branch,
          :266-271): softmax of the cls query over all keys, mean over heads, fp32 [B, N]."""
        if kind in self._PATCH_ATTN_PSCORES:
            B, N, H, D = q.shape
            fused = self._fused_patch_score(kind, H, D, N)
            if fused and lse is not None:
                return K.patch_attention_prob_from_lse(q.reshape(B * N, H, D), kv, self.attn.scale, lse)
            return K.patch_attention_prob(q.reshape(B * N, H, D), kv, self.attn.scale,
                                          K.PATTN_LSE if fused else K.PATTN_DENSE)
        if kind in self._PSEUDO_ATTN_PSCORES:
            qp = K.pseudo_query(q[:, q.shape[1] - num_patches:])
            return K.query_attention_prob(qp, kv, self.attn.scale, out_dtype=torch.bfloat16)
        return K.query_attention_prob(q[:, 0], kv, self.attn.scale)

    # -- plan bookkeeping (block.py:358-940) --------------------------------------------------------

    @staticmethod
    def _tensor_cache_signature(t: Tensor | None):
        if t is None:
            return None
        try:
            version = t._version
        except RuntimeError:
            version = None
        return (t.data_ptr(), tuple(t.shape), tuple(t.stride()), t.storage_offset(), str(t.device), str(t.dtype),
                version)

    @classmethod
    def _shared_partial_token_plan_key(cls, *, dindice, mobile_pscore_hint, num_pretokens, num_tokens,
                                       token_keep_ratio, token_keep_thres, server_pscore, server_pscore_weight,
                                       mobile_pscore, mobile_pscore_weight, pscore_fusion):
        """Plans are shared across layers only when the score does not depend on the layer
        (block.py:709-741): server weight 0, or a layer-mean server score."""
        if server_pscore_weight != 0.0 and server_pscore not in cls._LAYERMEAN_SERVER_PSCORES:
            return None
        return ("partial_token", cls._tensor_cache_signature(dindice), cls._tensor_cache_signature(mobile_pscore_hint),
                num_pretokens, num_tokens, float(token_keep_ratio), token_keep_thres, server_pscore,
                float(server_pscore_weight), mobile_pscore, float(mobile_pscore_weight), pscore_fusion)

    @classmethod
    def _get_partial_token_plan_cache(cls, cache_feature: Dict) -> Dict:
        pc = cache_feature.setdefault(cls._PARTIAL_TOKEN_PLAN_CACHE_KEY, {})
        if not isinstance(pc, dict):
            raise RuntimeError(f"{cls._PARTIAL_TOKEN_PLAN_CACHE_KEY} must be a dict")
        return pc

    @classmethod
    def _invalidate_partial_token_derived_caches(cls, cache_feature: Dict) -> None:
        cache_feature.pop(cls._PARTIAL_TOKEN_PLAN_CACHE_KEY, None)
        for key in [k for k in cache_feature if k.startswith("_shared_")]:
            cache_feature.pop(key, None)

    def _resolve_mobile_patch_scores(self, mobile_pscore, hint, dindice_patches, *, num_pretokens, num_tokens):
        """block.py:638-667."""
        if mobile_pscore not in self._MOBILE_HINT_PSCORE_ALIASES or hint is None:
            return None
        if hint.shape[0] != dindice_patches.shape[0]:
            raise RuntimeError(f"Mobile pscore hint batch mismatch: hint={tuple(hint.shape)} "
                               f"candidates={tuple(dindice_patches.shape)}")
        if hint.shape[1] == num_tokens - num_pretokens:
            return hint.gather(1, dindice_patches - num_pretokens)
        if hint.shape[1] == num_tokens:
            return hint.gather(1, dindice_patches)
        raise RuntimeError(f"Unsupported mobile pscore hint shape {tuple(hint.shape)} for num_tokens={num_tokens}, "
                           f"num_pretokens={num_pretokens}")

    @staticmethod
    def _combine_patch_scores(server, server_w, mobile, mobile_w, fusion):
        """block.py:669-687."""
        combined = server_w * server
        if mobile is None or mobile_w == 0.0:
            return combined
        term = mobile_w * mobile.to(dtype=combined.dtype)
        if fusion == "multiply":
            return combined * term
        if fusion == "geo_mean":
            return torch.sqrt(torch.clamp(combined * term, min=0.0))
        return combined + term

    def _resolve_server_token_scores(self, cache_feature: Dict, tag: str, server_pscore: str) -> Tensor:
        """block.py:862-940 (layer-mean averaging over this stack, the per-stack random control)."""
        if server_pscore in self._LAYERMEAN_SERVER_PSCORES:
            stack = tag.rstrip("0123456789")
            ck = f"_shared_{server_pscore}_server_pscore_mean_{stack}"
            cached = cache_feature.get(ck)
            if cached is not None:
                return cached
            keys = tuple(sorted(k for k, v in cache_feature.items()
                                if k.endswith("_server_pscore") and isinstance(v, Tensor)
                                and k[: -len("_server_pscore")].rstrip("0123456789") == stack))
            if not keys:
                raise KeyError(f"Missing cached *_server_pscore entries for stack '{stack}'. "
                               "They must be produced during approx.")
            ts = [cache_feature[k] for k in keys]
            if any(t.shape != ts[0].shape for t in ts[1:]):
                raise RuntimeError("Cannot average server pscores across layers with inconsistent shapes")
            mean = torch.stack(ts, dim=0).mean(dim=0)
            cache_feature[ck] = mean.detach()
            cache_feature[f"{ck}_keys"] = keys
            return mean
        scores = cache_feature.get(f"{tag}_server_pscore")
        if scores is None:
            raise KeyError(f"Missing cached {tag}_server_pscore. It must be produced during approx.")
        if server_pscore == "random":
            stack = tag.rstrip("0123456789")
            key = f"_shared_random_server_pscore_{stack}"
            cached = cache_feature.get(key)
            if cached is None:
                cached = torch.rand_like(scores)
                cache_feature[key] = cached
            return cached
        return scores

    _PLAN_STAT_KEYS = ("_token_pscore_kept_mass_total", "_token_pscore_full_mass_total",
                       "_partial_token_kept_patch_total", "_partial_token_full_patch_total",
                       "_partial_token_sample_total")

    @staticmethod
    def _accumulate_partial_token_plan_stats(cache_feature: Dict, plan: PartialTokenQueryPlan, scale: float = 1.0):
        """block.py:790-844: running kept / full score mass and patch counts, total = total + value
        (value * scale when scale != 1) for the five statistics, as fresh tensors; all five in one
        multi-tensor launch. A missing total starts from the value itself, which equals 0 + value
        here: the plan's statistics already carry the + 0 (plan_stats)."""
        keys = SelfAttentionBlock._PLAN_STAT_KEYS
        vals = [plan.kept_pscore_mass, plan.full_pscore_mass, plan.kept_patch_total, plan.full_patch_total,
                plan.sample_total]
        if scale != 1.0:
            vals = list(torch._foreach_mul(vals, scale))
        prev = [cache_feature.get(k) for k in keys]
        if all(p is None for p in prev) and scale == 1.0:
            for k, v in zip(keys, vals):
                cache_feature[k] = v
            return
        prev = [v.new_zeros((), dtype=torch.float32) if p is None else p for p, v in zip(prev, vals)]
        for k, t in zip(keys, torch._foreach_add(prev, vals)):
            cache_feature[k] = t

    @annotate("build_packed_query_state")
    def _build_query_plan(self, x: Tensor, dindice: Tensor, rope, cache_feature: Dict, tag: str, kw: dict,
                          num_pretokens: int) -> PartialTokenQueryPlan:
        B, N, _ = x.shape
        dindice_patches = dindice[:, num_pretokens:]
        mobile = None
        if kw["mobile_pscore"] != "none" and kw["mobile_pscore_weight"] != 0.0:
            mobile = self._resolve_mobile_patch_scores(kw["mobile_pscore"], kw["mobile_pscore_hint"], dindice_patches,
                                                       num_pretokens=num_pretokens, num_tokens=N)
        if kw["server_pscore_weight"] == 0.0:
            server = x.new_zeros((B, dindice_patches.shape[1]), dtype=torch.float32)
        else:
            server = self._resolve_server_token_scores(cache_feature, tag, kw["server_pscore"]).gather(1,
                                                                                                       dindice_patches)
        if (kw["server_pscore_weight"] == 0.0 and kw["mobile_pscore_weight"] == 1.0 and mobile is not None
                and mobile.dtype == torch.float32 and kw["pscore_fusion"] not in ("multiply", "geo_mean")):
            # 0 * 0 + 1 * mobile is mobile itself (up to the sign of a zero score, which ranks and
            # sums the same): no launches for the combine.
            combined = mobile
        else:
            combined = self._combine_patch_scores(server, kw["server_pscore_weight"], mobile,
                                                  kw["mobile_pscore_weight"], kw["pscore_fusion"])
        cvm = kw.get("candidate_valid_mask")
        if cvm is not None:
            combined = combined.masked_fill(~cvm.to(combined.device), float("-inf"))
        Pn = dindice_patches.shape[1]
        scores = combined.to(torch.float32).contiguous()
        thres = kw["token_keep_thres"]
        all_valid = True
        if thres is None:                                       # top-k (block.py:377-394, 397-490)
            ratio = float(kw["token_keep_ratio"])
            k = Pn if ratio >= 1.0 else min(int(Pn * ratio), Pn)
            tp = K.topk_plan(scores, k, dindice.contiguous(), num_pretokens, N)
            valid = None
        elif kw["token_keep_cap"] > 0:                          # fixed width, sync-free (block.py:492-560)
            width = max(0, min(int(kw["token_keep_cap"]), Pn))
            tp = K.threshold_plan(scores, thres, dindice.contiguous(), num_pretokens, width, padded=False,
                                  num_tokens=N)
            valid = None
        else:                                                   # padded (block.py:562-621)
            # The width is the largest kept count, read back to the host as the reference's .item()
            # does (block.py:570); rows past an image's count are not queries.
            _, counts = K.threshold_keep(scores, thres)
            counts_h = counts.cpu()
            width = int(counts_h.max()) if B > 0 else 0
            if num_pretokens == 0 and width > 0 and int(counts_h.min()) == 0:
                raise NotImplementedError("padded threshold plan with num_pretokens == 0: an image that keeps no "
                                          "candidate has no row to stand in for its padding; set token_keep_cap")
            tp = K.threshold_plan(scores, thres, dindice.contiguous(), num_pretokens, width, padded=True,
                                  num_tokens=N)
            valid = tp.query_valid
            all_valid = bool(B <= 1 or valid.numel() == 0 or bool((counts_h == width).all()))
        T = tp.update_indice.shape[1]
        if valid is None:
            valid = torch.ones((B, T), device=x.device, dtype=torch.bool)
        qs = PackedQueryState(
            active_batch_idx=tp.active_batch_idx, active_pos_idx=tp.active_pos_idx,
            active_token_idx=tp.active_token_idx, query_valid_mask=valid,
            active_query_pos_padded=torch.arange(T, device=x.device, dtype=torch.long).unsqueeze(0).expand(B, -1),
            active_query_mask=valid, all_valid=all_valid, active_patch_mask=tp.active_patch_mask,
            active_rope_idx=tp.active_rope_idx, row_slot=tp.row_slot)
        keep = tp.keep_mask
        stats = K.plan_stats(scores, keep)  # block.py:762-788 in one launch
        return PartialTokenQueryPlan(
            update_indice=tp.update_indice, fixed_query_state=qs, server_patch_scores=server.detach(),
            mobile_patch_scores=None if mobile is None else mobile.detach(), combined_patch_scores=combined.detach(),
            kept_pscore_mass=stats[0], full_pscore_mass=stats[1], kept_patch_total=stats[2],
            full_patch_total=stats[3], sample_total=stats[4])

    # -- the correction step (block.py:942-1191) ---------------------------------------------------

    def _prepare_correction(self, x: Tensor, dindice: Tensor, rope, cache_feature: Dict, tag: str, kwargs: Dict):
        """Options, the (cached) query plan and its statistics, the per-tag score keys and the cache
        tensors of one correction block (block.py:942-1110). Returns (plan, plan_key, kv, bos)."""
        debug = bool(kwargs.get("debug", False))
        kw = {
            "token_keep_ratio": kwargs.get("token_keep_ratio", 0.2),
            "token_keep_thres": None if kwargs.get("token_keep_thres") in (None, "", "null", "None")
            else float(kwargs["token_keep_thres"]),
            # > 0 with a threshold: the fixed-width, sync-free builder (block.py:949-951, 1055-1062)
            "token_keep_cap": int(kwargs.get("token_keep_cap", 0) or 0),
            "server_pscore_weight": float(kwargs.get("server_pscore_weight", 1.0)),
            "server_pscore": str(kwargs.get("server_pscore", "cls_attn_prob")),
            "mobile_pscore": str(kwargs.get("mobile_pscore", "none")),
            "mobile_pscore_weight": float(kwargs.get("mobile_pscore_weight", 0.0)),
            "mobile_pscore_hint": kwargs.get("mobile_pscore_hint"),
            "pscore_fusion": str(kwargs.get("pscore_fusion", "add")).lower(),
            "candidate_valid_mask": kwargs.get("candidate_valid_mask"),
        }
        if kw["pscore_fusion"] not in ("add", "multiply", "geo_mean"):
            kw["pscore_fusion"] = "add"
        if kw["server_pscore"] not in self._VALID_SERVER_PSCORES:
            raise ValueError(f"Unknown server_pscore '{kw['server_pscore']}'. "
                             f"Available values: {sorted(self._VALID_SERVER_PSCORES)}")
        if x.dtype != torch.bfloat16 or x.dim() != 3:
            raise ValueError("correct_partial_token expects x [B, N, C] bf16")
        B, N, C = x.shape
        num_pretokens = kwargs.get("num_pretokens")
        if num_pretokens is None:
            num_pretokens = N - rope[0].shape[0]
        num_pretokens = int(num_pretokens)

        key = self._shared_partial_token_plan_key(
            dindice=dindice, mobile_pscore_hint=kw["mobile_pscore_hint"] if kw["mobile_pscore_weight"] != 0.0 else None,
            num_pretokens=num_pretokens, num_tokens=N, token_keep_ratio=kw["token_keep_ratio"],
            token_keep_thres=kw["token_keep_thres"], server_pscore=kw["server_pscore"],
            server_pscore_weight=kw["server_pscore_weight"], mobile_pscore=kw["mobile_pscore"],
            mobile_pscore_weight=kw["mobile_pscore_weight"], pscore_fusion=kw["pscore_fusion"])
        plan = None
        if key is not None:
            plan = self._get_partial_token_plan_cache(cache_feature).get(key)
            if plan is not None and not isinstance(plan, PartialTokenQueryPlan):
                raise RuntimeError("Corrupt partial-token query-plan cache entry")
        hit = plan is not None
        if plan is None:
            plan = self._build_query_plan(x, dindice, rope, cache_feature, tag, kw, num_pretokens)
            if key is not None:
                self._get_partial_token_plan_cache(cache_feature)[key] = plan
        if not hit:
            scale = float(kwargs.get("partial_token_plan_stat_scale", 1.0)) if key is not None else 1.0
            self._accumulate_partial_token_plan_stats(cache_feature, plan, scale=scale)
        if plan.mobile_patch_scores is not None:
            cache_feature[f"{tag}_mobile_pscore_sel"] = plan.mobile_patch_scores
        cache_feature[f"{tag}_server_pscore_sel"] = plan.server_patch_scores
        cache_feature[f"{tag}_combined_pscore"] = plan.combined_patch_scores
        if debug:
            cache_feature[f"{tag}_update_indice"] = plan.update_indice

        kv = cache_feature[f"{tag}_kv"]
        bos = cache_feature[f"{tag}_blocks_out_sum"]
        if kv.dtype != torch.bfloat16 or bos.dtype != torch.bfloat16:
            raise ValueError("the correction cache ({tag}_kv, {tag}_blocks_out_sum) must be bf16")
        if not bos.is_contiguous():
            raise ValueError("{tag}_blocks_out_sum must be contiguous")
        return plan, key, kv, bos

    def _correct_rows(self, x_act: Tensor, rope, kv: Tensor, qs: PackedQueryState, xn: Tensor | None = None,
                      residual=None, xn_is_xhat: bool = False, next_block: "SelfAttentionBlock | None" = None):
        """The block's arithmetic on the packed selected rows (block.py:1111-1141): returns
        (x_attn, mlp); the K/V cache rows of the selected tokens are rewritten in place. `xn`, when
        given, is norm1(x_act) already computed (by the previous block's fused residual step).
        `residual` = (blocks_out_sum, next block's norm1 or None): when the last MLP product splits K,
        its reduce runs fused with the packed residual step, and the second value returned is then
        (x_new, norm1(x_new) or None) instead of mlp (see _mlp_scaled_residual). `next_block` (the block
        that runs next in a packed run, or None): the bf16 GEMMs read the weights of later launches
        into the caches from the CUs they leave idle -- qkv proj's, proj fc1's, fc1 fc2's (else
        norm2's launch does), fc2 the next block's qkv -- a cache hint only."""
        with trace_range("correct_attn"):
            if xn is None:   # block.py:1114 (an NVFP4 qkv linear's x_hat, written by the LayerNorm itself)
                ts1 = _fp4_scale(self.attn.qkv)
                xn = K.layer_norm(x_act, self.norm1.weight, self.norm1.bias, self.norm1.eps, nvfp4_scale=ts1)
                xn_is_xhat = ts1 is not None
            proj = self.attn.proj
            # A native FP8 proj takes the attention's output as e4m3 codes written by the attention itself
            # (its activation quantizer in the attention's store, one launch fewer).
            fp8_codes = (LP.low_precision_state(proj) == "fp8" and proj.native and self.attn.head_dim == 128)
            fc1 = self.mlp.fc1 if isinstance(self.mlp, Mlp) else None
            _, attn = self.attn._qkv_attention(xn, rope, kv, qs, xn_is_xhat,           # attention.py:415-523
                                               fp8_out=proj.act_inv_f32 if fp8_codes else None,
                                               warm=_bf16_weight(proj))
            g1 = self._gamma(self.ls1, x_act)
            # proj warms fc1's weight, fc1 fc2's (norm2's launch does where fc1's leaves no CU idle)
            fc2_w = self._mlp_prefetch()
            proj_warm = _bf16_weight(fc1) if _bf16_weight(proj) is not None else None
            fc1_warms = (fc2_w is not None and
                         K.linear_warm_slots(x_act.shape[0], fc1.out_features, fc1.in_features,
                                             _lib.EPI_BIAS_GELU) > 0)
            if fp8_codes:
                x_attn = proj.linear_codes(attn, proj.bias, "proj", epilogue=_lib.EPI_BIAS_LS_RESID, gamma=g1,
                                           resid=x_act)
            elif LP.low_precision_state(proj) == "fp4":                                  # proj_precision "fp4"
                x_attn = _fp4_linear(proj, attn, "proj", epilogue=_lib.EPI_BIAS_LS_RESID, gamma=g1, resid=x_act)
            else:
                x_attn = _linear_route(proj, attn, "proj", epilogue=_lib.EPI_BIAS_LS_RESID,  # attention.py:532 +
                                       gamma=g1, resid=x_act,                             # block.py:1129-1134
                                       **({} if proj_warm is None else {"warm": proj_warm}))
        with trace_range("correct_ffn"):
            ts2 = None if isinstance(self.mlp, Mlp) else _fp4_scale(self.mlp.w1)
            xn2 = K.layer_norm(x_attn, self.norm2.weight, self.norm2.bias, self.norm2.eps, nvfp4_scale=ts2,  # :1141
                               prefetch=None if fc1_warms else fc2_w)
            if residual is not None and ts2 is None:
                fused = self._mlp_scaled_residual(xn2, x_act, x_attn, qs, *residual)
                if fused is not None:
                    return x_attn, fused
            nb = next_block
            warm = (fc2_w if fc1_warms else None, None if nb is None else _bf16_weight(nb.attn.qkv))
            mlp = self._mlp_scaled(xn2, xn_is_xhat=ts2 is not None, warm=warm)
        return x_attn, mlp

    def _mlp_prefetch(self) -> Tensor | None:
        """fc2's weight (8 MB at ViT-L), read by the MLP's second GEMM after fc1 and otherwise fetched from
        HBM on first touch (measured at the headline: fc2 48.7 -> 43.7 us per block warmed): warmed by
        fc1's idle CUs in the correction, else by norm2's launch. bf16 Mlp only; None otherwise."""
        if isinstance(self.mlp, Mlp) and LP.low_precision_state(self.mlp.fc2) == "bf16":
            return self.mlp.fc2.weight
        return None

    def _mlp_scaled_residual(self, xn: Tensor, x_act: Tensor, x_attn: Tensor, qs: PackedQueryState, bos: Tensor,
                             next_norm):
        """_mlp_scaled followed by the packed residual step (block.py:1140-1186) and the next block's
        norm1, with the last product's split-K reduce and the residual step in one kernel: (x_new,
        norm1(x_new) or None), bit-identical to the unfused steps. None (nothing computed) unless the
        MLP is bf16 throughout (GELU fc1 / fc2, or SwiGLU w1 / w2 / w3 as plain linears), its last
        product splits K (small row counts: ViT-S / ViT-B, ViT-L keep 10 %) and the width is at most
        1024: the fused step runs a wave per row, which at the ViT-7B width (4096, w3 in two slices)
        was slower than the element-parallel reduce plus the residual step (pass 31.65 -> 31.77 ms),
        while ViT-S / ViT-B / ViT-L keep 10 % gained 4.5 / 1.8 / 1.3 %."""
        ln = None if next_norm is None else (next_norm.weight, next_norm.bias, next_norm.eps)
        M = xn.shape[0]
        if x_act.shape[1] > 1024:
            return None
        if isinstance(self.mlp, Mlp):
            fc1, last = self.mlp.fc1, self.mlp.fc2
        elif all(type(m) is nn.Linear for m in (self.mlp.w1, self.mlp.w2, self.mlp.w3)):
            fc1, last = None, self.mlp.w3
        else:
            return None
        if not K.linear_splits_k(M, last.out_features, last.in_features):
            return None
        g2 = self._gamma(self.ls2, xn)
        if fc1 is not None:
            h = K.linear(xn, fc1.weight, fc1.bias, epilogue=_lib.EPI_BIAS_GELU, site="fc1")
            site = "fc2"
        else:
            x2 = K.linear(xn, self.mlp.w2.weight, self.mlp.w2.bias, site="w2")
            h = K.linear(xn, self.mlp.w1.weight, self.mlp.w1.bias, epilogue=_lib.EPI_BIAS_SILU_MUL, resid=x2,
                         site="w1")
            site = "w3"
        out = K.linear_ls_packed_residual(h, last.weight, last.bias, g2, x_act, x_attn, qs.active_batch_idx,
                                          qs.active_token_idx, bos, ln, site=site)
        if out is None:  # an operand the fused step cannot take: the unfused last product and step
            mlp = K.linear(h, last.weight, last.bias, epilogue=_lib.EPI_BIAS_LS, gamma=g2, site=site)
            if ln is None:
                return K.packed_residual_persist(x_act, x_attn, mlp, qs.active_batch_idx, qs.active_token_idx,
                                                 bos), None
            return K.packed_residual_persist_ln(x_act, x_attn, mlp, qs.active_batch_idx, qs.active_token_idx, bos,
                                                *ln)
        return out

    @annotate("correct_partial_token")
    def correct_partial_token(self, x: Tensor, dindice: Tensor, rope, cache_feature: Dict, tag: str, **kwargs):
        plan, _, kv, bos = self._prepare_correction(x, dindice, rope, cache_feature, tag, kwargs)
        qs = plan.fixed_query_state
        inplace = bool(kwargs.get("inplace_residual_add", False)) and not torch.is_grad_enabled()
        xc = x if x.is_contiguous() else x.contiguous()
        out = xc if inplace else torch.empty_like(xc)
        M = qs.active_token_idx.numel()
        if M == 0:
            empty = xc.new_empty((0, xc.shape[-1]))
            return K.reconstruct_scatter_persist(xc, bos, qs.row_slot, empty, empty, empty, out=out), cache_feature

        x_act = K.gather_rows(xc, qs.active_batch_idx, qs.active_token_idx)          # block.py:1111
        x_attn, mlp = self._correct_rows(x_act, rope, kv, qs)
        out = K.reconstruct_scatter_persist(xc, bos, qs.row_slot, x_act, x_attn, mlp, out=out)  # :1140-1179
        if os.environ.get("APPCORR_PERSIST_TRACE") and not getattr(SelfAttentionBlock, "_persist_traced", False):
            SelfAttentionBlock._persist_traced = True
            print(f"[persist] blocks_out_sum write executed, tag={tag} rows={M}", flush=True)
        return out, cache_feature


@annotate("correct_blocks_packed")
def correct_blocks_packed(blocks, x: Tensor, dindice: Tensor, rope, cache_feature: Dict, tags, **kwargs):
    """A run of correction blocks with one query plan, the selected rows kept packed between blocks.

    Same results, bit for bit, as calling blocks[i].correct(...) in turn (block.py:942-1191 per
    block, the executor loop of dinov3_classifier.py:591-663): every block recomputes exactly the
    selected rows, and an unselected row only ever receives x + blocks_out_sum of each block, which
    does not depend on the correction. So the selected rows are gathered once, carried packed through
    the blocks (each block persists its blocks_out_sum rows and K/V rows as usual), and the full
    tensor is written once at the end: packed rows scattered back, every other row folded through
    the blocks' blocks_out_sum with the per-block bf16 rounding. Saves a gather and a full-tensor
    pass per block.

    Returns (x_out, cache_feature), or None when the blocks would not share one plan (the plan
    depends on per-layer server scores), in which case the caller runs the blocks one by one.
    """
    if not blocks:
        return x, cache_feature
    # Decided before anything is computed or cached: the plan is shared across blocks exactly when
    # _shared_partial_token_plan_key returns a key (server weight 0, or a layer-mean server score).
    server_w = float(kwargs.get("server_pscore_weight", 1.0))
    if server_w != 0.0 and str(kwargs.get("server_pscore", "cls_attn_prob")) not in \
            SelfAttentionBlock._LAYERMEAN_SERVER_PSCORES:
        return None
    plan0, key, _, _ = blocks[0]._prepare_correction(x, dindice, rope, cache_feature, tags[0], kwargs)
    if key is None:
        raise RuntimeError("packed correction run: the query plan is not shared across blocks")
    qs = plan0.fixed_query_state
    inplace = bool(kwargs.get("inplace_residual_add", False)) and not torch.is_grad_enabled()
    xc = x if x.is_contiguous() else x.contiguous()
    M = qs.active_token_idx.numel()
    # norm1 of the next block on x_p (from the gather for block 0, from the fused residual + LayerNorm
    # step after that), written as that block's NVFP4 qkv operand when xn_is_xhat
    xn, xn_is_xhat = None, False
    if M:
        ts0 = _fp4_scale(blocks[0].attn.qkv)
        n1 = blocks[0].norm1
        x_p, xn = K.gather_rows_ln(xc, qs.active_batch_idx, qs.active_token_idx, n1.weight, n1.bias, n1.eps,
                                   nvfp4_scale=ts0)
        xn_is_xhat = ts0 is not None
    else:
        x_p = xc.new_empty((0, xc.shape[-1]))
    bos_list = []
    for i, (blk, tag) in enumerate(zip(blocks, tags)):
        if i == 0:
            plan, kv, bos = plan0, cache_feature[f"{tag}_kv"], cache_feature[f"{tag}_blocks_out_sum"]
        else:
            plan, _, kv, bos = blk._prepare_correction(xc, dindice, rope, cache_feature, tag, kwargs)
        if plan is not plan0:
            raise RuntimeError("blocks of one packed run resolved different query plans")
        if x_p.shape[0] > 0:
            ts_next = _fp4_scale(blocks[i + 1].attn.qkv) if i + 1 < len(blocks) else None
            nxt = blocks[i + 1].norm1 if i + 1 < len(blocks) and ts_next is None else None
            x_attn, mlp = blk._correct_rows(x_p, rope, kv, qs, xn=xn, residual=(bos, nxt), xn_is_xhat=xn_is_xhat,
                                            next_block=blocks[i + 1] if i + 1 < len(blocks) else None)
            if isinstance(mlp, tuple):  # the residual step ran fused with the last MLP product
                x_p, xn = mlp
                xn_is_xhat = False
            elif i + 1 < len(blocks):
                n1 = blocks[i + 1].norm1
                x_p, xn = K.packed_residual_persist_ln(x_p, x_attn, mlp, qs.active_batch_idx, qs.active_token_idx,
                                                       bos, n1.weight, n1.bias, n1.eps, nvfp4_scale=ts_next)
                xn_is_xhat = ts_next is not None
            else:
                x_p = K.packed_residual_persist(x_p, x_attn, mlp, qs.active_batch_idx, qs.active_token_idx, bos)
        bos_list.append(bos)
    out = K.fold_residual_rows(xc, qs.row_slot, x_p, bos_list, out=xc if inplace else None, ptr_holder=cache_feature)
    return out, cache_feature
