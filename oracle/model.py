"""DINOv3 block restated on the CPU with torch: weights, RoPE tables, the approximate pass (cache
producer) and the partial-token correction pass. Test infrastructure only.

Reference files followed (ckswjd99-lab/AppCorr):
  model shapes / init        appcorr/models/dinov3/hub/backbones.py:201-237, 279-315, 318-371, 452-494;
                             models/vision_transformer.py:30-57 (init_weights_vit), 300-306
  RoPE tables                layers/rope_position_encoding.py:57-121 (base 100, "separate", fp32)
  rotate-half RoPE           layers/attention.py:24-36; triton_kernels/rope.py:120-183
  K-masked qkv bias          layers/attention.py:39-49 (+ mask init vision_transformer.py:46-49)
  approx pass                layers/block.py:312-349; layers/attention.py:215-278, 370-391
  correction pass            layers/block.py:942-1191; layers/attention.py:393-534
  MLP / SwiGLU               layers/ffn_layers.py:24-49, 60-115; LayerScale layers/layer_scale.py:28-29

Two arithmetic modes:
  "f64"  every product, sum and reduction in float64, rounded to bf16 exactly where the reference
         materialises a bf16 tensor (see the rounding points listed in `correct_block`). This is the
         parity oracle: the GPU may differ only by fp32 accumulation order.
  "bf16" the reference's own eager op sequence on bf16 CPU tensors (torch CPU kernels). Used only
         as the timed CPU baseline.
RoPE is fp32 arithmetic in both modes, as in the reference (its tables are fp32).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np
import torch
import torch.nn.functional as F


@dataclass(frozen=True)
class ViTConfig:
    name: str
    dim: int
    depth: int
    heads: int
    ffn: str            # "mlp" (fc1 -> GELU -> fc2) or "swiglu" (w1, w2 -> silu * -> w3)
    ffn_hidden: int
    qkv_bias: bool
    img_size: int
    patch_size: int = 16
    n_storage_tokens: int = 4
    ln_eps: float = 1e-5
    layerscale_init: float = 1e-5
    rope_base: float = 100.0

    @property
    def head_dim(self) -> int:
        return self.dim // self.heads

    @property
    def num_pretokens(self) -> int:
        return 1 + self.n_storage_tokens

    @property
    def grid(self) -> int:
        return self.img_size // self.patch_size

    @property
    def num_patches(self) -> int:
        return self.grid * self.grid

    @property
    def num_tokens(self) -> int:
        return self.num_pretokens + self.num_patches


# BASELINE.json configs (hub factories; ffn hidden per ffn_layers.py / SwiGLU 2/3 rule aligned to 64).
CONFIGS = {
    "vits16_224": ViTConfig("vits16_224", 384, 12, 6, "mlp", 1536, True, 224),
    "vitb16_512": ViTConfig("vitb16_512", 768, 12, 12, "mlp", 3072, True, 512),
    "vitl16_512": ViTConfig("vitl16_512", 1024, 24, 16, "mlp", 4096, True, 512),
    "vit7b16_1024": ViTConfig("vit7b16_1024", 4096, 40, 32, "swiglu", 8192, False, 1024),
}


def with_overrides(cfg: ViTConfig, **kw) -> ViTConfig:
    d = dict(cfg.__dict__)
    d.update(kw)
    return ViTConfig(**d)


# ------------------------------------------------------------------------------------------------
# Weights and inputs
# ------------------------------------------------------------------------------------------------


def make_block_weights(cfg: ViTConfig, seed: int = 0, *, gamma: float | None = None, bias_std: float = 0.0,
                       ln_std: float = 0.0, depth: int | None = None) -> list[dict]:
    """Per-block bf16 weights named like the reference module tree (block.py, attention.py).

    Linear weights ~ N(0, 0.02) (trunc_normal_ at +-2 is inert at that std), biases 0, LayerNorm
    (1, 0), LayerScale = layerscale_init (vision_transformer.py:41-57). `gamma`, `bias_std` and
    `ln_std` override these for stress tests that make every term of the block matter.
    """
    g = torch.Generator().manual_seed(seed)
    C, Hd = cfg.dim, cfg.ffn_hidden
    gam = cfg.layerscale_init if gamma is None else gamma

    def lin(o, i, bias=True):
        w = (torch.randn(o, i, generator=g) * 0.02).to(torch.bfloat16)
        b = (torch.randn(o, generator=g) * bias_std).to(torch.bfloat16) if bias else None
        return w, b

    def ln():
        w = (1.0 + torch.randn(C, generator=g) * ln_std).to(torch.bfloat16)
        b = (torch.randn(C, generator=g) * ln_std).to(torch.bfloat16)
        return w, b

    blocks = []
    for _ in range(cfg.depth if depth is None else depth):
        blk = {}
        blk["norm1.weight"], blk["norm1.bias"] = ln()
        blk["attn.qkv.weight"], qb = lin(3 * C, C, cfg.qkv_bias)
        if qb is not None:
            mask = torch.ones(3 * C, dtype=torch.bfloat16)
            mask[C: 2 * C] = 0  # K third of the bias is masked (vision_transformer.py:46-49)
            blk["attn.qkv.bias"] = qb
            blk["attn.qkv.bias_mask"] = mask
        blk["attn.proj.weight"], blk["attn.proj.bias"] = lin(C, C)
        blk["ls1.gamma"] = torch.full((C,), gam).to(torch.bfloat16)
        blk["norm2.weight"], blk["norm2.bias"] = ln()
        if cfg.ffn == "mlp":
            blk["mlp.fc1.weight"], blk["mlp.fc1.bias"] = lin(Hd, C)
            blk["mlp.fc2.weight"], blk["mlp.fc2.bias"] = lin(C, Hd)
        else:
            blk["mlp.w1.weight"], blk["mlp.w1.bias"] = lin(Hd, C)
            blk["mlp.w2.weight"], blk["mlp.w2.bias"] = lin(Hd, C)
            blk["mlp.w3.weight"], blk["mlp.w3.bias"] = lin(C, Hd)
        blk["ls2.gamma"] = torch.full((C,), gam).to(torch.bfloat16)
        blocks.append(blk)
    return blocks


def masked_qkv_bias(blk: dict) -> torch.Tensor | None:
    """LinearKMaskedBias.forward: bias * bias_mask (attention.py:47-49)."""
    b = blk.get("attn.qkv.bias")
    if b is None:
        return None
    return (b.double() * blk["attn.qkv.bias_mask"].double()).to(torch.bfloat16)


def make_inputs(cfg: ViTConfig, B: int, seed: int = 1):
    """Synthetic tokens: base embeddings N(0,1), residual delta ~ Laplace(0,1) on patch rows,
    full-resolution tokens = base + delta (bf16), importance = ||delta_p||_2 (fp32)."""
    g = torch.Generator().manual_seed(seed)
    N, P, C = cfg.num_tokens, cfg.num_patches, cfg.dim
    x_base = torch.randn(B, N, C, generator=g)
    u = torch.rand(B, P, C, generator=g, dtype=torch.float64) - 0.5
    delta = (-torch.sign(u) * torch.log1p(-2.0 * u.abs())).to(torch.float32)  # Laplace(0, 1)
    x_full = x_base.clone()
    x_full[:, cfg.num_pretokens:] += delta
    importance = torch.linalg.vector_norm(delta, dim=-1).to(torch.float32)
    return x_base.to(torch.bfloat16), x_full.to(torch.bfloat16), delta, importance


def full_dindice(cfg: ViTConfig, B: int) -> torch.Tensor:
    """One correction group covering every patch: [B, pre + P] = [0 .. N-1]."""
    return torch.arange(cfg.num_tokens, dtype=torch.long).unsqueeze(0).expand(B, -1).contiguous()


# ------------------------------------------------------------------------------------------------
# RoPE tables (rope_position_encoding.py:57-121)
# ------------------------------------------------------------------------------------------------


def rope_periods(cfg: ViTConfig, periods_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """base^(2i / (D/2)) for i < D/4, computed in fp32 (rope_position_encoding.py:110-113) and then
    held in the serving dtype: the reference casts the whole model, this persistent buffer
    included, with `model.to(dtype=torch.bfloat16)` (offload/server/model/dinov3_classifier.py:304;
    analysis/experiments/dinov3_correct_profile.py:60) after init_weights. fp32 `periods_dtype`
    gives the uncast module's periods."""
    D = cfg.head_dim
    p = cfg.rope_base ** (2 * torch.arange(D // 4, dtype=torch.float32) / (D // 2))
    return p.to(periods_dtype)


def rope_tables(cfg: ViTConfig, H: int | None = None, W: int | None = None,
                periods_dtype: torch.dtype = torch.bfloat16):
    """(sin, cos) [H*W, Dh] fp32 (rope_position_encoding.py:57-106): coordinates and angles in fp32,
    divided by the periods held in `periods_dtype` (bf16 for a bf16-served model), which fp32
    division promotes exactly to fp32 (:100)."""
    H = cfg.grid if H is None else H
    W = cfg.grid if W is None else W
    dt = torch.float32
    periods = rope_periods(cfg, periods_dtype)
    coords_h = torch.arange(0.5, H, dtype=dt) / H
    coords_w = torch.arange(0.5, W, dtype=dt) / W
    coords = torch.stack(torch.meshgrid(coords_h, coords_w, indexing="ij"), dim=-1).flatten(0, 1)
    coords = 2.0 * coords - 1.0
    angles = 2 * math.pi * coords[:, :, None] / periods[None, None, :]
    angles = angles.flatten(1, 2).tile(2)
    return torch.sin(angles), torch.cos(angles)


def rope_rotate(x: torch.Tensor, sin: torch.Tensor, cos: torch.Tensor) -> torch.Tensor:
    """(x * cos) + (rotate_half(x) * sin) in fp32, rounded to bf16 (attention.py:25-36)."""
    xf = x.to(torch.float32)
    x1, x2 = xf.chunk(2, dim=-1)
    rot = torch.cat([-x2, x1], dim=-1)
    return ((xf * cos) + (rot * sin)).to(torch.bfloat16)


# ------------------------------------------------------------------------------------------------
# Arithmetic primitives, f64 mode (explicit bf16 rounding) and bf16 mode (reference eager ops)
# ------------------------------------------------------------------------------------------------


def _f(t):
    return t.to(torch.float64)


def _rb(t):
    """Round to bf16 the way an fp32 kernel does: fp64 -> fp32 (nearest) -> bf16 (nearest even)."""
    return t.to(torch.float32).to(torch.bfloat16)


class _F64:
    @staticmethod
    def ln(x, w, b, eps):
        xf = _f(x)
        mean = xf.mean(-1, keepdim=True)
        var = ((xf - mean) ** 2).mean(-1, keepdim=True)
        return _rb((xf - mean) / torch.sqrt(var + eps) * _f(w) + _f(b))

    @staticmethod
    def linear(x, w, b):
        y = _f(x) @ _f(w).T
        if b is not None:
            y = y + _f(b)
        return _rb(y)

    @staticmethod
    def gelu(x):
        """Exact-erf GELU, 0.5 x (1 + erf(x / sqrt 2)), evaluated as 0.5 x erfc(-x / sqrt 2) so the
        negative tail keeps full relative accuracy (1 + erf cancels there)."""
        xf = _f(x)
        return _rb(0.5 * xf * torch.special.erfc(-xf / math.sqrt(2.0)))

    @staticmethod
    def silu_mul(x1, x2):
        s = _rb(_f(x1) * torch.sigmoid(_f(x1)))
        return _rb(_f(s) * _f(x2))

    @staticmethod
    def mul(a, g):
        return _rb(_f(a) * _f(g))

    @staticmethod
    def add(a, b):
        return _rb(_f(a) + _f(b))

    @staticmethod
    def sub(a, b):
        return _rb(_f(a) - _f(b))

    @staticmethod
    def fma_add(x, a, g):
        """x + a * g with one rounding (Triton fused_layerscale_add, token_update.py:33-41)."""
        return _rb((_f(x) + _f(a) * _f(g)).to(torch.float32))

    @staticmethod
    def sdpa(q, k, v, scale):
        """q [B, H, T, D], k/v [B, H, N, D] bf16 -> bf16, exact softmax in float64."""
        s = (_f(q) @ _f(k).transpose(-2, -1)) * scale
        p = torch.softmax(s, dim=-1)
        return _rb(p @ _f(v))


class _BF16:
    @staticmethod
    def ln(x, w, b, eps):
        return F.layer_norm(x, (x.shape[-1],), w, b, eps)

    @staticmethod
    def linear(x, w, b):
        return F.linear(x, w, b)

    @staticmethod
    def gelu(x):
        return F.gelu(x)

    @staticmethod
    def silu_mul(x1, x2):
        return F.silu(x1) * x2

    @staticmethod
    def mul(a, g):
        return a * g

    @staticmethod
    def add(a, b):
        return a + b

    @staticmethod
    def sub(a, b):
        return a - b

    @staticmethod
    def fma_add(x, a, g):
        return x + a * g

    @staticmethod
    def sdpa(q, k, v, scale):
        return F.scaled_dot_product_attention(q, k.contiguous(), v.contiguous(), scale=scale)


_MODES = {"f64": _F64, "bf16": _BF16}


def _mlp(ops, cfg: ViTConfig, blk: dict, x):
    if cfg.ffn == "mlp":
        h = ops.gelu(ops.linear(x, blk["mlp.fc1.weight"], blk["mlp.fc1.bias"]))
        return ops.linear(h, blk["mlp.fc2.weight"], blk["mlp.fc2.bias"])
    x1 = ops.linear(x, blk["mlp.w1.weight"], blk["mlp.w1.bias"])
    x2 = ops.linear(x, blk["mlp.w2.weight"], blk["mlp.w2.bias"])
    return ops.linear(ops.silu_mul(x1, x2), blk["mlp.w3.weight"], blk["mlp.w3.bias"])


# ------------------------------------------------------------------------------------------------
# Approximate pass (block.py:312-349; attention.py:215-278) -- produces the cache
# ------------------------------------------------------------------------------------------------


def server_score(kind: str, q: torch.Tensor, k: torch.Tensor, num_patches: int, scale: float) -> torch.Tensor:
    """The approx pass's {tag}_server_pscore (attention.py:241-273) from q, k [B, N, H, D] bf16 (after
    RoPE), with the reference's dispatch: patch_attn_prob(_layermean) -> dense mean over heads and
    queries (bf16 [B, N]; the layer-mean kind takes the fused fp32 key-side kernel's value for 32 heads
    of 128, attention.py:241-250 and attention_pscore.py:104-120); patch_pseudo_attn_prob(_layermean)
    -> the pseudo query's probabilities (bf16 [B, N]); every other kind -> cls_attn_prob (fp32 [B, N])."""
    from . import pscore as PS

    qn = q.float().numpy()
    kn = k.float().numpy()
    B, N, H, D = q.shape
    if kind in ("patch_attn_prob", "patch_attn_prob_layermean"):
        qh = np.ascontiguousarray(qn.transpose(0, 2, 1, 3))
        if kind == "patch_attn_prob_layermean" and H == 32 and D == 128 and 0 < N <= 4096:
            return torch.from_numpy(PS.patch_attn_prob_fused(qh, kn, scale)).to(torch.bfloat16)
        return torch.from_numpy(PS.patch_attn_prob(qh, kn, scale)).to(torch.bfloat16)
    if kind in ("patch_pseudo_attn_prob", "patch_pseudo_attn_prob_layermean"):
        qp = PS.pseudo_query(np.ascontiguousarray(qn[:, N - num_patches:].transpose(0, 2, 1, 3)))
        return torch.from_numpy(PS.query_attention_prob(qp, kn, scale)).to(torch.bfloat16)
    return torch.from_numpy(PS.query_attention_prob(np.ascontiguousarray(qn[:, 0]), kn, scale))


def approx_block(cfg: ViTConfig, blk: dict, x: torch.Tensor, rope, cache: dict, tag: str, mode: str = "f64",
                 server_pscore: str = "none"):
    """One approximate-pass block (the cache producer): {tag}_kv, {tag}_blocks_out_sum and, unless
    server_pscore is "none"/"disabled" (block.py:317-319 maps a zero server weight to "none"), the
    server score {tag}_server_pscore (attention.py:241-273)."""
    ops = _MODES[mode]
    B, N, C = x.shape
    H, D = cfg.heads, cfg.head_dim
    sin, cos = rope
    prefix = N - sin.shape[0]
    xn = ops.ln(x, blk["norm1.weight"], blk["norm1.bias"], cfg.ln_eps)
    qkv = ops.linear(xn, blk["attn.qkv.weight"], masked_qkv_bias(blk)).reshape(B, N, 3, H, D)
    kv = qkv[:, :, 1:].clone()
    q, k, v = qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2]
    q = torch.cat([q[:, :prefix], rope_rotate(q[:, prefix:], sin[None, :, None], cos[None, :, None])], dim=1)
    k = torch.cat([k[:, :prefix], rope_rotate(k[:, prefix:], sin[None, :, None], cos[None, :, None])], dim=1)
    kv[:, :, 0] = k
    cache[f"{tag}_kv"] = kv
    if server_pscore not in ("none", "disabled"):
        cache[f"{tag}_server_pscore"] = server_score(server_pscore, q, k, sin.shape[0], D ** -0.5)
    attn = ops.sdpa(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), D ** -0.5)
    attn = attn.transpose(1, 2).reshape(B, N, C)
    inc = ops.mul(ops.linear(attn, blk["attn.proj.weight"], blk["attn.proj.bias"]), blk["ls1.gamma"])
    x_attn = ops.add(x, inc)
    mlp = ops.mul(_mlp(ops, cfg, blk, ops.ln(x_attn, blk["norm2.weight"], blk["norm2.bias"], cfg.ln_eps)),
                  blk["ls2.gamma"])
    cache[f"{tag}_blocks_out_sum"] = ops.add(inc, mlp)
    return ops.add(x_attn, mlp), cache


def approx_pass(cfg: ViTConfig, blocks: list, x: torch.Tensor, rope, mode: str = "f64", server_pscore: str = "none"):
    cache: dict = {}
    for i, blk in enumerate(blocks):
        x, cache = approx_block(cfg, blk, x, rope, cache, f"layer{i}", mode, server_pscore)
    return x, cache


# ------------------------------------------------------------------------------------------------
# Correction pass (block.py:942-1191; attention.py:393-534)
# ------------------------------------------------------------------------------------------------


def qkv_rope_rows(cfg: ViTConfig, blk: dict, xn: torch.Tensor, plan, rope, mode: str = "f64",
                  lowp: dict | None = None):
    """q, k, v [M, H, D] of the selected rows from their norm1 output xn [M, C]: the qkv projection
    (attention.py:415; the low-precision route of `lowp["attn.qkv"]` when given) and RoPE on q and k of
    patch rows (attention.py:428-438); k and v are what the K/V cache rows receive (bf16 on store)."""
    ops = _MODES[mode]
    H, D = cfg.heads, cfg.head_dim
    M = xn.shape[0]
    sin, cos = rope
    if lowp is not None:
        from . import lowp as LPO
        qkv = LPO.linear_out(lowp["attn.qkv"], xn, blk["attn.qkv.weight"], blk.get("attn.qkv.bias")).reshape(M, 3, H, D)
    else:
        qkv = ops.linear(xn, blk["attn.qkv.weight"], masked_qkv_bias(blk)).reshape(M, 3, H, D)
    q, k, v = qkv[:, 0], qkv[:, 1], qkv[:, 2]
    pm = torch.from_numpy(plan.active_patch_mask)
    ri = torch.from_numpy(plan.active_rope_idx)
    s_sel, c_sel = sin[ri][:, None], cos[ri][:, None]
    q = torch.where(pm[:, None, None], rope_rotate(q, s_sel, c_sel), q)
    k = torch.where(pm[:, None, None], rope_rotate(k, s_sel, c_sel), k)
    return q, k, v


def correct_block(cfg: ViTConfig, blk: dict, x: torch.Tensor, plan, rope, cache: dict, tag: str,
                  mode: str = "f64", inplace_cache: bool = True, lowp: dict | None = None):
    """One partial-token correction block. `plan` is an oracle.plan.Plan (numpy) for this block: its
    active_* rows are the queries (compacted for the padded threshold builder), scattered into the
    padded [B, T] query buffer by (active_batch_idx, active_pos_idx) for the attention.

    `lowp` (SwiGLU blocks): {linear name: (kind, act_scale)} for "attn.qkv", "attn.proj", "mlp.w1",
    "mlp.w2", "mlp.w3", kind "fp4" or "fp8" -- the correction linears of the reference's low-precision
    controller after calibration (oracle/lowp.py); the rest of the block is unchanged.

    bf16 rounding points (reference materialisations): x_act (gather, exact); LN1 out; qkv out;
    q/k after RoPE (fp32 math); K/V cache rows; SDPA out; proj out; x_attn = x_act + g1 * proj
    (one rounding); LN2 out; fc1 out; GELU out; fc2 out; mlp = g2 * fc2; x + blocks_out_sum;
    x_attn + mlp; (x_attn - x_act); (x_attn - x_act) + mlp.
    """
    ops = _MODES[mode]
    B, N, C = x.shape
    H, D = cfg.heads, cfg.head_dim
    bi = torch.from_numpy(plan.active_batch_idx)
    ti = torch.from_numpy(plan.active_token_idx)
    M = bi.numel()
    T = plan.update_indice.shape[1]
    kv = cache[f"{tag}_kv"] if inplace_cache else cache[f"{tag}_kv"].clone()
    bos = cache[f"{tag}_blocks_out_sum"] if inplace_cache else cache[f"{tag}_blocks_out_sum"].clone()
    if M == 0:
        return ops.add(x, bos), cache

    x_act = x[bi, ti]                                                        # block.py:1111
    xn = ops.ln(x_act, blk["norm1.weight"], blk["norm1.bias"], cfg.ln_eps)   # :1114
    q, k, v = qkv_rope_rows(cfg, blk, xn, plan, rope, mode, lowp)            # attention.py:415-438
    if lowp is not None:
        from . import lowp as LPO
    kv[bi, ti, 0] = k                                                        # attention.py:444-454
    kv[bi, ti, 1] = v
    pi = torch.from_numpy(plan.active_pos_idx)
    q_pad = q.new_zeros((B, T, H, D))                                        # q_pad, BTHD (:456-495);
    q_pad[bi, pi] = q                                                        # pad rows are never read back
    attn = ops.sdpa(q_pad.transpose(1, 2), kv[:, :, 0].transpose(1, 2), kv[:, :, 1].transpose(1, 2), D ** -0.5)
    attn = attn.transpose(1, 2)[bi, pi].reshape(M, C)                        # :497-523
    if lowp is not None:
        proj = LPO.linear_out(lowp["attn.proj"], attn, blk["attn.proj.weight"], blk["attn.proj.bias"])
    else:
        proj = ops.linear(attn, blk["attn.proj.weight"], blk["attn.proj.bias"])  # :532
    x_attn = ops.fma_add(x_act, proj, blk["ls1.gamma"])                      # block.py:1129-1134
    xn2 = ops.ln(x_attn, blk["norm2.weight"], blk["norm2.bias"], cfg.ln_eps)
    if lowp is not None and lowp["mlp.w1"][0] == "fp4":
        mlp = LPO.swiglu_mlp(lowp, blk, xn2, blk["ls2.gamma"])
    elif lowp is not None:   # FP8: the unfused SwiGLU of ffn_layers.py:108-115 on FP8 linears
        x1 = LPO.linear_out(lowp["mlp.w1"], xn2, blk["mlp.w1.weight"], blk.get("mlp.w1.bias"))
        x2 = LPO.linear_out(lowp["mlp.w2"], xn2, blk["mlp.w2.weight"], blk.get("mlp.w2.bias"))
        h = ops.silu_mul(x1, x2)
        mlp = ops.mul(LPO.linear_out(lowp["mlp.w3"], h, blk["mlp.w3.weight"], blk.get("mlp.w3.bias")),
                      blk["ls2.gamma"])
    else:
        mlp = ops.mul(_mlp(ops, cfg, blk, xn2), blk["ls2.gamma"])            # :1141
    x_out = ops.add(x, bos)                                                  # :1143-1149
    x_out[bi, ti] = ops.add(x_attn, mlp)                                     # :1151-1158
    bos[bi, ti] = ops.add(ops.sub(x_attn, x_act), mlp)                       # :1177-1179
    cache[f"{tag}_kv"] = kv
    cache[f"{tag}_blocks_out_sum"] = bos
    return x_out, cache


def correct_pass(cfg: ViTConfig, blocks: list, x: torch.Tensor, plan, rope, cache: dict, mode: str = "f64"):
    """All blocks with one plan (the plan is cached across layers whenever the score does not depend
    on the layer, block.py:709-727; true for the mobile-hint score with server weight 0), or with one
    plan per block when `plan` is a list (a per-layer server score such as cls_attn_prob)."""
    plans = list(plan) if isinstance(plan, (list, tuple)) else [plan] * len(blocks)
    for i, blk in enumerate(blocks):
        x, cache = correct_block(cfg, blk, x, plans[i], rope, cache, f"layer{i}", mode)
    return x, cache
