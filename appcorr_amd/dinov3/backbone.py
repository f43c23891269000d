"""DINOv3 ViT backbone container: blocks, RoPE, token layout and the hub factory shapes.

Shapes and initialisation follow the reference factories (appcorr/models/dinov3/hub/backbones.py:
dinov3_vits16 :201-237, dinov3_vitb16 :279-315, dinov3_vitl16 :318-371, dinov3_vit7b16 :452-494) and
init_weights / init_weights_vit (models/vision_transformer.py:41-57, 300-306). Token layout is
[cls | 4 storage tokens | patches] (vision_transformer.py:308-338).

Only the block stack is on the accelerated path. Patch embedding and the final norm are fixture /
head plumbing (torch ops), used to turn images into tokens and features into logits.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn

from .. import kernels as K
from .layers import LayerScale, LinearKMaskedBias, SelfAttentionBlock
from .rope import RopePositionEmbedding


class DinoBackbone(nn.Module):
    def __init__(self, *, embed_dim: int, depth: int, num_heads: int, ffn_ratio: float, qkv_bias: bool,
                 ffn_layer: str = "mlp", n_storage_tokens: int = 4, layerscale_init: float | None = 1e-5,
                 norm_eps: float = 1e-5, mask_k_bias: bool = True, rope_base: float = 100.0, patch_size: int = 16,
                 in_chans: int = 3, device=None):
        super().__init__()
        self.embed_dim = embed_dim
        self.num_heads = num_heads
        self.patch_size = patch_size
        self.n_storage_tokens = n_storage_tokens
        self.patch_embed = nn.Conv2d(in_chans, embed_dim, kernel_size=patch_size, stride=patch_size, device=device)
        self.cls_token = nn.Parameter(torch.zeros(1, 1, embed_dim, device=device))
        self.storage_tokens = nn.Parameter(torch.zeros(1, n_storage_tokens, embed_dim, device=device))
        self.rope_embed = RopePositionEmbedding(embed_dim, num_heads=num_heads, base=rope_base, device=device)
        self.blocks = nn.ModuleList([
            SelfAttentionBlock(embed_dim, num_heads, ffn_ratio=ffn_ratio, qkv_bias=qkv_bias, init_values=layerscale_init,
                               norm_eps=norm_eps, ffn_layer=ffn_layer, mask_k_bias=mask_k_bias, device=device)
            for _ in range(depth)
        ])
        self.norm = nn.LayerNorm(embed_dim, eps=norm_eps, device=device)

    @property
    def num_pretokens(self) -> int:
        return 1 + self.n_storage_tokens

    @torch.no_grad()
    def init_weights(self, generator: torch.Generator | None = None) -> "DinoBackbone":
        """Linear ~ trunc_normal(0.02) (drawn from `generator`, on the generator's device), biases 0,
        K-bias mask, LayerNorm (1, 0), LayerScale = init value, cls/storage ~ N(0, 0.02)."""
        gdev = generator.device if generator is not None else None

        def normal_(p, std):
            r = torch.randn(p.shape, generator=generator, device=gdev)
            p.copy_((r * std).clamp_(-2.0, 2.0).to(p.dtype))

        normal_(self.cls_token, 0.02)
        normal_(self.storage_tokens, 0.02)
        for m in self.modules():
            if isinstance(m, nn.Linear):
                normal_(m.weight, 0.02)
                if m.bias is not None:
                    m.bias.zero_()
                if isinstance(m, LinearKMaskedBias) and m.bias is not None:
                    o = m.out_features
                    m.bias_mask.fill_(1)
                    m.bias_mask[o // 3: 2 * o // 3].fill_(0)
            elif isinstance(m, nn.LayerNorm):
                m.reset_parameters()
            elif isinstance(m, LayerScale):
                m.reset_parameters()
        return self

    def prepare_tokens(self, images: torch.Tensor) -> tuple[torch.Tensor, tuple[int, int]]:
        """[B, 3, H, W] -> tokens [B, 5 + HW/256, C] (vision_transformer.py:308-338), fixture plumbing."""
        x = self.patch_embed(images.to(self.patch_embed.weight.dtype))
        B, C, H, W = x.shape
        x = x.flatten(2).transpose(1, 2)
        pre = torch.cat([self.cls_token, self.storage_tokens], dim=1).expand(B, -1, -1).to(x.dtype)
        return torch.cat([pre, x], dim=1), (H, W)

    def final_norm(self, x: torch.Tensor) -> torch.Tensor:
        return K.layer_norm(x.contiguous(), self.norm.weight, self.norm.bias, self.norm.eps)


_FACTORY = {
    # name: (embed_dim, depth, heads, ffn_ratio, qkv_bias, ffn_layer)
    "vits16": (384, 12, 6, 4.0, True, "mlp"),
    "vitb16": (768, 12, 12, 4.0, True, "mlp"),
    "vitl16": (1024, 24, 16, 4.0, True, "mlp"),
    "vit7b16": (4096, 40, 32, 3.0, False, "swiglu64"),
}


def dinov3_backbone(name: str, *, depth: int | None = None, layerscale_init: float | None = 1e-5, device=None,
                    dtype: torch.dtype = torch.bfloat16, seed: int | None = 0) -> DinoBackbone:
    """Random-init DINOv3 backbone of a hub shape ('vits16', 'vitb16', 'vitl16', 'vit7b16')."""
    key = name.replace("dinov3_", "")
    if key not in _FACTORY:
        raise ValueError(f"unknown DINOv3 backbone {name!r}; choose from {sorted(_FACTORY)}")
    dim, d, heads, ratio, qkv_bias, ffn = _FACTORY[key]
    # Built on the target device and drawn from a generator there (the ViT-7B stack holds 6.7e9
    # weights); on the CPU when no device is given.
    m = DinoBackbone(embed_dim=dim, depth=d if depth is None else depth, num_heads=heads, ffn_ratio=ratio,
                     qkv_bias=qkv_bias, ffn_layer=ffn, layerscale_init=layerscale_init, device=device)
    if seed is not None:
        m.init_weights(torch.Generator(device=device if device is not None else "cpu").manual_seed(seed))
    # Every floating parameter and buffer moves to the serving dtype, as the reference's
    # `model.to(dtype=torch.bfloat16)` does (offload/server/model/dinov3_classifier.py:304;
    # analysis/experiments/dinov3_correct_profile.py:60). That includes the RoPE `periods` buffer
    # (rope_position_encoding.py:50-53): the tables are then computed in fp32 from bf16-rounded
    # periods (rope_position_encoding.py:100), which is what the reference serves.
    for p in m.parameters():
        p.data = p.data.to(dtype)
    for buf in m.buffers():
        if buf.is_floating_point():
            buf.data = buf.data.to(dtype)
    return m.to(device) if device is not None else m


def dinov3_vits16(**kw):
    return dinov3_backbone("vits16", **kw)


def dinov3_vitb16(**kw):
    return dinov3_backbone("vitb16", **kw)


def dinov3_vitl16(**kw):
    return dinov3_backbone("vitl16", **kw)


def dinov3_vit7b16(**kw):
    return dinov3_backbone("vit7b16", **kw)
