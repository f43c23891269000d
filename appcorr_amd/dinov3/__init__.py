"""DINOv3 block stack with the partial-token approx / correct passes on gfx950 kernels."""

from .backbone import DinoBackbone, dinov3_backbone, dinov3_vit7b16, dinov3_vitb16, dinov3_vitl16, dinov3_vits16
from .layers import (
    LayerScale,
    LinearKMaskedBias,
    Mlp,
    PackedQueryState,
    PartialTokenQueryPlan,
    SelfAttention,
    SelfAttentionBlock,
    SwiGLUFFN,
)
from .rope import RopePositionEmbedding

__all__ = [
    "DinoBackbone", "dinov3_backbone", "dinov3_vits16", "dinov3_vitb16", "dinov3_vitl16", "dinov3_vit7b16",
    "LayerScale", "LinearKMaskedBias", "Mlp", "SwiGLUFFN", "SelfAttention", "SelfAttentionBlock",
    "PackedQueryState", "PartialTokenQueryPlan", "RopePositionEmbedding",
]
