"""2-D axial RoPE tables, the positional input of the correction path.

Same parametrisation as the reference's RopePositionEmbedding in eval mode
(appcorr/models/dinov3/layers/rope_position_encoding.py:16-121): periods base^(2i / (D/2)) for
i < D/4, coordinates at patch centres normalised per axis ("separate") to [-1, 1], angles tiled to
the full head dim. Tables are built once per (H, W) with torch on the target device (setup work,
not part of the per-block path) and handed to every block as (sin, cos), each [H*W, Dh] fp32.

`self.dtype` (fp32, the hub factories' `pos_embed_rope_dtype`) sets the dtype of the coordinates
and of the tables; the `periods` buffer follows the module's dtype casts like any buffer, so a
backbone served in bf16 divides by bf16-rounded periods, as the reference does
(rope_position_encoding.py:47-53, 100).
"""

from __future__ import annotations

import math

import torch
from torch import nn


class RopePositionEmbedding(nn.Module):
    def __init__(self, embed_dim: int, *, num_heads: int, base: float = 100.0, normalize_coords: str = "separate",
                 dtype: torch.dtype = torch.float32, device=None):
        super().__init__()
        if embed_dim % (4 * num_heads) != 0:
            raise ValueError("embed_dim must be divisible by 4 * num_heads")
        if normalize_coords not in ("min", "max", "separate"):
            raise ValueError(f"unknown normalize_coords {normalize_coords!r}")
        self.D_head = embed_dim // num_heads
        self.base = base
        self.normalize_coords = normalize_coords
        self.dtype = dtype
        q = self.D_head // 4
        periods = base ** (2 * torch.arange(q, device=device, dtype=dtype) / (self.D_head // 2))
        self.register_buffer("periods", periods, persistent=True)

    def forward(self, *, H: int, W: int) -> tuple[torch.Tensor, torch.Tensor]:
        dd = {"device": self.periods.device, "dtype": self.dtype}
        if self.normalize_coords == "max":
            den_h = den_w = max(H, W)
        elif self.normalize_coords == "min":
            den_h = den_w = min(H, W)
        else:
            den_h, den_w = H, W
        ch = torch.arange(0.5, H, **dd) / den_h
        cw = torch.arange(0.5, W, **dd) / den_w
        coords = torch.stack(torch.meshgrid(ch, cw, indexing="ij"), dim=-1).flatten(0, 1)
        coords = 2.0 * coords - 1.0
        angles = 2 * math.pi * coords[:, :, None] / self.periods[None, None, :]
        angles = angles.flatten(1, 2).tile(2)
        return torch.sin(angles), torch.cos(angles)
