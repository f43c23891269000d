"""Per-block precision routing for the approx and correct passes.

Mirrors DINOv3CorrectPrecisionController / DINOv3ApproxPrecisionController
(offload/server/model/dinov3_precision.py:172-629, 632-1010): `run_block` picks the block to run,
calls its `correct` / `approx` without autograd, and keeps the public contract that activations and
the K/V cache leave the block as bf16 (:972-985); `event_metadata` reports the route taken.

Correction precision (:632-1010):
  "bf16" / "auto"  the bf16 MFMA GEMMs;
  "fp4"            each block's qkv, mlp.w1, mlp.w2, mlp.w3 in NVFP4 (w1 / w2 sharing one quantized
                   activation) and attn.proj in `fp4_proj_precision` (FP8 by default);
  "fp8"            all five correction linears in FP8.
The low-precision linears (appcorr_amd/dinov3/lowp.py) exist only for blocks with exactly the five
eligible linears (SwiGLU, ViT-7B). They calibrate for `fp4_calib_events` events (exact bf16 GEMMs with
an amax observer) and freeze their static activation scales at the start of the next event
(:889-937). An explicit "fp8" / "fp4" request whose path cannot be built (a GELU-MLP model, no GPU)
raises RuntimeError at construction, as `_handle_fp8_unavailable` / `_handle_fp4_unavailable` do
(:723-731). `correct_compile` and `correct_bucket_rows` are accepted; launches here are fixed-shape
kernels (HIP graphs replace torch.compile), so neither changes the arithmetic.
"""

from __future__ import annotations

from typing import Any, Dict

import torch
from torch import nn


class DINOv3CorrectPrecisionController:
    def __init__(self, blocks: nn.ModuleList, *, precision: str = "bf16", device: torch.device | None = None,
                 compile_enabled: bool = False, fp4_calib_events: int = 1, fp4_proj_precision: str = "fp8",
                 bucket_rows: int = 0) -> None:
        if precision not in ("bf16", "auto", "fp8", "fp4"):
            raise ValueError(f"unknown correct_precision {precision!r}")
        self.blocks = blocks
        self.precision = precision
        self.device = device
        self.compile_enabled = bool(compile_enabled)
        self.fp4_calib_events = max(0, int(fp4_calib_events))
        self.fp4_proj_precision = str(fp4_proj_precision)
        self.bucket_rows = max(0, int(bucket_rows))
        self.lowp_blocks: list | None = None
        self.unavailable_reason: str | None = None
        self._calib_remaining: int | None = None
        self._event_routes: Dict[str, tuple[str, int]] = {}
        if precision in ("fp8", "fp4"):
            self._initialize_low_precision(precision)

    def _handle_unavailable(self, precision: str, reason: str) -> None:
        """Record why a low-precision path is unavailable; an explicit request for it is an error
        (dinov3_precision.py:723-731)."""
        self.unavailable_reason = reason
        if self.precision == precision:
            raise RuntimeError(f"correct_precision={precision!r} is unavailable: {reason}")

    def _initialize_low_precision(self, precision: str) -> None:
        """Convert every block's five correction linears (dinov3_precision.py:734-887)."""
        from appcorr_amd.dinov3 import lowp as LP

        dev = torch.device(self.device) if self.device is not None else None
        if dev is None or dev.type != "cuda" or not torch.cuda.is_available():
            self._handle_unavailable(precision, f"{precision.upper()} requires a GPU")
            return
        if precision == "fp4" and self.fp4_proj_precision not in ("fp8", "fp4"):
            self._handle_unavailable(precision, f"unknown fp4_proj_precision {self.fp4_proj_precision!r}")
            return
        converted, n4, n8 = [], 0, 0
        try:
            for block in self.blocks:
                blk, a, b = LP.convert_block(block, precision, proj_precision=self.fp4_proj_precision,
                                             bucket_rows=self.bucket_rows)
                converted.append(blk)
                n4 += a
                n8 += b
        except (RuntimeError, ValueError) as exc:
            self._handle_unavailable(precision, str(exc))
            return
        expected = len(self.blocks) * len(LP.LOW_PRECISION_LINEAR_SUFFIXES)
        if n4 + n8 != expected:
            self._handle_unavailable(precision, f"converted {n4 + n8} Linear layers, expected {expected}")
            return
        self.lowp_blocks = converted
        self.lowp_counts = {"fp4": n4, "fp8": n8}
        self._calib_remaining = max(1, self.fp4_calib_events)

    @classmethod
    def from_config(cls, blocks: nn.ModuleList, config: Any, device: torch.device):
        return cls(blocks, precision=getattr(config, "correct_precision", "bf16"), device=device,
                   compile_enabled=getattr(config, "correct_compile", False),
                   fp4_calib_events=getattr(config, "correct_fp4_calib_events", 1),
                   fp4_proj_precision=getattr(config, "correct_fp4_proj_precision", "fp8"),
                   bucket_rows=getattr(config, "correct_bucket_rows", 0))

    @property
    def fp4_available(self) -> bool:
        return self.precision == "fp4" and self.lowp_blocks is not None

    @property
    def fp8_available(self) -> bool:
        return self.precision == "fp8" and self.lowp_blocks is not None

    @property
    def calibrating(self) -> bool:
        return self._calib_remaining is not None

    def _freeze_static_scales(self) -> None:
        """Bake each linear's observed amax into its static scale (dinov3_precision.py:889-937). A linear
        that saw nothing keeps observing on the exact bf16 route and the freeze is retried next event."""
        from appcorr_amd.dinov3 import lowp as LP

        pending = 0
        for blk in self.lowp_blocks:
            for mod in blk.modules():
                if isinstance(mod, LP._LowPrecisionLinear) and not mod.freeze_activation_scale():
                    pending += 1
        self._calib_remaining = 0 if pending else None

    def begin_event(self) -> None:
        """Convert at the start of the event after the last calibration event, so the observers have
        seen data (dinov3_precision.py:939-951)."""
        self._event_routes = {}
        if self._calib_remaining is not None:
            if self._calib_remaining > 0:
                self._calib_remaining -= 1
            else:
                self._freeze_static_scales()

    def _effective_precision(self) -> str:
        if self.precision in ("fp8", "fp4"):
            return self.precision if self.lowp_blocks is not None else "bf16"
        return "bf16"

    def _block(self, layer_idx: int) -> nn.Module:
        return self.lowp_blocks[layer_idx] if self._effective_precision() in ("fp8", "fp4") else self.blocks[layer_idx]

    def run_block(self, layer_idx: int, x: torch.Tensor, dindice: torch.Tensor, rope: Any, cache: Dict[str, Any],
                  tag: str, *, source_key: str = "default", **kwargs: Any):
        rows = int(x.shape[0] * x.shape[1]) if x.dim() == 3 else int(x.shape[0])
        self._event_routes[source_key] = (self._effective_precision(), rows)
        with torch.no_grad():
            out, cache = self._block(layer_idx).correct(x, dindice, rope, cache, tag, **kwargs)
        if out.dtype != torch.bfloat16:
            out = out.to(torch.bfloat16)
        for key, value in list(cache.items()):
            if (key.startswith(f"{tag}_") and key.endswith("_kv") and torch.is_tensor(value)
                    and torch.is_floating_point(value) and value.dtype != torch.bfloat16):
                cache[key] = value.to(torch.bfloat16)
        return out, cache

    def run_blocks_packed(self, layer_range: range, x: torch.Tensor, dindice: torch.Tensor, rope: Any,
                          cache: Dict[str, Any], **kwargs: Any):
        """The blocks of layer_range in one packed correction run (the selected rows stay packed between
        blocks; bit-identical to run_block over the same layers). Records the same per-layer routes as
        run_block. Returns None, with nothing run or recorded, when the query plan is per-layer."""
        from appcorr_amd.dinov3.layers import correct_blocks_packed

        if kwargs.get("appcorr_method", "partial_token") != "partial_token":
            return None
        blocks = [self._block(i) for i in layer_range]
        tags = [f"layer{i}" for i in layer_range]
        with torch.no_grad():
            res = correct_blocks_packed(blocks, x, dindice, rope, cache, tags, **kwargs)
        if res is None:
            return None
        rows = int(x.shape[0] * x.shape[1]) if x.dim() == 3 else int(x.shape[0])
        for i in layer_range:
            self._event_routes[f"layer{i}"] = (self._effective_precision(), rows)
        return res

    def event_metadata(self) -> Dict[str, Any]:
        routes = self._event_routes.values()
        eff = {p for p, _ in routes}
        effective = "none" if not eff else (next(iter(eff)) if len(eff) == 1 else "mixed")
        meta = {
            "correct_precision_requested": self.precision,
            "correct_precision_effective": effective,
            "correct_precision_rows": sorted({r for _, r in routes}),
            "correct_fp8_sources": sum(p == "fp8" for p, _ in routes),
            "correct_fp4_sources": sum(p == "fp4" for p, _ in routes),
            "correct_bf16_sources": sum(p == "bf16" for p, _ in routes),
        }
        if self.unavailable_reason:
            meta["correct_precision_unavailable_reason"] = self.unavailable_reason
        return meta


class DINOv3ApproxPrecisionController:
    """bf16 approx pass (the cache producer) through the same kernels."""

    def __init__(self, blocks: nn.ModuleList, *, precision: str = "bf16", device=None) -> None:
        self.blocks = blocks
        self.precision = precision
        self._event_routes: Dict[str, tuple[str, int]] = {}

    @classmethod
    def from_config(cls, blocks: nn.ModuleList, config: Any, device: torch.device):
        return cls(blocks, precision=getattr(config, "precision", "bf16"), device=device)

    def begin_event(self) -> None:
        self._event_routes = {}

    def run_block(self, layer_idx: int, x: torch.Tensor, rope: Any, cache: Dict[str, Any], tag: str, *,
                  source_key: str = "default", **kwargs: Any):
        self._event_routes[source_key] = ("bf16", int(x.shape[0] * x.shape[1]))
        with torch.no_grad():
            out, cache = self.blocks[layer_idx].approx(x, rope, cache, tag, **kwargs)
        return out, cache

    def event_metadata(self) -> Dict[str, Any]:
        return {"approx_precision_requested": self.precision, "approx_precision_effective": "bf16"}
