"""Per-block precision routing for the approx and correct passes.

Mirrors DINOv3CorrectPrecisionController / DINOv3ApproxPrecisionController
(offload/server/model/dinov3_precision.py:172-629, 632-1010): `run_block` picks the block to run,
calls its `correct` / `approx` without autograd, and keeps the public contract that activations and
the K/V cache leave the block as bf16 (:972-985); `event_metadata` reports the route taken.

Precision: the correction GEMMs run in bf16 on MFMA. An explicit `correct_precision` of "fp8" or
"fp4" whose low-precision path is unavailable raises RuntimeError at construction, as the
reference's `_handle_fp8_unavailable` / `_handle_fp4_unavailable` do (:723-731); "bf16" and "auto"
run bf16.
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
        self.unavailable_reason = None
        self._event_routes: Dict[str, tuple[str, int]] = {}
        if precision in ("fp8", "fp4"):
            self._handle_unavailable(precision, f"{precision} correction linears are not part of this build")

    def _handle_unavailable(self, precision: str, reason: str) -> None:
        """Record why a low-precision path is unavailable; an explicit request for it is an error
        (dinov3_precision.py:723-731)."""
        self.unavailable_reason = reason
        if self.precision == precision:
            raise RuntimeError(f"correct_precision={precision!r} is unavailable: {reason}")

    @classmethod
    def from_config(cls, blocks: nn.ModuleList, config: Any, device: torch.device):
        return cls(blocks, precision=getattr(config, "correct_precision", "bf16"), device=device,
                   compile_enabled=getattr(config, "correct_compile", False),
                   fp4_calib_events=getattr(config, "correct_fp4_calib_events", 1),
                   fp4_proj_precision=getattr(config, "correct_fp4_proj_precision", "fp8"),
                   bucket_rows=getattr(config, "correct_bucket_rows", 0))

    def begin_event(self) -> None:
        self._event_routes = {}

    def _effective_precision(self) -> str:
        return "bf16"

    def run_block(self, layer_idx: int, x: torch.Tensor, dindice: torch.Tensor, rope: Any, cache: Dict[str, Any],
                  tag: str, *, source_key: str = "default", **kwargs: Any):
        rows = int(x.shape[0] * x.shape[1]) if x.dim() == 3 else int(x.shape[0])
        self._event_routes[source_key] = (self._effective_precision(), rows)
        with torch.no_grad():
            out, cache = self.blocks[layer_idx].correct(x, dindice, rope, cache, tag, **kwargs)
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
        blocks = [self.blocks[i] for i in layer_range]
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
        eff = {p for p, _ in self._event_routes.values()}
        effective = "none" if not eff else (next(iter(eff)) if len(eff) == 1 else "mixed")
        meta = {
            "correct_precision_requested": self.precision,
            "correct_precision_effective": effective,
            "correct_precision_rows": sorted({r for _, r in self._event_routes.values()}),
            "correct_fp8_sources": 0,
            "correct_fp4_sources": 0,
            "correct_bf16_sources": sum(p == "bf16" for p, _ in self._event_routes.values()),
        }
        if self.unavailable_reason:
            meta["correct_precision_fallback_reason"] = self.unavailable_reason
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
