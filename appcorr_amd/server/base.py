"""ModelExecutor: the plugin / operator interface the worker drives (one method per OpType).

Same abstract surface and DINOv3 precision hooks as the reference's offload/server/model/base.py:8-171
(configure_* / begin_* / run_dinov3_*_block / *_event_metadata, _normalize_patch_score_map, and the
abstract load_model ... get_final_results). The per-layer correction call
`run_dinov3_correct_block(layer_idx, x, dindice, rope, cache, tag, *, source_key, **kwargs)` is the
drop-in boundary of the accelerated path.
"""

from __future__ import annotations

from abc import ABC, abstractmethod
from typing import Any, Dict

import torch

from .protocol import Task


class ModelExecutor(ABC):
    def __init__(self, device: torch.device):
        self.device = device
        self.model = None
        self._dinov3_approx_precision = None
        self._dinov3_correct_precision = None

    def configure_dinov3_approx_precision(self, backbone: torch.nn.Module, config: Any):
        from .precision import DINOv3ApproxPrecisionController

        self._dinov3_approx_precision = DINOv3ApproxPrecisionController.from_config(backbone.blocks, config,
                                                                                    self.device)

    def begin_dinov3_approx_event(self):
        if self._dinov3_approx_precision is None:
            raise RuntimeError("DINOv3 approximate precision is not configured")
        self._dinov3_approx_precision.begin_event()

    def run_dinov3_approx_block(self, layer_idx: int, x: torch.Tensor, rope, cache: Dict[str, Any], tag: str, *,
                                source_key: str = "default", **kwargs):
        if self._dinov3_approx_precision is None:
            raise RuntimeError("DINOv3 approximate precision is not configured")
        return self._dinov3_approx_precision.run_block(layer_idx, x, rope, cache, tag, source_key=source_key,
                                                       **kwargs)

    def dinov3_approx_event_metadata(self) -> Dict[str, Any]:
        return {} if self._dinov3_approx_precision is None else self._dinov3_approx_precision.event_metadata()

    def configure_dinov3_correct_precision(self, backbone: torch.nn.Module, config: Any):
        from .precision import DINOv3CorrectPrecisionController

        self._dinov3_correct_precision = DINOv3CorrectPrecisionController.from_config(backbone.blocks, config,
                                                                                      self.device)

    def begin_dinov3_correct_event(self):
        if self._dinov3_correct_precision is None:
            raise RuntimeError("DINOv3 correct precision is not configured")
        self._dinov3_correct_precision.begin_event()

    def run_dinov3_correct_block(self, layer_idx: int, x: torch.Tensor, dindice: torch.Tensor, rope,
                                 cache: Dict[str, Any], tag: str, *, source_key: str = "default", **kwargs):
        if self._dinov3_correct_precision is None:
            raise RuntimeError("DINOv3 correct precision is not configured")
        return self._dinov3_correct_precision.run_block(layer_idx, x, dindice, rope, cache, tag,
                                                        source_key=source_key, **kwargs)

    def dinov3_correct_event_metadata(self) -> Dict[str, Any]:
        return {} if self._dinov3_correct_precision is None else self._dinov3_correct_precision.event_metadata()

    @staticmethod
    def _normalize_patch_score_map(score_map: torch.Tensor | None) -> torch.Tensor | None:
        """Row-normalise a [B, P] score map (reference base.py:114-123)."""
        if score_map is None:
            return None
        if score_map.ndim != 2:
            raise ValueError(f"Expected a 2D score map, got shape {tuple(score_map.shape)}")
        sums = score_map.sum(dim=1, keepdim=True, dtype=torch.float32)
        denom = sums.clamp_min(torch.finfo(torch.float32).eps).to(dtype=score_map.dtype)
        return score_map / denom

    @abstractmethod
    def load_model(self, model_name: str, config: Any):
        ...

    @abstractmethod
    def preprocess(self, batch_data: Any, task: Task, context: Dict[str, Any], config: Any):
        ...

    @abstractmethod
    def prepare_tokens(self, task: Task, context: Dict[str, Any], config: Any):
        ...

    @abstractmethod
    def approx_forward(self, params: Dict[str, Any], context: Dict[str, Any], config: Any):
        ...

    @abstractmethod
    def correct_forward(self, params: Dict[str, Any], context: Dict[str, Any], config: Any):
        ...

    @abstractmethod
    def head_inference(self, task: Task, context: Dict[str, Any], config: Any) -> Dict[str, Any]:
        ...

    @abstractmethod
    def full_inference(self, task: Task, context: Dict[str, Any], config: Any):
        ...

    @abstractmethod
    def decide_exit(self, task: Task, context: Dict[str, Any], config: Any) -> Dict[str, Any]:
        ...

    @abstractmethod
    def get_final_results(self, task: Task, context: Dict[str, Any], config: Any) -> Dict[int, Any]:
        ...
