"""Executor-side drop-in for offload/server/model (the worker's plugin API for the correction path)."""

import torch

from .base import ModelExecutor
from .protocol import (ExperimentConfig, InferenceResult, Instruction, OpType, Patch, Task, default_appcorr_kwargs,
                       normalize_appcorr_kwargs)


def get_model_executor(name: str, device: torch.device) -> ModelExecutor:
    """Registry (reference offload/server/model/__init__.py:4-40), DINOv3 classifier executor only."""
    if "dinov3" in name and not any(t in name for t in ("detector", "segmentor", "depther")):
        from .dinov3_classifier import DINOv3ClassifierExecutor

        return DINOv3ClassifierExecutor(device)
    raise ValueError(f"Unknown model executor for: {name} (this build provides dinov3_classifier)")


__all__ = ["ModelExecutor", "get_model_executor", "ExperimentConfig", "InferenceResult", "Instruction", "OpType",
           "Patch", "Task", "default_appcorr_kwargs", "normalize_appcorr_kwargs"]
