"""roctx ranges around the stages of the correction path, the counterpart of the reference's NVTX
annotations (appcorr/models/dinov3/layers/block.py:274,288,942,1104,1137; worker.py:509-525).

torch's `torch.cuda.nvtx` calls go to roctx on ROCm builds, so `rocprofv3 --marker-trace` (or any
roctx consumer) shows them; without a consumer a push / pop pair costs well under a microsecond of
host time, and nothing on the device. When the marker library is unusable the ranges are no-ops.
"""

from __future__ import annotations

import contextlib
import functools

try:
    import torch.cuda.nvtx as _nvtx

    _nvtx.range_push("appcorr_amd")
    _nvtx.range_pop()
    _ENABLED = True
except Exception:  # no marker library in this torch build
    _nvtx = None
    _ENABLED = False


@contextlib.contextmanager
def trace_range(name: str):
    """A named roctx range around the enclosed host code (and the launches it enqueues)."""
    if not _ENABLED:
        yield
        return
    _nvtx.range_push(name)
    try:
        yield
    finally:
        _nvtx.range_pop()


def annotate(name: str):
    """Decorator form of trace_range."""
    def deco(fn):
        @functools.wraps(fn)
        def wrapper(*args, **kwargs):
            with trace_range(name):
                return fn(*args, **kwargs)
        return wrapper
    return deco
