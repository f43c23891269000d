"""bf16 bit helpers (numpy). Test infrastructure only.

bf16 values are carried as uint16 bit patterns. Rounding from fp32 is round-to-nearest-even, the
rounding of torch's c10::BFloat16 (used by every bf16 tensor the reference materialises).
"""

from __future__ import annotations

import numpy as np
import torch


def f32_to_bf16_bits(a) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bits. uint32 arithmetic: the rounding increment carries out
    of 32 bits only for NaN patterns (|u| > 0x7F800000), whose result is replaced by the quiet NaN."""
    u = np.asarray(a, dtype=np.float32).view(np.uint32)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    r = np.asarray((u >> np.uint32(16)) & np.uint32(1), dtype=np.uint32)
    r += u
    r += np.uint32(0x7FFF)
    r >>= np.uint32(16)
    return np.where(nan, np.uint16(0x7FC0), r.astype(np.uint16))


def bf16_bits_to_f32(b) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(a) -> np.ndarray:
    """fp32 array -> nearest bf16 value, as fp32."""
    return bf16_bits_to_f32(f32_to_bf16_bits(a))


def torch_bf16_to_bits(t: torch.Tensor) -> np.ndarray:
    assert t.dtype == torch.bfloat16
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def bits_to_torch_bf16(b: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(b, dtype=np.uint16).view(np.int16)).view(torch.bfloat16)
