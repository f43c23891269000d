"""Top-k token selection and the packed query plan, restated in numpy. Test infrastructure only.

Follows appcorr/models/dinov3/layers/block.py:
  _select_patch_keep_mask           :358-395  (k = min(int(P * ratio), P); k == 0 -> none; k == P -> all)
  _build_packed_query_state_fixed_k :397-442  (kept indices sorted ascending; pretokens first)
  _build_packed_query_state_all_keep:444-490
  _compute_partial_token_plan_stats :762-788  (plan_stats)
and the PackedQueryState fields of attention.py:64-74.

torch.topk leaves the order of equal scores unspecified (block.py:385-390); the selection here
ranks by (score descending, candidate index ascending), with -0.0 == +0.0 and NaN above +inf. The
HIP kernel implements the same rule; agreement with torch.topk on tied inputs is "parity unpinned".
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np


def keep_count(num_candidates: int, token_keep_ratio: float) -> int:
    """block.py:378 -- Python int arithmetic on a static shape."""
    return min(int(num_candidates * token_keep_ratio), num_candidates)


def topk_keep(scores: np.ndarray, k: int) -> np.ndarray:
    """Kept candidate indices per row, sorted ascending: [B, k] int64."""
    s = np.asarray(scores, dtype=np.float32)
    B, P = s.shape
    if k <= 0:
        return np.zeros((B, 0), dtype=np.int64)
    if k >= P:
        return np.broadcast_to(np.arange(P, dtype=np.int64), (B, P)).copy()
    out = np.empty((B, k), dtype=np.int64)
    idx = np.arange(P)
    for b in range(B):
        row = s[b].astype(np.float64)
        isnan = np.isnan(row)
        key = np.where(isnan, 0.0, -row)  # -(-0.0) == -(0.0) under float compare
        order = np.lexsort((idx, key, ~isnan))  # NaN first, then score descending, then index
        out[b] = np.sort(order[:k])
    return out


@dataclass
class Plan:
    update_indice: np.ndarray      # [B, T]
    active_batch_idx: np.ndarray   # [M]
    active_pos_idx: np.ndarray     # [M]
    active_token_idx: np.ndarray   # [M]
    active_patch_mask: np.ndarray  # [M] bool
    active_rope_idx: np.ndarray    # [M]
    keep_mask: np.ndarray          # [B, P] bool
    row_slot: np.ndarray           # [B, N] int32 (packed row or -1)


def build_plan(scores: np.ndarray, k: int, dindice: np.ndarray, num_pretokens: int, num_tokens: int) -> Plan:
    dindice = np.asarray(dindice, dtype=np.int64)
    B = dindice.shape[0]
    P = dindice.shape[1] - num_pretokens
    kept = topk_keep(scores, k)
    pre = dindice[:, :num_pretokens]
    patches = dindice[:, num_pretokens:]
    upd = np.concatenate([pre, np.take_along_axis(patches, kept, axis=1)], axis=1)
    T = upd.shape[1]
    tok = upd.reshape(-1)
    keep_mask = np.zeros((B, P), dtype=bool)
    np.put_along_axis(keep_mask, kept, True, axis=1)
    row_slot = np.full((B, num_tokens), -1, dtype=np.int32)
    for b in range(B):
        for s in range(T):
            t = upd[b, s]
            if 0 <= t < num_tokens:
                row_slot[b, t] = b * T + s
    return Plan(
        update_indice=upd,
        active_batch_idx=np.repeat(np.arange(B, dtype=np.int64), T),
        active_pos_idx=np.tile(np.arange(T, dtype=np.int64), B),
        active_token_idx=tok.copy(),
        active_patch_mask=tok >= num_pretokens,
        active_rope_idx=np.maximum(tok - num_pretokens, 0),
        keep_mask=keep_mask,
        row_slot=row_slot,
    )


def plan_stats(scores: np.ndarray, keep: np.ndarray) -> np.ndarray:
    """block.py:762-788, in float64: (sum(scores * keep), sum(scores), sum(keep), B * P, B).
    keep enters the product as 0.0 / 1.0, so an unkept -inf (or any NaN) score makes the first sum
    NaN, as (scores * keep.to(scores.dtype)).sum() does."""
    s = np.asarray(scores, dtype=np.float64)
    kf = np.asarray(keep, dtype=bool).astype(np.float64)
    B, P = s.shape
    with np.errstate(invalid="ignore"):
        kept_mass = float((s * kf).sum())
    return np.array([kept_mass, float(s.sum()), float(kf.sum()), float(B * P), float(B)], dtype=np.float64)
