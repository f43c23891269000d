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


# ------------------------------------------------------------------------------------------------
# Threshold selection (block.py:374-376) and its two builders (block.py:492-560, 562-621)
# ------------------------------------------------------------------------------------------------


def threshold_keep(scores: np.ndarray, thres: float) -> np.ndarray:
    """block.py:374-376, `combined_patch_scores >= token_keep_thres`: torch compares an fp32 tensor with
    a Python float in fp32, the float rounded to the nearest fp32 first; NaN is never kept."""
    s = np.asarray(scores, dtype=np.float32)
    with np.errstate(invalid="ignore"):
        return s >= np.float32(thres)


@dataclass
class ThresholdPlan(Plan):
    """The reference's PackedQueryState for threshold selection (its active_* are the compacted rows
    at query_valid_mask), plus `rows`: the same plan at a fixed B x T packed layout in which every slot
    that is not a query repeats its image's last valid row -- the layout the GPU path runs."""
    query_valid_mask: np.ndarray = None   # [B, T] bool
    kept_count: np.ndarray = None         # [B] int64
    all_valid: bool = True
    rows: Plan = None


def _rows_plan(upd_rows: np.ndarray, valid: np.ndarray, keep: np.ndarray, num_pretokens: int,
               num_tokens: int) -> Plan:
    B, T = upd_rows.shape
    tok = upd_rows.reshape(-1)
    row_slot = np.full((B, num_tokens), -1, dtype=np.int32)
    for b in range(B):
        for s in range(T):
            t = upd_rows[b, s]
            if valid[b, s] and 0 <= t < num_tokens and row_slot[b, t] < 0:
                row_slot[b, t] = b * T + s          # the first slot that holds the token
    return Plan(update_indice=upd_rows, active_batch_idx=np.repeat(np.arange(B, dtype=np.int64), T),
                active_pos_idx=np.tile(np.arange(T, dtype=np.int64), B), active_token_idx=tok.copy(),
                active_patch_mask=tok >= num_pretokens, active_rope_idx=np.maximum(tok - num_pretokens, 0),
                keep_mask=keep, row_slot=row_slot)


def threshold_plan(scores: np.ndarray, thres: float, dindice: np.ndarray, num_pretokens: int, num_tokens: int,
                   keep_cap: int = 0) -> ThresholdPlan:
    """keep_cap > 0: _build_packed_query_state_thres_static (block.py:492-560) -- width
    K = min(keep_cap, P); slot j of image b holds its kept candidate number min(j, count_b - 1) in
    candidate order (candidate 0 when it keeps none), so a row keeping more than K drops its last kept
    candidates; every slot is a query.
    keep_cap == 0: _build_packed_query_state (block.py:562-621) -- width = the largest kept count;
    slots past an image's count hold token 0 and are not queries; the active rows are the queries in
    row-major order; all_valid is True for B <= 1 or no slots, else whether every count equals the
    largest."""
    dindice = np.asarray(dindice, dtype=np.int64)
    B = dindice.shape[0]
    P = dindice.shape[1] - num_pretokens
    keep = threshold_keep(scores, thres).reshape(B, P)
    count = keep.sum(axis=1).astype(np.int64)
    pre = dindice[:, :num_pretokens]
    patches = dindice[:, num_pretokens:]
    kept = [np.flatnonzero(keep[b]) for b in range(B)]
    static = keep_cap > 0
    W = max(0, min(int(keep_cap), P)) if static else (int(count.max()) if B else 0)
    upd_p = np.zeros((B, W), dtype=np.int64)
    valid_p = np.zeros((B, W), dtype=bool)
    rows_p = np.zeros((B, W), dtype=np.int64)
    for b in range(B):
        c = int(count[b])
        for j in range(W):
            if static:
                cand = int(kept[b][min(j, c - 1)]) if c > 0 else 0
                upd_p[b, j] = rows_p[b, j] = patches[b, cand]
                valid_p[b, j] = True
            elif j < c:
                upd_p[b, j] = rows_p[b, j] = patches[b, kept[b][j]]
                valid_p[b, j] = True
            else:
                # not a query: token 0 in update_indice; the packed row repeats the last valid row
                last = patches[b, kept[b][c - 1]] if c > 0 else (pre[b, -1] if num_pretokens > 0 else 0)
                rows_p[b, j] = last
    upd = np.concatenate([pre, upd_p], axis=1)
    valid = np.concatenate([np.ones((B, num_pretokens), dtype=bool), valid_p], axis=1)
    rows_tok = np.concatenate([pre, rows_p], axis=1)
    bi, pi = np.nonzero(valid)
    tok = upd[bi, pi]
    T = upd.shape[1]
    if static:
        all_valid = True
    else:
        all_valid = True if (B <= 1 or valid.size == 0) else bool(np.all(count == W))
    rows = _rows_plan(rows_tok, valid, keep, num_pretokens, num_tokens)
    return ThresholdPlan(update_indice=upd, active_batch_idx=bi.astype(np.int64), active_pos_idx=pi.astype(np.int64),
                         active_token_idx=tok.astype(np.int64), active_patch_mask=tok >= num_pretokens,
                         active_rope_idx=np.maximum(tok - num_pretokens, 0), keep_mask=keep, row_slot=rows.row_slot,
                         query_valid_mask=valid, kept_count=count, all_valid=all_valid, rows=rows)
