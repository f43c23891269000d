"""Pixel-residual importance and image-residual token pruning, restated in numpy. Test infrastructure only.

Follows offload/server/model/dinov3_classifier.py:
  _compute_patch_residual_rms         :91-122   (curr - prev in fp32, per patch sqrt(mean(d^2)))
  _apply_image_residual_token_pruning :124-197  (threshold or top-min_keep, masses, compaction)
and offload/policies/transmission/progressive.py:14-22 (a residual crop's RMS / energy).

The reductions are evaluated exactly (float64 sums of fp32 squares, exact for integer pixels and for
the quantised float inputs the tests use) and rounded once; the reference's torch / numpy fp32
reductions land within a few ulp of that (tests/test_oracle_importance.py). The top-min_keep set
uses oracle.plan.topk_keep's tie rule (lower candidate index first, NaN largest); torch.topk's
order among equal residuals is "parity unpinned", as for the top-k plan.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .plan import topk_keep

L2, ENERGY, RMS = 0, 1, 2


def patch_residual_score(curr: np.ndarray, prev: np.ndarray | None, ph: int, pw: int, mode: int = RMS,
                         image_idx: np.ndarray | None = None) -> np.ndarray:
    """curr / prev [B, H, W, C] -> [n, (H/ph) * (W/pw)] fp32 (n = len(image_idx) or B)."""
    c = np.asarray(curr)
    if image_idx is not None:
        c = c[np.asarray(image_idx)]
    d = c.astype(np.float32)
    if prev is not None:
        p = np.asarray(prev)
        if image_idx is not None:
            p = p[np.asarray(image_idx)]
        d = d - p.astype(np.float32)                     # fp32 residual
    B, H, W, C = d.shape
    gh, gw = H // ph, W // pw
    sq = (d * d).astype(np.float32)                      # fp32 squares, as materialised
    sq = sq.reshape(B, gh, ph, gw, pw, C).transpose(0, 1, 3, 2, 4, 5).reshape(B, gh * gw, ph * pw * C)
    tot = sq.astype(np.float64).sum(axis=2)
    if mode == ENERGY:
        return tot.astype(np.float32)
    if mode == RMS:
        mean = (tot / float(ph * pw * C)).astype(np.float32)
        return np.sqrt(mean.astype(np.float64)).astype(np.float32)
    return np.sqrt(tot.astype(np.float32).astype(np.float64)).astype(np.float32)


@dataclass
class Pruned:
    pruned_dindice: np.ndarray     # [B, pre + width]
    kept_patch_count: np.ndarray   # [B]
    full_patch_count: np.ndarray   # [B]
    kept_residual_mass: np.ndarray  # [B] fp32
    full_residual_mass: np.ndarray  # [B] fp32
    kept_local_idx: np.ndarray     # [B, width]
    keep: np.ndarray               # [B, P] bool


def residual_prune(dindice: np.ndarray, spatial: np.ndarray, rms: np.ndarray | None, threshold: float,
                   min_keep: int) -> Pruned:
    """dinov3_classifier.py:124-197 on dindice [B, pre + P], spatial [B, P] (patch indices) and the
    per-image residual RMS map rms [B, G]."""
    dindice = np.asarray(dindice, dtype=np.int64)
    spatial = np.asarray(spatial, dtype=np.int64)
    B, P = spatial.shape
    pre = dindice.shape[1] - P
    full_count = np.full(B, P, dtype=np.int64)
    zeros = np.zeros(B, dtype=np.float32)
    full_idx = np.broadcast_to(np.arange(P, dtype=np.int64), (B, P)).copy()
    if rms is None or P == 0:
        return Pruned(dindice, full_count.copy(), full_count, zeros, zeros.copy(), full_idx, np.ones((B, P), bool))
    r = np.take_along_axis(np.asarray(rms, dtype=np.float32), spatial, axis=1)
    with np.errstate(invalid="ignore"):
        keep = r >= np.float32(threshold)
        if min_keep > 0:
            k = min(min_keep, P)
            np.put_along_axis(keep, topk_keep(r, k), True, axis=1)
        full_mass = r.astype(np.float64).sum(axis=1).astype(np.float32)
        kept_mass = (r * keep.astype(np.float32)).astype(np.float64).sum(axis=1).astype(np.float32)
    count = keep.sum(axis=1).astype(np.int64)
    W = int(count.max()) if B else 0
    if W == P:       # some image keeps every candidate: nothing is pruned (:166-174)
        return Pruned(dindice, count, full_count, kept_mass, full_mass, full_idx, keep)
    kept_sp = np.zeros((B, W), dtype=np.int64)
    local = np.zeros((B, W), dtype=np.int64)
    for b in range(B):
        idx = np.flatnonzero(keep[b])
        kept_sp[b, :idx.size] = spatial[b, idx]
        local[b, :idx.size] = idx
    pruned = np.concatenate([dindice[:, :pre], kept_sp + pre], axis=1)
    return Pruned(pruned, count, full_count, kept_mass, full_mass, local, keep)
