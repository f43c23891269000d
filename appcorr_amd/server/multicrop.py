"""Batched correction of several crops (or images) that carry their own caches and candidate lists.

The segmentation executor of the reference corrects the crops of a request together so that every
correction GEMM sees all their selected rows at once (offload/server/model/dinov3_segmentor_m2f.py:
1499-1656): candidate lists are padded to a common length with invalid slots, crops whose shapes
agree are grouped into buckets, each bucket's per-layer caches are concatenated along the batch,
the correction blocks run once over the bucket with `candidate_valid_mask`, and the updated caches
are split back to their crops (:1707-1785). This module is that caller side, built on the block's
own threshold / top-k plan kernels. It reads nothing back from the device except in union_dindices
(the per-row unique lengths, which torch.unique needs on the host there as in the reference); whether
a bucket has padded slots is known from the host-side candidate counts.

Padded candidate slots repeat the crop's last real candidate and score -inf, so neither a threshold
nor top-k selects them; with a threshold the kept set of each crop is exactly the one it has alone
(top-k takes k from the padded candidate count, as in the reference).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Callable, Dict, List, Sequence

import torch


@dataclass
class CropItem:
    """One crop of a batched correction: tokens [b, N, C], dindice [b, pre + P_i], the crop's own cache
    (keys f"{prefix}layer{l}_kv" / "_blocks_out_sum" / "_server_pscore") and optional mobile hint."""
    input_tokens: torch.Tensor
    dindice: torch.Tensor
    num_pre: int
    cache: Dict[str, Any]
    rope: Any = None
    mobile_pscore_hint: torch.Tensor | None = None
    prefix: str = ""
    cand_valid: torch.Tensor | None = field(default=None, repr=False)
    n_padded: int = 0  # padded candidate slots per row (set by pad_crop_candidates)


def pad_crop_candidates(items: Sequence[CropItem]) -> None:
    """dinov3_segmentor_m2f.py:1506-1520: pad every candidate list to the longest one by repeating its
    last real candidate, and mark the padded slots invalid (in place)."""
    if not items:
        return
    max_cand = max(int(it.dindice.shape[1]) - it.num_pre for it in items)
    for it in items:
        d = it.dindice
        n_cand = int(d.shape[1]) - it.num_pre
        valid = torch.ones((d.shape[0], n_cand), dtype=torch.bool, device=d.device)
        it.n_padded = 0
        if 0 < n_cand < max_cand:
            pad = max_cand - n_cand
            it.dindice = torch.cat([d, d[:, -1:].expand(-1, pad)], dim=1)
            valid = torch.cat([valid, torch.zeros((d.shape[0], pad), dtype=torch.bool, device=d.device)], dim=1)
            it.n_padded = pad
        it.cand_valid = valid


def _rope_key(rope) -> Any:
    if rope is None:
        return None
    return tuple((t.data_ptr(), tuple(t.shape), str(t.dtype)) for t in rope)


def batch_key(it: CropItem) -> tuple:
    """Crops batch together when token shapes, candidate count, dtype, RoPE tables and hint layout
    agree (dinov3_segmentor_m2f.py:1522-1532)."""
    hint = it.mobile_pscore_hint
    return (tuple(it.input_tokens.shape[1:]), int(it.dindice.shape[1]), str(it.input_tokens.dtype), _rope_key(it.rope),
            None if hint is None else (tuple(hint.shape[1:]), str(hint.dtype)))


def build_batch_cache(items: Sequence[CropItem], start_l: int, end_l: int, *, server_pscore: str,
                      server_pscore_weight: float, tag_prefix: str = "batch_") -> Dict[str, Any] | None:
    """dinov3_segmentor_m2f.py:1707-1745: concatenate the crops' per-layer caches along the batch.
    Server scores of every layer up to end_l are included for a layer-mean score. None when a needed
    entry is missing or the crops' tensors disagree in shape, dtype or device."""
    out: Dict[str, Any] = {}
    layers = range(0, end_l) if server_pscore.endswith("_layermean") else range(start_l, end_l)

    def cat(ts):
        t0 = ts[0]
        if any(t.shape[1:] != t0.shape[1:] or t.dtype != t0.dtype or t.device != t0.device for t in ts):
            return None
        return torch.cat(ts, dim=0)

    for l in layers:
        ts = [it.cache.get(f"{it.prefix}layer{l}_server_pscore") for it in items]
        if any(t is None for t in ts):
            if server_pscore_weight != 0.0 and start_l <= l < end_l:
                return None
            continue
        c = cat(ts)
        if c is None:
            return None
        out[f"{tag_prefix}layer{l}_server_pscore"] = c
    for l in range(start_l, end_l):
        for suffix in ("_kv", "_blocks_out_sum"):
            ts = [it.cache.get(f"{it.prefix}layer{l}{suffix}") for it in items]
            if any(t is None for t in ts):
                return None
            c = cat(ts)
            if c is None:
                return None
            out[f"{tag_prefix}layer{l}{suffix}"] = c
    return out


def scatter_batch_cache(items: Sequence[CropItem], batch_cache: Dict[str, Any], start_l: int, end_l: int,
                        tag_prefix: str = "batch_") -> None:
    """dinov3_segmentor_m2f.py:1754-1778: split both `_kv` and `_blocks_out_sum` of every layer back to
    the crops as fresh tensors (the corrected K/V rows and the persisted increments)."""
    off = 0
    for it in items:
        n = int(it.input_tokens.shape[0])
        for l in range(start_l, end_l):
            for suffix in ("_kv", "_blocks_out_sum"):
                t = batch_cache.get(f"{tag_prefix}layer{l}{suffix}")
                if t is not None:
                    it.cache[f"{it.prefix}layer{l}{suffix}"] = t[off:off + n].detach().clone()
        off += n


# dinov3_segmentor_m2f.py:68-80
_TOTAL_KEYS = ("_attn_prob_mass_used_total", "_attn_prob_mass_full_total", "_token_prune_kept_patch_total",
               "_token_prune_full_patch_total", "_token_prune_kept_residual_mass_total",
               "_token_prune_full_residual_mass_total", "_token_pscore_kept_mass_total", "_token_pscore_full_mass_total",
               "_partial_token_kept_patch_total", "_partial_token_full_patch_total", "_partial_token_sample_total")


def add_batch_total_stats(dst_cache: Dict[str, Any], batch_cache: Dict[str, Any]) -> None:
    """dinov3_segmentor_m2f.py:1780-1785: fold the batch's plan statistics into one crop's cache."""
    for k in _TOTAL_KEYS:
        v = batch_cache.get(k)
        if v is not None:
            dst_cache[k] = dst_cache.get(k, v.new_zeros((), dtype=torch.float32)) + v


def union_dindices(dindices: List[torch.Tensor]) -> torch.Tensor:
    """dinov3_segmentor_m2f.py:1836-1843: per-row sorted union of several index lists (all rows must
    end up with the same length)."""
    if not dindices:
        raise ValueError("union_dindices needs at least one index list")
    merged = torch.cat(dindices, dim=1)
    rows = [torch.unique(r, sorted=True) for r in merged]
    if any(r.numel() != rows[0].numel() for r in rows):
        raise RuntimeError("union_dindices: rows of different lengths")
    return torch.stack(rows, dim=0)


RunBlock = Callable[..., tuple]


def correct_crops_batched(run_block: RunBlock, items: List[CropItem], start_l: int, end_l: int,
                          **correct_kwargs) -> List[torch.Tensor]:
    """Pad, bucket, batch and correct layers [start_l, end_l) of every crop; returns each crop's
    corrected tokens and leaves each crop's cache updated (dinov3_segmentor_m2f.py:1499-1656).

    `run_block(layer_idx, x, dindice, rope, cache, tag, source_key=..., **kw)` is the executor's
    per-layer correction call (run_dinov3_correct_block). Raises if a bucket's caches cannot be
    batched (the reference then returns False and falls back to per-crop correction)."""
    pad_crop_candidates(items)
    buckets: Dict[tuple, List[int]] = {}
    for i, it in enumerate(items):
        buckets.setdefault(batch_key(it), []).append(i)
    server_pscore = str(correct_kwargs.get("server_pscore", "cls_attn_prob"))
    server_w = float(correct_kwargs.get("server_pscore_weight", 1.0))
    out: List[torch.Tensor | None] = [None] * len(items)
    for idx in buckets.values():
        group = [items[i] for i in idx]
        bc = build_batch_cache(group, start_l, end_l, server_pscore=server_pscore, server_pscore_weight=server_w)
        if bc is None:
            raise RuntimeError("crops of one bucket have caches that cannot be batched")
        x = torch.cat([it.input_tokens for it in group], dim=0)
        dind = torch.cat([it.dindice for it in group], dim=0)
        # nothing padded (known on the host): no mask
        cv = torch.cat([it.cand_valid for it in group], dim=0) if any(it.n_padded for it in group) else None
        hints = [it.mobile_pscore_hint for it in group]
        hint = None if any(h is None for h in hints) else torch.cat(hints, dim=0)
        for l in range(start_l, end_l):
            tag = f"batch_layer{l}"
            x, bc = run_block(l, x, dind, group[0].rope, bc, tag, source_key=tag, mobile_pscore_hint=hint,
                              candidate_valid_mask=cv, **correct_kwargs)
        scatter_batch_cache(group, bc, start_l, end_l)
        add_batch_total_stats(group[0].cache, bc)
        for i, xs in zip(idx, torch.split(x, [int(it.input_tokens.shape[0]) for it in group], dim=0)):
            out[i] = xs
    return out
