"""Shared helpers for the parity tests."""

from __future__ import annotations

import numpy as np
import torch


def bits(t: torch.Tensor) -> np.ndarray:
    """Raw bit pattern of a tensor as a numpy array (bf16 -> uint16, others via their byte view)."""
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    if t.dtype == torch.bool:
        return t.numpy().view(np.uint8)
    return t.numpy()


def assert_bits_equal(got: torch.Tensor, ref, what: str = ""):
    g = bits(got)
    r = bits(ref) if isinstance(ref, torch.Tensor) else np.asarray(ref)
    assert g.shape == r.shape, f"{what}: shape {g.shape} vs {r.shape}"
    bad = np.flatnonzero(g.reshape(-1) != r.reshape(-1))
    assert bad.size == 0, f"{what}: {bad.size} of {g.size} elements differ, first at {bad[:5]}"


def bf16_ulp(x: np.ndarray) -> np.ndarray:
    """Spacing of bf16 values at |x| (2^(e-7)), with a floor at the smallest normal spacing."""
    a = np.abs(np.asarray(x, dtype=np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0**-126)))
    return 2.0 ** (e - 7)


def assert_bf16_close(got: torch.Tensor, ref: torch.Tensor, *, max_ulps: float = 1.0, max_frac_off: float = 0.01,
                      atol: float = 0.0, what: str = ""):
    """bf16 results computed with a different fp32 accumulation order than the oracle: every element
    within `max_ulps` bf16 ulps (+ atol) of the oracle, and at most `max_frac_off` of them not equal."""
    g = got.detach().float().cpu().numpy().astype(np.float64)
    r = ref.detach().float().cpu().numpy().astype(np.float64)
    assert g.shape == r.shape, f"{what}: shape {g.shape} vs {r.shape}"
    assert np.isfinite(g).all(), f"{what}: non-finite output"
    diff = np.abs(g - r)
    lim = max_ulps * bf16_ulp(r) + atol
    worst = np.argmax(diff - lim)
    assert (diff <= lim).all(), (f"{what}: max excess at {np.unravel_index(worst, g.shape)}: got {g.flat[worst]}, "
                                 f"ref {r.flat[worst]}, diff {diff.flat[worst]}, limit {lim.flat[worst]}")
    frac = float((diff > 0).mean())
    assert frac <= max_frac_off, f"{what}: {frac:.4%} of elements differ (limit {max_frac_off:.2%})"


def ulp_stats(got: torch.Tensor, ref: torch.Tensor):
    """(max, mean) of |got - ref| in units of the bf16 ulp at the reference, and the fraction differing."""
    g = got.detach().float().cpu().numpy().astype(np.float64)
    r = ref.detach().float().cpu().numpy().astype(np.float64)
    u = np.abs(g - r) / bf16_ulp(r)
    return float(u.max()), float(u.mean()), float((g != r).mean())


def assert_ulps(got: torch.Tensor, ref: torch.Tensor, *, max_ulps: float, mean_ulps: float, what: str = ""):
    """Statistical bf16 agreement for results several roundings downstream of an accumulation-order
    difference: no element beyond max_ulps, and the average error well below one ulp."""
    mx, mean, frac = ulp_stats(got, ref)
    assert np.isfinite(got.detach().float().cpu().numpy()).all(), f"{what}: non-finite output"
    assert mx <= max_ulps and mean <= mean_ulps, (f"{what}: max {mx:.2f} ulp (limit {max_ulps}), mean {mean:.4f} ulp "
                                                  f"(limit {mean_ulps}), {frac:.3%} differ")


def assert_propagated_close(got: torch.Tensor, ref: torch.Tensor, *, max_ulps: float = 8.0,
                            floor_rel: float = 2.0 ** -6, mean_rel: float = 2.0 ** -9, floor_abs=None,
                            what: str = ""):
    """Agreement for outputs several bf16 roundings downstream of fp32-vs-fp64 accumulation.

    Each element within max_ulps ulp of the oracle, or within floor_rel * rms(oracle) for values that
    come out of a cancellation (a one-ulp flip of a summand of size ~rms shows up there as an absolute
    error of ~2^-8 rms); and the mean absolute error below mean_rel * mean|oracle| (2^-9: half a bf16
    ulp on average)."""
    g = got.detach().float().cpu().numpy().astype(np.float64)
    r = ref.detach().float().cpu().numpy().astype(np.float64)
    assert g.shape == r.shape and np.isfinite(g).all(), f"{what}: shape/finite"
    d = np.abs(g - r)
    u = bf16_ulp(r)
    floor = floor_rel * float(np.sqrt((r ** 2).mean()))
    if floor_abs is not None:  # elementwise floor, e.g. the ulp of the summands of a difference
        floor = np.maximum(floor, np.asarray(floor_abs, dtype=np.float64))
    bad = (d > max_ulps * u) & (d > floor)
    assert not bad.any(), (f"{what}: {int(bad.sum())} elements beyond {max_ulps} ulp and the floor; "
                           f"worst {float(d[bad].max())}")
    mean, scale = float(d.mean()), float(np.abs(r).mean())
    assert mean <= mean_rel * scale, f"{what}: mean |error| {mean:.3g} > {mean_rel:.3g} * mean|ref| ({scale:.3g})"


def close_stats(got: torch.Tensor, ref: torch.Tensor):
    d = (got.detach().float().cpu() - ref.detach().float().cpu()).abs()
    return float(d.max()), float(d.mean())
