"""Tensor-level wrappers over the gfx950 C ABI.

The names and argument meaning follow the reference's kernel wrappers so call sites read the same
(reference: appcorr/models/dinov3/layers/triton_kernels/{token_update,rope,nvfp4_fused}.py). One
behavioural difference is deliberate: where a reference wrapper returned False/None on an
unsupported layout (and `note_fallback` raised by default), these raise `OudjatKernelError` /
`ValueError` directly. There is no eager fallback.

Every launch is enqueued on torch's current stream of the tensors' device and returns without
synchronising.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _lib
from ._lib import call

P = ctypes.c_void_p

# Optional live timing of launch sites: every launch at a site named in `_probe["tags"]` is bracketed
# by a pair of timing events on the launch stream (used by bench.py for the roofline). Sites are the
# kernels' roles in the pass: "qkv", "proj", "fc1", "fc2", "w1", "w2", "w3", "attention", ...
_probe: dict = {"tags": frozenset(), "events": {}}


def set_probe(tags) -> None:
    """Probe the named launch sites (a name, an iterable of names, or None for none)."""
    if tags is None:
        tags = ()
    elif isinstance(tags, str):
        tags = (tags,)
    _probe["tags"] = frozenset(tags)
    _probe["events"] = {}


def probe_events() -> dict:
    """{site: [(start event, end event), ...]} of the probed launches since set_probe."""
    return _probe["events"]


def _launch(tag: str, t: torch.Tensor, name: str, *args) -> None:
    if tag not in _probe["tags"]:
        call(name, *args)
        return
    s = torch.cuda.current_stream(t.device)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(s)
    call(name, *args)
    e1.record(s)
    _probe["events"].setdefault(tag, []).append((e0, e1))


def _ptr(t: torch.Tensor | None) -> P:
    return P(0 if t is None else t.data_ptr())


def _stream(t: torch.Tensor) -> P:
    return P(_lib.stream_of(t))


def _require_cuda(*tensors: torch.Tensor | None) -> None:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError("appcorr_amd kernels run on the GPU only; got a CPU tensor (no CPU fallback exists)")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} vs {t.device}")


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def _index(t: torch.Tensor, name: str) -> torch.Tensor:
    _require(t.dtype == torch.long and t.dim() == 1, f"{name} must be a 1-D int64 tensor")
    return t.contiguous()


def trailing_is_packed(t: torch.Tensor, first_row_dim: int) -> bool:
    """True when dims >= first_row_dim form one contiguous run (a row), whatever the outer strides.

    Same acceptance rule as the reference's `_trailing_is_packed` (token_update.py:390-404): a view
    like qkv_new[:, 1:] has row stride 3C but its 2C row elements are contiguous.
    """
    expected = 1
    for d in range(t.dim() - 1, first_row_dim - 1, -1):
        if t.shape[d] != 1 and t.stride(d) != expected:
            return False
        expected *= t.shape[d]
    return True


def _row_elems(t: torch.Tensor, first_row_dim: int) -> int:
    n = 1
    for d in range(first_row_dim, t.dim()):
        n *= t.shape[d]
    return n


# ------------------------------------------------------------------------------------------------
# Row movement (token_update.py:352-473, 257-347, 10-60)
# ------------------------------------------------------------------------------------------------


def gather_rows(src: torch.Tensor, batch_idx: torch.Tensor, token_idx: torch.Tensor) -> torch.Tensor:
    """`src[batch_idx, token_idx]` as a new contiguous tensor of shape [n, *src.shape[2:]]."""
    _require_cuda(src, batch_idx, token_idx)
    _require(src.dim() >= 2 and trailing_is_packed(src, 2), "gather_rows: src rows (dims 2..) must be packed")
    bi, ti = _index(batch_idx, "batch_idx"), _index(token_idx, "token_idx")
    _require(bi.numel() == ti.numel(), "gather_rows: index length mismatch")
    n = bi.numel()
    out = torch.empty((n, *src.shape[2:]), device=src.device, dtype=src.dtype)
    row_bytes = _row_elems(src, 2) * src.element_size()
    if n == 0 or row_bytes == 0:
        return out
    es = src.element_size()
    _launch("gather_rows", src, "oudjat_gather_rows", _ptr(src), src.stride(0) * es, src.stride(1) * es, row_bytes, _ptr(bi), _ptr(ti), n,
         _ptr(out), row_bytes, _stream(src))
    return out


def scatter_rows(dst: torch.Tensor, batch_idx: torch.Tensor, token_idx: torch.Tensor, src: torch.Tensor) -> bool:
    """`dst[batch_idx, token_idx] = src` in place; (batch, token) pairs must be unique. Returns True."""
    _require_cuda(dst, batch_idx, token_idx, src)
    _require(dst.dim() >= 2 and trailing_is_packed(dst, 2), "scatter_rows: dst rows (dims 2..) must be packed")
    _require(src.dim() >= 1 and trailing_is_packed(src, 1), "scatter_rows: src rows (dims 1..) must be packed")
    _require(src.dtype == dst.dtype, "scatter_rows: dtype mismatch")
    bi, ti = _index(batch_idx, "batch_idx"), _index(token_idx, "token_idx")
    n = bi.numel()
    _require(ti.numel() == n and src.shape[0] == n, "scatter_rows: length mismatch")
    row = _row_elems(dst, 2)
    _require(_row_elems(src, 1) == row, f"scatter_rows: row width mismatch ({_row_elems(src, 1)} vs {row})")
    if n == 0 or row == 0:
        return True
    es = dst.element_size()
    _launch("scatter_rows", dst, "oudjat_scatter_rows", _ptr(dst), dst.stride(0) * es, dst.stride(1) * es, row * es, _ptr(bi), _ptr(ti), n,
         _ptr(src), src.stride(0) * es, _stream(dst))
    return True


def active_token_update(x_base: torch.Tensor, active_batch_idx: torch.Tensor, active_token_idx: torch.Tensor,
                        x_attn_active: torch.Tensor, x_delta_active: torch.Tensor, *,
                        clone_base: bool = True) -> torch.Tensor:
    """x_out = x_base (cloned unless clone_base=False); x_out[b_i, t_i] = x_attn_i + x_delta_i (bf16)."""
    _require_cuda(x_base, active_batch_idx, active_token_idx, x_attn_active, x_delta_active)
    x_out = x_base.clone() if clone_base else x_base
    n = active_batch_idx.numel()
    if n == 0:
        return x_out
    _require(x_out.dtype == torch.bfloat16 and x_out.dim() == 3 and x_out.stride(2) == 1,
             "active_token_update: x_base must be [B, N, C] bf16 with contiguous rows")
    a = x_attn_active.to(torch.bfloat16).contiguous()
    d = x_delta_active.to(torch.bfloat16).contiguous()
    C = x_out.shape[2]
    _require(a.shape == (n, C) and d.shape == (n, C), "active_token_update: [n, C] sources required")
    call("oudjat_active_token_update", _ptr(x_out), x_out.stride(0), x_out.stride(1),
         _ptr(_index(active_batch_idx, "batch")), _ptr(_index(active_token_idx, "token")), n, _ptr(a), C, _ptr(d),
         C, C, _stream(x_out))
    return x_out


def fused_layerscale_add(x: torch.Tensor, x_attn: torch.Tensor, gamma: torch.Tensor) -> torch.Tensor:
    """out = x + x_attn * gamma (gamma broadcast over the last dim), bf16."""
    _require_cuda(x, x_attn, gamma)
    _require(x.dtype == x_attn.dtype == gamma.dtype == torch.bfloat16, "fused_layerscale_add: bf16 only")
    _require(x.shape == x_attn.shape and x.is_contiguous() and x_attn.is_contiguous(),
             "fused_layerscale_add: contiguous tensors of one shape required")
    C = x.shape[-1]
    g = gamma.contiguous()
    _require(g.numel() == C, "fused_layerscale_add: gamma must have C entries")
    out = torch.empty_like(x)
    rows = x.numel() // C if C else 0
    call("oudjat_fused_layerscale_add", _ptr(x), _ptr(x_attn), _ptr(g), rows, C, _ptr(out), _stream(x))
    return out


def reconstruct_scatter_persist(x: torch.Tensor, blocks_out_sum: torch.Tensor, row_slot: torch.Tensor,
                                x_act: torch.Tensor, x_attn: torch.Tensor, mlp: torch.Tensor,
                                out: torch.Tensor | None = None) -> torch.Tensor:
    """Fused block.py:1140-1179: x_out = x + blocks_out_sum off the selected rows; on them
    x_out = x_attn + mlp and blocks_out_sum = (x_attn - x_act) + mlp (in place). `out` may alias x."""
    _require_cuda(x, blocks_out_sum, row_slot, x_act, x_attn, mlp, out)
    _require(x.dtype == blocks_out_sum.dtype == torch.bfloat16, "reconstruct_scatter_persist: bf16 only")
    _require(x.is_contiguous() and blocks_out_sum.is_contiguous() and x.shape == blocks_out_sum.shape,
             "reconstruct_scatter_persist: contiguous x / blocks_out_sum of one shape required")
    _require(row_slot.dtype == torch.int32 and row_slot.is_contiguous() and row_slot.numel() * x.shape[-1] == x.numel(),
             "reconstruct_scatter_persist: row_slot must be int32 with one entry per row")
    for t, nm in ((x_act, "x_act"), (x_attn, "x_attn"), (mlp, "mlp")):
        _require(t.dtype == torch.bfloat16 and t.is_contiguous() and t.shape[-1] == x.shape[-1],
                 f"reconstruct_scatter_persist: {nm} must be contiguous bf16 [M, C]")
    if out is None:
        out = torch.empty_like(x)
    C = x.shape[-1]
    _launch("reconstruct", x, "oudjat_reconstruct_scatter_persist", _ptr(x), _ptr(blocks_out_sum), _ptr(row_slot), _ptr(x_act),
         _ptr(x_attn), _ptr(mlp), x.numel() // C, C, _ptr(out), _stream(x))
    return out


def packed_residual_persist(x_act: torch.Tensor, x_attn: torch.Tensor, mlp: torch.Tensor, batch_idx: torch.Tensor,
                            token_idx: torch.Tensor, blocks_out_sum: torch.Tensor) -> torch.Tensor:
    """Selected rows kept packed: returns x_new = x_attn + mlp (bf16) and writes
    blocks_out_sum[b_i, t_i] = (x_attn - x_act) + mlp in place (block.py:1140-1179, selected rows)."""
    _require_cuda(x_act, x_attn, mlp, batch_idx, token_idx, blocks_out_sum)
    for t, nm in ((x_act, "x_act"), (x_attn, "x_attn"), (mlp, "mlp")):
        _require(t.dtype == torch.bfloat16 and t.dim() == 2 and t.is_contiguous() and t.shape == x_act.shape,
                 f"packed_residual_persist: {nm} must be contiguous bf16 [M, C]")
    M, C = x_act.shape
    _require(blocks_out_sum.dim() == 3 and blocks_out_sum.shape[2] == C and blocks_out_sum.stride(2) == 1,
             "packed_residual_persist: blocks_out_sum must be [B, N, C] with contiguous rows")
    x_new = torch.empty_like(x_act)
    _launch("packed_residual", x_act, "oudjat_packed_residual_persist", _ptr(x_act), _ptr(x_attn), _ptr(mlp), M, C,
            _ptr(_index(batch_idx, "batch_idx")), _ptr(_index(token_idx, "token_idx")), _ptr(blocks_out_sum),
            blocks_out_sum.stride(0), blocks_out_sum.stride(1), _ptr(x_new), _stream(x_act))
    return x_new


def _nvfp4_scale(ts: torch.Tensor | None, what: str) -> torch.Tensor | None:
    if ts is not None:
        _require(ts.dtype == torch.float32 and ts.numel() == 1 and ts.is_cuda,
                 f"{what}: the NVFP4 tensor scale must be one fp32 value on the device")
    return ts


def packed_residual_persist_ln(x_act: torch.Tensor, x_attn: torch.Tensor, mlp: torch.Tensor, batch_idx: torch.Tensor,
                               token_idx: torch.Tensor, blocks_out_sum: torch.Tensor, ln_weight: torch.Tensor,
                               ln_bias: torch.Tensor, eps: float, nvfp4_scale: torch.Tensor | None = None):
    """packed_residual_persist fused with the next block's first LayerNorm: returns (x_new, LN(x_new)),
    the LayerNorm bit-identical to layer_norm(x_new) (block.py:1140-1179, then :1114 of the next block).
    With nvfp4_scale (the next qkv linear's NVFP4 activation scale) the second tensor is instead the
    NVFP4 operand x_hat of LN(x_new), as nvfp4_quantize_dequantize would give it."""
    _require_cuda(x_act, x_attn, mlp, batch_idx, token_idx, blocks_out_sum, ln_weight, ln_bias)
    ts = _nvfp4_scale(nvfp4_scale, "packed_residual_persist_ln")
    for t, nm in ((x_act, "x_act"), (x_attn, "x_attn"), (mlp, "mlp")):
        _require(t.dtype == torch.bfloat16 and t.dim() == 2 and t.is_contiguous() and t.shape == x_act.shape,
                 f"packed_residual_persist_ln: {nm} must be contiguous bf16 [M, C]")
    M, C = x_act.shape
    _require(blocks_out_sum.dim() == 3 and blocks_out_sum.shape[2] == C and blocks_out_sum.stride(2) == 1,
             "packed_residual_persist_ln: blocks_out_sum must be [B, N, C] with contiguous rows")
    _require(ln_weight.dtype == ln_bias.dtype == torch.bfloat16 and ln_weight.numel() == C == ln_bias.numel(),
             "packed_residual_persist_ln: bf16 LayerNorm parameters of size C")
    x_new = torch.empty_like(x_act)
    ln_out = torch.empty_like(x_act)
    args = (_ptr(x_act), _ptr(x_attn), _ptr(mlp), M, C, _ptr(_index(batch_idx, "batch_idx")),
            _ptr(_index(token_idx, "token_idx")), _ptr(blocks_out_sum), blocks_out_sum.stride(0),
            blocks_out_sum.stride(1), _ptr(x_new), _ptr(ln_weight.contiguous()), _ptr(ln_bias.contiguous()), float(eps))
    if ts is None:
        _launch("packed_residual", x_act, "oudjat_packed_residual_persist_ln", *args, _ptr(ln_out), _stream(x_act))
    else:
        _launch("packed_residual", x_act, "oudjat_packed_residual_persist_ln_nvfp4", *args, _ptr(ts), _ptr(ln_out),
                _stream(x_act))
    return x_new, ln_out


def linear_splits_k(M: int, N: int, K: int) -> bool:
    """Whether an M x N x K LayerScale product (fc2, w3) splits K given a workspace."""
    key = ("gemm", M, N, K, _lib.EPI_BIAS_LS)
    elems = _WS_ELEMS.get(key)
    if elems is None:
        elems = int(_lib.load().oudjat_linear_workspace_elems(M, N, K, _lib.EPI_BIAS_LS))
        _WS_ELEMS[key] = elems
    return elems > 0


def linear_warm_slots(M: int, N: int, K: int, epilogue: int) -> int:
    """Warming workgroups `linear(..., warm=...)` adds for an M x N x K product with this epilogue (0:
    its tiles fill the GPU or it splits K, and the region is not read)."""
    key = ("warm", M, N, K, int(epilogue))
    n = _WS_ELEMS.get(key)
    if n is None:
        n = int(_lib.load().oudjat_linear_warm_slots(M, N, K, int(epilogue)))
        _WS_ELEMS[key] = n
    return n


def linear_ls_packed_residual(h: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None, gamma: torch.Tensor,
                              x_act: torch.Tensor, x_attn: torch.Tensor, batch_idx: torch.Tensor,
                              token_idx: torch.Tensor, blocks_out_sum: torch.Tensor, ln=None, site: str = "fc2"):
    """mlp = bf16(bf16(h . W^T + bias) * gamma) split K, its reduce fused with packed_residual_persist_ln
    (or packed_residual_persist when `ln` is None): returns (x_new, LN(x_new) or None), bit-identical to
    linear(..., EPI_BIAS_LS) followed by that residual step. `ln` = (weight, bias, eps) of the next block's
    norm1. Returns None when the product does not split K or an operand is not 16-byte aligned (the
    caller then runs the two steps)."""
    M, Kd = h.shape
    N = weight.shape[0]
    if not linear_splits_k(M, N, Kd):
        return None
    tensors = [h, weight, gamma, x_act, x_attn] + ([bias] if bias is not None else [])
    if ln is not None:
        tensors += [ln[0], ln[1]]
    if any(t.data_ptr() % 16 for t in tensors) or h.stride(1) != 1 or weight.stride(1) != 1:
        return None
    _require_cuda(h, weight, bias, gamma, x_act, x_attn, batch_idx, token_idx, blocks_out_sum)
    _require(x_act.shape == x_attn.shape == (M, N) and x_act.is_contiguous() and x_attn.is_contiguous()
             and x_act.dtype == x_attn.dtype == torch.bfloat16, "linear_ls_packed_residual: x_act / x_attn [M, N] bf16")
    _require(blocks_out_sum.dim() == 3 and blocks_out_sum.shape[2] == N and blocks_out_sum.stride(2) == 1,
             "linear_ls_packed_residual: blocks_out_sum must be [B, N, C] with contiguous rows")
    elems = int(_lib.load().oudjat_linear_workspace_elems(M, N, Kd, _lib.EPI_BIAS_LS))
    ws = _stream_workspace(h, elems)
    slices = ctypes.c_int64(0)
    _launch(site, h, "oudjat_linear_splitk_partial", _ptr(h), M, Kd, h.stride(0), _ptr(weight), N, weight.stride(0),
            _ptr(ws), ws.numel(), ctypes.addressof(slices), _stream(h))
    x_new = torch.empty_like(x_act)
    ln_out = torch.empty_like(x_act) if ln is not None else None
    lw, lb, eps = (ln[0].contiguous(), ln[1].contiguous(), float(ln[2])) if ln is not None else (None, None, 0.0)
    _launch("packed_residual", x_act, "oudjat_splitk_ls_packed_residual", _ptr(ws), slices.value, _ptr(bias),
            _ptr(gamma.contiguous()), 1.0, _ptr(x_act), _ptr(x_attn), M, N, _ptr(_index(batch_idx, "batch_idx")),
            _ptr(_index(token_idx, "token_idx")), _ptr(blocks_out_sum), blocks_out_sum.stride(0),
            blocks_out_sum.stride(1), _ptr(x_new), _ptr(lw), _ptr(lb), eps, _ptr(ln_out), _stream(x_act))
    return x_new, ln_out


POINTER_ARRAYS_KEY = "_oudjat_device_pointer_arrays"


def device_pointer_array(ptrs, device, holder: dict | None = None) -> torch.Tensor:
    """Device int64 array of the given addresses.

    With a `holder` (the session's cache dict, which owns the tensors the addresses point at) the
    array is built once per distinct address list and kept in holder[POINTER_ARRAYS_KEY], so repeated
    calls copy nothing from the host and can run inside a captured HIP graph: the array lives exactly
    as long as the dict that keeps its tensors alive. An array is dropped only when the holder no
    longer holds every tensor it points at (a graph recorded over those tensors could not be replayed
    anyway). Without a holder a fresh array is copied from the host on every call."""
    if holder is None:
        return torch.tensor(list(ptrs), dtype=torch.int64).to(device)
    store = holder.setdefault(POINTER_ARRAYS_KEY, {})
    key = (str(device), tuple(int(p) for p in ptrs))
    t = store.get(key)
    if t is None:
        live = {v.data_ptr() for v in holder.values() if isinstance(v, torch.Tensor)}
        for stale in [k for k in store if not set(k[1]) <= live]:
            del store[stale]
        t = torch.tensor(list(key[1]), dtype=torch.int64).to(device)
        store[key] = t
    return t


def fold_residual_rows(x: torch.Tensor, row_slot: torch.Tensor, x_packed: torch.Tensor, blocks_out_sums,
                       out: torch.Tensor | None = None, ptr_holder: dict | None = None) -> torch.Tensor:
    """x [B, N, C] after a run of correction blocks whose selected rows stayed packed: selected rows from
    x_packed [M, C] (row_slot [B, N] int32 maps a token to its packed row), the other rows
    x + bos_0 + ... + bos_{L-1} with a bf16 rounding after each addition. `out` may alias x.
    `ptr_holder`: the dict owning the blocks_out_sum tensors (see device_pointer_array)."""
    _require_cuda(x, row_slot, x_packed, out, *blocks_out_sums)
    _require(x.dtype == torch.bfloat16 and x.is_contiguous() and x.dim() == 3, "fold_residual_rows: x [B, N, C] bf16")
    for b in blocks_out_sums:
        _require(b.dtype == torch.bfloat16 and b.is_contiguous() and b.shape == x.shape,
                 "fold_residual_rows: blocks_out_sum tensors must be contiguous and shaped like x")
    _require(row_slot.dtype == torch.int32 and row_slot.is_contiguous() and row_slot.numel() * x.shape[2] == x.numel(),
             "fold_residual_rows: row_slot must be int32 [B, N]")
    _require(x_packed.dtype == torch.bfloat16 and x_packed.is_contiguous() and x_packed.shape[-1] == x.shape[2],
             "fold_residual_rows: x_packed must be contiguous bf16 [M, C]")
    if out is None:
        out = torch.empty_like(x)
    ptrs = device_pointer_array([b.data_ptr() for b in blocks_out_sums] or [0], x.device, ptr_holder)
    C = x.shape[2]
    _launch("fold", x, "oudjat_fold_residual_rows", _ptr(x), x.numel() // C, C, _ptr(row_slot), _ptr(x_packed),
            _ptr(ptrs), len(blocks_out_sums), _ptr(out), _stream(x))
    return out


# ------------------------------------------------------------------------------------------------
# Plan (block.py:358-490)
# ------------------------------------------------------------------------------------------------


@dataclass
class TopkPlan:
    update_indice: torch.Tensor      # [B, T] int64
    active_batch_idx: torch.Tensor   # [M] int64
    active_pos_idx: torch.Tensor     # [M] int64
    active_token_idx: torch.Tensor   # [M] int64
    active_patch_mask: torch.Tensor  # [M] bool
    active_rope_idx: torch.Tensor    # [M] int64
    keep_mask: torch.Tensor          # [B, P] bool
    row_slot: torch.Tensor | None    # [B, N] int32 (packed row of each token or -1)


def topk_plan(scores: torch.Tensor, k: int, dindice: torch.Tensor, num_pretokens: int,
              num_tokens: int | None = None) -> TopkPlan:
    """Select the k highest-scoring candidates per row and build the packed query plan on device.

    scores [B, P] fp32 (combined patch scores), dindice [B, num_pretokens + P] int64. Ties go to the
    lower candidate index. `num_tokens` (N) additionally requests the token -> packed-row map.
    """
    _require_cuda(scores, dindice)
    _require(scores.dtype == torch.float32 and scores.dim() == 2 and scores.stride(1) == 1,
             "topk_plan: scores must be [B, P] fp32 with contiguous rows")
    _require(dindice.dtype == torch.long and dindice.dim() == 2 and dindice.stride(1) == 1,
             "topk_plan: dindice must be [B, pre + P] int64 with contiguous rows")
    B, Pn = scores.shape
    _require(dindice.shape[0] == B and dindice.shape[1] == num_pretokens + Pn, "topk_plan: dindice shape mismatch")
    k = int(k)
    _require(0 <= k <= Pn, f"topk_plan: k={k} outside [0, {Pn}]")
    T = num_pretokens + k
    dev = scores.device
    upd = torch.empty((B, T), device=dev, dtype=torch.long)
    abat = torch.empty((B * T,), device=dev, dtype=torch.long)
    apos = torch.empty_like(abat)
    atok = torch.empty_like(abat)
    pmask = torch.empty((B * T,), device=dev, dtype=torch.bool)
    ridx = torch.empty_like(abat)
    keep = torch.empty((B, Pn), device=dev, dtype=torch.bool)
    slot = None
    if num_tokens is not None:
        slot = torch.empty((B, int(num_tokens)), device=dev, dtype=torch.int32)
    _launch("topk_plan", scores, "oudjat_topk_plan", _ptr(scores), B, Pn, scores.stride(0), k, _ptr(dindice), dindice.stride(0),
         num_pretokens, 0 if num_tokens is None else int(num_tokens), _ptr(upd), _ptr(abat), _ptr(apos), _ptr(atok),
         _ptr(pmask), _ptr(ridx), _ptr(keep), _ptr(slot), _stream(scores))
    return TopkPlan(upd, abat, apos, atok, pmask, ridx, keep, slot)


@dataclass
class ThresholdPlan(TopkPlan):
    query_valid: torch.Tensor | None = None   # [B, T] bool
    kept_count: torch.Tensor | None = None    # [B] int32


def _check_threshold_scores(scores: torch.Tensor, what: str):
    _require(scores.dtype == torch.float32 and scores.dim() == 2 and (scores.numel() == 0 or scores.stride(1) == 1),
             f"{what}: scores must be [B, P] fp32 with contiguous rows")


def threshold_keep(scores: torch.Tensor, thres: float) -> tuple[torch.Tensor, torch.Tensor]:
    """keep = scores >= thres (fp32 compare, block.py:374-376) and the kept count per image:
    (keep [B, P] bool, kept_count [B] int32)."""
    _require_cuda(scores)
    _check_threshold_scores(scores, "threshold_keep")
    B, Pn = scores.shape
    keep = torch.empty((B, Pn), device=scores.device, dtype=torch.bool)
    cnt = torch.empty((B,), device=scores.device, dtype=torch.int32)
    _launch("threshold_keep", scores, "oudjat_threshold_keep", _ptr(scores), B, Pn, max(scores.stride(0), Pn),
            float(thres), _ptr(keep), _ptr(cnt), _stream(scores))
    return keep, cnt


def threshold_plan(scores: torch.Tensor, thres: float, dindice: torch.Tensor, num_pretokens: int, width: int,
                   padded: bool, num_tokens: int | None = None) -> ThresholdPlan:
    """Threshold selection and its packed plan at `width` patch slots per image (T = pre + width).

    padded=False: the fixed-width builder of token_keep_cap (block.py:492-560) -- slots past an
    image's kept count repeat its last kept candidate (candidate 0 if none), all valid.
    padded=True: the padded builder (block.py:562-621) at width = the largest kept count --
    update_indice holds 0 and query_valid False past the count; the packed rows repeat the image's
    last valid row, so the rows at query_valid are the reference's compacted active rows.
    """
    _require_cuda(scores, dindice)
    _check_threshold_scores(scores, "threshold_plan")
    _require(dindice.dtype == torch.long and dindice.dim() == 2 and dindice.stride(1) == 1,
             "threshold_plan: dindice must be [B, pre + P] int64 with contiguous rows")
    B, Pn = scores.shape
    _require(dindice.shape[0] == B and dindice.shape[1] == num_pretokens + Pn, "threshold_plan: dindice shape mismatch")
    width = int(width)
    _require(0 <= width <= Pn, f"threshold_plan: width={width} outside [0, {Pn}]")
    T = num_pretokens + width
    dev = scores.device
    upd = torch.empty((B, T), device=dev, dtype=torch.long)
    abat = torch.empty((B * T,), device=dev, dtype=torch.long)
    apos = torch.empty_like(abat)
    atok = torch.empty_like(abat)
    pmask = torch.empty((B * T,), device=dev, dtype=torch.bool)
    ridx = torch.empty_like(abat)
    qvalid = torch.empty((B, T), device=dev, dtype=torch.bool)
    keep = torch.empty((B, Pn), device=dev, dtype=torch.bool)
    cnt = torch.empty((B,), device=dev, dtype=torch.int32)
    slot = None
    if num_tokens is not None:
        slot = torch.empty((B, int(num_tokens)), device=dev, dtype=torch.int32)
    _launch("threshold_plan", scores, "oudjat_threshold_plan", _ptr(scores), B, Pn, max(scores.stride(0), Pn),
            float(thres), width, 1 if padded else 0, _ptr(dindice), dindice.stride(0), num_pretokens,
            0 if num_tokens is None else int(num_tokens), _ptr(upd), _ptr(abat), _ptr(apos), _ptr(atok), _ptr(pmask),
            _ptr(ridx), _ptr(qvalid), _ptr(keep), _ptr(cnt), _ptr(slot), _stream(scores))
    return ThresholdPlan(upd, abat, apos, atok, pmask, ridx, keep, slot, qvalid, cnt)


def plan_stats(scores: torch.Tensor, keep: torch.Tensor) -> torch.Tensor:
    """The plan's statistics in one launch (block.py:762-788): fp32 [5] = (sum(scores * keep),
    sum(scores), sum(keep), B * P, B) for scores [B, P] fp32 and the bool keep mask [B, P]."""
    _require_cuda(scores, keep)
    _require(scores.dtype == torch.float32 and scores.dim() == 2 and (scores.numel() == 0 or scores.stride(1) == 1),
             "plan_stats: scores must be [B, P] fp32 with contiguous rows")
    _require(keep.dtype == torch.bool and keep.shape == scores.shape and keep.is_contiguous(),
             "plan_stats: keep must be a contiguous bool mask shaped like scores")
    B, Pn = scores.shape
    out = torch.empty((5,), device=scores.device, dtype=torch.float32)
    _launch("plan_stats", scores, "oudjat_plan_stats", _ptr(scores), B, Pn, max(scores.stride(0), Pn), _ptr(keep),
            _ptr(out), _stream(scores))
    return out


def patch_importance(delta: torch.Tensor, mode: int = _lib.IMPORTANCE_L2) -> torch.Tensor:
    """Per-row reduction of a residual delta [..., D] fp32: L2 norm, energy or RMS -> [...]."""
    _require_cuda(delta)
    _require(delta.dtype == torch.float32 and delta.stride(-1) == 1, "patch_importance: fp32, contiguous rows")
    d2 = delta.reshape(-1, delta.shape[-1])
    out = torch.empty(d2.shape[0], device=delta.device, dtype=torch.float32)
    _launch("importance", delta, "oudjat_patch_importance", _ptr(d2), d2.shape[0], d2.shape[1], d2.stride(0), int(mode), _ptr(out),
         _stream(delta))
    return out.view(delta.shape[:-1])


_PIXEL_DTYPES = {torch.uint8: 0, torch.int16: 1, torch.float32: 2}


def patch_residual_score(curr: torch.Tensor, prev: torch.Tensor | None, patch: tuple[int, int],
                         mode: int = _lib.IMPORTANCE_RMS, image_idx: torch.Tensor | None = None) -> torch.Tensor:
    """Per-patch score of the pixel residual curr - prev of HWC images [B, H, W, C] (uint8, int16 or
    fp32; prev None: curr already is the residual) -> [n, (H/ph) * (W/pw)] fp32, n = len(image_idx) or B.
    RMS is dinov3_classifier.py:91-122; RMS / ENERGY of one residual crop is progressive.py:14-22."""
    _require_cuda(curr, prev, image_idx)
    _require(curr.dim() == 4 and curr.is_contiguous() and curr.dtype in _PIXEL_DTYPES,
             "patch_residual_score: curr must be a contiguous [B, H, W, C] uint8 / int16 / fp32 tensor")
    _require(prev is None or (prev.shape == curr.shape and prev.dtype == curr.dtype and prev.is_contiguous()),
             "patch_residual_score: prev must match curr")
    _require(image_idx is None or (image_idx.dtype == torch.long and image_idx.dim() == 1 and image_idx.is_contiguous()),
             "patch_residual_score: image_idx must be a contiguous int64 vector")
    B, H, W, C = curr.shape
    ph, pw = patch
    n = B if image_idx is None else image_idx.numel()
    out = torch.empty((n, (H // ph) * (W // pw)), device=curr.device, dtype=torch.float32)
    _launch("residual_score", curr, "oudjat_patch_residual_score", _ptr(curr), _ptr(prev), _PIXEL_DTYPES[curr.dtype],
            B, _ptr(image_idx), n, H, W, C, ph, pw, int(mode), _ptr(out), _stream(curr))
    return out


@dataclass
class ResidualPruneKeep:
    keep: torch.Tensor          # [B, P] bool
    kept_count: torch.Tensor    # [B] int32
    kept_mass: torch.Tensor     # [B] fp32
    full_mass: torch.Tensor     # [B] fp32


def residual_prune_keep(rms: torch.Tensor, spatial: torch.Tensor, threshold: float, min_keep: int) -> ResidualPruneKeep:
    """The kept set of image-residual token pruning (dinov3_classifier.py:143-160): keep a candidate
    whose residual RMS reaches `threshold` or that is among the `min_keep` largest of its image."""
    _require_cuda(rms, spatial)
    _require(rms.dtype == torch.float32 and rms.dim() == 2 and rms.stride(1) == 1, "residual_prune_keep: rms [B, G] fp32")
    _require(spatial.dtype == torch.long and spatial.dim() == 2 and spatial.shape[0] == rms.shape[0]
             and (spatial.numel() == 0 or spatial.stride(1) == 1), "residual_prune_keep: spatial [B, P] int64")
    B, P = spatial.shape
    dev = rms.device
    keep = torch.empty((B, P), device=dev, dtype=torch.bool)
    cnt = torch.empty((B,), device=dev, dtype=torch.int32)
    km = torch.empty((B,), device=dev, dtype=torch.float32)
    fm = torch.empty((B,), device=dev, dtype=torch.float32)
    _launch("residual_prune", rms, "oudjat_residual_prune_keep", _ptr(rms), B, max(rms.stride(0), rms.shape[1]),
            rms.shape[1], _ptr(spatial), max(spatial.stride(0), P), P, float(threshold), int(min_keep), _ptr(keep),
            _ptr(cnt), _ptr(km), _ptr(fm), _stream(rms))
    return ResidualPruneKeep(keep, cnt, km, fm)


def residual_prune_compact(keep: torch.Tensor, spatial: torch.Tensor, dindice: torch.Tensor, num_pretokens: int,
                           width: int) -> tuple[torch.Tensor, torch.Tensor]:
    """(pruned_dindice [B, pre + width], kept_local_idx [B, width]) of dinov3_classifier.py:163-196."""
    _require_cuda(keep, spatial, dindice)
    B, P = spatial.shape
    _require(keep.dtype == torch.bool and keep.shape == (B, P) and keep.is_contiguous(), "residual_prune_compact: keep")
    _require(dindice.dtype == torch.long and dindice.dim() == 2 and dindice.stride(1) == 1 and dindice.shape[0] == B,
             "residual_prune_compact: dindice [B, pre + P] int64")
    _require(0 <= width <= P, f"residual_prune_compact: width {width} outside [0, {P}]")
    pruned = torch.empty((B, num_pretokens + width), device=keep.device, dtype=torch.long)
    local = torch.empty((B, width), device=keep.device, dtype=torch.long)
    _launch("residual_prune", keep, "oudjat_residual_prune_compact", _ptr(keep), B, P, _ptr(spatial),
            max(spatial.stride(0), P), _ptr(dindice), dindice.stride(0), num_pretokens, width, _ptr(pruned),
            _ptr(local), _stream(keep))
    return pruned, local


# ------------------------------------------------------------------------------------------------
# LayerNorm, RoPE, QKV post-processing (block.py:1114,1141; rope.py:186-240; attention.py:415-454)
# ------------------------------------------------------------------------------------------------


def layer_norm(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, eps: float = 1e-5,
               out: torch.Tensor | None = None, nvfp4_scale: torch.Tensor | None = None,
               prefetch: torch.Tensor | None = None) -> torch.Tensor:
    """LayerNorm of bf16 rows (fp32 statistics). With nvfp4_scale (the consuming linear's NVFP4 activation
    scale) the result is instead the NVFP4 operand x_hat of LayerNorm(x), as nvfp4_quantize_dequantize
    would give it on the LayerNorm output.

    prefetch: a contiguous device tensor (a weight read by a later kernel) that the same launch reads
    once, a word per 128-byte line, so that it is in the last-level cache when that kernel runs; the
    output is unchanged (bf16 path only)."""
    _require_cuda(x, weight, bias, prefetch)
    _require(x.dtype == weight.dtype == bias.dtype == torch.bfloat16, "layer_norm: bf16 only")
    ts = _nvfp4_scale(nvfp4_scale, "layer_norm")
    C = x.shape[-1]
    x2 = x.reshape(-1, C)
    _require(x2.stride(1) == 1, "layer_norm: rows must be contiguous")
    if out is None:
        out = torch.empty(x.shape, device=x.device, dtype=x.dtype)
    o2 = out.view(-1, C)
    if ts is None and prefetch is not None:
        _require(prefetch.is_contiguous() and prefetch.device == x.device, "layer_norm: prefetch must be a contiguous "
                 "tensor on the rows' device")
        _launch("layernorm", x, "oudjat_layernorm_rows_prefetch", _ptr(x2), x2.shape[0], C, x2.stride(0),
                _ptr(weight.contiguous()), _ptr(bias.contiguous()), float(eps), _ptr(o2), o2.stride(0),
                _ptr(prefetch), prefetch.numel() * prefetch.element_size(), _stream(x))
    elif ts is None:
        _launch("layernorm", x, "oudjat_layernorm_rows", _ptr(x2), x2.shape[0], C, x2.stride(0),
                _ptr(weight.contiguous()), _ptr(bias.contiguous()), float(eps), _ptr(o2), o2.stride(0), _stream(x))
    else:
        _launch("layernorm", x, "oudjat_layernorm_rows_nvfp4", _ptr(x2), x2.shape[0], C, x2.stride(0),
                _ptr(weight.contiguous()), _ptr(bias.contiguous()), float(eps), _ptr(ts), _ptr(o2), o2.stride(0),
                _stream(x))
    return out


def residual_pair(inc: torch.Tensor, x_attn: torch.Tensor, mlp: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(bf16(inc + mlp), bf16(x_attn + mlp)) of three same-shape bf16 tensors with contiguous rows, in one
    launch: the approximate block's cached blocks_out_sum and its output (block.py:336-347)."""
    _require_cuda(inc, x_attn, mlp)
    _require(inc.shape == x_attn.shape == mlp.shape and inc.dtype == x_attn.dtype == mlp.dtype == torch.bfloat16
             and inc.is_contiguous() and x_attn.is_contiguous() and mlp.is_contiguous(),
             "residual_pair: three contiguous bf16 tensors of one shape")
    C = inc.shape[-1]
    rows = inc.numel() // max(C, 1)
    bos, out = torch.empty_like(inc), torch.empty_like(inc)
    _launch("residual", inc, "oudjat_residual_pair", _ptr(inc), _ptr(x_attn), _ptr(mlp), rows, C, _ptr(bos),
            _ptr(out), _stream(inc))
    return bos, out


def gather_rows_ln(src: torch.Tensor, batch_idx: torch.Tensor, token_idx: torch.Tensor, weight: torch.Tensor,
                   bias: torch.Tensor, eps: float = 1e-5,
                   nvfp4_scale: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """(gather_rows(src, batch_idx, token_idx), layer_norm of those rows) in one launch, bit-identical to
    the two calls; src [B, N, C] bf16 with contiguous rows. With nvfp4_scale the second result is the
    NVFP4 operand x_hat of the LayerNorm, as layer_norm(..., nvfp4_scale=) gives it."""
    _require_cuda(src, batch_idx, token_idx, weight, bias)
    _require(src.dim() == 3 and src.stride(2) == 1 and src.dtype == weight.dtype == bias.dtype == torch.bfloat16,
             "gather_rows_ln: src must be [B, N, C] bf16 with contiguous rows")
    ts = _nvfp4_scale(nvfp4_scale, "gather_rows_ln")
    bi, ti = _index(batch_idx, "batch_idx"), _index(token_idx, "token_idx")
    _require(bi.numel() == ti.numel(), "gather_rows_ln: index length mismatch")
    n, C = bi.numel(), src.shape[2]
    x_out = torch.empty((n, C), device=src.device, dtype=src.dtype)
    ln_out = torch.empty((n, C), device=src.device, dtype=src.dtype)
    if n == 0:
        return x_out, ln_out
    _launch("gather_rows", src, "oudjat_gather_rows_ln", _ptr(src), src.stride(0), src.stride(1), C, _ptr(bi),
            _ptr(ti), n, _ptr(weight.contiguous()), _ptr(bias.contiguous()), float(eps), _ptr(ts), _ptr(x_out),
            _ptr(ln_out), _stream(src))
    return x_out, ln_out


def apply_rope_active_inplace(q_active: torch.Tensor, k_active: torch.Tensor, rope, patch_mask: torch.Tensor,
                              rope_idx: torch.Tensor) -> None:
    """Rotate-half RoPE on [T, H, Dh] q and k views in place, fp32 math; rows with patch_mask False
    are untouched. Same contract as apply_rope_active_inplace_triton (rope.py:186-240)."""
    sin, cos = rope
    _require_cuda(q_active, k_active, patch_mask, rope_idx, sin, cos)
    _require(q_active.dim() == 3 and q_active.shape == k_active.shape, "rope: q/k must be [T, H, D] of one shape")
    _require(q_active.dtype == k_active.dtype == torch.bfloat16, "rope: bf16 q/k only")
    _require(sin.dtype == cos.dtype == torch.float32 and sin.stride(-1) == 1 and cos.stride(-1) == 1
             and sin.stride(0) == cos.stride(0), "rope: fp32 sin/cos tables with matching contiguous rows")
    _require(patch_mask.dim() == 1 and rope_idx.dim() == 1 and patch_mask.is_contiguous() and rope_idx.is_contiguous(),
             "rope: patch_mask and rope_idx must be contiguous 1-D")
    n, H, D = q_active.shape
    _require(patch_mask.shape[0] == n and rope_idx.shape[0] == n, "rope: one mask/idx entry per row")
    _require(q_active.stride(2) == 1 and k_active.stride(2) == 1, "rope: head dim must be contiguous")
    if n == 0 or D == 0:
        return
    call("oudjat_rope_active_inplace", _ptr(q_active), q_active.stride(0), q_active.stride(1), _ptr(k_active),
         k_active.stride(0), k_active.stride(1), _ptr(sin), _ptr(cos), sin.stride(0), _ptr(patch_mask.to(torch.bool)),
         _ptr(rope_idx), n, H, D, _stream(q_active))


def qkv_rope_kv_scatter(qkv: torch.Tensor, rope, patch_mask: torch.Tensor, rope_idx: torch.Tensor,
                        batch_idx: torch.Tensor, token_idx: torch.Tensor, kv_cache: torch.Tensor,
                        q_out: torch.Tensor, scale: float | None = None, bias: torch.Tensor | None = None) -> None:
    """qkv [M, 3, H, Dh] -> RoPE on q/k of patch rows; k, v rows written into kv_cache [B, N, 2, H, Dh]
    in place; q written to q_out [M, H, Dh]. With `scale` (an NVFP4 qkv linear), qkv is that linear's raw
    product and each value first becomes bf16(raw * scale + bias) (scale_bias's arithmetic)."""
    sin, cos = rope
    _require_cuda(qkv, patch_mask, rope_idx, batch_idx, token_idx, kv_cache, q_out, sin, cos, bias)
    if scale is not None:
        M, three, H, Dh = qkv.shape
        _require(bias is None or (bias.dtype == torch.bfloat16 and bias.numel() == 3 * H * Dh),
                 "qkv_rope_kv_scatter: bias must be bf16 [3 H Dh]")
        _require(three == 3 and qkv.is_contiguous() and qkv.dtype == torch.bfloat16, "qkv must be contiguous [M,3,H,Dh]")
        _require(kv_cache.dim() == 5 and kv_cache.shape[2:] == (2, H, Dh) and trailing_is_packed(kv_cache, 2),
                 "kv_cache must be [B, N, 2, H, Dh] with packed rows")
        _require(q_out.is_contiguous() and q_out.shape == (M, H, Dh), "q_out must be contiguous [M, H, Dh]")
        _launch("qkv_post", qkv, "oudjat_qkv_rope_kv_scatter_scaled", _ptr(qkv), M, H, Dh, float(scale),
                _ptr(None if bias is None else bias.contiguous()), _ptr(sin), _ptr(cos), sin.stride(0),
                _ptr(patch_mask), _ptr(rope_idx), _ptr(batch_idx), _ptr(token_idx), _ptr(kv_cache),
                kv_cache.stride(0), kv_cache.stride(1), _ptr(q_out), _stream(qkv))
        return
    M, three, H, Dh = qkv.shape
    _require(three == 3 and qkv.is_contiguous() and qkv.dtype == torch.bfloat16, "qkv must be contiguous [M,3,H,Dh]")
    _require(kv_cache.dim() == 5 and kv_cache.shape[2:] == (2, H, Dh) and trailing_is_packed(kv_cache, 2),
             "kv_cache must be [B, N, 2, H, Dh] with packed rows")
    _require(q_out.is_contiguous() and q_out.shape == (M, H, Dh), "q_out must be contiguous [M, H, Dh]")
    _launch("qkv_post", qkv, "oudjat_qkv_rope_kv_scatter", _ptr(qkv), M, H, Dh, _ptr(sin), _ptr(cos), sin.stride(0), _ptr(patch_mask),
         _ptr(rope_idx), _ptr(batch_idx), _ptr(token_idx), _ptr(kv_cache), kv_cache.stride(0), kv_cache.stride(1),
         _ptr(q_out), _stream(qkv))


def qkv_fusable(H: int, Dh: int) -> bool:
    """Shapes the fused QKV + RoPE + K/V-write GEMM supports (otherwise: linear, then qkv_rope_kv_scatter)."""
    return Dh % 16 == 0 and 128 % Dh == 0 and (H * Dh) % 128 == 0


def linear_qkv_rope_kv(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None, rope,
                       patch_mask: torch.Tensor, rope_idx: torch.Tensor, batch_idx: torch.Tensor,
                       token_idx: torch.Tensor, kv_cache: torch.Tensor, q_out: torch.Tensor,
                       acc_scale: float = 1.0, raw_bf16: bool = False, warm: torch.Tensor | None = None) -> None:
    """One kernel for attention.py:415-454: qkv = x . weight^T + bias, RoPE on q and k of patch rows,
    k and v written into kv_cache [B, N, 2, H, Dh] rows (b, t) in place, q written to q_out [M, H, Dh].
    The qkv tensor itself is never materialised. `acc_scale` multiplies the fp32 accumulator before
    its first rounding (an FP8 GEMM's per-tensor scales). raw_bf16: an NVFP4 linear (x and weight its
    x_hat operands, acc_scale its output scale): qkv = bf16(bf16(x . weight^T) * acc_scale + bias).
    `warm`: a tensor (the weight of a later launch) read into the caches from the CUs the launch leaves
    idle, where it leaves any (a cache hint; the results do not depend on it)."""
    sin, cos = rope
    _require_cuda(x, weight, bias, patch_mask, rope_idx, batch_idx, token_idx, kv_cache, q_out, sin, cos)
    M, Kd = x.shape
    _require(x.dtype == weight.dtype == torch.bfloat16 and x.stride(1) == 1 and weight.stride(1) == 1,
             "linear_qkv_rope_kv: bf16 operands with contiguous rows")
    _require(kv_cache.dim() == 5 and kv_cache.shape[2] == 2 and trailing_is_packed(kv_cache, 2),
             "linear_qkv_rope_kv: kv_cache must be [B, N, 2, H, Dh] with packed rows")
    H, Dh = kv_cache.shape[3], kv_cache.shape[4]
    _require(weight.shape == (3 * H * Dh, Kd), "linear_qkv_rope_kv: weight must be [3 H Dh, K]")
    _require(q_out.is_contiguous() and q_out.shape == (M, H, Dh), "linear_qkv_rope_kv: q_out must be contiguous [M, H, Dh]")
    _require(sin.dtype == cos.dtype == torch.float32 and sin.stride(1) == 1 and cos.stride() == sin.stride(),
             "linear_qkv_rope_kv: fp32 RoPE tables with contiguous rows")
    args = [_ptr(x), M, Kd, x.stride(0), _ptr(weight), weight.stride(0),
            _ptr(None if bias is None else bias.contiguous()), H, Dh, _ptr(sin), _ptr(cos), sin.stride(0),
            _ptr(patch_mask), _ptr(_index(rope_idx, "rope_idx")), _ptr(_index(batch_idx, "batch_idx")),
            _ptr(_index(token_idx, "token_idx")), _ptr(kv_cache), kv_cache.stride(0), kv_cache.stride(1), _ptr(q_out),
            float(acc_scale)]
    if warm is not None and not raw_bf16:
        _require_cuda(warm)
        _require(warm.is_contiguous(), "linear_qkv_rope_kv: warm must be contiguous")
        _launch("qkv", x, "oudjat_linear_qkv_rope_kv_warm", *args, _ptr(warm), warm.numel() * warm.element_size(),
                _stream(x))
        return
    entry = "oudjat_linear_qkv_rope_kv_nvfp4" if raw_bf16 else "oudjat_linear_qkv_rope_kv"
    _launch("qkv", x, entry, *args, _stream(x))


def linear_swiglu_nvfp4(xh: torch.Tensor, w2_hat: torch.Tensor, x1: torch.Tensor, s1: float,
                        b1: torch.Tensor | None, s2: float, b2: torch.Tensor | None, tensor_scale: torch.Tensor,
                        site: str = "w2") -> torch.Tensor:
    """w2's NVFP4 GEMM with the SwiGLU of the pair and w3's activation quantizer in its epilogue: from the
    shared operand xh [M, K], w2's weight x_hat [N, K] and w1's bf16 output x1 [M, N], the NVFP4 operand
    of bf16(silu(x1 s1 + b1) (bf16(xh . w2^T) s2 + b2)) with w3's tensor scale -- swiglu_scaled(x1, s1, b1,
    linear(xh, w2_hat), s2, b2, nvfp4_scale=tensor_scale) in one launch. N % 256 == 0."""
    _require_cuda(xh, w2_hat, x1, b1, b2, tensor_scale)
    M, Kd = xh.shape
    N = w2_hat.shape[0]
    _require(xh.dtype == w2_hat.dtype == x1.dtype == torch.bfloat16 and xh.stride(1) == 1 and w2_hat.stride(1) == 1
             and w2_hat.shape[1] == Kd and x1.shape == (M, N) and x1.stride(1) == 1,
             "linear_swiglu_nvfp4: bf16 xh [M, K], w2_hat [N, K], x1 [M, N] with contiguous rows")
    ts = _nvfp4_scale(tensor_scale, "linear_swiglu_nvfp4")
    out = torch.empty((M, N), device=xh.device, dtype=torch.bfloat16)
    _launch(site, xh, "oudjat_linear_swiglu_nvfp4", _ptr(xh), M, Kd, xh.stride(0), _ptr(w2_hat), N, w2_hat.stride(0),
            _ptr(x1), x1.stride(0), float(s1), _ptr(None if b1 is None else b1.contiguous()), float(s2),
            _ptr(None if b2 is None else b2.contiguous()), _ptr(ts), _ptr(out), out.stride(0), _stream(xh))
    return out


def linear_qkv_rope_kv_fp8(x8: torch.Tensor, w8: torch.Tensor, bias: torch.Tensor | None, rope,
                           patch_mask: torch.Tensor, rope_idx: torch.Tensor, batch_idx: torch.Tensor,
                           token_idx: torch.Tensor, kv_cache: torch.Tensor, q_out: torch.Tensor,
                           acc_scale: float) -> None:
    """linear_qkv_rope_kv on e4m3fn codes (uint8 x8 [M, K], w8 [3 H Dh, K]) on the FP8 MFMA: the FP8 qkv
    linear (fp8_fast_linear.py:174-196) with its scales on the accumulator, then RoPE and the K/V write."""
    sin, cos = rope
    _require_cuda(x8, w8, bias, patch_mask, rope_idx, batch_idx, token_idx, kv_cache, q_out, sin, cos)
    M, Kd = x8.shape
    _require(x8.dtype == w8.dtype == torch.uint8 and x8.stride(1) == 1 and w8.stride(1) == 1,
             "linear_qkv_rope_kv_fp8: e4m3 code (uint8) operands with contiguous rows")
    _require(kv_cache.dim() == 5 and kv_cache.shape[2] == 2 and trailing_is_packed(kv_cache, 2),
             "linear_qkv_rope_kv_fp8: kv_cache must be [B, N, 2, H, Dh] with packed rows")
    H, Dh = kv_cache.shape[3], kv_cache.shape[4]
    _require(w8.shape == (3 * H * Dh, Kd), "linear_qkv_rope_kv_fp8: weight must be [3 H Dh, K]")
    _require(q_out.is_contiguous() and q_out.shape == (M, H, Dh), "linear_qkv_rope_kv_fp8: q_out must be contiguous")
    _require(sin.dtype == cos.dtype == torch.float32 and sin.stride(1) == 1 and cos.stride() == sin.stride(),
             "linear_qkv_rope_kv_fp8: fp32 RoPE tables with contiguous rows")
    _launch("qkv", x8, "oudjat_linear_qkv_rope_kv_fp8", _ptr(x8), M, Kd, x8.stride(0), _ptr(w8), w8.stride(0),
            _ptr(None if bias is None else bias.contiguous()), H, Dh, _ptr(sin), _ptr(cos), sin.stride(0),
            _ptr(patch_mask), _ptr(_index(rope_idx, "rope_idx")), _ptr(_index(batch_idx, "batch_idx")),
            _ptr(_index(token_idx, "token_idx")), _ptr(kv_cache), kv_cache.stride(0), kv_cache.stride(1), _ptr(q_out),
            float(acc_scale), _stream(x8))


# ------------------------------------------------------------------------------------------------
# GEMM and attention
# ------------------------------------------------------------------------------------------------


def fp8_gemm_supported(in_features: int, out_features: int) -> bool:
    """Whether linear_fp8 (the native FP8 MFMA GEMM) takes a weight of this shape: K % 128, N % 256."""
    return in_features % 128 == 0 and out_features % 256 == 0


def linear_fp8(x8: torch.Tensor, w8: torch.Tensor, bias: torch.Tensor | None = None, *, acc_scale: float,
               epilogue: int = _lib.EPI_BIAS, gamma: torch.Tensor | None = None, resid: torch.Tensor | None = None,
               out: torch.Tensor | None = None, site: str = "linear") -> torch.Tensor:
    """bf16 epilogue(acc * acc_scale + bias) with acc = x8 . w8^T over e4m3fn codes (uint8 x8 [.., K],
    w8 [N, K]) on the FP8 MFMA: torch._scaled_mm of FastFP8Linear with its per-tensor scales
    (fp8_fast_linear.py:174-196). Epilogues as `linear` (no GELU)."""
    _require_cuda(x8, w8, bias, gamma, resid, out)
    _require(x8.dtype == w8.dtype == torch.uint8, "linear_fp8: e4m3 code (uint8) operands")
    K = x8.shape[-1]
    N = w8.shape[0]
    _require(w8.shape[1] == K and w8.stride(1) == 1, "linear_fp8: weight must be [N, K] with contiguous rows")
    x2 = x8.reshape(-1, K)
    _require(x2.stride(1) == 1, "linear_fp8: input rows must be contiguous")
    M = x2.shape[0]
    if out is None:
        out = torch.empty((*x8.shape[:-1], N), device=x8.device, dtype=torch.bfloat16)
    o2 = out.view(-1, N)
    r2 = None
    if resid is not None:
        r2 = resid.reshape(-1, N)
        _require(r2.stride(1) == 1 and r2.shape[0] == M, "linear_fp8: resid must be [M, N] with contiguous rows")
    _launch(site, x8, "oudjat_linear_fp8", _ptr(x2), M, K, x2.stride(0), _ptr(w8), N, w8.stride(0),
            _ptr(None if bias is None else bias.contiguous()), int(epilogue),
            _ptr(None if gamma is None else gamma.contiguous()), _ptr(r2), 0 if r2 is None else r2.stride(0), _ptr(o2),
            o2.stride(0), float(acc_scale), _stream(x8))
    return out


def linear_fp8_kernel_name(M: int, N: int, K: int, epilogue: int = _lib.EPI_BIAS) -> str:
    """Demangled name of the kernel `linear_fp8` launches (epilogue 5: linear_qkv_rope_kv_fp8)."""
    buf = ctypes.create_string_buffer(256)
    call("oudjat_linear_fp8_kernel_name", M, N, K, epilogue, buf, len(buf))
    return buf.value.decode()


def linear_kernel_name(M: int, N: int, K: int, epilogue: int = _lib.EPI_BIAS) -> str:
    """Demangled name (as profilers print it) of the kernel `linear` launches for an M x N x K product."""
    buf = ctypes.create_string_buffer(256)
    call("oudjat_linear_kernel_name", M, N, K, epilogue, buf, len(buf))
    return buf.value.decode()


_WS_ELEMS: dict = {}
_STREAM_WS: dict = {}
_RETIRED_WS: dict = {}


def _stream_workspace(x: torch.Tensor, elems: int) -> torch.Tensor:
    """fp32 scratch of one launch sequence (split-K GEMM partials, attention key parts): a buffer per
    (device, stream), grown to the largest need and reused by every launch on that stream (launches
    on one stream run in order, and none keeps data in it past its own launches). A buffer that is
    outgrown stays allocated (listed under its stream in _RETIRED_WS): a HIP graph recorded earlier on
    that stream holds its address, and freeing it would let the allocator hand the memory to a tensor
    that the graph's replays would then overwrite. graphs.capture takes a recorded stream's buffers
    out of both tables (take_stream_workspaces), so each graph owns the scratch its kernels use."""
    skey = (x.device, _lib.stream_of(x))
    buf = _STREAM_WS.get(skey)
    if buf is None or buf.numel() < elems:
        if buf is not None:  # grown geometrically, so few buffers are ever retired
            _RETIRED_WS.setdefault(skey, []).append(buf)
            elems = max(elems, 2 * buf.numel())
        buf = torch.empty(elems, device=x.device, dtype=torch.float32)
        _STREAM_WS[skey] = buf
    return buf


def take_stream_workspaces(device: torch.device, stream: int) -> list:
    """Remove and return every scratch buffer created for launches on `stream` (raw hipStream_t) of
    `device`: the current one and those it outgrew. The caller keeps them alive as long as anything
    recorded on that stream may still run; later launches on the stream get a fresh buffer."""
    skey = (torch.device(device), stream)
    bufs = _RETIRED_WS.pop(skey, [])
    cur = _STREAM_WS.pop(skey, None)
    return bufs + ([cur] if cur is not None else [])


def _gemm_workspace(x: torch.Tensor, M: int, N: int, K: int, epilogue: int) -> torch.Tensor | None:
    """The split-K scratch of one GEMM (None: this shape never splits)."""
    key = ("gemm", M, N, K, epilogue)
    elems = _WS_ELEMS.get(key)
    if elems is None:
        elems = int(_lib.load().oudjat_linear_workspace_elems(M, N, K, epilogue))
        _WS_ELEMS[key] = elems
    return _stream_workspace(x, elems) if elems > 0 else None


def linear(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None, *,
           epilogue: int = _lib.EPI_BIAS, gamma: torch.Tensor | None = None, resid: torch.Tensor | None = None,
           out: torch.Tensor | None = None, site: str = "linear", acc_scale: float = 1.0,
           warm: torch.Tensor | None = None) -> torch.Tensor:
    """bf16 x[..., K] . weight[N, K]^T with a fused epilogue (see include/oudjat.h). `site` names the
    launch for the timing probe ("proj", "fc1", "fc2", "w1", "w2", "w3", ...). `acc_scale` multiplies
    the fp32 accumulator before the epilogue's first rounding (an FP8 GEMM's per-tensor scales); with
    `epilogue | EPI_RAW_BF16` (an NVFP4 linear) the accumulator is rounded to bf16 before it. `warm`: a
    tensor (the weight of a later launch) read into the caches from the CUs the launch leaves idle,
    where it leaves any (a cache hint; the results do not depend on it)."""
    _require_cuda(x, weight, bias, gamma, resid, out)
    _require(x.dtype == weight.dtype == torch.bfloat16, "linear: bf16 only")
    K = x.shape[-1]
    N = weight.shape[0]
    _require(weight.shape[1] == K and weight.stride(1) == 1, "linear: weight must be [N, K] with contiguous rows")
    x2 = x.reshape(-1, K)
    _require(x2.stride(1) == 1, "linear: input rows must be contiguous")
    M = x2.shape[0]
    if out is None:
        out = torch.empty((*x.shape[:-1], N), device=x.device, dtype=torch.bfloat16)
    o2 = out.view(-1, N)
    r2 = None
    if resid is not None:
        r2 = resid.reshape(-1, N)
        _require(r2.stride(1) == 1 and r2.shape[0] == M, "linear: resid must be [M, N] with contiguous rows")
    ws = _gemm_workspace(x, M, N, K, int(epilogue))
    args = [_ptr(x2), M, K, x2.stride(0), _ptr(weight), N, weight.stride(0),
            _ptr(None if bias is None else bias.contiguous()), int(epilogue),
            _ptr(None if gamma is None else gamma.contiguous()), _ptr(r2), 0 if r2 is None else r2.stride(0), _ptr(o2),
            o2.stride(0), float(acc_scale), _ptr(ws), 0 if ws is None else ws.numel()]
    if warm is not None:
        _require_cuda(warm)
        _require(warm.is_contiguous(), "linear: warm must be contiguous")
        _launch(site, x, "oudjat_linear_bf16_warm", *args, _ptr(warm), warm.numel() * warm.element_size(), _stream(x))
    else:
        _launch(site, x, "oudjat_linear_bf16", *args, _stream(x))
    return out


def sparse_query_attention(q: torch.Tensor, kv_cache: torch.Tensor, T: int, scale: float,
                           out: torch.Tensor | None = None, lse: torch.Tensor | None = None) -> torch.Tensor:
    """softmax(q . K^T * scale) . V per image over all cached keys.

    q [B*T, H, Dh] packed (rows b*T + t), kv_cache [B, N, 2, H, Dh] (K post-RoPE), -> [B*T, H*Dh].
    lse: optional contiguous fp32 [B, H, T] that receives each query's row log-sum-exp of the scaled
    scores (what cuDNN's SDPA returns beside its output, attention_pscore.py:136-168)."""
    _require_cuda(q, kv_cache, lse)
    _require(q.dtype == kv_cache.dtype == torch.bfloat16, "attention: bf16 only")
    B, N, two, H, Dh = kv_cache.shape
    _require(two == 2 and kv_cache.stride(4) == 1 and kv_cache.stride(3) == Dh, "attention: kv heads must be packed")
    _require(q.dim() == 3 and q.shape[1:] == (H, Dh) and q.shape[0] == B * T and q.stride(2) == 1
             and q.stride(1) == Dh, "attention: q must be [B*T, H, Dh] with packed heads")
    if out is None:
        out = torch.empty((B * T, H * Dh), device=q.device, dtype=torch.bfloat16)
    if lse is not None:
        _require(lse.dtype == torch.float32 and lse.is_contiguous() and tuple(lse.shape) == (B, H, T),
                 "attention: lse must be contiguous fp32 [B, H, T]")
        _launch("attention", q, "oudjat_sparse_query_attention_lse", _ptr(q), q.stride(0), B, T, H, Dh,
                _ptr(kv_cache), kv_cache.stride(0), kv_cache.stride(1), kv_cache.stride(2), kv_cache.stride(3), N,
                float(scale), _ptr(out), out.stride(0), _ptr(lse), _stream(q))
        return out
    key = ("attention", B, T, H, Dh, N)
    elems = _WS_ELEMS.get(key)
    if elems is None:
        elems = int(_lib.load().oudjat_sparse_query_attention_workspace_elems(B, T, H, Dh, N))
        _WS_ELEMS[key] = elems
    if elems > 0:
        # Few (image, head) pairs: the keys are split over several workgroups per pair and merged.
        ws = _stream_workspace(q, elems)
        _launch("attention", q, "oudjat_sparse_query_attention_ws", _ptr(q), q.stride(0), B, T, H, Dh, _ptr(kv_cache),
                kv_cache.stride(0), kv_cache.stride(1), kv_cache.stride(2), kv_cache.stride(3), N, float(scale),
                _ptr(out), out.stride(0), _ptr(ws), ws.numel(), _stream(q))
        return out
    _launch("attention", q, "oudjat_sparse_query_attention", _ptr(q), q.stride(0), B, T, H, Dh, _ptr(kv_cache), kv_cache.stride(0),
         kv_cache.stride(1), kv_cache.stride(2), kv_cache.stride(3), N, float(scale), _ptr(out), out.stride(0),
         _stream(q))
    return out


def sparse_query_attention_fp8(q: torch.Tensor, kv_cache: torch.Tensor, T: int, scale: float,
                               act_inv_scale: torch.Tensor) -> torch.Tensor:
    """sparse_query_attention's output as the e4m3fn codes (uint8 [B*T, H*Dh]) of FastFP8Linear's
    activation quantizer with the device scalar act_inv_scale (fp32, the bf16 inverse scale), in the
    attention's own store: fp8_quantize(sparse_query_attention(...), act_inv_scale) bit for bit. Dh = 128."""
    _require_cuda(q, kv_cache, act_inv_scale)
    _require(q.dtype == kv_cache.dtype == torch.bfloat16, "attention: bf16 only")
    B, N, two, H, Dh = kv_cache.shape
    _require(two == 2 and kv_cache.stride(4) == 1 and kv_cache.stride(3) == Dh, "attention: kv heads must be packed")
    _require(q.dim() == 3 and q.shape[1:] == (H, Dh) and q.shape[0] == B * T and q.stride(2) == 1
             and q.stride(1) == Dh, "attention: q must be [B*T, H, Dh] with packed heads")
    _require(act_inv_scale.dtype == torch.float32 and act_inv_scale.numel() == 1, "attention: fp32 scalar scale")
    out = torch.empty((B * T, H * Dh), device=q.device, dtype=torch.uint8)
    _launch("attention", q, "oudjat_sparse_query_attention_fp8", _ptr(q), q.stride(0), B, T, H, Dh, _ptr(kv_cache),
            kv_cache.stride(0), kv_cache.stride(1), kv_cache.stride(2), kv_cache.stride(3), N, float(scale),
            _ptr(act_inv_scale), _ptr(out), out.stride(0), _stream(q))
    return out


# ------------------------------------------------------------------------------------------------
# Server scores of the approximate pass (attention.py:246-273)
# ------------------------------------------------------------------------------------------------


def _kv_k_view_ok(kv_cache: torch.Tensor) -> None:
    _require(kv_cache.dim() == 5 and kv_cache.shape[2] == 2 and kv_cache.stride(4) == 1
             and kv_cache.dtype == torch.bfloat16, "pscore: kv_cache must be [B, N, 2, H, Dh] bf16 with packed heads")


def query_attention_prob(q: torch.Tensor, kv_cache: torch.Tensor, scale: float, *, out_dtype=torch.float32,
                         workspace: torch.Tensor | None = None) -> torch.Tensor:
    """mean_h softmax_n(bf16(bf16(q[b, h] . K[b, n, h]) * scale)) with torch's bf16 rounding points ->
    [B, N] (attention.py:267-271 with q = the cls query; :260-261 with the pseudo query).

    q [B, H, Dh] (any strides with a contiguous head dim), kv_cache [B, N, 2, H, Dh] (K after RoPE).
    out_dtype float32 (cls_attn_prob) or bfloat16 (the pseudo score); the values are bf16 either way.
    `workspace` (fp32, >= B*H*N elements) is scratch; one is allocated when not given."""
    _require_cuda(q, kv_cache, workspace)
    _kv_k_view_ok(kv_cache)
    B, N, _, H, Dh = kv_cache.shape
    _require(q.dim() == 3 and q.shape == (B, H, Dh) and q.stride(2) == 1 and q.dtype == torch.bfloat16,
             "query_attention_prob: q must be [B, H, Dh] bf16 with a contiguous head dim")
    _require(out_dtype in (torch.float32, torch.bfloat16), "query_attention_prob: out_dtype fp32 or bf16")
    if workspace is None:
        workspace = torch.empty((B * H * N,), device=q.device, dtype=torch.float32)
    _require(workspace.dtype == torch.float32 and workspace.is_contiguous() and workspace.numel() >= B * H * N,
             "query_attention_prob: workspace must be contiguous fp32 with B*H*N elements")
    out = torch.empty((B, N), device=q.device, dtype=out_dtype)
    _launch("pscore", q, "oudjat_query_attention_prob", _ptr(q), q.stride(0), q.stride(1), B, H, Dh, _ptr(kv_cache),
            kv_cache.stride(0), kv_cache.stride(1), kv_cache.stride(3), N, float(scale), _ptr(workspace), _ptr(out),
            N, int(out_dtype == torch.bfloat16), _stream(q))
    return out


PATTN_DENSE = 0   # patch_attn_prob: torch's bf16 rounding points (attention.py:251-253)
PATTN_LSE = 1     # the fused key-side sum from the row log-sum-exp (attention_pscore.py:20-98)


def patch_attention_prob(q: torch.Tensor, kv_cache: torch.Tensor, scale: float, mode: int = PATTN_DENSE,
                         workspace: torch.Tensor | None = None) -> torch.Tensor:
    """The mean attention probability of every key over heads and all queries -> [B, N] bf16.

    q [B * N, H, Dh] (the approx pass's packed queries after RoPE, contiguous heads), kv_cache
    [B, N, 2, H, Dh] (K after RoPE). `workspace` (fp32, >= oudjat_patch_attention_prob_workspace_elems)
    holds the row statistics and partial column sums; one is allocated when not given."""
    _require_cuda(q, kv_cache, workspace)
    _kv_k_view_ok(kv_cache)
    B, N, _, H, Dh = kv_cache.shape
    _require(q.dim() == 3 and q.shape == (B * N, H, Dh) and q.stride(2) == 1 and q.stride(1) == Dh
             and q.dtype == torch.bfloat16, "patch_attention_prob: q must be [B*N, H, Dh] bf16 with packed heads")
    need = int(_lib.load().oudjat_patch_attention_prob_workspace_elems(B, N, H, int(mode)))
    if workspace is None:
        workspace = torch.empty((need,), device=q.device, dtype=torch.float32)
    _require(workspace.dtype == torch.float32 and workspace.is_contiguous() and workspace.numel() >= need,
             f"patch_attention_prob: workspace must be contiguous fp32 with {need} elements")
    out = torch.empty((B, N), device=q.device, dtype=torch.bfloat16)
    _launch("pscore", q, "oudjat_patch_attention_prob", _ptr(q), q.stride(0), B, N, H, Dh, _ptr(kv_cache),
            kv_cache.stride(0), kv_cache.stride(1), kv_cache.stride(3), float(scale), int(mode), _ptr(workspace),
            _ptr(out), N, _stream(q))
    return out


def patch_attention_prob_from_lse(q: torch.Tensor, kv_cache: torch.Tensor, scale: float,
                                  lse: torch.Tensor, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """PATTN_LSE's key-side score from the attention's own row log-sum-exp (lse [B, H, N] fp32, as
    sparse_query_attention(..., lse=) writes it for T = N): one pass over the scores instead of three
    (attention_pscore.py:172-241 after cuDNN's LSE). Same q / kv_cache contract as
    patch_attention_prob; `workspace` (fp32, >= B*H*N) takes the partial column sums, one is allocated
    when not given."""
    _require_cuda(q, kv_cache, lse, workspace)
    _kv_k_view_ok(kv_cache)
    B, N, _, H, Dh = kv_cache.shape
    _require(q.dim() == 3 and q.shape == (B * N, H, Dh) and q.stride(2) == 1 and q.stride(1) == Dh
             and q.dtype == torch.bfloat16, "patch_attention_prob: q must be [B*N, H, Dh] bf16 with packed heads")
    _require(lse.dtype == torch.float32 and lse.is_contiguous() and tuple(lse.shape) == (B, H, N),
             "patch_attention_prob: lse must be contiguous fp32 [B, H, N]")
    if workspace is None:
        workspace = torch.empty((B * H * N,), device=q.device, dtype=torch.float32)
    _require(workspace.dtype == torch.float32 and workspace.is_contiguous() and workspace.numel() >= B * H * N,
             "patch_attention_prob: workspace must be contiguous fp32 with B*H*N elements")
    out = torch.empty((B, N), device=q.device, dtype=torch.bfloat16)
    _launch("pscore", q, "oudjat_patch_attention_prob_lse", _ptr(q), q.stride(0), B, N, H, Dh, _ptr(kv_cache),
            kv_cache.stride(0), kv_cache.stride(1), kv_cache.stride(3), float(scale), _ptr(lse), _ptr(workspace),
            _ptr(out), N, _stream(q))
    return out


def pseudo_query(q_patch: torch.Tensor) -> torch.Tensor:
    """The pseudo query of patch_pseudo_attn_prob (attention.py:254-259): q_patch [B, P, H, Dh] (patch
    queries after RoPE, any strides with a contiguous head dim) -> [B, H, Dh] bf16."""
    _require_cuda(q_patch)
    _require(q_patch.dim() == 4 and q_patch.dtype == torch.bfloat16 and q_patch.stride(3) == 1,
             "pseudo_query: q_patch must be [B, P, H, Dh] bf16 with a contiguous head dim")
    B, P, H, Dh = q_patch.shape
    out = torch.empty((B, H, Dh), device=q_patch.device, dtype=torch.bfloat16)
    _launch("pscore", q_patch, "oudjat_pseudo_query", _ptr(q_patch), q_patch.stride(0), q_patch.stride(1),
            q_patch.stride(2), B, P, H, Dh, _ptr(out), _stream(q_patch))
    return out


# ------------------------------------------------------------------------------------------------
# NVFP4 (nvfp4_fused.py:119-145; fp4_fast_linear.py:221-283)
# ------------------------------------------------------------------------------------------------


def nvfp4_scale_numel(M: int, K: int) -> int:
    return -(-M // 128) * -(-K // 64) * 512


def quantize_nvfp4_swizzled(x: torch.Tensor, tensor_scale: torch.Tensor):
    """x [M, K] bf16 -> (qdata uint8 [M, K/2], swizzled e4m3 block scales float8_e4m3fn [tiles*512])."""
    _require_cuda(x, tensor_scale)
    _require(x.dim() == 2 and x.dtype == torch.bfloat16 and x.stride(1) == 1, "nvfp4: x must be [M, K] bf16 rows")
    M, K = x.shape
    _require(K % 16 == 0, f"nvfp4: K must be a multiple of the 16-element block, got {K}")
    ts = tensor_scale.reshape(1).to(torch.float32)
    qdata = torch.empty((M, K // 2), device=x.device, dtype=torch.uint8)
    scale = torch.empty((nvfp4_scale_numel(M, K),), device=x.device, dtype=torch.uint8)
    _launch("nvfp4_quantize", x, "oudjat_nvfp4_quantize", _ptr(x), M, K, x.stride(0), _ptr(ts), _ptr(qdata), _ptr(scale), _stream(x))
    return qdata, scale.view(torch.float8_e4m3fn)


def dequantize_nvfp4(qdata: torch.Tensor, scale: torch.Tensor, tensor_scale: torch.Tensor) -> torch.Tensor:
    """Inverse of quantize_nvfp4_swizzled: bf16 [M, K]."""
    _require_cuda(qdata, scale, tensor_scale)
    M, K2 = qdata.shape
    K = 2 * K2
    _require(qdata.dtype == torch.uint8 and qdata.is_contiguous(), "nvfp4: qdata must be contiguous uint8")
    s = scale.reshape(-1).view(torch.uint8)
    _require(s.numel() == nvfp4_scale_numel(M, K), "nvfp4: scale buffer size mismatch")
    ts = tensor_scale.reshape(1).to(torch.float32)
    out = torch.empty((M, K), device=qdata.device, dtype=torch.bfloat16)
    _launch("nvfp4_dequantize", qdata, "oudjat_nvfp4_dequantize", _ptr(qdata), _ptr(s), _ptr(ts), M, K, _ptr(out), out.stride(0), _stream(qdata))
    return out


def _rows_bf16(x: torch.Tensor, what: str) -> torch.Tensor:
    _require(x.dtype == torch.bfloat16 and x.stride(-1) == 1, f"{what}: bf16 with contiguous rows required")
    x2 = x.reshape(-1, x.shape[-1])
    _require(x2.stride(1) == 1, f"{what}: rows must be contiguous")
    return x2


def nvfp4_quantize_dequantize(x: torch.Tensor, tensor_scale: torch.Tensor, *, packed: bool = False):
    """The NVFP4 operand of an FP4 linear (fp4_fast_linear.py:171-219): xhat = e2m1(q) * e4m3(s), the
    block-scaled values without the tensor scale, as bf16 [.., K] (exact). With packed=True also
    returns the reference's (qdata, scales) bytes: (xhat, qdata, scales)."""
    _require_cuda(x, tensor_scale)
    x2 = _rows_bf16(x, "nvfp4_quantize_dequantize")
    M, K = x2.shape
    _require(K % 16 == 0, f"nvfp4: K must be a multiple of the 16-element block, got {K}")
    ts = tensor_scale.reshape(1).to(torch.float32)
    xhat = torch.empty(x.shape, device=x.device, dtype=torch.bfloat16)
    q = s = None
    if packed:
        q = torch.empty((M, K // 2), device=x.device, dtype=torch.uint8)
        s = torch.empty((nvfp4_scale_numel(M, K),), device=x.device, dtype=torch.uint8)
    _launch("nvfp4_qdq", x, "oudjat_nvfp4_quantize_dequantize", _ptr(x2), M, K, x2.stride(0), _ptr(ts), _ptr(q),
            _ptr(s), _ptr(xhat), K, _stream(x))
    return (xhat, q, s.view(torch.float8_e4m3fn)) if packed else xhat


FP8_ACTIVATION = 0   # e4m3(clamp(x * inv_scale)), fp32 product (the compiled activation quantizer)
FP8_WEIGHT = 1       # e4m3(clamp(bf16(x / bf16(scale))))      (the eager weight quantizer)


def fp8_quantize_dequantize(x: torch.Tensor, scale: torch.Tensor, mode: int = FP8_ACTIVATION) -> torch.Tensor:
    """FastFP8Linear's e4m3 operand as its exact bf16 value (fp8_fast_linear.py:71-73, 123-125).
    `scale`: a device scalar -- the bf16 inverse scale for FP8_ACTIVATION, the fp32 scale for FP8_WEIGHT."""
    _require_cuda(x, scale)
    x2 = _rows_bf16(x, "fp8_quantize_dequantize")
    M, K = x2.shape
    s = scale.reshape(1).to(torch.float32)
    out = torch.empty(x.shape, device=x.device, dtype=torch.bfloat16)
    _launch("fp8_qdq", x, "oudjat_fp8_quantize_dequantize", _ptr(x2), M, K, x2.stride(0), _ptr(s), int(mode), _ptr(out),
            K, _stream(x))
    return out


def fp8_quantize(x: torch.Tensor, scale: torch.Tensor, mode: int = FP8_ACTIVATION) -> torch.Tensor:
    """FastFP8Linear's e4m3 operand as its e4m3fn codes, uint8 [.., K] (the same quantizer as
    fp8_quantize_dequantize). `scale`: an fp32 device scalar (the bf16 inverse scale's value for
    FP8_ACTIVATION, the fp32 scale for FP8_WEIGHT)."""
    _require_cuda(x, scale)
    _require(scale.dtype == torch.float32 and scale.numel() == 1, "fp8_quantize: scale must be one fp32 value")
    x2 = _rows_bf16(x, "fp8_quantize")
    M, K = x2.shape
    out = torch.empty(x.shape, device=x.device, dtype=torch.uint8)
    _launch("fp8_q", x, "oudjat_fp8_quantize", _ptr(x2), M, K, x2.stride(0), _ptr(scale), int(mode), _ptr(out), K,
            _stream(x))
    return out


def scale_bias(x: torch.Tensor, scale: float, bias: torch.Tensor | None = None, gamma: torch.Tensor | None = None,
               out: torch.Tensor | None = None) -> torch.Tensor:
    """bf16(x * scale + bias), then bf16(. * gamma) when gamma is given (scale_bias_inplace_triton,
    token_update.py:571-617, and the LayerScale after it). `out` may be x (in place)."""
    _require_cuda(x, bias, gamma, out)
    x2 = _rows_bf16(x, "scale_bias")
    M, N = x2.shape
    for t, nm in ((bias, "bias"), (gamma, "gamma")):
        _require(t is None or (t.dtype == torch.bfloat16 and t.numel() == N), f"scale_bias: {nm} must be bf16 [N]")
    if out is None:
        out = torch.empty(x.shape, device=x.device, dtype=torch.bfloat16)
    o2 = out.reshape(-1, N)
    _launch("scale_bias", x, "oudjat_scale_bias_rows", _ptr(x2), M, N, x2.stride(0), float(scale),
            _ptr(None if bias is None else bias.contiguous()), _ptr(None if gamma is None else gamma.contiguous()),
            _ptr(o2), o2.stride(0), _stream(x))
    return out


def swiglu_scaled(x1: torch.Tensor, s1: float, b1: torch.Tensor | None, x2: torch.Tensor, s2: float,
                  b2: torch.Tensor | None, nvfp4_scale: torch.Tensor | None = None) -> torch.Tensor:
    """silu(x1 * s1 + b1) * (x2 * s2 + b2) -> bf16, written into x1 (fused_swiglu_epilogue_triton,
    token_update.py:620-669). With nvfp4_scale (the NVFP4 w3 linear's activation scale) x1 receives
    instead the NVFP4 operand x_hat of that output."""
    _require_cuda(x1, x2, b1, b2)
    _require(x1.shape == x2.shape and x1.is_contiguous() and x2.is_contiguous() and x1.dtype == x2.dtype == torch.bfloat16,
             "swiglu_scaled: contiguous bf16 tensors of one shape")
    _require((b1 is None) == (b2 is None), "swiglu_scaled: both biases or neither")
    ts = _nvfp4_scale(nvfp4_scale, "swiglu_scaled")
    N = x1.shape[-1]
    M = x1.numel() // N if N else 0
    args = (_ptr(x1), float(s1), _ptr(None if b1 is None else b1.contiguous()), _ptr(x2), float(s2),
            _ptr(None if b2 is None else b2.contiguous()), M, N)
    if ts is None:
        _launch("swiglu", x1, "oudjat_swiglu_scaled", *args, _ptr(x1), _stream(x1))
    else:
        _launch("swiglu", x1, "oudjat_swiglu_scaled_nvfp4", *args, _ptr(ts), _ptr(x1), _stream(x1))
    return x1


def amax_update(x: torch.Tensor, amax: torch.Tensor) -> None:
    """amax = max(amax, max |x|) in place (a device fp32 scalar; NaN propagates)."""
    _require_cuda(x, amax)
    _require(amax.dtype == torch.float32 and amax.numel() == 1 and amax.is_contiguous(), "amax_update: fp32 scalar")
    x2 = _rows_bf16(x, "amax_update")
    call("oudjat_amax_update", _ptr(x2), x2.shape[0], x2.shape[1], x2.stride(0), _ptr(amax), _stream(x))


# Reference spellings, for call sites written against the Triton wrappers.
gather_rows_triton = gather_rows
scatter_rows_triton = scatter_rows
active_token_update_triton = active_token_update
apply_rope_active_inplace_triton = apply_rope_active_inplace
