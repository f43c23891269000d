"""The no-alloc server-score entry point (oudjat_query_attention_prob_noalloc) against the entry point
that takes a workspace, through the C ABI: bit-identical results on two calls in a row, the second
smaller than the first (the library's scratch array keeps the first call's contents), and sizes
beyond the array rejected before any launch."""

import ctypes

import pytest
import torch

from appcorr_amd import _lib
from appcorr_amd import kernels as K

pytestmark = pytest.mark.gpu

P = ctypes.c_void_p


def _noalloc(q, kv, scale, out_dtype=torch.float32):
    B, N, _, H, Dh = kv.shape
    out = torch.empty((B, N), device=q.device, dtype=out_dtype)
    _lib.call("oudjat_query_attention_prob_noalloc", P(q.data_ptr()), q.stride(0), q.stride(1), B, H, Dh,
              P(kv.data_ptr()), kv.stride(0), kv.stride(1), kv.stride(3), N, float(scale), P(out.data_ptr()), N,
              int(out_dtype == torch.bfloat16), P(torch.cuda.current_stream(q.device).cuda_stream))
    return out


def _case(B, H, N, Dh, seed, dev):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(B, N, H, Dh, generator=g) * 2.0).to(torch.bfloat16).to(dev)
    kv = torch.randn(B, N, 2, H, Dh, generator=g).to(torch.bfloat16).to(dev)
    return q, kv


def test_noalloc_equals_workspace_entry_point(dev):
    for (B, H, N, Dh, dt) in [(4, 32, 4101, 128, torch.float32), (2, 16, 1029, 64, torch.bfloat16)]:
        print(f"noalloc B={B} H={H} N={N} Dh={Dh} {dt}", flush=True)
        assert B * H * N <= _lib.QUERY_PROB_NOALLOC_MAX
        q, kv = _case(B, H, N, Dh, N, dev)
        want = K.query_attention_prob(q[:, 0], kv, Dh ** -0.5, out_dtype=dt)
        got = _noalloc(q[:, 0], kv, Dh ** -0.5, dt)
        torch.cuda.synchronize()
        assert got.dtype == want.dtype and torch.equal(got.view(torch.int16) if dt == torch.bfloat16 else got,
                                                       want.view(torch.int16) if dt == torch.bfloat16 else want)


def test_noalloc_rejects_sizes_beyond_the_scratch_array(dev):
    B, H, N, Dh = 16, 32, 4101, 128     # 2.1M > 1M elements: refused on the host, nothing launched
    q = torch.zeros(B, H, Dh, device=dev, dtype=torch.bfloat16)
    kv = torch.zeros(1, 1, 2, H, Dh, device=dev, dtype=torch.bfloat16).expand(B, N, 2, H, Dh)
    with pytest.raises(_lib.OudjatKernelError) as ei:
        _noalloc(q, kv, Dh ** -0.5)
    assert ei.value.status_name == "OUDJAT_ERR_TOO_LARGE"
