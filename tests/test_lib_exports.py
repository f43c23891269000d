"""CPU checks of the C ABI: the library loads, exports every symbol include/oudjat.h declares, and
rejects bad arguments with the documented status before any launch (so these run without a GPU)."""

import ctypes
import re
from pathlib import Path

import pytest

from appcorr_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "oudjat.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(oudjat_[a-z0-9_]+)\s*\(", text)))


def test_library_loads_and_abi_version():
    lib = _lib.load()
    assert lib.oudjat_abi_version() == _lib.ABI_VERSION


def test_every_declared_symbol_is_exported_and_bound():
    lib = _lib.load()
    decl = declared_functions()
    assert len(decl) >= 18
    for name in decl:
        assert hasattr(lib, name), f"{name} declared in oudjat.h but not exported"
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature in appcorr_amd._lib"
    assert set(_lib.SIGNATURES) == set(decl)


def test_status_strings():
    lib = _lib.load()
    for code in range(7):
        assert lib.oudjat_status_string(code)
    assert lib.oudjat_status_string(0) == b"ok"


NULL = ctypes.c_void_p(0)


def _expect(status_name, fn, *args):
    with pytest.raises(_lib.OudjatKernelError) as ei:
        _lib.call(fn, *args)
    assert ei.value.status_name == status_name, str(ei.value)


def test_linear_rejects_bad_shapes_before_launch():
    # K not a multiple of 64
    _expect("OUDJAT_ERR_UNSUPPORTED_SHAPE", "oudjat_linear_bf16", ctypes.c_void_p(16), 4, 100, 100,
            ctypes.c_void_p(16), 64, 100, NULL, 0, NULL, NULL, 0, ctypes.c_void_p(16), 64, 1.0, NULL, 0, NULL)
    # bad epilogue id
    _expect("OUDJAT_ERR_INVALID_ARGUMENT", "oudjat_linear_bf16", NULL, 4, 64, 64, NULL, 64, 64, NULL, 9, NULL, NULL, 0,
            NULL, 64, 1.0, NULL, 0, NULL)
    # LayerScale epilogue without gamma
    _expect("OUDJAT_ERR_INVALID_ARGUMENT", "oudjat_linear_bf16", ctypes.c_void_p(16), 4, 64, 64, ctypes.c_void_p(16),
            64, 64, NULL, 3, NULL, NULL, 0, ctypes.c_void_p(16), 64, 1.0, NULL, 0, NULL)
    # misaligned A
    _expect("OUDJAT_ERR_UNSUPPORTED_LAYOUT", "oudjat_linear_bf16", ctypes.c_void_p(18), 4, 64, 64,
            ctypes.c_void_p(16), 64, 64, NULL, 0, NULL, NULL, 0, ctypes.c_void_p(16), 64, 1.0, NULL, 0, NULL)
    # the raw-bf16 flag does not combine with GELU; it needs a 16-byte aligned bias
    _expect("OUDJAT_ERR_INVALID_ARGUMENT", "oudjat_linear_bf16", ctypes.c_void_p(16), 4, 64, 64, ctypes.c_void_p(16),
            64, 64, NULL, _lib.EPI_BIAS_GELU | _lib.EPI_RAW_BF16, NULL, NULL, 0, ctypes.c_void_p(16), 64, 1.0, NULL,
            0, NULL)
    _expect("OUDJAT_ERR_UNSUPPORTED_LAYOUT", "oudjat_linear_bf16", ctypes.c_void_p(16), 4, 64, 64, ctypes.c_void_p(16),
            64, 64, ctypes.c_void_p(24), _lib.EPI_BIAS | _lib.EPI_RAW_BF16, NULL, NULL, 0, ctypes.c_void_p(16), 64, 1.0,
            NULL, 0, NULL)


def test_swiglu_nvfp4_gemm_rejects_bad_arguments():
    # N not a multiple of 256; one bias only
    _expect("OUDJAT_ERR_UNSUPPORTED_SHAPE", "oudjat_linear_swiglu_nvfp4", ctypes.c_void_p(16), 4, 64, 64,
            ctypes.c_void_p(16), 128, 64, ctypes.c_void_p(16), 128, 1.0, NULL, 1.0, NULL, ctypes.c_void_p(16),
            ctypes.c_void_p(16), 128, NULL)
    _expect("OUDJAT_ERR_INVALID_ARGUMENT", "oudjat_linear_swiglu_nvfp4", ctypes.c_void_p(16), 4, 64, 64,
            ctypes.c_void_p(16), 256, 64, ctypes.c_void_p(16), 256, 1.0, ctypes.c_void_p(16), 1.0, NULL,
            ctypes.c_void_p(16), ctypes.c_void_p(16), 256, NULL)


def test_low_precision_entry_points_reject_bad_arguments():
    # row length not a multiple of 8 / 16, a bad mode, one of qdata / scales only
    _expect("OUDJAT_ERR_UNSUPPORTED_SHAPE", "oudjat_fp8_quantize_dequantize", ctypes.c_void_p(16), 4, 12, 16,
            ctypes.c_void_p(16), 0, ctypes.c_void_p(16), 16, NULL)
    _expect("OUDJAT_ERR_INVALID_ARGUMENT", "oudjat_fp8_quantize_dequantize", ctypes.c_void_p(16), 4, 16, 16,
            ctypes.c_void_p(16), 2, ctypes.c_void_p(16), 16, NULL)
    _expect("OUDJAT_ERR_UNSUPPORTED_SHAPE", "oudjat_nvfp4_quantize_dequantize", ctypes.c_void_p(16), 4, 24, 24,
            ctypes.c_void_p(16), NULL, NULL, ctypes.c_void_p(16), 24, NULL)
    _expect("OUDJAT_ERR_INVALID_ARGUMENT", "oudjat_nvfp4_quantize_dequantize", ctypes.c_void_p(16), 4, 32, 32,
            ctypes.c_void_p(16), ctypes.c_void_p(16), NULL, ctypes.c_void_p(16), 32, NULL)
    _expect("OUDJAT_ERR_INVALID_ARGUMENT", "oudjat_swiglu_scaled", ctypes.c_void_p(16), 1.0, ctypes.c_void_p(16),
            ctypes.c_void_p(16), 1.0, NULL, 4, 64, ctypes.c_void_p(16), NULL)
    _expect("OUDJAT_ERR_UNSUPPORTED_LAYOUT", "oudjat_scale_bias_rows", ctypes.c_void_p(18), 4, 64, 64, 1.0, NULL, NULL,
            ctypes.c_void_p(16), 64, NULL)


def test_topk_plan_rejects_bad_k_and_too_large():
    args = [NULL] * 10
    _expect("OUDJAT_ERR_INVALID_ARGUMENT", "oudjat_topk_plan", NULL, 2, 10, 10, 11, NULL, 15, 5, 15, *args[:9])
    _expect("OUDJAT_ERR_TOO_LARGE", "oudjat_topk_plan", ctypes.c_void_p(16), 1, 20000, 20000, 5,
            ctypes.c_void_p(16), 20005, 5, 0, *([ctypes.c_void_p(16)] * 6), NULL, NULL, NULL)


def test_nvfp4_rejects_k_not_multiple_of_16():
    _expect("OUDJAT_ERR_UNSUPPORTED_SHAPE", "oudjat_nvfp4_quantize", NULL, 4, 24, 24, NULL, NULL, NULL, NULL)
    _expect("OUDJAT_ERR_UNSUPPORTED_SHAPE", "oudjat_nvfp4_dequantize", NULL, NULL, NULL, 4, 24, NULL, 24, NULL)


def test_attention_rejects_unsupported_head_dim():
    _expect("OUDJAT_ERR_UNSUPPORTED_SHAPE", "oudjat_sparse_query_attention", ctypes.c_void_p(16), 96, 1, 4, 1, 96,
            ctypes.c_void_p(16), 0, 0, 0, 0, 8, 0.1, ctypes.c_void_p(16), 96, NULL)
    _expect("OUDJAT_ERR_UNSUPPORTED_SHAPE", "oudjat_sparse_query_attention_lse", ctypes.c_void_p(16), 96, 1, 4, 1,
            96, ctypes.c_void_p(16), 0, 0, 0, 0, 8, 0.1, ctypes.c_void_p(16), 96, ctypes.c_void_p(16), NULL)


def test_lse_entry_points_reject_bad_arguments():
    # no lse buffer for a non-empty call
    _expect("OUDJAT_ERR_INVALID_ARGUMENT", "oudjat_sparse_query_attention_lse", ctypes.c_void_p(16), 128, 1, 4, 1,
            128, ctypes.c_void_p(16), 0, 0, 0, 0, 8, 0.1, ctypes.c_void_p(16), 128, NULL, NULL)
    # misaligned lse
    _expect("OUDJAT_ERR_UNSUPPORTED_LAYOUT", "oudjat_sparse_query_attention_lse", ctypes.c_void_p(16), 128, 1, 4, 1,
            128, ctypes.c_void_p(16), 2048, 256, 128, 128, 8, 0.1, ctypes.c_void_p(16), 128, ctypes.c_void_p(18), NULL)
    _expect("OUDJAT_ERR_UNSUPPORTED_SHAPE", "oudjat_patch_attention_prob_lse", ctypes.c_void_p(16), 96, 1, 8, 1, 96,
            ctypes.c_void_p(16), 0, 0, 96, 0.1, ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16), 8, NULL)
    _expect("OUDJAT_ERR_INVALID_ARGUMENT", "oudjat_patch_attention_prob_lse", ctypes.c_void_p(16), 128, 1, 8, 1, 128,
            ctypes.c_void_p(16), 0, 0, 128, 0.1, NULL, ctypes.c_void_p(16), ctypes.c_void_p(16), 8, NULL)
    _expect("OUDJAT_ERR_INVALID_ARGUMENT", "oudjat_patch_attention_prob_lse", ctypes.c_void_p(16), 128, 1, 8, 1, 128,
            ctypes.c_void_p(16), 0, 0, 128, 0.1, ctypes.c_void_p(16), NULL, ctypes.c_void_p(16), 8, NULL)
    # zero-sized calls touch nothing
    _lib.call("oudjat_sparse_query_attention_lse", NULL, 128, 0, 4, 1, 128, NULL, 0, 0, 0, 0, 8, 0.1, NULL, 128,
              NULL, NULL)
    _lib.call("oudjat_patch_attention_prob_lse", NULL, 128, 0, 8, 1, 128, NULL, 0, 0, 128, 0.1, NULL, NULL, NULL, 8,
              NULL)


def test_attention_fp8_rejects_bad_arguments():
    # Dh = 64 has no FP8-output kernel; a null scale; a misaligned output row stride
    _expect("OUDJAT_ERR_UNSUPPORTED_SHAPE", "oudjat_sparse_query_attention_fp8", ctypes.c_void_p(16), 64, 1, 4, 1, 64,
            ctypes.c_void_p(16), 1024, 128, 64, 64, 8, 0.1, ctypes.c_void_p(16), ctypes.c_void_p(16), 64, NULL)
    _expect("OUDJAT_ERR_INVALID_ARGUMENT", "oudjat_sparse_query_attention_fp8", ctypes.c_void_p(16), 128, 1, 4, 1,
            128, ctypes.c_void_p(16), 2048, 256, 128, 128, 8, 0.1, NULL, ctypes.c_void_p(16), 128, NULL)
    _expect("OUDJAT_ERR_UNSUPPORTED_LAYOUT", "oudjat_sparse_query_attention_fp8", ctypes.c_void_p(16), 128, 1, 4, 1,
            128, ctypes.c_void_p(16), 2048, 256, 128, 128, 8, 0.1, ctypes.c_void_p(16), ctypes.c_void_p(16), 130, NULL)
    _lib.call("oudjat_sparse_query_attention_fp8", NULL, 128, 0, 4, 1, 128, NULL, 0, 0, 0, 0, 8, 0.1, NULL, NULL,
              128, NULL)


def test_layernorm_prefetch_rejects_bad_regions():
    """The cache-warming region is checked before anything else (here with zero rows, so no GPU)."""
    _expect("OUDJAT_ERR_INVALID_ARGUMENT", "oudjat_layernorm_rows_prefetch", NULL, 0, 1024, 1024, NULL, NULL, 1e-5,
            NULL, 1024, NULL, 4096, NULL)
    _expect("OUDJAT_ERR_INVALID_ARGUMENT", "oudjat_layernorm_rows_prefetch", NULL, 0, 1024, 1024, NULL, NULL, 1e-5,
            NULL, 1024, ctypes.c_void_p(256), -128, NULL)
    _expect("OUDJAT_ERR_UNSUPPORTED_LAYOUT", "oudjat_layernorm_rows_prefetch", NULL, 0, 1024, 1024, NULL, NULL, 1e-5,
            NULL, 1024, ctypes.c_void_p(258), 4096, NULL)
    _lib.call("oudjat_layernorm_rows_prefetch", NULL, 0, 1024, 1024, NULL, NULL, 1e-5, NULL, 1024,
              ctypes.c_void_p(256), 4096, NULL)
    _lib.call("oudjat_layernorm_rows_prefetch", NULL, 0, 1024, 1024, NULL, NULL, 1e-5, NULL, 1024, NULL, 0, NULL)


def test_gemm_warm_regions_are_checked_first():
    """The GEMMs' cache-warming region is checked before anything else (zero rows: no GPU)."""
    lin = ("oudjat_linear_bf16_warm", NULL, 0, 1024, 1024, NULL, 1024, 1024, NULL, 0, NULL, NULL, 0, NULL, 1024, 1.0,
           NULL, 0)
    _expect("OUDJAT_ERR_INVALID_ARGUMENT", *lin, NULL, 4096, NULL)
    _expect("OUDJAT_ERR_INVALID_ARGUMENT", *lin, ctypes.c_void_p(256), -128, NULL)
    _expect("OUDJAT_ERR_UNSUPPORTED_LAYOUT", *lin, ctypes.c_void_p(258), 4096, NULL)
    _lib.call(*lin, ctypes.c_void_p(256), 4096, NULL)
    _lib.call(*lin, NULL, 0, NULL)
    qkv = ("oudjat_linear_qkv_rope_kv_warm", NULL, 0, 1024, 1024, NULL, 1024, NULL, 16, 64, NULL, NULL, 64, NULL, NULL,
           NULL, NULL, NULL, 0, 0, NULL, 1.0)
    _expect("OUDJAT_ERR_INVALID_ARGUMENT", *qkv, NULL, 4096, NULL)
    _expect("OUDJAT_ERR_UNSUPPORTED_LAYOUT", *qkv, ctypes.c_void_p(258), 4096, NULL)
    _lib.call(*qkv, ctypes.c_void_p(256), 4096, NULL)


def test_zero_sized_calls_are_noops():
    # Nothing to do -> OK without touching any pointer (and without a GPU).
    _lib.call("oudjat_gather_rows", NULL, 0, 0, 2048, NULL, NULL, 0, NULL, 2048, NULL)
    _lib.call("oudjat_scatter_rows", NULL, 0, 0, 2048, NULL, NULL, 0, NULL, 2048, NULL)
    _lib.call("oudjat_layernorm_rows", NULL, 0, 1024, 1024, NULL, NULL, 1e-5, NULL, 1024, NULL)
    _lib.call("oudjat_nvfp4_quantize", NULL, 0, 1024, 1024, NULL, NULL, NULL, NULL)
    _lib.call("oudjat_layernorm_rows_nvfp4", NULL, 0, 1024, 1024, NULL, NULL, 1e-5, NULL, NULL, 1024, NULL)


def test_wrappers_refuse_cpu_tensors():
    import torch

    from appcorr_amd import kernels as K

    x = torch.zeros(2, 8, 64, dtype=torch.bfloat16)
    idx = torch.zeros(3, dtype=torch.long)
    with pytest.raises(ValueError, match="GPU only"):
        K.gather_rows(x, idx, idx)


def test_linear_kernel_name_reports_a_gemm_kernel():
    """Host-only introspection (no GPU work): the name of the kernel a linear launch would use."""
    from appcorr_amd import _lib
    from appcorr_amd import kernels as K

    name = K.linear_kernel_name(4176, 4096, 1024, _lib.EPI_BIAS_GELU)
    assert name.startswith("oudjat::gemm_bf16_") and name.endswith(", 1>"), name
    assert K.linear_kernel_name(64, 64, 64).startswith("oudjat::gemm_bf16_")


def test_fp8_gemm_entry_points_reject_bad_arguments():
    """The native FP8 GEMM: K % 128, N % 256, 16-byte rows, no GELU, all checked before any launch."""
    A, W, C = ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16)
    ok = dict(M=4, K=128, lda=128, N=256, ldw=128)

    def lin(epi=0, **kv):
        a = dict(ok, **kv)
        return ("oudjat_linear_fp8", A, a["M"], a["K"], a["lda"], W, a["N"], a["ldw"], NULL, epi, NULL, NULL, 0, C,
                a["N"], 1.0, NULL)

    _expect("OUDJAT_ERR_UNSUPPORTED_SHAPE", *lin(K=192, lda=192))
    _expect("OUDJAT_ERR_UNSUPPORTED_SHAPE", *lin(N=192))
    _expect("OUDJAT_ERR_UNSUPPORTED_LAYOUT", *lin(lda=136))
    _expect("OUDJAT_ERR_INVALID_ARGUMENT", *lin(epi=1))   # GELU: not an FP8 route
    _expect("OUDJAT_ERR_INVALID_ARGUMENT", *lin(epi=3))   # LayerScale without gamma
    _expect("OUDJAT_ERR_UNSUPPORTED_SHAPE", "oudjat_fp8_quantize", ctypes.c_void_p(16), 4, 12, 16,
            ctypes.c_void_p(16), 0, ctypes.c_void_p(16), 16, NULL)
    _expect("OUDJAT_ERR_INVALID_ARGUMENT", "oudjat_linear_qkv_rope_kv_fp8", A, 4, 128, 128, W, 128, NULL, 2, 64,
            NULL, NULL, 0, NULL, NULL, NULL, NULL, NULL, 0, 0, NULL, 1.0, NULL)
    from appcorr_amd import kernels as K
    assert K.linear_fp8_kernel_name(1656, 12288, 4096, 5) == "oudjat::gemm_bf16_pp_kernel<192, 256, 5, true>"
    assert K.linear_fp8_kernel_name(1656, 4096, 8192, 3) == "oudjat::gemm_bf16_pp_kernel<128, 256, 3, true>"
    assert K.fp8_gemm_supported(4096, 12288) and not K.fp8_gemm_supported(384, 1152)
