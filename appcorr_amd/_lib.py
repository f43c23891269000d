"""ctypes binding of liboudjat_hip.so (declared in include/oudjat.h).

The library is the only compute path: there is no eager or CPU fallback anywhere in the package. If
the library is missing or fails its self-test, every entry point raises.

torch is imported before the library is opened so that the HIP runtime torch ships with
(libamdhip64.so.7) is the one the library binds to; both share that SONAME.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch  # noqa: F401  -- must be loaded before the HIP library, see module docstring

LIB_PATH = Path(__file__).resolve().parent / "liboudjat_hip.so"
ABI_VERSION = 18

OK = 0
STATUS_NAMES = {
    0: "OUDJAT_OK",
    1: "OUDJAT_ERR_INVALID_ARGUMENT",
    2: "OUDJAT_ERR_UNSUPPORTED_SHAPE",
    3: "OUDJAT_ERR_UNSUPPORTED_LAYOUT",
    4: "OUDJAT_ERR_TOO_LARGE",
    5: "OUDJAT_ERR_LAUNCH",
    6: "OUDJAT_ERR_HIP",
}

EPI_BIAS = 0
EPI_BIAS_GELU = 1
EPI_BIAS_LS_RESID = 2
EPI_BIAS_LS = 3
EPI_BIAS_SILU_MUL = 4
EPI_RAW_BF16 = 16  # flag: round the accumulator to bf16 before the scale and bias (NVFP4 linears)

QUERY_PROB_NOALLOC_MAX = 1 << 20  # OUDJAT_QUERY_PROB_NOALLOC_MAX: fp32 elements of the no-alloc scratch array

IMPORTANCE_L2 = 0
IMPORTANCE_ENERGY = 1
IMPORTANCE_RMS = 2


class OudjatUnavailable(RuntimeError):
    """The HIP library is not built or cannot be loaded. There is no fallback path."""


class OudjatKernelError(RuntimeError):
    """A library entry point returned a non-OK status (nothing was launched, or the launch failed)."""

    def __init__(self, func: str, status: int, message: str):
        self.func = func
        self.status = status
        self.status_name = STATUS_NAMES.get(status, f"status {status}")
        super().__init__(f"{func}: {self.status_name}: {message}")


_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float

# name -> argtypes (every function returns int status unless listed in _RESTYPES)
SIGNATURES: dict[str, list] = {
    "oudjat_abi_version": [],
    "oudjat_status_string": [_i32],
    "oudjat_last_error": [],
    "oudjat_selftest": [_p],
    "oudjat_patch_importance": [_p, _i64, _i64, _i64, _i32, _p, _p],
    "oudjat_topk_plan": [_p, _i64, _i64, _i64, _i64, _p, _i64, _i64, _i64, _p, _p, _p, _p, _p, _p, _p, _p, _p],
    "oudjat_threshold_keep": [_p, _i64, _i64, _i64, _f32, _p, _p, _p],
    "oudjat_patch_attention_prob": [_p, _i64, _i64, _i64, _i64, _i64, _p, _i64, _i64, _i64, _f32, _i32, _p, _p, _i64,
                                    _p],
    "oudjat_patch_residual_score": [_p, _p, _i32, _i64, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i32, _p, _p],
    "oudjat_residual_prune_keep": [_p, _i64, _i64, _i64, _p, _i64, _i64, _f32, _i64, _p, _p, _p, _p, _p],
    "oudjat_residual_prune_compact": [_p, _i64, _i64, _p, _i64, _p, _i64, _i64, _i64, _p, _p, _p],
    "oudjat_threshold_plan": [_p, _i64, _i64, _i64, _f32, _i64, _i32, _p, _i64, _i64, _i64, _p, _p, _p, _p, _p, _p,
                              _p, _p, _p, _p, _p],
    "oudjat_plan_stats": [_p, _i64, _i64, _i64, _p, _p, _p],
    "oudjat_gather_rows": [_p, _i64, _i64, _i64, _p, _p, _i64, _p, _i64, _p],
    "oudjat_scatter_rows": [_p, _i64, _i64, _i64, _p, _p, _i64, _p, _i64, _p],
    "oudjat_active_token_update": [_p, _i64, _i64, _p, _p, _i64, _p, _i64, _p, _i64, _i64, _p],
    "oudjat_reconstruct_scatter_persist": [_p, _p, _p, _p, _p, _p, _i64, _i64, _p, _p],
    "oudjat_fused_layerscale_add": [_p, _p, _p, _i64, _i64, _p, _p],
    "oudjat_rope_active_inplace": [_p, _i64, _i64, _p, _i64, _i64, _p, _p, _i64, _p, _p, _i64, _i64, _i64, _p],
    "oudjat_qkv_rope_kv_scatter": [_p, _i64, _i64, _i64, _p, _p, _i64, _p, _p, _p, _p, _p, _i64, _i64, _p, _p],
    "oudjat_layernorm_rows": [_p, _i64, _i64, _i64, _p, _p, _f32, _p, _i64, _p],
    "oudjat_layernorm_rows_prefetch": [_p, _i64, _i64, _i64, _p, _p, _f32, _p, _i64, _p, _i64, _p],
    "oudjat_linear_bf16": [_p, _i64, _i64, _i64, _p, _i64, _i64, _p, _i32, _p, _p, _i64, _p, _i64, _f32, _p, _i64,
                           _p],
    "oudjat_linear_bf16_warm": [_p, _i64, _i64, _i64, _p, _i64, _i64, _p, _i32, _p, _p, _i64, _p, _i64, _f32, _p,
                                _i64, _p, _i64, _p],
    "oudjat_linear_workspace_elems": [_i64, _i64, _i64, _i32],
    "oudjat_linear_warm_slots": [_i64, _i64, _i64, _i32],
    "oudjat_linear_splitk_partial": [_p, _i64, _i64, _i64, _p, _i64, _i64, _p, _i64, _p, _p],
    "oudjat_splitk_ls_packed_residual": [_p, _i64, _p, _p, _f32, _p, _p, _i64, _i64, _p, _p, _p, _i64, _i64, _p, _p,
                                         _p, _f32, _p, _p],
    "oudjat_linear_kernel_name": [_i64, _i64, _i64, _i32, ctypes.c_char_p, _i64],
    "oudjat_packed_residual_persist": [_p, _p, _p, _i64, _i64, _p, _p, _p, _i64, _i64, _p, _p],
    "oudjat_packed_residual_persist_ln": [_p, _p, _p, _i64, _i64, _p, _p, _p, _i64, _i64, _p, _p, _p, _f32, _p, _p],
    "oudjat_fold_residual_rows": [_p, _i64, _i64, _p, _p, _p, _i64, _p, _p],
    "oudjat_linear_qkv_rope_kv": [_p, _i64, _i64, _i64, _p, _i64, _p, _i64, _i64, _p, _p, _i64, _p, _p, _p, _p, _p,
                                  _i64, _i64, _p, _f32, _p],
    "oudjat_linear_qkv_rope_kv_warm": [_p, _i64, _i64, _i64, _p, _i64, _p, _i64, _i64, _p, _p, _i64, _p, _p, _p, _p,
                                       _p, _i64, _i64, _p, _f32, _p, _i64, _p],
    "oudjat_linear_swiglu_nvfp4": [_p, _i64, _i64, _i64, _p, _i64, _i64, _p, _i64, _f32, _p, _f32, _p, _p, _p, _i64,
                                   _p],
    "oudjat_linear_qkv_rope_kv_nvfp4": [_p, _i64, _i64, _i64, _p, _i64, _p, _i64, _i64, _p, _p, _i64, _p, _p, _p,
                                        _p, _p, _i64, _i64, _p, _f32, _p],
    "oudjat_sparse_query_attention": [_p, _i64, _i64, _i64, _i64, _i64, _p, _i64, _i64, _i64, _i64, _i64, _f32, _p,
                                      _i64, _p],
    "oudjat_sparse_query_attention_ws": [_p, _i64, _i64, _i64, _i64, _i64, _p, _i64, _i64, _i64, _i64, _i64, _f32,
                                         _p, _i64, _p, _i64, _p],
    "oudjat_sparse_query_attention_workspace_elems": [_i64, _i64, _i64, _i64, _i64],
    "oudjat_sparse_query_attention_fp8": [_p, _i64, _i64, _i64, _i64, _i64, _p, _i64, _i64, _i64, _i64, _i64, _f32,
                                          _p, _p, _i64, _p],
    "oudjat_sparse_query_attention_lse": [_p, _i64, _i64, _i64, _i64, _i64, _p, _i64, _i64, _i64, _i64, _i64, _f32,
                                          _p, _i64, _p, _p],
    "oudjat_patch_attention_prob_workspace_elems": [_i64, _i64, _i64, _i32],
    "oudjat_residual_pair": [_p, _p, _p, _i64, _i64, _p, _p, _p],
    "oudjat_gather_rows_ln": [_p, _i64, _i64, _i64, _p, _p, _i64, _p, _p, _f32, _p, _p, _p, _p],
    "oudjat_patch_attention_prob_lse": [_p, _i64, _i64, _i64, _i64, _i64, _p, _i64, _i64, _i64, _f32, _p, _p, _p,
                                        _i64, _p],
    "oudjat_nvfp4_quantize": [_p, _i64, _i64, _i64, _p, _p, _p, _p],
    "oudjat_nvfp4_dequantize": [_p, _p, _p, _i64, _i64, _p, _i64, _p],
    "oudjat_query_attention_prob": [_p, _i64, _i64, _i64, _i64, _i64, _p, _i64, _i64, _i64, _i64, _f32, _p, _p, _i64,
                                    _i32, _p],
    "oudjat_pseudo_query": [_p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p, _p],
    "oudjat_nvfp4_quantize_dequantize": [_p, _i64, _i64, _i64, _p, _p, _p, _p, _i64, _p],
    "oudjat_fp8_quantize_dequantize": [_p, _i64, _i64, _i64, _p, _i32, _p, _i64, _p],
    "oudjat_fp8_quantize": [_p, _i64, _i64, _i64, _p, _i32, _p, _i64, _p],
    "oudjat_layernorm_rows_nvfp4": [_p, _i64, _i64, _i64, _p, _p, _f32, _p, _p, _i64, _p],
    "oudjat_packed_residual_persist_ln_nvfp4": [_p, _p, _p, _i64, _i64, _p, _p, _p, _i64, _i64, _p, _p, _p, _f32,
                                                _p, _p, _p],
    "oudjat_swiglu_scaled_nvfp4": [_p, _f32, _p, _p, _f32, _p, _i64, _i64, _p, _p, _p],
    "oudjat_qkv_rope_kv_scatter_scaled": [_p, _i64, _i64, _i64, _f32, _p, _p, _p, _i64, _p, _p, _p, _p, _p, _i64,
                                          _i64, _p, _p],
    "oudjat_linear_fp8": [_p, _i64, _i64, _i64, _p, _i64, _i64, _p, _i32, _p, _p, _i64, _p, _i64, _f32, _p],
    "oudjat_linear_qkv_rope_kv_fp8": [_p, _i64, _i64, _i64, _p, _i64, _p, _i64, _i64, _p, _p, _i64, _p, _p, _p, _p,
                                      _p, _i64, _i64, _p, _f32, _p],
    "oudjat_linear_fp8_kernel_name": [_i64, _i64, _i64, _i32, ctypes.c_char_p, _i64],
    "oudjat_scale_bias_rows": [_p, _i64, _i64, _i64, _f32, _p, _p, _p, _i64, _p],
    "oudjat_swiglu_scaled": [_p, _f32, _p, _p, _f32, _p, _i64, _i64, _p, _p],
    "oudjat_amax_update": [_p, _i64, _i64, _i64, _p, _p],
    "oudjat_query_attention_prob_noalloc": [_p, _i64, _i64, _i64, _i64, _i64, _p, _i64, _i64, _i64, _i64, _f32, _p,
                                            _i64, _i32, _p],
}
_RESTYPES = {"oudjat_status_string": ctypes.c_char_p, "oudjat_last_error": ctypes.c_char_p,
             "oudjat_linear_workspace_elems": ctypes.c_int64, "oudjat_linear_warm_slots": ctypes.c_int64,
             "oudjat_sparse_query_attention_workspace_elems": ctypes.c_int64,
             "oudjat_patch_attention_prob_workspace_elems": ctypes.c_int64}

_lock = threading.Lock()
_lib = None
_selftest_ok: set[int] = set()


def load() -> ctypes.CDLL:
    """Open the library (once) and declare every exported signature."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise OudjatUnavailable(
                f"{LIB_PATH} is not built; run `python -m appcorr_amd.build` "
                "(or __graft_entry__.build()). There is no non-HIP fallback."
            )
        try:
            lib = ctypes.CDLL(str(LIB_PATH))
        except OSError as exc:
            raise OudjatUnavailable(f"cannot load {LIB_PATH}: {exc}") from exc
        for name, argtypes in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = _RESTYPES.get(name, ctypes.c_int)
        got = lib.oudjat_abi_version()
        if got != ABI_VERSION:
            raise OudjatUnavailable(f"{LIB_PATH} has ABI version {got}, expected {ABI_VERSION}; rebuild it")
        _lib = lib
    return _lib


def call(name: str, *args) -> None:
    """Call an entry point and raise OudjatKernelError on a non-OK status."""
    lib = load()
    status = getattr(lib, name)(*args)
    if status != OK:
        msg = lib.oudjat_last_error()
        raise OudjatKernelError(name, status, msg.decode() if msg else "")


def stream_of(t: torch.Tensor) -> int:
    """Raw hipStream_t of torch's current stream on the tensor's device."""
    return torch.cuda.current_stream(t.device).cuda_stream


def verify_runtime(device: torch.device | int | None = None) -> bool:
    """Run the library's self-test kernel once per device (raises on failure).

    Mirrors verify_triton_runtime (appcorr/models/dinov3/layers/triton_kernels/_strict.py:74-125):
    prove at start-up that device code actually runs here rather than at the first correction.
    """
    if not torch.cuda.is_available():
        raise OudjatUnavailable("no HIP device is visible; the correction path runs only on a GPU")
    dev = torch.device("cuda", torch.cuda.current_device() if device is None else torch.device(device).index or 0)
    if dev.index in _selftest_ok:
        return True
    with torch.cuda.device(dev):
        call("oudjat_selftest", ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream))
    _selftest_ok.add(dev.index)
    return True


def exported_symbols() -> list[str]:
    return list(SIGNATURES)


def lib_path() -> str:
    return os.fspath(LIB_PATH)
