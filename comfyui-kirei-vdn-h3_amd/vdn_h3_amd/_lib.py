"""ctypes binding of ``libvdnh3.so`` (the C ABI declared in ``include/vdnh3.h``).

The library is loaded from this directory only. A missing or unloadable library is a
hard error: there is no CPU or eager-PyTorch fallback for any op of this package.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().with_name("libvdnh3.so")

VDNH3_OK = 0
VDNH3_ERR_INVALID = 1
VDNH3_ERR_RUNTIME = 2
VDNH3_ERR_LINALG = 3

ANCHOR_MODE_CODES = {"none": 0, "columns": 1, "rows": 2, "both": 3}

_c_int, _c_i32, _c_i64, _c_size, _c_float, _vp = (
    ctypes.c_int, ctypes.c_int32, ctypes.c_int64, ctypes.c_size_t, ctypes.c_float, ctypes.c_void_p)
_p_i32 = ctypes.POINTER(ctypes.c_int32)
_p_i64 = ctypes.POINTER(ctypes.c_int64)

# name -> (restype, argtypes); every symbol of include/vdnh3.h
SIGNATURES = {
    "vdnh3_last_error": (ctypes.c_char_p, []),
    "vdnh3_abi_version": (_c_int, []),
    "vdnh3_window_plan_size": (_c_int, [_c_int, _c_int, _c_int, _c_int, _c_int, _p_i32, _c_int, _c_int, _c_int,
                                        _p_i32, _p_i32, _p_i64]),
    "vdnh3_window_plan_build": (_c_int, [_c_int, _c_int, _c_int, _c_int, _c_int, _p_i32, _c_int, _c_int, _c_int,
                                         _p_i32, _c_i32, _p_i32, _c_i32]),
    "vdnh3_window_block_m": (_c_int, []),
    "vdnh3_window_block_n": (_c_int, []),
    "vdnh3_window_workspace_bytes": (_c_size, [_c_int, _c_int, _c_int]),
    "vdnh3_window_attn_fwd": (_c_int, [_vp, _c_i64, _c_i64, _vp, _c_i64, _c_i64, _vp, _c_i64, _c_i64,
                                       _vp, _c_i64, _c_i64, _vp, _c_i64,
                                       _c_int, _c_int, _c_int, _c_float,
                                       _vp, _c_i32, _vp, _vp, _c_size, _vp]),
    "vdnh3_window_vt_prepass": (_c_int, [_vp, _c_i64, _c_i64, _c_int, _c_int, _c_int, _vp, _c_size, _vp]),
    "vdnh3_window_attn_prepared": (_c_int, [_vp, _c_i64, _c_i64, _vp, _c_i64, _c_i64, _vp, _c_i64, _c_i64,
                                            _vp, _c_i64, _c_int, _c_int, _c_int, _c_float,
                                            _vp, _c_i32, _vp, _vp, _c_size, _vp]),
    "vdnh3_window_norm_workspace_bytes": (_c_size, [_c_int, _c_int, _c_int, _c_int]),
    "vdnh3_window_qkv_prepass": (_c_int, [_vp, _c_i64, _c_i64, _vp, _c_float, _vp, _c_i64, _c_i64, _vp, _c_float,
                                          _vp, _c_i64, _c_i64, _vp, _c_i64, _c_int, _c_int, _c_int, _c_int,
                                          _vp, _c_size, _vp]),
    "vdnh3_window_attn_qnorm": (_c_int, [_vp, _c_i64, _c_i64, _vp, _c_float, _vp, _c_i64, _c_i64, _vp, _c_i64,
                                         _c_int, _c_int, _c_int, _c_float, _vp, _c_i32, _vp, _vp, _c_size, _vp]),
    "vdnh3_gemm": (_c_int, [_c_int, _vp, _c_i64, _vp, _c_i64, _vp, _c_i64, _c_int, _c_int, _c_int,
                            _vp, _c_int, _vp, _c_int, _c_float, _vp, _c_int, _c_int, _c_int, _c_int, _c_int, _vp]),
    "vdnh3_quant_rows": (_c_int, [_c_int, _vp, _c_i64, _c_int, _c_int, _vp, _c_i64, _vp, _vp]),
    "vdnh3_quant_tensor_f8": (_c_int, [_vp, _c_i64, _vp, _vp, _vp, _vp]),
    "vdnh3_quant_tensor_f8_noalloc": (_c_int, [_vp, _c_i64, _vp, _vp, _vp]),
    "vdnh3_quant_tensor_f8_noalloc_max_elements": (_c_size, []),
    "vdnh3_frame_stats": (_c_int, [_vp, _c_i64, _c_i64, _vp, _c_i64, _c_i64, _c_int, _vp, _c_i64, _c_int,
                                   _c_int, _c_int, _c_int, _vp, _vp, _vp]),
    "vdnh3_short_conv": (_c_int, [_vp, _c_i64, _c_i64, _vp, _c_int, _c_int, _vp, _c_int, _c_int, _c_int, _c_int,
                                  _c_int, _c_int, _c_int, _vp, _c_i64, _c_i64, _vp]),
    "vdnh3_short_conv_batch": (_c_int, [_vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
                                        _vp]),
    "vdnh3_delta_factor": (_c_int, [_vp, _vp, _vp, _vp, _vp, _c_float, _vp, _c_int, _c_int, _vp]),
    "vdnh3_sana_factor": (_c_int, [_vp, _vp, _vp, _vp, _vp, _c_float, _c_int, _c_int, _c_int, _vp]),
    "vdnh3_delta_scan": (_c_int, [_vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _vp]),
    "vdnh3_readout": (_c_int, [_vp, _c_i64, _c_i64, _c_int, _vp, _vp, _vp, _vp, _vp, _c_int, _vp, _vp, _c_i64,
                               _vp, _c_i64, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _vp]),
    "vdnh3_readout_fused_gate": (_c_int, [_vp, _c_i64, _c_i64, _c_int, _vp, _vp, _vp, _vp, _vp, _c_int, _vp, _vp,
                                          _c_i64, _vp, _vp, _vp, _c_i64, _c_int, _c_int, _c_int, _c_int, _c_int,
                                          _c_int, _vp]),
    "vdnh3_frame_mean": (_c_int, [_vp, _c_i64, _c_int, _c_int, _c_int, _vp, _vp]),
    "vdnh3_linear_f32": (_c_int, [_vp, _c_i64, _vp, _c_int, _c_i64, _vp, _vp, _c_i64, _c_int, _c_int, _c_int,
                                  _vp]),
    "vdnh3_alpha_decay": (_c_int, [_vp, _vp, _vp, _c_int, _c_int, _c_int, _vp]),
    "vdnh3_alpha_logsum": (_c_int, [_vp, _c_int, _c_int, _c_int, _vp, _vp]),
    "vdnh3_fill_rows_bf16": (_c_int, [_vp, _c_i64, _c_int, _c_int, _c_float, _vp]),
    "vdnh3_qk_rmsnorm": (_c_int, [_vp, _c_i64, _c_i64, _vp, _c_i64, _c_i64, _vp, _vp, _c_float, _c_float,
                                  _vp, _c_i64, _c_i64, _vp, _c_i64, _c_i64, _c_int, _c_int, _c_int, _vp]),
    "vdnh3_qk_rmsnorm_rope": (_c_int, [_vp, _c_i64, _c_i64, _vp, _c_i64, _c_i64, _vp, _vp, _c_float, _vp, _c_i64,
                                       _c_int, _vp, _c_i64, _c_i64, _vp, _c_i64, _c_i64, _c_int, _c_int, _c_int,
                                       _vp]),
    "vdnh3_gdn_workspace_bytes": (_c_size, [_c_int, _c_int, _c_int]),
    "vdnh3_gdn_chunk_fwd": (_c_int, [_vp, _c_i64, _c_i64, _vp, _c_i64, _c_i64, _vp, _c_i64, _c_i64, _vp, _c_i64,
                                     _vp, _c_i64, _vp, _vp, _vp, _c_i64, _c_i64, _c_int, _c_int, _c_int, _vp,
                                     _c_size, _vp]),
    "vdnh3_gdn_segments": (_c_int, [_c_int, _c_int, _c_int]),
    "vdnh3_gdn_prep": (_c_int, [_vp, _c_i64, _c_i64, _vp, _c_i64, _c_i64, _vp, _c_i64, _c_i64, _vp, _c_i64, _vp,
                                _c_i64, _c_int, _c_int, _c_int, _c_int, _vp, _c_size, _vp]),
    "vdnh3_gdn_scan": (_c_int, [_vp, _vp, _vp, _c_i64, _c_i64, _c_int, _c_int, _c_int, _c_int, _vp, _c_size, _vp]),
    "vdnh3_rmsnorm_modulate": (_c_int, [_vp, _c_i64, _vp, _c_float, _vp, _vp, _c_i64, _c_int, _vp, _c_int, _vp,
                                        _c_i64, _c_int, _c_int, _vp]),
    "vdnh3_gated_residual": (_c_int, [_vp, _c_i64, _vp, _c_i64, _c_int, _vp, _c_int, _vp, _c_i64, _vp, _c_i64,
                                      _c_int, _c_int, _vp]),
    "vdnh3_swiglu": (_c_int, [_vp, _c_i64, _c_int, _c_int, _vp, _c_i64, _vp]),
    "vdnh3_swiglu_quant_rows": (_c_int, [_c_int, _vp, _c_i64, _c_int, _c_int, _vp, _c_i64, _vp, _vp]),
    "vdnh3_head_gate": (_c_int, [_vp, _c_i64, _c_i64, _vp, _c_i64, _vp, _c_i64, _c_int, _c_int, _c_int, _vp]),
    "vdnh3_mfma_peak": (_c_int, [_c_int, _vp, _vp, _c_int, _c_int, _vp, _vp]),
    "vdnh3_mfma_peak_ops": (ctypes.c_double, [_c_int, _c_int, _c_int]),
}

_lock = threading.Lock()
_lib = None


class LibraryMissingError(RuntimeError):
    """libvdnh3.so is not built or cannot be loaded."""


def lib():
    """The loaded library (raises ``LibraryMissingError`` if it is not built)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise LibraryMissingError(
                    f"{LIB_PATH} is not built; run `python -m vdn_h3_amd._build` or __graft_entry__.build()")
            try:
                handle = ctypes.CDLL(str(LIB_PATH))
            except OSError as exc:
                raise LibraryMissingError(f"cannot load {LIB_PATH}: {exc}") from exc
            for name, (restype, argtypes) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = restype
                fn.argtypes = argtypes
            _lib = handle
    return _lib


def last_error() -> str:
    return (lib().vdnh3_last_error() or b"").decode(errors="replace")


def check(rc: int, what: str) -> None:
    """Map a VDNH3_* status to the exception type the reference raises."""
    if rc == VDNH3_OK:
        return
    message = f"{what}: {last_error()}"
    if rc == VDNH3_ERR_INVALID:
        raise ValueError(message)
    if rc == VDNH3_ERR_LINALG:
        raise torch.linalg.LinAlgError(message)
    raise RuntimeError(message)


def ptr(tensor) -> ctypes.c_void_p | None:
    """Device (or host) address of a tensor, ``None`` for ``None``."""
    if tensor is None:
        return None
    return ctypes.c_void_p(tensor.data_ptr())


def stream_handle(device: torch.device) -> ctypes.c_void_p:
    """Raw hipStream_t of torch's current stream on ``device``."""
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def forward_only(what: str, *tensors) -> None:
    """The HIP ops have no backward: in gradient mode an input that requires grad is an error, since the
    result would silently carry no gradient."""
    if torch.is_grad_enabled() and any(isinstance(t, torch.Tensor) and t.requires_grad for t in tensors):
        raise RuntimeError(f"{what} is forward-only (no backward) and an input requires grad; "
                           "call it under torch.no_grad() or torch.inference_mode()")


def require_device(*tensors) -> torch.device:
    """All tensors must live on one GPU; the HIP path has no CPU fallback."""
    device = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError("vdn_h3_amd ops run on a ROCm GPU only (got a CPU tensor); "
                               "there is no CPU fallback")
        if device is None:
            device = t.device
        elif t.device != device:
            raise RuntimeError(f"tensors on different devices: {device} and {t.device}")
    return device
