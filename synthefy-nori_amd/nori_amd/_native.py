"""ctypes binding of libnori_hip.so (the C ABI declared in include/nori_hip.h).

The library is the product path: every operator in this package runs one of its
kernels on the current HIP stream of the tensor's device. There is no CPU fallback;
calling an operator on CPU tensors, or without the built library, raises.
"""

from __future__ import annotations

import ctypes
import os

import torch

LIBRARY = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libnori_hip.so")

NORI_OK, NORI_ERR_INVALID, NORI_ERR_RUNTIME, NORI_ERR_UNSUPPORTED, NORI_ERR_OUT_OF_MEMORY = range(5)
NORI_F32, NORI_F16, NORI_BF16, NORI_I8 = range(4)
SCALE_DIV_TRUE, SCALE_DIV_RECIP = 0, 1
ATTN_MERGE = 1
NOALLOC_SCRATCH_BYTES = 32 << 20  # NORI_NOALLOC_SCRATCH_BYTES
ABI_VERSION = 3  # NORI_ABI_VERSION: the signatures below

_DTYPE_CODES = {
    torch.float32: NORI_F32,
    torch.float16: NORI_F16,
    torch.bfloat16: NORI_BF16,
    torch.int8: NORI_I8,
}

# Every symbol include/nori_hip.h declares, with its ctypes signature.
_vp, _i64, _i32, _u32, _f32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_uint32, ctypes.c_float
SIGNATURES: dict[str, tuple[object, list]] = {
    "nori_abi_version": (ctypes.c_int, []),
    "nori_last_error": (ctypes.c_char_p, []),
    "nori_kv_quantize_int8": (
        ctypes.c_int,
        [_vp, _i32, _i64, _i64, _i32, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _i32, _vp],
    ),
    "nori_kv_dequantize_int8": (
        ctypes.c_int,
        [_vp, _vp, _i64, _i64, _i32, _i64, _i64, _i64, _i64, _vp, _i32, _i64, _i64, _vp],
    ),
    "nori_rms_norm": (ctypes.c_int, [_vp, _i32, _i64, _i32, _i64, _vp, _i32, _f32, _vp, _i64, _vp]),
    "nori_rms_norm_to": (ctypes.c_int, [_vp, _i32, _i64, _i32, _i64, _vp, _i32, _f32, _vp, _i32, _i64, _vp]),
    "nori_icl_attention": (
        ctypes.c_int,
        [
            _vp, _i32, _i64, _i64, _i32, _i32, _i64, _i64, _i64,  # q
            _vp, _i32, _vp, _i64, _i32, _i64, _i64, _i64, _i64, _i64, _i64,  # kv
            _f32,  # scale
            _vp, _i32, _i64, _i64, _i64,  # out
            _vp, _u32, _vp, _i64, _vp,  # lse, flags, workspace, bytes, stream
        ],
    ),
    "nori_icl_attention_qk": (
        ctypes.c_int,
        [
            _vp, _i32, _i64, _i64, _i32, _i32, _i64, _i64, _i64,  # q
            _vp, _i32, _vp, _i64, _i32, _i64, _i64, _i64, _i64, _i64, _i64,  # kv
            _f32,  # scale
            _vp, _i32, _i64, _i64, _i64,  # out
            _vp, _u32, _vp, _i64, _vp, _vp,  # lse, flags, workspace, bytes, prologue, stream
        ],
    ),
    "nori_icl_attention_workspace_size": (_i64, [_i64, _i64, _i32, _i32, _i64]),
    "nori_icl_attention_takes_prologue": (_i32, [_i64, _i64, _i32, _i32, _i64, _i32, _i32, _i32]),
    "nori_icl_attention_noalloc": (
        ctypes.c_int,
        [
            _vp, _i32, _i64, _i64, _i32, _i32, _i64, _i64, _i64,  # q
            _vp, _i32, _vp, _i64, _i32, _i64, _i64, _i64, _i64, _i64, _i64,  # kv
            _f32,  # scale
            _vp, _i32, _i64, _i64, _i64,  # out
            _vp, _u32, _vp,  # lse, flags, stream
        ],
    ),
    "nori_residual_add": (ctypes.c_int, [_vp, _vp, _i32, _f32, _i64, _vp, _vp]),
    "nori_silu_mul": (ctypes.c_int, [_vp, _i32, _i64, _i32, _i64, _vp, _i64, _vp]),
    "nori_layer_norm": (ctypes.c_int, [_vp, _i32, _i64, _i32, _i64, _vp, _vp, _f32, _i32, _vp, _i32, _i64, _vp]),
    "nori_swiglu_mlp": (ctypes.c_int, [_vp, _i32, _i64, _i32, _i64, _vp, _vp, _i32, _vp, _i64, _vp]),
    "nori_qass_gate": (ctypes.c_int, [_vp, _i32, _i64, _i32, _i32, _i64, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _i64, _vp]),
    "nori_residual_add_rms_norm": (ctypes.c_int, [_vp, _vp, _i32, _vp, _f32, _i64, _i32, _f32, _vp, _vp, _i32, _i64, _i64,
                                                  _i64, _vp]),
    "nori_kv_project_quantize_int8": (
        ctypes.c_int,
        [_vp, _i32, _i64, _i64, _i32, _i64, _i64, _i32, _f32, _vp, _i32, _i64, _i32, _i32,
         _vp, _i64, _i64, _vp, _i64, _i64, _i32, _vp, _i64, _vp],
    ),
    "nori_kv_project_quantize_int8_workspace_size": (_i64, [_i32, _i64, _i64, _i32, _i32]),
    "nori_kv_project_quantize_int8_workspace_bytes": (_i64, [_i32, _i64, _i64, _i32, _i32, _i32, _i32]),
    "nori_linear_f16": (
        ctypes.c_int, [_vp, _i64, _i64, _i64, _i32, _i64, _i64, _i64, _vp, _i64, _i32, _vp, _i64, _i64, _i64, _vp],
    ),
    "nori_swiglu_mlp_residual_rms_norm": (
        ctypes.c_int,
        [_vp, _i32, _i64, _i32, _i64, _vp, _vp, _i32, _f32, _vp, _i64, _i32, _f32, _vp, _i64, _i64, _i64, _vp],
    ),
    "nori_layer_norm_cells": (
        ctypes.c_int,
        [_vp, _i32, _i64, _i64, _i64, _i32, _i64, _vp, _vp, _f32, _vp, _vp, _i64, _vp, _f32, _vp, _vp],
    ),
    "nori_cell_tokens": (
        ctypes.c_int,
        [_vp, _i64, _i64, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _f32, _vp, _vp, _i32, _vp, _i32, _vp, _vp, _vp],
    ),
    "nori_linear_f16_residual_rms_norm": (
        ctypes.c_int,
        [_vp, _i64, _i64, _i64, _i32, _i64, _i64, _i64, _vp, _i64, _f32, _vp, _i64, _i64, _i64, _f32, _vp, _i64, _i64,
         _i64, _vp],
    ),
    "nori_mfma_f16_probe": (ctypes.c_int, [_vp, _i64, _i32, _vp, _i64, _vp]),
    "nori_mfma_f16_probe_flop": (_i64, [_i64]),
    "nori_quant_f16_scale_probe": (ctypes.c_int, [_vp, _i64, _vp, _vp, _vp]),
}

_lib: ctypes.CDLL | None = None


def library_path() -> str:
    return LIBRARY


def lib() -> ctypes.CDLL:
    """Load libnori_hip.so (once). Raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIBRARY):
            raise RuntimeError(
                f"{LIBRARY} is not built; run `python -c 'import __graft_entry__ as g; g.build()'` "
                "(or python synthefy-nori_amd/nori_amd/build.py) first"
            )
        handle = ctypes.CDLL(LIBRARY)
        handle.nori_abi_version.restype = ctypes.c_int
        found = handle.nori_abi_version()
        if found != ABI_VERSION:
            raise RuntimeError(f"{LIBRARY} has ABI version {found}, this package binds version {ABI_VERSION}; rebuild it")
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = handle
    return _lib


def check(status: int, what: str) -> None:
    """Map a nori_status to the exception type the reference raises for the same failure."""
    if status == NORI_OK:
        return
    message = f"{what}: {lib().nori_last_error().decode(errors='replace')}"
    if status == NORI_ERR_INVALID:
        raise ValueError(message)
    if status == NORI_ERR_UNSUPPORTED:
        raise NotImplementedError(message)
    if status == NORI_ERR_OUT_OF_MEMORY:
        raise torch.cuda.OutOfMemoryError(message)
    raise RuntimeError(message)


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dtype]
    except KeyError:
        raise NotImplementedError(f"nori_amd kernels do not take {dtype}") from None


def require_device(*tensors: torch.Tensor) -> torch.device:
    """All tensors must live on one ROCm device; the kernels have no CPU path."""
    device = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(
                f"nori_amd kernels run on a ROCm GPU; got a tensor on {t.device}. "
                "Move the cache and queries to the GPU (there is no CPU fallback)."
            )
        if device is None:
            device = t.device
        elif t.device != device:
            raise RuntimeError(f"tensors on different devices: {device} and {t.device}")
    if device is None:
        raise ValueError("no tensor given")
    return device


def stream_of(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


class QKPrologue(ctypes.Structure):
    """``nori_qk_prologue``: per-head q/k RMS norm gains, eps and a q multiplier."""

    _fields_ = [
        ("q_weight", ctypes.c_void_p),
        ("k_weight", ctypes.c_void_p),
        ("weight_dtype", ctypes.c_int),
        ("eps", ctypes.c_float),
        ("q_mult", ctypes.c_float),
    ]
