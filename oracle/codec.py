"""ctypes front end of the C oracle (oracle/nori_oracle.c) for the int8 cache codec.

TEST INFRASTRUCTURE ONLY: the checker that the HIP kernels are compared with. Only
tests/, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import this module. Nothing in the product package imports it.

Restates ``quantize_int8`` / ``dequantize_int8``
(src/synthefy_nori/model/kv_cache_scaling.py:29-41) with torch's per-op rounding
in the tensor dtype; see the header of nori_oracle.c for the exact semantics and the
CPU/GPU difference in ``m / 127.0``.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
SOURCE = os.path.join(HERE, "nori_oracle.c")
LIBRARY = os.path.join(HERE, "libnori_oracle.so")

F32, F16, BF16 = 0, 1, 2
DIV_TRUE, DIV_RECIP = 0, 1  # torch on CPU, torch on a GPU

_lib = None


def build(force: bool = False) -> str:
    """Compile nori_oracle.c into libnori_oracle.so beside it (gcc, -O2, no fast-math)."""
    if force or not os.path.exists(LIBRARY) or os.path.getmtime(LIBRARY) < os.path.getmtime(SOURCE):
        tmp = LIBRARY + ".tmp"
        subprocess.run(
            ["gcc", "-O2", "-fPIC", "-shared", "-fno-fast-math", "-ffp-contract=off", "-o", tmp, SOURCE, "-lm"],
            check=True,
        )
        os.replace(tmp, LIBRARY)
    return LIBRARY


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIBRARY):
            build()
        _lib = ctypes.CDLL(LIBRARY)
        vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        _lib.oracle_quantize_int8.argtypes = [vp, i32, i64, i32, i32, vp, vp]
        _lib.oracle_dequantize_int8.argtypes = [vp, vp, i64, i32, vp, i32]
        _lib.oracle_round_f32_array.argtypes = [vp, i64, i32, vp]
        _lib.oracle_f32_to_f16_array.argtypes = [vp, i64, vp]
        _lib.oracle_f32_to_bf16_array.argtypes = [vp, i64, vp]
        _lib.oracle_rms_norm.argtypes = [vp, vp, i32, i64, i32, ctypes.c_double, vp]
        for f in (
            _lib.oracle_quantize_int8,
            _lib.oracle_dequantize_int8,
            _lib.oracle_round_f32_array,
            _lib.oracle_f32_to_f16_array,
            _lib.oracle_f32_to_bf16_array,
            _lib.oracle_rms_norm,
        ):
            f.restype = None
    return _lib


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def bits_dtype_code(bits: np.ndarray, dtype: str) -> tuple[np.ndarray, int]:
    """Map (array, dtype name) to the raw array the C oracle reads and its dtype code.

    ``bits`` holds float32 values for "f32", float16 values for "f16", and uint16
    bf16 bit patterns for "bf16".
    """
    if dtype == "f32":
        return np.ascontiguousarray(bits, dtype=np.float32), F32
    if dtype == "f16":
        return np.ascontiguousarray(bits, dtype=np.float16), F16
    if dtype == "bf16":
        return np.ascontiguousarray(bits, dtype=np.uint16), BF16
    raise ValueError(f"unknown dtype {dtype!r}")


def quantize_int8(src: np.ndarray, dtype: str, div_mode: int = DIV_TRUE) -> tuple[np.ndarray, np.ndarray]:
    """Quantize the last axis of ``src``: returns (int8 codes of src.shape, fp32 scales of shape[:-1]+(1,))."""
    raw, code = bits_dtype_code(src, dtype)
    d = raw.shape[-1]
    n_vec = raw.size // d if d else 0
    codes = np.empty(raw.shape, dtype=np.int8)
    scales = np.empty(raw.shape[:-1] + (1,), dtype=np.float32)
    lib().oracle_quantize_int8(_ptr(raw), code, n_vec, d, div_mode, _ptr(codes), _ptr(scales))
    return codes, scales


def dequantize_int8(codes: np.ndarray, scales: np.ndarray, dtype: str) -> np.ndarray:
    """Dequantize to ``dtype``; bf16 results are returned as uint16 bit patterns."""
    codes = np.ascontiguousarray(codes, dtype=np.int8)
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    d = codes.shape[-1]
    out_dtype = {"f32": np.float32, "f16": np.float16, "bf16": np.uint16}[dtype]
    out = np.empty(codes.shape, dtype=out_dtype)
    lib().oracle_dequantize_int8(
        _ptr(codes), _ptr(scales), codes.size // d, d, _ptr(out), {"f32": F32, "f16": F16, "bf16": BF16}[dtype]
    )
    return out


def round_f32(x: np.ndarray, dtype: str) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().oracle_round_f32_array(_ptr(x), x.size, {"f32": F32, "f16": F16, "bf16": BF16}[dtype], _ptr(y))
    return y


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, dtype=np.uint16)
    lib().oracle_f32_to_f16_array(_ptr(x), x.size, _ptr(y))
    return y


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, dtype=np.uint16)
    lib().oracle_f32_to_bf16_array(_ptr(x), x.size, _ptr(y))
    return y


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def rms_norm(x: np.ndarray, weight: np.ndarray | None, dtype: str, eps: float) -> np.ndarray:
    """RMSNorm over the last axis (layer.py:233-258), double statistic, one rounding to ``dtype``."""
    raw, code = bits_dtype_code(x, dtype)
    cols = raw.shape[-1]
    w = None if weight is None else bits_dtype_code(weight, dtype)[0]
    out = np.empty_like(raw)
    lib().oracle_rms_norm(_ptr(raw), None if w is None else _ptr(w), code, raw.size // cols, cols, eps, _ptr(out))
    return out
