"""Projections of the attention sublayers: ``F.linear`` under fp16 autocast on the HIP kernel.

``linear(x, weight)`` is ``torch.nn.functional.linear(x, weight)`` for fp16 operands (what the
reference's projections compute under the GPU's fp16 autocast, layer.py:651-683, 1114-1160):
fp32 sums of fp16 products, rounded once to fp16. ``nori_linear_f16`` (csrc/linear.hip) reads
x and writes the output through strides -- a token subset of each row, a slice of a stacked
output buffer (``out``), the transposed [table, group, row] view of a cell buffer -- without
copies. ``linear`` routes to it the shapes where it is the faster of the two (same-box A/B
against the library GEMM: inner width 128 and up to 256 output columns, e.g. 655,360 rows x
128 -> 128 in 78 against 110 us; at inner width 256 or wider outputs the library GEMM was as
fast or faster); everything else (other dtypes, widths or shapes, short operands, CPU
tensors) is ``F.linear``. The two differ only in the order of the fp32 sums.
"""

from __future__ import annotations

import ctypes

import torch

from . import _native as nat

__all__ = ["linear", "linear_residual_norm", "takes_kernel"]

_WIDTHS = (128,)  # inner widths routed to the kernel (it also takes 256, where the library GEMM was faster)
_MAX_N = 256      # output widths up to this (past it the library GEMM was as fast or faster)
_MIN_ROWS = 4096  # below this the library GEMM's launch is as cheap


def _row_levels(t: torch.Tensor) -> list[tuple[int, int]] | None:
    """The rows of ``t`` [..., C] as at most three (count, stride) levels, outer first (adjacent
    leading dims merged where their strides chain), or None when they need more levels."""
    merged: list[tuple[int, int]] = []
    for size, stride in zip(t.shape[:-1], t.stride()[:-1]):
        size, stride = int(size), int(stride)
        if size == 1:
            continue
        if merged and merged[-1][1] == stride * size:
            merged[-1] = (merged[-1][0] * size, stride)
        else:
            merged.append((size, stride))
    return merged if len(merged) <= 3 else None


def _common_grid(*tensors: torch.Tensor) -> tuple | None:
    """((n_outer, n_mid, n_inner), strides of each tensor ...): one three-level row grid
    addressing the rows of every tensor (same leading shape) in the same order, or None. The
    grid's levels are the union of the tensors' level boundaries; a tensor level that spans
    several grid levels gives each of them its stride times the rows inside it."""
    per = [_row_levels(t) for t in tensors]
    if any(levels is None for levels in per):
        return None
    bounds = set()
    for levels in per:
        prod = 1
        for count, _ in reversed(levels):
            prod *= count
            bounds.add(prod)
    counts, prev = [], 1  # inner first
    for b in sorted(bounds):
        if b % prev:
            return None
        counts.append(b // prev)
        prev = b
    if len(counts) > 3:
        return None
    strides = []
    for levels in per:
        st, gi = [], 0
        for count, stride in reversed(levels):
            inside, mult = 1, 1
            while gi < len(counts) and inside * counts[gi] <= count:
                st.append(stride * mult)
                mult *= counts[gi]
                inside *= counts[gi]
                gi += 1
            if inside != count:
                return None
        strides.append(st)
    pad = 3 - len(counts)
    grid = tuple([1] * pad + counts[::-1])
    return (grid,) + tuple(tuple([0] * pad + st[::-1]) for st in strides)


def takes_kernel(x: torch.Tensor, weight: torch.Tensor, *, any_width: bool = False) -> bool:
    """Whether ``linear(x, weight)`` runs on the HIP kernel (``any_width``: whether the kernel
    can take the operands at all, whatever the routing rule says)."""
    if not (x.is_cuda and x.dtype == torch.float16 and weight.dtype == torch.float16 and weight.dim() == 2):
        return False
    k = int(x.shape[-1])
    widths = (128, 256) if any_width else _WIDTHS
    if k not in widths or int(weight.shape[1]) != k or int(weight.shape[0]) % 4:
        return False
    if not any_width and int(weight.shape[0]) > _MAX_N:
        return False
    if x.stride(-1) != 1:
        return False
    if weight.stride(-1) != 1 or weight.stride(0) % 8 or weight.data_ptr() % 16 or x.data_ptr() % 16:
        return False
    if x.numel() // k < _MIN_ROWS:
        return False
    levels = _row_levels(x)
    return levels is not None and all(st % 8 == 0 for _, st in levels)


def linear(x: torch.Tensor, weight: torch.Tensor, out: torch.Tensor | None = None, *,
           any_width: bool = False) -> torch.Tensor:
    """``F.linear(x, weight)`` (no bias) -> [..., N]; with ``out`` (a view of that shape, any
    row strides) the result is written there and ``out`` returned. ``any_width`` takes the
    kernel for every shape it can (a caller whose strided ``out`` would otherwise cost a copy)."""
    if not takes_kernel(x, weight, any_width=any_width):
        y = torch.nn.functional.linear(x, weight)
        if out is None:
            return y
        out.copy_(y)
        return out
    n = int(weight.shape[0])
    if out is None:
        out = torch.empty(tuple(x.shape[:-1]) + (n,), dtype=torch.float16, device=x.device)
    elif tuple(out.shape) != tuple(x.shape[:-1]) + (n,) or out.dtype != torch.float16 or out.device != x.device:
        raise ValueError(f"out {tuple(out.shape)} {out.dtype} is not the [..., {n}] fp16 result of x {tuple(x.shape)}")
    common = _common_grid(x, out)
    if common is None or out.stride(-1) != 1 or out.data_ptr() % 8 or any(st % 4 for st in common[2]):
        out.copy_(linear(x, weight))
        return out
    (no, nm, ni), (xo, xm, xr), (yo, ym, yr) = common
    nat.check(
        nat.lib().nori_linear_f16(
            ctypes.c_void_p(x.data_ptr()), no, nm, ni, int(x.shape[-1]), xo, xm, xr,
            ctypes.c_void_p(weight.data_ptr()), int(weight.stride(0)), n,
            ctypes.c_void_p(out.data_ptr()), yo, ym, yr, nat.stream_of(x.device),
        ),
        "linear_f16",
    )
    return out


def linear_residual_norm(a: torch.Tensor, weight: torch.Tensor, stream: torch.Tensor, alpha: float, eps: float,
                         out: torch.Tensor | None = None) -> torch.Tensor | None:
    """``stream += alpha * F.linear(a, weight)`` in place, then the RMSNorm (no weight, ``eps``)
    of the updated stream rows in fp16, in one kernel (``nori_linear_f16_residual_rms_norm``):
    bit for bit ``linear`` followed by the fused residual + norm pass. ``a`` [..., K] fp16,
    ``weight`` [K, K] fp16 (K 128 or 256), ``stream`` [..., K] fp32 with ``a``'s leading shape
    (any row strides: e.g. the [table, row, group] cells beside an attention output in
    [table, group, row] order), ``out`` the same shape in fp16 (new and laid out like
    ``stream`` when None). Returns the normalized rows, or None where the kernel does not take
    the operands (nothing is then written)."""
    k = int(a.shape[-1])
    if not (a.is_cuda and a.dtype == torch.float16 and weight.dtype == torch.float16 and stream.dtype == torch.float32
            and k in (128, 256) and tuple(weight.shape) == (k, k) and tuple(stream.shape) == tuple(a.shape)
            and stream.device == a.device and weight.device == a.device):
        return None
    if a.stride(-1) != 1 or stream.stride(-1) != 1 or weight.stride(-1) != 1:
        return None
    if out is None:
        out = torch.empty_like(stream, dtype=torch.float16)
    elif tuple(out.shape) != tuple(a.shape) or out.dtype != torch.float16 or out.stride(-1) != 1:
        return None
    common = _common_grid(a, stream, out)
    if common is None:
        return None
    (no, nm, ni), sa, sx, sy = common
    if (a.data_ptr() % 16 or any(st % 8 for st in sa) or weight.data_ptr() % 16 or weight.stride(0) % 8
            or stream.data_ptr() % 16 or any(st % 4 for st in sx) or out.data_ptr() % 8 or any(st % 4 for st in sy)):
        return None
    nat.check(
        nat.lib().nori_linear_f16_residual_rms_norm(
            ctypes.c_void_p(a.data_ptr()), no, nm, ni, k, *sa, ctypes.c_void_p(weight.data_ptr()), int(weight.stride(0)),
            float(alpha), ctypes.c_void_p(stream.data_ptr()), *sx, float(eps), ctypes.c_void_p(out.data_ptr()), *sy,
            nat.stream_of(a.device),
        ),
        "linear_f16_residual_rms_norm",
    )
    return out
