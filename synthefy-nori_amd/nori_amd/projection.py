"""Projections of the attention sublayers: ``F.linear`` under fp16 autocast on the HIP kernel.

``linear(x, weight)`` is ``torch.nn.functional.linear(x, weight)`` for fp16 operands (what the
reference's projections compute under the GPU's fp16 autocast, layer.py:651-683, 1114-1160):
fp32 sums of fp16 products, rounded once to fp16. ``nori_linear_f16`` (csrc/linear.hip) reads
x and writes the output through strides -- a token subset of each row, or a slice of a stacked
output buffer (``out``) -- without copies. ``linear`` routes to it the shapes where it is the
faster of the two (same-box A/B against the library GEMM: inner width 128 and up to 256 output
columns, e.g. 655,360 rows x 128 -> 128 in 78 against 110 us; at inner width 256 or wider
outputs the library GEMM was as fast or faster); everything else (other dtypes, widths or
shapes, short operands, CPU tensors) is ``F.linear``. The two differ only in the order of the
fp32 sums.
"""

from __future__ import annotations

import ctypes

import torch

from . import _native as nat

__all__ = ["linear", "takes_kernel"]

_WIDTHS = (128,)  # inner widths routed to the kernel (it also takes 256, where the library GEMM was faster)
_MAX_N = 256      # output widths up to this (past it the library GEMM was as fast or faster)
_MIN_ROWS = 4096  # below this the library GEMM's launch is as cheap


def _row_levels(t: torch.Tensor) -> list[tuple[int, int]] | None:
    """The rows of ``t`` [..., C] as at most two (count, stride) levels, outer first (adjacent
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
    if len(merged) > 2:
        return None
    return merged


def _common_grid(x: torch.Tensor, y: torch.Tensor) -> tuple[int, int, int, int, int, int] | None:
    """(n_outer, n_inner, x outer stride, x row stride, y outer stride, y row stride): one
    two-level row grid addressing the rows of x and of y (same leading shape) in the same
    order, or None."""
    lx, ly = _row_levels(x), _row_levels(y)
    if lx is None or ly is None:
        return None
    rows = x.numel() // max(int(x.shape[-1]), 1)
    grid = lx if len(lx) == 2 else (ly if len(ly) == 2 else [(1, 0), (rows, lx[0][1] if lx else 0)])
    outer, inner = grid[0][0], grid[1][0]

    def on_grid(levels):
        if len(levels) == 2:
            return (levels[0][1], levels[1][1]) if (levels[0][0], levels[1][0]) == (outer, inner) else None
        stride = levels[0][1] if levels else 0
        return inner * stride, stride

    gx, gy = on_grid(lx), on_grid(ly)
    if gx is None or gy is None:
        return None
    return outer, inner, gx[0], gx[1], gy[0], gy[1]


def takes_kernel(x: torch.Tensor, weight: torch.Tensor) -> bool:
    """Whether ``linear(x, weight)`` runs on the HIP kernel."""
    if not (x.is_cuda and x.dtype == torch.float16 and weight.dtype == torch.float16 and weight.dim() == 2):
        return False
    k = int(x.shape[-1])
    if k not in _WIDTHS or int(weight.shape[1]) != k or int(weight.shape[0]) % 4 or int(weight.shape[0]) > _MAX_N:
        return False
    if x.stride(-1) != 1:
        return False
    if weight.stride(-1) != 1 or weight.stride(0) % 8 or weight.data_ptr() % 16 or x.data_ptr() % 16:
        return False
    if x.numel() // k < _MIN_ROWS:
        return False
    levels = _row_levels(x)
    return levels is not None and all(st % 8 == 0 for _, st in levels)


def linear(x: torch.Tensor, weight: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """``F.linear(x, weight)`` (no bias) -> [..., N]; with ``out`` (a view of that shape, any
    row strides) the result is written there and ``out`` returned."""
    if not takes_kernel(x, weight):
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
    grid = _common_grid(x, out)
    if grid is None or out.stride(-1) != 1 or out.data_ptr() % 8 or grid[4] % 4 or grid[5] % 4:
        out.copy_(linear(x, weight))
        return out
    nat.check(
        nat.lib().nori_linear_f16(
            ctypes.c_void_p(x.data_ptr()), grid[0], grid[1], int(x.shape[-1]), grid[2], grid[3],
            ctypes.c_void_p(weight.data_ptr()), int(weight.stride(0)), n,
            ctypes.c_void_p(out.data_ptr()), grid[4], grid[5], nat.stream_of(x.device),
        ),
        "linear_f16",
    )
    return out
