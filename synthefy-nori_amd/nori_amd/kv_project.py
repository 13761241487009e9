"""Fused context-cache write on libnori_hip.so: (RMSNorm ->) K/V projection -> int8 cache rows.

On the GPU the reference writes an int8 cross cache in three passes over HBM: the RMSNorm of
the context rows (src/synthefy_nori/model/layer.py:251-258), the K/V projection
``MultiheadAttention.project_kv_cache`` (layer.py:651-683; fp16 under the inference
autocast, predictor.py:2674) writing the fp16 K/V, and ``quantize_int8``
(kv_cache_scaling.py:29-37) reading them back to write codes and scales. ``project_quantize_kv``
is one kernel: the fp16 K/V exist only in LDS, so the HBM traffic per context row drops from
read x + write/read fp16 K/V + write codes to read x + write codes.

Semantics are those of the fp16 autocast path: operands rounded to fp16, fp32 sums, the K/V
rounded once to fp16, then the exact fp16 quantizer. The sums run in MFMA order rather than
the library GEMM's, so a K/V value can differ from torch's in its last bit and its code by one.
"""

from __future__ import annotations

import torch

from . import _native as nat
from .kv_cache_scaling import _split_strides, _vector_layout

_FLOATS = (torch.float32, torch.float16, torch.bfloat16)


def _row_view(t: torch.Tensor, lead: int) -> torch.Tensor | None:
    """``t`` with every axis after the first ``lead`` folded into one row axis, or None."""
    try:
        return t.view(*t.shape[:lead], -1)
    except RuntimeError:
        return None


def fusable(x: torch.Tensor, weight: torch.Tensor, head_dim: int) -> bool:
    """Whether ``project_quantize_kv`` takes these operands as they are (dtype, widths, alignment)."""
    if x.dtype not in _FLOATS or weight.dtype not in _FLOATS or x.device.type != "cuda" or weight.device != x.device:
        return False
    if head_dim % 4 or head_dim > 128 or x.shape[-1] != weight.shape[-1] or weight.dim() != 2 or x.shape[-1] > 1024:
        return False
    if x.stride(-1) != 1 or weight.stride(-1) != 1:
        return False
    xe, we = x.element_size(), weight.element_size()
    embed = x.shape[-1]
    if (embed * xe) % 16 or (embed * we) % 16 or x.data_ptr() % 16 or weight.data_ptr() % 16:
        return False
    return all((s * xe) % 16 == 0 for s in x.stride()[:-1]) and (weight.stride(0) * we) % 16 == 0


def project_quantize_kv(
    x: torch.Tensor,
    weight: torch.Tensor,
    kv_heads: int,
    head_dim: int,
    *,
    norm_eps: float | None = None,
    out: tuple[torch.Tensor, torch.Tensor] | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """int8 cache rows of ``x`` [..., E] under the K/V projection ``weight`` [2*kv_heads*head_dim, E].

    ``weight`` holds the K heads then the V heads (the reference's
    ``qkv_proj_weight[1:].reshape(2 * H * D, E)``); ``norm_eps`` applies an RMSNorm without
    an elementwise weight to each row first. Returns ``(codes [..., 2, kv_heads, head_dim]
    int8, scales [..., 2, kv_heads, 1] fp32)``, or fills ``out`` -- views of that shape such
    as a row slice of a preallocated cache payload -- and returns it.

    Raises:
        ValueError: on mismatched shapes or dtypes.
        NotImplementedError: for operands the kernel does not take (``fusable``).
        RuntimeError: when the kernel reports an error.
    """
    if weight.dim() != 2 or weight.shape[0] != 2 * kv_heads * head_dim:
        raise ValueError(
            f"weight {tuple(weight.shape)} is not [2 * {kv_heads} * {head_dim}, E] for {kv_heads} heads of {head_dim}"
        )
    if x.dim() < 1 or x.shape[-1] != weight.shape[1]:
        raise ValueError(f"x {tuple(x.shape)} does not end in the projection's embed width {weight.shape[1]}")
    device = nat.require_device(x, weight)
    lead = tuple(x.shape[:-1])
    if out is None:
        codes = torch.empty(lead + (2, kv_heads, head_dim), dtype=torch.int8, device=device)
        scales = torch.empty(lead + (2, kv_heads, 1), dtype=torch.float32, device=device)
    else:
        codes, scales = out
        nat.require_device(codes, scales)
        if codes.dtype != torch.int8 or scales.dtype != torch.float32:
            raise ValueError(f"out must be (int8 codes, fp32 scales), got ({codes.dtype}, {scales.dtype})")
        if tuple(codes.shape) != lead + (2, kv_heads, head_dim) or tuple(scales.shape) != lead + (2, kv_heads, 1):
            raise ValueError(
                f"out shapes {tuple(codes.shape)}/{tuple(scales.shape)} do not match rows {lead} of "
                f"2 x {kv_heads} x {head_dim}"
            )
    if not fusable(x, weight, head_dim):
        raise NotImplementedError(
            f"project_quantize_kv does not take x {x.dtype} {tuple(x.shape)} strides {x.stride()} with weight "
            f"{weight.dtype} {tuple(weight.shape)} and head_dim {head_dim} (needs 16-byte aligned rows of whole "
            "16-byte chunks, embed up to 1024 and head_dim a multiple of 4 up to 128)"
        )
    if x.numel() == 0:
        return codes, scales
    if x.dtype == torch.float32 and weight.dtype != torch.float16:
        # the kernel takes its weights as f16 (the autocast cast, round to nearest); as f16
        # they stream through the one-pass kernel's LDS at half the bytes
        weight = weight.to(torch.float16)
    _launch(x, weight, kv_heads, head_dim, norm_eps, codes, scales, device)
    return codes, scales


def _launch(x, weight, kv_heads, head_dim, norm_eps, codes, scales, device) -> None:
    lead = x.dim() - 1
    x_layout = _vector_layout(x)
    c_rows = _row_view(codes, lead)
    s_rows = _row_view(scales, lead)
    c_str = s_str = None
    if x_layout is not None and c_rows is not None and s_rows is not None:
        n_outer, n_inner = x_layout[0], x_layout[1]
        c_str = _split_strides(_vector_layout(c_rows), n_outer, n_inner)
        s_str = _split_strides(_vector_layout(s_rows), n_outer, n_inner)
    if c_str is None or s_str is None:
        if lead < 2:
            raise NotImplementedError("project_quantize_kv cannot address these output rows")
        # three or more levels of row addressing: one launch per index of the first axis
        for i in range(x.shape[0]):
            _launch(x[i], weight, kv_heads, head_dim, norm_eps, codes[i], scales[i], device)
        return
    n_outer, n_inner, x_outer, x_row = x_layout
    norm = int(norm_eps is not None)
    lib = nat.lib()
    ws_bytes = int(lib.nori_kv_project_quantize_int8_workspace_bytes(
        nat.dtype_code(x.dtype), n_outer, n_inner, x.shape[-1], norm, nat.dtype_code(weight.dtype), head_dim))
    # the f16 operand rows (torch's caching allocator keeps the buffer for the next slice)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=device) if ws_bytes > 0 else None
    nat.check(
        lib.nori_kv_project_quantize_int8(
            x.data_ptr(), nat.dtype_code(x.dtype), n_outer, n_inner, x.shape[-1], x_outer, x_row,
            norm, float(norm_eps if norm_eps is not None else 0.0),
            weight.data_ptr(), nat.dtype_code(weight.dtype), weight.stride(0), kv_heads, head_dim,
            codes.data_ptr(), c_str[0], c_str[1], scales.data_ptr(), s_str[0], s_str[1],
            nat.SCALE_DIV_RECIP, nat.ptr(ws), ws_bytes, nat.stream_of(device),
        ),
        "project_quantize_kv",
    )


class FusedKVRows:
    """A row slice of a context cache still to be projected: context rows plus the K/V weight.

    ``x`` is [B, G, n, E] (the layer's rows of the slice, batch and feature groups first); it
    stands for the projected slice [B * G, n, 2, kv_heads, head_dim] of the reference's
    ``project_kv_cache``, whose ``shape`` and ``dtype`` it reports. The cache containers'
    ``from_row_slices`` accept it in place of that slice and write its codes straight into
    their storage with ``project_quantize_kv``.
    """

    def __init__(self, x: torch.Tensor, weight: torch.Tensor, kv_heads: int, head_dim: int, norm_eps: float | None):
        if x.dim() != 4:
            raise ValueError(f"FusedKVRows takes rows [B, G, n, E], got {tuple(x.shape)}")
        self.x = x
        self.weight = weight
        self.kv_heads = int(kv_heads)
        self.head_dim = int(head_dim)
        self.norm_eps = norm_eps
        b, g, n, _ = x.shape
        self.shape = torch.Size((b * g, n, 2, self.kv_heads, self.head_dim))
        self.dtype = torch.float16
        self.device = x.device

    def _grid(self, t: torch.Tensor) -> torch.Tensor:
        return t.view(*self.x.shape[:3], *t.shape[2:])

    def quantize(self) -> tuple[torch.Tensor, torch.Tensor]:
        codes = torch.empty(self.shape, dtype=torch.int8, device=self.device)
        scales = torch.empty(tuple(self.shape[:-1]) + (1,), dtype=torch.float32, device=self.device)
        self.quantize_into(codes, scales)
        return codes, scales

    def quantize_into(self, codes: torch.Tensor, scales: torch.Tensor) -> None:
        project_quantize_kv(
            self.x, self.weight, self.kv_heads, self.head_dim, norm_eps=self.norm_eps,
            out=(self._grid(codes), self._grid(scales)),
        )


def fp16_autocast(device: torch.device) -> bool:
    """True inside ``torch.autocast`` on ``device`` with fp16 as the autocast dtype (inference on the GPU)."""
    if device.type != "cuda":
        return False
    return bool(torch.is_autocast_enabled(device.type)) and torch.get_autocast_dtype(device.type) == torch.float16
