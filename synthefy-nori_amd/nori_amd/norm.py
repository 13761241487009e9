"""Row-wise kernels of libnori_hip.so around the attention: RMSNorm (drop-in for ``RMSNorm``,
src/synthefy_nori/model/layer.py:233-258), the deep-norm residual update and the SwiGLU gate."""

from __future__ import annotations

import ctypes

import torch
import torch.nn as nn

from . import _native as nat


def _strided_rows(t: torch.Tensor, cols: int) -> tuple[int, int] | None:
    """(rows, row stride) when ``t``'s rows of ``cols`` contiguous elements sit at one stride."""
    if t.stride(-1) != 1 or (t.dim() > 1 and t.shape[-1] != cols):
        return None
    lead = [(n, st) for n, st in zip(t.shape[:-1], t.stride()[:-1]) if n != 1]
    if not lead:
        return 1, cols
    for (n_outer, s_outer), (n_inner, s_inner) in zip(lead, lead[1:]):
        if s_outer != n_inner * s_inner:
            return None
    rows = 1
    for n, _ in lead:
        rows *= n
    return rows, lead[-1][1]


def rms_norm_(x: torch.Tensor, weight: torch.Tensor | None = None, eps: float = 1e-5) -> torch.Tensor:
    """In-place ``rms_norm`` over the last axis of a row view, e.g. the K half of a projected
    [..., 2, H, D] K/V tensor taken one head at a time: rows of D contiguous elements at one
    stride. Each row is read whole before it is written."""
    if x.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise NotImplementedError(f"rms_norm takes float32/float16/bfloat16, got {x.dtype}")
    device = nat.require_device(x, weight)
    cols = int(x.shape[-1])
    layout = _strided_rows(x, cols)
    if layout is None:
        raise ValueError(f"rms_norm_ needs rows at one stride, got shape {tuple(x.shape)} strides {x.stride()}")
    rows, stride = layout
    w = None if weight is None else weight.reshape(cols).contiguous()
    if x.numel() == 0:
        return x
    nat.check(
        nat.lib().nori_rms_norm(
            x.data_ptr(), nat.dtype_code(x.dtype), rows, cols, stride,
            nat.ptr(w), nat.dtype_code(w.dtype) if w is not None else nat.NORI_F32, float(eps),
            x.data_ptr(), stride, nat.stream_of(device),
        ),
        "rms_norm",
    )
    return x


def rms_norm(
    x: torch.Tensor, normalized_shape, weight: torch.Tensor | None = None, eps: float = 1e-5, *,
    out_dtype: torch.dtype | None = None, out: torch.Tensor | None = None,
) -> torch.Tensor:
    """x * rsqrt(mean(x^2) + eps) (* weight) over the trailing ``normalized_shape`` axes.

    The native ``F.rms_norm`` semantics (layer.py:253): statistic and product in fp32,
    one rounding to x's dtype, then the weight multiply. ``out_dtype`` (fp16 or bf16, for an
    fp32 ``x``) writes that result rounded once more to ``out_dtype``: the value
    ``rms_norm(x).to(out_dtype)`` has, in one pass. ``out`` (x's shape, rows at one stride, its
    dtype the output dtype) receives the rows in place of a new tensor -- e.g. a slice of a
    buffer that stacks several normalized operands.
    """
    if out is not None:
        return _rms_norm_into(x, normalized_shape, weight, eps, out)
    if isinstance(normalized_shape, int):
        normalized_shape = (normalized_shape,)
    normalized_shape = tuple(normalized_shape)
    if tuple(x.shape[-len(normalized_shape):]) != normalized_shape:
        raise ValueError(f"input {tuple(x.shape)} does not end in normalized_shape {normalized_shape}")
    if x.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise NotImplementedError(f"rms_norm takes float32/float16/bfloat16, got {x.dtype}")
    device = nat.require_device(x, weight)
    cols = 1
    for s in normalized_shape:
        cols *= int(s)
    x2 = x.reshape(-1, cols)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    rows = x2.shape[0]
    out_dtype = x.dtype if out_dtype is None else out_dtype
    y = torch.empty((rows, cols), dtype=out_dtype, device=device)
    w = None
    if weight is not None:
        w = weight.reshape(cols)
        if not w.is_contiguous():
            w = w.contiguous()
    nat.check(
        nat.lib().nori_rms_norm_to(
            x2.data_ptr(), nat.dtype_code(x.dtype), rows, cols, x2.stride(0),
            nat.ptr(w), nat.dtype_code(w.dtype) if w is not None else nat.NORI_F32, float(eps),
            y.data_ptr(), nat.dtype_code(out_dtype), y.stride(0), nat.stream_of(device),
        ),
        "rms_norm",
    )
    return y.reshape(x.shape)


def _rms_norm_into(x, normalized_shape, weight, eps, out):
    cols = 1
    for n in (normalized_shape,) if isinstance(normalized_shape, int) else normalized_shape:
        cols *= int(n)
    if tuple(out.shape) != tuple(x.shape):
        raise ValueError(f"rms_norm out {tuple(out.shape)} does not match x {tuple(x.shape)}")
    device = nat.require_device(x, weight, out)
    src = _strided_rows(x, cols)
    if src is None:
        x = x.contiguous()
        src = _strided_rows(x, cols)
    dst = _strided_rows(out, cols)
    if dst is None or dst[0] != src[0]:
        raise ValueError(f"rms_norm out needs rows of {cols} at one stride, got strides {out.stride()}")
    w = None if weight is None else weight.reshape(cols).contiguous()
    if x.numel():
        nat.check(
            nat.lib().nori_rms_norm_to(
                x.data_ptr(), nat.dtype_code(x.dtype), src[0], cols, src[1],
                nat.ptr(w), nat.dtype_code(w.dtype) if w is not None else nat.NORI_F32, float(eps),
                out.data_ptr(), nat.dtype_code(out.dtype), dst[1], nat.stream_of(device),
            ),
            "rms_norm",
        )
    return out


def operand_dtype(x: torch.Tensor) -> torch.dtype:
    """The dtype a projection of ``x`` computes in: the autocast dtype for an fp32 ``x`` under
    fp16/bf16 autocast on the GPU, else x's own."""
    if x.dtype == torch.float32 and x.is_cuda and torch.is_autocast_enabled("cuda"):
        dt = torch.get_autocast_dtype("cuda")
        if dt in (torch.float16, torch.bfloat16):
            return dt
    return x.dtype


def projection_operand(norm: "RMSNorm", x: torch.Tensor) -> torch.Tensor:
    """``norm(x)`` for a caller that only feeds it to projections (F.linear / nn.Linear).

    Under fp16 or bf16 autocast on the GPU, such a projection casts the norm's fp32 output to
    the autocast dtype before its GEMM; here the norm kernel writes that rounded value
    directly (bit for bit the same operand), saving the fp32 write and the cast's read and
    write. Elsewhere it is ``norm(x)``.
    """
    if isinstance(norm, RMSNorm) and x.dtype == torch.float32 and x.is_cuda and torch.is_autocast_enabled("cuda"):
        dt = torch.get_autocast_dtype("cuda")
        if dt in (torch.float16, torch.bfloat16):
            return rms_norm(x, norm.normalized_shape, norm.weight, norm.eps, out_dtype=dt)
    return norm(x)


class RMSNorm(nn.Module):
    """RMSNorm with the reference constructor and state dict (layer.py:233-258), computed by HIP."""

    def __init__(self, normalized_shape, eps=1e-5, elementwise_affine=False, device=None, dtype=None):
        super().__init__()
        if isinstance(normalized_shape, int):
            normalized_shape = (normalized_shape,)
        self.normalized_shape = tuple(normalized_shape)
        self.eps = eps
        self.elementwise_affine = elementwise_affine
        self.use_native = True
        if elementwise_affine:
            self.weight = nn.Parameter(torch.ones(self.normalized_shape, device=device, dtype=dtype))
        else:
            self.register_parameter("weight", None)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return rms_norm(x, self.normalized_shape, self.weight, self.eps)


def residual_add(x: torch.Tensor, u: torch.Tensor, alpha: float, *, inplace: bool = False) -> torch.Tensor:
    """``x + alpha * u`` for an fp32 residual stream and a sublayer output of the same shape, in
    one pass on the GPU (``nori_residual_add``) with torch's rounding: ``alpha * u`` formed in
    fp32 and rounded to u's dtype, then the fp32 sum. ``inplace`` writes the sum over x (same
    values). Other operands take the torch expression."""
    if not (
        x.is_cuda and x.dtype == torch.float32 and u.dtype in (torch.float32, torch.float16, torch.bfloat16)
        and u.device == x.device and tuple(u.shape) == tuple(x.shape) and x.is_contiguous() and u.is_contiguous()
    ):
        if inplace:
            return x.add_(alpha * u)
        return x + alpha * u
    out = x if inplace else torch.empty_like(x)
    nat.check(
        nat.lib().nori_residual_add(
            x.data_ptr(), u.data_ptr(), nat.dtype_code(u.dtype), float(alpha), x.numel(), out.data_ptr(),
            nat.stream_of(x.device),
        ),
        "residual_add",
    )
    return out


def _grouped_rows(t: torch.Tensor, cols: int) -> tuple[int, int, int, int] | None:
    """(rows, group, group stride, row stride) when ``t``'s rows of ``cols`` contiguous elements
    sit in groups of ``group`` rows at one stride, the groups at another -- e.g. a slice
    [B, n, g, cols] of a [B, n, g + k, cols] token buffer -- or None."""
    if t.stride(-1) != 1 or t.shape[-1] != cols:
        return None
    lead = [(n, st) for n, st in zip(t.shape[:-1], t.stride()[:-1]) if n != 1]
    if not lead:
        return 1, 1, cols, cols

    def consistent(dims):
        return all(so == ni * si for (_, so), (ni, si) in zip(dims, dims[1:]))

    split = len(lead) - 1
    while split > 0 and consistent(lead[split - 1:]):
        split -= 1
    inner, outer = lead[split:], lead[:split]
    if not consistent(outer):
        return None
    group = 1
    for n, _ in inner:
        group *= n
    rows = group
    for n, _ in outer:
        rows *= n
    return rows, group, (outer[-1][1] if outer else group * inner[-1][1]), inner[-1][1]


def _row_levels(t: torch.Tensor) -> tuple[int, int, int, int, int] | None:
    """(d1, d2, s0, s1, s2) such that row r = (i0 * d1 + i1) * d2 + i2 of ``t`` (rows over its
    leading axes in order, each of its last axis' contiguous elements) starts at element
    i0 * s0 + i1 * s1 + i2 * s2 -- at most three row levels after merging axes that follow each
    other in memory -- or None."""
    if t.stride(-1) != 1:
        return None
    dims = []
    for n, st in zip(t.shape[:-1], t.stride()[:-1]):
        if n == 1:
            continue
        if dims and dims[-1][1] == n * st:
            dims[-1] = (dims[-1][0] * n, st)
        else:
            dims.append((n, st))
    if len(dims) > 3:
        return None
    dims = [(1, 0)] * (3 - len(dims)) + dims
    return dims[1][0], dims[2][0], dims[0][1], dims[1][1], dims[2][1]


def residual_add_norm(x: torch.Tensor, u: torch.Tensor, alpha: float, norm: "RMSNorm", *,
                      out_dtype: torch.dtype | None = None, out: torch.Tensor | None = None,
                      x_out: torch.Tensor | None = None) -> torch.Tensor:
    """``x += alpha * u`` in place (``residual_add``'s rounding), then ``norm`` of the updated x,
    in one HIP pass (``nori_residual_add_rms_norm``), bit for bit the two separate calls.
    ``x_out`` (contiguous fp32, x's shape) takes the sum instead of x, which is then left as
    it is.

    ``norm`` is an ``RMSNorm`` without weight over x's trailing width. The result is written in
    ``out_dtype`` (default x's; a projection operand under autocast passes ``operand_dtype(x)``,
    the value ``projection_operand`` gives) or into ``out`` (x's shape, rows in groups at two
    strides -- e.g. a slice of a token buffer). Operands the kernel does not take (non-fp32 or
    non-contiguous streams, a norm with a weight, rows past 1024 elements) run the two calls.
    """
    ns = tuple(norm.normalized_shape)
    cols = 1
    for n in ns:
        cols *= int(n)
    dt = (out.dtype if out is not None else (x.dtype if out_dtype is None else out_dtype))
    xo = x if x_out is None else x_out
    fused = (
        isinstance(norm, RMSNorm) and norm.weight is None and x.is_cuda and x.dtype == torch.float32
        and x.is_contiguous() and tuple(u.shape) == tuple(x.shape) and u.device == x.device
        and xo.dtype == torch.float32 and xo.is_contiguous() and tuple(xo.shape) == tuple(x.shape)
        and u.dtype in (torch.float32, torch.float16, torch.bfloat16) and dt in (torch.float32, torch.float16, torch.bfloat16)
        and tuple(x.shape[-len(ns):]) == ns and cols % 4 == 0 and cols <= 1024
    )
    u_levels = None if not fused or u.is_contiguous() else _row_levels(u)
    if fused and (u.is_contiguous() or u_levels is not None):
        y = out if out is not None else torch.empty(x.shape, dtype=dt, device=x.device)
        layout = _grouped_rows(y, cols) if out is not None else (x.numel() // cols, 1, cols, cols)
        if layout is not None and layout[0] == x.numel() // cols:
            rows, group, gstride, rstride = layout
            levels = None if u_levels is None else (ctypes.c_int64 * 5)(*u_levels)
            rc = nat.lib().nori_residual_add_rms_norm(
                x.data_ptr(), u.data_ptr(), nat.dtype_code(u.dtype), levels, float(alpha), rows, cols,
                float(norm.eps), xo.data_ptr(), y.data_ptr(), nat.dtype_code(dt), group, gstride, rstride,
                nat.stream_of(x.device),
            )
            if rc == nat.NORI_OK:
                return y
            if rc != nat.NORI_ERR_UNSUPPORTED:
                nat.check(rc, "residual_add_rms_norm")
    if x_out is None:
        residual_add(x, u, alpha, inplace=True)
    else:
        x_out.copy_(residual_add(x, u, alpha))
        x = x_out
    if out is None:
        if dt == x.dtype:
            return norm(x)
        return rms_norm(x, ns, None, norm.eps, out_dtype=dt)
    if _strided_rows(out, cols) is not None:
        return rms_norm(x, ns, None, norm.eps, out=out)
    for j in range(out.shape[-2]):  # rows at two strides: one call per index of the group axis
        rms_norm(x[..., j, :], ns, None, norm.eps, out=out[..., j, :])
    return out


def layer_norm(
    x: torch.Tensor,
    weight: torch.Tensor | None,
    bias: torch.Tensor | None,
    eps: float,
    relu: bool = False,
    out_dtype: torch.dtype | None = None,
) -> torch.Tensor:
    """``F.layer_norm`` over the last axis (then ``relu`` when asked) in one HIP pass
    (``nori_layer_norm``): fp32 statistics and affine, the result rounded once to
    ``out_dtype`` (default: x's dtype) -- under fp16 autocast the fp16 operand of the F.linear
    that follows (ref encoders.py:118-276, 432-585)."""
    cols = x.shape[-1]
    out_dtype = out_dtype or x.dtype
    device = nat.require_device(x)
    x2 = x.reshape(-1, cols)
    if x2.stride(-1) != 1 or x2.stride(0) % 4 or x2.data_ptr() % (4 * x2.element_size()):
        x2 = x2.contiguous()
    w = None if weight is None else weight.detach().to(device=device, dtype=torch.float32).contiguous()
    b = None if bias is None else bias.detach().to(device=device, dtype=torch.float32).contiguous()
    out = torch.empty((x2.shape[0], cols), dtype=out_dtype, device=device)
    nat.check(
        nat.lib().nori_layer_norm(
            x2.data_ptr(), nat.dtype_code(x.dtype), x2.shape[0], cols, x2.stride(0),
            None if w is None else w.data_ptr(), None if b is None else b.data_ptr(), float(eps), int(relu),
            out.data_ptr(), nat.dtype_code(out_dtype), cols, nat.stream_of(device),
        ),
        "layer_norm",
    )
    return out.view(*x.shape[:-1], cols)


# Widths (in = out features) the fused SwiGLU kernel is built for.
FUSED_MLP_WIDTHS = (128, 256, 352)


def swiglu_mlp(x: torch.Tensor, gate_up: torch.Tensor, down: torch.Tensor, hidden: int) -> torch.Tensor:
    """The whole fp16 SwiGLU feed-forward ``(silu(x Wg^T) * (x Wu^T)) Wd^T`` in one HIP kernel
    (``nori_swiglu_mlp``): ``gate_up`` [2 * hidden, width] (gate rows, then up rows) and
    ``down`` [width, hidden], fp16 and contiguous, ``hidden`` padded to a multiple of 32 with
    zero rows/columns; x [..., width] fp16 with width in FUSED_MLP_WIDTHS. SwiGLUMLP.forward
    under fp16 autocast (layer.py:261-274) without writing the hidden activations out."""
    width = x.shape[-1]
    if gate_up.shape != (2 * hidden, width) or down.shape != (width, hidden):
        raise ValueError(
            f"swiglu_mlp: weights {tuple(gate_up.shape)} / {tuple(down.shape)} do not match width {width}, hidden {hidden}"
        )
    device = nat.require_device(x, gate_up, down)
    x2 = x.reshape(-1, width)
    if x2.stride(-1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    gate_up, down = gate_up.contiguous(), down.contiguous()
    out = torch.empty((x2.shape[0], width), dtype=x.dtype, device=device)
    nat.check(
        nat.lib().nori_swiglu_mlp(
            x2.data_ptr(), nat.dtype_code(x.dtype), x2.shape[0], width, x2.stride(0), gate_up.data_ptr(),
            down.data_ptr(), hidden, out.data_ptr(), width, nat.stream_of(device),
        ),
        "swiglu_mlp",
    )
    return out.view(*x.shape[:-1], width)


def swiglu_mlp_residual_norm(x: torch.Tensor, gate_up: torch.Tensor, down: torch.Tensor, hidden: int,
                             stream: torch.Tensor, alpha: float, eps: float, norm_width: int,
                             out: torch.Tensor | None = None) -> torch.Tensor | None:
    """``stream += alpha * swiglu_mlp(x, ...)`` in place, then the RMSNorm (no weight, ``eps``)
    of every ``norm_width`` columns of the updated stream rows in fp16, in one kernel
    (``nori_swiglu_mlp_residual_rms_norm``), bit for bit ``swiglu_mlp`` followed by
    ``residual_add_norm``. x [..., width] fp16; stream fp32, contiguous, holding x's rows of
    width columns (its last axis ``norm_width``); ``out`` fp16 in stream's shape (any two-level
    row layout ``residual_add_norm`` takes, e.g. a slice of a token buffer), new and contiguous
    when None. Returns the normalized rows, or None where the kernel does not take the operands
    (nothing is then written)."""
    width = int(x.shape[-1])
    if not (x.is_cuda and x.dtype == torch.float16 and stream.dtype == torch.float32 and stream.is_contiguous()
            and stream.device == x.device and stream.numel() == x.numel() and stream.shape[-1] == norm_width
            and (width, norm_width) in ((128, 128), (256, 128), (256, 256))
            and gate_up.shape == (2 * hidden, width) and down.shape == (width, hidden)):
        return None
    x2 = x.reshape(-1, width)
    if x2.stride(-1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16 or stream.data_ptr() % 16:
        return None
    rows = x2.shape[0]
    groups = rows * (width // norm_width)
    if out is None:
        out = torch.empty(stream.shape, dtype=torch.float16, device=x.device)
    if out.dtype != torch.float16 or out.numel() != stream.numel() or out.shape[-1] != norm_width:
        return None
    layout = _grouped_rows(out, norm_width)
    if layout is None or layout[0] != groups or out.data_ptr() % 8:
        return None
    _, group, gstride, rstride = layout
    nat.check(
        nat.lib().nori_swiglu_mlp_residual_rms_norm(
            x2.data_ptr(), nat.NORI_F16, rows, width, x2.stride(0), gate_up.contiguous().data_ptr(),
            down.contiguous().data_ptr(), hidden, float(alpha), stream.data_ptr(), width, norm_width, float(eps),
            out.data_ptr(), group, gstride, rstride, nat.stream_of(x.device),
        ),
        "swiglu_mlp_residual_rms_norm",
    )
    return out


QASS_GATE_HIDDEN = 64


def qass_gate(q: torch.Tensor, w1: torch.Tensor, b1: torch.Tensor, w2: torch.Tensor, b2: torch.Tensor,
              base_scale: torch.Tensor) -> torch.Tensor:
    """QASS "full" scaling ``q * base_scale * (1 + tanh(gate_mlp(q)))`` in one HIP pass
    (``nori_qass_gate``): q [..., H, D] fp16, the gate MLP's weights w1 [64, D], b1 [64], w2
    [D, 64], b2 [D] and base_scale [H, D], all fp16. QASSMaxScaling.forward under fp16
    autocast (layer.py:316-456), with each op's fp16 rounding."""
    h, d = q.shape[-2], q.shape[-1]
    if w1.shape != (QASS_GATE_HIDDEN, d) or w2.shape != (d, QASS_GATE_HIDDEN) or b1.shape != (QASS_GATE_HIDDEN,) \
            or b2.shape != (d,) or base_scale.numel() != h * d:
        raise ValueError(f"qass_gate: weights do not match {h} heads of {d}")
    device = nat.require_device(q, w1, b1, w2, b2, base_scale)
    q3 = q.reshape(-1, h, d)
    if q3.stride(-1) != 1 or q3.stride(-2) != d or q3.stride(0) % 4 or q3.data_ptr() % 8:
        q3 = q3.contiguous()
    w1, b1, w2, b2 = w1.contiguous(), b1.contiguous(), w2.contiguous(), b2.contiguous()
    bs = base_scale.reshape(h, d).contiguous()
    out = torch.empty((q3.shape[0], h, d), dtype=q.dtype, device=device)
    nat.check(
        nat.lib().nori_qass_gate(
            q3.data_ptr(), nat.dtype_code(q.dtype), q3.shape[0], h, d, q3.stride(0), w1.data_ptr(), b1.data_ptr(),
            w2.data_ptr(), b2.data_ptr(), QASS_GATE_HIDDEN, bs.data_ptr(), out.data_ptr(), h * d, nat.stream_of(device),
        ),
        "qass_gate",
    )
    return out.view(q.shape)


def silu_mul(gu: torch.Tensor, hidden: int) -> torch.Tensor:
    """``F.silu(gu[..., :hidden]) * gu[..., hidden:]`` for the [gate | up] output of a stacked
    projection, in gu's dtype with torch's rounding of the two ops, one HIP pass
    (``nori_silu_mul``). SwiGLUMLP.forward's gate (layer.py:261-274)."""
    if gu.shape[-1] != 2 * hidden:
        raise ValueError(f"silu_mul expects the [gate | up] width {2 * hidden}, got {gu.shape[-1]}")
    device = nat.require_device(gu)
    g2 = gu.reshape(-1, 2 * hidden)
    if g2.stride(-1) != 1:
        g2 = g2.contiguous()
    out = torch.empty((g2.shape[0], hidden), dtype=gu.dtype, device=device)
    nat.check(
        nat.lib().nori_silu_mul(
            g2.data_ptr(), nat.dtype_code(gu.dtype), g2.shape[0], hidden, g2.stride(0), out.data_ptr(), hidden,
            nat.stream_of(device),
        ),
        "silu_mul",
    )
    return out.view(*gu.shape[:-1], hidden)
