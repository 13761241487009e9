"""GPU parity of RMSNorm (layer.py:233-258) against the oracle and torch's F.rms_norm.

Tolerance: the kernel forms the statistic in fp32 and rounds once to the dtype, so it
may differ from the float64 oracle and from torch's native kernel by one unit in the
last place of the output dtype (the reference documents 1 bf16 ulp between its own
native and decomposed variants, predictor.py:247-250). Per element:
|got - ref| <= 1 ulp(ref) of the dtype (fp32: 4 ulp, different summation order).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import nori_amd
from oracle import codec

pytestmark = pytest.mark.gpu

ULP_BITS = {torch.float32: 23, torch.float16: 10, torch.bfloat16: 7}
ULPS = {torch.float32: 4, torch.float16: 1, torch.bfloat16: 1}


def ulp(x: torch.Tensor, dtype) -> torch.Tensor:
    a = x.abs().double().clamp_min(torch.finfo(dtype).tiny)
    return torch.exp2(torch.floor(torch.log2(a)) - ULP_BITS[dtype])


def oracle(x: torch.Tensor, w: torch.Tensor | None, eps: float) -> torch.Tensor:
    c = x.cpu()
    if c.dtype == torch.bfloat16:
        raw = c.view(torch.int16).numpy().view(np.uint16)
        wr = None if w is None else w.cpu().view(torch.int16).numpy().view(np.uint16)
        out = codec.rms_norm(raw, wr, "bf16", eps)
        return torch.from_numpy(out.view(np.int16)).view(torch.bfloat16)
    name = "f32" if c.dtype == torch.float32 else "f16"
    out = codec.rms_norm(c.numpy(), None if w is None else w.cpu().numpy(), name, eps)
    return torch.from_numpy(out)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("cols", [44, 64, 128, 352, 560, 100, 3])
@pytest.mark.parametrize("affine", [False, True])
def test_rms_norm_within_one_ulp(cuda, dtype, cols, affine):
    g = torch.Generator(device=cuda).manual_seed(cols)
    x = (torch.randn(3, 37, cols, generator=g, device=cuda) * 3).to(dtype)
    w = (torch.rand(cols, generator=g, device=cuda) + 0.5).to(dtype) if affine else None
    eps = 1e-6 if affine else 1e-5
    got = nori_amd.rms_norm(x, cols, w, eps)
    assert got.dtype == dtype and got.shape == x.shape
    ref = oracle(x, w, eps).to(cuda)
    tol = ULPS[dtype] * ulp(ref, dtype) * (2 if affine else 1)
    assert torch.all((got.double() - ref.double()).abs() <= tol)
    nat = torch.nn.functional.rms_norm(x, (cols,), weight=w, eps=eps)
    assert torch.all((got.double() - nat.double()).abs() <= 2 * tol)


def test_rms_norm_module_and_strided_rows(cuda):
    m = nori_amd.RMSNorm(128, eps=1e-5).to(cuda)
    x = torch.randn(2, 300, 9, 128, device=cuda, dtype=torch.bfloat16)
    y = m(x)
    ref = torch.nn.functional.rms_norm(x, (128,), eps=1e-5)
    assert (y.float() - ref.float()).abs().max() <= 2 * 2.0**-7 * ref.float().abs().max()
    # a non-contiguous row view (the [:, :eval_pos] slices of layer.py) takes the same path
    xs = x[:, ::3]
    ys = nori_amd.rms_norm(xs, 128, None, 1e-5)
    assert torch.equal(ys, m(xs.contiguous()))
    assert nori_amd.rms_norm(torch.empty(0, 64, device=cuda), 64).shape == (0, 64)


@pytest.mark.gpu
@pytest.mark.parametrize("cols", [64, 128, 44, 352])
@pytest.mark.parametrize("out_dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("affine", [False, True])
def test_norm_written_in_the_autocast_dtype_equals_norm_then_cast(cuda, cols, out_dtype, affine):
    """nori_rms_norm_to: an fp32 row written as fp16/bf16 is bit for bit the fp32 norm cast to
    that dtype -- the operand an autocast projection would make of it (chunked path for
    whole 16-byte chunks, element-wise path for 44-wide rows)."""
    from nori_amd.norm import RMSNorm, projection_operand, rms_norm

    g = torch.Generator().manual_seed(cols)
    x = (torch.randn(1000, cols, generator=g) * 3.0).to(cuda)
    w = (1.0 + 0.3 * torch.randn(cols, generator=g)).to(cuda) if affine else None
    got = rms_norm(x, cols, w, 1e-5, out_dtype=out_dtype)
    exp = rms_norm(x, cols, w, 1e-5).to(out_dtype)
    assert got.dtype == out_dtype and torch.equal(got, exp)
    norm = RMSNorm(cols, eps=1e-5, elementwise_affine=affine).to(cuda)
    if affine:
        with torch.no_grad():
            norm.weight.copy_(w)
    with torch.autocast("cuda", dtype=out_dtype):
        op = projection_operand(norm, x)
    assert op.dtype == out_dtype and torch.equal(op, norm(x).to(out_dtype))
    assert projection_operand(norm, x).dtype == torch.float32  # no autocast: the norm itself


@pytest.mark.gpu
@pytest.mark.parametrize("udtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("n", [4096 * 33, 1001])
def test_residual_add_equals_the_torch_expression(cuda, udtype, n):
    """nori_residual_add: x + alpha * u bit for bit as torch evaluates it (the product rounded
    to u's dtype, then the fp32 sum), on the vector path (n a multiple of 4, aligned) and the
    element path (n = 1001); the in-row two-phase residual updates use it."""
    from nori_amd.norm import residual_add

    g = torch.Generator().manual_seed(n)
    x = (torch.randn(n, generator=g) * 5).to(cuda)
    u = (torch.randn(n, generator=g) * 3).to(udtype).to(cuda)
    alpha = 18 ** -0.5
    got = residual_add(x, u, alpha)
    assert torch.equal(got, x + alpha * u)
    # a strided update takes the torch expression itself
    x2 = torch.randn(64, 8, device=cuda)
    u2 = torch.randn(8, 64, device=cuda).to(udtype).t()
    assert torch.equal(residual_add(x2, u2, alpha), x2 + alpha * u2)


@pytest.mark.gpu
@pytest.mark.parametrize("udtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("out_dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("cols", [128, 256, 44, 1024])
def test_residual_add_norm_equals_the_two_calls(cuda, udtype, out_dtype, cols):
    """nori_residual_add_rms_norm: the residual update and the norm of its result in one pass
    equal nori_residual_add followed by nori_rms_norm_to bit for bit -- the stream and the
    normalized rows -- also written into a slice of a token buffer (rows in groups at two
    strides); rows past the kernel's width take the two calls."""
    from nori_amd.norm import RMSNorm, residual_add, residual_add_norm, rms_norm

    g = torch.Generator().manual_seed(cols)
    x = (torch.randn(3, 37, 4, cols, generator=g) * 5).to(cuda)
    u = (torch.randn(3, 37, 4, cols, generator=g) * 3).to(udtype).to(cuda)
    alpha = 18 ** -0.5
    norm = RMSNorm(cols, eps=1e-5)
    ref_x = residual_add(x, u, alpha)
    ref_y = rms_norm(ref_x, cols, None, 1e-5, out_dtype=out_dtype if out_dtype != torch.float32 else None)
    got_x = x.clone()
    got_y = residual_add_norm(got_x, u, alpha, norm, out_dtype=out_dtype)
    assert got_y.dtype == out_dtype
    assert torch.equal(got_x, ref_x) and torch.equal(got_y, ref_y)
    # into the first 4 of 6 token slots of a buffer
    buf = torch.full((3, 37, 6, cols), 7.0, dtype=out_dtype, device=cuda)
    got_x = x.clone()
    residual_add_norm(got_x, u, alpha, norm, out=buf[:, :, :4])
    assert torch.equal(got_x, ref_x) and torch.equal(buf[:, :, :4], ref_y) and bool((buf[:, :, 4:] == 7.0).all())
    # a transposed update (a column attention's [batch, groups, rows] output over a
    # [batch, rows, groups] stream): rows at three strides
    u_t = u.transpose(1, 2).contiguous().transpose(1, 2)
    assert not u_t.is_contiguous()
    got_x = x.clone()
    got_y = residual_add_norm(got_x, u_t, alpha, norm, out_dtype=out_dtype)
    assert torch.equal(got_x, ref_x) and torch.equal(got_y, ref_y)
    # rows wider than the kernel's 1024 elements take the two calls
    wide = RMSNorm(2 * cols + 1024, eps=1e-5)
    xw = torch.randn(5, 2 * cols + 1024, device=cuda)
    uw = torch.randn(5, 2 * cols + 1024, device=cuda).to(udtype)
    ref = rms_norm(residual_add(xw, uw, alpha), 2 * cols + 1024, None, 1e-5)
    xg = xw.clone()
    assert torch.equal(residual_add_norm(xg, uw, alpha, wide), ref)
