"""GPU parity of the fp16 projection kernel (``nori_amd.projection.linear``, csrc/linear.hip).

It replaces ``F.linear`` of fp16 operands (the reference's projections under the GPU's fp16
autocast, layer.py:651-683, 1114-1160). Bars:
  * bit-exact (``torch.equal``) with ``F.linear`` and with the float64 product rounded to fp16
    on operands whose products and sums are exact in fp32 (multiples of 1/8 and 1/64 over a
    few hundred terms), where the order of the fp32 sums cannot matter;
  * on Gaussian operands, within one fp16 rounding of the float64 product (the fp32 sums of the
    kernel and of the library GEMM may round differently in the last bit);
  * strided views -- a token subset of each row as x, a slice of a stacked buffer as the
    output -- give the same values as the contiguous call, and nothing outside the slice is
    written;
  * row counts that are not a multiple of the kernel's 256-row blocks, output widths that are
    not a multiple of its 128-column chunks, and both inner widths.
"""

from __future__ import annotations

import pytest
import torch

import ctypes

from nori_amd import _native as nat
from nori_amd import projection

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def fp32_gemm_reductions():
    # the library GEMM sums in fp32 throughout, as the kernel does
    flag = torch.backends.cuda.matmul.allow_fp16_reduced_precision_reduction
    torch.backends.cuda.matmul.allow_fp16_reduced_precision_reduction = False
    yield
    torch.backends.cuda.matmul.allow_fp16_reduced_precision_reduction = flag


def dyadic(shape, step, lim, gen, device):
    k = int(lim / step)
    return (torch.randint(-k, k + 1, shape, generator=gen) * step).to(torch.float16).to(device)


def kernel_linear(x, w):
    """The kernel itself on a contiguous [rows, k] x, whatever ``linear`` would route."""
    y = torch.empty(x.shape[0], w.shape[0], dtype=torch.float16, device=x.device)
    nat.check(nat.lib().nori_linear_f16(ctypes.c_void_p(x.data_ptr()), 1, 1, x.shape[0], x.shape[1], 0, 0, x.stride(0),
                                        ctypes.c_void_p(w.data_ptr()), w.stride(0), w.shape[0],
                                        ctypes.c_void_p(y.data_ptr()), 0, 0, y.stride(0), nat.stream_of(x.device)),
              "linear_f16")
    return y


@pytest.mark.parametrize("k", [128, 256])
@pytest.mark.parametrize("rows,n", [(4096, 128), (5000, 256), (65536 + 77, 768), (4100, 100), (8192, 36)])
def test_exact_sums_bit_exact(cuda, k, rows, n):
    g = torch.Generator().manual_seed(rows + n + k)
    x = dyadic((rows, k), 1 / 8, 4.0, g, cuda)
    w = dyadic((n, k), 1 / 64, 1.0, g, cuda)
    assert projection.takes_kernel(x, w) == (k == 128 and n <= 256)
    y = kernel_linear(x, w)
    ref = torch.nn.functional.linear(x, w)
    assert y.dtype == torch.float16 and y.shape == (rows, n)
    assert torch.equal(y, ref)
    exact = (x.double() @ w.double().t()).to(torch.float16)
    assert torch.equal(y, exact)


@pytest.mark.parametrize("k", [128, 256])
def test_gaussian_within_one_rounding(cuda, k):
    g = torch.Generator(device=cuda).manual_seed(5 + k)
    x = torch.randn(300_001, k, generator=g, device=cuda).to(torch.float16)
    w = (torch.randn(384, k, generator=g, device=cuda) / k ** 0.5).to(torch.float16)
    y = kernel_linear(x, w)
    exact = x.double() @ w.double().t()
    # |y - exact| <= half an fp16 ulp of exact plus the fp32 summation error (k terms, each
    # partial sum rounded: at most k * 2^-24 * sum |x w|)
    ulp = torch.clamp(exact.abs(), min=2.0 ** -14).log2().floor().exp2() * 2.0 ** -10
    mag = x.double().abs() @ w.double().abs().t()
    err = (y.double() - exact).abs()
    assert bool((err <= 0.5 * ulp + k * 2.0 ** -24 * mag).all())
    # against the library GEMM: both within that bound of the exact product, so within twice it
    # of each other (near zero the fp32 sums' rounding exceeds an fp16 ulp of the result)
    lib = torch.nn.functional.linear(x, w)
    diff = (y.double() - lib.double()).abs()
    print(f"[parity] linear_f16 k={k}: {float((diff > 0).float().mean()):.2e} of outputs differ from F.linear, "
          f"{float((diff > ulp).float().mean()):.2e} by more than an fp16 ulp", flush=True)
    assert bool((diff <= ulp + 2 * k * 2.0 ** -24 * mag).all())


def test_strided_views_in_place(cuda):
    # the two-phase feature attention's operands: rows of 6 tokens, x the first 4 tokens of each
    # row, the output a slice of a stacked [row, token, 768] buffer
    g = torch.Generator(device=cuda).manual_seed(9)
    tokens = torch.randn(3000, 6, 128, generator=g, device=cuda).to(torch.float16)
    w = (torch.randn(640, 128, generator=g, device=cuda) / 11.3).to(torch.float16)
    cells = tokens[:, :4]
    assert projection.takes_kernel(cells, w[:256])
    buf = torch.full((3000, 6, 768), 7.0, dtype=torch.float16, device=cuda)
    out = buf[:, :4, :256]
    assert projection.linear(cells, w[:256], out=out) is out
    ref = kernel_linear(cells.contiguous().view(-1, 128), w[:256]).view(3000, 4, 256)
    assert torch.equal(out, ref)
    assert bool((buf[:, :4, 256:] == 7.0).all()) and bool((buf[:, 4:] == 7.0).all())
    # a token subset as x with a contiguous result, and a column slice of a 3-D view as out
    targets = tokens[:, 4:]
    assert projection.takes_kernel(targets, w[:128])
    assert torch.equal(projection.linear(targets, w[:128]), projection.linear(targets.contiguous(), w[:128]))
    q = buf[:, 4:, 640:]
    projection.linear(targets, w[512:], out=q)
    assert torch.equal(q, kernel_linear(targets.contiguous().view(-1, 128), w[512:]).view(3000, 2, 128))
    # wider outputs go to the library GEMM; out= still lands in the slice
    wide = buf[:, :4, :640]
    projection.linear(cells, w, out=wide)
    assert torch.equal(wide, torch.nn.functional.linear(cells, w))


def test_transposed_cell_view(cuda):
    # the column attention's operands: cells [table, row, group, width] read as the transposed
    # [table, group, row] view (three row levels), and its first rows as the K/V operand
    g = torch.Generator(device=cuda).manual_seed(12)
    cells = torch.randn(40, 320, 4, 128, generator=g, device=cuda).to(torch.float16)
    cols = cells.transpose(1, 2)
    w = (torch.randn(256, 128, generator=g, device=cuda) / 11.3).to(torch.float16)
    for x in (cols, cols[:, :, :256]):
        assert projection.takes_kernel(x, w)
        y = projection.linear(x, w)
        assert y.is_contiguous() and y.shape == x.shape[:-1] + (256,)
        assert torch.equal(y, kernel_linear(x.contiguous().view(-1, 128), w).view(y.shape))


def test_falls_back_where_the_kernel_does_not_apply(cuda):
    g = torch.Generator(device=cuda).manual_seed(1)
    small = torch.randn(100, 128, generator=g, device=cuda).to(torch.float16)
    odd_k = torch.randn(8192, 96, generator=g, device=cuda).to(torch.float16)
    fp32 = torch.randn(8192, 128, generator=g, device=cuda)
    w = torch.randn(64, 128, generator=g, device=cuda).to(torch.float16)
    assert not projection.takes_kernel(small, w)
    assert not projection.takes_kernel(odd_k, torch.randn(64, 96, device=cuda).to(torch.float16))
    assert not projection.takes_kernel(fp32, w.float())
    assert torch.equal(projection.linear(small, w), torch.nn.functional.linear(small, w))
