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


# ---------------------------------------------------------------- projection + residual + norm
# ``projection.linear_residual_norm`` (nori_linear_f16_residual_rms_norm) replaces the output
# projection of an attention sublayer followed by the deep-norm residual update and the next
# RMSNorm (reference two_phase.py:198, 209, 220-225, 264, 271-272; layer.py:251-253). Bars:
#   * bit-exact (stream and normalized rows) against the projection kernel followed by the
#     fused residual + norm kernel, which the norm tests pin to torch;
#   * the stream bit-exact against torch's own expression ``x + alpha * u`` on the same u, the
#     normalized rows within one fp16 ulp of ``F.rms_norm`` (the order of the fp32 sum of
#     squares differs).

ALPHA = 0.20412415  # (12 + 12) ** -0.5, a deep-norm alpha


def separate_passes(a, w, x, alpha, eps):
    from nori_amd.norm import RMSNorm, residual_add_norm

    k = a.shape[-1]
    u = kernel_linear(a.contiguous().view(-1, k), w).view(a.shape)
    xr = x.clone()
    y = residual_add_norm(xr, u, alpha, RMSNorm(k, eps=eps), out_dtype=torch.float16)
    return u, xr, y


@pytest.mark.parametrize("k", [128, 256])
@pytest.mark.parametrize("rows", [256, 4097, 70_001])
def test_residual_norm_equals_the_separate_passes(cuda, k, rows):
    g = torch.Generator(device=cuda).manual_seed(rows + k)
    a = torch.randn(rows, k, generator=g, device=cuda).to(torch.float16)
    w = (torch.randn(k, k, generator=g, device=cuda) / k ** 0.5).to(torch.float16)
    x = torch.randn(rows, k, generator=g, device=cuda) * 3.0
    u, x_ref, y_ref = separate_passes(a, w, x, ALPHA, 1e-5)
    xs = x.clone()
    y = projection.linear_residual_norm(a, w, xs, ALPHA, 1e-5)
    assert y is not None and y.dtype == torch.float16 and y.shape == (rows, k)
    assert torch.equal(xs, x_ref)
    assert torch.equal(y, y_ref)
    # torch's expression on the same u: fp16 u * alpha rounded to fp16, added to the fp32 stream
    assert torch.equal(xs, x + ALPHA * u)
    ref = torch.nn.functional.rms_norm(x + ALPHA * u, (k,), None, 1e-5)
    ulp = torch.clamp(ref.abs(), min=2.0 ** -14).log2().floor().exp2() * 2.0 ** -10
    assert bool(((y.float() - ref).abs() <= ulp).all())


def test_residual_norm_rows_in_another_order(cuda):
    # the column attention: its output in [table, group, row] order, the cell stream in
    # [table, row, group] order, the normalized cells written in the stream's layout
    g = torch.Generator(device=cuda).manual_seed(3)
    b, n, gr, k = 5, 700, 4, 128
    cells = torch.randn(b, n, gr, k, generator=g, device=cuda) * 2.0
    atten = torch.randn(b, gr, n, k, generator=g, device=cuda).to(torch.float16)
    w = (torch.randn(k, k, generator=g, device=cuda) / 11.3).to(torch.float16)
    a = atten.transpose(1, 2)
    _, x_ref, y_ref = separate_passes(a, w, cells, ALPHA, 1e-5)
    xs = cells.clone()
    y = projection.linear_residual_norm(a, w, xs, ALPHA, 1e-5)
    assert y.is_contiguous() and y.shape == cells.shape
    assert torch.equal(xs, x_ref) and torch.equal(y, y_ref)
    # the same through a transposed view of the stream: the output follows the stream's layout
    xs = cells.clone()
    yt = projection.linear_residual_norm(atten, w, xs.transpose(1, 2), ALPHA, 1e-5)
    assert torch.equal(xs, x_ref) and torch.equal(yt.transpose(1, 2), y_ref)


def test_residual_norm_into_a_slice(cuda):
    g = torch.Generator(device=cuda).manual_seed(4)
    rows, k = 3000, 128
    a = torch.randn(rows, 4, k, generator=g, device=cuda).to(torch.float16)
    w = (torch.randn(k, k, generator=g, device=cuda) / 11.3).to(torch.float16)
    x = torch.randn(rows, 4, k, generator=g, device=cuda)
    buf = torch.full((rows, 6, k), 7.0, dtype=torch.float16, device=cuda)
    _, x_ref, y_ref = separate_passes(a, w, x, ALPHA, 1e-6)
    xs = x.clone()
    assert projection.linear_residual_norm(a, w, xs, ALPHA, 1e-6, out=buf[:, :4]) is not None
    assert torch.equal(xs, x_ref) and torch.equal(buf[:, :4], y_ref)
    assert bool((buf[:, 4:] == 7.0).all())


def test_residual_norm_declines_what_it_does_not_take(cuda):
    g = torch.Generator(device=cuda).manual_seed(5)
    a = torch.randn(4096, 128, generator=g, device=cuda).to(torch.float16)
    w = torch.randn(128, 128, generator=g, device=cuda).to(torch.float16)
    x = torch.randn(4096, 128, generator=g, device=cuda)
    before = x.clone()
    assert projection.linear_residual_norm(a, w[:64], x, ALPHA, 1e-5) is None        # output width != inner
    assert projection.linear_residual_norm(a.float(), w.float(), x, ALPHA, 1e-5) is None  # not fp16
    assert projection.linear_residual_norm(a[:, :96], w[:96, :96], x[:, :96], ALPHA, 1e-5) is None
    assert projection.linear_residual_norm(a, w, x.half(), ALPHA, 1e-5) is None       # stream not fp32
    assert torch.equal(x, before)


def test_two_phase_steps_take_the_fused_pass(cuda, monkeypatch):
    """A cell layer and a row layer under fp16 autocast: every attention update whose next norm
    is an fp16 operand goes through the fused kernel, and the result matches the separate
    projection + residual + norm passes to within the fp16 roundings of the updates (at these
    row counts the separate projection is the library GEMM, which sums in another order)."""
    from nori_amd import two_phase

    torch.manual_seed(0)
    layer = two_phase.CellLayer2P(128, 2, 256, target_tokens=2, target_heads=4, target_hidden_dim=682,
                                  deepnorm_alpha=ALPHA, device=cuda, dtype=torch.float32).eval()
    row_layer = two_phase.RowLayer2P(256, 4, 682, deepnorm_alpha=ALPHA, device=cuda, dtype=torch.float32).eval()
    g = torch.Generator(device=cuda).manual_seed(6)
    cells = torch.randn(3, 96, 4, 128, generator=g, device=cuda)
    targets = torch.randn(3, 96, 2, 128, generator=g, device=cuda)
    memory = torch.randn(3, 96, 4, 256, generator=g, device=cuda).to(torch.float16)
    calls = []
    fused = projection.linear_residual_norm

    def spy(a, *args, **kw):
        y = fused(a, *args, **kw)
        calls.append((int(a.shape[-1]), y is not None))
        return y

    def run(take):
        monkeypatch.setattr(two_phase, "linear_residual_norm", spy if take else (lambda *a, **k: None))
        with torch.no_grad(), torch.autocast("cuda", dtype=torch.float16):
            c, t = layer(cells, targets, 64)
            r = row_layer(t.reshape(3, 96, 256), 64, memory)
        return c, t, r

    c1, t1, r1 = run(True)
    assert calls and all(took for _, took in calls)
    assert sorted(set(k for k, _ in calls)) == [128, 256]
    c0, t0, r0 = run(False)
    for got, ref in ((c1, c0), (t1, t0), (r1, r0)):
        scale = ref.abs().amax()
        assert float((got - ref).abs().amax()) <= 2e-3 * float(scale)
