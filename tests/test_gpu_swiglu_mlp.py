"""The fused SwiGLU feed-forward kernel (nori_swiglu_mlp) on the GPU.

SwiGLUMLP.forward (ref src/synthefy_nori/model/layer.py:261-274) under fp16 autocast is three
ops, each rounding to fp16: the gate/up projection, silu(gate) * up, the down projection. The
checks here:

* against an emulation of exactly those roundings with exact (float64) sums on the CPU:
  the kernel sums in fp32 in its own order and takes silu from the hardware exp2 and
  reciprocal, so an intermediate may land one fp16 ulp away; the outputs are held to
  |y - y_ref| <= 2^-8 * max|y_ref| (measured: at most 3.6e-4, about 2^-11.5);
* against the unfused GPU sequence (hipBLASLt projections + nori_silu_mul), same bound
  (measured: at most 5.9e-4; 99.96 % of the outputs bit-identical);
* shapes: every width the kernel is built for, hidden widths padded up to whole 32-unit chunks
  (8, 40, 682), ragged row counts, a strided operand, zero rows;
* the module: SwiGLUMLP under autocast takes the kernel, and matches its unfused path.
"""
import pytest
import torch

from nori_amd import layer as nl
from nori_amd.norm import FUSED_MLP_WIDTHS, silu_mul, swiglu_mlp

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)


def _weights(width: int, hidden: int, seed: int):
    """Stacked fp16 weights as SwiGLUMLP._stacked_weights lays them out for the kernel: [gate |
    up] rows [2 hp, width] and down [width, hp], hp = hidden padded to a multiple of 32 with
    zeros."""
    g = torch.Generator().manual_seed(seed)
    hp = (hidden + 31) // 32 * 32
    gate_up = torch.zeros(2 * hp, width)
    gate_up[:hidden] = torch.randn(hidden, width, generator=g) / width**0.5
    gate_up[hp : hp + hidden] = torch.randn(hidden, width, generator=g) / width**0.5
    down = torch.zeros(width, hp)
    down[:, :hidden] = torch.randn(width, hidden, generator=g) / hidden**0.5
    return gate_up.half().to(DEV), down.half().to(DEV), hp


def _emulated(x: torch.Tensor, gate_up: torch.Tensor, down: torch.Tensor, hp: int) -> torch.Tensor:
    """The unfused fp16 sequence's roundings with exact sums (float64 on the CPU)."""
    gu = (x.double().cpu() @ gate_up.double().cpu().T).half().float()
    g, u = gu[:, :hp], gu[:, hp:]
    s = (g / (1.0 + torch.exp(-g))).half().float()
    a = (s * u).half()
    return (a.double() @ down.double().cpu().T).half()


def _unfused(x: torch.Tensor, gate_up: torch.Tensor, down: torch.Tensor, hp: int) -> torch.Tensor:
    gu = torch.nn.functional.linear(x, gate_up)
    return torch.nn.functional.linear(silu_mul(gu, hp), down)


def _rel_err(y: torch.Tensor, ref: torch.Tensor) -> float:
    ref = ref.float().cpu()
    return float((y.float().cpu() - ref).abs().max() / ref.abs().max().clamp_min(1e-30))


TOL = 2.0**-8


@pytest.mark.parametrize("width", FUSED_MLP_WIDTHS)
@pytest.mark.parametrize("hidden,rows", [(256, 300), (682, 37), (40, 1), (8, 129)])
def test_against_exact_sum_emulation(width, hidden, rows):
    gate_up, down, hp = _weights(width, hidden, seed=width + hidden)
    x = torch.randn(rows, width, generator=torch.Generator().manual_seed(rows)).half().to(DEV)
    print(f"swiglu_mlp width {width} hidden {hidden} rows {rows}", flush=True)
    y = swiglu_mlp(x, gate_up, down, hp)
    torch.cuda.synchronize()
    err = _rel_err(y, _emulated(x, gate_up, down, hp))
    print(f"  max |y - y_ref| / max |y_ref| = {err:.3e}", flush=True)
    assert bool(torch.isfinite(y).all())
    assert err <= TOL


@pytest.mark.parametrize("width", FUSED_MLP_WIDTHS)
def test_against_unfused_sequence(width):
    hidden = int(2 * (3 * width) / 3)  # SwiGLUMLP(width, 3 * width): hidden 2 * width
    gate_up, down, hp = _weights(width, hidden, seed=7 * width)
    x = torch.randn(5000, width, generator=torch.Generator().manual_seed(3)).half().to(DEV)
    print(f"swiglu_mlp vs unfused, width {width} rows 5000", flush=True)
    y = swiglu_mlp(x, gate_up, down, hp)
    ref = _unfused(x, gate_up, down, hp)
    torch.cuda.synchronize()
    err = _rel_err(y, ref)
    same = float((y == ref).float().mean())
    print(f"  max rel err {err:.3e}, bit-identical fraction {same:.4f}", flush=True)
    assert err <= TOL


def test_strided_operand_and_empty_rows():
    gate_up, down, hp = _weights(256, 682, seed=11)
    base = torch.randn(400, 264, generator=torch.Generator().manual_seed(5)).half().to(DEV)
    x = base[:, :256]  # row stride 264
    print("swiglu_mlp strided operand", flush=True)
    y = swiglu_mlp(x, gate_up, down, hp)
    ref = swiglu_mlp(x.contiguous(), gate_up, down, hp)
    torch.cuda.synchronize()
    assert torch.equal(y, ref)
    empty = swiglu_mlp(x[:0], gate_up, down, hp)
    assert empty.shape == (0, 256)


def test_config5_shapes_fill_whole_grids():
    """The two-phase model's two sublayers at the many-small-tables size: cells (width 128,
    hidden 256, 655,360 rows) and target rows (width 256, hidden 688, 163,840 rows),
    checked on sampled rows against the emulation."""
    for width, hidden, rows in ((128, 256, 655_360), (256, 682, 163_840)):
        gate_up, down, hp = _weights(width, hidden, seed=width)
        x = torch.randn(rows, width, device=DEV, dtype=torch.float16)
        print(f"swiglu_mlp width {width} hidden {hidden} rows {rows}", flush=True)
        y = swiglu_mlp(x, gate_up, down, hp)
        idx = torch.randperm(rows, generator=torch.Generator().manual_seed(1))[:2048].to(DEV)
        err = _rel_err(y[idx], _emulated(x[idx], gate_up, down, hp))
        print(f"  sampled max rel err {err:.3e}", flush=True)
        assert bool(torch.isfinite(y).all())
        assert err <= TOL


def test_module_takes_the_fused_kernel_under_autocast():
    torch.manual_seed(0)
    mlp = nl.SwiGLUMLP(128, 384, 128, has_bias=False, device=DEV, dtype=torch.float32)
    x = torch.randn(3, 700, 128, device=DEV)
    calls = []
    real = nl.swiglu_mlp

    def spy(*a, **k):
        calls.append(1)
        return real(*a, **k)

    nl.swiglu_mlp = spy
    try:
        with torch.inference_mode(), torch.autocast("cuda", dtype=torch.float16):
            y = mlp(x)
            mlp.fused = False
            ref = mlp(x)
    finally:
        nl.swiglu_mlp = real
        mlp.fused = True
    torch.cuda.synchronize()
    assert calls == [1]
    assert y.dtype == torch.float16 and y.shape == (3, 700, 128)
    assert _rel_err(y, ref) <= TOL
    # fp32 without autocast, and a width the kernel lacks, keep the unfused path
    with torch.inference_mode():
        out32 = mlp(x)
    assert out32.dtype == torch.float32
    wide = nl.SwiGLUMLP(96, 288, 96, has_bias=False, device=DEV, dtype=torch.float32)
    with torch.inference_mode(), torch.autocast("cuda", dtype=torch.float16):
        assert wide(torch.randn(10, 96, device=DEV)).shape == (10, 96)


# ---------------------------------------------------------------- with the residual update + norm
# nori_swiglu_mlp_residual_rms_norm: the MLP, then stream += alpha * y and the next RMSNorm
# (reference two_phase.py:209, 220-225, 271-272): bit for bit swiglu_mlp followed by the fused
# residual + norm kernel (which the norm tests pin to torch), for every width / norm-width pair
# it is built for, ragged row counts and an output that is a slice of a token buffer.

ALPHA = 18 ** -0.5


@pytest.mark.parametrize("width,norm_width,hidden", [(128, 128, 256), (256, 128, 682), (256, 256, 1024)])
@pytest.mark.parametrize("rows", [1, 77, 5000])
def test_residual_norm_epilogue_equals_the_separate_kernels(width, norm_width, hidden, rows):
    from nori_amd.norm import RMSNorm, residual_add_norm, swiglu_mlp_residual_norm

    gate_up, down, hp = _weights(width, hidden, seed=width + hidden + rows)
    g = torch.Generator(device=DEV).manual_seed(rows)
    x = torch.randn(rows, width, generator=g, device=DEV).half()
    stream = torch.randn(rows, width // norm_width, norm_width, generator=g, device=DEV) * 2.0
    u = swiglu_mlp(x, gate_up, down, hp)
    ref_stream = stream.clone()
    ref = residual_add_norm(ref_stream, u.view(stream.shape), ALPHA, RMSNorm(norm_width, eps=1e-5),
                            out_dtype=torch.float16)
    got_stream = stream.clone()
    got = swiglu_mlp_residual_norm(x, gate_up, down, hp, got_stream, ALPHA, 1e-5, norm_width)
    assert got is not None and got.shape == stream.shape and got.dtype == torch.float16
    assert torch.equal(got_stream, ref_stream)
    assert torch.equal(got, ref)


def test_residual_norm_epilogue_into_token_slices():
    # the two-phase cell layer: the cells' MLP into the first 4 token slots of each row, the
    # target row MLP (width 256, two 128-wide tokens) into the last 2
    from nori_amd.norm import RMSNorm, residual_add_norm, swiglu_mlp_residual_norm

    b, n, gr = 3, 700, 4
    g = torch.Generator(device=DEV).manual_seed(5)
    tokens = torch.full((b, n, gr + 2, 128), 7.0, dtype=torch.float16, device=DEV)
    ref_tokens = tokens.clone()
    cells = torch.randn(b, n, gr, 128, generator=g, device=DEV)
    targets = torch.randn(b, n, 2, 128, generator=g, device=DEV)
    xc = torch.randn(b, n, gr, 128, generator=g, device=DEV).half()
    xt = torch.randn(b, n, 256, generator=g, device=DEV).half()
    wc = _weights(128, 256, seed=1)
    wt = _weights(256, 682, seed=2)
    rc, rt = cells.clone(), targets.clone()
    residual_add_norm(rc, swiglu_mlp(xc, *wc).view(rc.shape), ALPHA, RMSNorm(128, eps=1e-5), out=ref_tokens[:, :, :gr])
    residual_add_norm(rt, swiglu_mlp(xt, *wt).view(rt.shape), ALPHA, RMSNorm(128, eps=1e-5), out=ref_tokens[:, :, gr:])
    assert swiglu_mlp_residual_norm(xc, *wc, cells, ALPHA, 1e-5, 128, out=tokens[:, :, :gr]) is not None
    assert swiglu_mlp_residual_norm(xt, *wt, targets, ALPHA, 1e-5, 128, out=tokens[:, :, gr:]) is not None
    assert torch.equal(cells, rc) and torch.equal(targets, rt)
    assert torch.equal(tokens, ref_tokens)


def test_residual_norm_epilogue_declines_what_it_does_not_take():
    from nori_amd.norm import swiglu_mlp_residual_norm

    gate_up, down, hp = _weights(352, 1056, seed=3)
    x = torch.randn(64, 352, device=DEV).half()
    stream = torch.randn(64, 352, device=DEV)
    assert swiglu_mlp_residual_norm(x, gate_up, down, hp, stream, ALPHA, 1e-5, 352) is None  # width 352
    gate_up, down, hp = _weights(128, 256, seed=4)
    x = torch.randn(64, 128, device=DEV).half()
    assert swiglu_mlp_residual_norm(x, gate_up, down, hp, torch.randn(64, 128, device=DEV).half(), ALPHA, 1e-5,
                                    128) is None  # fp16 stream
