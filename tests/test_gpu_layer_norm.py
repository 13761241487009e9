"""The LayerNorm kernel (nori_layer_norm) on the GPU.

nn.LayerNorm in the cell encoder (ref src/synthefy_nori/model/encoders.py:118-276, 432-585):
fp32 statistics (mean, biased variance) and affine; under fp16 autocast the result feeds an
F.linear that rounds it to fp16. Checked against F.layer_norm in float64 on the CPU, then the
affine, the ReLU and the rounding to the output dtype:

* fp32 output: |y - y_ref| <= 2e-6 * (1 + |y_ref|) (the statistics summed in another order);
* fp16 / bf16 output: within one ulp of the output dtype of the rounded reference;
* widths: the grouped path (16, 128, 256: 4, 32 and 64 lanes a row) and the one-wavefront-a-
  row path (96, 1000), ragged row counts, a strided input, no affine, zero rows;
* the module: the two-phase model's cell encoder under autocast against its fp32 CPU run.
"""
import pytest
import torch

from nori_amd.norm import layer_norm

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)


def _reference(x, w, b, eps, relu, out_dtype):
    y = torch.nn.functional.layer_norm(x.double().cpu(), (x.shape[-1],), None, None, eps)
    if w is not None:
        y = y * w.double().cpu()
    if b is not None:
        y = y + b.double().cpu()
    if relu:
        y = y.clamp_min(0.0)
    return y


def _check(y, ref, out_dtype):
    y = y.double().cpu()
    if out_dtype == torch.float32:
        err = float(((y - ref).abs() / (1.0 + ref.abs())).max())
        assert err <= 2e-6, err
        return err
    rounded = ref.to(out_dtype).double()
    ulp = 2.0**-10 if out_dtype == torch.float16 else 2.0**-7
    tol = ulp * rounded.abs().clamp_min(2.0**-14)
    bad = (y - rounded).abs() > tol
    assert not bool(bad.any()), float((y - rounded).abs().max())
    return float((y != rounded).double().mean())


@pytest.mark.parametrize("cols", [16, 128, 256, 96, 1000])
@pytest.mark.parametrize("x_dtype,out_dtype", [
    (torch.float16, torch.float32), (torch.float16, torch.float16), (torch.float32, torch.float16),
    (torch.float32, torch.float32), (torch.bfloat16, torch.bfloat16),
])
def test_against_float64_reference(cols, x_dtype, out_dtype):
    g = torch.Generator().manual_seed(cols)
    rows = 777
    x = (torch.randn(rows, cols, generator=g) * 3.0 + 0.5).to(x_dtype).to(DEV)
    w = (torch.rand(cols, generator=g) + 0.5).to(DEV)
    b = (torch.randn(cols, generator=g) * 0.1).to(DEV)
    for relu in (False, True):
        print(f"layer_norm cols {cols} {x_dtype} -> {out_dtype} relu {relu}", flush=True)
        y = layer_norm(x, w, b, 1e-5, relu=relu, out_dtype=out_dtype)
        torch.cuda.synchronize()
        assert y.dtype == out_dtype and y.shape == x.shape
        diff = _check(y, _reference(x, w, b, 1e-5, relu, out_dtype), out_dtype)
        print(f"  {diff:.3e}", flush=True)


def test_matches_torch_fp32_on_device():
    x = torch.randn(65536, 128, device=DEV, dtype=torch.float16)
    w = torch.rand(128, device=DEV) + 0.5
    b = torch.randn(128, device=DEV)
    y = layer_norm(x, w, b, 1e-5, out_dtype=torch.float32)
    ref = torch.nn.functional.layer_norm(x.float(), (128,), w, b, 1e-5)
    torch.cuda.synchronize()
    assert float((y - ref).abs().max()) <= 4e-6 * float(ref.abs().max())


def test_strided_no_affine_and_empty():
    base = torch.randn(300, 136, device=DEV)
    x = base[:, :128]
    y = layer_norm(x, None, None, 1e-6)
    ref = layer_norm(x.contiguous(), None, None, 1e-6)
    torch.cuda.synchronize()
    assert torch.equal(y, ref)
    _check(y, _reference(x, None, None, 1e-6, False, torch.float32), torch.float32)
    assert layer_norm(x[:0], None, None, 1e-5).shape == (0, 128)


def test_cell_encoder_under_autocast():
    """MaskEmbEncoder with the RBF numeric embedding (the two-phase model's cell encoder):
    the GPU forward under fp16 autocast, whose three norms run on the kernel, against the same
    module in fp32 on the CPU (torch's LayerNorm)."""
    from nori_amd.encoders import MaskEmbEncoder

    torch.manual_seed(0)
    enc = MaskEmbEncoder(
        num_features=2, emsize=128, mask_embedding_size=128, numeric_embed_type="RBF",
        RBF_config=dict(token_embed_dim=8, n_kernels=16, sigma=0.5, use_learn_sigma=False,
                        use_learn_embeddings=False, use_original_features=False),
    ).eval()
    x = torch.randn(2, 64, 4, 2) * 3.0
    x[0, :3, 1, 0] = float("nan")
    with torch.inference_mode():
        ref = enc({"data": x.clone()})["data"]
        enc_gpu = enc.to(DEV)
        with torch.autocast("cuda", dtype=torch.float16):
            out = enc_gpu({"data": x.to(DEV)})["data"]
    torch.cuda.synchronize()
    assert out.dtype == torch.float32 and out.shape == ref.shape
    err = float((out.cpu() - ref).abs().max() / ref.abs().max())
    print(f"cell encoder under autocast vs fp32 CPU: {err:.3e}", flush=True)
    assert err <= 2e-2  # fp16 projections against fp32 ones


@pytest.mark.parametrize("cols", [128, 96])
def test_relu_keeps_nan_rows(cols):
    # an inf or NaN cell (an fp16 projection that overflowed) makes its row's statistics NaN;
    # the fused ReLU keeps NaN as torch.relu does, so predict still sees the non-finite output
    x = torch.randn(40, cols, device=DEV)
    x[3, 5] = float("inf")
    x[7, 0] = float("nan")
    w = torch.rand(cols, device=DEV) + 0.5
    b = torch.randn(cols, device=DEV)
    y = layer_norm(x, w, b, 1e-5, relu=True, out_dtype=torch.float32)
    ref = torch.relu(torch.nn.functional.layer_norm(x, (cols,), w, b, 1e-5))
    torch.cuda.synchronize()
    assert bool(torch.isnan(y[3]).all()) and bool(torch.isnan(y[7]).all())
    assert torch.equal(torch.isnan(y), torch.isnan(ref))
    ok = ~torch.isnan(ref)
    assert float((y[ok] - ref[ok]).abs().max()) <= 4e-6 * float(ref[ok].abs().max())
