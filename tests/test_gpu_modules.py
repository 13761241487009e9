"""Module-level routes into the HIP attention kernel.

* QASS "log_only" on the MFMA path (the two-phase column/row attentions): the log-n multiply
  rides on the kernel's logit scale instead of a separate fp16 multiply over q
  (QASSMaxScaling.forward, layer.py:433-456). Same module, fold on and off, under fp16
  autocast at the config-5 column-attention shape (320 queries over 256 context keys): the
  only difference is one f16 rounding of q, so the outputs agree to 5e-3.
* The combined-QKV feature attention over a row's tokens at a width past the short-context
  kernel (51 tokens, nori-100m's token groups): the MFMA kernel, against the float64 oracle
  on the same projected q/k/v.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from nori_amd.layer import MultiheadAttention
from oracle import attention as oa
from parity import check_relative

pytestmark = pytest.mark.gpu


def _module(cuda, embed, heads, **kw):
    torch.manual_seed(7)
    mod = MultiheadAttention(embed_dim=embed, num_heads=heads, dropout=0.0, **kw).to(cuda).eval()
    if mod.q_norm is not None:  # gains away from 1, so the norms' gains are exercised
        with torch.no_grad():
            mod.q_norm.weight.uniform_(0.5, 1.5)
            mod.k_norm.weight.uniform_(0.5, 1.5)
    return mod


@pytest.mark.parametrize("n_ctx", [256, 1])
def test_log_only_qass_fold_matches_separate_multiply(cuda, n_ctx):
    mod = _module(cuda, 128, 2, qkv_combined=False, use_qassmax=True, qass_mode="log_only", qk_norm=True)
    g = torch.Generator(device="cpu").manual_seed(3)
    cells = torch.randn(2, 3, 320, 128, generator=g).to(cuda)  # [tables, columns, rows, width]
    outs = {}
    with torch.inference_mode(), torch.autocast("cuda", dtype=torch.float16):
        for fold in (True, False):
            mod.fold_log_only_qass = fold
            outs[fold] = mod(cells, x_kv=cells[:, :, :n_ctx])[0].float()
    mod.fold_log_only_qass = True
    err = (outs[True] - outs[False]).abs().max().item()
    print(f"[parity] QASS log_only fold vs separate multiply, {n_ctx} keys: max abs {err:.3e}", flush=True)
    assert err <= 5e-3
    if n_ctx == 1:
        # one key: every query reads that key's value whatever its scale, and no log-n factor applies
        assert mod.log_only_logit_scale(1, torch.float16) == 1.0 / math.sqrt(64)


def test_wide_combined_qkv_feature_attention_runs_on_the_kernel(cuda):
    tokens, embed, heads = 51, 112, 2
    mod = _module(cuda, embed, heads, qkv_combined=True)
    g = torch.Generator(device="cpu").manual_seed(5)
    x = torch.randn(1, 300, tokens, embed, generator=g).to(cuda)  # [tables, rows, tokens, width]
    with torch.inference_mode():
        out = mod(x)[0]
        qkv = torch.einsum("... s, j h d s -> ... j h d", x.reshape(-1, tokens, embed), mod.qkv_proj_weight)
        ref, _ = oa.attention_f64(*(qkv[:, :, j].double().cpu().numpy() for j in range(3)))
        d = embed // heads
        ref = torch.from_numpy(ref).reshape(300, tokens, heads * d)
        w_out = mod.out_proj_weight.double().cpu().reshape(heads * d, embed)
        expected = (ref @ w_out).reshape(1, 300, tokens, embed)
    check_relative(out, expected, 1e-3, "51-token combined-QKV feature attention vs float64 oracle")
    assert np.isfinite(out.cpu().numpy()).all()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("hidden", [170, 341, 64])
def test_silu_mul_is_torch_silu_times_up(cuda, dtype, hidden):
    # the SwiGLU gate of one stacked [gate | up] projection against torch's own two ops in the
    # same dtype (F.silu then *), element for element; widths with and without the 4-wide path
    from nori_amd.norm import silu_mul

    g = torch.Generator(device="cpu").manual_seed(hidden)
    gu = (torch.randn(777, 2 * hidden, generator=g) * 3).to(dtype).to(cuda)
    got = silu_mul(gu, hidden)
    exp = torch.nn.functional.silu(gu[:, :hidden]) * gu[:, hidden:]
    diff = (got.float() - exp.float()).abs()
    ulp = exp.float().abs() * (2.0**-10 if dtype == torch.float16 else 2.0**-7 if dtype == torch.bfloat16 else 2.0**-23)
    mismatches = int((got != exp).sum())
    print(f"[parity] silu_mul {dtype} hidden {hidden}: {mismatches} of {exp.numel()} differ from torch", flush=True)
    assert bool((diff <= ulp + 1e-30).all()), "silu_mul differs from torch by more than one unit in the last place"
    assert mismatches <= exp.numel() // 1000


def test_swiglu_module_matches_separate_projections(cuda):
    from nori_amd.layer import SwiGLUMLP

    torch.manual_seed(11)
    mlp = SwiGLUMLP(128, 256, 128, has_bias=False, device=cuda, dtype=torch.float32)
    x = torch.randn(4, 300, 128, device=cuda)
    results = []
    for step in range(2):
        if step:
            with torch.no_grad():
                mlp.w_up.weight.mul_(0.5)  # a changed weight rebuilds the stacked one
        with torch.inference_mode(), torch.autocast("cuda", dtype=torch.float16):
            results.append((mlp(x), mlp.w_down(torch.nn.functional.silu(mlp.w_gate(x)) * mlp.w_up(x))))
    for a, b in results:
        check_relative(a, b, 2e-3, "stacked SwiGLU vs separate gate/up projections (fp16 autocast)")


@pytest.mark.parametrize("layer_arch,alpha", [("smf", 18**-0.5), ("fmfmsm", None)])
def test_dense_layer_residual_chain_is_bit_exact(cuda, layer_arch, alpha):
    """The dense layer's pre-norm residual updates formed in the same pass as the next norm's
    operand (``_add_then_steps``, ``nori_residual_add_rms_norm``) against the separate
    ``residual + deepnorm_alpha * update`` (the fp32 buffer cast to the update's dtype, as
    torch applies it) and norm of each step (layer.py:1444-1445), under fp16 autocast and in
    fp32. alpha 18^-1/2 is not an fp16 value, so the cast matters.

    * bit-identical streams when the sublayers are deterministic functions of their operands
      (the library GEMMs may pick split-K kernels whose sums are not reproducible run to run);
    * with the layer's own sublayers, the two orders agree to a relative 1e-3."""
    from nori_amd.layer import EncoderBaseLayer

    torch.manual_seed(5)
    layer = EncoderBaseLayer(
        nhead=4, embed_dim=128, hid_dim=384, pre_norm=True, activation="swiglu", norm_type="rmsnorm",
        layer_arch=layer_arch, deepnorm_alpha=alpha, device=cuda,
    ).eval()
    pre_steps, seq_step, post_steps, _ = layer._cache_steps()
    steps = list(pre_steps) or list(post_steps)
    assert layer.deepnorm_alpha is None or layer.deepnorm_alpha.device.type == "cpu"
    _chain_cases(layer, steps, cuda, layer_arch)
    layer.to(cuda)  # the buffer on the device: torch casts it to the update's dtype first
    _chain_cases(layer, steps, cuda, layer_arch)


def _chain_cases(layer, steps, cuda, layer_arch):
    x = torch.randn(2, 40, 9, 128, device=cuda)
    update = torch.randn(2, 40, 9, 128, device=cuda) * 2.0
    own_steps = list(layer.layer_steps)
    synthetic = [lambda op, k=k: (torch.tanh(op.float() * (1.1 + 0.3 * k)) * 3.0).to(op.dtype) for k in range(len(own_steps))]
    for sublayers, exact in ((synthetic, True), (own_steps, False)):
        layer.layer_steps = sublayers
        for autocast in (True, False):
            with torch.inference_mode(), torch.autocast("cuda", dtype=torch.float16, enabled=autocast):
                u = update.half() if autocast else update
                ref = layer._residual_add(x, u)
                for step in steps:
                    ref = layer._run_non_sequence_step(ref, step_idx=step, feature_atten_mask=None, eval_pos=40)
                x0 = x.clone()
                got = layer._add_then_steps(x, u, steps, None, 40)
            torch.cuda.synchronize()
            assert torch.equal(x, x0), "the input stream was modified"
            if exact:
                assert torch.equal(got, ref), f"{layer_arch} autocast={autocast}: max diff {float((got - ref).abs().max())}"
            else:
                check_relative(got, ref, 1e-3, f"{layer_arch} residual chain with the layer's sublayers")
    layer.layer_steps = own_steps
