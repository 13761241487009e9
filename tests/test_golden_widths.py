"""Model-level parity at the long-context models' head widths, 44 and 56 (tests/width_cases.py).

tests/golden/width_goldens.npz holds the reference's own outputs (tests/golden/
make_width_golden.py, run on the CPU) for two-layer stacks and two-layer models with two heads
of 44 (embed 88, 33 tokens a row) and of 56 (embed 112, 51 tokens a row), QASS "full", a few
hundred context rows: in fp32 (full-precision and int8 caches) and under the reference's own
fp16 autocast (int8 cache). These shapes take, in composition, what the narrower goldens do
not: the attention's folded mode (head widths not a multiple of 16: the padding columns that
carry the running max and the denominator, the optimistic scan), K/V staged at d 44 / 56, the
few-token kernel over 33 and 51 tokens (fp16 queries, so under autocast), the QASS gate kernel
at those widths, and the fused cache write (``fused_cache_write=True``).

Bars (max|got - exp| / max|exp|, printed by every check):
* fp32 on the GPU against the reference's fp32 run: 1e-3, the prediction bar;
* fp16 autocast on the GPU against the reference's fp16 autocast run (made on the CPU with CUDA
  autocast's op policy, tests/golden/cuda_autocast_policy.py): the prediction bar, or
  1.5 times the reference's own spread if that is larger -- the largest change of the
  reference's fp16 outputs when only the order of the context rows (so of its sums) changes,
  measured by the golden recipe over three orders and stored beside the outputs. An fp16 run
  cannot be reproduced more closely than its own summation order allows.
CPU tests: the seeded weights hash to the ones the reference ran with, and load strictly.
"""

from __future__ import annotations

import json
import os

import numpy as np
import pytest
import torch

import regressor_case as case
import width_cases as wc
from nori_amd import layer as NL
from nori_amd import transformer as NT
from parity import PREDICTION_BAR, check_relative

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "width_goldens.npz")
SPREAD_FACTOR = 1.5


@pytest.fixture(scope="module")
def gold():
    with np.load(GOLDEN, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def make_stack(gold, tag):
    c = wc.STACKS[tag]
    stack = NL.LayerStack([NL.EncoderBaseLayer(**wc.layer_kwargs(c)) for _ in range(c["layers"])]).eval()
    scales = json.loads(str(gold[f"{tag}/weight_scales"]))
    stack.load_state_dict(wc.seeded_state(stack.state_dict(), scales, 40 + list(wc.STACKS).index(tag)), strict=True)
    return stack


def make_model(gold, tag):
    model = NT.FeaturesTransformer(**wc.model_config(wc.MODELS[tag])).eval()
    scales = json.loads(str(gold[f"{tag}/weight_scales"]))
    state = wc.seeded_state(model.state_dict(), scales, 50 + list(wc.MODELS).index(tag), wc.head_name(model))
    model.load_state_dict(state, strict=True)
    return model


def autocast_bar(gold, key):
    return max(PREDICTION_BAR, SPREAD_FACTOR * float(gold[key]))


def check(got, exp, bar, what):
    got = torch.as_tensor(got).detach().float().cpu()
    exp = torch.as_tensor(exp)
    assert tuple(got.shape) == tuple(exp.shape), (tuple(got.shape), tuple(exp.shape))
    return check_relative(got, exp, bar, what)


# ------------------------------------------------------------------------------- CPU
@pytest.mark.parametrize("tag", list(wc.STACKS))
def test_stack_weights_are_the_ones_the_reference_ran(gold, tag):
    assert case.weights_sha256(make_stack(gold, tag)) == str(gold[f"{tag}/weights_sha256"])


@pytest.mark.parametrize("tag", list(wc.MODELS))
def test_model_weights_are_the_ones_the_reference_ran(gold, tag):
    assert case.weights_sha256(make_model(gold, tag)) == str(gold[f"{tag}/weights_sha256"])


def test_fixture_spreads_are_recorded(gold):
    for tag in wc.STACKS:
        for name in ("spread_test_out_int8_ac", "spread_train_out_int8_ac"):
            assert 0.0 < float(gold[f"{tag}/{name}"]) < 1e-2
    for tag in wc.MODELS:
        assert 0.0 < float(gold[f"{tag}/spread_pred_int8_ac"]) < 1e-2


# ------------------------------------------------------------------------------- GPU
@pytest.mark.gpu
@pytest.mark.parametrize("tag", list(wc.STACKS))
@pytest.mark.parametrize("quant", [False, True])
def test_stack_fp32_matches_reference(gold, cuda, tag, quant):
    stack = make_stack(gold, tag).to(cuda)
    x_train, x_test = (torch.from_numpy(a).to(cuda) for a in wc.stack_inputs(tag))
    sfx = "int8" if quant else "fp"
    print(f"{tag} fp32 {sfx}: {tuple(x_train.shape)} context, {tuple(x_test.shape)} queries", flush=True)
    with torch.inference_mode():
        train_out, caches = stack.build_train_cache(x_train, quantize_kv_cache=quant, device=cuda)
        test_out = stack.forward_test_with_cache(x_test, caches)
    check(train_out[:, ::wc.ROW_STEP], gold[f"{tag}/train_out_{sfx}"], PREDICTION_BAR, f"{tag} fp32 {sfx} context rows")
    check(test_out[:, ::wc.QUERY_STEP], gold[f"{tag}/test_out_{sfx}"], PREDICTION_BAR, f"{tag} fp32 {sfx} query rows")
    if quant:
        # layer 0's codes come from the inputs through one norm and one projection: within one
        d = (caches[0]["seq_kv"].device_payload()[0][:, : wc.CODE_ROWS].cpu().numpy().astype(np.int32)
             - gold[f"{tag}/codes0"].astype(np.int32))
        print(f"[parity] {tag} layer-0 codes: {np.mean(d != 0):.2e} differ by one", flush=True)
        assert np.abs(d).max() <= 1 and np.mean(d != 0) < 0.01


@pytest.mark.gpu
@pytest.mark.parametrize("tag", list(wc.STACKS))
@pytest.mark.parametrize("fused", [False, True])
def test_stack_fp16_autocast_matches_reference_autocast(gold, cuda, tag, fused):
    stack = make_stack(gold, tag).to(cuda)
    x_train, x_test = (torch.from_numpy(a).to(cuda) for a in wc.stack_inputs(tag))
    what = f"{tag} fp16 autocast int8 ({'fused' if fused else 'default'} cache write)"
    print(what, flush=True)
    with torch.inference_mode(), torch.autocast("cuda", dtype=torch.float16):
        train_out, caches = stack.build_train_cache(x_train, quantize_kv_cache=True, device=cuda,
                                                    fused_cache_write=fused)
        test_out = stack.forward_test_with_cache(x_test, caches)
    check(train_out[:, ::wc.ROW_STEP], gold[f"{tag}/train_out_int8_ac"],
          autocast_bar(gold, f"{tag}/spread_train_out_int8_ac"), what + ", context rows")
    check(test_out[:, ::wc.QUERY_STEP], gold[f"{tag}/test_out_int8_ac"],
          autocast_bar(gold, f"{tag}/spread_test_out_int8_ac"), what + ", query rows")
    d = (caches[0]["seq_kv"].device_payload()[0][:, : wc.CODE_ROWS].cpu().numpy().astype(np.int32)
         - gold[f"{tag}/codes0_ac"].astype(np.int32))
    print(f"[parity] {what} layer-0 codes: {np.mean(d != 0):.2e} differ by one, max {np.abs(d).max()}", flush=True)
    assert np.abs(d).max() <= 1 and np.mean(d != 0) < 0.02


@pytest.mark.gpu
@pytest.mark.parametrize("tag", list(wc.MODELS))
def test_model_fp32_matches_reference(gold, cuda, tag):
    c = wc.MODELS[tag]
    model = make_model(gold, tag).to(cuda)
    x_np, y_np = wc.model_table(tag)
    x, y = torch.from_numpy(x_np).to(cuda), torch.from_numpy(y_np).to(cuda)
    n_ctx = c["n_ctx"]
    for cache_dtype in ("bf16", "int8"):
        print(f"{tag} fp32 {cache_dtype} cache: {n_ctx} context rows, {c['features']} features", flush=True)
        with torch.inference_mode():
            ctx = model.build_context_cache(x[:, :n_ctx], y, cache_dtype=cache_dtype)
            pred = model.apply_context_cache(x[:, n_ctx:], ctx)
        check(pred, gold[f"{tag}/pred_{cache_dtype}"], PREDICTION_BAR, f"{tag} fp32 {cache_dtype} predictions")


@pytest.mark.gpu
@pytest.mark.parametrize("tag", list(wc.MODELS))
@pytest.mark.parametrize("fused", [False, True])
def test_model_fp16_autocast_matches_reference_autocast(gold, cuda, tag, fused):
    c = wc.MODELS[tag]
    model = make_model(gold, tag).to(cuda)
    x_np, y_np = wc.model_table(tag)
    x, y = torch.from_numpy(x_np).to(cuda), torch.from_numpy(y_np).to(cuda)
    n_ctx = c["n_ctx"]
    what = f"{tag} fp16 autocast int8 predictions ({'fused' if fused else 'default'} cache write)"
    print(what, flush=True)
    with torch.inference_mode(), torch.autocast("cuda", dtype=torch.float16):
        ctx = model.build_context_cache(x[:, :n_ctx], y, cache_dtype="int8", fused_cache_write=fused)
        pred = model.apply_context_cache(x[:, n_ctx:], ctx)
    check(pred, gold[f"{tag}/pred_int8_ac"], autocast_bar(gold, f"{tag}/spread_pred_int8_ac"), what)
    check(pred, gold[f"{tag}/pred_int8"], max(PREDICTION_BAR, 4 * float(gold[f"{tag}/spread_pred_int8_ac"])),
          what + " against the fp32 run")
