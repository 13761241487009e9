"""Parity of the per-layer cache path with the reference's own outputs.

tests/golden/layer_cache_goldens.npz holds weights, inputs and outputs of the reference's
``MultiheadAttention`` cache methods (layer.py:651-745, QASS :433-456) and of a two-layer
``LayerStack`` of nori-6m-flagged ``EncoderBaseLayer``s (build_train_cache /
forward_test_with_cache, layer.py:1771-1967, 2058-2108), run on the CPU in fp32 by
tests/golden/make_golden.py. Cases: a multi-head cache (Hkv = H) and a shared-head cache
(Hkv = 1), full-precision and int8 caches, dense and blockwise (host-streamed) attention.

CPU tests: the fixture loads without pickle, and this package's modules accept the
reference's state dicts strictly (same parameter names and shapes).
GPU tests: the same computation through the HIP kernels. Attention runs on f16 MFMA with
fp32 accumulation against the reference's fp32 CPU path. Every output is held to a relative
error max|got - exp| / max|exp| <= 1e-3, the bar for predictions; the measured figures
(printed by each check) are at most 4e-4 on attention outputs and below 1e-5 downstream of
the layer norms.
The int8 codes are compared with the reference's CPU codes up to the scale-rounding
difference between torch's CPU division and its GPU reciprocal multiply.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch
from parity import PREDICTION_BAR, check_relative

from nori_amd import layer as NL
from nori_amd.kv_cache_scaling import BlockwiseSeqKV, ScalableSeqKV

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "layer_cache_goldens.npz")


@pytest.fixture(scope="module")
def gold():
    with np.load(GOLDEN, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def weights(gold, prefix):
    n = len(prefix) + 3
    return {k[n:]: torch.from_numpy(v) for k, v in gold.items() if k.startswith(prefix + "/w.")}


def make_attn():
    return NL.MultiheadAttention(32, 2, qkv_combined=False, use_qassmax=True, qass_mode="full").eval()


def make_stack(gold, tag):
    e, h, hid, nl, cross = (int(v) for v in gold[f"{tag}/config"])
    layers = [
        NL.EncoderBaseLayer(
            nhead=h, embed_dim=e, hid_dim=hid, pre_norm=True, activation="swiglu", layer_arch="smf",
            seq_attn_isolated=True, cross_share_all_kv_heads=bool(cross), use_qassmax=True, norm_type="rmsnorm",
            deepnorm_alpha=nl ** -0.5, qass_mode="full",
        )
        for _ in range(nl)
    ]
    return NL.LayerStack(layers).eval()


def check(got, exp, bar=PREDICTION_BAR):
    """max|got - exp| / max|exp| <= bar (relative 1e-3 by default, the bar for predictions)."""
    got = torch.as_tensor(got).detach()
    exp = torch.as_tensor(exp)
    assert tuple(got.shape) == tuple(exp.shape), (tuple(got.shape), tuple(exp.shape))
    test = os.environ.get("PYTEST_CURRENT_TEST", "?").split(" ")[0]
    return check_relative(got, exp, bar, test)


# ------------------------------------------------------------------------------- CPU
def test_fixture_loads_without_pickle_and_is_consistent(gold):
    for tag in ("attn_mha", "attn_mqa"):
        x_ctx, x_q = gold[f"{tag}/x_ctx"], gold[f"{tag}/x_q"]
        kv, codes, scales = gold[f"{tag}/kv"], gold[f"{tag}/codes"], gold[f"{tag}/scales"]
        b, g, n, e = x_ctx.shape
        hkv = 1 if tag == "attn_mqa" else 2
        assert kv.shape == (b * g, n, 2, hkv, e // 2) and codes.dtype == np.int8 and codes.shape == kv.shape
        assert scales.shape == kv.shape[:-1] + (1,)
        assert gold[f"{tag}/out_dense"].shape == x_q.shape
        # the reference's own CPU quantizer is per-vector absmax: the absmax element codes to +-127
        assert np.all(np.abs(codes).max(axis=-1) == 127)
    for tag in ("stack", "stack_mqa"):
        assert gold[f"{tag}/test_out_int8"].shape == gold[f"{tag}/x_test"].shape


@pytest.mark.parametrize("tag", ["attn_mha", "attn_mqa"])
def test_attention_module_takes_the_reference_state_dict(gold, tag):
    attn = make_attn()
    attn.load_state_dict(weights(gold, tag), strict=True)


@pytest.mark.parametrize("tag", ["stack", "stack_mqa"])
def test_layer_stack_takes_the_reference_state_dict(gold, tag):
    stack = make_stack(gold, tag)
    stack.load_state_dict(weights(gold, tag), strict=True)


def test_bounded_build_levers_are_validated_as_the_reference_does(gold):
    """layer.py:1822-1855: the streamed builds need a row cap, host offload (streaming) or a
    resident int8 cache (hybrid), and serial attention refuses every bounded build."""
    stack = make_stack(gold, "stack")
    x = torch.from_numpy(gold["stack/x_train"])
    with pytest.raises(ValueError, match="context_row_chunk"):
        stack.build_train_cache(x.clone(), stream_context=True, offload_kv_cache=True)
    with pytest.raises(ValueError, match="offload_kv_cache=True"):
        stack.build_train_cache(x.clone(), stream_context=True, fit_row_chunk=32)
    with pytest.raises(ValueError, match="hybrid resident INT8 prefill requires"):
        stack.build_train_cache(x.clone(), _hybrid_resident_int8_prefill=True, fit_row_chunk=32)
    with pytest.raises(ValueError, match="CPU-resident"):
        stack.layers[0].forward_train_cache(
            x.clone().to("meta"), fit_row_chunk=32, stream_context=True, offload_kv_cache=True
        )
    serial = make_stack(gold, "stack")
    for layer in serial.layers:
        layer.seq_attn_serial = True
    with pytest.raises(NotImplementedError, match="serial sequence attention"):
        serial.build_train_cache(x.clone(), fit_row_chunk=32)


# ------------------------------------------------------------------------------- GPU
@pytest.mark.gpu
@pytest.mark.parametrize("tag", ["attn_mha", "attn_mqa"])
def test_attention_cache_paths_match_reference(gold, cuda, tag):
    attn = make_attn()
    attn.load_state_dict(weights(gold, tag), strict=True)
    attn = attn.to(cuda)
    x_ctx = torch.from_numpy(gold[f"{tag}/x_ctx"]).to(cuda)
    x_q = torch.from_numpy(gold[f"{tag}/x_q"]).to(cuda)
    with torch.inference_mode():
        cache = attn.project_kv_cache(x_ctx, copy_first_head_kv=(tag == "attn_mqa"))
        check(cache["kv"], gold[f"{tag}/kv"], 1e-5)
        dense, _ = attn.forward_with_kv_cache(x_q, cache)
        check(dense, gold[f"{tag}/out_dense"])
        # the int8 cache the reference built, consumed by the kernel as codes + scales
        ref_scal = ScalableSeqKV.from_payload(
            torch.from_numpy(gold[f"{tag}/codes"]).to(cuda), torch.from_numpy(gold[f"{tag}/scales"]).to(cuda), 2, 3,
            dtype=torch.float32,
        )
        check(attn.forward_with_kv_cache(x_q, ref_scal)[0], gold[f"{tag}/out_int8"])
        # this package's own int8 cache of the same K/V
        scal = ScalableSeqKV(cache["kv"], cache["batch"], cache["groups"], quantize=True, device=cuda)
        codes = scal.device_payload()[0].cpu().numpy().astype(np.int32)
        ref_codes = gold[f"{tag}/codes"].astype(np.int32)
        assert np.abs(codes - ref_codes).max() <= 1 and np.mean(codes != ref_codes) < 0.01
        check(attn.forward_with_kv_cache(x_q, scal)[0], gold[f"{tag}/out_int8"])
        # host-streamed blockwise int8 cache, ragged blocks (64, 1, rest)
        n = cache["kv"].shape[1]
        bw = BlockwiseSeqKV.from_row_slices(
            (cache["kv"][:, a:b] for a, b in ((0, 64), (64, 65), (65, n))), cache["batch"], cache["groups"],
            quantize=True, device=cuda, dtype=cache["kv"].dtype, offload=True,
        )
        check(attn.forward_with_kv_cache(x_q, bw)[0], gold[f"{tag}/out_blockwise_int8"])


@pytest.mark.gpu
@pytest.mark.parametrize("tag", ["stack", "stack_mqa"])
@pytest.mark.parametrize("quant", [False, True])
def test_layer_stack_cache_build_and_apply_match_reference(gold, cuda, tag, quant):
    stack = make_stack(gold, tag)
    stack.load_state_dict(weights(gold, tag), strict=True)
    stack = stack.to(cuda)
    x_train = torch.from_numpy(gold[f"{tag}/x_train"]).to(cuda)
    x_test = torch.from_numpy(gold[f"{tag}/x_test"]).to(cuda)
    sfx = "int8" if quant else "fp"
    with torch.inference_mode():
        train_out, caches = stack.build_train_cache(x_train, quantize_kv_cache=quant, device=cuda)
        check(train_out, gold[f"{tag}/train_out_{sfx}"])
        if quant:
            for c in caches:
                assert isinstance(c["seq_kv"], ScalableSeqKV) and c["seq_kv"].device_payload()[0].dtype == torch.int8
            # layer 0's cache comes from the inputs through one norm and one projection, so its
            # codes match the reference's up to the division difference; deeper layers inherit
            # the attention's f16 rounding (~1e-3), which moves codes near a rounding boundary
            d = caches[0]["seq_kv"].device_payload()[0].cpu().numpy().astype(np.int32) - gold[f"{tag}/codes0"].astype(np.int32)
            assert np.abs(d).max() <= 1 and np.mean(d != 0) < 0.01
        test_out = stack.forward_test_with_cache(x_test, caches)
        check(test_out, gold[f"{tag}/test_out_{sfx}"])


# the bounded builds: the reference's own row-chunked / streamed / hybrid outputs (100 context
# rows in chunks of 32, tests/golden/make_golden.py)
ROW_CHUNK = 32
BOUNDED = [("rowchunk", False), ("rowchunk", True), ("stream", False), ("stream", True), ("hybrid", True)]


@pytest.mark.gpu
@pytest.mark.parametrize("tag", ["stack", "stack_mqa"])
@pytest.mark.parametrize("mode,quant", BOUNDED)
def test_bounded_layer_stack_builds_match_reference(gold, cuda, tag, mode, quant):
    stack = make_stack(gold, tag)
    stack.load_state_dict(weights(gold, tag), strict=True)
    stack = stack.to(cuda)
    streamed = mode != "rowchunk"
    # the streamed builds read the context rows from host memory and stage a row chunk at a time
    x_train = torch.from_numpy(gold[f"{tag}/x_train"]).clone()
    if not streamed:
        x_train = x_train.to(cuda)
    x_test = torch.from_numpy(gold[f"{tag}/x_test"]).to(cuda)
    kwargs = dict(quantize_kv_cache=quant, fit_row_chunk=ROW_CHUNK, device=cuda)
    if mode == "stream":
        kwargs.update(stream_context=True, offload_kv_cache=True)
    elif mode == "hybrid":
        kwargs.update(_hybrid_resident_int8_prefill=True)
    sfx = "int8" if quant else "fp"
    with torch.inference_mode():
        train_out, caches = stack.build_train_cache(x_train, **kwargs)
        assert train_out.device.type == ("cpu" if streamed else "cuda")
        check(train_out, gold[f"{tag}/train_out_{mode}_{sfx}"])
        for c in caches:
            skv = c["seq_kv"]
            if mode == "rowchunk":
                assert isinstance(skv, ScalableSeqKV if quant else dict)
            else:
                assert isinstance(skv, BlockwiseSeqKV) and skv.quantized == quant
                # streamed caches live on the host; the hybrid one is one resident int8 payload
                assert skv.offloaded == (mode == "stream")
                assert (skv.resident_payload() is not None) == (mode == "hybrid")
        test_out = stack.forward_test_with_cache(x_test, caches)
        check(test_out, gold[f"{tag}/test_out_{mode}_{sfx}"])
