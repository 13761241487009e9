"""Parity of the context-cache API with the reference's own outputs.

tests/golden/layer_cache_goldens.npz ("ctx_a", "ctx_b") holds the weights, a feature table
with NaN / +inf / -inf cells and a constant column, and the outputs of the reference's
``FeaturesTransformer.build_context_cache`` / ``apply_context_cache``
(src/synthefy_nori/model/transformer.py:813-1078) run on the CPU in fp32 by
tests/golden/make_golden.py: the encoded context tokens, the captured context statistics,
layer 0's K/V cache (fp and int8), the layer stack's output for the query rows and the
quantile predictions, for reduced random-init models with nori-6m's flags.

CPU tests: the state dicts load strictly; the preprocessing and encoders reproduce the
reference's context tokens and statistics (fp32 on both sides, up to summation order); the
unsupported levers raise; the query-chunk OOM ladder halves and reports as the reference's.
GPU tests: the whole build/apply through the HIP kernels. The layer K/V cache from the
context encode is fp32 end to end: device and host differ only in summation order, which
the normalizations amplify to ~3e-4 relative at worst. The layer stack's output and the
quantile predictions are held to a relative error max|got - exp| / max|exp| <= 1e-3, the
bar for predictions (measured near 2e-6; each check prints its figure).
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch
from parity import PREDICTION_BAR, check_relative

from nori_amd import transformer as NT

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "layer_cache_goldens.npz")
# Mirrors the configurations tests/golden/make_golden.py builds the reference models with.
VARIANTS = {
    "a": dict(pos="none", remove_outliers=False, cross_share=False, column_y=True),
    "b": dict(pos="subortho", remove_outliers=True, cross_share=True, column_y=False),
}


def config(v):
    return dict(
        preprocess_config_x=dict(
            num_features=2, nan_handling_enabled=True, normalize_on_train_only=True, normalize_x=True,
            remove_outliers=v["remove_outliers"], normalize_by_used_features=True,
        ),
        encoder_config_x=dict(
            num_features=2, embedding_size=32, mask_embedding_size=32, encoder_use_bias=True, numeric_embed_type="RBF",
            RBF_config=dict(token_embed_dim=8, n_kernels=16, sigma=0.5, use_learn_sigma=False,
                            use_learn_embeddings=False, use_original_features=False),
        ),
        encoder_config_y=dict(num_inputs=1, embedding_size=32, nan_handling_y_encoder=True, max_num_classes=10),
        decoder_config=dict(num_classes=10, num_reg_quantiles=7, regression_loss="pinball",
                            regression_quantiles=[0.05, 0.1, 0.25, 0.5, 0.75, 0.9, 0.95]),
        nlayers=2, nhead=2, embed_dim=32, hid_dim=48, features_per_group=2, dropout=0.0, pre_norm=True,
        activation="swiglu", norm_type="rmsnorm", deepnorm_alpha=2 ** -0.5, layer_arch="smf",
        feature_positional_embedding_type=v["pos"], seq_attn_isolated=True, cross_share_all_kv_heads=v["cross_share"],
        use_qassmax=True, qass_mode="full", use_target_aware_embedding=True, use_column_specific_y_aware=v["column_y"],
    )


@pytest.fixture(scope="module")
def gold():
    with np.load(GOLDEN, allow_pickle=False) as f:
        return {k: f[k] for k in f.files if k.startswith("ctx_")}


def make_model(gold, tag, device="cpu"):
    model = NT.FeaturesTransformer(**config(VARIANTS[tag])).eval()
    prefix = f"ctx_{tag}/w."
    model.load_state_dict({k[len(prefix):]: torch.from_numpy(v) for k, v in gold.items() if k.startswith(prefix)}, strict=True)
    model = model.to(device)
    if f"ctx_{tag}/feature_pos_emb" in gold:  # the fixture holds the subortho draw fixed
        fixed = torch.from_numpy(gold[f"ctx_{tag}/feature_pos_emb"])
        model.make_feature_positional_embeddings = lambda n_groups, *, device, dtype: fixed.to(device, dtype)
    return model


def table(gold, tag, device="cpu"):
    x = torch.from_numpy(gold[f"ctx_{tag}/x"]).to(device)
    y = torch.from_numpy(gold[f"ctx_{tag}/y"]).to(device)
    return x, y, int(gold[f"ctx_{tag}/n_ctx"])


def check(got, exp, bar=PREDICTION_BAR):
    """max|got - exp| / max|exp| <= bar (relative 1e-3 by default, the bar for predictions)."""
    got = torch.as_tensor(got).detach()
    exp = torch.as_tensor(exp)
    assert tuple(got.shape) == tuple(exp.shape), (tuple(got.shape), tuple(exp.shape))
    test = os.environ.get("PYTEST_CURRENT_TEST", "?").split(" ")[0]
    return check_relative(got, exp, bar, test)


def encode_context(model, x, y, n_ctx):
    """The context half of build_context_cache up to the layer stack: (tokens, statistics)."""
    seen = {}

    def capture(tokens, *args, **kwargs):
        seen["tokens"] = tokens
        raise StopIteration

    model.transformer_encoder.build_train_cache = capture
    with pytest.raises(StopIteration):
        model.build_context_cache(x[:, :n_ctx], y[:, :n_ctx])
    return seen["tokens"]


# ------------------------------------------------------------------------------- CPU
@pytest.mark.parametrize("tag", ["a", "b"])
def test_model_takes_the_reference_state_dict(gold, tag):
    make_model(gold, tag)


@pytest.mark.parametrize("tag", ["a", "b"])
def test_context_encoding_matches_reference_tokens_and_statistics(gold, tag):
    # preprocessing (NaN fill, outlier clip, normalization, valid-feature scaling), the RBF x
    # encoder, the y encoder and the target-aware embedding, all fp32 / fp64 torch on the CPU
    model = make_model(gold, tag)
    x, y, n_ctx = table(gold, tag)
    with torch.inference_mode():
        tokens = encode_context(model, x, y, n_ctx)
        x_dict, _ = model._build_x_preprocess_inputs(x[:, :n_ctx], n_ctx)
        pre = model.x_preprocess(x_dict)
    exp = gold[f"ctx_{tag}/tokens"]
    assert tokens.shape == exp.shape
    np.testing.assert_allclose(tokens.numpy(), exp, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(pre["_nan_mean"].numpy(), gold[f"ctx_{tag}/nan_mean"], rtol=1e-6, atol=1e-6)
    assert np.array_equal(pre["_valid_feature_num"].numpy(), gold[f"ctx_{tag}/valid_feature_num"])
    for k, v in pre["_norm_stats"].items():
        np.testing.assert_allclose(v.numpy(), gold[f"ctx_{tag}/norm_{k}"], rtol=1e-6, atol=1e-6)


def test_query_rows_use_the_frozen_context_statistics(gold):
    # encoding query rows alone with the captured context statistics equals encoding them as
    # the tail of the whole table (the transductive semantics the cache must keep)
    model = make_model(gold, "b")
    x, _, n_ctx = table(gold, "b")
    with torch.inference_mode():
        whole, _ = model._build_x_preprocess_inputs(x, n_ctx)
        whole = model.process_4_x(model.x_preprocess(whole))
        ctx, _ = model._build_x_preprocess_inputs(x[:, :n_ctx], n_ctx)
        ctx = model.x_preprocess(ctx)
        q, _ = model._build_x_preprocess_inputs(x[:, n_ctx:], x.shape[1] - n_ctx)
        q["_frozen_norm_stats"] = ctx["_norm_stats"]
        q["_frozen_nan_mean"] = ctx["_nan_mean"]
        q["_frozen_valid_feature_num"] = ctx["_valid_feature_num"]
        q = model.process_4_x(model.x_preprocess(q))
    torch.testing.assert_close(q["data"], whole["data"][:, n_ctx:], rtol=0, atol=0, equal_nan=True)


def test_unsupported_and_invalid_levers_raise(gold):
    model = make_model(gold, "a")
    x, y, n_ctx = table(gold, "a")
    with pytest.raises(ValueError, match="requires a concrete context_row_chunk"):
        model.build_context_cache(x[:, :n_ctx], y[:, :n_ctx], stream_context=True, offload_kv_cache=True)
    with pytest.raises(ValueError, match="hybrid resident INT8 prefill requires"):
        model.build_context_cache(x[:, :n_ctx], y[:, :n_ctx], _hybrid_resident_int8_prefill=True, fit_row_chunk=32)
    with pytest.raises(ValueError, match="requires CPU x_train"):
        model.build_context_cache(x[:, :n_ctx].to("meta"), y[:, :n_ctx], stream_context=True, offload_kv_cache=True,
                                  fit_row_chunk=32)
    with pytest.raises(ValueError, match="stream_context requires offload_kv_cache"):
        model.build_context_cache(x[:, :n_ctx], y[:, :n_ctx], stream_context=True, fit_row_chunk=32)
    with pytest.raises(ValueError, match="concrete cache_dtype"):
        model.build_context_cache(x[:, :n_ctx], y[:, :n_ctx], cache_dtype="fp8")
    two_phase = NT.FeaturesTransformer(
        **config(VARIANTS["a"]), two_phase_config={"target_tokens": 1, "row_layers": 1, "row_heads": 2, "row_hidden_dim": 32}
    )
    with pytest.raises(NotImplementedError, match="two-phase"):
        two_phase.build_context_cache(x[:, :n_ctx], y[:, :n_ctx])
    cfg = config(VARIANTS["a"])
    cfg["preprocess_config_x"] = dict(cfg["preprocess_config_x"], normalize_on_train_only=False)
    with pytest.raises(NotImplementedError, match="normalize_on_train_only"):
        NT.FeaturesTransformer(**cfg).build_context_cache(x[:, :n_ctx], y[:, :n_ctx])


def test_query_chunks_halve_on_out_of_memory(gold):
    # the OOM ladder of apply_context_cache (transformer.py:1051-1078), driven from the host: the
    # layer stack runs out of memory on chunks wider than 5 rows
    model = make_model(gold, "a")
    x, _, n_ctx = table(gold, "a")
    n_q = x.shape[1] - n_ctx
    widths = []

    def stack(tokens, caches, feature_atten_mask=None):
        if tokens.shape[1] > 5:
            raise torch.cuda.OutOfMemoryError("synthetic")
        widths.append(tokens.shape[1])
        return tokens

    model.transformer_encoder.forward_test_with_cache = stack
    model.encoder_out_norm = torch.nn.Identity()
    context = NT.ContextCache(caches=[], feature_pos_emb=None, norm_stats=None, y_train=torch.from_numpy(gold["ctx_a/y"][:, :n_ctx]),
                              eval_pos=n_ctx)
    events = []
    with torch.inference_mode():
        out = model.apply_context_cache(x[:, n_ctx:], context, row_chunk_size=16, query_chunk_attempt_callback=lambda c, e: events.append((c, e)))
    assert out.shape == (2, n_q, 7)
    assert events == [(16, "oom"), (8, "oom"), (4, "success")]
    assert sum(widths) == n_q and max(widths) == 4
    with pytest.raises(torch.cuda.OutOfMemoryError):
        model.apply_context_cache(x[:, n_ctx:], context, row_chunk_size=16, adaptive_query_chunk=False)


# ------------------------------------------------------------------------------- GPU
@pytest.mark.gpu
@pytest.mark.parametrize("tag", ["a", "b"])
@pytest.mark.parametrize("cache_dtype", ["bf16", "int8"])
def test_build_and_apply_match_reference(gold, cuda, tag, cache_dtype):
    model = make_model(gold, tag, cuda)
    x, y, n_ctx = table(gold, tag, cuda)
    seen = {}
    stack_apply = model.transformer_encoder.forward_test_with_cache

    def capture(*args, **kwargs):
        seen["out"] = stack_apply(*args, **kwargs)
        return seen["out"]

    model.transformer_encoder.forward_test_with_cache = capture
    with torch.inference_mode():
        ctx = model.build_context_cache(x[:, :n_ctx], y[:, :n_ctx], cache_dtype=cache_dtype)
        pred = model.apply_context_cache(x[:, n_ctx:], ctx)
    assert ctx.eval_pos == n_ctx and len(ctx.caches) == 2
    assert np.array_equal(ctx.valid_feature_num.cpu().numpy(), gold[f"ctx_{tag}/valid_feature_num"])
    check(ctx.nan_mean, gold[f"ctx_{tag}/nan_mean"], 1e-5)
    if cache_dtype == "bf16":
        check(ctx.caches[0]["seq_kv"]["kv"], gold[f"ctx_{tag}/kv0"], 1e-3)
    else:
        d = ctx.caches[0]["seq_kv"].device_payload()[0].cpu().numpy().astype(np.int32) - gold[f"ctx_{tag}/codes0"].astype(np.int32)
        assert np.abs(d).max() <= 1 and np.mean(d != 0) < 0.01
    check(seen["out"], gold[f"ctx_{tag}/stack_out_{cache_dtype}"])
    check(pred, gold[f"ctx_{tag}/pred_{cache_dtype}"])


@pytest.mark.gpu
def test_forward_cached_regression_and_chunked_apply_agree(gold, cuda):
    model = make_model(gold, "a", cuda)
    x, y, n_ctx = table(gold, "a", cuda)
    with torch.inference_mode():
        ctx = model.build_context_cache(x[:, :n_ctx], y[:, :n_ctx], cache_dtype="int8")
        whole = model.apply_context_cache(x[:, n_ctx:], ctx)
        chunked = model.apply_context_cache(x[:, n_ctx:], ctx, row_chunk_size=7)
        again = model.apply_context_cache(x[:, n_ctx:], ctx)  # the bundle is not mutated
        pair = model.forward_cached_regression(x, y, n_ctx, cache_dtype="int8")
    torch.testing.assert_close(again, whole, rtol=0, atol=0)
    torch.testing.assert_close(pair, whole, rtol=0, atol=0)
    # chunks change only the query count of each attention launch (same per-row arithmetic
    # up to the kernel's per-launch schedule)
    torch.testing.assert_close(chunked, whole, rtol=1e-4, atol=1e-4)


# the bounded builds (tests/golden/make_golden.py): row-chunked, host-streamed and hybrid
# resident-int8 context builds in chunks of 32 context rows, applied in query chunks of 16
ROW_CHUNK = 32
BOUNDED = [("rowchunk", "bf16"), ("rowchunk", "int8"), ("stream", "bf16"), ("stream", "int8"), ("hybrid", "int8")]


@pytest.mark.gpu
@pytest.mark.parametrize("tag", ["a", "b"])
@pytest.mark.parametrize("mode,cache_dtype", BOUNDED)
def test_bounded_context_builds_match_reference(gold, cuda, tag, mode, cache_dtype):
    model = make_model(gold, tag, cuda)
    streamed = mode != "rowchunk"
    # the streamed builds and their apply keep the raw tables on the host
    x, y, n_ctx = table(gold, tag, "cpu" if streamed else cuda)
    kwargs = dict(fit_row_chunk=ROW_CHUNK)
    if mode == "stream":
        kwargs.update(stream_context=True, offload_kv_cache=True)
    elif mode == "hybrid":
        kwargs.update(_hybrid_resident_int8_prefill=True)
    with torch.inference_mode():
        ctx = model.build_context_cache(x[:, :n_ctx], y[:, :n_ctx], cache_dtype=cache_dtype, **kwargs)
        pred = model.apply_context_cache(x[:, n_ctx:], ctx, row_chunk_size=16)
    assert ctx.eval_pos == n_ctx and len(ctx.caches) == 2
    if streamed:
        # the query target embedding is drawn once from the context mean; the context targets
        # are not kept
        assert ctx.query_y_embedding is not None and ctx.y_train.shape[1] == 0
        for c in ctx.caches:
            assert c["seq_kv"].offloaded == (mode == "stream")
    check(pred, gold[f"ctx_{tag}/pred_{mode}_{cache_dtype}"])
