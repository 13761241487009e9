"""Write golden vectors for the cached sequence-attention layer path and the context-cache API.

Runs the reference's own model code (synthefy_nori.model.layer, .kv_cache_scaling,
.encoders and .transformer: src/synthefy_nori/model/layer.py:459-1162, 1164-1967,
2058-2108; transformer.py:12-61, 564-1139; encoders.py:12-1009) on the CPU in fp32, on
reduced random-init modules built with nori-6m's flags (smf arch, pre-norm RMSNorm, SwiGLU,
deepnorm alpha, isolated sequence attentions, QASS "full", RBF numeric embedding,
target-aware y embedding, a quantile head), and stores their weights, inputs and outputs as
arrays. Nothing else pins these functions: they compose preprocessing statistics, encoders,
projections, QASS, attention, norms and MLPs whose composition has no closed form.

Only this container holds the reference (at /root/reference); the committed product of this
script is the .npz data beside it, never the reference's code. The package's parent
``__init__`` files are skipped (they pull in the product API's optional dependencies): the
model modules import only torch, numpy and einops.

Usage: python tests/golden/make_golden.py   (writes tests/golden/layer_cache_goldens.npz)
"""

from __future__ import annotations

import os
import sys
import types

import numpy as np
import torch

REFERENCE_SRC = "/root/reference/src"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "layer_cache_goldens.npz")


def load_reference():
    for name, sub in (("synthefy_nori", "synthefy_nori"), ("synthefy_nori.model", "synthefy_nori/model")):
        mod = types.ModuleType(name)
        mod.__path__ = [os.path.join(REFERENCE_SRC, sub)]
        sys.modules[name] = mod
    import synthefy_nori.model.kv_cache_scaling as kv_mod
    import synthefy_nori.model.layer as layer_mod

    return layer_mod, kv_mod


# Reduced random-init FeaturesTransformer configurations with nori-6m's flags (model v2-lite:
# SwiGLU, pre-norm RMSNorm, deepnorm alpha, RBF numeric embedding, smf layers, isolated
# sequence attentions, QASS "full", target-aware + column-specific y embedding, a pinball
# quantile head; scripts/train.sh:40-47, 146-148; training/cli.py:1309-1314, 344-352).
# Variant "b" switches on the subortho feature embedding (drawn once, then held fixed so the
# fixture is reproducible), outlier removal, and the shared-head cross cache.
CTX_VARIANTS = {
    "a": dict(pos="none", remove_outliers=False, cross_share=False, column_y=True),
    "b": dict(pos="subortho", remove_outliers=True, cross_share=True, column_y=False),
}


# Bounded cache builds and the cache dtypes each is run with: row-chunked (fit_row_chunk), host
# streamed (stream_context, host-offloaded caches) and the hybrid resident-int8 prefill.
ROW_CHUNK = 32
BOUNDED_BUILDS = (("rowchunk", (False, True)), ("stream", (False, True)), ("hybrid", (True,)))
BOUNDED_KWARGS = {
    "rowchunk": {},
    "stream": dict(stream_context=True, offload_kv_cache=True),
    "hybrid": dict(_hybrid_resident_int8_prefill=True),
}


def ctx_config(v):
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


def ctx_table(gen, b, n, f):
    """Feature table with NaN, +inf, -inf cells, a constant column and a target."""
    x = torch.randn(b, n, f, generator=gen) * torch.tensor([1.0, 3.0, 0.2, 10.0, 1.0])[:f]
    x[:, :, 2] = 0.5  # constant column: not a valid feature
    cells = torch.rand(b, n, f, generator=gen)
    x[cells < 0.05] = float("nan")
    x[(cells > 0.97) & (cells < 0.985)] = float("inf")
    x[cells >= 0.985] = float("-inf")
    y = torch.nan_to_num(x[:, :, 0], nan=0.0, posinf=1.0, neginf=-1.0) * 0.7 + torch.randn(b, n, generator=gen) * 0.1
    return x, y


def perturb_qass(attn, gen):
    """QASS initializes its last layers to zero (q * log n); give them small weights so the
    learned base and gate terms are exercised."""
    if attn.qassmax is None:
        return
    for mlp in (attn.qassmax.base_mlp, attn.qassmax.gate_mlp):
        if mlp is None:
            continue
        with torch.no_grad():
            mlp[-1].weight.copy_(torch.randn(mlp[-1].weight.shape, generator=gen) * 0.1)
            mlp[-1].bias.copy_(torch.randn(mlp[-1].bias.shape, generator=gen) * 0.1)


def row_slices(t, widths):
    start = 0
    for w in widths:
        yield t[:, start : start + w]
        start += w


def main():
    L, K = load_reference()
    torch.set_num_threads(4)
    out: dict[str, np.ndarray] = {}

    def put(prefix, name, t):
        out[f"{prefix}/{name}"] = t.detach().cpu().numpy()

    # ---------------------------------------------------------------- a6 / a7: one attention
    for tag, copy_first in (("mha", False), ("mqa", True)):
        torch.manual_seed(10)
        E, H = 32, 2
        attn = L.MultiheadAttention(E, H, qkv_combined=False, use_qassmax=True, qass_mode="full").eval()
        gen = torch.Generator().manual_seed(11)
        perturb_qass(attn, gen)
        x_ctx = torch.randn(2, 3, 100, E, generator=gen)  # [B, G, N, E] (rows/features transposed)
        x_q = torch.randn(2, 3, 37, E, generator=gen)
        with torch.inference_mode():
            cache = attn.project_kv_cache(x_ctx, copy_first_head_kv=copy_first)
            dense = attn.forward_with_kv_cache(x_q, cache)[0]
            scal = K.ScalableSeqKV(cache["kv"], cache["batch"], cache["groups"], quantize=True, device=torch.device("cpu"))
            int8 = attn.forward_with_kv_cache(x_q, scal)[0]
            bw = K.BlockwiseSeqKV.from_row_slices(
                row_slices(cache["kv"], (64, 1, 35)), cache["batch"], cache["groups"], quantize=True,
                device=torch.device("cpu"), dtype=cache["kv"].dtype, offload=True,
            )
            blockwise = attn.forward_with_kv_cache(x_q, bw)[0]
        p = f"attn_{tag}"
        for k, v in attn.state_dict().items():
            put(p, "w." + k, v)
        put(p, "x_ctx", x_ctx)
        put(p, "x_q", x_q)
        put(p, "kv", cache["kv"])
        put(p, "codes", scal._q)
        put(p, "scales", scal._scale)
        put(p, "out_dense", dense)
        put(p, "out_int8", int8)
        put(p, "out_blockwise_int8", blockwise)

    # ---------------------------------------------------------------- a12 / a13: a two-layer stack
    for tag, cross_share in (("stack", False), ("stack_mqa", True)):
        torch.manual_seed(20)
        E, H, HID, NL = 32, 2, 48, 2
        layers = [
            L.EncoderBaseLayer(
                nhead=H, embed_dim=E, hid_dim=HID, pre_norm=True, activation="swiglu", layer_arch="smf",
                seq_attn_isolated=True, cross_share_all_kv_heads=cross_share, use_qassmax=True,
                norm_type="rmsnorm", deepnorm_alpha=NL ** -0.5, qass_mode="full",
            ).eval()
            for _ in range(NL)
        ]
        gen = torch.Generator().manual_seed(21)
        for layer in layers:
            for attn in layer.sequence_attentions:
                perturb_qass(attn, gen)
            for m in layer.modules():
                if isinstance(m, L.RMSNorm):
                    m.use_native = True  # the serving setting (utils/loading.py:272-277)
        stack = L.LayerStack(layers).eval()
        x_train = torch.randn(2, 100, 3, E, generator=gen)  # [B, N, G, E]
        x_test = torch.randn(2, 29, 3, E, generator=gen)
        p = tag
        with torch.inference_mode():
            for quant in (False, True):
                xt = x_train.clone()
                xt_out, caches = stack.build_train_cache(xt, quantize_kv_cache=quant, device=torch.device("cpu"))
                y = stack.forward_test_with_cache(x_test.clone(), caches)
                sfx = "int8" if quant else "fp"
                put(p, f"train_out_{sfx}", xt_out)
                put(p, f"test_out_{sfx}", y)
                for i, c in enumerate(caches):
                    skv = c["seq_kv"]
                    if quant:
                        put(p, f"codes{i}", skv._q)
                        put(p, f"scales{i}", skv._scale)
            # the bounded builds (layer.py:1482-1769): 100 context rows in chunks of 32, the last
            # one ragged; row-chunked (memsaving), host-streamed, and the hybrid resident-int8 prefill
            for mode, quants in BOUNDED_BUILDS:
                for quant in quants:
                    kwargs = dict(quantize_kv_cache=quant, fit_row_chunk=ROW_CHUNK, device=torch.device("cpu"))
                    kwargs.update(BOUNDED_KWARGS[mode])
                    xt_out, caches = stack.build_train_cache(x_train.clone(), **kwargs)
                    y = stack.forward_test_with_cache(x_test.clone(), caches)
                    sfx = "int8" if quant else "fp"
                    put(p, f"train_out_{mode}_{sfx}", xt_out)
                    put(p, f"test_out_{mode}_{sfx}", y)
        for k, v in stack.state_dict().items():
            put(p, "w." + k, v)
        put(p, "x_train", x_train)
        put(p, "x_test", x_test)
        out[f"{p}/config"] = np.array([E, H, HID, NL, int(cross_share)], dtype=np.int64)

    # ---------------------------------------------------------------- a14: context-cache API
    import synthefy_nori.model.transformer as T

    for tag, v in CTX_VARIANTS.items():
        torch.manual_seed(30)
        model = T.FeaturesTransformer(**ctx_config(v)).eval()
        gen = torch.Generator().manual_seed(31)
        for m in model.modules():
            if isinstance(m, L.RMSNorm):
                m.use_native = True
            if isinstance(m, L.MultiheadAttention):
                perturb_qass(m, gen)
        with torch.no_grad():
            # random init leaves the head's output near its bias; spread the quantiles and scale
            # the head so the predictions move by O(1) with the inputs
            model.reg_y_decoder[-1].bias.copy_(torch.linspace(-1.0, 1.0, 7))
            model.reg_y_decoder[-1].weight.mul_(30.0)
        p = f"ctx_{tag}"
        if v["pos"] == "subortho":
            fixed = model.make_feature_positional_embeddings(3, device=torch.device("cpu"), dtype=torch.float32).detach()
            model.make_feature_positional_embeddings = lambda n_groups, *, device, dtype, e=fixed: e.to(device, dtype)
            put(p, "feature_pos_emb", fixed)
        x, y = ctx_table(gen, 2, 113, 5)
        n_ctx = 90
        seen = {}
        stack_apply = model.transformer_encoder.forward_test_with_cache

        def capture(*args, _f=stack_apply, **kwargs):  # the layer stack's output for the query rows
            seen["out"] = _f(*args, **kwargs)
            return seen["out"]

        model.transformer_encoder.forward_test_with_cache = capture
        stack_build = model.transformer_encoder.build_train_cache

        def capture_tokens(tokens, *args, _f=stack_build, **kwargs):  # the encoded context tokens
            seen["tokens"] = tokens
            return _f(tokens, *args, **kwargs)

        model.transformer_encoder.build_train_cache = capture_tokens
        with torch.inference_mode():
            for cache_dtype in ("bf16", "int8"):
                ctx = model.build_context_cache(x[:, :n_ctx], y[:, :n_ctx], cache_dtype=cache_dtype)
                pred = model.apply_context_cache(x[:, n_ctx:], ctx)
                put(p, f"pred_{cache_dtype}", pred)
                put(p, f"stack_out_{cache_dtype}", seen["out"])
                if cache_dtype == "int8":
                    put(p, "codes0", ctx.caches[0]["seq_kv"]._q)
                else:
                    put(p, "kv0", ctx.caches[0]["seq_kv"]["kv"])
            put(p, "tokens", seen["tokens"])
            for k, t in (ctx.norm_stats or {}).items():
                put(p, f"norm_{k}", t)
            put(p, "nan_mean", ctx.nan_mean)
            put(p, "valid_feature_num", ctx.valid_feature_num)
            # the bounded context builds (transformer.py:1169-1301 for the streamed ones), applied
            # in query chunks of 16
            for mode, quants in BOUNDED_BUILDS:
                for quant in quants:
                    cache_dtype = "int8" if quant else "bf16"
                    kwargs = dict(fit_row_chunk=ROW_CHUNK)
                    if mode == "stream":
                        kwargs.update(stream_context=True, offload_kv_cache=True)
                    elif mode == "hybrid":
                        kwargs.update(_hybrid_resident_int8_prefill=True)
                    ctx = model.build_context_cache(x[:, :n_ctx], y[:, :n_ctx], cache_dtype=cache_dtype, **kwargs)
                    pred = model.apply_context_cache(x[:, n_ctx:], ctx, row_chunk_size=16)
                    put(p, f"pred_{mode}_{cache_dtype}", pred)
        for k, t in model.state_dict().items():
            put(p, "w." + k, t)
        put(p, "x", x)
        put(p, "y", y)
        out[f"{p}/n_ctx"] = np.array(n_ctx, dtype=np.int64)

    np.savez_compressed(OUT, **out)
    total = sum(v.nbytes for v in out.values())
    print(f"wrote {OUT}: {len(out)} arrays, {total / 1e6:.2f} MB uncompressed")


if __name__ == "__main__":
    main()
