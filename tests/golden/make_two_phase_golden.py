"""Write golden vectors for the two-phase encoder (Nori 1.5) and its prompt-quantile PLE cells.

Runs the reference's own model code (synthefy_nori.model.transformer with
.two_phase, .encoders and .layer: src/synthefy_nori/model/two_phase.py:1-486,
transformer.py:370-562, encoders.py:309-585, 972-1009) on the CPU in fp32, on reduced
random-init two-phase models built with Nori 1.5's flags (RBF + prompt-quantile PLE cell
tokens, SwiGLU, RMSNorm, target-aware + column-specific y embedding, a pinball quantile head;
the reference's tests/test_model_v3.py:21-56 builds the same kind of model), and stores their
weights, inputs and outputs as arrays. Nothing else pins these functions: the composition of
preprocessing, PLE edges, cell/row layers and decoders has no closed form.

Only this container holds the reference (at /root/reference); the committed product of this
script is the .npz data beside it, never the reference's code. The package's parent
``__init__`` files are skipped (they pull in the product API's optional dependencies).

Usage: python tests/golden/make_two_phase_golden.py   (writes tests/golden/two_phase_goldens.npz)
"""

from __future__ import annotations

import os
import sys
import types

import numpy as np
import torch

REFERENCE_SRC = "/root/reference/src"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "two_phase_goldens.npz")

TWO_PHASE = dict(target_tokens=2, row_layers=2, row_heads=4, row_hidden_dim=96)
PLE_BINS = 8
# Variant "a": two features per group, no positional embedding. Variant "b": one feature per
# group and the subortho feature embedding (its draw is recorded so the fixture is fixed).
VARIANTS = {"a": dict(fpg=2, pos="none"), "b": dict(fpg=1, pos="subortho")}
ROWS, EVAL_POS, FEATURES = 40, 28, 5


def load_reference():
    for name, sub in (("synthefy_nori", "synthefy_nori"), ("synthefy_nori.model", "synthefy_nori/model")):
        mod = types.ModuleType(name)
        mod.__path__ = [os.path.join(REFERENCE_SRC, sub)]
        sys.modules[name] = mod
    import synthefy_nori.model.encoders as encoders_mod
    import synthefy_nori.model.layer as layer_mod
    import synthefy_nori.model.transformer as transformer_mod

    return layer_mod, transformer_mod, encoders_mod


def model_config(v):
    fpg = v["fpg"]
    return dict(
        preprocess_config_x=dict(
            num_features=fpg, nan_handling_enabled=True, normalize_on_train_only=True, normalize_x=True,
            remove_outliers=False, normalize_by_used_features=True, prompt_quantile_ple_bins=PLE_BINS,
        ),
        encoder_config_x=dict(
            num_features=fpg, embedding_size=32, mask_embedding_size=32, encoder_use_bias=True, numeric_embed_type="RBF",
            RBF_config=dict(token_embed_dim=8, n_kernels=16, sigma=0.5, use_learn_sigma=False,
                            use_learn_embeddings=False, use_original_features=False),
            prompt_quantile_ple_bins=PLE_BINS,
        ),
        encoder_config_y=dict(num_inputs=1, embedding_size=32, nan_handling_y_encoder=True, max_num_classes=10),
        decoder_config=dict(num_reg_quantiles=9, regression_loss="pinball"),
        nlayers=2, nhead=2, embed_dim=32, hid_dim=64, features_per_group=fpg, dropout=0.0, pre_norm=True,
        activation="swiglu", norm_type="rmsnorm", deepnorm_alpha=4 ** -0.5,
        feature_positional_embedding_type=v["pos"], use_target_aware_embedding=True, use_column_specific_y_aware=True,
        use_qassmax=True, qass_mode="log_only", omit_feature_decoder=True, two_phase_config=dict(TWO_PHASE),
    )


def table(gen):
    """Two tables of 40 rows x 5 features: NaN, +inf, -inf cells, a constant column (zero-width
    PLE bins), a column with repeated values, and a target."""
    x = torch.randn(2, ROWS, FEATURES, generator=gen) * torch.tensor([1.0, 3.0, 0.2, 10.0, 1.0])
    x[:, :, 2] = 0.5
    x[:, :, 4] = torch.randint(0, 3, (2, ROWS), generator=gen).float()
    cells = torch.rand(2, ROWS, FEATURES, generator=gen)
    x[cells < 0.05] = float("nan")
    x[(cells > 0.97) & (cells < 0.985)] = float("inf")
    x[cells >= 0.985] = float("-inf")
    y = torch.nan_to_num(x[:, :, 0], nan=0.0, posinf=1.0, neginf=-1.0) * 0.7 + torch.randn(2, ROWS, generator=gen) * 0.1
    return x, y


def main():
    L, T, E = load_reference()
    torch.set_num_threads(4)
    out: dict[str, np.ndarray] = {}

    def put(name, t):
        out[name] = t.detach().cpu().numpy() if torch.is_tensor(t) else np.asarray(t)

    for tag, v in VARIANTS.items():
        torch.manual_seed(30)
        model = T.FeaturesTransformer(**model_config(v)).eval()
        gen = torch.Generator().manual_seed(31)
        with torch.no_grad():
            for m in model.modules():
                if isinstance(m, L.RMSNorm):
                    m.use_native = True  # the serving setting (utils/loading.py:272-277)
                    if m.weight is not None:  # the per-head q/k norm gains start at one
                        m.weight.mul_(1.0 + 0.2 * torch.randn(m.weight.shape, generator=gen))
        x, y = table(gen)
        y_ctx = y[:, :EVAL_POS]
        drawn = []
        if v["pos"] == "subortho":
            model.feature_positional_embedding.register_forward_hook(lambda mod, inp, res: drawn.append(res.detach().clone()))
        p = f"tp_{tag}"
        with torch.no_grad():
            pre, _ = model._build_x_preprocess_inputs(x.clone(), EVAL_POS)
            pre = model.x_preprocess(pre)
            edges = pre["_prompt_quantile_ple_reference"]["edges"]
            ple = E.PromptQuantilePLEEncoder.encode(pre["data"], pre["_prompt_quantile_ple_reference"])
            torch.manual_seed(32)
            reg = model(x=x.clone(), y=y_ctx.clone(), eval_pos=EVAL_POS, task_type="reg")
            torch.manual_seed(32)
            rows = model(x=x.clone(), y=y_ctx.clone(), eval_pos=EVAL_POS, task_type="reg", return_embeddings=True)
            # the chunked encoder on the same embedded cells (its own entry point, :380-486)
            captured = {}

            def grab(mod, args, kwargs):
                captured["cells"] = args[0].detach().clone()
                captured["y"] = args[1].detach().clone()

            h = model.transformer_encoder.register_forward_pre_hook(grab, with_kwargs=True)
            torch.manual_seed(32)
            model(x=x.clone(), y=y_ctx.clone(), eval_pos=EVAL_POS, task_type="reg")
            h.remove()
            chunked = model.transformer_encoder.forward_chunked(
                captured["cells"].clone(), captured["y"], EVAL_POS, row_chunk=16, column_chunk=2,
                compute_device=torch.device("cpu"),
            )
        for k, w in model.state_dict().items():
            put(f"{p}/w.{k}", w)
        put(f"{p}/x", x)
        put(f"{p}/y", y_ctx)
        put(f"{p}/pre_data", pre["data"])
        put(f"{p}/pre_mask", pre["mask"])
        put(f"{p}/ple_edges", edges)
        put(f"{p}/ple_coords", ple)
        put(f"{p}/reg", reg)
        put(f"{p}/rows", rows)
        put(f"{p}/enc_cells", captured["cells"])
        put(f"{p}/enc_y", captured["y"])
        put(f"{p}/chunked_rows", chunked)
        if drawn:
            put(f"{p}/feature_pos_emb", drawn[0])
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT}: {len(out)} arrays, {os.path.getsize(OUT) / 1e6:.2f} MB")


if __name__ == "__main__":
    main()
