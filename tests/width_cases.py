"""Model-level cases at the long-context models' head widths (44 and 56), shared by
tests/golden/make_width_golden.py, which runs the reference's own modules on them, and
tests/test_golden_widths.py, which holds this package's HIP path to the reference's outputs.

Two heads of 44 (embed 88) and of 56 (embed 112): the head widths of the nori-30m and nori-100m
models (src/synthefy_nori/model/layer.py:859-861), which are not multiples of 16, so the cached
attention runs its folded mode (the running max and the denominator carried by padding
columns); 33 and 51 tokens a row (64 and 100 features, two per token, plus the target token),
the row widths of the long-context and batched tables, so the feature attention over a row's
tokens runs on the few-token kernel under fp16 autocast; QASS "full"; a few hundred context
rows. Each case is one layer stack (``LayerStack.build_train_cache`` /
``forward_test_with_cache``) or one model (``FeaturesTransformer.build_context_cache`` /
``apply_context_cache``) with nori-6m's flags.

The tables, inputs and weights are drawn from numpy's default_rng (the same bits on every
machine): every random parameter is uniform with the mean and standard deviation the reference
constructor gives it (a table measured once by the golden recipe and stored with the fixture),
so the fixture carries that table and the weights' SHA-256, not the weights.
"""

from __future__ import annotations

import numpy as np
import torch

# tag -> (embed, heads, hidden, layers, tokens a row (stacks) / features (models), context rows, query rows)
STACKS = {
    "stack44": dict(embed=88, heads=2, hid=264, layers=2, tokens=33, n_ctx=256, n_q=64),
    "stack56": dict(embed=112, heads=2, hid=336, layers=2, tokens=51, n_ctx=192, n_q=48),
}
MODELS = {
    "ctx44": dict(embed=88, heads=2, hid=264, layers=2, features=64, n_ctx=300, n_q=64),
    "ctx56": dict(embed=112, heads=2, hid=336, layers=2, features=100, n_ctx=200, n_q=48),
}
QUANTILES = [0.05, 0.1, 0.25, 0.5, 0.75, 0.9, 0.95]
# context-row permutations whose outputs measure the fp16-autocast run's own sensitivity to
# summation order (the outputs are invariant to the order of the context rows)
SPREAD_PERMUTATIONS = 3
# the fixture keeps the context rows' outputs of every ROW_STEP-th row and layer 0's int8 codes of
# the first CODE_ROWS context rows
ROW_STEP = 16
CODE_ROWS = 16
# and the query rows' outputs of every QUERY_STEP-th query row
QUERY_STEP = 2


def layer_kwargs(c: dict) -> dict:
    return dict(
        nhead=c["heads"], embed_dim=c["embed"], hid_dim=c["hid"], pre_norm=True, activation="swiglu", layer_arch="smf",
        seq_attn_isolated=True, cross_share_all_kv_heads=False, use_qassmax=True, norm_type="rmsnorm",
        deepnorm_alpha=c["layers"] ** -0.5, qass_mode="full",
    )


def model_config(c: dict) -> dict:
    e = c["embed"]
    return dict(
        preprocess_config_x=dict(num_features=2, nan_handling_enabled=True, normalize_on_train_only=True,
                                 normalize_x=True, remove_outliers=False, normalize_by_used_features=True),
        encoder_config_x=dict(num_features=2, embedding_size=e, mask_embedding_size=e, encoder_use_bias=True,
                              numeric_embed_type="RBF",
                              RBF_config=dict(token_embed_dim=8, n_kernels=16, sigma=0.5, use_learn_sigma=False,
                                              use_learn_embeddings=False, use_original_features=False)),
        encoder_config_y=dict(num_inputs=1, embedding_size=e, nan_handling_y_encoder=True, max_num_classes=10),
        decoder_config=dict(num_classes=10, num_reg_quantiles=len(QUANTILES), regression_loss="pinball",
                            regression_quantiles=list(QUANTILES)),
        nlayers=c["layers"], nhead=c["heads"], embed_dim=e, hid_dim=c["hid"], features_per_group=2, dropout=0.0,
        pre_norm=True, activation="swiglu", norm_type="rmsnorm", deepnorm_alpha=c["layers"] ** -0.5,
        layer_arch="smf", feature_positional_embedding_type="none", seq_attn_isolated=True,
        cross_share_all_kv_heads=False, use_qassmax=True, qass_mode="full", use_target_aware_embedding=True,
        use_column_specific_y_aware=True,
    )


def stack_inputs(tag: str):
    """x_train [1, n_ctx, tokens, embed], x_test [1, n_q, tokens, embed], float32 N(0, 1)."""
    c = STACKS[tag]
    rng = np.random.default_rng(100 + c["embed"])
    x_train = rng.standard_normal((1, c["n_ctx"], c["tokens"], c["embed"])).astype(np.float32)
    x_test = rng.standard_normal((1, c["n_q"], c["tokens"], c["embed"])).astype(np.float32)
    return x_train, x_test


def model_table(tag: str):
    """x [1, n_ctx + n_q, features] float32 N(0, 1) with 5 % NaN cells, y [1, n_ctx] a nonlinear
    target (a sum of pairwise products over the first features, scaled, plus noise)."""
    c = MODELS[tag]
    rng = np.random.default_rng(200 + c["embed"])
    n, f = c["n_ctx"] + c["n_q"], c["features"]
    x = rng.standard_normal((1, n, f))
    y = (x[..., 0:16:2] * x[..., 1:16:2]).sum(-1) / 4.0 + 0.5 * x[..., 16] + 0.1 * rng.standard_normal((1, n))
    x[rng.random(x.shape) < 0.05] = np.nan
    return x.astype(np.float32), y[:, : c["n_ctx"]].astype(np.float32)


def permutations(n: int) -> list[np.ndarray]:
    return [np.random.default_rng(300 + s).permutation(n) for s in range(SPREAD_PERMUTATIONS)]


def relative(a, b) -> float:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    s = np.abs(b).max()
    return float(np.abs(a - b).max() / (s if s > 0 else 1.0))


def seeded_state(template: dict, scales: dict, seed: int, head: str | None = None) -> dict:
    """A state dict with the keys and shapes of ``template``, each random parameter (sorted by
    name) mean + std * sqrt(3) * (2u - 1) with u from numpy's default_rng(seed) and the (mean,
    std) of ``scales``, constants (std 0) at their value. The QASS MLPs' output layers, which the
    constructor zeroes, get small weights from the same stream (so the base and gate terms are
    exercised); ``head`` names a quantile head's output layer, whose bias then spreads over
    [-1, 1] and whose weight is scaled by 30, so the predictions move by O(1) with the inputs."""
    rng = np.random.default_rng(seed)
    new = {}
    for name in sorted(template):
        mean, std = scales[name]
        shape = tuple(template[name].shape)
        if std == 0.0:
            values = np.full(shape, mean, dtype=np.float64)
        else:
            values = mean + std * np.sqrt(3.0) * (2.0 * rng.random(shape) - 1.0)
        if ".qassmax." in name and name.rsplit(".", 2)[-2] == "2":  # the QASS MLPs' output layers
            values = 0.1 * np.sqrt(3.0) * (2.0 * rng.random(shape) - 1.0)
        new[name] = values
    if head is not None:
        n = new[f"{head}.bias"].shape[0]
        new[f"{head}.bias"] = np.linspace(-1.0, 1.0, n)
        new[f"{head}.weight"] = new[f"{head}.weight"] * 30.0
    return {k: torch.from_numpy(v.astype(np.float32)) for k, v in new.items()}


def head_name(model) -> str:
    return f"reg_y_decoder.{len(model.reg_y_decoder) - 1}"
