"""Parity of the two-phase encoder (Nori 1.5) and its PLE cell tokens with the reference's outputs.

tests/golden/two_phase_goldens.npz ("tp_a": two features per group; "tp_b": one feature per
group with the subortho feature embedding held fixed) holds the weights, a table with NaN /
+inf / -inf cells, a constant column and a column of repeated values, and what the
reference's ``FeaturesTransformer.forward`` (src/synthefy_nori/model/transformer.py:370-562,
two_phase.py:287-486) computes from it on the CPU in fp32 (tests/golden/make_two_phase_golden.py):
the preprocessed cells, the prompt-quantile PLE edges and coordinates (encoders.py:309-429),
the quantile predictions of the query rows, the row states, the encoder input and the
chunked encoder's row states.

CPU tests: the state dicts load strictly; the preprocessing chain and the PLE edges and
coordinates match the reference (fp32 on both sides; the edges are order statistics and
interpolations of the same values); the PLE token split and the refusals of the reference's
tests/test_model_v3.py hold. GPU tests: the whole forward and the chunked encoder through
the HIP attention and norm kernels, held to a relative error max|got - exp| / max|exp| <=
1e-3 on the row states and the quantile predictions (measured near 1e-6, printed by each
check); and the reference's own property that a query row never sees another
(test_model_v3.py:69-84).
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch
from parity import PREDICTION_BAR, check_relative

from nori_amd import transformer as NT
from nori_amd.encoders import MaskEmbEncoder, PromptQuantilePLEEncoder

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "two_phase_goldens.npz")
PLE_BINS = 8
EVAL_POS = 28
# Mirrors the configurations tests/golden/make_two_phase_golden.py builds the reference models with.
VARIANTS = {"a": dict(fpg=2, pos="none"), "b": dict(fpg=1, pos="subortho")}
RBF = dict(token_embed_dim=8, n_kernels=16, sigma=0.5, use_learn_sigma=False, use_learn_embeddings=False,
           use_original_features=False)


def config(v):
    fpg = v["fpg"]
    return dict(
        preprocess_config_x=dict(
            num_features=fpg, nan_handling_enabled=True, normalize_on_train_only=True, normalize_x=True,
            remove_outliers=False, normalize_by_used_features=True, prompt_quantile_ple_bins=PLE_BINS,
        ),
        encoder_config_x=dict(
            num_features=fpg, embedding_size=32, mask_embedding_size=32, encoder_use_bias=True, numeric_embed_type="RBF",
            RBF_config=dict(RBF), prompt_quantile_ple_bins=PLE_BINS,
        ),
        encoder_config_y=dict(num_inputs=1, embedding_size=32, nan_handling_y_encoder=True, max_num_classes=10),
        decoder_config=dict(num_reg_quantiles=9, regression_loss="pinball"),
        nlayers=2, nhead=2, embed_dim=32, hid_dim=64, features_per_group=fpg, dropout=0.0, pre_norm=True,
        activation="swiglu", norm_type="rmsnorm", deepnorm_alpha=4 ** -0.5,
        feature_positional_embedding_type=v["pos"], use_target_aware_embedding=True, use_column_specific_y_aware=True,
        use_qassmax=True, qass_mode="log_only", omit_feature_decoder=True,
        two_phase_config=dict(target_tokens=2, row_layers=2, row_heads=4, row_hidden_dim=96),
    )


@pytest.fixture(scope="module")
def gold():
    with np.load(GOLDEN, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def make_model(gold, tag, device="cpu"):
    model = NT.FeaturesTransformer(**config(VARIANTS[tag])).eval()
    prefix = f"tp_{tag}/w."
    model.load_state_dict({k[len(prefix):]: torch.from_numpy(v) for k, v in gold.items() if k.startswith(prefix)}, strict=True)
    model = model.to(device)
    if f"tp_{tag}/feature_pos_emb" in gold:  # the fixture holds the subortho draw fixed
        fixed = torch.from_numpy(gold[f"tp_{tag}/feature_pos_emb"])
        model.make_feature_positional_embeddings = lambda n_groups, *, device, dtype: fixed.to(device, dtype)
    return model


def table(gold, tag, device="cpu"):
    return torch.from_numpy(gold[f"tp_{tag}/x"]).to(device), torch.from_numpy(gold[f"tp_{tag}/y"]).to(device)


def check(got, exp, bar=PREDICTION_BAR):
    """max|got - exp| / max|exp| <= bar (relative 1e-3 by default, the bar for predictions)."""
    got = torch.as_tensor(got).detach()
    exp = torch.as_tensor(exp)
    assert tuple(got.shape) == tuple(exp.shape), (tuple(got.shape), tuple(exp.shape))
    test = os.environ.get("PYTEST_CURRENT_TEST", "?").split(" ")[0]
    return check_relative(got, exp, bar, test)


# ------------------------------------------------------------------------------- CPU
@pytest.mark.parametrize("tag", ["a", "b"])
def test_model_takes_the_reference_state_dict(gold, tag):
    model = make_model(gold, tag)
    assert model.supports_context_cache is False
    assert model.cls_y_encoder is None and model.cls_y_decoder is None and model.cls_target_aware_embedding is None
    assert not any(p.requires_grad for p in model.reg_y_encoder.parameters())
    assert model.reg_y_decoder[0].in_features == 64  # K * cell_dim


@pytest.mark.parametrize("tag", ["a", "b"])
def test_preprocessing_and_ple_edges_match_reference(gold, tag):
    model = make_model(gold, tag)
    x, _ = table(gold, tag)
    with torch.no_grad():
        pre, _ = model._build_x_preprocess_inputs(x.clone(), EVAL_POS)
        pre = model.x_preprocess(pre)
    np.testing.assert_allclose(pre["data"].numpy(), gold[f"tp_{tag}/pre_data"], rtol=1e-6, atol=1e-6)
    assert np.array_equal(pre["mask"].numpy(), gold[f"tp_{tag}/pre_mask"])
    edges = pre[PromptQuantilePLEEncoder.reference_key]["edges"]
    np.testing.assert_allclose(edges.numpy(), gold[f"tp_{tag}/ple_edges"], rtol=1e-6, atol=1e-6)
    # the constant column has one edge value, so every bin of it is closed
    assert bool((edges[..., 1:] == edges[..., :1]).all(-1).any())
    coords = PromptQuantilePLEEncoder.encode(pre["data"], pre[PromptQuantilePLEEncoder.reference_key])
    np.testing.assert_allclose(coords.numpy(), gold[f"tp_{tag}/ple_coords"], rtol=1e-6, atol=1e-6)


def test_ple_edges_closed_forms():
    """Edges of a column are its context quantiles: with n valid values ranked v_0..v_{n-1}, edge
    i of b bins is v at rank (n - 1) i / b, linearly interpolated; invalid and query cells are
    ignored; a column without valid context cells has zero edges. Coordinates are cumulative."""
    enc = PromptQuantilePLEEncoder(4)
    ctx = torch.tensor([3.0, 1.0, float("nan"), 2.0, 5.0, 4.0])  # valid: 1 2 3 4 5
    x = torch.cat((ctx, torch.tensor([100.0, -100.0]))).view(1, 8, 1, 1)  # two query rows
    empty = torch.full((1, 8, 1, 1), float("nan"))
    data = torch.cat((x, empty), dim=2)
    mask = torch.zeros_like(data, dtype=torch.int32)
    out = enc({"data": data, "mask": mask, "eval_pos": 6})
    edges = out[enc.reference_key]["edges"]
    assert torch.equal(edges[0, 0, 0], torch.tensor([1.0, 2.0, 3.0, 4.0, 5.0]))
    assert torch.equal(edges[0, 1, 0], torch.zeros(5))
    # a masked cell is not a context value either
    mask2 = mask.clone()
    mask2[0, 4, 0, 0] = 1  # drops 5.0: valid 1 2 3 4 -> ranks (3 i / 4)
    e2 = enc({"data": data, "mask": mask2, "eval_pos": 6})[enc.reference_key]["edges"][0, 0, 0]
    assert torch.allclose(e2, torch.tensor([1.0, 1.75, 2.5, 3.25, 4.0]))
    coords = PromptQuantilePLEEncoder.encode(torch.tensor([0.0, 2.5, 9.0, float("nan")]).view(1, 4, 1, 1), {"edges": edges[:, :1]})
    assert torch.equal(coords[0, :, 0, 0], torch.tensor(
        [[0.0, 0.0, 0.0, 0.0], [1.0, 0.5, 0.0, 0.0], [1.0, 1.0, 1.0, 1.0], [0.0, 0.0, 0.0, 0.0]]))
    frozen = enc({"data": data, "mask": mask, "eval_pos": 1, enc.frozen_reference_key: {"edges": edges}})
    assert torch.equal(frozen[enc.reference_key]["edges"], edges)
    with pytest.raises(ValueError, match="expected"):
        enc({"data": data, "mask": mask, enc.frozen_reference_key: {"edges": edges[..., :3]}})
    with pytest.raises(ValueError, match="non-empty context"):
        enc({"data": data, "mask": mask, "eval_pos": 0})


def test_ple_bins_split_the_cell_token_and_refuse_bad_configs():
    """tests/test_model_v3.py:119-133 and encoders.py:469-480."""
    dense = MaskEmbEncoder(1, 32, 32, numeric_embed_type="RBF", RBF_config=dict(RBF))
    assert dense.numeric_mlp.out_layer.out_features == 32
    with_ple = MaskEmbEncoder(1, 32, 32, numeric_embed_type="RBF", RBF_config=dict(RBF), prompt_quantile_ple_bins=8)
    assert with_ple.numeric_mlp.out_layer.out_features == 24
    with pytest.raises(TypeError, match="reference is required"):
        with_ple({"data": torch.randn(1, 4, 2, 1)})
    for bins, kw, msg in ((1, {}, "at least 2"), (-1, {}, "negative"), (32, {}, "smaller"),
                          (8, dict(numeric_embed_type="linear"), "only with the RBF")):
        args = dict(numeric_embed_type="RBF", RBF_config=dict(RBF))
        args.update(kw)
        with pytest.raises(ValueError, match=msg):
            MaskEmbEncoder(1, 32, 32, prompt_quantile_ple_bins=bins, **args)


def test_two_phase_refusals(gold):
    """tests/test_model_v3.py:59-67, 87-94: regression only; no context cache."""
    model = make_model(gold, "a")
    x, y = table(gold, "a")
    with pytest.raises(ValueError, match="regression only"):
        model(x=x, y=y, eval_pos=EVAL_POS, task_type="cls")
    with pytest.raises(NotImplementedError, match="two-phase"):
        model.forward_cached_regression(x, y, eval_pos=EVAL_POS)
    with pytest.raises(NotImplementedError, match="two-phase"):
        model.build_context_cache(x[:, :EVAL_POS], y)
    with pytest.raises(ValueError, match="divisible by row_heads"):
        cfg = config(VARIANTS["a"])
        cfg["two_phase_config"]["row_heads"] = 5
        NT.FeaturesTransformer(**cfg)


# ------------------------------------------------------------------------------- GPU
@pytest.mark.gpu
@pytest.mark.parametrize("tag", ["a", "b"])
def test_forward_matches_reference(gold, cuda, tag):
    model = make_model(gold, tag, cuda)
    x, y = table(gold, tag, cuda)
    with torch.inference_mode():
        reg = model(x=x, y=y, eval_pos=EVAL_POS, task_type="reg")
        rows = model(x=x, y=y, eval_pos=EVAL_POS, task_type="reg", return_embeddings=True)
    assert reg.shape == (2, 12, 9) and rows.shape == (2, 40, 64)
    check(rows, gold[f"tp_{tag}/rows"])
    check(reg, gold[f"tp_{tag}/reg"])


@pytest.mark.gpu
@pytest.mark.parametrize("tag", ["a", "b"])
@pytest.mark.parametrize("residual", ["cuda", "cpu"])
def test_chunked_encoder_matches_reference(gold, cuda, tag, residual):
    """forward_chunked with the table resident on the GPU, and with it in host memory."""
    model = make_model(gold, tag, cuda)
    home = cuda if residual == "cuda" else torch.device("cpu")
    # forward_chunked overwrites the table in place: hand it a copy of the fixture
    cells = torch.from_numpy(gold[f"tp_{tag}/enc_cells"].copy()).to(home)
    y = torch.from_numpy(gold[f"tp_{tag}/enc_y"])
    out = model.transformer_encoder.forward_chunked(cells, y, EVAL_POS, row_chunk=16, column_chunk=2, compute_device=cuda)
    assert out.device.type == home.type
    check(out, gold[f"tp_{tag}/chunked_rows"])
    whole, _ = model.transformer_encoder(torch.from_numpy(gold[f"tp_{tag}/enc_cells"]).to(cuda), y.to(cuda), EVAL_POS)
    check(out, whole, 1e-3)


@pytest.mark.gpu
@pytest.mark.parametrize("tag", ["a", "b"])
def test_query_rows_never_see_each_other(gold, cuda, tag):
    """tests/test_model_v3.py:69-84: perturbing the last query row (and every query label)
    changes only that row's prediction."""
    model = make_model(gold, tag, cuda)
    x, y = table(gold, tag, cuda)
    full_y = torch.cat((y, torch.full((2, 12), 1000.0, device=cuda)), dim=1)
    with torch.inference_mode():
        full = model(x=x, y=y, eval_pos=EVAL_POS, task_type="reg")
        x_alt = x.clone()
        x_alt[:, -1] = torch.randn(x.shape[2], device=cuda)
        alt = model(x=x_alt, y=full_y, eval_pos=EVAL_POS, task_type="reg")
    assert torch.allclose(full[:, :-1], alt[:, :-1], atol=1e-5)
    assert not torch.allclose(full[:, -1], alt[:, -1], atol=1e-5)
