"""GPU parity of the cell-token kernel (``nori_cell_tokens``, csrc/cell_tokens.hip), which
forms the two-phase model's cell tokens under fp16 autocast (MaskEmbEncoder.forward with the
scientific-notation RBF embedding and prompt-quantile PLE coordinates, reference
model/encoders.py:118-276, 309-429, 432-585).

Bars, on cells that exercise every branch (NaN, 0, +-inf, negative values, magnitudes past
the exponent clamp at 1e-9 and 1e9, values below, inside and above the PLE edges, bins of
zero width, a column without context values):
  * the PLE channels and the mask-embedding rows: bit-exact against the module's torch ops;
  * the RBF channels against a torch restatement that takes the same gate table: within one
    fp16 ulp (only the output projection's fp32 sums differ in order), and 99 % bit-exact;
  * the RBF channels against the module's own torch ops (whose gate MLP runs over every cell,
    not over the table's 40 rows): within 4 fp16 ulps of the output's scale;
  * the encoder's output (after the fusion network) within 2e-3 of the torch path's.
"""

from __future__ import annotations

import pytest
import torch

from nori_amd import encoders
from nori_amd.norm import layer_norm

pytestmark = pytest.mark.gpu


def make_encoder(n_kernels, device, nan_to_zero=False):
    torch.manual_seed(11)
    enc = encoders.MaskEmbEncoder(
        num_features=2, emsize=128, mask_embedding_size=128, numeric_embed_type="RBF",
        RBF_config=dict(token_embed_dim=8, n_kernels=n_kernels, sigma=0.5, use_learn_sigma=False,
                        use_learn_embeddings=False, use_original_features=False),
        prompt_quantile_ple_bins=32, nan_to_zero=nan_to_zero,
    )
    return enc.to(device).eval()


def make_cells(device, b=3, s=300, g=4, f=2, ctx=200):
    gen = torch.Generator().manual_seed(7)
    x = torch.randn(b, s, g, f, generator=gen) * 3.0
    x = x * torch.exp(torch.randn(b, s, g, f, generator=gen) * 4.0)   # magnitudes over many decades
    flat = x.view(-1)
    special = torch.tensor([0.0, -0.0, float("nan"), float("inf"), float("-inf"), 1e-12, -3e-11, 5e12, -7e15, 1.0,
                            10.0, 0.1, 9.999999, 1e9, 1e-9, -1e-9])
    flat[: special.numel()] = special
    flat[500:520] = float("nan")
    x[0, :, 1, 0] = 2.5             # a constant column: every bin has zero width
    x[1, :ctx, 2, 1] = float("nan")  # a column without context values: zero edges
    valid = torch.isfinite(x)
    ple = encoders.PromptQuantilePLEEncoder(32)
    edges = ple._context_edges(x, valid, ctx)["edges"]
    return x.to(device), {"edges": edges.to(device)}


def torch_tokens(enc, x, reference, table=None):
    """The fusion network's operand as the module's torch ops form it (with ``table``: the
    gate from that table instead of the gate MLP over every cell)."""
    b, s, g, f = x.shape
    xs = x.unsqueeze(-1)
    missing = torch.isnan(xs)
    xs = xs.masked_fill(missing, 0.0)
    rbf = enc.numeric_mlp
    if table is None:
        emb = rbf(xs)
    else:
        xw = xs.squeeze(-1).double()
        m, e = rbf._mantissa_exponent(xw)
        c = rbf.centers.double().view(1, 1, 1, 1, -1)
        r = torch.exp(-((m.unsqueeze(-1) - c) ** 2) / (2 * (rbf.sigma ** 2))).float()
        row = (xw < 0).long() * 20 + (e < 0).long() * 10 + e.abs() % 10
        pre = r * table[row, 0] + table[row, 1]
        op = layer_norm(pre, rbf.norm.weight, rbf.norm.bias, rbf.norm.eps, out_dtype=torch.float16)
        emb = rbf.out_layer(op)
    coords = encoders.PromptQuantilePLEEncoder.encode(xs.squeeze(-1), reference).to(emb.dtype)
    emb = torch.cat((emb, coords), dim=-1)
    if not enc.nan_to_zero:
        emb = torch.where(missing, enc.mask_embedding.expand_as(emb), emb)
    return emb.flatten(3).to(torch.float16)


def fp16_ulp(t):
    return torch.clamp(t.float().abs(), min=2.0 ** -14).log2().floor().exp2() * 2.0 ** -10


@pytest.mark.parametrize("n_kernels", [16, 32])
@pytest.mark.parametrize("nan_to_zero", [False, True])
def test_cell_tokens_match_the_torch_ops(cuda, n_kernels, nan_to_zero):
    enc = make_encoder(n_kernels, cuda, nan_to_zero)
    x, reference = make_cells(cuda)
    inp = {"data": x, encoders.PromptQuantilePLEEncoder.reference_key: reference}
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.float16):
        h = enc._tokens_on_device(x, inp)
        assert h is not None and h.dtype == torch.float16 and h.shape == (3, 300, 4, 256)
        table = enc.numeric_mlp.gate_table(cuda)
        ref_table = torch_tokens(enc, x, reference, table)
        ref_module = torch_tokens(enc, x, reference)
    hv = h.view(3, 300, 4, 2, 128)
    rt = ref_table.view(3, 300, 4, 2, 128)
    rm = ref_module.view(3, 300, 4, 2, 128)
    # PLE channels and the NaN cells' rows: exact
    assert torch.equal(hv[..., 96:], rt[..., 96:])
    miss = torch.isnan(x)
    if not nan_to_zero:
        assert torch.equal(hv[miss], rt[miss])
    # RBF channels against the same gate table: the output projection's sum order only
    d = (hv[..., :96].float() - rt[..., :96].float()).abs()
    assert bool((d <= fp16_ulp(rt[..., :96])).all())
    exact = float((d == 0).float().mean())
    print(f"[parity] cell_tokens n_kernels={n_kernels}: {exact:.4f} of RBF channels bit-exact vs the table restatement",
          flush=True)
    assert exact >= 0.99
    # against the module's own gate MLP over every cell
    d = (hv[..., :96].float() - rm[..., :96].float()).abs()
    assert float(d.max()) <= 4 * 2.0 ** -10 * float(rm[..., :96].float().abs().max())


@pytest.mark.parametrize("n_kernels", [16, 32])
def test_encoder_output_with_and_without_the_kernel(cuda, n_kernels, monkeypatch):
    enc = make_encoder(n_kernels, cuda)
    x, reference = make_cells(cuda)
    outs = []
    for fused in (True, False):
        if not fused:
            monkeypatch.setattr(encoders.MaskEmbEncoder, "_tokens_on_device", lambda self, x, inp: None)
        inp = {"data": x.clone(), encoders.PromptQuantilePLEEncoder.reference_key: reference}
        with torch.no_grad(), torch.autocast("cuda", dtype=torch.float16):
            outs.append(enc(inp)["data"].float())
    assert outs[0].shape == (3, 300, 4, 128)
    assert float((outs[0] - outs[1]).abs().max()) <= 2e-3 * float(outs[1].abs().max())


def test_fp32_and_unsupported_configurations_take_the_torch_ops(cuda):
    enc = make_encoder(16, cuda)
    x, reference = make_cells(cuda)
    inp = {"data": x, encoders.PromptQuantilePLEEncoder.reference_key: reference}
    with torch.no_grad():
        assert enc._tokens_on_device(x, inp) is None  # no autocast: the fp32 model's ops
    enc.numeric_mlp.n_kernels = 8
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.float16):
        assert enc._tokens_on_device(x, inp) is None


# ---------------------------------------------------------------- the cells' last norm + additions
# ``nori_layer_norm_cells`` replaces the cell encoder's last LayerNorm, the feature positional
# embedding and the target-aware row bias of the two-phase forward (reference
# transformer.py:467-470, 1080-1132). Bars: query rows (no row bias) bit-exact against the
# separate norm kernel + torch's ops; context rows within a few fp32 ulps (the gate's dot
# product is summed in another order).

TWO_PHASE = dict(
    preprocess_config_x=dict(num_features=2, nan_handling_enabled=True, normalize_on_train_only=True, normalize_x=True,
                             remove_outliers=False, normalize_by_used_features=True, prompt_quantile_ple_bins=32),
    encoder_config_x=dict(num_features=2, embedding_size=128, mask_embedding_size=128, encoder_use_bias=True,
                          numeric_embed_type="RBF",
                          RBF_config=dict(token_embed_dim=8, n_kernels=16, sigma=0.5, use_learn_sigma=False,
                                          use_learn_embeddings=False, use_original_features=False),
                          prompt_quantile_ple_bins=32),
    encoder_config_y=dict(num_inputs=1, embedding_size=128, nan_handling_y_encoder=True, max_num_classes=10),
    decoder_config=dict(num_reg_quantiles=999, regression_loss="pinball"),
    nlayers=2, nhead=2, embed_dim=128, hid_dim=384, features_per_group=2, dropout=0.0, pre_norm=True,
    activation="swiglu", norm_type="rmsnorm", deepnorm_alpha=4 ** -0.5, feature_positional_embedding_type="subortho",
    use_target_aware_embedding=True, use_column_specific_y_aware=True, use_qassmax=True, qass_mode="log_only",
    omit_feature_decoder=True, two_phase_config=dict(target_tokens=2, row_layers=1, row_heads=4, row_hidden_dim=256),
)


@pytest.mark.parametrize("autocast", [True, False])
@pytest.mark.parametrize("gated", [True, False])
def test_layer_norm_cells_match_the_separate_ops(cuda, autocast, gated):
    import nori_amd

    torch.manual_seed(3)
    model = nori_amd.FeaturesTransformer(**TWO_PHASE).eval().to(cuda)
    with torch.no_grad():
        model.column_y_aware_alpha.fill_(0.3)
        model.reg_target_aware_embedding.weight.normal_(0.0, 0.5)
        model.reg_target_aware_embedding.bias.normal_(0.0, 0.5)
    if not gated:
        model.use_column_specific_y_aware = False
    ln = model.encoder_x[0].fusion_network[4]
    with torch.no_grad():
        ln.weight.normal_(1.0, 0.2)
        ln.bias.normal_(0.0, 0.2)
    b, s, g, ep = 3, 200, 4, 150
    gen = torch.Generator(device=cuda).manual_seed(9)
    h = torch.randn(b, s, g, 128, generator=gen, device=cuda) * 2.0 + 0.5
    y = torch.randn(b, s, generator=gen, device=cuda)
    y[:, ep:] = float("nan")
    dt = torch.float32
    h = h.half() if autocast else h
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.float16, enabled=autocast):
        pos = model.make_feature_positional_embeddings(g, device=cuda, dtype=dt)
        fused = model._finish_cells(h, (ln, dt), pos, y, ep)
        cells = layer_norm(h, ln.weight, ln.bias, ln.eps, out_dtype=dt)
        ref = model._finish_cells(cells, None, pos, y, ep)
    assert fused.dtype == torch.float32 and fused.shape == (b, s, g, 128)
    assert torch.equal(fused[:, ep:], ref[:, ep:])
    if not gated:
        assert torch.equal(fused, ref)
    d = (fused[:, :ep] - ref[:, :ep]).abs()
    assert float(d.max()) <= 8 * 2.0 ** -24 * float(ref[:, :ep].abs().max())
