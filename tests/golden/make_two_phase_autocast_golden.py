"""Write golden vectors for the two-phase encoder (Nori 1.5) at its own widths, in fp32 and under
fp16 autocast.

Runs the reference's own model code (synthefy_nori.model.transformer with .two_phase, .encoders
and .layer: src/synthefy_nori/model/two_phase.py:1-486, transformer.py:370-562,
encoders.py:118-585) on the CPU, on a random-init two-phase model with Nori 1.5's widths --
128-wide cells with 2 heads of 64, 32-bin prompt-quantile PLE cells beside a 96-wide RBF
embedding, 2 target tokens (256-wide target and row streams, 4 heads of 64), SwiGLU hidden
widths 256 and 682 -- but 2 cell and 2 row layers and a small table, so that the GPU runs it
through the kernels these widths select (the cell-token kernel, the cells' last norm with the
positional and target-aware additions, the output projection + residual + norm, the SwiGLU
with its residual epilogue, the short-context attention with its q/k prologue).

Two runs of the same weights and table:
* fp32 (the reference's CPU setting);
* ``torch.autocast("cpu", dtype=torch.float16)`` with CUDA autocast's op policy
  (tests/golden/cuda_autocast_policy.py): the dtypes a GPU run of the reference computes in,
  its predictor's own mode (predictor.py:3208-3217); with its spread -- the largest relative
  change of the query rows' predictions and row states when the same fp16 run takes the
  context rows in three other orders (the outputs do not depend on that order except through
  the order of the sums).
The subortho feature embedding's draw of each run is recorded so the test can hold it fixed.
The model's matrices are redrawn by tests/golden/weight_draws.py at the scale of the
reference's own initialisation and stored as a seed and a scale only.

Only this container holds the reference (at /root/reference); the committed product of this
script is the .npz data beside it, never the reference's code.

Usage: python tests/golden/make_two_phase_autocast_golden.py
(writes tests/golden/two_phase_autocast_goldens.npz)
"""

from __future__ import annotations

import os
import sys
import types

import numpy as np
import torch

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
from cuda_autocast_policy import cuda_policy  # noqa: E402
from weight_draws import pack  # noqa: E402

REFERENCE_SRC = "/root/reference/src"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "two_phase_autocast_goldens.npz")

ROWS, EVAL_POS, FEATURES = 40, 28, 8


def load_reference():
    for name, sub in (("synthefy_nori", "synthefy_nori"), ("synthefy_nori.model", "synthefy_nori/model")):
        mod = types.ModuleType(name)
        mod.__path__ = [os.path.join(REFERENCE_SRC, sub)]
        sys.modules[name] = mod
    import synthefy_nori.model.layer as layer_mod
    import synthefy_nori.model.transformer as transformer_mod

    return layer_mod, transformer_mod


def model_config():
    return dict(
        preprocess_config_x=dict(
            num_features=2, nan_handling_enabled=True, normalize_on_train_only=True, normalize_x=True,
            remove_outliers=False, normalize_by_used_features=True, prompt_quantile_ple_bins=32,
        ),
        encoder_config_x=dict(
            num_features=2, embedding_size=128, mask_embedding_size=128, encoder_use_bias=True, numeric_embed_type="RBF",
            RBF_config=dict(token_embed_dim=8, n_kernels=16, sigma=0.5, use_learn_sigma=False,
                            use_learn_embeddings=False, use_original_features=False),
            prompt_quantile_ple_bins=32,
        ),
        encoder_config_y=dict(num_inputs=1, embedding_size=128, nan_handling_y_encoder=True, max_num_classes=10),
        decoder_config=dict(num_reg_quantiles=9, regression_loss="pinball"),
        nlayers=2, nhead=2, embed_dim=128, hid_dim=384, features_per_group=2, dropout=0.0, pre_norm=True,
        activation="swiglu", norm_type="rmsnorm", deepnorm_alpha=4 ** -0.5, feature_positional_embedding_type="subortho",
        use_target_aware_embedding=True, use_column_specific_y_aware=True, use_qassmax=True, qass_mode="log_only",
        omit_feature_decoder=True, two_phase_config=dict(target_tokens=2, row_layers=2, row_heads=4, row_hidden_dim=1024),
    )


def table(gen):
    """Two tables of 40 rows x 8 features: NaN, +inf, -inf cells, a constant column (zero-width
    PLE bins), a column of repeated values, magnitudes over several decades, and a target."""
    scale = torch.tensor([1.0, 3.0, 0.2, 10.0, 1.0, 100.0, 0.01, 2.0])
    x = torch.randn(2, ROWS, FEATURES, generator=gen) * scale
    x[:, :, 2] = 0.5
    x[:, :, 4] = torch.randint(0, 3, (2, ROWS), generator=gen).float()
    cells = torch.rand(2, ROWS, FEATURES, generator=gen)
    x[cells < 0.05] = float("nan")
    x[(cells > 0.97) & (cells < 0.985)] = float("inf")
    x[cells >= 0.985] = float("-inf")
    finite = torch.nan_to_num(x, nan=0.0, posinf=1.0, neginf=-1.0)
    y = finite[:, :, 0] * 0.7 - 0.3 * finite[:, :, 1] * finite[:, :, 7] + torch.randn(2, ROWS, generator=gen) * 0.1
    return x, y


def main():
    L, T = load_reference()
    torch.set_num_threads(4)
    torch.manual_seed(40)
    model = T.FeaturesTransformer(**model_config()).eval()
    gen = torch.Generator().manual_seed(41)
    with torch.no_grad():
        for m in model.modules():
            if isinstance(m, L.RMSNorm):
                m.use_native = True  # the serving setting (utils/loading.py:272-277)
                if m.weight is not None:  # the per-head q/k norm gains start at one
                    m.weight.mul_(1.0 + 0.2 * torch.randn(m.weight.shape, generator=gen))
        # the column-specific target-aware mix starts near zero (sigmoid(-5)); move it so it counts
        model.column_y_aware_alpha.fill_(0.5)
        stored, full = pack({k: v.numpy() for k, v in model.state_dict().items()})
        model.load_state_dict({k: torch.from_numpy(v) for k, v in full.items()}, strict=True)
    x, y = table(gen)
    y_ctx = y[:, :EVAL_POS]
    drawn = []
    model.feature_positional_embedding.register_forward_hook(lambda mod, inp, res: drawn.append(res.detach().clone()))
    out: dict[str, np.ndarray] = {}

    def put(name, t):
        out[name] = t.detach().cpu().numpy() if torch.is_tensor(t) else np.asarray(t)

    def run(xx, yy, autocast):
        drawn.clear()
        with torch.inference_mode(), torch.autocast("cpu", dtype=torch.float16, enabled=autocast):
            with cuda_policy():
                torch.manual_seed(42)
                reg = model(x=xx.clone(), y=yy.clone(), eval_pos=EVAL_POS, task_type="reg")
                torch.manual_seed(42)
                rows = model(x=xx.clone(), y=yy.clone(), eval_pos=EVAL_POS, task_type="reg", return_embeddings=True)
        return reg.float(), rows.float(), drawn[0]

    reg32, rows32, pos32 = run(x, y_ctx, False)
    reg16, rows16, pos16 = run(x, y_ctx, True)

    def rel(a, b):
        return float((a.double() - b.double()).abs().max() / b.double().abs().max())

    spread = {"reg": 0.0, "query_rows": 0.0}
    for seed in range(3):
        perm = torch.from_numpy(np.random.default_rng(400 + seed).permutation(EVAL_POS))
        order = torch.cat((perm, torch.arange(EVAL_POS, ROWS)))
        reg_p, rows_p, _ = run(x[:, order], y_ctx[:, perm], True)
        spread["reg"] = max(spread["reg"], rel(reg_p, reg16))
        spread["query_rows"] = max(spread["query_rows"], rel(rows_p[:, EVAL_POS:], rows16[:, EVAL_POS:]))

    out.update(stored)
    put("x", x)
    put("y", y_ctx)
    put("fp32/reg", reg32)
    put("fp32/rows", rows32)
    put("fp32/feature_pos_emb", pos32)
    put("ac/reg", reg16)
    put("ac/rows", rows16)
    put("ac/feature_pos_emb", pos16)
    for k, v in spread.items():
        put(f"ac/spread/{k}", np.array(v))
    put("ac/vs_fp32/reg", np.array(rel(reg16, reg32)))
    put("ac/vs_fp32/query_rows", np.array(rel(rows16[:, EVAL_POS:], rows32[:, EVAL_POS:])))
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT}: {len(out)} arrays, {os.path.getsize(OUT) / 1e6:.2f} MB")
    print("fp16 autocast: spread over context orders " + ", ".join(f"{k} {v:.2e}" for k, v in spread.items())
          + f"; vs fp32: reg {rel(reg16, reg32):.2e}, query rows {rel(rows16[:, EVAL_POS:], rows32[:, EVAL_POS:]):.2e}")


if __name__ == "__main__":
    main()
