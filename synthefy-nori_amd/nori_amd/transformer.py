"""Drop-in for the context-cache API of ``synthefy_nori.model.transformer``.

``FeaturesTransformer`` here has the reference's constructor, module tree and parameter
names (src/synthefy_nori/model/transformer.py:70-369), so a reference state dict loads with
``strict=True``, and implements its cached-regression entry points:

* ``build_context_cache`` (:813-959): preprocess and encode the context rows once --
  ``NanEncoder`` -> ``NormalizationEncoder`` -> ``ValidFeatureEncoder`` with their context
  statistics captured, the x and y encoders, the target-aware embedding -- then run the
  layer stack's cache build, each layer's sequence K/V quantized to the int8 cache on the
  HIP codec as soon as the layer produces it; returns a ``ContextCache`` (:12-61);
* ``apply_context_cache`` (:961-1078): encode query rows with the frozen context
  statistics and score them through the cached layers (query -> context attention on the
  HIP kernel, over the int8 payload directly), in query chunks that halve on
  ``torch.cuda.OutOfMemoryError``;
* ``forward_cached_regression`` (:716-811): the build/apply pair;
* the bounded builds: ``fit_row_chunk`` (row-chunked layer builds) and ``stream_context`` /
  the hybrid resident-int8 prefill (``_build_context_cache_streaming``, :1169-1301), which
  keep the context rows and every full-N tensor on the host and stage ``fit_row_chunk`` rows
  at a time.

With a ``two_phase_config`` the model is Nori 1.5 ("Model v3", regression only): the
transformer encoder is the two-phase encoder (``nori_amd.two_phase``, two_phase.py) and
``forward`` runs it over context and query rows together (:370-562, ``_forward_two_phase``
:525-562), every attention on the HIP kernel. It has no context cache (the reference's
``supports_context_cache`` is False): the cache entry points raise ``NotImplementedError``,
as the reference's do (:763-764, 839-840). The uncached forward of the dense layer stack is
not part of this package (it raises); the dense models run through the cache entry points.
"""

from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass
from typing import Any, Callable, Literal

import torch
import torch.nn as nn
from torch.amp import autocast

from . import _native as nat
from .encoders import (
    MaskEmbEncoder,
    PromptQuantilePLEEncoder,
    get_cls_y_encoder,
    get_reg_y_encoder,
    get_x_encoder,
    preprocesss_4_x,
)
from .layer import EncoderBaseLayer, LayerStack
from .two_phase import TwoPhaseEncoder
from .norm import RMSNorm, layer_norm

__all__ = ["ContextCache", "FeaturesTransformer"]


@dataclass
class ContextCache:
    """Query-independent encoding of a fixed context table (reference transformer.py:12-61):
    per-layer sequence K/V caches, the feature positional embedding drawn for the context,
    the context's normalization statistics, NaN fill and valid-feature count (re-applied,
    frozen, to query rows), the context targets and the context row count."""

    caches: list
    feature_pos_emb: torch.Tensor | None
    norm_stats: dict | None
    y_train: torch.Tensor
    eval_pos: int
    nan_mean: torch.Tensor | None = None
    valid_feature_num: torch.Tensor | None = None
    query_y_embedding: torch.Tensor | None = None


def _regression_head(decoder_config: dict) -> tuple[str, tuple[float, ...], int]:
    """(loss, quantile levels, head width) as the reference resolves them (:142-183)."""
    width = int(decoder_config.get("num_reg_quantiles", 1))
    loss = decoder_config.get("regression_loss")
    if loss is None:  # legacy configs only recorded the head width
        loss = "mse" if width == 1 else "pinball"
    loss = str(loss)
    levels: tuple[float, ...] = ()
    if loss == "pinball":
        given = decoder_config.get("regression_quantiles")
        if given is None:
            levels = tuple((i + 1.0) / (width + 1.0) for i in range(width))
        else:
            levels = tuple(float(q) for q in given)
            if len(levels) != width:
                raise ValueError(
                    f"decoder_config.regression_quantiles length {len(levels)} does not match num_reg_quantiles={width}"
                )
            if any(not math.isfinite(q) or not 0.0 < q < 1.0 for q in levels) or any(
                a >= b for a, b in zip(levels, levels[1:])
            ):
                raise ValueError("decoder_config.regression_quantiles must be strictly increasing values in (0, 1)")
    return loss, levels, width


def _bar_borders(mode: str, n: int, low: float, high: float) -> torch.Tensor:
    """Bin edges of the bar-distribution head (:189-220): N(0,1) quantiles with +-8 ends, or
    uniform."""
    if mode == "normal_quantile":
        try:
            from scipy.stats import norm

            edges = norm.ppf(torch.linspace(0.0, 1.0, n + 1, dtype=torch.float32).numpy())
            edges[0], edges[-1] = -8.0, 8.0
            return torch.from_numpy(edges).float()
        except ImportError:
            pass
    return torch.linspace(low, high, n + 1, dtype=torch.float32)


class FeaturesTransformer(nn.Module):
    """Reference ``FeaturesTransformer`` (transformer.py:67-1301), cached regression paths."""

    def __init__(
        self,
        *,
        preprocess_config_x: dict[str, Any],
        encoder_config_x: dict[str, Any],
        encoder_config_y: dict[str, Any],
        decoder_config: dict[str, Any],
        nlayers: int,
        nhead: int,
        embed_dim: int,
        hid_dim: int,
        feature_positional_embedding_type: Literal["none", "subortho", "learned"] = "subortho",
        feature_positional_embedding_num_slots: int = 1000,
        mask_prediction: bool = False,
        features_per_group: int = 2,
        dropout: float = 0,
        pre_norm: bool = False,
        activation: str = "gelu",
        layer_norm_eps: float = 1e-5,
        device: torch.device | None = None,
        dtype: torch.dtype | None = None,
        recompute_attn: bool = False,
        mlp_use_residual: bool = False,
        layer_arch: str = "fmfmsm",
        norm_type: str = "layernorm",
        deepnorm_alpha: float | None = None,
        use_target_aware_embedding: bool = False,
        use_column_specific_y_aware: bool = False,
        use_logn_attention: bool = False,
        use_learnable_attn_temperature: bool = False,
        attn_n_ref: float = 1024.0,
        omit_feature_decoder: bool = False,
        two_phase_config: dict[str, Any] | None = None,
        **layer_kwargs: Any,
    ):
        super().__init__()
        if mlp_use_residual:
            raise ValueError(
                "mlp_use_residual=True is unsupported: every MLP sublayer already uses the transformer's outer "
                "residual connection. This legacy flag was a no-op; leave it false or remove it from the config."
            )
        self.preprocess_config_x = preprocess_config_x
        self.encoder_config_x = encoder_config_x
        self.encoder_config_y = encoder_config_y
        self.decoder_config = decoder_config
        self.feature_positional_embedding_type = feature_positional_embedding_type
        self.nlayers, self.nhead, self.embed_dim, self.hid_dim = nlayers, nhead, embed_dim, hid_dim
        self.mask_prediction = mask_prediction
        self.features_per_group = int(features_per_group)
        if self.features_per_group < 1:
            raise ValueError("features_per_group must be at least 1")
        self.dropout, self.pre_norm, self.activation = dropout, pre_norm, activation
        self.layer_norm_eps, self.device, self.dtype = layer_norm_eps, device, dtype
        self.recompute_attn = recompute_attn
        self.mlp_use_residual = False
        self.layer_arch, self.norm_type, self.deepnorm_alpha = layer_arch, norm_type, deepnorm_alpha
        self.omit_feature_decoder = bool(omit_feature_decoder)
        self.two_phase_config = dict(two_phase_config) if two_phase_config else None
        two_phase = self.two_phase_config is not None
        self.regression_loss, self.regression_quantiles, self.num_reg_quantiles = _regression_head(decoder_config)
        self.num_bars = int(decoder_config.get("num_bars", self.num_reg_quantiles))
        self.bar_borders_low = float(decoder_config.get("bar_borders_low", -10.0))
        self.bar_borders_high = float(decoder_config.get("bar_borders_high", 10.0))
        self.bar_borders_mode = str(decoder_config.get("bar_borders_mode", "uniform"))
        if self.regression_loss == "bar_distribution":
            self.register_buffer(
                "bar_borders_buffer",
                _bar_borders(self.bar_borders_mode, self.num_bars, self.bar_borders_low, self.bar_borders_high),
                persistent=True,
            )
        else:
            self.bar_borders_buffer = None
        self.use_target_aware_embedding = use_target_aware_embedding
        self.use_column_specific_y_aware = use_column_specific_y_aware
        self.column_y_aware_alpha = (
            nn.Parameter(torch.tensor(-5.0, device=device, dtype=dtype if dtype else torch.float32))
            if use_column_specific_y_aware
            else None
        )
        self.target_aware_scale = 1.0
        self.max_num_classes = int(encoder_config_y.get("max_num_classes", decoder_config.get("num_classes", 10)))
        self.use_logn_attention = use_logn_attention
        self.use_learnable_attn_temperature = use_learnable_attn_temperature
        self.attn_n_ref = float(attn_n_ref)

        self.encoder_x = get_x_encoder(**encoder_config_x)
        self.cls_y_encoder = None if two_phase else get_cls_y_encoder(**encoder_config_y)
        self.reg_y_encoder = get_reg_y_encoder(**encoder_config_y)
        if use_target_aware_embedding:
            self.cls_target_aware_embedding = (
                None if two_phase else nn.Embedding(self.max_num_classes, embed_dim, device=device, dtype=dtype)
            )
            self.reg_target_aware_embedding = nn.Linear(1, embed_dim, device=device, dtype=dtype)
            if self.cls_target_aware_embedding is not None:
                nn.init.normal_(self.cls_target_aware_embedding.weight, std=0.02)
            nn.init.normal_(self.reg_target_aware_embedding.weight, std=0.02)
            nn.init.zeros_(self.reg_target_aware_embedding.bias)
        else:
            self.cls_target_aware_embedding = None
            self.reg_target_aware_embedding = None
        if two_phase:
            cfg = self.two_phase_config
            self.transformer_encoder = TwoPhaseEncoder(
                embed_dim,
                nhead,
                hid_dim,
                target_tokens=int(cfg["target_tokens"]),
                cell_layers=nlayers,
                row_layers=int(cfg["row_layers"]),
                row_heads=int(cfg["row_heads"]),
                row_hidden_dim=int(cfg["row_hidden_dim"]),
                task_type="reg",
                max_num_classes=self.max_num_classes,
                layer_norm_eps=layer_norm_eps,
                device=device,
                dtype=dtype,
            )
            # the single y-token encoder is unused by the two-phase path; kept for the state-dict schema
            for parameter in self.reg_y_encoder.parameters():
                parameter.requires_grad_(False)
            decoder_width = self.transformer_encoder.width
        else:
            self.transformer_encoder = self._dense_stack(
                nlayers, embed_dim=embed_dim, hid_dim=hid_dim, nhead=nhead, dropout=dropout, pre_norm=pre_norm,
                activation=activation, layer_norm_eps=layer_norm_eps, device=device, dtype=dtype,
                recompute_attn=recompute_attn, layer_arch=layer_arch, norm_type=norm_type, deepnorm_alpha=deepnorm_alpha,
                use_logn_attention=use_logn_attention, use_learnable_attn_temperature=use_learnable_attn_temperature,
                **layer_kwargs,
            )
            decoder_width = embed_dim
        self.supports_context_cache = not two_phase
        if not pre_norm:
            self.encoder_out_norm = nn.Identity()
        elif norm_type == "rmsnorm":
            self.encoder_out_norm = RMSNorm(embed_dim, eps=layer_norm_eps, elementwise_affine=False)
        else:
            self.encoder_out_norm = nn.LayerNorm(embed_dim, eps=layer_norm_eps, elementwise_affine=False)
        self.cls_y_decoder = (
            None
            if two_phase
            else nn.Sequential(nn.Linear(embed_dim, hid_dim), nn.GELU(), nn.Linear(hid_dim, decoder_config["num_classes"]))
        )
        self.reg_y_decoder = nn.Sequential(
            nn.Linear(decoder_width, hid_dim), nn.LayerNorm(hid_dim), nn.GELU(), nn.Linear(hid_dim, self.num_reg_quantiles)
        )
        self._finish_init(
            embed_dim=embed_dim, hid_dim=hid_dim, feature_positional_embedding_type=feature_positional_embedding_type,
            feature_positional_embedding_num_slots=feature_positional_embedding_num_slots,
            preprocess_config_x=preprocess_config_x,
        )

    def _dense_stack(self, nlayers: int, *, embed_dim, hid_dim, nhead, dropout, pre_norm, activation, layer_norm_eps,
                     device, dtype, recompute_attn, layer_arch, norm_type, deepnorm_alpha, use_logn_attention,
                     use_learnable_attn_temperature, **layer_kwargs) -> LayerStack:
        """The dense layer stack of nori-6m/30m/100m."""
        return LayerStack(
            [
                EncoderBaseLayer(
                    embed_dim=embed_dim,
                    hid_dim=hid_dim,
                    nhead=nhead,
                    dropout=dropout,
                    pre_norm=pre_norm,
                    activation=activation,
                    layer_norm_eps=layer_norm_eps,
                    device=device,
                    dtype=dtype,
                    recompute_attn=recompute_attn,
                    mlp_use_residual=False,
                    layer_arch=layer_arch,
                    norm_type=norm_type,
                    deepnorm_alpha=deepnorm_alpha,
                    use_logn_attention=use_logn_attention,
                    use_learnable_attn_temperature=use_learnable_attn_temperature,
                    attn_n_ref=self.attn_n_ref,
                    **layer_kwargs,
                )
                for _ in range(nlayers)
            ]
        )

    def _finish_init(self, *, embed_dim, hid_dim, feature_positional_embedding_type, feature_positional_embedding_num_slots,
                     preprocess_config_x) -> None:
        self.feature_decoder = (
            None
            if self.omit_feature_decoder
            else nn.Sequential(
                nn.Linear(embed_dim, hid_dim), nn.LayerNorm(hid_dim), nn.GELU(), nn.Linear(hid_dim, self.features_per_group)
            )
        )
        if feature_positional_embedding_type == "learned":
            self.feature_positional_embedding = nn.Embedding(feature_positional_embedding_num_slots, embed_dim)
            nn.init.normal_(self.feature_positional_embedding.weight, std=0.02)
            self.feature_positional_embedding_num_slots = feature_positional_embedding_num_slots
        elif feature_positional_embedding_type == "subortho":
            self.feature_positional_embedding = nn.Linear(embed_dim // 4, embed_dim)
        self.x_preprocess = preprocesss_4_x(**preprocess_config_x)

    # ------------------------------------------------------------------ row encoding
    def _build_x_preprocess_inputs(self, x: torch.Tensor, eval_pos: int) -> tuple[dict[str, Any], int]:
        """{"data", "mask" (non-finite), "eval_pos"}, zero-padded to whole feature groups and
        viewed as [B, S, groups, features_per_group] (:564-605)."""
        b, s, f = x.shape
        pad = (-f) % self.features_per_group
        out: dict[str, Any] = {"data": x, "mask": (~torch.isfinite(x)).to(torch.int32).to(x.device)}
        for key in ("data", "mask"):
            v = out[key]
            if pad:
                v = torch.cat((v, torch.zeros(b, s, pad, device=v.device, dtype=v.dtype)), dim=-1)
            out[key] = v.reshape(b, s, v.shape[2] // self.features_per_group, self.features_per_group)
        out["eval_pos"] = eval_pos
        return out, pad

    _ROW_KEYS = frozenset(
        {"data", "mask", "nan_encoding", "_conditional_landmark_coordinates", "_conditional_landmark_embedding",
         "_frozen_column_deepset_rbf"}
    )

    def _slice_preprocessed_x(self, preprocessed_x: dict[str, Any], row_slice: slice, total_rows: int) -> dict[str, Any]:
        """Row-slice the per-row tensors of a preprocessed dict, pass the rest through (:607-626)."""
        return {
            k: (v[:, row_slice].contiguous()
                if k in self._ROW_KEYS and torch.is_tensor(v) and v.dim() >= 2 and v.shape[1] == total_rows else v)
            for k, v in preprocessed_x.items()
        }

    def make_feature_positional_embeddings(self, n_groups: int, *, device: torch.device, dtype: torch.dtype):
        """One embedding per feature group: a fresh orthogonal draw projected (subortho), or a
        random subset of learned slots (:628-648)."""
        kind = self.feature_positional_embedding_type
        if kind == "subortho":
            with autocast(device_type=device.type, enabled=False):
                basis = torch.randn((n_groups, self.embed_dim // 4), device=device, dtype=torch.float32)
                torch.nn.init.orthogonal_(basis)
            return self.feature_positional_embedding(basis.to(dtype))
        if kind == "learned":
            slots = torch.randperm(self.feature_positional_embedding_num_slots, device=device)[:n_groups]
            return self.feature_positional_embedding(slots).to(dtype)
        if kind is None or kind == "none":
            return None
        raise ValueError(f"Unknown feature_positional_embedding_type={kind}")

    def apply_feature_positional_embeddings(self, x: torch.Tensor, embs: torch.Tensor | None) -> torch.Tensor:
        return x if embs is None else x + embs[None, None, :, :]

    def _encode_x_rows(self, preprocessed_x, row_slice: slice, *, total_rows: int, feature_pos_emb):
        part = self._slice_preprocessed_x(preprocessed_x, row_slice, total_rows)
        return self.apply_feature_positional_embeddings(self.encoder_x(part)["data"], feature_pos_emb)

    def _encode_y_full(self, y: torch.Tensor, *, total_rows: int, eval_pos: int, task_type: Literal["reg", "cls"]):
        """(raw targets padded with NaN to total_rows, y-encoder embedding with rows >= eval_pos
        masked to NaN) (:671-714)."""
        yv = y.unsqueeze(-1)
        if yv.shape[1] < total_rows:
            yv = torch.cat(
                (yv, torch.full((yv.shape[0], total_rows - yv.shape[1], yv.shape[2]), float("nan"), device=yv.device, dtype=yv.dtype)),
                dim=1,
            )
        target_aware_y = yv.squeeze(-1).clone()
        rows = torch.arange(total_rows, device=yv.device).view(1, -1, 1)
        masked = torch.where(rows >= eval_pos, torch.tensor(float("nan"), device=yv.device, dtype=yv.dtype), yv)
        enc = self.cls_y_encoder if task_type == "cls" else self.reg_y_encoder
        return target_aware_y, enc({"data": masked, "eval_pos": eval_pos})["data"].squeeze(2)

    def apply_target_aware_embedding(self, x: torch.Tensor, y: torch.Tensor, *, task_type: Literal["reg", "cls"], eval_pos: int):
        """Add an embedding of each context row's target to all its tokens (zeros for query
        rows), optionally gated per feature group by its alignment with that embedding and
        mixed by sigmoid(alpha) (:1080-1132)."""
        scale = float(getattr(self, "target_aware_scale", 1.0))
        if not self.use_target_aware_embedding or eval_pos <= 0 or abs(scale) < 1e-8:
            return x
        if task_type == "cls":
            idx = torch.clamp(y[:, :eval_pos].to(torch.long), min=0, max=self.max_num_classes - 1)
            ctx = self.cls_target_aware_embedding(idx).to(x.dtype)
        else:
            ctx = self.reg_target_aware_embedding(y[:, :eval_pos].unsqueeze(-1).to(x.dtype)).to(x.dtype)
        bias = torch.cat([ctx, ctx.new_zeros(x.shape[0], x.shape[1] - eval_pos, self.embed_dim)], dim=1)
        if scale != 1.0:
            bias = bias * scale
        row_bias = bias.unsqueeze(2)
        if self.use_column_specific_y_aware and self.column_y_aware_alpha is not None:
            gate = torch.sigmoid((x * row_bias).sum(dim=-1) * (1.0 / self.embed_dim**0.5)).unsqueeze(-1)
            alpha = torch.sigmoid(self.column_y_aware_alpha).to(x.dtype)
            return x + (1.0 - alpha) * row_bias + alpha * (row_bias * gate)
        return x + row_bias

    def _finish_cells(self, cells: torch.Tensor, last_norm, pos: torch.Tensor | None, y: torch.Tensor,
                      eval_pos: int) -> torch.Tensor:
        """The cell tokens the two-phase encoder takes: the cell encoder's output (``last_norm``:
        its last LayerNorm still to apply, as (module, output dtype)), the feature positional
        embedding and the target-aware row bias (:467-470, 1080-1132). On the GPU the three are
        one pass (``nori_layer_norm_cells``) where it takes the configuration."""
        scale = float(getattr(self, "target_aware_scale", 1.0))
        target_aware = self.use_target_aware_embedding and eval_pos > 0 and abs(scale) >= 1e-8
        if last_norm is not None:
            ln, out_dtype = last_norm
            b, s, g, e = cells.shape
            fused = (
                out_dtype == torch.float32 and cells.dtype in (torch.float16, torch.float32) and e in (64, 128, 256)
                and (pos is None or tuple(pos.shape) == (g, e)) and (not target_aware or scale == 1.0)
                and (not target_aware or self.reg_target_aware_embedding is not None)
                and cells.stride(-1) == 1 and cells.is_contiguous()
            )
            if fused:
                ctx = alpha = None
                if target_aware:
                    ctx = self.reg_target_aware_embedding(y[:, :eval_pos].unsqueeze(-1).to(out_dtype)).to(out_dtype)
                    ctx = ctx.contiguous()
                    if self.use_column_specific_y_aware and self.column_y_aware_alpha is not None:
                        alpha = torch.sigmoid(self.column_y_aware_alpha).to(out_dtype).reshape(1)
                out = torch.empty((b, s, g, e), dtype=torch.float32, device=cells.device)
                pos32 = None if pos is None else pos.to(torch.float32).contiguous()
                w = None if ln.weight is None else ln.weight.float().contiguous()
                bias = None if ln.bias is None else ln.bias.float().contiguous()
                ptr = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())
                nat.check(
                    nat.lib().nori_layer_norm_cells(
                        ptr(cells), nat.dtype_code(cells.dtype), b, s, g, e, e, ptr(w), ptr(bias), float(ln.eps),
                        ptr(pos32), ptr(ctx), eval_pos if ctx is not None else 0, ptr(alpha), 1.0 / self.embed_dim ** 0.5,
                        ptr(out), nat.stream_of(cells.device),
                    ),
                    "layer_norm_cells",
                )
                return out
            cells = layer_norm(cells, ln.weight, ln.bias, ln.eps, out_dtype=out_dtype)
        cells = self.apply_feature_positional_embeddings(cells, pos)
        return self.apply_target_aware_embedding(cells, y.clone(), task_type="reg", eval_pos=eval_pos)

    def process_4_x(self, data: dict):
        """Originally non-finite cells become NaN again after preprocessing (:1134-1139)."""
        data["data"] = torch.where(data["mask"].to(torch.bool), float("nan"), data["data"])
        return data

    # ------------------------------------------------------------ full forward (two-phase)
    def forward(
        self,
        x: torch.Tensor,
        y: torch.Tensor,
        eval_pos: int,
        y_type: torch.Tensor | None = None,
        task_type: Literal["reg", "cls"] = "cls",
        calculate_sample_attention: bool = False,
        calculate_feature_attention: bool = False,
        return_embeddings: bool = False,
        **kwargs: Any,
    ):
        """Context rows [0, eval_pos) and query rows [eval_pos, S) through the model together
        (:370-523, ``_forward_two_phase`` :525-562). x [B, S, F], y [B, >= eval_pos].

        Runs the two-phase encoder of Nori 1.5: the rows are preprocessed (context statistics
        and PLE edges from the context rows only), encoded into cell tokens with the feature
        positional and target-aware embeddings, passed through the cell and row layers, and
        the query rows' row states decoded into quantiles [B, S - eval_pos, Q]. With
        ``return_embeddings`` it returns the row states [B, S, width]; with ``mask_prediction``
        the reference's dict. The dense layer stack's uncached forward is not part of this
        package: dense models run through ``forward_cached_regression``.
        """
        if self.two_phase_config is None:
            raise NotImplementedError(
                "the uncached forward of the dense layer stack is not implemented here; use "
                "forward_cached_regression or build_context_cache / apply_context_cache"
            )
        assert x is not None and y is not None, "x and y must not be none"
        assert eval_pos > 0, "eval_pos must be a positive number"
        assert len(x.shape) == 3, "x must be [Batch, seq, Feature]"
        assert len(y.shape) == 2, "y must be [Batch, label]"
        assert eval_pos < x.shape[1] and eval_pos <= y.shape[1], (
            "The split point between train x and test x must be less than the feature dimension of x, "
            "and less than or equal to the label dimension of y"
        )
        if task_type != "reg":
            raise ValueError("the two-phase encoder (Model v3) supports regression only; pass task_type='reg'")
        if calculate_sample_attention or calculate_feature_attention:
            raise NotImplementedError("attention-score diagnostics are not computed by the HIP attention path")
        seq_len = x.shape[1]
        x_dict, n_pad = self._build_x_preprocess_inputs(x, eval_pos)
        pre = self.process_4_x(self.x_preprocess(x_dict))
        pre[MaskEmbEncoder.defer_last_norm_key] = x.is_cuda
        encoded = self.encoder_x(pre)
        cells, last_norm = encoded["data"], encoded.pop(MaskEmbEncoder.last_norm_key, None)
        out_dtype = cells.dtype if last_norm is None else last_norm[1]
        pos = self.make_feature_positional_embeddings(cells.shape[2], device=cells.device, dtype=out_dtype)
        if y.shape[1] < seq_len:
            y = torch.cat((y, torch.full((y.shape[0], seq_len - y.shape[1]), float("nan"), device=y.device, dtype=y.dtype)), 1)
        cells = self._finish_cells(cells, last_norm, pos, y, eval_pos)
        positions = torch.arange(seq_len, device=y.device).view(1, -1)
        y_masked = torch.where(positions >= eval_pos, torch.tensor(float("nan"), device=y.device, dtype=y.dtype), y)
        row_states, cell_states = self.transformer_encoder(cells, y_masked, eval_pos, inplace=True)
        if return_embeddings:
            return row_states
        reg_output = self.reg_y_decoder(row_states[:, eval_pos:])
        if not self.mask_prediction:
            return reg_output
        skip = self.feature_decoder is None or getattr(self, "_skip_feature_decoder", False)
        return {
            "reg_output": reg_output,
            "feature_pred": None if skip else self.feature_decoder(cell_states),
            "process_config": {
                "n_x_padding": n_pad,
                "features_per_group": self.features_per_group,
                "num_used_features": pre.get("_valid_feature_num"),
                "mean_for_normalization": pre.get("_norm_mean"),
                "std_for_normalization": pre.get("_norm_std"),
            },
        }

    def _require_context_cache(self) -> None:
        if self.two_phase_config is not None:
            raise NotImplementedError("context caching is not implemented for the two-phase encoder")
        if any(isinstance(step, PromptQuantilePLEEncoder) for step in self.x_preprocess):
            raise NotImplementedError("the context cache does not carry prompt-quantile PLE edges to query rows")

    # ------------------------------------------------------------ context-cache API
    def forward_cached_regression(
        self,
        x: torch.Tensor,
        y: torch.Tensor,
        eval_pos: int,
        *,
        row_chunk_size: int | None = None,
        cache_dtype: str = "bf16",
        offload_kv_cache: bool = False,
        fit_row_chunk: int | None = None,
        adaptive_query_chunk: bool = True,
        quantize_kv_cache: bool | None = None,
        adaptive_oom_chunk: bool | None = None,
    ) -> torch.Tensor:
        """Cached prediction of rows [eval_pos, S) against context rows [0, eval_pos): the
        build/apply pair (:716-811)."""
        self._require_context_cache()
        if quantize_kv_cache is not None and cache_dtype == "bf16":
            cache_dtype = "int8" if quantize_kv_cache else "bf16"
        if adaptive_oom_chunk is not None:
            adaptive_query_chunk = bool(adaptive_oom_chunk)
        if cache_dtype not in ("bf16", "int8"):
            raise ValueError(
                "forward_cached_regression takes a concrete cache_dtype of 'bf16' or 'int8', "
                f"got {cache_dtype!r}. Deciding which one is worth it needs the device budget."
            )
        if self.mask_prediction:
            raise NotImplementedError("forward_cached_regression requires mask_prediction=False")
        if x is None or y is None:
            raise AssertionError("x and y must not be none")
        if eval_pos <= 0:
            raise AssertionError("eval_pos must be a positive number")
        if len(x.shape) != 3:
            raise AssertionError("x must be [Batch, seq, Feature]")
        if len(y.shape) != 2:
            raise AssertionError("y must be [Batch, label]")
        if eval_pos >= x.shape[1] or eval_pos > y.shape[1]:
            raise AssertionError("Invalid eval_pos for cached regression")
        bundle = self.build_context_cache(
            x[:, :eval_pos], y[:, :eval_pos], cache_dtype=cache_dtype, offload_kv_cache=offload_kv_cache,
            fit_row_chunk=fit_row_chunk,
        )
        return self.apply_context_cache(
            x[:, eval_pos:], bundle, row_chunk_size=row_chunk_size, adaptive_query_chunk=adaptive_query_chunk
        )

    def build_context_cache(
        self,
        x_train: torch.Tensor,
        y_train: torch.Tensor,
        *,
        cache_dtype: str = "bf16",
        offload_kv_cache: bool = False,
        fit_row_chunk: int | None = None,
        quantize_kv_cache: bool | None = None,
        stream_context: bool = False,
        _hybrid_resident_int8_prefill: bool = False,
        fused_cache_write: bool = False,
    ) -> ContextCache:
        """Encode the context table once into a ``ContextCache`` (:813-959).

        int8 caches are written as the reference writes them: the K/V projection (the library
        GEMM), then the exact quantizer, so codes and scales are bit for bit the reference
        expression's on the same device. ``fused_cache_write`` (int8 caches under fp16 autocast)
        opts into the fused projection + quantizer kernel instead: one pass, the fp16 K/V never
        stored, but its MFMA summation order can move a code by one where a K/V value sits on an
        fp16 rounding boundary.
        """
        self._require_context_cache()
        if quantize_kv_cache is not None and cache_dtype == "bf16":
            cache_dtype = "int8" if quantize_kv_cache else "bf16"
        if cache_dtype not in ("bf16", "int8"):
            raise ValueError(f"build_context_cache takes a concrete cache_dtype of 'bf16' or 'int8', got {cache_dtype!r}.")
        if self.mask_prediction:
            raise NotImplementedError("build_context_cache requires mask_prediction=False")
        cfg = self.preprocess_config_x
        if not bool(cfg.get("normalize_on_train_only", True)) and (
            bool(cfg.get("normalize_x", False)) or bool(cfg.get("remove_outliers", False))
        ):
            raise NotImplementedError(
                "build_context_cache cannot preserve normalize_on_train_only=False: that transductive configuration "
                "derives preprocessing statistics from context and query rows together; use the uncached forward path"
            )
        if x_train is None or y_train is None:
            raise AssertionError("x_train and y_train must not be None")
        if len(x_train.shape) != 3:
            raise AssertionError("x_train must be [Batch, seq, Feature]")
        if len(y_train.shape) != 2:
            raise AssertionError("y_train must be [Batch, label]")
        eval_pos = x_train.shape[1]
        if eval_pos <= 0:
            raise AssertionError("x_train must have at least one context row")
        if y_train.shape[1] < eval_pos:
            raise AssertionError("y_train must cover all context rows")
        if _hybrid_resident_int8_prefill and (stream_context or offload_kv_cache or cache_dtype != "int8" or fit_row_chunk is None):
            raise ValueError(
                "hybrid resident INT8 prefill requires cache_dtype='int8', offload_kv_cache=False, "
                "stream_context=False, and a concrete context_row_chunk"
            )
        if stream_context or _hybrid_resident_int8_prefill:
            if stream_context and not offload_kv_cache:
                raise ValueError("stream_context requires offload_kv_cache=True")
            if fit_row_chunk is None:
                what = "stream_context" if stream_context else "hybrid resident INT8 prefill"
                raise ValueError(f"{what} requires a concrete context_row_chunk")
            return self._build_context_cache_streaming(
                x_train, y_train[:, :eval_pos], cache_dtype=cache_dtype, fit_row_chunk=fit_row_chunk,
                _hybrid_resident_int8_prefill=_hybrid_resident_int8_prefill, fused_cache_write=fused_cache_write,
            )

        x_dict, _ = self._build_x_preprocess_inputs(x_train, eval_pos)
        pre = self.x_preprocess(x_dict)
        stats = pre.get("_norm_stats") or {}
        norm_stats = {k: v.detach() for k, v in stats.items()} if stats else None
        nan_mean = pre.get("_nan_mean")
        nan_mean = nan_mean.detach() if isinstance(nan_mean, torch.Tensor) else None
        valid = pre.get("_valid_feature_num")
        valid = valid.detach() if isinstance(valid, torch.Tensor) else None
        pre = self.process_4_x(pre)
        data = pre["data"]
        pos_emb = self.make_feature_positional_embeddings(data.shape[2], device=data.device, dtype=data.dtype)
        target_aware_y, y_emb = self._encode_y_full(y_train[:, :eval_pos], total_rows=eval_pos, eval_pos=eval_pos, task_type="reg")
        x_enc = self._encode_x_rows(pre, slice(0, eval_pos), total_rows=eval_pos, feature_pos_emb=pos_emb)
        x_enc = self.apply_target_aware_embedding(x_enc, target_aware_y[:, :eval_pos], task_type="reg", eval_pos=eval_pos)
        tokens = torch.cat((x_enc, y_emb[:, :eval_pos].unsqueeze(2)), dim=2)
        _, caches = self.transformer_encoder.build_train_cache(
            tokens,
            feature_atten_mask=None,
            quantize_kv_cache=cache_dtype == "int8",
            offload_kv_cache=offload_kv_cache,
            fit_row_chunk=fit_row_chunk,
            device=data.device,
            fused_cache_write=fused_cache_write,
        )
        return ContextCache(
            caches=caches,
            feature_pos_emb=pos_emb,
            norm_stats=norm_stats,
            y_train=y_train[:, :eval_pos].detach(),
            eval_pos=eval_pos,
            nan_mean=nan_mean,
            valid_feature_num=valid,
        )

    def _build_context_cache_streaming(
        self, x_train: torch.Tensor, y_train: torch.Tensor, *, cache_dtype: str, fit_row_chunk: int,
        _hybrid_resident_int8_prefill: bool = False, fused_cache_write: bool = False,
    ) -> ContextCache:
        """Context cache with no full-N tensor on the device (reference transformer.py:1169-1301).

        The context statistics come from one pass over the raw table on the host; the rows are
        then preprocessed with those statistics frozen and encoded ``fit_row_chunk`` at a time on
        the device, and their tokens collected on the host, where the streamed layer builds read
        them. The query rows' (always NaN-masked) target embedding is drawn once from the
        context mean and kept in the bundle.
        """
        if x_train.device.type != "cpu" or y_train.device.type != "cpu":
            mode = "hybrid resident INT8 prefill" if _hybrid_resident_int8_prefill else "stream_context"
            raise ValueError(f"{mode} requires CPU x_train/y_train; upload only row chunks, not the full training matrix")
        device = next(self.parameters()).device
        eval_pos = x_train.shape[1]
        x_dict, _ = self._build_x_preprocess_inputs(x_train, eval_pos)
        pre = self.x_preprocess(x_dict)
        stats = pre.get("_norm_stats") or {}
        norm_stats = {k: v.detach() for k, v in stats.items()} if stats else None
        nan_mean = pre.get("_nan_mean")
        nan_mean = nan_mean.detach() if isinstance(nan_mean, torch.Tensor) else None
        valid = pre.get("_valid_feature_num")
        valid = valid.detach() if isinstance(valid, torch.Tensor) else None
        n_groups = (x_train.shape[2] + self.features_per_group - 1) // self.features_per_group
        pos_emb = self.make_feature_positional_embeddings(int(n_groups), device=device, dtype=x_train.dtype)
        del x_dict, pre, stats

        y_values = y_train.unsqueeze(-1)
        y_finite = torch.isfinite(y_values)
        y_nan_mean = torch.where(y_finite, y_values, torch.zeros_like(y_values)).sum(dim=1) / y_finite.sum(dim=1).clamp_min(1)
        y_nan_mean = y_nan_mean.to(device)
        query_y = {
            "data": torch.full((y_train.shape[0], 1, 1), float("nan"), device=device, dtype=y_train.dtype),
            "eval_pos": 1,
            "_frozen_nan_mean": y_nan_mean,
        }
        query_y_embedding = self.reg_y_encoder(query_y)["data"].squeeze(2).detach()

        tokens = None
        for r0 in range(0, eval_pos, fit_row_chunk):
            r1 = min(r0 + fit_row_chunk, eval_pos)
            width = r1 - r0
            chunk, _ = self._build_x_preprocess_inputs(x_train[:, r0:r1], width)
            if norm_stats is not None:
                chunk["_frozen_norm_stats"] = norm_stats
            if nan_mean is not None:
                chunk["_frozen_nan_mean"] = nan_mean
            if valid is not None:
                chunk["_frozen_valid_feature_num"] = valid
            chunk = self.process_4_x(self.x_preprocess(chunk))
            staged = {k: v.to(device) if isinstance(v, torch.Tensor) else v for k, v in chunk.items()}
            x_enc = self._encode_x_rows(staged, slice(0, width), total_rows=width, feature_pos_emb=pos_emb)
            y_rows = y_train[:, r0:r1].to(device)
            x_enc = self.apply_target_aware_embedding(x_enc, y_rows, eval_pos=width, task_type="reg")
            y_enc = self.reg_y_encoder({"data": y_rows.unsqueeze(-1), "eval_pos": width, "_frozen_nan_mean": y_nan_mean})
            host = torch.cat((x_enc, y_enc["data"].squeeze(2).unsqueeze(2)), dim=2).detach().to("cpu")
            if tokens is None:
                tokens = torch.empty((x_train.shape[0], eval_pos, *host.shape[2:]), dtype=host.dtype, device="cpu")
            tokens[:, r0:r1].copy_(host)
            del chunk, staged, x_enc, y_rows, y_enc, host
        if tokens is None:
            raise ValueError("stream_context received an empty context")

        _, caches = self.transformer_encoder.build_train_cache(
            tokens,
            feature_atten_mask=None,
            quantize_kv_cache=cache_dtype == "int8",
            offload_kv_cache=not _hybrid_resident_int8_prefill,
            fit_row_chunk=fit_row_chunk,
            device=device,
            stream_context=not _hybrid_resident_int8_prefill,
            _hybrid_resident_int8_prefill=_hybrid_resident_int8_prefill,
            fused_cache_write=fused_cache_write,
        )
        return ContextCache(
            caches=caches,
            feature_pos_emb=pos_emb,
            norm_stats=norm_stats,
            y_train=y_train[:, :0].detach(),
            eval_pos=eval_pos,
            nan_mean=nan_mean,
            valid_feature_num=valid,
            query_y_embedding=query_y_embedding,
        )

    def apply_context_cache(
        self,
        x_test: torch.Tensor,
        context: ContextCache,
        *,
        row_chunk_size: int | None = None,
        adaptive_query_chunk: bool = True,
        query_chunk_attempt_callback: Callable[[int, Literal["success", "oom"]], None] | None = None,
    ) -> torch.Tensor:
        """Score query rows against a prebuilt ``ContextCache``; mutates nothing on it
        (:961-1078). Returns ``[B, Nq, num_reg_quantiles]``."""
        self._require_context_cache()
        if self.mask_prediction:
            raise NotImplementedError("apply_context_cache requires mask_prediction=False")
        if len(x_test.shape) != 3:
            raise AssertionError("x_test must be [Batch, seq, Feature]")
        eval_pos = context.eval_pos
        n_test = x_test.shape[1]
        if n_test <= 0:
            raise AssertionError("x_test must have at least one query row")
        x_dict, _ = self._build_x_preprocess_inputs(x_test, n_test)
        dev = x_test.device
        if context.norm_stats is not None:
            x_dict["_frozen_norm_stats"] = {k: v.to(dev) for k, v in context.norm_stats.items()}
        if context.nan_mean is not None:
            x_dict["_frozen_nan_mean"] = context.nan_mean.to(dev)
        if context.valid_feature_num is not None:
            x_dict["_frozen_valid_feature_num"] = context.valid_feature_num.to(dev)
        pre = self.process_4_x(self.x_preprocess(x_dict))

        streamed = context.query_y_embedding is not None
        if not streamed:
            # a query target is NaN-masked whatever its value; encoding [context y ; NaN] keeps the
            # y encoder's context statistics, and its tail is every query row's embedding
            _, y_full = self._encode_y_full(context.y_train, total_rows=eval_pos + n_test, eval_pos=eval_pos, task_type="reg")
            y_query = y_full[:, eval_pos:]

        def run(start: int, end: int) -> torch.Tensor:
            if streamed:
                width = end - start
                device = next(self.parameters()).device
                part = self._slice_preprocessed_x(pre, slice(start, end), n_test)
                part = {k: v.to(device) if isinstance(v, torch.Tensor) else v for k, v in part.items()}
                xq = self._encode_x_rows(part, slice(0, width), total_rows=width, feature_pos_emb=context.feature_pos_emb)
                yq = context.query_y_embedding.to(device).expand(-1, width, -1)
            else:
                xq = self._encode_x_rows(pre, slice(start, end), total_rows=n_test, feature_pos_emb=context.feature_pos_emb)
                yq = y_query[:, start:end]
            out = self.transformer_encoder.forward_test_with_cache(
                torch.cat((xq, yq.unsqueeze(2)), dim=2), context.caches, feature_atten_mask=None
            )
            return self.reg_y_decoder(self.encoder_out_norm(out)[:, :, -1])

        chunk = n_test if row_chunk_size is None or row_chunk_size <= 0 else row_chunk_size
        outputs = []
        start = 0
        while start < n_test:
            end = min(start + chunk, n_test)
            try:
                outputs.append(run(start, end))
                start = end
            except torch.cuda.OutOfMemoryError:
                if query_chunk_attempt_callback is not None:
                    query_chunk_attempt_callback(chunk, "oom")
                # halve and keep the smaller chunk: what failed is a property of the request
                if not adaptive_query_chunk or chunk <= 1:
                    raise
                torch.cuda.empty_cache()
                chunk = max(1, chunk // 2)
        if query_chunk_attempt_callback is not None:
            query_chunk_attempt_callback(chunk, "success")
        return torch.cat(outputs, dim=1)
