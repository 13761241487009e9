"""Drop-in for the input encoders of ``synthefy_nori.model.encoders`` on the cached
regression path (the context encode of ``build_context_cache`` and the query encode of
``apply_context_cache``).

Same class names, constructor signatures and parameter names as the reference
(src/synthefy_nori/model/encoders.py), so a reference ``FeaturesTransformer`` state dict
loads into ``nori_amd.transformer.FeaturesTransformer`` with ``strict=True``:

* the x preprocessing chain ``preprocesss_4_x`` (:972-1009): ``NanEncoder`` (:588-653),
  ``NormalizationEncoder`` (:825-885) and ``ValidFeatureEncoder`` (:656-724), each with the
  frozen-statistics path the context cache uses to encode query rows with context stats;
* the x encoder ``get_x_encoder`` (:888-926): ``MaskEmbEncoder`` (:432-585) over the
  scientific-notation ``RBFembedding`` (:118-276, float64) or the linear numeric MLP;
* the regression y encoder ``get_reg_y_encoder`` (:945-969): ``NanEncoder`` +
  ``LinearEncoder`` (:80-115);
* the classification y encoder's modules (``EmbYEncoderStep`` :727-782,
  ``MulticlassTargetEncoder`` :785-822), kept for the state-dict schema.

* the prompt-quantile piecewise-linear cell coordinates of Nori 1.5
  (``PromptQuantilePLEEncoder`` :309-429): per-column context quantile edges built in the
  preprocessing chain, expanded into the last channels of each cell token by ``MaskEmbEncoder``.

These are small per-row torch expressions around the hot path (a few elementwise passes
and GEMMs of width E); they run as torch ops on the device the tensors live on. The PBLD
numeric embedding is not part of the nori models and raises ``NotImplementedError``.
"""

from __future__ import annotations

import ctypes
from typing import Any

import torch
import torch.nn as nn
from torch.nn.init import orthogonal_

from . import _native as nat
from .norm import layer_norm

__all__ = [
    "EmbYEncoderStep",
    "LinearEncoder",
    "MaskEmbEncoder",
    "MulticlassTargetEncoder",
    "NanEncoder",
    "NormalizationEncoder",
    "PromptQuantilePLEEncoder",
    "RBFembedding",
    "ValidFeatureEncoder",
    "calc_mean",
    "calc_std",
    "drop_outliers",
    "get_cls_y_encoder",
    "get_reg_y_encoder",
    "get_x_encoder",
    "normalize_mean0_std1",
    "preprocesss_4_x",
]


# ------------------------------------------------------------------- statistics (:12-77)
def calc_mean(x: torch.Tensor, dim: int):
    """Mean over the finite entries along ``dim`` and their count (at least 1) (:12-16)."""
    ok = torch.isfinite(x)
    count = ok.sum(dim=dim).clip(min=1)
    return torch.where(ok, x, torch.zeros_like(x)).sum(dim=dim) / count, count


def calc_std(x: torch.Tensor, dim: int, mean_v: torch.Tensor | None = None, value_num: torch.Tensor | None = None):
    """Sample standard deviation over the finite entries, n-1 clipped at 1 (:19-28)."""
    if mean_v is None or value_num is None:
        mean_v, value_num = calc_mean(x, dim)
    ok = torch.isfinite(x)
    sq = torch.where(ok, torch.square(mean_v.unsqueeze(dim) - x), torch.zeros_like(x))
    return torch.sqrt(sq.sum(dim=dim) / (value_num - 1).clip(min=1))


def _bounds(data: torch.Tensor, std_sigma: float, dim: int):
    mean, n = calc_mean(data, dim=dim)
    half = calc_std(data, dim=dim, mean_v=mean, value_num=n) * std_sigma
    return mean - half, mean + half


def drop_outliers(
    x: torch.Tensor,
    std_sigma: float = 4,
    eval_pos: int = -1,
    lower: torch.Tensor | None = None,
    upper: torch.Tensor | None = None,
    dim: int = 1,
):
    """Soft-clip to [mean - k std, mean + k std] of the context, the bounds computed twice
    (the second time without the first pass's outliers) unless given (:31-57)."""
    if lower is None:
        ctx = x[:, :eval_pos].clone()
        lower, upper = _bounds(ctx, std_sigma, dim)
        ctx[(ctx > upper.unsqueeze(dim)) | (ctx < lower.unsqueeze(dim))] = float("nan")
        lower, upper = _bounds(ctx, std_sigma, dim)
    x = torch.maximum(lower.unsqueeze(dim) - torch.log(1 + torch.abs(x)), x)
    x = torch.minimum(upper.unsqueeze(dim) + torch.log(1 + torch.abs(x)), x)
    return x, lower, upper


def normalize_mean0_std1(
    x: torch.Tensor,
    eval_pos: int = -1,
    clip: bool = True,
    dim: int = 1,
    mean: torch.Tensor | None = None,
    std: torch.Tensor | None = None,
):
    """(x - mean) / std with context statistics (std + 1e-20; 1 for a single row), clipped to
    +-100 (:60-77)."""
    if mean is None:
        mean, n = calc_mean(x[:, :eval_pos], dim=dim)
        std = calc_std(x[:, :eval_pos], dim=dim, mean_v=mean, value_num=n) + 1e-20
        if x.shape[1] == 1 or eval_pos == 1:
            std[:] = 1.0
    x = (x - mean.unsqueeze(1).expand_as(x)) / std.unsqueeze(1).expand_as(x)
    if clip:
        x = torch.clip(x, min=-100, max=100)
    return x, mean, std


# ------------------------------------------------------------------------------ steps
class LinearEncoder(nn.Module):
    """Concatenate ``in_keys`` on the last axis and apply one Linear (:80-115)."""

    def __init__(
        self,
        num_features: int,
        emsize: int,
        nan_to_zero: bool = False,
        bias: bool = True,
        in_keys: list[str] = ["data"],
        out_key: str = "data",
    ):
        super().__init__()
        self.layer = nn.Linear(num_features, emsize, bias=bias)
        self.nan_to_zero = nan_to_zero
        self.in_keys = in_keys
        self.out_key = out_key

    def forward(self, input: dict[str, Any]) -> dict[str, Any]:
        absent = [k for k in self.in_keys if k not in input]
        assert not absent, f"Missing encoder inputs: {absent}"
        x = torch.cat([input[k] for k in self.in_keys], dim=-1)
        if self.nan_to_zero:
            x = torch.nan_to_num(x, nan=0.0, posinf=0.0, neginf=0.0)
        input[self.out_key] = self.layer(x)
        return input


def _operand_dtype(dtype: torch.dtype) -> torch.dtype:
    """The dtype an F.linear on the current device computes in: the autocast dtype when
    autocast is on, else the given one."""
    return torch.get_autocast_dtype("cuda") if torch.is_autocast_enabled("cuda") else dtype


class RBFembedding(nn.Module):
    """Scientific-notation RBF embedding of a scalar (:118-276).

    |x| = m * 10^e with m in [0, 10) and |e| <= 10^digits - 1; m is expanded over Gaussian
    kernels on a fixed grid of centers (float64 on the device), then modulated by a gate
    (sigmoid) and shift (tanh) computed from embeddings of sign(x), sign(e) and the digits of
    |e|, layer-normed and projected.
    """

    def __init__(
        self,
        embedding_size: int = 96,
        exponent_digits: int = 1,
        token_embed_dim: int = 32,
        n_kernels: int = 32,
        sigma: float = 1.05,
        use_learn_sigma: bool = False,
        center_range: tuple = (0.0, 10.0),
        use_learn_embeddings: bool = False,
        as_tokenizer: bool = False,
        use_original_features: bool = False,
        dtype: torch.dtype = torch.float32,
    ):
        super().__init__()
        self.dtype = dtype
        self.n_kernels = n_kernels
        self.exponent_digits = exponent_digits
        self.as_tokenizer = as_tokenizer
        self.use_original_features = use_original_features
        lo, hi = center_range
        grid = (
            torch.tensor([(lo + hi) / 2.0], dtype=torch.float32)
            if n_kernels <= 1
            else torch.linspace(lo, hi, steps=n_kernels, dtype=torch.float32)
        )
        self.register_buffer("centers", grid, persistent=False)
        if use_learn_sigma:
            self.sigma = nn.Parameter(torch.tensor(sigma, dtype=dtype))
        else:
            self.register_buffer("sigma", torch.tensor(sigma, dtype=dtype))
        if exponent_digits > 0:
            self.sign_embedding = nn.Embedding(2, token_embed_dim, dtype=dtype)
            self.exp_sign_embedding = nn.Embedding(2, token_embed_dim, dtype=dtype)
            self.exp_digit_embedding = nn.Embedding(10, token_embed_dim, dtype=dtype)
            for emb in (self.sign_embedding, self.exp_sign_embedding, self.exp_digit_embedding):
                emb.weight.requires_grad = bool(use_learn_embeddings)
            self.gate_mlp = nn.Sequential(
                nn.Linear((exponent_digits + 2) * token_embed_dim, 4 * token_embed_dim, dtype=dtype),
                nn.GELU(),
                nn.Linear(4 * token_embed_dim, 2 * n_kernels, dtype=dtype),
            )
        else:
            self.sign_embedding = self.exp_sign_embedding = self.exp_digit_embedding = None
            self.gate_mlp = None
        self.norm = nn.LayerNorm(n_kernels, dtype=dtype)
        self.out_layer = nn.Linear(n_kernels + (1 if use_original_features else 0), embedding_size, dtype=dtype)

    def _load_from_state_dict(self, state_dict, prefix, local_metadata, strict, missing_keys, unexpected_keys, error_msgs):
        # Some checkpoints persisted the (deterministic) centers; accept the key only when it
        # holds the canonical grid, so a different grid still fails a strict load (:178-217).
        key = prefix + "centers"
        saved = state_dict.get(key)
        grid = self.centers.detach()
        if torch.is_tensor(saved) and saved.shape == grid.shape and torch.equal(saved.to(grid.device, grid.dtype), grid):
            state_dict = dict(state_dict)
            del state_dict[key]
        super()._load_from_state_dict(state_dict, prefix, local_metadata, strict, missing_keys, unexpected_keys, error_msgs)

    def _mantissa_exponent(self, xw: torch.Tensor):
        mag = torch.abs(xw)
        zero = mag == 0
        top = 10**self.exponent_digits - 1
        e = torch.clamp(torch.floor(torch.log10(torch.where(zero, torch.ones_like(mag), mag))), -top, top).to(torch.int64)
        m = mag / (10.0 ** e.to(xw.dtype))
        return torch.where(zero, torch.zeros_like(m), m), e

    def gate_table(self, device: torch.device) -> torch.Tensor:
        """[40, 2, n_kernels]: sigmoid(gamma) and tanh(beta) of the gate for every row the gate
        MLP can see -- row 20 s + 10 t + d for sign s of x, sign t of the exponent and exponent
        digit d (one exponent digit) -- through the module's own embeddings, gate MLP and
        activations under the current autocast state; cached until a weight or that state
        changes."""
        params = [self.sign_embedding.weight, self.exp_sign_embedding.weight, self.exp_digit_embedding.weight]
        params += [p for p in self.gate_mlp.parameters()]
        state = (torch.is_autocast_enabled("cuda"), torch.get_autocast_dtype("cuda"))
        key = (device, state) + tuple((p.data_ptr(), p._version) for p in params)
        cached = getattr(self, "_gate_table", None)
        if cached is None or cached[0] != key:
            with torch.no_grad():
                r = torch.arange(40, device=device)
                parts = [self.sign_embedding(r // 20), self.exp_sign_embedding((r // 10) % 2), self.exp_digit_embedding(r % 10)]
                gb = self.gate_mlp(torch.cat(parts, dim=-1).to(self.dtype))
                gamma, beta = torch.split(gb, self.n_kernels, dim=-1)
                table = torch.stack((torch.sigmoid(gamma), torch.tanh(beta)), dim=1).contiguous()
            cached = self._gate_table = (key, table)
        return cached[1]

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x = x.squeeze(-1)
        rows = x.shape[0]
        work = torch.float32 if x.device.type == "mps" else torch.float64
        xw = x.to(work)
        if self.gate_mlp is not None:
            m, e = self._mantissa_exponent(xw)
        else:
            m, e = xw, None
        c = self.centers.to(work).view((1,) * m.dim() + (self.n_kernels,))
        rbf = torch.exp(-((m.unsqueeze(-1) - c) ** 2) / (2 * (self.sigma**2))).to(self.dtype)
        if self.gate_mlp is not None:
            parts = [self.sign_embedding((xw < 0).long()), self.exp_sign_embedding((e < 0).long())]
            mag = e.abs()
            # most significant exponent digit first
            for p in reversed(range(self.exponent_digits)):
                parts.append(self.exp_digit_embedding((mag // (10**p)) % 10))
            gb = self.gate_mlp(torch.cat(parts, dim=-1).to(self.dtype))
            gamma, beta = torch.split(gb, self.n_kernels, dim=-1)
            pre = rbf * torch.sigmoid(gamma) + torch.tanh(beta)
            if pre.is_cuda:
                # the norm on the HIP kernel, written as the operand out_layer computes with
                # (fp16 under fp16 autocast: the same rounding of the same fp32 value)
                op = _operand_dtype(pre.dtype) if not self.use_original_features else pre.dtype
                rbf = layer_norm(pre, self.norm.weight, self.norm.bias, self.norm.eps, out_dtype=op)
            else:
                rbf = self.norm(pre)
        if self.use_original_features:
            rbf = torch.cat([rbf, x.unsqueeze(-1)], dim=-1)
        out = self.out_layer(rbf if rbf.dtype == _operand_dtype(self.dtype) else rbf.to(self.dtype))
        return out if self.as_tokenizer else out.reshape(rows, -1)


class PromptQuantilePLEEncoder(nn.Module):
    """Context-only quantile edges for piecewise-linear cell coordinates (:309-429).

    Preprocessing step: for every (table, group, feature) column it stores ``n_bins + 1``
    edges, the quantiles at levels 0, 1/n_bins, ..., 1 of the column's valid context cells
    (finite and not masked), linearly interpolated between order statistics; a column without
    valid cells gets zero edges. Query rows never influence the edges, and a caller may pass
    edges built earlier under ``frozen_reference_key``. ``encode`` turns cell values into the
    coordinates ``MaskEmbEncoder`` appends to each cell token.
    """

    reference_key = "_prompt_quantile_ple_reference"
    frozen_reference_key = "_frozen_prompt_quantile_ple_reference"

    def __init__(self, n_bins: int):
        super().__init__()
        if n_bins < 2:
            raise ValueError("prompt-quantile PLE requires at least 2 bins")
        self.n_bins = int(n_bins)
        self.register_buffer(
            "quantile_levels", torch.linspace(0.0, 1.0, self.n_bins + 1, dtype=torch.float32), persistent=False
        )

    def _context_edges(self, x: torch.Tensor, valid: torch.Tensor, eval_pos: int) -> dict[str, torch.Tensor]:
        ctx, ok = x[:, :eval_pos], valid[:, :eval_pos]
        # invalid cells rank last, so the k-th valid value of a column sits at index k
        ranked = torch.where(ok, ctx, torch.full_like(ctx, float("inf"))).permute(0, 2, 3, 1).sort(dim=-1).values
        n_valid = ok.sum(dim=1)  # [B, G, F]
        rank = (n_valid - 1).clamp(min=0).to(x.dtype).unsqueeze(-1) * self.quantile_levels.to(x.device, x.dtype)
        below, above = rank.floor().to(torch.long), rank.ceil().to(torch.long)
        lo, hi = ranked.gather(-1, below), ranked.gather(-1, above)
        edges = lo + (rank - below.to(rank.dtype)) * (hi - lo)
        edges = torch.where(n_valid.unsqueeze(-1) > 0, edges, torch.zeros_like(edges))
        return {"edges": edges.detach()}

    def _checked(self, reference: dict, x: torch.Tensor) -> dict[str, torch.Tensor]:
        edges = reference.get("edges")
        if not isinstance(edges, torch.Tensor):
            raise TypeError("prompt-quantile PLE reference is missing tensor 'edges'")
        want = (x.shape[0], x.shape[2], x.shape[3], self.n_bins + 1)
        if tuple(edges.shape) != want:
            raise ValueError(f"prompt-quantile PLE reference has shape {tuple(edges.shape)}, expected {want}")
        return {"edges": edges.to(device=x.device, dtype=x.dtype)}

    def forward(self, input: dict[str, Any]) -> dict[str, Any]:
        x, mask = input.get("data"), input.get("mask")
        if not isinstance(x, torch.Tensor) or not isinstance(mask, torch.Tensor):
            raise TypeError("PromptQuantilePLEEncoder requires tensor data and mask inputs")
        if x.dim() != 4 or mask.shape != x.shape:
            raise ValueError("PromptQuantilePLEEncoder expects data and mask shaped [batch, rows, groups, features]")
        frozen = input.get(self.frozen_reference_key)
        if frozen is None:
            eval_pos = int(input["eval_pos"])
            if eval_pos <= 0 or eval_pos > x.shape[1]:
                raise ValueError(f"eval_pos must select a non-empty context prefix, got {eval_pos} for {x.shape[1]} rows")
            reference = self._context_edges(x, torch.isfinite(x) & ~mask.to(torch.bool), eval_pos)
        elif isinstance(frozen, dict):
            reference = frozen
        else:
            raise TypeError("_frozen_prompt_quantile_ple_reference must be a dictionary")
        input[self.reference_key] = self._checked(reference, x)
        return input

    @staticmethod
    def encode(x: torch.Tensor, reference: dict[str, torch.Tensor]) -> torch.Tensor:
        """Coordinates [B, S, G, F, n_bins] of cells x [B, S, G, F]: channel i is
        clamp((x - e_i) / (e_{i+1} - e_i), 0, 1), so bins below the value read 1, its own bin
        the fraction, bins above 0. A bin of zero width and a non-finite cell read 0."""
        edges = reference["edges"].to(device=x.device, dtype=x.dtype)
        left = edges[..., :-1].unsqueeze(-2)
        width = (edges[..., 1:] - edges[..., :-1]).unsqueeze(-2)
        open_bin = width > 0
        values = x.permute(0, 2, 3, 1).unsqueeze(-1)  # [B, G, F, S, 1]
        coords = ((values - left) / torch.where(open_bin, width, torch.ones_like(width))).clamp(0.0, 1.0)
        coords = torch.where(torch.isfinite(values) & open_bin, coords, torch.zeros_like(coords))
        return coords.permute(0, 3, 1, 2, 4).contiguous()


class MaskEmbEncoder(nn.Module):
    """Per-cell numeric embedding, a learned vector for missing cells, and a fusion MLP over a
    group's cells (:432-585). With ``prompt_quantile_ple_bins`` > 0 (Nori 1.5) the numeric
    embedding fills the first E - bins channels of a cell token and the cell's PLE
    coordinates the rest."""

    def __init__(
        self,
        num_features: int,
        emsize: int,
        mask_embedding_size: int,
        numeric_embed_type: str = "linear",
        RBF_config: dict | None = None,
        PBLD_config: dict | None = None,
        prompt_quantile_ple_bins: int = 0,
        nan_to_zero: bool = False,
        bias: bool = True,
        in_keys: list[str] = ["data"],
        out_key: str = "data",
    ):
        super().__init__()
        bins = int(prompt_quantile_ple_bins)
        if bins < 0:
            raise ValueError("prompt_quantile_ple_bins cannot be negative")
        if bins == 1:
            raise ValueError("prompt_quantile_ple_bins must be 0 (disabled) or at least 2")
        if bins >= emsize:
            raise ValueError("prompt_quantile_ple_bins must be smaller than the embedding dimension")
        if bins and in_keys != ["data"]:
            raise ValueError("prompt-quantile PLE requires in_keys=['data']")
        if bins and numeric_embed_type != "RBF":
            raise ValueError("prompt-quantile PLE is supported only with the RBF numeric encoder")
        self.embedding_dim = emsize
        self.mask_embedding_size = mask_embedding_size
        self.in_keys = in_keys
        self.out_key = out_key
        self.prompt_quantile_ple_bins = bins
        self.mask_embedding = nn.Parameter(torch.randn(mask_embedding_size))
        self.numeric_embed_type = numeric_embed_type
        half = emsize // 2
        if numeric_embed_type == "linear":
            self.numeric_mlp = nn.Sequential(
                nn.Linear(1, half), nn.LayerNorm(half), nn.ReLU(), nn.Linear(half, emsize), nn.LayerNorm(emsize), nn.ReLU()
            )
        elif numeric_embed_type == "RBF":
            cfg = dict(RBF_config or {})
            for key, only in (("input_transform", "scientific"), ("compute_dtype", "float64"), ("use_raw_input_residual", False)):
                if key in cfg and cfg[key] != only:
                    raise ValueError(f"Unsupported RBF_config options in this release: {{{key!r}: {cfg[key]!r}}}")
            self.numeric_mlp = RBFembedding(
                embedding_size=emsize - bins,
                exponent_digits=1,
                token_embed_dim=cfg["token_embed_dim"],
                n_kernels=cfg["n_kernels"],
                sigma=cfg["sigma"],
                use_learn_sigma=cfg["use_learn_sigma"],
                use_learn_embeddings=cfg["use_learn_embeddings"],
                center_range=(0.0, 10.0),
                use_original_features=cfg["use_original_features"],
                as_tokenizer=True,
            )
        elif numeric_embed_type == "PBLD":
            raise NotImplementedError("the PBLD numeric embedding is not part of the cached nori models")
        else:
            raise ValueError(f"Invalid numeric_embed_type: {numeric_embed_type}")
        self.fusion_network = nn.Sequential(
            nn.Linear(num_features * emsize, emsize, bias=bias),
            nn.LayerNorm(emsize),
            nn.ReLU(),
            nn.Linear(emsize, emsize, bias=bias),
            nn.LayerNorm(emsize),
        )
        self.nan_to_zero = nan_to_zero

    def forward(self, input: dict[str, Any]) -> dict[str, Any]:
        absent = [k for k in self.in_keys if k not in input]
        assert not absent, f"Missing encoder inputs: {absent}"
        x = torch.cat([input[k] for k in self.in_keys], dim=-1)
        b, s, g, _ = x.shape
        h = self._tokens_on_device(x, input) if x.is_cuda else None
        if h is not None:
            input[self.out_key] = self._fusion_on_device(h, input).view(b, s, g, -1)
            return input
        x = x.unsqueeze(-1)
        missing = torch.isnan(x)
        x = x.masked_fill(missing, 0.0)
        emb = self.numeric_mlp(x)
        if self.prompt_quantile_ple_bins:
            reference = input.get(PromptQuantilePLEEncoder.reference_key)
            if not isinstance(reference, dict):
                raise TypeError("prompt-quantile PLE reference is required when the tokenizer is enabled")
            emb = torch.cat((emb, PromptQuantilePLEEncoder.encode(x.squeeze(-1), reference).to(emb.dtype)), dim=-1)
        if not self.nan_to_zero:
            emb = torch.where(missing, self.mask_embedding.expand_as(emb), emb)
        h = emb.flatten(3)
        input[self.out_key] = (self._fusion_on_device(h, input) if h.is_cuda else self.fusion_network(h)).view(b, s, g, -1)
        return input

    def _tokens_on_device(self, x: torch.Tensor, input: dict[str, Any]) -> torch.Tensor | None:
        """The fusion network's fp16 operand [b, s, g, features * E] straight from the cell
        values under fp16 autocast (``nori_cell_tokens``: masked fill, RBF embedding, PLE
        coordinates and the mask embedding in one pass; the values torch's ops give, up to the
        order of the LayerNorm's and the output projection's fp32 sums), or None where the
        kernel does not take the configuration."""
        rbf = self.numeric_mlp
        if not (torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") == torch.float16
                and isinstance(rbf, RBFembedding) and rbf.gate_mlp is not None and rbf.exponent_digits == 1
                and not rbf.use_original_features and rbf.n_kernels in (16, 32) and self.prompt_quantile_ple_bins == 32
                and rbf.out_layer.out_features == 96 and self.embedding_dim == 128 and x.dtype == torch.float32
                and (self.nan_to_zero or self.mask_embedding.numel() == 128)):
            return None
        reference = input.get(PromptQuantilePLEEncoder.reference_key)
        if not isinstance(reference, dict):
            return None
        edges = reference["edges"]
        b, s, g, f = x.shape
        if tuple(edges.shape) != (b, g, f, 33) or edges.device != x.device:
            return None
        dev = x.device
        key = (dev,) + tuple((p.data_ptr(), p._version) for p in rbf.out_layer.parameters())
        cached = getattr(self, "_out16", None)
        if cached is None or cached[0] != key:
            with torch.no_grad():
                bias = rbf.out_layer.bias
                cached = self._out16 = (key, rbf.out_layer.weight.to(dev, torch.float16).contiguous(),
                                        None if bias is None else bias.to(dev, torch.float16).contiguous())
        w16, b16 = cached[1:]
        table = rbf.gate_table(dev)
        x = x.contiguous()
        edges = edges.to(torch.float32).contiguous()
        ln_w = None if rbf.norm.weight is None else rbf.norm.weight.float().contiguous()
        ln_b = None if rbf.norm.bias is None else rbf.norm.bias.float().contiguous()
        mask = None if self.nan_to_zero else self.mask_embedding.float().contiguous()
        h = torch.empty((b, s, g, f * self.embedding_dim), dtype=torch.float16, device=dev)
        ptr = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())
        nat.check(
            nat.lib().nori_cell_tokens(
                ptr(x), b, s, g, f, rbf.n_kernels, ptr(rbf.centers.float().contiguous()), ptr(rbf.sigma.float().reshape(1)),
                ptr(table), ptr(ln_w), ptr(ln_b), float(rbf.norm.eps), ptr(w16), ptr(b16), 96, ptr(edges), 32, ptr(mask),
                ptr(h), nat.stream_of(dev),
            ),
            "cell_tokens",
        )
        return h

    # A caller that applies the last LayerNorm itself (fused with what follows it) sets this key
    # in the input dict; the encoder then leaves the norm out, and returns it under
    # ``last_norm_key`` as (module, output dtype).
    defer_last_norm_key = "_defer_last_norm"
    last_norm_key = "_last_norm"

    def _fusion_on_device(self, h: torch.Tensor, input: dict[str, Any] | None = None) -> torch.Tensor:
        """fusion_network (Linear -> LayerNorm -> ReLU -> Linear -> LayerNorm) with the norms on
        the HIP kernel: the first writes the ReLU'd operand of the second Linear in the dtype it
        computes in, the second the fp32 (autocast) or input-dtype output torch's would."""
        lin1, ln1, _, lin2, ln2 = self.fusion_network
        h = lin1(h)
        h = layer_norm(h, ln1.weight, ln1.bias, ln1.eps, relu=True, out_dtype=_operand_dtype(h.dtype))
        h = lin2(h)
        autocast = torch.is_autocast_enabled("cuda")
        out_dtype = torch.float32 if autocast else h.dtype
        if input is not None and input.get(self.defer_last_norm_key):
            input[self.last_norm_key] = (ln2, out_dtype)
            return h
        return layer_norm(h, ln2.weight, ln2.bias, ln2.eps, out_dtype=out_dtype)


class NanEncoder(nn.Module):
    """Fill NaN/+-inf with the context column mean (or the frozen one) and emit a signed
    indicator channel: nan -> -2, +inf -> 2, -inf -> 4 (:588-653)."""

    def __init__(
        self,
        nan_value: float = -2.0,
        inf_value: float = 2.0,
        neg_info_value: float = 4.0,
        in_keys: list[str] = ["data"],
        out_key: str = "nan_encoding",
    ):
        super().__init__()
        self.nan_value = nan_value
        self.inf_value = inf_value
        self.neg_info_value = neg_info_value
        self.in_keys = in_keys
        self.out_key = out_key

    def forward(self, input: dict[str, Any]) -> dict[str, Any]:
        x: torch.Tensor = input[self.in_keys[0]]
        fill = input.get("_frozen_nan_mean")
        if fill is None:
            fill, _ = calc_mean(x[:, : input["eval_pos"], :], dim=1)
        input["_nan_mean"] = fill
        nan = torch.isnan(x)
        pinf = torch.isinf(x) & (x > 0)
        ninf = torch.isinf(x) & (x < 0)
        zero = torch.zeros_like(x)
        indicator = torch.where(nan, self.nan_value, torch.where(pinf, self.inf_value, torch.where(ninf, self.neg_info_value, zero)))
        input[self.in_keys[0]] = torch.where(nan | pinf | ninf, fill.unsqueeze(1).expand_as(x), x)
        input[self.out_key] = indicator
        return input


class ValidFeatureEncoder(nn.Module):
    """Scale by sqrt(num_features / valid features of the context) and zero-pad to
    ``num_features`` (:656-724). A feature is valid when the context holds more than one
    finite, originally present value and they are not all equal."""

    def __init__(
        self,
        num_features: int,
        nan_normalize: bool = True,
        sqrt_normalize: bool = True,
        in_keys: list[str] = ["data"],
        out_key: str = "data",
    ):
        super().__init__()
        self.num_features = num_features
        self.nan_normalize = nan_normalize
        self.sqrt_normalize = sqrt_normalize
        self.in_keys = in_keys
        self.out_key = out_key
        self.valid_feature_num = None

    def forward(self, input: dict[str, Any]) -> dict[str, Any]:
        x: torch.Tensor = input[self.in_keys[0]]
        valid = input.get("_frozen_valid_feature_num")
        if valid is None:
            ep = int(input["eval_pos"])
            ctx = x[:, :ep]
            orig = input.get("mask")
            if self.in_keys[0] == "data" and isinstance(orig, torch.Tensor) and orig.shape == x.shape:
                ctx = torch.where(orig[:, :ep].to(torch.bool), torch.full_like(ctx, float("nan")), ctx)
            ok = torch.isfinite(ctx)
            lo = torch.where(ok, ctx, torch.full_like(ctx, float("inf"))).amin(dim=1)
            hi = torch.where(ok, ctx, torch.full_like(ctx, float("-inf"))).amax(dim=1)
            usable = (ok.sum(dim=1) > 1) & (lo != hi)
            valid = torch.clip(usable.sum(-1).unsqueeze(-1), min=1)
        self.valid_feature_num = valid.detach()
        input["_valid_feature_num"] = valid
        if self.nan_normalize:
            if self.sqrt_normalize:
                x = x * torch.sqrt(self.num_features / valid).unsqueeze(1).expand_as(x)
            else:
                x = x * (self.num_features / valid)
        pad = torch.zeros(*x.shape[:-1], self.num_features - x.shape[-1], device=x.device, dtype=x.dtype)
        input[self.out_key] = torch.cat([x, pad], -1)
        return input


class NormalizationEncoder(nn.Module):
    """Outlier soft-clip and mean-0/std-1 normalization with context statistics, or with the
    frozen ones a context cache carries (:825-885)."""

    def __init__(
        self,
        train_only: bool,
        normalize_x: bool,
        remove_outliers: bool,
        std_sigma: float = 4.0,
        in_keys: list[str] = ["data"],
        out_key: str = "data",
    ):
        super().__init__()
        self.train_only = train_only
        self.normalize_x = normalize_x
        self.remove_outliers = remove_outliers
        self.std_sigma = std_sigma
        self.in_keys = in_keys
        self.out_key = out_key
        self.mean = None
        self.std = None

    def forward(self, input: dict[str, Any]) -> dict[str, Any]:
        x = input[self.in_keys[0]]
        pos = input["eval_pos"] if self.train_only else x.shape[1]
        frozen = input.get("_frozen_norm_stats") or {}
        used: dict[str, torch.Tensor] = {}
        if self.remove_outliers:
            x, used["lower"], used["upper"] = drop_outliers(
                x, eval_pos=pos, std_sigma=self.std_sigma, lower=frozen.get("lower"), upper=frozen.get("upper")
            )
        if self.normalize_x:
            x, mean, std = normalize_mean0_std1(x, eval_pos=pos, mean=frozen.get("mean"), std=frozen.get("std"))
            self.mean, self.std = mean.detach(), std.detach()
            input["_norm_mean"], input["_norm_std"] = mean, std
            used["mean"], used["std"] = mean, std
        input[self.out_key] = x
        input["_norm_stats"] = used
        return input


class EmbYEncoderStep(nn.Module):
    """Class-index embedding for context targets and a mask vector for query rows; rows of
    one orthogonal (n_classes + 1) x emsize matrix (:727-782)."""

    def __init__(self, *, emsize: int, n_classes: int = 10, in_keys: list[str] = ["data"], out_key: str = "data"):
        super().__init__()
        assert emsize > n_classes + 1, f"emsize ({emsize}) must be >= n_classes+1 ({n_classes + 1}) for orthogonal initialization"
        basis = torch.empty(n_classes + 1, emsize)
        orthogonal_(basis)
        self.y_embedding = nn.Embedding(n_classes, emsize)
        self.y_embedding.weight.data = basis[:n_classes].clone()
        self.y_mask = nn.Embedding(1, emsize)
        self.y_mask.weight.data = basis[n_classes:].clone()
        self.in_keys = in_keys
        self.out_key = out_key

    def forward(self, input: dict[str, Any]) -> dict[str, Any]:
        y = input[self.in_keys[0]].int()
        ep = input["eval_pos"]
        input[self.out_key] = torch.cat([self.y_embedding(y[:, :ep]), self.y_mask(torch.zeros_like(y[:, ep:]))], dim=1)
        return input


class MulticlassTargetEncoder(nn.Module):
    """Rank-remap class labels to 0..K-1 over the classes present in the context (:785-822)."""

    MAX_CLASSES: int = 10

    def __init__(self, in_keys: list[str] = ["data"], out_key: str = "data"):
        super().__init__()
        self.in_keys = in_keys
        self.out_key = out_key

    def forward(self, input: dict[str, Any]) -> dict[str, Any]:
        x: torch.Tensor = input[self.in_keys[0]]
        ids = torch.arange(self.MAX_CLASSES, device=x.device, dtype=x.dtype)
        present = (x[:, : input["eval_pos"], :] == ids).any(dim=1).long()
        rank = torch.cumsum(present, dim=1) - present  # classes present below each index
        idx = x[:, :, 0].long().clamp(0, self.MAX_CLASSES - 1)
        input[self.out_key] = torch.gather(rank, 1, idx).unsqueeze(-1).to(x.dtype)
        return input


# -------------------------------------------------------------------------- factories
def get_x_encoder(
    *,
    num_features: int,
    embedding_size: int,
    mask_embedding_size: int,
    encoder_use_bias: bool,
    numeric_embed_type: str = "linear",
    RBF_config: dict | None = None,
    PBLD_config: dict | None = None,
    prompt_quantile_ple_bins: int = 0,
    in_keys: list = ["data"],
    nan_to_zero: bool = False,
):
    """``nn.Sequential(MaskEmbEncoder)`` over ``in_keys`` (:888-926)."""
    assert isinstance(in_keys, list), "The type of in_keys must be a list!"
    return nn.Sequential(
        MaskEmbEncoder(
            num_features=num_features * len(in_keys),
            emsize=embedding_size,
            mask_embedding_size=mask_embedding_size,
            nan_to_zero=nan_to_zero,
            bias=encoder_use_bias,
            in_keys=in_keys,
            RBF_config=RBF_config,
            PBLD_config=PBLD_config,
            prompt_quantile_ple_bins=prompt_quantile_ple_bins,
            numeric_embed_type=numeric_embed_type,
        )
    )


def get_cls_y_encoder(*, num_inputs: int, embedding_size: int, nan_handling_y_encoder: bool, max_num_classes: int) -> nn.Module:
    """[NanEncoder] -> [MulticlassTargetEncoder] -> EmbYEncoderStep (:929-942)."""
    steps: list[nn.Module] = []
    if nan_handling_y_encoder:
        steps.append(NanEncoder(in_keys=["data"], out_key="nan_encoding"))
    if max_num_classes >= 2:
        steps.append(MulticlassTargetEncoder())
    steps.append(EmbYEncoderStep(emsize=embedding_size, n_classes=max_num_classes))
    return nn.Sequential(*steps)


def get_reg_y_encoder(*, num_inputs: int, embedding_size: int, nan_handling_y_encoder: bool, max_num_classes: int = 10) -> nn.Module:
    """[NanEncoder] -> LinearEncoder over the value (and its NaN indicator) (:945-969)."""
    steps: list[nn.Module] = []
    keys = ["data"]
    if nan_handling_y_encoder:
        steps.append(NanEncoder(in_keys=["data"], out_key="nan_encoding"))
        keys.append("nan_encoding")
    steps.append(
        LinearEncoder(
            num_features=num_inputs * len(keys),
            emsize=embedding_size,
            nan_to_zero=not nan_handling_y_encoder,
            in_keys=keys,
            out_key="data",
        )
    )
    return nn.Sequential(*steps)


def preprocesss_4_x(
    *,
    num_features: int,
    nan_handling_enabled: bool,
    normalize_on_train_only: bool,
    normalize_x: bool,
    remove_outliers: bool,
    normalize_by_used_features: bool,
    prompt_quantile_ple_bins: int = 0,
):
    """[NanEncoder] -> NormalizationEncoder -> ValidFeatureEncoder [-> PromptQuantilePLEEncoder]
    (:972-1009)."""
    steps: list[nn.Module] = []
    if nan_handling_enabled:
        steps.append(NanEncoder(in_keys=["data"], out_key="nan_encoding"))
    steps.append(NormalizationEncoder(train_only=normalize_on_train_only, normalize_x=normalize_x, remove_outliers=remove_outliers))
    steps.append(ValidFeatureEncoder(num_features=num_features, nan_normalize=normalize_by_used_features))
    if prompt_quantile_ple_bins:
        steps.append(PromptQuantilePLEEncoder(prompt_quantile_ple_bins))
    return nn.Sequential(*steps)
