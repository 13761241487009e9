"""The two-phase encoder of Nori 1.5 ("Model v3", src/synthefy_nori/model/two_phase.py), planned
around the HIP kernels.

What it computes is the reference's: a cell phase (per cell layer: column attention of each
cell over its column's context cells; a context-only row attention of each row's target
stream; SwiGLU MLPs for cells and targets; a decoupled feature attention inside each row),
the boundary (target tokens flattened into one row vector, context labels embedded into it
again, final cell states projected into a read-back memory), then a row phase (context-only
row attention, a read-back from the row's own cells, a SwiGLU MLP). Every update is a
deep-norm residual ``x + alpha * u`` with alpha = (cell layers + row layers)^-1/2; every
attention has per-head q/k RMS norms and QASS "log_only". Module and parameter names are the
reference's state-dict keys, so its checkpoints load with ``strict=True``.

How it is laid out here:

* Two fp32 residual streams per batch of tables, the cells ``[B, R, G, C]`` and the target
  stream ``[B, R, K, C]`` (whose ``[B, R, K * C]`` view is the row vector of the row phase),
  updated in place by the fused residual kernel (``nori_residual_add``: one pass, torch's
  rounding of ``x + alpha * u``).
* Every RMS norm that feeds a projection writes the projection's operand dtype directly.
* The decoupled feature attention is one GEMM: the per-token norms of cells and targets
  write one ``[B, R, G + K, C]`` operand buffer, and the q/k/v weights of both of its
  attentions are stacked, so the operand is read once. Each attention then reads its q and
  K/V as strided views of that projection -- the cell queries attend to every token, the
  target queries to the cells -- with its q/k norms and log-n factor applied as the
  short-context kernel loads the rows.
* The MLPs are ``SwiGLUMLP``: one stacked gate/up GEMM, the HIP SwiGLU gate, the down GEMM.
* Column and row attentions over the context rows run on the MFMA attention kernel.
"""

from __future__ import annotations

import torch
from torch import nn

from .layer import MultiheadAttention, SwiGLUMLP
from .norm import RMSNorm, operand_dtype, projection_operand, residual_add, residual_add_norm, swiglu_mlp_residual_norm
from .projection import linear as proj_linear
from .projection import linear_residual_norm, takes_kernel

__all__ = [
    "CellLayer2P",
    "DecoupledFeatureAttention",
    "FullColumnAttention",
    "RowLayer2P",
    "TargetStreamEncoder",
    "TwoPhaseEncoder",
]


def _icl_attention_module(width: int, heads: int, device, dtype, cudnn_hint: bool = False) -> MultiheadAttention:
    """The attention every sublayer of the encoder uses (two_phase.py:34-50): separate Q/KV
    projections, per-head q/k RMS norms, QASS "log_only"."""
    return MultiheadAttention(
        embed_dim=width, num_heads=heads, qkv_combined=False, dropout=0.0, use_qassmax=True, qass_mode="log_only",
        device=device, dtype=dtype, qk_norm=True, reuse_projected_kv_storage=True, prefer_cudnn_inference=cudnn_hint,
    )


def _plain_norm(width: int, eps: float) -> RMSNorm:
    return RMSNorm(width, eps=eps, elementwise_affine=False)


def _accumulate(stream: torch.Tensor, update: torch.Tensor, alpha: float, then: RMSNorm | None = None, *,
                operand: bool = True, out: torch.Tensor | None = None) -> torch.Tensor | None:
    """stream += alpha * update (deep-norm residual), in place. With ``then``, also returns the
    next sublayer's normalized stream -- ``projection_operand(then, stream)`` when ``operand``,
    else ``then(stream)`` -- formed in the same pass (``residual_add_norm``), or writes it into
    ``out``."""
    if then is None:
        residual_add(stream, update.reshape(stream.shape), alpha, inplace=True)
        return None
    dt = operand_dtype(stream) if operand else stream.dtype
    return residual_add_norm(stream, update.reshape(stream.shape), alpha, then, out_dtype=dt, out=out)


def _linear_accumulate(a: torch.Tensor, weight: torch.Tensor, stream: torch.Tensor, alpha: float, then: RMSNorm | None,
                       project, *, operand: bool = True, out: torch.Tensor | None = None) -> torch.Tensor | None:
    """``_accumulate(stream, project(), alpha, then, ...)`` where ``project()`` is ``F.linear(a,
    weight)`` under fp16 autocast: ``a`` [..., K] with ``stream``'s leading shape (any row
    strides), ``weight`` [K, K] in the projection dtype. When the next norm is formed in the
    fp16 operand dtype, the projection, the residual update and the norm run as one kernel
    (``linear_residual_norm``: u never reaches memory) wherever it takes the operands."""
    if (then is not None and operand and a.is_cuda and then.weight is None
            and tuple(then.normalized_shape) == (int(stream.shape[-1]),)
            and operand_dtype(stream) == torch.float16 and weight.dtype == torch.float16):
        y = linear_residual_norm(a, weight, stream, alpha, then.eps, out=out)
        if y is not None:
            return y
    return _accumulate(stream, project(), alpha, then, operand=operand, out=out)


def _attend_accumulate(attn: MultiheadAttention, atten: torch.Tensor, stream: torch.Tensor, alpha: float,
                       then: RMSNorm | None = None, *, operand: bool = True) -> torch.Tensor | None:
    """``stream += alpha * attn.project_out(atten)`` (then the next norm, as ``_accumulate``):
    ``atten`` the attention output [..., H, D] with ``stream``'s leading shape, any row strides."""
    a = atten.reshape(*atten.shape[:-2], -1)
    w_o = attn._linear_weights(atten.device)[2] if atten.is_cuda else None
    if w_o is None:
        return _accumulate(stream, attn.project_out(atten), alpha, then, operand=operand)
    return _linear_accumulate(a, w_o, stream, alpha, then, lambda: attn.project_out(atten), operand=operand)


def _mlp_accumulate(mlp: SwiGLUMLP, x: torch.Tensor, stream: torch.Tensor, alpha: float, then: RMSNorm | None,
                    *, operand: bool = True, out: torch.Tensor | None = None) -> torch.Tensor | None:
    """``_accumulate(stream, mlp(x), alpha, then, ...)``: with the next norm formed in the fp16
    operand dtype, the fused SwiGLU kernel applies the residual update and the norm itself
    (``swiglu_mlp_residual_norm``: the MLP output never reaches memory) wherever it takes the
    operands. ``stream`` holds x's rows (its last axis the norm's width)."""
    if (then is not None and operand and x.is_cuda and then.weight is None and mlp.fuses(x)
            and tuple(then.normalized_shape) == (int(stream.shape[-1]),)
            and operand_dtype(stream) == torch.float16):
        gate_up, _, down, hidden = mlp._stacked_weights(x, multiple=32)
        y = swiglu_mlp_residual_norm(x.to(torch.float16), gate_up, down, hidden, stream, alpha, then.eps,
                                     int(stream.shape[-1]), out=out)
        if y is not None:
            return y
    return _accumulate(stream, mlp(x), alpha, then, operand=operand, out=out)


def _row_vectors(targets: torch.Tensor) -> torch.Tensor:
    """The [batch, n, K * width] row-vector view of a target stream [batch, n, K, width] (a view:
    updates through it land in the stream)."""
    return targets.view(*targets.shape[:2], -1)


def _put(dst: torch.Tensor, src: torch.Tensor) -> None:
    """dst[...] = src, skipped when src already is dst's memory (a chunk worked on in place)."""
    if src.data_ptr() != dst.data_ptr() or src.device != dst.device or src.stride() != dst.stride():
        dst.copy_(src)


def _over_keys(attn: MultiheadAttention, queries: torch.Tensor, keys: torch.Tensor) -> torch.Tensor:
    """``queries`` [batch, groups, n, width] attend over the third axis of ``keys``
    [batch, groups, m, width]; the output projection is applied (two_phase.py:53-55)."""
    return attn(x=queries, x_kv=keys, copy_first_head_kv=False)[0]


class TargetStreamEncoder(nn.Module):
    """The K target tokens of each row from its label (two_phase.py:58-107): a GELU MLP of the
    value for regression or a class embedding; rows whose label is not finite (the query rows)
    take the learned query vector. ``y`` [batch, rows] -> [batch, rows, K, cell_dim]."""

    def __init__(self, cell_dim: int, target_tokens: int, *, task_type: str, max_num_classes: int, device=None,
                 dtype=None):
        super().__init__()
        self.cell_dim, self.target_tokens, self.task_type = int(cell_dim), int(target_tokens), task_type
        self.width = width = self.cell_dim * self.target_tokens
        self.mlp = None
        self.class_embedding = None
        if task_type == "reg":
            self.mlp = nn.Sequential(nn.Linear(1, width // 2, device=device, dtype=dtype), nn.GELU(),
                                     nn.Linear(width // 2, width, device=device, dtype=dtype))
        if task_type == "cls":
            self.class_embedding = nn.Embedding(max_num_classes, width, device=device, dtype=dtype)
        self.query_embedding = nn.Parameter(torch.empty(width, device=device, dtype=dtype))
        nn.init.normal_(self.query_embedding, std=0.02)

    def forward(self, y: torch.Tensor) -> torch.Tensor:
        known = torch.isfinite(y)
        label = y.masked_fill(~known, 0.0)
        if self.mlp is not None:
            tokens = self.mlp(label[..., None].to(self.mlp[0].weight.dtype))
        else:
            n_classes = self.class_embedding.num_embeddings
            tokens = self.class_embedding(label.long().clamp(0, n_classes - 1))
        tokens = torch.where(known[..., None], tokens, self.query_embedding.to(tokens.dtype))
        return tokens.unflatten(-1, (self.target_tokens, self.cell_dim))


class FullColumnAttention(nn.Module):
    """Holds the column attention (two_phase.py:110-119): a cell attends to the context cells of
    its column. ``forward`` takes the normalized cells [batch, rows, groups, width]."""

    def __init__(self, cell_dim: int, heads: int, *, device, dtype):
        super().__init__()
        self.sequence_attentions = nn.ModuleList([_icl_attention_module(cell_dim, heads, device, dtype, cudnn_hint=True)])

    def forward(self, normed_cells: torch.Tensor, eval_pos: int) -> torch.Tensor:
        columns = normed_cells.transpose(1, 2)  # [batch, groups, rows, width]
        return _over_keys(self.sequence_attentions[0], columns, columns[:, :, :eval_pos]).transpose(1, 2)

    def attend(self, normed_cells: torch.Tensor, eval_pos: int) -> torch.Tensor:
        """``forward`` before the output projection: the attention output [batch, rows, groups,
        H, D] as a view of the [batch, groups, rows] result (rows in the cells' order)."""
        b, n, g, _ = normed_cells.shape
        attn = self.sequence_attentions[0]
        columns = normed_cells.transpose(1, 2)
        out = attn.attend(columns, columns[:, :, :eval_pos])  # [batch * groups, rows, H, D]
        return out.view(b, g, n, attn.num_heads, attn.head_dim).transpose(1, 2)


class DecoupledFeatureAttention(nn.Module):
    """Holds the feature attention inside a row (two_phase.py:122-138): attention 0 lets the
    cells read every token of the row, attention 1 lets the target tokens read the cells, and
    ``target_mix`` mixes the K target read-outs. The stacked projection of both is built by
    ``stacked_weight``; ``forward`` takes the normalized [cells | targets] token buffer."""

    def __init__(self, cell_dim: int, heads: int, target_tokens: int, *, device, dtype):
        super().__init__()
        self.target_tokens = int(target_tokens)
        self.feature_attentions = nn.ModuleList([_icl_attention_module(cell_dim, heads, device, dtype) for _ in range(2)])
        width = cell_dim * self.target_tokens
        self.target_mix = nn.Linear(width, width, bias=False, device=device, dtype=dtype)
        nn.init.normal_(self.target_mix.weight, std=0.02)

    def stacked_weight(self, dtype: torch.dtype, device) -> torch.Tensor:
        """[k0; v0; q0; k1; v1; q1] projection weight [6 * H * D, width] in ``dtype`` (attention 0
        reads the K/V of every token and the queries of the cells, attention 1 the K/V of the
        cells and the queries of the target tokens: in this order each token's projections are
        one or two contiguous row ranges), cached until a weight changes."""
        parts = [m.qkv_proj_weight for m in self.feature_attentions]
        key = (dtype, device) + tuple((p.data_ptr(), p._version) for p in parts)
        cached = getattr(self, "_stacked", None)
        if cached is None or cached[0] != key:
            with torch.no_grad():
                w = torch.cat([torch.cat([p[1], p[2], p[0]]).reshape(-1, p.shape[-1]) for p in parts])
                w = w.to(device=device, dtype=dtype)
            cached = self._stacked = (key, w)
        return cached[1]

    def forward(self, tokens: torch.Tensor, n_cells: int) -> tuple[torch.Tensor, torch.Tensor]:
        """``tokens`` [batch, rows, groups + K, width]: the normalized cells, then the normalized
        target tokens of each row. Returns (cell update [batch, rows, groups, width], target
        update [batch, rows, K, width])."""
        b, r, _, width = tokens.shape
        cell_out, readout = self.attend(tokens, n_cells)
        cells_out = self.feature_attentions[0].project_out(cell_out)
        return cells_out, self.target_mix(readout).view(b, r, self.target_tokens, width)

    def mix_weight(self, dtype: torch.dtype, device) -> torch.Tensor:
        """``target_mix``'s weight in ``dtype`` (the projection dtype), cached until it changes."""
        p = self.target_mix.weight
        key = (dtype, device, p.data_ptr(), p._version)
        cached = getattr(self, "_mix", None)
        if cached is None or cached[0] != key:
            with torch.no_grad():
                cached = self._mix = (key, p.to(device=device, dtype=dtype).contiguous())
        return cached[1]

    def attend(self, tokens: torch.Tensor, n_cells: int) -> tuple[torch.Tensor, torch.Tensor]:
        """``forward`` before the cells' output projection and ``target_mix``: (the cell
        attention's output [batch, rows, groups, H, D], the target read-out [batch, rows,
        K * width] that ``target_mix`` takes)."""
        b, r, t, width = tokens.shape
        a0, a1 = self.feature_attentions
        h, d = a0.num_heads, a0.head_dim
        hd = h * d
        flat = tokens.reshape(b * r, t, width)
        w = self.stacked_weight(tokens.dtype, tokens.device)
        cells, targets = flat[:, :n_cells], flat[:, n_cells:]
        if takes_kernel(cells, w, any_width=True) and takes_kernel(targets, w, any_width=True):
            # only the projections each token's attentions read, into one buffer (slots
            # [k0 v0 q0 k1 v1 q1] per token; the others stay unwritten): the cells' k0 v0 q0 k1
            # v1, the target tokens' k0 v0 and q1 -- 28 % fewer outputs than projecting every
            # token through all six
            proj = torch.empty((b * r, t, 6 * hd), dtype=tokens.dtype, device=tokens.device)
            proj_linear(cells, w[: 5 * hd], out=proj[:, :n_cells, : 5 * hd], any_width=True)
            proj_linear(targets, w[: 2 * hd], out=proj[:, n_cells:, : 2 * hd], any_width=True)
            proj_linear(targets, w[5 * hd:], out=proj[:, n_cells:, 5 * hd:], any_width=True)
        else:
            proj = torch.nn.functional.linear(flat, w)
        proj = proj.view(b * r, t, 6, h, d)     # [row, token, k0 v0 q0 k1 v1 q1, head, d]
        cell_q = proj[:, :n_cells, 2]
        all_kv = proj[:, :, 0:2]                # every token of the row: K then V
        target_q = proj[:, n_cells:, 5]
        cell_kv = proj[:, :n_cells, 3:5]        # the cells only
        cell_out = a0.attend_projected(cell_q, all_kv).view(b, r, n_cells, h, d)
        readout = a1.project_out(a1.attend_projected(target_q, cell_kv))
        return cell_out, readout.reshape(b, r, -1)


class CellLayer2P(nn.Module):
    """A cell-phase layer (two_phase.py:141-232). Norms: ``cell_norms`` (column attention, MLP,
    feature attention) over a cell, ``target_norms`` (row attention and MLP over the row vector
    of K target tokens, feature attention over one token); all without gains. Its steps take the
    two residual streams and update them in place; ``forward`` runs them in order."""

    def __init__(self, cell_dim: int, heads: int, hidden_dim: int, *, target_tokens: int, target_heads: int,
                 target_hidden_dim: int, deepnorm_alpha: float, layer_norm_eps: float = 1e-5, device=None, dtype=None):
        super().__init__()
        self.cell_dim, self.target_tokens = int(cell_dim), int(target_tokens)
        self.target_width = self.cell_dim * self.target_tokens
        self.deepnorm_alpha = float(deepnorm_alpha)
        eps = layer_norm_eps
        self.cell_norms = nn.ModuleList([_plain_norm(self.cell_dim, eps) for _ in range(3)])
        self.target_norms = nn.ModuleList(
            [_plain_norm(self.target_width, eps), _plain_norm(self.target_width, eps), _plain_norm(self.cell_dim, eps)]
        )
        self.column_attention = FullColumnAttention(self.cell_dim, heads, device=device, dtype=dtype)
        self.sequence_attentions = nn.ModuleList([_icl_attention_module(self.target_width, target_heads, device, dtype)])
        self.mlp = nn.ModuleList([
            SwiGLUMLP(self.cell_dim, hidden_dim, self.cell_dim, has_bias=False, device=device, dtype=dtype),
            SwiGLUMLP(self.target_width, target_hidden_dim, self.target_width, has_bias=False, device=device, dtype=dtype),
        ])
        self.feature_attention = DecoupledFeatureAttention(self.cell_dim, heads, self.target_tokens, device=device,
                                                           dtype=dtype)

    def forward(self, cells: torch.Tensor, targets: torch.Tensor, eval_pos: int) -> tuple[torch.Tensor, torch.Tensor]:
        """Out-of-place form: returns the updated (cells, targets); the inputs are left as they are."""
        cells, targets = cells.clone(), targets.contiguous().clone()
        cell_op = self.column_step(cells, eval_pos, then=True)
        rows = _row_vectors(targets)
        row_op = self.target_row_step(rows, self.row_operand(rows), eval_pos, then=True)
        self.row_local_steps(cells, targets, cell_op, row_op)
        return cells, targets

    # --- steps on the streams (in place). Each step may take its normalized input, and with
    # ``then`` returns the normalized input of the step after it from the same pass as its
    # residual update (so a stream is not read again for the next norm).
    def column_step(self, cells: torch.Tensor, eval_pos: int, normed: torch.Tensor | None = None,
                    then: bool = False) -> torch.Tensor | None:
        """Each cell reads its column's context cells. Reads whole columns: a slice of the
        groups axis may be passed. ``normed``: the cells through ``cell_norms[0]``; ``then``:
        return the cells through ``cell_norms[1]`` (the cell MLP's operand)."""
        if normed is None:
            normed = projection_operand(self.cell_norms[0], cells)
        atten = self.column_attention.attend(normed, eval_pos)
        del normed
        return _attend_accumulate(self.column_attention.sequence_attentions[0], atten, cells, self.deepnorm_alpha,
                                  self.cell_norms[1] if then else None)

    def row_operand(self, rows: torch.Tensor) -> torch.Tensor:
        """The normalized row vectors the target-stream row attention reads, [batch, 1, n, width]."""
        return projection_operand(self.target_norms[0], rows).unsqueeze(1)

    def target_row_step(self, rows: torch.Tensor, normed: torch.Tensor, eval_pos: int | None = None,
                        context: torch.Tensor | None = None, then: bool = False) -> torch.Tensor | None:
        """The row vectors ``rows`` [batch, n, width] (normalized: ``normed``) read the context
        rows' normalized vectors: ``context``, or the first ``eval_pos`` of ``normed``. ``then``:
        return the rows through ``target_norms[1]`` (the target MLP's operand)."""
        keys = normed[:, :, :eval_pos] if context is None else context
        attn = self.sequence_attentions[0]
        atten = attn.attend(normed, keys).view(*rows.shape[:-1], attn.num_heads, attn.head_dim)
        return _attend_accumulate(attn, atten, rows, self.deepnorm_alpha, self.target_norms[1] if then else None)

    def row_local_steps(self, cells: torch.Tensor, targets: torch.Tensor, cell_operand: torch.Tensor | None = None,
                        row_operand: torch.Tensor | None = None,
                        then: tuple[RMSNorm | None, RMSNorm | None, bool] | None = None):
        """The MLPs, then the feature attention: each row reads only itself, so any slice of rows
        may be passed. ``targets`` [batch, n, K, width] (its row-vector view is what the target
        MLP transforms). ``cell_operand`` / ``row_operand``: the MLPs' normalized inputs.
        ``then`` = (cell norm, target-row norm, operand): return the streams through those norms
        (in the projection dtype when ``operand``), from the feature attention's update passes."""
        alpha = self.deepnorm_alpha
        rows = _row_vectors(targets)
        if cell_operand is None:
            cell_operand = projection_operand(self.cell_norms[1], cells)
        if row_operand is None:
            row_operand = projection_operand(self.target_norms[1], rows)
        # the two MLP updates, each with the feature attention's norm of its stream written
        # token by token into the attention's operand buffer
        b, n, g, w = cells.shape
        tokens = torch.empty((b, n, g + self.target_tokens, w), dtype=operand_dtype(cells), device=cells.device)
        _mlp_accumulate(self.mlp[0], cell_operand, cells, alpha, self.cell_norms[2], out=tokens[:, :, :g])
        del cell_operand
        _mlp_accumulate(self.mlp[1], row_operand, targets, alpha, self.target_norms[2], out=tokens[:, :, g:])
        del row_operand
        fa = self.feature_attention
        cell_out, readout = fa.attend(tokens, g)
        del tokens
        cell_norm, row_norm, operand = (None, None, True) if then is None else then
        cell_next = _attend_accumulate(fa.feature_attentions[0], cell_out, cells, alpha, cell_norm, operand=operand)
        mix = fa.mix_weight(readout.dtype, readout.device) if readout.is_cuda else None
        row_next = _linear_accumulate(readout, mix, rows, alpha, row_norm, lambda: fa.target_mix(readout),
                                      operand=operand) if mix is not None else \
            _accumulate(rows, fa.target_mix(readout), alpha, row_norm, operand=operand)
        return None if then is None else (cell_next, row_next)


class RowLayer2P(nn.Module):
    """A row-phase layer (two_phase.py:235-284): context-only row attention, a read-back of the
    row's own cells, a SwiGLU MLP. Steps update the row stream in place."""

    def __init__(self, width: int, heads: int, hidden_dim: int, *, deepnorm_alpha: float, layer_norm_eps: float = 1e-5,
                 device=None, dtype=None):
        super().__init__()
        self.deepnorm_alpha = float(deepnorm_alpha)
        self.attn_norm = _plain_norm(width, layer_norm_eps)
        self.mlp_norm = _plain_norm(width, layer_norm_eps)
        self.readback_norm = _plain_norm(width, layer_norm_eps)
        self.sequence_attentions = nn.ModuleList([_icl_attention_module(width, heads, device, dtype)])
        self.feature_attentions = nn.ModuleList([_icl_attention_module(width, heads, device, dtype)])
        self.mlp = nn.ModuleList([SwiGLUMLP(width, hidden_dim, width, has_bias=False, device=device, dtype=dtype)])

    def forward(self, rows: torch.Tensor, eval_pos: int, cell_memory: torch.Tensor) -> torch.Tensor:
        """Out-of-place form: returns the updated rows; ``rows`` is left as it is."""
        rows = rows.clone()
        query = self.context_step(rows, self.row_operand(rows), eval_pos, then=True)
        self.readback_steps(rows, cell_memory, query)
        return rows

    def row_operand(self, rows: torch.Tensor) -> torch.Tensor:
        return projection_operand(self.attn_norm, rows).unsqueeze(1)

    def context_step(self, rows: torch.Tensor, normed: torch.Tensor, eval_pos: int | None = None,
                     context: torch.Tensor | None = None, then: bool = False) -> torch.Tensor | None:
        """``rows`` [batch, n, width] (normalized: ``normed``) read the context rows' normalized
        vectors: ``context``, or the first ``eval_pos`` of ``normed``. ``then``: return the rows
        through ``readback_norm`` (the read-back query)."""
        keys = normed[:, :, :eval_pos] if context is None else context
        attn = self.sequence_attentions[0]
        atten = attn.attend(normed, keys).view(*rows.shape[:-1], attn.num_heads, attn.head_dim)
        return _attend_accumulate(attn, atten, rows, self.deepnorm_alpha, self.readback_norm if then else None)

    def readback_steps(self, rows: torch.Tensor, cell_memory: torch.Tensor, query: torch.Tensor | None = None,
                       then: RMSNorm | None = None, operand: bool = True) -> torch.Tensor | None:
        """The row reads its own cells ``cell_memory`` [batch, n, groups, width], then the MLP;
        each row reads only itself. ``query``: the rows through ``readback_norm``; ``then``:
        return the rows through that norm after the MLP's update (in the projection dtype
        when ``operand``)."""
        alpha = self.deepnorm_alpha
        if query is None:
            query = projection_operand(self.readback_norm, rows)
        attn = self.feature_attentions[0]
        atten = attn.attend(query.unsqueeze(2), cell_memory).view(*rows.shape[:-1], attn.num_heads, attn.head_dim)
        del query
        mlp_in = _attend_accumulate(attn, atten, rows, alpha, self.mlp_norm)
        return _mlp_accumulate(self.mlp[0], mlp_in, rows, alpha, then, operand=operand)


class TwoPhaseEncoder(nn.Module):
    """Cell layers, the boundary and row layers of Nori 1.5 (two_phase.py:287-486).

    ``forward`` / ``forward_chunked`` take the embedded cells [batch, rows, groups, cell_dim] and
    the labels [batch, rows] (not finite on query rows) and return the normalized row states
    [batch, rows, K * cell_dim] (``forward`` also the final cell states)."""

    def __init__(self, cell_dim: int, heads: int, hidden_dim: int, *, target_tokens: int, cell_layers: int,
                 row_layers: int, row_heads: int, row_hidden_dim: int, task_type: str, max_num_classes: int,
                 layer_norm_eps: float = 1e-5, device=None, dtype=None):
        super().__init__()
        if cell_layers <= 0 or target_tokens <= 0 or row_heads <= 0 or row_layers < 0:
            raise ValueError("two-phase encoder needs positive cell-layer, token and head counts and row_layers >= 0")
        self.cell_dim, self.target_tokens, self.task_type = int(cell_dim), int(target_tokens), task_type
        self.width = self.cell_dim * self.target_tokens
        if self.width % int(row_heads):
            raise ValueError("two-phase target width (target_tokens * embed_dim) must be divisible by row_heads")
        self.num_cell_layers, self.num_row_layers = int(cell_layers), int(row_layers)
        self.gradient_checkpointing = False
        alpha = (self.num_cell_layers + self.num_row_layers) ** -0.5
        self.deepnorm_alpha = alpha
        self.target_encoder = TargetStreamEncoder(self.cell_dim, self.target_tokens, task_type=task_type,
                                                  max_num_classes=max_num_classes, device=device, dtype=dtype)
        if task_type == "cls":
            self.row_y_encoder = nn.Embedding(max_num_classes, self.width, device=device, dtype=dtype)
        else:
            self.row_y_encoder = nn.Sequential(nn.Linear(1, self.width, device=device, dtype=dtype),
                                               nn.LayerNorm(self.width, device=device, dtype=dtype))
        layers: list[nn.Module] = [
            CellLayer2P(self.cell_dim, heads, hidden_dim, target_tokens=self.target_tokens, target_heads=row_heads,
                        target_hidden_dim=row_hidden_dim, deepnorm_alpha=alpha, layer_norm_eps=layer_norm_eps,
                        device=device, dtype=dtype)
            for _ in range(self.num_cell_layers)
        ]
        self.cell_to_row = nn.Linear(self.cell_dim, self.width, bias=False, device=device, dtype=dtype)
        layers += [
            RowLayer2P(self.width, row_heads, row_hidden_dim, deepnorm_alpha=alpha, layer_norm_eps=layer_norm_eps,
                       device=device, dtype=dtype)
            for _ in range(self.num_row_layers)
        ]
        self.layers = nn.ModuleList(layers)
        self.cell_out_norm = _plain_norm(self.cell_dim, layer_norm_eps)
        self.row_out_norm = _plain_norm(self.width, layer_norm_eps)

    @property
    def cell_layers(self):
        return self.layers[: self.num_cell_layers]

    @property
    def row_layers(self):
        return self.layers[self.num_cell_layers :]

    def label_embedding(self, context_y: torch.Tensor) -> torch.Tensor:
        """What the boundary adds to the context rows' vectors: [batch, n] labels -> [batch, n, width]."""
        labels = torch.nan_to_num(context_y)
        if isinstance(self.row_y_encoder, nn.Embedding):
            return self.row_y_encoder(labels.long().clamp(0, self.row_y_encoder.num_embeddings - 1))
        return self.row_y_encoder(labels[..., None].to(self.row_y_encoder[0].weight.dtype))

    def _require_context(self, eval_pos: int, n_rows: int) -> None:
        if not 0 < eval_pos <= n_rows:
            raise ValueError("two-phase encoder requires a non-empty context prefix")

    def forward(self, cells: torch.Tensor, y: torch.Tensor, eval_pos: int, inplace: bool = False,
                **_: object) -> tuple[torch.Tensor, torch.Tensor]:
        """``inplace``: the cell stream is updated in ``cells`` itself (a caller's own temporary)
        instead of in a copy."""
        self._require_context(eval_pos, cells.shape[1])
        cells = cells if inplace else cells.clone()  # the streams are updated in place
        targets = self.target_encoder(y).to(cells.dtype).contiguous()
        rows = _row_vectors(targets)
        # every residual update hands the next sublayer its normalized stream (one pass)
        cell_layers = list(self.cell_layers)
        col_op = row_op = cell_states = None
        for i, layer in enumerate(cell_layers):
            mlp_op = layer.column_step(cells, eval_pos, normed=col_op, then=True)
            if row_op is None:
                row_op = layer.row_operand(rows)
            tmlp_op = layer.target_row_step(rows, row_op, eval_pos, then=True)
            if i + 1 < len(cell_layers):
                nxt = cell_layers[i + 1]
                col_op, row_op = layer.row_local_steps(cells, targets, mlp_op, tmlp_op,
                                                       then=(nxt.cell_norms[0], nxt.target_norms[0], True))
                row_op = row_op.unsqueeze(1)
            else:
                # the last update of the cells gives the cell states; the rows take the labels next
                cell_states, _ = layer.row_local_steps(cells, targets, mlp_op, tmlp_op,
                                                       then=(self.cell_out_norm, None, False))
        rows[:, :eval_pos] += self.label_embedding(y[:, :eval_pos]).to(rows.dtype)
        if cell_states is None:
            cell_states = self.cell_out_norm(cells)
        memory = self.cell_to_row(cell_states)
        row_layers = list(self.row_layers)
        row_op, out = None, None
        for i, layer in enumerate(row_layers):
            if row_op is None:
                row_op = layer.row_operand(rows)
            query = layer.context_step(rows, row_op, eval_pos, then=True)
            if i + 1 < len(row_layers):
                row_op = layer.readback_steps(rows, memory, query, then=row_layers[i + 1].attn_norm).unsqueeze(1)
            else:
                out = layer.readback_steps(rows, memory, query, then=self.row_out_norm, operand=False)
        return (self.row_out_norm(rows) if out is None else out), cell_states

    @torch.no_grad()
    def forward_chunked(self, cells: torch.Tensor, y: torch.Tensor, eval_pos: int, *, row_chunk: int, column_chunk: int,
                        compute_device: torch.device) -> torch.Tensor:
        """``forward``'s normalized row states without the whole table on ``compute_device``
        (two_phase.py:380-486). ``cells`` lives on its home device (the GPU or host memory) and
        is overwritten; the target stream is kept beside it. Per cell layer the column step runs
        ``column_chunk`` columns at a time; the row attentions take the context rows' normalized
        vectors once per layer and run ``row_chunk`` rows at a time, as do all the row-local
        steps (each chunk projects its own read-back memory). Matches ``forward`` up to the
        reassociation of smaller batches. Returns [batch, rows, width] on the home device."""
        self._require_context(eval_pos, cells.shape[1])
        home = cells.device
        n_batch, n_rows, n_groups, _ = cells.shape
        chunks = [slice(r, min(r + row_chunk, n_rows)) for r in range(0, n_rows, row_chunk)]
        y = y.to(compute_device)
        targets = torch.empty((n_batch, n_rows, self.target_tokens, self.cell_dim), dtype=cells.dtype, device=home)

        def load(t: torch.Tensor) -> torch.Tensor:
            return t.to(compute_device).contiguous()

        for part in chunks:
            targets[:, part] = self.target_encoder(y[:, part]).to(cells.dtype).to(home)
        rows = targets.view(n_batch, n_rows, self.width)

        for layer in self.cell_layers:
            for g0 in range(0, n_groups, column_chunk):
                cols = slice(g0, min(g0 + column_chunk, n_groups))
                block = load(cells[:, :, cols])
                layer.column_step(block, eval_pos)
                _put(cells[:, :, cols], block)
            context = layer.row_operand(load(rows[:, :eval_pos]))  # from the layer's input rows
            for part in chunks:
                c, t = load(cells[:, part]), load(targets[:, part])
                r = _row_vectors(t)
                layer.target_row_step(r, layer.row_operand(r), context=context)
                layer.row_local_steps(c, t)
                _put(cells[:, part], c)
                _put(targets[:, part], t)
            del context

        # the boundary: context labels go into the row vectors; cells become the final states
        for part in chunks:
            n_ctx = min(max(eval_pos - part.start, 0), part.stop - part.start)
            if n_ctx:
                r = load(rows[:, part.start : part.start + n_ctx])
                r += self.label_embedding(y[:, part.start : part.start + n_ctx]).to(r.dtype)
                _put(rows[:, part.start : part.start + n_ctx], r)
            _put(cells[:, part], self.cell_out_norm(load(cells[:, part])))

        for layer in self.row_layers:
            context = layer.row_operand(load(rows[:, :eval_pos]))
            for part in chunks:
                r = load(rows[:, part])
                layer.context_step(r, layer.row_operand(r), context=context)
                layer.readback_steps(r, self.cell_to_row(load(cells[:, part])))
                _put(rows[:, part], r)
            del context

        out = None
        for part in chunks:
            normed = self.row_out_norm(load(rows[:, part]))
            if out is None:
                out = torch.empty((n_batch, n_rows, self.width), dtype=normed.dtype, device=home)
            _put(out[:, part], normed)
        return out
