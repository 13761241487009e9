"""Query-row -> context attention over the cached K/V, on libnori_hip.so.

Mirrors the cached-attention half of ``MultiheadAttention`` in the reference
(src/synthefy_nori/model/layer.py):

* ``compute_attention_by_torch``'s dense path over a ``{"kv"}`` dict or a
  ``ScalableSeqKV`` (layer.py:936-1049, fed by forward_with_kv_cache :707-730);
* ``compute_attention_blockwise`` over a ``BlockwiseSeqKV``: one launch over the whole
  resident int8 payload, or one launch per host-streamed block merged by the exact LSE
  rule of layer.py:914-920 (CPU scan :777-839, GPU flex scan :841-934).

Queries are ``[BG, Q, H, D]`` (the layout ``forward_with_kv_cache`` builds at
layer.py:703-706) and caches ``[BG, N, 2, Hkv, D]``. The default logit scale is
1/sqrt(D), as SDPA and the blockwise paths use (layer.py:798, 857).
"""

from __future__ import annotations

import ctypes
import math

import torch

from . import _native as nat
from .kv_cache_scaling import BlockwiseSeqKV, ScalableSeqKV


def _kv_strides(kv: torch.Tensor) -> tuple[int, int, int]:
    """(bg, row, half) element strides of a [BG, N, 2, Hkv, D] tensor whose heads are packed."""
    return kv.stride(0), kv.stride(1), kv.stride(2)


def _packed_heads(kv: torch.Tensor) -> bool:
    d = kv.shape[-1]
    return kv.stride(-1) == 1 and (kv.shape[3] == 1 or kv.stride(3) == d)


def workspace_bytes(bg: int, nq: int, heads: int, d: int, nk: int) -> int:
    return int(nat.lib().nori_icl_attention_workspace_size(bg, nq, heads, d, nk))


def takes_prologue(bg: int, nq: int, heads: int, d: int, nk: int, kv_dtype: torch.dtype, key_norm: bool,
                   q_dtype: torch.dtype = torch.float16) -> bool:
    """Whether ``icl_attention(..., qk_prologue=...)`` runs for these sizes: on the short-context
    kernel (few queries over few keys) and on resident-context launches (fp16 queries, up to 256
    keys read by many queries; a key norm there needs an fp16 cache) -- the launch planner's
    answer (``nori_icl_attention_takes_prologue``)."""
    return bool(nat.lib().nori_icl_attention_takes_prologue(bg, nq, heads, d, nk, nat.dtype_code(kv_dtype),
                                                            1 if key_norm else 0, nat.dtype_code(q_dtype)))


def short_context(nq: int, nk: int) -> bool:
    """Whether the attention runs on the short-context kernel: few queries over few keys (the
    planner's rule, short_context() in csrc/icl_attention_kernel.h)."""
    return nq <= 64 and nk <= 128 and nq * nk <= 2048


def icl_attention(
    q: torch.Tensor,
    kv: torch.Tensor,
    kv_scales: torch.Tensor | None = None,
    *,
    scale: float | None = None,
    out: torch.Tensor | None = None,
    lse: torch.Tensor | None = None,
    merge: bool = False,
    workspace: torch.Tensor | None = None,
    qk_prologue: dict | None = None,
) -> torch.Tensor:
    """softmax(scale * q k^T) v for every (bg, query, head); returns ``out`` ([BG, Q, H, D]).

    kv: int8 codes [BG, N, 2, Hkv, D] with ``kv_scales`` [BG, N, 2, Hkv, 1] fp32, or a
    float16/bfloat16/float32 cache of the same shape (``kv_scales`` None).
    lse: optional fp32 [BG, H, Q] natural-log LSE output.
    merge: treat ``out`` (fp32) and ``lse`` as a running output/LSE of earlier key
    blocks and fold this block in (layer.py:915-920).
    workspace: optional uint8 device buffer of at least ``workspace_bytes(...)`` bytes for
    the split-context partials; allocated per call when omitted.
    qk_prologue: ``{"q_weight", "k_weight", "eps", "q_mult"}`` -- per-head RMS norms of the
    raw q and K rows (gains of d elements, or None) and a multiply of the normed q, applied
    as the kernel loads them, rounded as the separate passes round them
    (``nori_icl_attention_qk``). Only where ``takes_prologue`` says so (short-context shapes
    with full-precision caches, resident-context launches); the library refuses it elsewhere.
    """
    if q.dim() != 4:
        raise ValueError(f"query must be [BG, Q, H, D], got {tuple(q.shape)}")
    if kv.dim() != 5 or kv.shape[2] != 2:
        raise ValueError(f"streamed K/V block must be [BG, K, 2, Hkv, D], got {tuple(kv.shape)}")
    bg, nq, heads, d = q.shape
    if kv.shape[0] != bg:
        raise ValueError(f"K/V batch {kv.shape[0]} does not match query batch {bg}")
    if kv.shape[-1] != d:
        raise ValueError(f"streamed K/V head width must match query head width {d}, got {kv.shape[-1]}")
    kv_heads = kv.shape[3]
    if heads % kv_heads:
        raise ValueError(f"query heads {heads} cannot attend to {kv_heads} K/V heads")
    nk = kv.shape[1]
    if nk == 0:
        raise ValueError("empty K/V cache")
    device = nat.require_device(q, kv, kv_scales, out, lse)
    if kv.dtype == torch.int8:
        if kv_scales is None:
            raise ValueError("int8 cache without scales")
        if tuple(kv_scales.shape) != tuple(kv.shape[:-1]) + (1,):
            raise ValueError(f"scales {tuple(kv_scales.shape)} do not match codes {tuple(kv.shape)}")
        if kv_scales.dtype != torch.float32:
            kv_scales = kv_scales.float()
    if q.stride(-1) != 1:
        q = q.contiguous()
    if not _packed_heads(kv) or (kv.dtype == torch.int8 and any(s % 4 for s in _kv_strides(kv))):
        kv = kv.contiguous()
    if kv_scales is not None and (kv_scales.shape[3] > 1 and kv_scales.stride(3) != 1):
        kv_scales = kv_scales.contiguous()
    if out is None:
        out = torch.empty(q.shape, dtype=torch.float32 if merge else q.dtype, device=device)
    elif tuple(out.shape) != tuple(q.shape) or out.stride(-1) != 1:
        raise ValueError(f"out must be a [BG, Q, H, D] tensor with a contiguous last axis, got {tuple(out.shape)}")
    if merge and (out.dtype != torch.float32 or lse is None):
        raise ValueError("merging needs an fp32 running output and an LSE tensor")
    if lse is not None and (tuple(lse.shape) != (bg, heads, nq) or not lse.is_contiguous() or lse.dtype != torch.float32):
        raise ValueError(f"lse must be a contiguous fp32 [BG, H, Q] tensor, got {tuple(lse.shape)}")
    if scale is None:
        scale = 1.0 / math.sqrt(float(d))
    ws_bytes = workspace_bytes(bg, nq, heads, d, nk)
    if workspace is None or workspace.numel() < ws_bytes:
        workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=device) if ws_bytes > 0 else None
    elif workspace.device != device or workspace.dtype != torch.uint8 or not workspace.is_contiguous():
        raise ValueError("workspace must be a contiguous uint8 tensor on the query's device")
    kvb, kvr, kvh = _kv_strides(kv)
    scb = scr = sch = 0
    if kv_scales is not None:
        scb, scr, sch = kv_scales.stride(0), kv_scales.stride(1), kv_scales.stride(2)
    common = (
        q.data_ptr(), nat.dtype_code(q.dtype), bg, nq, heads, d, q.stride(0), q.stride(1), q.stride(2),
        kv.data_ptr(), nat.dtype_code(kv.dtype), nat.ptr(kv_scales), nk, kv_heads, kvb, kvr, kvh, scb, scr, sch,
        float(scale),
        out.data_ptr(), nat.dtype_code(out.dtype), out.stride(0), out.stride(1), out.stride(2),
        nat.ptr(lse), nat.ATTN_MERGE if merge else 0, nat.ptr(workspace), ws_bytes,
    )
    if qk_prologue is None:
        nat.check(nat.lib().nori_icl_attention(*common, nat.stream_of(device)), "icl_attention")
        return out
    gains = [qk_prologue.get("q_weight"), qk_prologue.get("k_weight")]
    gains = [None if g is None else g.reshape(d).contiguous() for g in gains]
    present = [g for g in gains if g is not None]
    nat.require_device(q, *present)
    if len({g.dtype for g in present}) > 1:
        gains = [None if g is None else g.float() for g in gains]
        present = [g for g in gains if g is not None]
    pro = nat.QKPrologue(
        nat.ptr(gains[0]), nat.ptr(gains[1]), nat.dtype_code(present[0].dtype) if present else nat.NORI_F32,
        float(qk_prologue.get("eps", 0.0)), float(qk_prologue.get("q_mult", 1.0)),
    )
    nat.check(
        nat.lib().nori_icl_attention_qk(*common, ctypes.addressof(pro), nat.stream_of(device)), "icl_attention_qk"
    )
    return out


def attend_dense(q: torch.Tensor, kv_cache, *, scale: float | None = None) -> torch.Tensor:
    """Dense cached attention over a ``{"kv"}`` dict or ``ScalableSeqKV`` (layer.py:707-730, 936-1049).

    An int8 ``ScalableSeqKV`` is consumed as codes + scales; nothing is dequantized in HBM.
    """
    if isinstance(kv_cache, BlockwiseSeqKV):
        return compute_attention_blockwise(q, kv_cache, sdpa_scale=scale)
    if isinstance(kv_cache, ScalableSeqKV):
        payload, scales = kv_cache.device_payload()
        return icl_attention(q, payload, scales, scale=scale)
    return icl_attention(q, kv_cache["kv"], scale=scale)


def compute_attention_blockwise(q: torch.Tensor, kv_cache: BlockwiseSeqKV, *, sdpa_scale: float | None = None) -> torch.Tensor:
    """Exact-context attention over a ``BlockwiseSeqKV`` (layer.py:747-934). Returns [BG, Q, H, D] in q.dtype."""
    if kv_cache.device != q.device:
        raise RuntimeError(
            "streamed K/V cache device does not match the query/model device: "
            f"cache={kv_cache.device}, query={q.device}; rebuild the context cache"
        )
    batch_groups, n_query, n_heads, head_dim = q.shape
    scale = (1.0 / math.sqrt(float(head_dim))) if sdpa_scale is None else sdpa_scale
    resident = kv_cache.resident_payload()
    if resident is not None:
        payload, scales = resident
        return icl_attention(q, payload, scales, scale=scale)
    running_output = torch.zeros((batch_groups, n_query, n_heads, head_dim), dtype=torch.float32, device=q.device)
    running_lse = torch.full((batch_groups, n_heads, n_query), float("-inf"), dtype=torch.float32, device=q.device)
    if kv_cache.offloaded:
        _streamed_scan(q, kv_cache, scale, running_output, running_lse)
    else:
        # device-resident blocks in separate allocations: merged launch by launch, nothing staged
        kv_cache.max_staged_rows = 0
        for payload, scales in kv_cache.device_blocks():
            icl_attention(q, payload, scales, scale=scale, out=running_output, lse=running_lse, merge=True)
    return running_output.to(q.dtype)


_COPY_STREAMS: dict[int, torch.cuda.Stream] = {}


def _copy_stream(device: torch.device) -> torch.cuda.Stream:
    """One host-to-device staging stream per device, at the default priority."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if idx not in _COPY_STREAMS:
        _COPY_STREAMS[idx] = torch.cuda.Stream(device=device)
    return _COPY_STREAMS[idx]


def _streamed_scan(q, kv_cache: BlockwiseSeqKV, scale: float, running_output, running_lse) -> None:
    """Scan the host blocks of an offloaded cache with the copy of block i+1 overlapping the
    attention over block i (layer.py:841-934 stages and computes each block in turn).

    Blocks are copied on a staging stream into two device slots sized for the largest block;
    the compute stream waits for a block's copy, and the staging stream waits for the compute
    on a slot before overwriting it. Host blocks built from device slices are pinned, so the
    copies run asynchronously; from pageable memory they are synchronous and merely correct.
    """
    device = q.device
    compute = torch.cuda.current_stream(device)
    copier = _copy_stream(device)
    blocks = kv_cache.host_blocks()
    kv_cache.max_staged_rows = 0
    if not blocks:
        return
    batch_groups = q.shape[0]
    first_payload, first_scale = blocks[0]
    row_elems = math.prod(first_payload.shape[2:])
    cap = batch_groups * kv_cache.max_block_rows * row_elems
    slots = [torch.empty(cap, dtype=first_payload.dtype, device=device) for _ in range(2)]
    scale_slots = None
    if first_scale is not None:
        scale_cap = batch_groups * kv_cache.max_block_rows * math.prod(first_scale.shape[2:])
        scale_slots = [torch.empty(scale_cap, dtype=torch.float32, device=device) for _ in range(2)]
    for t in slots + (scale_slots or []):
        t.record_stream(copier)  # used on the staging stream as well
    released: list[torch.cuda.Event | None] = [None, None]
    copier.wait_stream(compute)  # queries, outputs and slots exist before the first copy
    for i, (payload, stored_scale) in enumerate(blocks):
        if payload.ndim != 5 or payload.shape[0] != batch_groups:
            raise ValueError(f"streamed K/V block must be [BG, K, 2, Hkv, D], got {tuple(payload.shape)}")
        j = i % 2
        with torch.cuda.stream(copier):
            if released[j] is not None:
                copier.wait_event(released[j])
            staged = slots[j][: payload.numel()].view(payload.shape)
            staged.copy_(payload, non_blocking=True)
            staged_scale = None
            if stored_scale is not None:
                staged_scale = scale_slots[j][: stored_scale.numel()].view(stored_scale.shape)
                staged_scale.copy_(stored_scale, non_blocking=True)
            ready = torch.cuda.Event()
            ready.record(copier)
        compute.wait_event(ready)
        kv_cache.max_staged_rows = max(kv_cache.max_staged_rows, int(payload.shape[1]))
        icl_attention(q, staged, staged_scale, scale=scale, out=running_output, lse=running_lse, merge=True)
        done = torch.cuda.Event()
        done.record(compute)
        released[j] = done
