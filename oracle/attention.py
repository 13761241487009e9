"""CPU oracle for query-row -> context attention over a K/V cache.

TEST INFRASTRUCTURE ONLY: the checker for the HIP attention kernel and the CPU
baseline that ``bench.py`` times. Only tests/, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it.

Three restatements, each citing the reference lines it follows (paths relative to
the reference repo root):

* ``attention_f64`` -- textbook softmax(q k^T * scale) v in float64 numpy, with
  the natural-log LSE, over ``[BG, Q, H, D]`` queries and ``[BG, K, Hkv, D]`` keys;
  query head h reads K/V head ``h // (H // Hkv)`` (layer.py:108-111, the
  ``enable_gqa`` rule of SDPA used at layer.py:956, 1047-1049).
* ``blockwise_attention_fp32`` -- the CPU online-softmax scan of
  ``MultiheadAttention.compute_attention_blockwise`` (layer.py:777-839): fp32
  running max / denominator / numerator over K/V blocks, with the same 256 MiB
  score-workspace row cap (layer.py:21-26, 778-785). This is what the reference
  runs on CPU, so it is the CPU baseline.
* ``lse_merge`` -- the exact fp32 merge of per-block (output, LSE) pairs used by
  the GPU blockwise path (layer.py:914-920).

Pins (tests/test_oracle_attention.py): torch's SDPA on CPU, closed forms (one key,
identical keys, one-hot logits), the LSE-merge identity over ragged splits,
GQA == repeat_interleave, and zero-padding invariance of the head width.
"""

from __future__ import annotations

import math

import numpy as np

BLOCKWISE_SCORE_WORKSPACE_BYTES = 256 * 1024**2  # layer.py:25


def _group(n_heads: int, kv_heads: int) -> int:
    if kv_heads <= 0 or n_heads % kv_heads:
        raise ValueError(f"query heads {n_heads} cannot attend to {kv_heads} K/V heads")
    return n_heads // kv_heads


def attention_f64(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float | None = None):
    """q [BG,Q,H,D], k/v [BG,K,Hkv,D] -> (out [BG,Q,H,D] float64, lse [BG,H,Q] float64)."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    bg, nq, h, d = q.shape
    hkv = k.shape[2]
    rep = _group(h, hkv)
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    kx = np.repeat(k, rep, axis=2)  # head h -> kv head h // rep
    vx = np.repeat(v, rep, axis=2)
    logits = np.einsum("bqhd,bkhd->bhqk", q, kx) * scale
    mx = logits.max(axis=-1, keepdims=True)
    w = np.exp(logits - mx)
    den = w.sum(axis=-1, keepdims=True)
    out = np.einsum("bhqk,bkhd->bqhd", w / den, vx)
    lse = (np.log(den) + mx)[..., 0]
    return out, lse


def lse_merge(out_a, lse_a, out_b, lse_b):
    """Merge two normalized partial attentions (layer.py:915-920).

    out_*: [BG,H,Q,D], lse_*: [BG,H,Q] (natural log). Works for numpy or torch inputs.
    """
    new = np.logaddexp(lse_a, lse_b)
    wa = np.exp(lse_a - new)[..., None]
    wb = np.exp(lse_b - new)[..., None]
    return out_a * wa + out_b * wb, new


def blockwise_attention_fp32(q, kv_blocks, scale: float | None = None):
    """fp32 online softmax over K/V blocks, as run on CPU by the reference (layer.py:777-839).

    q: torch tensor [BG,Q,H,D]; kv_blocks: iterable of torch tensors [BG,Kb,2,Hkv,D].
    Returns torch [BG,Q,H,D] in q's dtype. Each stored block is re-sliced to the
    score-workspace row cap exactly like ``iter_kv_blocks(block_rows=...)``.
    """
    import torch

    batch_groups, n_query, n_heads, head_dim = q.shape
    score_bytes_per_key_row = batch_groups * n_heads * n_query * 4
    score_limited_rows = max(1, BLOCKWISE_SCORE_WORKSPACE_BYTES // max(score_bytes_per_key_row, 1))
    running_max = torch.full((batch_groups, n_heads, n_query, 1), float("-inf"), dtype=torch.float32)
    denominator = torch.zeros_like(running_max)
    numerator = torch.zeros((batch_groups, n_heads, n_query, head_dim), dtype=torch.float32)
    scale = (1.0 / math.sqrt(float(head_dim))) if scale is None else scale
    q_fp32 = q.to(torch.float32)
    for stored in kv_blocks:
        rows = stored.shape[1]
        step = min(rows, score_limited_rows)
        for start in range(0, rows, step):
            kv_block = stored[:, start : start + step]
            k, v = kv_block.unbind(dim=2)
            rep = _group(n_heads, k.shape[2])
            if rep != 1:
                k = k.repeat_interleave(rep, dim=2)
                v = v.repeat_interleave(rep, dim=2)
            logits = torch.einsum("bqhd,bkhd->bhqk", q_fp32, k.to(torch.float32)) * scale
            block_max = logits.amax(dim=-1, keepdim=True)
            new_max = torch.maximum(running_max, block_max)
            old_scale = torch.where(denominator > 0, torch.exp(running_max - new_max), torch.zeros_like(new_max))
            logits.sub_(new_max).exp_()
            block_denominator = logits.sum(dim=-1, keepdim=True)
            block_numerator = torch.einsum("bhqk,bkhd->bhqd", logits, v.to(torch.float32))
            numerator = numerator * old_scale + block_numerator
            denominator = denominator * old_scale + block_denominator
            running_max = new_max
    return (numerator / denominator).to(q.dtype).permute(0, 2, 1, 3)
