"""CPU restatement of the cached sequence-attention step that bench.py times on the GPU.

TEST INFRASTRUCTURE ONLY: the CPU baseline of ``bench.py`` (and the tests that pin it).
Only tests/, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it; the product package never does.

The reference runs its CPU inference in fp32 (src/synthefy_nori/inference/predictor.py:318-321
turns mixed precision off on the CPU), so everything here is fp32 torch on the host, using
every thread torch is given:

* ``quantize_int8`` -- the reference's int8 cache codec on an fp32 cache
  (model/kv_cache_scaling.py:29-37): per head vector, scale = max|t| (at least 1e-12) / 127,
  codes = round-half-even(t / scale) clamped to [-127, 127];
* ``dequantized_blocks`` -- the stored int8 cache read back in row blocks as the reference's
  blockwise reader does (kv_cache_scaling.py:40-41, 292-330: codes.float() * scale);
* ``sequence_attention_step`` -- one query batch through one layer's cached sequence
  attention as the workload composes it (model/layer.py:1945-1953 with
  ``forward_with_kv_cache``, :685-745): RMSNorm without weight (layer.py:251-253), the Q
  projection, attention over the dequantized cache with the CPU online-softmax scan
  (oracle.attention.blockwise_attention_fp32, layer.py:777-839), the output projection and the
  deepnorm residual x + alpha * out.

Pins (tests/test_oracle_sublayer.py): ``quantize_int8`` equals the C oracle's fp32 codec (itself
pinned to the reference's golden codes) bit for bit; ``sequence_attention_step`` equals a
float64 composition (textbook attention) to fp32 rounding; dequantized blocks joined equal the
whole-cache dequantization.
"""

from __future__ import annotations

import torch

from .attention import blockwise_attention_fp32

# the reference's blockwise reader stores the cache in blocks of this many rows when it streams
# (a block is dequantized, scanned and dropped; kv_cache_scaling.py:292-330)
BLOCK_ROWS = 32768


def quantize_int8(t: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(codes int8, scales fp32 [..., 1]) of an fp32 cache ``t`` [..., D] (kv_cache_scaling.py:29-37)."""
    if t.dtype != torch.float32:
        raise ValueError(f"the CPU cache is fp32, got {t.dtype}")
    amax = torch.amax(t.abs(), dim=-1, keepdim=True)
    scale = torch.clamp(amax, min=1e-12) / 127.0
    codes = torch.round(t / scale).clamp_(-127, 127).to(torch.int8)
    return codes, scale


def dequantized_blocks(codes: torch.Tensor, scales: torch.Tensor, block_rows: int = BLOCK_ROWS):
    """Yield the fp32 cache rows [BG, n, 2, Hkv, D] block by block (kv_cache_scaling.py:40-41)."""
    rows = codes.shape[1]
    for a in range(0, rows, block_rows):
        yield codes[:, a : a + block_rows].to(torch.float32) * scales[:, a : a + block_rows]


def rms_norm(x: torch.Tensor, eps: float) -> torch.Tensor:
    """x * rsqrt(mean(x^2) + eps) over the last axis, fp32 (layer.py:251-253, no weight)."""
    return x * torch.rsqrt(x.pow(2).mean(dim=-1, keepdim=True) + eps)


def sequence_attention_step(x, wq, wo, codes, scales, *, heads: int, head_dim: int, alpha: float, eps: float = 1e-5,
                            block_rows: int = BLOCK_ROWS):
    """One query batch x [BG, Q, E] (fp32) through one layer's cached sequence attention.

    wq [H*D, E] is the Q projection, wo [H, D, E] the output projection, (codes, scales) the
    layer's int8 cache [BG, N, 2, Hkv, D] / [BG, N, 2, Hkv, 1]. Returns x + alpha * out.
    """
    bg, nq, _ = x.shape
    q = torch.nn.functional.linear(rms_norm(x, eps), wq).view(bg, nq, heads, head_dim)
    o = blockwise_attention_fp32(q, dequantized_blocks(codes, scales, block_rows))
    return x + alpha * torch.einsum("bqhd,hde->bqe", o, wo)
