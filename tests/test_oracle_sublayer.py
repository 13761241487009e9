"""Pins of oracle/sublayer.py, the CPU restatement that bench.py's CPU baseline times.

* ``quantize_int8`` (torch, fp32 cache) equals the C oracle's fp32 codec bit for bit -- the
  codec that tests/test_oracle_codec.py pins to the reference's golden codes -- including
  all-zero vectors (scale 1e-12 / 127) and vectors with one dominant entry;
* the dequantized blocks, joined, equal the whole-cache dequantization, for ragged blocks;
* ``sequence_attention_step`` equals the same step composed in float64 with the textbook
  attention (oracle.attention.attention_f64) up to fp32 rounding, for grouped K/V heads and a
  ragged last block.
"""

from __future__ import annotations

import numpy as np
import torch

from oracle import codec
from oracle import sublayer as osl
from oracle.attention import attention_f64


def test_quantizer_matches_the_c_codec():
    g = torch.Generator().manual_seed(11)
    t = torch.randn(5, 37, 2, 3, 44, generator=g) * torch.rand(5, 37, 2, 3, 1, generator=g) * 10.0
    t[0, 0, 0, 0] = 0.0  # an all-zero vector
    t[1, 2, 1, 2, 7] = 1e4  # one dominant entry
    codes, scales = osl.quantize_int8(t)
    ref_codes, ref_scales = codec.quantize_int8(t.numpy(), "f32", codec.DIV_TRUE)
    assert np.array_equal(codes.numpy(), ref_codes)
    assert np.array_equal(scales.numpy().view(np.uint32), ref_scales.view(np.uint32))
    assert not codes[0, 0, 0, 0].any()


def test_dequantized_blocks_join_to_the_whole_cache():
    g = torch.Generator().manual_seed(12)
    codes, scales = osl.quantize_int8(torch.randn(2, 75, 2, 2, 8, generator=g))
    whole = codes.float() * scales
    joined = torch.cat(list(osl.dequantized_blocks(codes, scales, block_rows=16)), dim=1)
    assert torch.equal(joined, whole)


def test_step_matches_a_float64_composition():
    g = torch.Generator().manual_seed(13)
    bg, nq, embed, heads, hkv, d, nk, alpha, eps = 3, 5, 24, 4, 2, 12, 70, 0.3, 1e-5
    x = torch.randn(bg, nq, embed, generator=g)
    wq = torch.randn(heads * d, embed, generator=g) * embed ** -0.5
    wo = torch.randn(heads, d, embed, generator=g) * 0.2
    codes, scales = osl.quantize_int8(torch.randn(bg, nk, 2, hkv, d, generator=g))
    got = osl.sequence_attention_step(x, wq, wo, codes, scales, heads=heads, head_dim=d, alpha=alpha, eps=eps,
                                      block_rows=16)

    x64 = x.double().numpy()
    xn = x64 / np.sqrt((x64 ** 2).mean(axis=-1, keepdims=True) + eps)
    q = (xn @ wq.double().numpy().T).reshape(bg, nq, heads, d)
    kv = codes.double().numpy() * scales.double().numpy()
    out, _ = attention_f64(q, kv[:, :, 0], kv[:, :, 1])
    exp = x64 + alpha * np.einsum("bqhd,hde->bqe", out, wo.double().numpy())
    err = np.abs(got.double().numpy() - exp).max() / np.abs(exp).max()
    assert err < 2e-6, err
