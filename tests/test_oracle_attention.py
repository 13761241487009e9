"""Pins the attention oracle (oracle/attention.py) on the CPU.

The oracle restates softmax attention with GQA, the fp32 online-softmax block scan of
layer.py:777-839 and the LSE merge of layer.py:914-920. Checks that would catch a wrong
scale, a swapped head mapping, a dropped max-subtraction or a wrong merge weight:

* torch's SDPA on CPU (an independent implementation) in float64;
* closed forms: one key returns its value; identical keys average the values;
* the LSE merge over ragged splits equals one softmax (test_flex_attention_fallback.py:135-180);
* GQA equals repeat_interleave of K/V heads (test_flex_attention_fallback.py:68-74);
* zero-padding the head width leaves the result unchanged at a fixed scale
  (test_blockwise_context_attention.py:316-363);
* the fp32 block scan equals the float64 attention within the reference's fp32
  tolerance 2e-5 (test_blockwise_context_attention.py:172), including when the score
  workspace cap re-slices the blocks (:204-233).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attention as oa


def _rand(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape)


@pytest.mark.parametrize("heads,kv_heads", [(2, 2), (4, 1), (8, 2)])
def test_attention_f64_matches_torch_sdpa(heads, kv_heads):
    q = _rand((3, 7, heads, 16), 1)
    k = _rand((3, 13, kv_heads, 16), 2)
    v = _rand((3, 13, kv_heads, 16), 3)
    out, lse = oa.attention_f64(q, k, v)
    tq, tk, tv = (torch.from_numpy(a).permute(0, 2, 1, 3) for a in (q, k, v))
    ref = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, enable_gqa=heads != kv_heads)
    np.testing.assert_allclose(out, ref.permute(0, 2, 1, 3).numpy(), rtol=1e-12, atol=1e-12)
    # lse against logsumexp of explicitly formed logits
    kx = np.repeat(k, heads // kv_heads, axis=2)
    logits = np.einsum("bqhd,bkhd->bhqk", q, kx) / 4.0
    np.testing.assert_allclose(lse, torch.logsumexp(torch.from_numpy(logits), -1).numpy(), rtol=1e-12)


def test_closed_forms():
    q = _rand((1, 4, 2, 8), 4)
    v = _rand((1, 1, 2, 8), 5)
    out, lse = oa.attention_f64(q, _rand((1, 1, 2, 8), 6), v)
    np.testing.assert_allclose(out, np.broadcast_to(v, out.shape), rtol=1e-14)
    # identical keys: uniform weights, output = mean of values, lse = logit + log(n)
    k = np.broadcast_to(_rand((1, 1, 2, 8), 7), (1, 9, 2, 8))
    v = _rand((1, 9, 2, 8), 8)
    out, lse = oa.attention_f64(q, k, v, scale=0.5)
    np.testing.assert_allclose(out, np.broadcast_to(v.mean(axis=1, keepdims=True), out.shape), rtol=1e-12, atol=1e-14)
    logit = np.einsum("bqhd,bhd->bhq", q, k[:, 0]) * 0.5
    np.testing.assert_allclose(lse, logit + np.log(9), rtol=1e-12)


def test_lse_merge_over_ragged_splits_equals_one_softmax():
    q = _rand((2, 5, 4, 8), 9)
    k = _rand((2, 23, 4, 8), 10)
    v = _rand((2, 23, 4, 8), 11)
    full, full_lse = oa.attention_f64(q, k, v)
    run_o, run_l = None, None
    for a, b in ((0, 3), (3, 4), (4, 15), (15, 23)):
        o, l = oa.attention_f64(q, k[:, a:b], v[:, a:b])
        o = o.transpose(0, 2, 1, 3)  # [BG, H, Q, D] as the merge takes it
        if run_o is None:
            run_o, run_l = o, l
        else:
            run_o, run_l = oa.lse_merge(run_o, run_l, o, l)
    np.testing.assert_allclose(run_o.transpose(0, 2, 1, 3), full, rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(run_l, full_lse, rtol=1e-12)


def test_gqa_equals_repeat_interleave():
    q = _rand((2, 6, 6, 8), 12)
    k = _rand((2, 11, 2, 8), 13)
    v = _rand((2, 11, 2, 8), 14)
    grouped, _ = oa.attention_f64(q, k, v)
    expanded, _ = oa.attention_f64(q, np.repeat(k, 3, axis=2), np.repeat(v, 3, axis=2))
    np.testing.assert_allclose(grouped, expanded, rtol=1e-14)
    # head h reads kv head h // 3: changing kv head 1 must only move query heads 3..5
    k2 = k.copy()
    k2[:, :, 1] += _rand(k2[:, :, 1].shape, 18)
    moved, _ = oa.attention_f64(q, k2, v)
    assert np.allclose(moved[:, :, :3], grouped[:, :, :3]) and not np.allclose(moved[:, :, 3:], grouped[:, :, 3:])


@pytest.mark.parametrize("d,dpad", [(44, 64), (56, 64), (8, 16)])
def test_zero_padding_the_head_width_is_invisible(d, dpad):
    q = _rand((1, 5, 4, d), 15)
    k = _rand((1, 9, 4, d), 16)
    v = _rand((1, 9, 4, d), 17)
    out, _ = oa.attention_f64(q, k, v)
    pad = lambda a: np.concatenate([a, np.zeros(a.shape[:-1] + (dpad - d,))], axis=-1)  # noqa: E731
    padded, _ = oa.attention_f64(pad(q), pad(k), pad(v), scale=d**-0.5)
    np.testing.assert_allclose(padded[..., :d], out, rtol=1e-13)
    assert np.all(padded[..., d:] == 0)


@pytest.mark.parametrize("kv_heads", [1, 4])
def test_blockwise_scan_matches_f64(kv_heads, monkeypatch):
    torch.manual_seed(0)
    q = torch.randn(2, 7, 4, 16)
    kv = torch.randn(2, 37, 2, kv_heads, 16)
    blocks = [kv[:, :10], kv[:, 10:11], kv[:, 11:37]]
    got = oa.blockwise_attention_fp32(q, blocks)
    exp, _ = oa.attention_f64(q.numpy(), kv[:, :, 0].numpy(), kv[:, :, 1].numpy())
    np.testing.assert_allclose(got.numpy(), exp, rtol=2e-5, atol=2e-5)
    # a tiny score workspace forces every stored block to be re-sliced into 2-row pieces
    monkeypatch.setattr(oa, "BLOCKWISE_SCORE_WORKSPACE_BYTES", 2 * 2 * 4 * 7 * 4)
    got2 = oa.blockwise_attention_fp32(q, blocks)
    np.testing.assert_allclose(got2.numpy(), exp, rtol=2e-5, atol=2e-5)
