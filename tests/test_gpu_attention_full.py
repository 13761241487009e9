"""Attention parity at the sizes the throughput is measured on, one launch each.

* The long-context shape: nori-30m block dims (33 token groups, 8 heads of 44) over a
  65,536-row int8 context with 1,024 query rows -- the bench's dominant kernel, with its whole
  units and its split tail (group 32's units run over context ranges merged by the second
  kernel).
* The batched shape: nori-100m block dims (32 tables x 51 token groups, 10 heads of 56) over
  8,192 int8 context rows with 2,048 query rows.

The cache comes from the HIP quantizer over N(0,1) fp16 K/V with 2 % of channels scaled x8;
queries are N(0,1). Every launch covers the whole shape; the float64 oracle
(oracle/attention.py) is evaluated on sampled (group, head) units -- whole units and split
ones, both query tiles, the last rows -- over the exact values the cache holds. Bars: the
reference's bf16 attention tolerance assert_close(rtol=2e-2, atol=2e-2)
(tests/test_blockwise_context_attention.py:172, 403) for outputs, the derived rounding bound
for the LSE; every output and LSE of the launch is finite.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import nori_amd
from test_gpu_attention import check, lse_bound, reference

pytestmark = pytest.mark.gpu


def int8_cache(bg, nk, hkv, d, device, seed, chunk=64):
    """Codes and scales of N(0,1) fp16 K/V with 2 % of the channels scaled x8, quantized by the
    HIP codec a few groups at a time (the fp16 tensor of a whole batched layer is not needed)."""
    g = torch.Generator(device=device).manual_seed(seed)
    ch = torch.randperm(d, generator=torch.Generator().manual_seed(seed))[: max(1, round(0.02 * d))].to(device)
    codes = torch.empty(bg, nk, 2, hkv, d, dtype=torch.int8, device=device)
    scales = torch.empty(bg, nk, 2, hkv, 1, dtype=torch.float32, device=device)
    for b0 in range(0, bg, chunk):
        b1 = min(bg, b0 + chunk)
        kv = torch.randn(b1 - b0, nk, 2, hkv, d, generator=g, device=device, dtype=torch.float16)
        kv[..., ch] *= 8.0
        c, s = nori_amd.quantize_int8(kv)
        codes[b0:b1] = c
        scales[b0:b1] = s
        del kv, c, s
    return codes, scales


def sampled_parity(q, codes, scales, out, lse, units, rows):
    """Oracle check of (group, head) units over query rows ``rows`` (MHA cache: head h reads K/V head h)."""
    for b, h in units:
        qs = q[b : b + 1, rows, h : h + 1]
        values = codes[b : b + 1, :, :, h : h + 1].double() * scales[b : b + 1, :, :, h : h + 1].double()
        exp, exp_lse = reference(qs, values)
        print(f"  unit (group {b}, head {h}): {len(rows)} query rows", flush=True)
        check(out[b : b + 1, rows, h : h + 1], exp)
        err = (lse[b : b + 1, h : h + 1, rows].double().cpu() - exp_lse).abs().numpy()
        assert (err <= lse_bound(qs, values, 1)).all(), f"LSE error {err.max():.3e}"


def test_long_context_64k_one_launch(cuda):
    bg, h, d, nq, nk = 33, 8, 44, 1024, 65536
    print(f"long-context attention: bg {bg}, heads {h}, d {d}, {nq} queries over {nk} int8 rows", flush=True)
    codes, scales = int8_cache(bg, nk, h, d, cuda, seed=2)
    q = torch.randn(bg, nq, h, d, generator=torch.Generator(device=cuda).manual_seed(3), device=cuda,
                    dtype=torch.float16)
    lse = torch.empty(bg, h, nq, device=cuda)
    out = nori_amd.icl_attention(q, codes, scales, lse=lse)
    torch.cuda.synchronize(cuda)
    assert bool(torch.isfinite(out).all()) and bool(torch.isfinite(lse).all())
    rows = list(range(0, 32)) + list(range(496, 528)) + list(range(992, 1024))
    # groups 0-31 run as whole units; group 32 is the split tail
    sampled_parity(q, codes, scales, out, lse, [(0, 0), (13, 3), (31, 7), (32, 0), (32, 5)], rows)


def test_batched_nori100m_shape_one_launch(cuda):
    bg, h, d, nq, nk = 32 * 51, 10, 56, 2048, 8192
    print(f"batched attention: bg {bg}, heads {h}, d {d}, {nq} queries over {nk} int8 rows", flush=True)
    codes, scales = int8_cache(bg, nk, h, d, cuda, seed=4, chunk=204)
    q = torch.randn(bg, nq, h, d, generator=torch.Generator(device=cuda).manual_seed(5), device=cuda,
                    dtype=torch.float16)
    lse = torch.empty(bg, h, nq, device=cuda)
    out = nori_amd.icl_attention(q, codes, scales, lse=lse)
    torch.cuda.synchronize(cuda)
    assert bool(torch.isfinite(out).all()) and bool(torch.isfinite(lse).all())
    rows = list(range(0, 16)) + list(range(504, 520)) + list(range(1528, 1544)) + list(range(2032, 2048))
    sampled_parity(q, codes, scales, out, lse, [(0, 0), (777, 4), (1200, 9), (1631, 2)], rows)
