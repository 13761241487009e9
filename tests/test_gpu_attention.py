"""GPU parity of query-row -> context attention over the (int8) K/V cache.

Checked against the float64 oracle (oracle/attention.py) evaluated on the exact values
the cache holds (codes x scales for int8 caches). Tolerance is the reference's bf16
attention bar, assert_close(rtol=2e-2, atol=2e-2), i.e. |got - exp| <= 2e-2 + 2e-2*|exp|
(tests/test_blockwise_context_attention.py:172, 403); the assertion messages report the
max and mean absolute errors, which sit near 1e-3.
Covers the dense path, GQA/MQA, every supported head width, context lengths that are not
multiples of the 64-row block, query counts that are not multiples of the 256-row tile,
the split-context schedule, large logits (lazy max rescaling), the LSE output, the
running-output merge (layer.py:915-920), and the BlockwiseSeqKV host-streamed and
resident-int8 paths.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import nori_amd
from nori_amd import attention as attn
from nori_amd.kv_cache_scaling import BlockwiseSeqKV, ScalableSeqKV
from oracle import attention as oa

pytestmark = pytest.mark.gpu

TOL = 2e-2


def make_cache(bg, nk, hkv, d, device, seed, dtype=torch.float16, outliers=True):
    g = torch.Generator().manual_seed(seed)
    kv = torch.randn(bg, nk, 2, hkv, d, generator=g)
    if outliers:
        ch = torch.randperm(d, generator=g)[: max(1, round(0.02 * d))]
        kv[..., ch] *= 8.0
    return kv.to(dtype).to(device)


def make_queries(bg, nq, h, d, device, seed, dtype=torch.bfloat16, gain=1.0):
    g = torch.Generator().manual_seed(seed + 1000)
    return (torch.randn(bg, nq, h, d, generator=g) * gain).to(dtype).to(device)


def reference(q, kv_values, scale=None):
    """float64 oracle over the values the cache represents: kv_values [BG, N, 2, Hkv, D]."""
    kvv = kv_values.double().cpu().numpy()
    out, lse = oa.attention_f64(q.double().cpu().numpy(), kvv[:, :, 0], kvv[:, :, 1], scale)
    return torch.from_numpy(out), torch.from_numpy(lse)


def check(got, exp, tol=TOL):
    """|got - exp| <= tol + tol * |exp| elementwise: torch.testing.assert_close(rtol=tol, atol=tol),
    the criterion of the reference's own bf16 attention tests."""
    exp = exp.double()
    err = (got.double().cpu() - exp).abs()
    bound = tol + tol * exp.abs()
    worst = int(torch.argmax(err - bound))
    assert bool((err <= bound).all()), (
        f"max abs err {err.max().item():.3e} (mean {err.mean().item():.2e}); worst excess at flat index {worst}: "
        f"got {got.double().cpu().flatten()[worst].item():.5f} vs {exp.flatten()[worst].item():.5f}"
    )


@pytest.mark.parametrize("d", [8, 16, 44, 56, 64, 128])
@pytest.mark.parametrize("heads,kv_heads", [(2, 2), (4, 1)])
def test_int8_cache_matches_oracle(cuda, d, heads, kv_heads):
    bg, nq, nk = 3, 300, 331
    kv = make_cache(bg, nk, kv_heads, d, cuda, seed=d + heads)
    codes, scales = nori_amd.quantize_int8(kv)
    q = make_queries(bg, nq, heads, d, cuda, seed=d)
    lse = torch.empty(bg, heads, nq, device=cuda)
    got = nori_amd.icl_attention(q, codes, scales, lse=lse)
    assert got.dtype == q.dtype and got.shape == q.shape
    values = codes.double() * scales.double()
    exp, exp_lse = reference(q, values)
    check(got, exp)
    err = (lse.double().cpu() - exp_lse).abs().numpy()
    bound = lse_bound(q, values, heads // kv_heads)
    assert (err <= bound).all(), f"lse err {err.max():.3e} exceeds its rounding bound by {(err - bound).max():.3e}"


def lse_bound(q, values, group):
    """Rounding bound of the kernel's LSE (natural log). The logit MFMA multiplies f16
    operands: K dequantized to f16 (code x scale, one rounding; exact codes where the kernel
    keeps them) and Q rounded to f16 after the scale*log2(e) prescale, so logit j of query i
    is off by at most 2u * scale * sum_d |k_jd q_id| (u = 2^-11, plus fp32 accumulation
    slack); the LSE, a smooth maximum, moves by at most the largest logit error, and the
    denominator's f16 probabilities add a relative u."""
    u = 2.0**-11
    d = q.shape[-1]
    absk = np.repeat(np.abs(values[:, :, 0].cpu().numpy()), group, axis=2)  # [BG, N, H, D]
    absq = np.abs(q.double().cpu().numpy())  # [BG, Q, H, D]
    worst = np.einsum("bjhd,bihd->bhij", absk, absq).max(-1)  # [BG, H, Q]
    return 2.5 * u * worst / math.sqrt(d) + 3 * u


@pytest.mark.parametrize("kv_dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_full_precision_cache_matches_oracle(cuda, kv_dtype):
    kv = make_cache(2, 200, 2, 64, cuda, seed=3, dtype=kv_dtype)
    q = make_queries(2, 77, 2, 64, cuda, seed=3, dtype=torch.float16)
    got = nori_amd.icl_attention(q, kv)
    exp, _ = reference(q, kv)
    check(got, exp)


@pytest.mark.parametrize("nk", [1, 5, 63, 64, 65])
@pytest.mark.parametrize("nq", [1, 31, 257])
def test_ragged_lengths(cuda, nk, nq):
    kv = make_cache(2, nk, 2, 44, cuda, seed=nk)
    codes, scales = nori_amd.quantize_int8(kv)
    q = make_queries(2, nq, 2, 44, cuda, seed=nq)
    got = nori_amd.icl_attention(q, codes, scales)
    exp, _ = reference(q, codes.double() * scales.double())
    check(got, exp)


SHORT_CACHES = {"i8": torch.float16, "f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}


@pytest.mark.parametrize("d", [4, 8, 16, 44, 64, 128])
@pytest.mark.parametrize("kv_kind", ["i8", "f16", "bf16", "f32"])
@pytest.mark.parametrize("nq,nk", [(5, 7), (1, 1), (64, 32), (16, 128)])
def test_short_context_path(cuda, d, kv_kind, nq, nk):
    """Few queries over few keys (nq <= 64, nk <= 128, nq * nk <= 2048) take the VALU kernel:
    the in-row attentions of the two-phase encoder (fp16 caches with 8 or more queries and at
    most 64 keys take the few-token MFMA kernel instead). GQA (4 query heads on 2 K/V
    heads), the LSE output, and the running-output merge of two context halves."""
    bg, heads, kv_heads = 37, 4, 2
    kv = make_cache(bg, nk, kv_heads, d, cuda, seed=d + nk, dtype=SHORT_CACHES[kv_kind])
    q = make_queries(bg, nq, heads, d, cuda, seed=d + nq, dtype=torch.float16)
    if kv_kind == "i8":
        codes, scales = nori_amd.quantize_int8(kv)
        values = codes.double() * scales.double()
        call = lambda sl, **kw: nori_amd.icl_attention(q, codes[:, sl], scales[:, sl], **kw)  # noqa: E731
    else:
        values = kv.double()
        call = lambda sl, **kw: nori_amd.icl_attention(q, kv[:, sl], **kw)  # noqa: E731
    lse = torch.empty(bg, heads, nq, device=cuda)
    got = call(slice(0, nk), lse=lse)
    exp, exp_lse = reference(q, values)
    check(got, exp)
    assert ((lse.double().cpu() - exp_lse).abs().numpy() <= lse_bound(q, values, heads // kv_heads)).all()
    if nk > 1:
        run = torch.zeros(bg, nq, heads, d, device=cuda)
        lse2 = torch.full((bg, heads, nq), float("-inf"), device=cuda)
        for sl in (slice(0, nk // 2), slice(nk // 2, nk)):
            call(sl, out=run, lse=lse2, merge=True)
        check(run, exp)


def test_split_context_schedule(cuda):
    # one small (bg, head, query tile) grid over a long context: the kernel splits the
    # context across workgroups and merges the partial (O, LSE) pairs
    bg, h, nq, nk, d = 1, 2, 100, 5000, 64
    assert attn.workspace_bytes(bg, nq, h, d, nk) > 0
    kv = make_cache(bg, nk, h, d, cuda, seed=11)
    codes, scales = nori_amd.quantize_int8(kv)
    q = make_queries(bg, nq, h, d, cuda, seed=11)
    lse = torch.empty(bg, h, nq, device=cuda)
    got = nori_amd.icl_attention(q, codes, scales, lse=lse)
    values = codes.double() * scales.double()
    exp, exp_lse = reference(q, values)
    check(got, exp)
    assert ((lse.double().cpu() - exp_lse).abs().numpy() <= lse_bound(q, values, 1)).all()


def test_tail_split_matches_whole_units(cuda):
    # 33 groups x 8 heads x 2 query tiles = 528 work units on 256 slots: two full rounds run
    # whole, the 16 units of the third round (group 32, query tiles fastest) are split over
    # the idle slots and merged by the second kernel. Called through the C ABI twice -- with
    # the workspace (tail split) and without (every unit whole): the whole units are computed
    # identically by both calls, and group 32 matches the oracle either way.
    from nori_amd import _native as nat

    bg, h, nq, nk, d = 33, 8, 1024, 4096, 44
    ws = attn.workspace_bytes(bg, nq, h, d, nk)
    assert ws > 0
    kv = make_cache(bg, nk, h, d, cuda, seed=41)
    codes, scales = nori_amd.quantize_int8(kv)
    del kv
    q = make_queries(bg, nq, h, d, cuda, seed=41, dtype=torch.float32)
    workspace = torch.empty(ws, dtype=torch.uint8, device=cuda)
    results = []
    for buf, nbytes in ((workspace, ws), (None, 0)):
        out = torch.empty_like(q)
        lse = torch.empty(bg, h, nq, device=cuda)
        nat.check(
            nat.lib().nori_icl_attention(
                q.data_ptr(), nat.dtype_code(q.dtype), bg, nq, h, d, q.stride(0), q.stride(1), q.stride(2),
                codes.data_ptr(), nat.dtype_code(codes.dtype), scales.data_ptr(), nk, h,
                codes.stride(0), codes.stride(1), codes.stride(2), scales.stride(0), scales.stride(1), scales.stride(2),
                1.0 / math.sqrt(d), out.data_ptr(), nat.dtype_code(out.dtype), out.stride(0), out.stride(1),
                out.stride(2), lse.data_ptr(), 0, nat.ptr(buf), nbytes, nat.stream_of(cuda),
            ),
            "icl_attention",
        )
        results.append((out, lse))
    (o_split, l_split), (o_whole, l_whole) = results
    assert torch.equal(o_split[:32], o_whole[:32]) and torch.equal(l_split[:32], l_whole[:32])
    values = (codes[32:].double() * scales[32:].double()).cpu()
    exp, exp_lse = reference(q[32:], values)
    for o, lse in ((o_split, l_split), (o_whole, l_whole)):
        check(o[32:], exp)
        assert ((lse[32:].double().cpu() - exp_lse).abs().numpy() <= lse_bound(q[32:], values, 1)).all()


@pytest.mark.parametrize("d", [44, 64])
@pytest.mark.parametrize("gain", [4.0, 12.0])
def test_large_logits_exercise_rescaling(cuda, gain, d):
    # QASS multiplies queries by ~log(n) (layer.py:433-456): logits of tens of units, where the
    # running max must move between blocks; the first block is deliberately weak. d = 44 runs
    # the kernel that carries the running max inside the logit MFMA, d = 64 the one that
    # subtracts it on the VALU.
    bg, nq, nk = 2, 64, 700
    kv = make_cache(bg, nk, 2, d, cuda, seed=21)
    kv[:, :64] *= 0.05
    codes, scales = nori_amd.quantize_int8(kv)
    q = make_queries(bg, nq, 2, d, cuda, seed=21, gain=gain)
    got = nori_amd.icl_attention(q, codes, scales)
    exp, _ = reference(q, codes.double() * scales.double())
    check(got, exp)


@pytest.mark.parametrize("d,nq", [(44, 600), (56, 600), (52, 200), (44, 64)])
def test_key_norm_ramp_moves_the_max_late(cuda, d, nq):
    # Key magnitudes grow 20x along the context, so blocks early in the scan satisfy the
    # per-block logit bound (|q| max|k| - m <= slack: the per-step max test is skipped) while
    # later blocks must move the running max by more than the slack, several times. A bound
    # that were too small would let probabilities past the slack through unrescaled. Logits
    # stay within what f16 Q and K resolve at the 2e-2 bar (|q| ~ 3 per element). Shapes: the
    # 16-wave kernels (d = 44 and 56, 600 queries), the 8-wave one (d = 52), the 2-wave one.
    bg, h, nk = 2, 2, 3000
    kv = make_cache(bg, nk, h, d, cuda, seed=41)
    ramp = torch.linspace(0.05, 1.0, nk, device=cuda).view(1, nk, 1, 1, 1)
    kv = (kv.float() * ramp).to(kv.dtype)
    codes, scales = nori_amd.quantize_int8(kv)
    q = make_queries(bg, nq, h, d, cuda, seed=41, gain=3.0)
    lse = torch.empty(bg, h, nq, device=cuda)
    got = nori_amd.icl_attention(q, codes, scales, lse=lse)
    values = codes.double() * scales.double()
    exp, exp_lse = reference(q, values)
    check(got, exp)
    assert torch.isfinite(lse).all()
    assert ((lse.double().cpu() - exp_lse).abs().numpy() <= lse_bound(q, values, 1)).all()


@pytest.mark.parametrize("d", [44, 56])
@pytest.mark.parametrize("lift", [11.0, 24.0])
def test_late_key_above_the_anchored_max(cuda, d, lift):
    # The folded kernels scan every block after the first without the per-step rescale test,
    # keeping the running max the first block anchored, and rescan a work unit with the test
    # on when a probability overflowed f16 on the way (its denominator turns inf/NaN). One key
    # late in a 2048-row context (block 14 of 16) is lifted `lift` log2 units above the logits of
    # every other key: 11 stays within f16 (probabilities up to 2^11 in the unchecked scan), 24
    # overflows and must be rescanned. Either way the output is that key's value row, within the
    # reference's bar, and the LSE within its rounding bound. d = 44 runs the prefetching
    # 16-wave kernel, d = 56 the one that reads K operands just before their MFMAs.
    bg, h, nq, nk = 2, 2, 300, 2048
    scale = 1.0 / math.sqrt(d)
    g = torch.Generator().manual_seed(61)
    q0 = torch.randn(bg, 1, h, d, generator=g)
    q = q0 + 0.05 * torch.randn(bg, nq, h, d, generator=g)
    kv = 0.3 * torch.randn(bg, nk, 2, h, d, generator=g)
    late = 1800
    # q0 . k* = lift * ln 2 / scale for the late key: logit lift log2 units above ~0
    kv[:, late, 0] = q0[:, 0] * (lift * math.log(2.0) / scale) / (q0[:, 0] ** 2).sum(-1, keepdim=True)
    codes, scales = nori_amd.quantize_int8(kv.to(torch.float16).to(cuda))
    q = q.to(torch.float16).to(cuda)
    lse = torch.empty(bg, h, nq, device=cuda)
    got = nori_amd.icl_attention(q, codes, scales, lse=lse)
    values = codes.double() * scales.double()
    exp, exp_lse = reference(q, values)
    check(got, exp)
    assert torch.isfinite(got).all() and torch.isfinite(lse).all()
    assert ((lse.double().cpu() - exp_lse).abs().numpy() <= lse_bound(q, values, 1)).all()


def test_merge_of_two_halves_equals_one_call(cuda):
    bg, h, nq, nk, d = 2, 4, 50, 300, 56
    kv = make_cache(bg, nk, 1, d, cuda, seed=31)
    codes, scales = nori_amd.quantize_int8(kv)
    q = make_queries(bg, nq, h, d, cuda, seed=31)
    run = torch.zeros(bg, nq, h, d, device=cuda)
    lse = torch.full((bg, h, nq), float("-inf"), device=cuda)
    for a, b in ((0, 130), (130, 300)):
        nori_amd.icl_attention(q, codes[:, a:b], scales[:, a:b], out=run, lse=lse, merge=True)
    values = codes.double() * scales.double()
    exp, exp_lse = reference(q, values)
    check(run, exp)
    assert ((lse.double().cpu() - exp_lse).abs().numpy() <= lse_bound(q, values, h)).all()


@pytest.mark.parametrize("d", [44, 56, 100])
def test_merge_with_split_context(cuda, d):
    # Long host blocks merged into a running output, each block's context split over idle
    # workgroup slots: the second kernel merges the split partials into the running output and
    # overwrites the running LSE. A row's lanes (d / 4 of them: 11 at d = 44, not a divisor of
    # the 64-lane wavefront) must all read the old LSE before it is overwritten. Two scans of
    # the same blocks give the same bits, and both match the oracle.
    bg, h, nq, half = 1, 2, 300, 5000
    assert attn.workspace_bytes(bg, nq, h, d, half) > 0
    kv = make_cache(bg, 2 * half, 1, d, cuda, seed=d + 7)
    codes, scales = nori_amd.quantize_int8(kv)
    q = make_queries(bg, nq, h, d, cuda, seed=d + 7)
    runs = []
    for _ in range(2):
        run = torch.zeros(bg, nq, h, d, device=cuda)
        lse = torch.full((bg, h, nq), float("-inf"), device=cuda)
        for a, b in ((0, half), (half, 2 * half)):
            nori_amd.icl_attention(q, codes[:, a:b], scales[:, a:b], out=run, lse=lse, merge=True)
        runs.append((run, lse))
    assert torch.equal(runs[0][0], runs[1][0]) and torch.equal(runs[0][1], runs[1][1])
    values = codes.double() * scales.double()
    exp, exp_lse = reference(q, values)
    check(runs[0][0], exp)
    assert ((runs[0][1].double().cpu() - exp_lse).abs().numpy() <= lse_bound(q, values, h)).all()


@pytest.mark.parametrize("offload", [True, False])
def test_blockwise_cache_paths(cuda, offload):
    bg, h, nq, d = 3, 2, 40, 44
    kv = make_cache(bg, 517, h, d, cuda, seed=41)
    cache = BlockwiseSeqKV.from_row_slices(
        (kv[:, a:b] for a, b in ((0, 200), (200, 201), (201, 517))), 1, bg, quantize=True, device=cuda,
        dtype=kv.dtype, offload=offload, n_rows=517,
    )
    dense = ScalableSeqKV(kv, 1, bg, quantize=True, device=cuda)
    q = make_queries(bg, nq, h, d, cuda, seed=41)
    got = nori_amd.compute_attention_blockwise(q, cache)
    payload, scales = dense.device_payload()
    exp, _ = reference(q, payload.double() * scales.double())
    check(got, exp)
    got_dense = nori_amd.attend_dense(q, dense)
    check(got_dense, exp)
    if offload:
        assert cache.max_staged_rows == 316 and cache.resident_gpu_bytes() == 0


@pytest.mark.parametrize("quantize", [True, False])
def test_streamed_scan_overlaps_many_blocks(cuda, quantize):
    # 13 host blocks (the last ragged) through the two staging slots: block i+1 is copied on the
    # staging stream while block i is attended; every slot is reused several times. The merged
    # result equals one launch over the same cache up to fp32 merge rounding, and a second scan
    # of the same cache gives the same bits.
    bg, h, nq, d, rows = 2, 2, 300, 44, 256
    nk = 12 * rows + 77
    kv = make_cache(bg, nk, h, d, cuda, seed=43)
    bounds = [(a, min(a + rows, nk)) for a in range(0, nk, rows)]
    cache = BlockwiseSeqKV.from_row_slices(
        (kv[:, a:b] for a, b in bounds), 1, bg, quantize=quantize, device=cuda, dtype=kv.dtype, offload=True,
    )
    assert len(cache.host_blocks()) == len(bounds) == 13 and cache.resident_gpu_bytes() == 0
    q = make_queries(bg, nq, h, d, cuda, seed=43)
    got = nori_amd.compute_attention_blockwise(q, cache)
    again = nori_amd.compute_attention_blockwise(q, cache)
    assert torch.equal(got, again) and cache.max_staged_rows == rows
    if quantize:
        codes, scales = nori_amd.quantize_int8(kv)
        whole = nori_amd.icl_attention(q, codes, scales)
        values = codes.double() * scales.double()
    else:
        whole = nori_amd.icl_attention(q, kv)
        values = kv
    torch.testing.assert_close(got.float(), whole.float(), rtol=1e-2, atol=2e-3)
    exp, _ = reference(q, values)
    check(got, exp)


def test_config2_attention(cuda):
    # isolated nori-6m ICL block: BG=9, 1024 queries over 4096 int8 context rows, H=2, D=64, bf16
    g = torch.Generator().manual_seed(1)
    q = torch.randn(9, 1024, 2, 64, generator=g)
    kv = torch.randn(9, 4096, 2, 2, 64, generator=g)
    ch = torch.randperm(128, generator=g)[:3]
    q.view(9, 1024, 128)[..., ch] *= 8.0
    kv.view(9, 4096, 2, 128)[..., ch] *= 8.0
    q = q.to(torch.bfloat16).to(cuda)
    kv = kv.to(torch.bfloat16).to(cuda)
    codes, scales = nori_amd.quantize_int8(kv)
    got = nori_amd.icl_attention(q, codes, scales)
    exp, _ = reference(q, codes.double() * scales.double(), 1 / math.sqrt(64))
    check(got, exp)
    # against torch SDPA over the fp32-dequantized cache: the reference's dense path as it runs
    # on the CPU (fp32 cache dtype). With x8 outlier channels in both Q and K the logits reach
    # ~200, where a bf16 dequantization alone moves outputs by O(1); fp32 keeps the check sharp.
    deq = nori_amd.dequantize_int8(codes, scales, torch.float32).cpu()
    k, v = deq.unbind(dim=2)
    sdpa = torch.nn.functional.scaled_dot_product_attention(
        q.cpu().float().permute(0, 2, 1, 3), k.permute(0, 2, 1, 3).contiguous(), v.permute(0, 2, 1, 3).contiguous()
    ).permute(0, 2, 1, 3)
    check(got, sdpa.double())


def test_shape_errors(cuda):
    q = torch.randn(2, 5, 3, 16, device=cuda, dtype=torch.bfloat16)
    kv = torch.randn(2, 7, 2, 2, 16, device=cuda, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="cannot attend"):
        nori_amd.icl_attention(q, kv)
    with pytest.raises(ValueError, match="head width"):
        nori_amd.icl_attention(q[..., :8], torch.randn(2, 7, 2, 3, 16, device=cuda))
    with pytest.raises(NotImplementedError):
        nori_amd.icl_attention(torch.randn(2, 5, 2, 6, device=cuda), torch.randn(2, 7, 2, 2, 6, device=cuda))


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("d", [16, 44, 64])
def test_qk_prologue_equals_separate_passes(cuda, dtype, d):
    """icl_attention(qk_prologue=...) -- the per-head q/k RMS norms with gains and the q
    multiply applied as the short-context kernel loads the rows -- against the same steps as
    separate passes (nori_amd.rms_norm over q and K, the q multiply in q's dtype, then the
    attention). Only the order of the mean-of-squares sums differs, so the results agree to
    within a unit or two of the last place of the normed values."""
    from nori_amd.norm import rms_norm

    bg, nq, nk, heads = 300, 4, 6, 2
    g = torch.Generator().manual_seed(d)
    q = (torch.randn(bg, nq, heads, d, generator=g) * 3).to(dtype).to(cuda)
    kv = (torch.randn(bg, nk, 2, heads, d, generator=g) * 3).to(dtype).to(cuda)
    qw = (1 + 0.3 * torch.randn(d, generator=g)).to(cuda)
    kw = (1 + 0.3 * torch.randn(d, generator=g)).to(cuda)
    mult = float(torch.tensor(math.log(nk), dtype=dtype))
    fused = nori_amd.icl_attention(q, kv, qk_prologue={"q_weight": qw, "k_weight": kw, "eps": 1e-6, "q_mult": mult})
    qn = rms_norm(q, d, qw, 1e-6) * torch.tensor(mult, dtype=dtype, device=cuda)
    kvn = kv.clone()
    kvn[:, :, 0] = rms_norm(kv[:, :, 0], d, kw, 1e-6)
    separate = nori_amd.icl_attention(qn, kvn)
    tol = 4e-3 if dtype == torch.float16 else 1e-5
    torch.testing.assert_close(fused.float(), separate.float(), rtol=tol, atol=tol)
    with pytest.raises(NotImplementedError):  # long contexts keep the separate passes
        long_kv = torch.randn(bg, 300, 2, heads, d, device=cuda).to(dtype)
        nori_amd.icl_attention(q, long_kv, qk_prologue={"q_weight": qw, "k_weight": kw, "eps": 1e-6, "q_mult": 1.0})


@pytest.mark.parametrize("d,nk", [(64, 256), (64, 200), (48, 256), (32, 97)])
@pytest.mark.parametrize("key_norm", [True, False])
def test_qk_prologue_on_resident_context_launches(cuda, d, nk, key_norm):
    """The q/k prologue on resident-context launches (384 tables x 2 heads, 320 queries over up
    to 256 keys: the two-phase encoder's column and row attentions): the query norm on the
    fragment as loaded (the row's halves in lanes l and l ^ 32), the key norm on the staged
    rows in LDS. Against the same steps as separate passes: only the order of the
    mean-of-squares sums differs, which moves a normed value by an fp16 ulp now and then; the
    sharp softmax here (|q| x 3, log-n factor 5.5) turns such a flip into up to ~1.5e-2 on a
    handful of outputs (33 of 15.7 M measured), so all outputs are held to 2e-2 and 99.99 % to
    4e-3 -- a systematic error moves most of them. An int8 cache takes the query norm alone."""
    from nori_amd.attention import takes_prologue
    from nori_amd.norm import rms_norm

    bg, nq, heads = 384, 320, 2
    g = torch.Generator().manual_seed(d + nk)
    q = (torch.randn(bg, nq, heads, d, generator=g) * 3).half().to(cuda)
    # un-normed keys at unit scale, so the logits are as sharp as with normed ones
    kv = (torch.randn(bg, nk, 2, heads, d, generator=g) * (3 if key_norm else 1)).half().to(cuda)
    qw = (1 + 0.3 * torch.randn(d, generator=g)).to(cuda)
    kw = (1 + 0.3 * torch.randn(d, generator=g)).to(cuda) if key_norm else None
    mult = float(torch.tensor(math.log(nk), dtype=torch.float16))
    print(f"resident prologue: d {d} nk {nk} key norm {key_norm}", flush=True)
    assert takes_prologue(bg, nq, heads, d, nk, torch.float16, key_norm)
    assert takes_prologue(bg, nq, heads, d, nk, torch.int8, False) and not takes_prologue(bg, nq, heads, d, nk, torch.int8, True)
    assert not takes_prologue(2, nq, heads, d, nk, torch.float16, key_norm)  # too few units: the ring kernel
    # resident-context launches take fp16 queries only: other query dtypes go to the ring kernel
    assert not takes_prologue(bg, nq, heads, d, nk, torch.float16, key_norm, q_dtype=torch.bfloat16)
    fused = nori_amd.icl_attention(q, kv, qk_prologue={"q_weight": qw, "k_weight": kw, "eps": 1e-6, "q_mult": mult})
    qn = rms_norm(q, d, qw, 1e-6) * torch.tensor(mult, dtype=torch.float16, device=cuda)
    kvn = kv.clone()
    if key_norm:
        kvn[:, :, 0] = rms_norm(kv[:, :, 0], d, kw, 1e-6)
    separate = nori_amd.icl_attention(qn, kvn)

    def agree(a, b):
        err = (a.float() - b.float()).abs()
        bound = 4e-3 + 4e-3 * b.float().abs()
        assert float((err <= bound).float().mean()) >= 0.9999, f"{int((err > bound).sum())} outputs past 4e-3"
        torch.testing.assert_close(a.float(), b.float(), rtol=2e-2, atol=2e-2)

    agree(fused, separate)
    if not key_norm:  # the query norm over an int8 cache
        codes, scales = nori_amd.quantize_int8(kv)
        fused8 = nori_amd.icl_attention(q, codes, scales, qk_prologue={"q_weight": qw, "k_weight": None, "eps": 1e-6,
                                                                       "q_mult": mult})
        agree(fused8, nori_amd.icl_attention(qn, codes, scales))


def test_two_phase_attention_module_takes_the_prologue(cuda):
    """MultiheadAttention with qk_norm and QASS "log_only" (the two-phase attention) computes
    the same output through the fused prologue as through its separate passes, under the fp16
    autocast of GPU inference."""
    from nori_amd.layer import MultiheadAttention

    torch.manual_seed(0)
    attn = MultiheadAttention(64, 2, qkv_combined=False, use_qassmax=True, qass_mode="log_only", qk_norm=True).to(cuda).eval()
    with torch.no_grad():
        attn.q_norm.weight.mul_(1 + 0.2 * torch.randn(32, device=cuda))
        attn.k_norm.weight.mul_(1 + 0.2 * torch.randn(32, device=cuda))
    x = torch.randn(50, 30, 4, 64, device=cuda)
    kv_src = torch.randn(50, 30, 6, 64, device=cuda)
    with torch.inference_mode(), torch.autocast("cuda", dtype=torch.float16):
        assert attn._fused_prologue(torch.empty(1, 4, 2, 32, device=cuda, dtype=torch.float16),
                                    torch.empty(1, 6, 2, 2, 32, device=cuda, dtype=torch.float16)) is not None
        fused = attn(x=x, x_kv=kv_src)[0]
        attn._fused_prologue = lambda q, kv: None
        separate = attn(x=x, x_kv=kv_src)[0]
    torch.testing.assert_close(fused.float(), separate.float(), rtol=5e-3, atol=5e-3)


def test_short_context_at_two_phase_scale(cuda):
    """The short-context kernel over the full grid of the nori-1-5-sized model's cell feature
    attention: 163,840 table rows x 2 heads x 4 queries over 6 keys, d 64, fp16 (1.3 M query
    rows in one launch), against a float32 torch evaluation of softmax(q k^T / sqrt(d)) v on
    the GPU, with the q/k prologue and without."""
    bg, nq, nk, heads, d = 163840, 4, 6, 2, 64
    g = torch.Generator(device=cuda).manual_seed(5)
    q = torch.randn(bg, nq, heads, d, generator=g, device=cuda).half()
    kv = torch.randn(bg, nk, 2, heads, d, generator=g, device=cuda).half()
    got = nori_amd.icl_attention(q, kv)
    qf = q.float().permute(0, 2, 1, 3).contiguous()                  # [bg, h, nq, d]
    kf = kv[:, :, 0].float().permute(0, 2, 3, 1).contiguous()       # [bg, h, d, nk]
    vf = kv[:, :, 1].float().permute(0, 2, 1, 3).contiguous()       # [bg, h, nk, d]
    p = torch.softmax(torch.matmul(qf, kf) / math.sqrt(d), dim=-1)
    exp = torch.matmul(p, vf).permute(0, 2, 1, 3)
    err = (got.float() - exp).abs()
    assert err.max().item() < 2e-3, f"max abs err {err.max().item():.3e}"
    ones = torch.ones(d, device=cuda)
    fused = nori_amd.icl_attention(q, kv, qk_prologue={"q_weight": ones, "k_weight": ones, "eps": 1e-6, "q_mult": 1.0})
    qn = q.float() * torch.rsqrt(q.float().pow(2).mean(-1, keepdim=True) + 1e-6)
    kn = kv[:, :, 0].float() * torch.rsqrt(kv[:, :, 0].float().pow(2).mean(-1, keepdim=True) + 1e-6)
    p = torch.softmax(torch.matmul(qn.permute(0, 2, 1, 3).contiguous(), kn.permute(0, 2, 3, 1).contiguous()) / math.sqrt(d), -1)
    exp = torch.matmul(p, vf).permute(0, 2, 1, 3)
    err = (fused.float() - exp).abs()
    assert err.max().item() < 4e-3, f"max abs err {err.max().item():.3e}"


def test_int8_scales_outside_the_f16_range(cuda):
    # Caches quantized from bf16 K/V may carry scales outside f16's range. Tiny ones (vectors
    # with amax ~1e-9, scales below f16's subnormals) dequantize to ~0 in the kernel: an
    # absolute error below 127 * 2^-25 per element, far inside the bar. Scales whose K/V values
    # exceed f16's range (127 * scale > 65504) are refused when a container hands the payload
    # to the kernel.
    bg, h, nq, nk, d = 2, 2, 40, 300, 44
    kv = make_cache(bg, nk, h, d, cuda, seed=51, dtype=torch.bfloat16)
    kv[:, 7:40] *= 1e-9
    cache = ScalableSeqKV(kv, 1, bg, quantize=True, device=cuda)
    payload, scales = cache.device_payload()
    assert float(scales.min()) < 2.0**-24
    q = make_queries(bg, nq, h, d, cuda, seed=51)
    got = nori_amd.attend_dense(q, cache)
    exp, _ = reference(q, payload.double() * scales.double())
    check(got, exp)
    big = ScalableSeqKV(make_cache(bg, nk, h, d, cuda, seed=52, dtype=torch.bfloat16) * 1e6, 1, bg, quantize=True,
                        device=cuda)
    with pytest.raises(NotImplementedError, match="fp16 range"):
        nori_amd.attend_dense(q, big)
    blocks = BlockwiseSeqKV.from_row_slices(iter([kv[:, :100] * 1e6, kv[:, 100:]]), 1, bg, quantize=True, device=cuda,
                                            offload=True)
    with pytest.raises(NotImplementedError, match="fp16 range"):
        nori_amd.compute_attention_blockwise(q, blocks)


@pytest.mark.parametrize("d", [8, 16, 44, 56, 64])
@pytest.mark.parametrize("nq,nk", [(51, 51), (33, 64), (64, 64), (40, 60), (64, 33), (33, 33), (17, 5), (9, 9), (8, 10)])
def test_few_token_tile_path(cuda, d, nq, nk):
    """8 to 64 fp16 queries over up to 64 fp16 keys take the few-token MFMA kernel (a
    wavefront per (b, h, 32-query tile), exact softmax over the unit's whole context): the
    feature attention over a row's tokens (33 tokens at 32 features, 51 at 50). GQA (4 query
    heads on 2 K/V heads) and the LSE output against the float64 oracle; a running-output
    merge keeps the long-context or the short-context kernel."""
    bg, heads, kv_heads = 29, 4, 2
    kv = make_cache(bg, nk, kv_heads, d, cuda, seed=3 * d + nk)
    q = make_queries(bg, nq, heads, d, cuda, seed=d + nq, dtype=torch.float16, gain=2.0)
    lse = torch.empty(bg, heads, nq, device=cuda)
    got = nori_amd.icl_attention(q, kv, lse=lse)
    exp, exp_lse = reference(q, kv.double())
    check(got, exp)
    assert ((lse.double().cpu() - exp_lse).abs().numpy() <= lse_bound(q, kv.double(), heads // kv_heads)).all()
    run = torch.zeros(bg, nq, heads, d, device=cuda)
    lse2 = torch.full((bg, heads, nq), float("-inf"), device=cuda)
    for sl in (slice(0, nk // 2), slice(nk // 2, nk)):
        nori_amd.icl_attention(q, kv[:, sl], out=run, lse=lse2, merge=True)
    check(run, exp)


def test_few_token_tile_path_at_the_config4_launch(cuda):
    """The 51 x 51 feature attention at the size one config-4 build launch has (65,536 rows =
    8 tables x 8,192 context rows, 10 heads of 56, q and K/V read out of one [rows, 51, 3, 10,
    56] fp16 projection, fp16 output): 96 sampled rows against the float64 oracle, and the rows
    bit for bit what a launch over those rows alone gives."""
    rows, tokens, heads, d = 65536, 51, 10, 56
    torch.manual_seed(4)
    qkv = torch.randn(rows, tokens, 3, heads, d, device=cuda, dtype=torch.float16)
    print(f"few-token attention at [{rows}, {tokens}, 3, {heads}, {d}]", flush=True)
    got = nori_amd.icl_attention(qkv[:, :, 0], qkv[:, :, 1:])
    pick = torch.randperm(rows, generator=torch.Generator().manual_seed(5))[:96].to(cuda)
    sub = qkv[pick]
    exp, _ = reference(sub[:, :, 0], sub[:, :, 1:].double())
    check(got[pick].float(), exp)
    assert torch.equal(nori_amd.icl_attention(sub[:, :, 0], sub[:, :, 1:]), got[pick])


def test_few_token_tile_path_on_a_qkv_projection(cuda):
    """The feature attention's own layout: q and K/V as strided views into one [rows, tokens,
    3, heads, d] projection (nori-100m dims: 51 tokens, 10 heads of 56), fp16 output."""
    rows, tokens, heads, d = 700, 51, 10, 56
    g = torch.Generator().manual_seed(9)
    qkv = torch.randn(rows, tokens, 3, heads, d, generator=g).half().to(cuda)
    got = nori_amd.icl_attention(qkv[:, :, 0], qkv[:, :, 1:])
    assert got.dtype == torch.float16
    exp, _ = reference(qkv[:, :, 0], qkv[:, :, 1:].double())
    check(got.float(), exp)


@pytest.mark.parametrize("d,kv_kind", [(64, "f16"), (64, "i8"), (32, "bf16"), (48, "f16")])
@pytest.mark.parametrize("nq,nk", [(320, 256), (300, 200), (640, 97)])
def test_resident_context_path(cuda, d, kv_kind, nq, nk):
    """Contexts of up to 256 keys read by more than 160 queries per (b, h), with at least two
    (b, h) units per CU, take the resident-context workgroups (10 wavefronts that stage the
    unit's whole context once): here 384 tables x 2 heads. They match the float64 oracle on a
    sample of tables; where the head width is a multiple of 16 (the VALU-mode scan, the same
    arithmetic as the ring kernel's) they give the ring kernel's bits, which a slice of two
    tables -- too few units for the resident path -- takes on the same rows."""
    bg, heads = 384, 2
    kv = make_cache(bg, nk, heads, d, cuda, seed=nq + nk + d, dtype=SHORT_CACHES[kv_kind])
    q = make_queries(bg, nq, heads, d, cuda, seed=nq + d, dtype=torch.float16, gain=2.0)
    print(f"resident path: d {d} {kv_kind} nq {nq} nk {nk}", flush=True)
    if kv_kind == "i8":
        codes, scales = nori_amd.quantize_int8(kv)
        got = nori_amd.icl_attention(q, codes, scales)
        ring = nori_amd.icl_attention(q[:2], codes[:2], scales[:2])
        values = codes[:3].double() * scales[:3].double()
    else:
        got = nori_amd.icl_attention(q, kv)
        ring = nori_amd.icl_attention(q[:2], kv[:2])
        values = kv[:3].double()
    exp, _ = reference(q[:3], values)
    check(got[:3], exp)
    assert torch.isfinite(got).all()
    if d % 16 == 0:
        assert torch.equal(got[:2], ring)
    else:
        check(got[:2], ring.float())


@pytest.mark.parametrize("offset", [1, 2])
def test_few_token_shape_with_a_query_view_off_the_4_element_grid(cuda, offset):
    """Few-token shapes whose query rows do not start on 4-element (8-byte) boundaries -- here
    heads of 44 read out of rows of 44 + offset elements at element offset 1 or 2 -- are
    routed to the kernels that read queries one element at a time (the few-token kernel reads
    them 8 bytes at a time) and still match the float64 oracle."""
    bg, nq, nk, heads, kv_heads, d = 13, 33, 33, 4, 2, 44
    kv = make_cache(bg, nk, kv_heads, d, cuda, seed=77)
    base = make_queries(bg, nq, heads, d + offset, cuda, seed=78, dtype=torch.float16, gain=2.0)
    q = base[..., offset:]
    assert q.stride(2) % 4 != 0 or q.storage_offset() % 4 != 0
    lse = torch.empty(bg, heads, nq, device=cuda)
    got = nori_amd.icl_attention(q, kv, lse=lse)
    exp, exp_lse = reference(q, kv.double())
    check(got, exp)
    assert ((lse.double().cpu() - exp_lse).abs().numpy() <= lse_bound(q, kv.double(), heads // kv_heads)).all()
    # the same values in an aligned view give the same answer to the bar
    check(nori_amd.icl_attention(q.contiguous(), kv), exp)
