"""GPU parity of the int8 cache codec: HIP kernel vs the oracle and vs torch on the GPU.

Bit-exact bar: codes and scales must equal, bit for bit,
  * the C oracle in its GPU scale mode (``m * fp32(1/127)``), and
  * the reference expression (kv_cache_scaling.py:35-37) executed by torch on the same
    device and dtype,
for every source dtype and head width, on config-2 shaped caches with outlier channels,
on special vectors, on strided destinations, and at config-3 size.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import nori_amd
from nori_amd.kv_cache_scaling import BlockwiseSeqKV, ScalableSeqKV
from oracle import codec

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.float16, torch.bfloat16]


def torch_reference(t: torch.Tensor):
    scale = t.abs().amax(dim=-1, keepdim=True).clamp_min(1e-12) / 127.0
    q = torch.clamp(torch.round(t / scale), -127, 127).to(torch.int8)
    return q, scale.to(torch.float32)


def oracle_quantize(t: torch.Tensor):
    c = t.detach().cpu()
    if c.dtype == torch.bfloat16:
        raw, name = c.view(torch.int16).numpy().view(np.uint16), "bf16"
    else:
        raw, name = c.numpy(), ("f32" if c.dtype == torch.float32 else "f16")
    return codec.quantize_int8(raw, name, codec.DIV_RECIP)


def outlier_cache(shape, dtype, device, seed, frac=0.02, factor=8.0):
    g = torch.Generator().manual_seed(seed)
    t = torch.randn(*shape, generator=g)
    d = shape[-1]
    ch = torch.randperm(d, generator=g)[: max(1, round(frac * d))]
    t[..., ch] *= factor
    return t.to(dtype).to(device)


def assert_bits_equal(codes, scales, ref_codes, ref_scales):
    assert torch.equal(codes.cpu(), ref_codes.cpu() if isinstance(ref_codes, torch.Tensor) else torch.from_numpy(ref_codes))
    a = scales.cpu().view(torch.int32)
    b = (ref_scales.cpu() if isinstance(ref_scales, torch.Tensor) else torch.from_numpy(ref_scales)).view(torch.int32)
    assert torch.equal(a, b)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("d", [4, 8, 16, 44, 56, 64, 128, 200])
def test_quantize_bit_exact(cuda, dtype, d):
    t = outlier_cache((3, 301, 2, 2, d), dtype, cuda, seed=d)
    t[0, 0] = torch.linspace(-1e-3, 1e-3, d, device=cuda).to(dtype)
    t[0, 1] = ((torch.arange(d, device=cuda) - d // 2) * 0.5).to(dtype)
    codes, scales = nori_amd.quantize_int8(t)
    assert codes.shape == t.shape and scales.shape == t.shape[:-1] + (1,)
    ref_q, ref_s = torch_reference(t)
    assert_bits_equal(codes, scales, ref_q, ref_s)
    o_q, o_s = oracle_quantize(t)
    assert_bits_equal(codes, scales, o_q, o_s)


def test_config2_cache_bit_exact(cuda):
    # nori-6m block dims: BG=9, 4096 context rows, Hkv=2, D=64, bf16 N(0,1), 3 channels x8
    t = outlier_cache((9, 4096, 2, 2, 64), torch.bfloat16, cuda, seed=1, frac=3 / 128)
    codes, scales = nori_amd.quantize_int8(t)
    ref_q, ref_s = torch_reference(t)
    assert_bits_equal(codes, scales, ref_q, ref_s)
    o_q, o_s = oracle_quantize(t)
    assert_bits_equal(codes, scales, o_q, o_s)


@pytest.mark.parametrize("dtype", DTYPES)
def test_special_vectors_match_torch(cuda, dtype):
    d = 16
    rows = [
        torch.zeros(d),
        torch.full((d,), 1e-30),
        torch.full((d,), 3e-8),  # fp16 scale underflows to 0
        torch.linspace(-6e4, 6e4, d),
        torch.tensor([1.0] * (d - 1) + [float("nan")]),
        torch.tensor([1.0] * (d - 1) + [float("inf")]),
        torch.tensor([-2.0] * (d - 1) + [float("-inf")]),
    ]
    t = torch.stack(rows).to(dtype).to(cuda)
    codes, scales = nori_amd.quantize_int8(t)
    ref_q, ref_s = torch_reference(t)
    assert torch.equal(codes.cpu(), ref_q.cpu())
    s, r = scales.cpu(), ref_s.cpu()
    assert torch.equal(torch.isnan(s), torch.isnan(r))
    assert torch.equal(s[~torch.isnan(s)], r[~torch.isnan(r)])
    o_q, _ = oracle_quantize(t)
    assert torch.equal(codes.cpu(), torch.from_numpy(o_q))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_every_absmax_matches_torch(cuda, dtype):
    """Each vector's absmax swept over the dtype's positive finite values -- every bf16 value
    (subnormal scales included), and for fp32 sixteen random significands at every exponent
    from 2^-149 to 2^127 -- with the other 15 values uniform in [-absmax, absmax]: codes and
    scales equal the reference expression on the same device and the oracle. (The fp16 sweep,
    every f16 absmax, is in tests/test_gpu_kv_project.py beside the fused write's.)"""
    g = torch.Generator().manual_seed(21)
    if dtype == torch.bfloat16:
        amax = (torch.arange(1, 0x7F80, dtype=torch.int32) << 16).view(torch.float32)
    else:
        e = torch.arange(-149, 128, dtype=torch.float64).repeat_interleave(16)
        m = 1.0 + torch.rand(e.numel(), generator=g, dtype=torch.float64)
        amax = (m * torch.pow(2.0, e)).clamp(max=3.4e38).float()
        amax = amax[torch.isfinite(amax) & (amax > 0)]
    d = 16
    vecs = (torch.rand(amax.numel(), d, generator=g, dtype=torch.float64) * 2 - 1) * amax.double()[:, None]
    vecs[:, 0] = amax.double() * torch.where(torch.rand(amax.numel(), generator=g) < 0.5, -1.0, 1.0).double()
    vecs = torch.gather(vecs, 1, torch.argsort(torch.rand(amax.numel(), d, generator=g), dim=1))
    t = vecs.to(dtype).to(cuda)
    assert torch.equal(t.abs().amax(-1).float().cpu(), amax.to(dtype).float())
    codes, scales = nori_amd.quantize_int8(t)
    ref_q, ref_s = torch_reference(t)
    assert_bits_equal(codes, scales, ref_q, ref_s)
    o_q, o_s = oracle_quantize(t)
    assert_bits_equal(codes, scales, o_q, o_s)


@pytest.mark.parametrize("dtype", DTYPES)
def test_dequantize_bit_exact(cuda, dtype):
    t = outlier_cache((2, 97, 2, 3, 44), torch.float32, cuda, seed=5)
    q, s = torch_reference(t)
    got = nori_amd.dequantize_int8(q, s, dtype)
    assert torch.equal(got.cpu(), (q.float() * s).to(dtype).cpu())
    name = {torch.float32: "f32", torch.float16: "f16", torch.bfloat16: "bf16"}[dtype]
    exp = codec.dequantize_int8(q.cpu().numpy(), s.cpu().numpy(), name)
    raw = got.cpu().view(torch.int16).numpy().view(np.uint16) if dtype == torch.bfloat16 else got.cpu().numpy()
    assert np.array_equal(raw.view(np.uint8), exp.view(np.uint8))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", [(1, 7, 2, 1, 20), (3, 33, 2, 2, 16), (2, 50, 2, 8, 44), (1, 9, 2, 3, 56), (2, 5, 2, 1, 128), (1, 11, 2, 2, 8)])
def test_dequantize_widths_and_row_slices(cuda, dtype, shape):
    # every head width class of the dequantizer (16-byte chunks that straddle two vectors, a
    # partial last chunk, widths below one chunk), whole tensors and row-slice views (two-level
    # addressing with an outer stride), against torch's own expression on the same device
    t = outlier_cache(shape, torch.float32, cuda, seed=shape[-1])
    q, s = torch_reference(t)
    got = nori_amd.dequantize_int8(q, s, dtype)
    assert torch.equal(got.cpu(), (q.float() * s).to(dtype).cpu())
    rows = slice(1, shape[1] - 1) if shape[1] > 2 else slice(0, shape[1])
    got_rows = nori_amd.dequantize_int8(q[:, rows], s[:, rows], dtype)
    assert torch.equal(got_rows.cpu(), (q[:, rows].float() * s[:, rows]).to(dtype).cpu())


def test_row_slices_into_preallocated_storage_equal_whole_tensor(cuda):
    # reference tests/test_blockwise_context_attention.py:31-61 and test_kv_cache_scaling.py:60-78
    kv = outlier_cache((3, 257, 2, 4, 44), torch.float16, cuda, seed=9)
    whole_q, whole_s = torch_reference(kv)
    cache = BlockwiseSeqKV.from_row_slices(
        (kv[:, a:b] for a, b in ((0, 64), (64, 100), (100, 257))), 3, 4, quantize=True, device=cuda,
        dtype=kv.dtype, offload=False, n_rows=257,
    )
    payload, scales = cache.resident_payload()
    assert_bits_equal(payload, scales, whole_q, whole_s)
    assert len({p.untyped_storage().data_ptr() for p, _ in cache.device_blocks()}) == 1
    dense = ScalableSeqKV(kv, 3, 4, quantize=True, device=cuda)
    assert torch.equal(torch.cat(list(cache.iter_kv_blocks()), dim=1), dense["kv"])
    built = ScalableSeqKV.from_row_slices(iter([kv[:, :100], kv[:, 100:]]), 3, 4, quantize=True, device=cuda)
    assert_bits_equal(*built.device_payload(), whole_q, whole_s)


def test_roundtrip_error_and_empty_input(cuda):
    t = torch.randn(4, 100, 2, 3, 16, device=cuda)
    q, s = nori_amd.quantize_int8(t)
    rel = (nori_amd.dequantize_int8(q, s, t.dtype) - t).abs().max() / t.abs().max()
    assert rel < 0.02
    e_q, e_s = nori_amd.quantize_int8(torch.empty(0, 5, 2, 1, 8, device=cuda))
    assert e_q.shape == (0, 5, 2, 1, 8) and e_s.shape == (0, 5, 2, 1, 1)


def test_config3_full_layer_bit_exact(cuda):
    # nori-30m dims: 33 token groups x 65536 rows x 2 x 8 heads x 44, fp16 (the GPU autocast dtype)
    g = torch.Generator(device=cuda).manual_seed(2)
    t = torch.randn((33, 65536, 2, 8, 44), generator=g, device=cuda, dtype=torch.float16)
    codes, scales = nori_amd.quantize_int8(t)
    ref_q, ref_s = torch_reference(t)
    assert torch.equal(codes, ref_q)
    assert torch.equal(scales.view(torch.int32), ref_s.view(torch.int32))
    # and the oracle on a sample of rows (codes are per-row, so a sample is exact)
    rows = torch.randint(0, 65536, (64,), generator=g, device=cuda)
    o_q, o_s = oracle_quantize(t[:, rows])
    assert_bits_equal(codes[:, rows], scales[:, rows], o_q, o_s)
