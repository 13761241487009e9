"""Host-side logic of the drop-in cache containers that needs no kernel (CPU tensors).

Mirrors the transport and error-behaviour checks of the reference's
tests/test_kv_cache_scaling.py and tests/test_blockwise_context_attention.py.
"""

from __future__ import annotations

import pytest
import torch

from nori_amd.kv_cache_scaling import BlockwiseSeqKV, ScalableSeqKV, _split_strides, _vector_layout, scale_caches


def _row_slices(kv, rows):
    start = 0
    for width in rows:
        yield kv[:, start : start + width]
        start += width


def test_scalable_identity_and_offload_without_quantization():
    kv = torch.randn(2, 50, 2, 4, 8)
    c = ScalableSeqKV(kv, 2, 5, quantize=False, offload=False, device=torch.device("cpu"))
    assert c["batch"] == 2 and c["groups"] == 5 and torch.equal(c["kv"], kv)
    c = ScalableSeqKV(kv, 2, 5, quantize=False, offload=True, device=torch.device("cpu"))
    assert torch.equal(c["kv"], kv) and c.resident_gpu_bytes() == 0
    with pytest.raises(KeyError):
        c["nope"]


def test_from_row_slices_reassembles_and_rejects_empty():
    kv = torch.randn(2, 100, 2, 3, 8)
    out = ScalableSeqKV.from_row_slices(iter([kv[:, i : i + 32] for i in range(0, 100, 32)]), 2, 3, quantize=False,
                                        device=torch.device("cpu"), dtype=kv.dtype)
    assert torch.equal(out["kv"], kv)
    with pytest.raises(ValueError):
        ScalableSeqKV.from_row_slices(iter([]), 1, 1, quantize=True, device=torch.device("cpu"), dtype=torch.float32)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_blockwise_transport_and_full_read_refusal(dtype):
    kv = torch.randn(2, 11, 2, 3, 4, dtype=dtype)
    cache = BlockwiseSeqKV.from_row_slices(_row_slices(kv, (3, 5, 3)), 1, 2, quantize=False,
                                           device=torch.device("cpu"), dtype=dtype)
    assert torch.equal(torch.cat(list(cache.iter_kv_blocks()), dim=1), kv)
    assert cache.resident_gpu_bytes() == 0 and cache.host_bytes() == kv.numel() * kv.element_size()
    assert cache.n_rows == 11 and cache.max_block_rows == 5 and cache.max_staged_rows == 5
    with pytest.raises(RuntimeError, match="cannot materialize a full layer"):
        cache["kv"]
    blocks = list(cache.iter_kv_blocks(block_rows=2))
    assert max(b.shape[1] for b in blocks) <= 2 and cache.max_staged_rows == 2
    with pytest.raises(ValueError):
        list(cache.iter_kv_blocks(block_rows=0))


def test_blockwise_resident_requires_int8_and_row_count():
    kv = torch.randn(1, 4, 2, 1, 4)
    with pytest.raises(ValueError, match="quantize=True"):
        BlockwiseSeqKV.from_row_slices(iter([kv]), 1, 1, quantize=False, device=torch.device("cpu"), offload=False, n_rows=4)
    with pytest.raises(ValueError, match="positive n_rows"):
        BlockwiseSeqKV.from_row_slices(iter([kv]), 1, 1, quantize=True, device=torch.device("cpu"), offload=False)
    with pytest.raises(ValueError):
        BlockwiseSeqKV([], 1, 1, device=torch.device("cpu"), dtype=torch.float32, quantized=False)


def test_scale_caches_is_a_noop_when_off():
    caches = [{"seq_kv": {"kv": torch.randn(1, 10, 2, 2, 4), "batch": 1, "groups": 1}}]
    assert scale_caches(caches) is caches and isinstance(caches[0]["seq_kv"], dict)


def test_vector_layout_collapses_leading_axes():
    kv = torch.empty(3, 100, 2, 4, 44)
    assert _vector_layout(kv) == (1, 3 * 100 * 2 * 4, 0, 44)
    view = kv[:, 10:30]  # a row slice of preallocated storage: two strided levels
    assert _vector_layout(view) == (3, 20 * 2 * 4, 100 * 2 * 4 * 44, 44)
    scales = torch.empty(3, 100, 2, 4, 1)[:, 10:30]
    assert _vector_layout(scales) == (3, 20 * 2 * 4, 100 * 2 * 4, 1)
    assert _vector_layout(torch.empty(2, 3, 8)[:, :, ::2]) is None  # last axis not contiguous
    assert _vector_layout(torch.empty(4, 5, 6, 8)[::2, ::2]) is None  # three levels


def test_split_strides_addresses_contiguous_outputs_of_a_sliced_source():
    # a row slice of a cache is two-level (3 x 800 vectors); the fresh contiguous codes and
    # scales that quantize_int8 allocates for it are single-level and must take that split
    src = torch.empty(3, 517, 2, 2, 44)[:, 0:200]
    so, si, sos, sis = _vector_layout(src)
    assert (so, si) == (3, 800)
    codes = torch.empty(src.shape, dtype=torch.int8)
    scales = torch.empty(tuple(src.shape[:-1]) + (1,))
    assert _split_strides(_vector_layout(codes), so, si) == (800 * 44, 44)
    assert _split_strides(_vector_layout(scales), so, si) == (800, 1)
    # element addresses agree with torch's own indexing
    o, i = 2, 517
    assert codes[o].reshape(-1, 44)[i].data_ptr() - codes.data_ptr() == o * 800 * 44 + i * 44
    # a two-level destination only takes its own split; mismatched counts are refused
    view = torch.empty(3, 517, 2, 2, 44)[:, 100:300]
    assert _split_strides(_vector_layout(view), 3, 800) == (517 * 4 * 44, 44)
    assert _split_strides(_vector_layout(view), 1, 2400) is None
    assert _split_strides(_vector_layout(codes), 4, 600) == (600 * 44, 44)
    assert _split_strides(_vector_layout(codes), 4, 601) is None
    assert _split_strides(None, 1, 1) is None


def test_fused_cache_write_is_taken_only_where_it_computes_the_same():
    # the fused (RMSNorm ->) projection -> int8 write replaces the separate steps only under the
    # GPU's fp16 autocast and for a row norm it can fold (none, or RMSNorm without a weight)
    from nori_amd import kv_project
    from nori_amd import layer as NL

    attn = NL.MultiheadAttention(64, 4, qkv_combined=False)
    cpu = torch.device("cpu")
    assert not kv_project.fp16_autocast(cpu)
    assert NL._fused_cache_write(attn, None, False, cpu) is None  # no fp16 autocast on the CPU
    with torch.autocast("cpu", dtype=torch.bfloat16):
        assert not kv_project.fp16_autocast(cpu)


def test_fused_rows_report_the_projected_slice_they_stand_for():
    from nori_amd.kv_project import FusedKVRows, fusable

    x = torch.randn(2, 3, 5, 64)  # [B, G, n, E]
    w = torch.randn(2 * 4 * 16, 64)
    rows = FusedKVRows(x, w, 4, 16, 1e-5)
    assert rows.shape == (6, 5, 2, 4, 16) and rows.dtype == torch.float16
    with pytest.raises(ValueError, match="B, G, n, E"):
        FusedKVRows(x[0], w, 4, 16, None)
    # host tensors are never taken by the kernel
    assert not fusable(x, w, 16)



def test_log_only_qass_logit_scale_rounds_log_n_in_the_query_dtype():
    # QASSMaxScaling.forward (layer.py:433-456) multiplies q by log(n) cast to q's dtype, and
    # returns q untouched for a single key; the folded logit scale carries exactly that factor
    import math

    from nori_amd.layer import MultiheadAttention

    mod = MultiheadAttention(embed_dim=128, num_heads=2, use_qassmax=True, qass_mode="log_only", qk_norm=True)
    for n in (2, 256, 65536, 70000):
        for dtype in (torch.float16, torch.bfloat16, torch.float32):
            factor = torch.tensor(math.log(n), dtype=dtype).item()
            assert mod.log_only_logit_scale(n, dtype) == factor / 8.0
    assert mod.log_only_logit_scale(256, torch.float16) != math.log(256) / 8.0  # the fp16 rounding is kept
    assert mod.log_only_logit_scale(1, torch.float16) == 1.0 / 8.0
    assert mod.log_only_logit_scale(0, torch.float32) == 1.0 / 8.0
