"""nori_icl_attention_noalloc: the attention entry point that allocates nothing.

Called through the C ABI, it must give exactly what nori_icl_attention gives with a
caller-provided workspace, on two calls in a row (the second smaller, so it reuses the scratch
the first one left behind), and refuse sizes whose split partials exceed the library's scratch
before doing any device work.
"""

from __future__ import annotations

import math

import pytest
import torch

from nori_amd import _native as nat

pytestmark = pytest.mark.gpu


def _case(bg, nq, heads, d, nk, kv_heads, kv_dtype, seed, device):
    g = torch.Generator(device="cpu").manual_seed(seed)
    q = torch.randn(bg, nq, heads, d, generator=g).to(torch.float16).to(device)
    kv = torch.randn(bg, nk, 2, kv_heads, d, generator=g)
    if kv_dtype == torch.int8:
        codes = torch.randint(-127, 128, kv.shape, generator=g, dtype=torch.int8).to(device)
        scales = (torch.rand(bg, nk, 2, kv_heads, 1, generator=g) * 0.05 + 1e-3).to(device)
        return q, codes, scales
    return q, kv.to(kv_dtype).to(device), None


def _args(q, kv, scales, out, lse, flags):
    bg, nq, heads, d = q.shape
    nk, kv_heads = kv.shape[1], kv.shape[3]
    sc = (0, 0, 0) if scales is None else (scales.stride(0), scales.stride(1), scales.stride(2))
    return [
        q.data_ptr(), nat.NORI_F16, bg, nq, heads, d, q.stride(0), q.stride(1), q.stride(2),
        kv.data_ptr(), nat.dtype_code(kv.dtype), nat.ptr(scales), nk, kv_heads,
        kv.stride(0), kv.stride(1), kv.stride(2), *sc,
        1.0 / math.sqrt(d),
        out.data_ptr(), nat.dtype_code(out.dtype), out.stride(0), out.stride(1), out.stride(2),
        nat.ptr(lse), flags,
    ]


def _run_pair(cuda, shape, kv_dtype, merge, seed):
    bg, nq, heads, d, nk, kv_heads = shape
    lib = nat.lib()
    need = lib.nori_icl_attention_workspace_size(bg, nq, heads, d, nk)
    print(f"no-alloc case {shape} cache {kv_dtype} merge={merge}: split scratch {need} bytes", flush=True)
    assert 0 < need <= nat.NOALLOC_SCRATCH_BYTES, "the case must run the split schedule inside the scratch"
    q, kv, scales = _case(bg, nq, heads, d, nk, kv_heads, kv_dtype, seed, cuda)
    out_dtype = torch.float32 if merge else torch.float16
    if merge:
        g = torch.Generator(device="cpu").manual_seed(seed + 1)
        out0 = torch.randn(bg, nq, heads, d, generator=g).to(cuda)
        lse0 = (torch.randn(bg, heads, nq, generator=g) + 3.0).to(cuda)
    else:
        out0 = torch.zeros(bg, nq, heads, d, dtype=out_dtype, device=cuda)
        lse0 = torch.zeros(bg, heads, nq, dtype=torch.float32, device=cuda)
    flags = nat.ATTN_MERGE if merge else 0
    stream = torch.cuda.current_stream(cuda).cuda_stream

    out_ref, lse_ref = out0.clone(), lse0.clone()
    workspace = torch.empty(need, dtype=torch.uint8, device=cuda)
    nat.check(lib.nori_icl_attention(*_args(q, kv, scales, out_ref, lse_ref, flags), workspace.data_ptr(), need, stream),
              "icl_attention")
    out_na, lse_na = out0.clone(), lse0.clone()
    nat.check(lib.nori_icl_attention_noalloc(*_args(q, kv, scales, out_na, lse_na, flags), stream), "icl_attention_noalloc")
    torch.cuda.synchronize(cuda)
    assert torch.isfinite(out_ref.float()).all()
    assert torch.equal(out_na, out_ref), (out_na.float() - out_ref.float()).abs().max().item()
    assert torch.equal(lse_na, lse_ref)


def test_noalloc_matches_workspace_entry_point_on_two_calls(cuda):
    # int8 cache at a 64k-row context (nori-30m head width), then a smaller ragged fp16 cache
    # merged into a running output, reusing the scratch the first call wrote
    _run_pair(cuda, (9, 1024, 2, 44, 65536, 2), torch.int8, merge=False, seed=11)
    _run_pair(cuda, (3, 300, 2, 44, 20000, 1), torch.float16, merge=True, seed=12)


def test_noalloc_refuses_sizes_beyond_its_scratch(cuda):
    lib = nat.lib()
    oversized = None
    for bg in (1, 3, 9, 33, 100):
        for nq in (256, 512, 1024, 2048):
            for heads in (2, 8):
                if lib.nori_icl_attention_workspace_size(bg, nq, heads, 128, 1 << 20) > nat.NOALLOC_SCRATCH_BYTES:
                    oversized = (bg, nq, heads)
                    break
            if oversized:
                break
        if oversized:
            break
    assert oversized is not None
    bg, nq, heads = oversized
    # null buffers: the size check comes before anything reads them
    args = [None, nat.NORI_F16, bg, nq, heads, 128, 0, 0, 0, None, nat.NORI_I8, None, 1 << 20, heads,
            0, 0, 0, 0, 0, 0, 1.0, None, nat.NORI_F16, 0, 0, 0, None, 0, None]
    assert lib.nori_icl_attention_noalloc(*args) == nat.NORI_ERR_UNSUPPORTED
    assert b"scratch" in lib.nori_last_error()
