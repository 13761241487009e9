"""GPU parity of the fused context-cache write: (RMSNorm ->) K/V projection -> int8 codes.

The unfused path it replaces is the reference's, on the GPU under fp16 autocast:
``F.linear`` (layer.py:676-679) writes fp16 K/V, ``quantize_int8`` (kv_cache_scaling.py:29-37)
codes them. Bars:
  * bit-exact on operands whose products and sums are exact in fp32 (multiples of 1/8 and
    1/16 over a few hundred terms), where the summation order cannot matter: codes and
    scales equal torch's autocast projection quantized by torch's own expression, and the
    oracle's quantizer applied to torch's fp16 K/V;
  * on Gaussian operands, where the fp32 sums of the MFMA and of the library GEMM round
    differently in the last bit now and then: every code within one of torch's and at most
    0.5% of them different, scales within one fp16 ulp;
  * row slices written through strided views equal the whole-tensor call bit for bit;
  * the layer's int8 cache builds under autocast -- the plain whole-context build and the
    bounded ones -- write the cache by the reference's separate steps by default, and take the
    fused write only with ``fused_cache_write=True``, which gives the same caches (codes within
    one, at most 1% of them different) and outputs as the default build, and the reference's
    fp32 outputs (its own run of the same stack, tests/golden/layer_cache_goldens.npz) to
    their tolerance;
  * the default build of a nori-30m layer (embed 352, 8 heads of 44) under autocast writes
    codes and scales equal (torch.equal) to torch's F.linear of the layer's own cache operand
    quantized by the reference expression on the same device.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import nori_amd
from nori_amd import layer as NL
from nori_amd.kv_cache_scaling import BlockwiseSeqKV, ScalableSeqKV
from oracle import codec

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.float16, torch.bfloat16]


@pytest.fixture(autouse=True)
def fp32_gemm_reductions():
    # the reference GEMMs sum in fp32 throughout, as the fused kernel does
    flag = torch.backends.cuda.matmul.allow_fp16_reduced_precision_reduction
    torch.backends.cuda.matmul.allow_fp16_reduced_precision_reduction = False
    yield
    torch.backends.cuda.matmul.allow_fp16_reduced_precision_reduction = flag


def torch_quantize(t):
    scale = t.abs().amax(dim=-1, keepdim=True).clamp_min(1e-12) / 127.0
    q = torch.clamp(torch.round(t / scale), -127, 127).to(torch.int8)
    return q, scale.to(torch.float32)


def autocast_projection(x, w, heads, d, eps=None):
    """The unfused GPU path: (rms_norm ->) F.linear under fp16 autocast -> [..., 2, heads, d] fp16."""
    if eps is not None:
        x = nori_amd.rms_norm(x, x.shape[-1], None, eps)
    with torch.autocast("cuda", dtype=torch.float16):
        kv = F.linear(x, w)
    assert kv.dtype == torch.float16
    return kv.view(*x.shape[:-1], 2, heads, d)


def dyadic(shape, step, lim, gen, device, dtype):
    k = int(lim / step)
    return (torch.randint(-k, k + 1, shape, generator=gen) * step).to(dtype).to(device)


@pytest.mark.parametrize("xdt", DTYPES)
@pytest.mark.parametrize("embed,heads,d", [(352, 8, 44), (64, 2, 16), (96, 1, 64), (200, 3, 20), (32, 4, 8)])
def test_exact_sums_bit_exact(cuda, xdt, embed, heads, d):
    g = torch.Generator().manual_seed(embed + d)
    x = dyadic((3, 131, embed), 1 / 8, 2.0, g, cuda, xdt)
    w = dyadic((2 * heads * d, embed), 1 / 16, 1.0, g, cuda, torch.float32)
    codes, scales = nori_amd.project_quantize_kv(x, w, heads, d)
    assert codes.shape == (3, 131, 2, heads, d) and scales.shape == (3, 131, 2, heads, 1)
    kv = autocast_projection(x, w, heads, d)
    ref_q, ref_s = torch_quantize(kv)
    assert torch.equal(codes, ref_q)
    assert torch.equal(scales.view(torch.int32), ref_s.view(torch.int32))
    o_q, o_s = codec.quantize_int8(kv.cpu().numpy(), "f16", codec.DIV_RECIP)
    assert np.array_equal(codes.cpu().numpy(), o_q)
    assert np.array_equal(scales.cpu().numpy().view(np.int32), o_s.view(np.int32))


def assert_codes_close(codes, scales, ref_q, ref_s, max_frac=5e-3):
    diff = (codes.int() - ref_q.int()).abs()
    assert int(diff.max()) <= 1
    frac = float((diff > 0).float().mean())
    print(f"[parity] int8 codes: {frac:.2e} of them differ by one (bar {max_frac:.0e})", flush=True)
    assert frac <= max_frac
    rel = ((scales - ref_s).abs() / ref_s.abs().clamp_min(1e-30)).max()
    assert float(rel) <= 2.0 ** -10


@pytest.mark.parametrize("xdt", DTYPES)
@pytest.mark.parametrize("norm", [False, True])
@pytest.mark.parametrize("embed,heads,d", [(352, 8, 44), (128, 2, 64), (48, 1, 12)])
def test_gaussian_matches_autocast_path(cuda, xdt, norm, embed, heads, d):
    g = torch.Generator(device=cuda).manual_seed(7 + embed)
    x = (3.0 * torch.randn(2, 517, embed, generator=g, device=cuda)).to(xdt)
    w = torch.randn(2 * heads * d, embed, generator=g, device=cuda) / embed ** 0.5
    eps = 1e-5 if norm else None
    codes, scales = nori_amd.project_quantize_kv(x, w, heads, d, norm_eps=eps)
    ref_q, ref_s = torch_quantize(autocast_projection(x, w, heads, d, eps))
    assert_codes_close(codes, scales, ref_q, ref_s)


def test_fp16_weight_and_strided_weight_rows(cuda):
    # the K/V rows of a packed [3, H, D, E] weight, as the layer passes them, in fp16
    g = torch.Generator().manual_seed(3)
    heads, d, embed = 4, 16, 64
    qkv = dyadic((3, heads, d, embed), 1 / 16, 1.0, g, cuda, torch.float16)
    w = qkv[1:].reshape(2 * heads * d, embed)
    x = dyadic((77, embed), 1 / 8, 2.0, g, cuda, torch.float32)
    codes, scales = nori_amd.project_quantize_kv(x, w, heads, d)
    ref_q, ref_s = torch_quantize(autocast_projection(x, w, heads, d))
    assert torch.equal(codes, ref_q) and torch.equal(scales, ref_s)
    # the shared-head weight: the first head's K and V rows only
    w1 = qkv[1:, 0].reshape(2 * d, embed).contiguous()
    codes1, scales1 = nori_amd.project_quantize_kv(x, w1, 1, d)
    assert torch.equal(codes1[:, :, 0], codes[:, :, 0]) and torch.equal(scales1[:, :, 0], scales[:, :, 0])


def test_row_slices_into_cache_storage(cuda):
    # rows [B, n, G, E] of a layer, written slice by slice into a [B*G, N, 2, H, D] payload, as
    # the bounded builds do; B = 2 needs three addressing levels (one launch per batch row)
    g = torch.Generator(device=cuda).manual_seed(11)
    b, n, grp, embed, heads, d = 2, 300, 5, 96, 2, 44
    x = torch.randn(b, n, grp, embed, generator=g, device=cuda)
    w = torch.randn(2 * heads * d, embed, generator=g, device=cuda) / embed ** 0.5
    whole_q, whole_s = nori_amd.project_quantize_kv(x.transpose(1, 2).contiguous(), w, heads, d, norm_eps=1e-5)
    payload = torch.full((b * grp, n, 2, heads, d), 99, dtype=torch.int8, device=cuda)
    scale = torch.full((b * grp, n, 2, heads, 1), -1.0, device=cuda)
    for r0, r1 in ((0, 64), (64, 65), (65, 300)):
        nori_amd.project_quantize_kv(
            x[:, r0:r1].transpose(1, 2), w, heads, d, norm_eps=1e-5,
            out=(payload[:, r0:r1].view(b, grp, r1 - r0, 2, heads, d),
                 scale[:, r0:r1].view(b, grp, r1 - r0, 2, heads, 1)),
        )
    assert torch.equal(payload, whole_q.view(b * grp, n, 2, heads, d))
    assert torch.equal(scale, whole_s.view(b * grp, n, 2, heads, 1))


def test_special_rows(cuda):
    # zero rows (scale = fp16(1e-12)/127 rounding), a row whose K/V overflow fp16 (inf -> NaN
    # scale handling as torch), and a single row
    heads, d, embed = 1, 16, 32
    w = torch.zeros(2 * d, embed, device=cuda)
    w[:d, 0] = 1.0
    w[d:, 1] = 1.0
    x = torch.zeros(3, embed, device=cuda)
    x[1, 0] = 7e4  # beyond fp16: K = inf
    x[2, 1] = 3.0
    codes, scales = nori_amd.project_quantize_kv(x, w, heads, d)
    ref_q, ref_s = torch_quantize(autocast_projection(x, w, heads, d))
    assert torch.equal(codes, ref_q)
    s, r = scales.cpu(), ref_s.cpu()
    assert torch.equal(torch.isnan(s), torch.isnan(r)) and torch.equal(s[~torch.isnan(s)], r[~torch.isnan(r)])
    one_q, one_s = nori_amd.project_quantize_kv(x[2:], w, heads, d)
    assert torch.equal(one_q, codes[2:]) and torch.equal(one_s, scales[2:])


def test_scale_and_reciprocal_over_every_f16_value(cuda):
    """The fused write's scale and reciprocal (nori_quant_f16_scale_probe) for all 65536 f16 bit
    patterns: s = f16(|m| / 127), the reference's scale (numpy's correctly rounded fp32 quotient,
    then f16), and y = the correctly rounded 1/s wherever the fast quotient uses it."""
    from nori_amd import _native as nat

    bits = torch.arange(65536, dtype=torch.int32).to(torch.int16).to(cuda)
    s = torch.empty(65536, device=cuda)
    y = torch.empty(65536, device=cuda)
    nat.check(nat.lib().nori_quant_f16_scale_probe(bits.data_ptr(), 65536, s.data_ptr(), y.data_ptr(),
                                                   nat.stream_of(cuda)), "quant_f16_scale_probe")
    m = np.abs(np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32))
    with np.errstate(divide="ignore", invalid="ignore"):
        s_ref = (m / np.float32(127)).astype(np.float16).astype(np.float32)
        y_ref = np.float32(1) / s_ref
    s, y = s.cpu().numpy(), y.cpu().numpy()
    nan = np.isnan(s_ref)
    assert np.array_equal(np.isnan(s), nan) and np.array_equal(s[~nan], s_ref[~nan])
    fast = (s_ref >= 2.0 ** -96) & (s_ref <= 2.0 ** 96)
    # every nonzero finite scale (absmax below 63.5 f16 subnormal steps gives scale 0)
    assert np.array_equal(fast, np.isfinite(s_ref) & (s_ref > 0)) and fast.sum() > 60000
    assert np.array_equal(y[fast].view(np.uint32), y_ref[fast].view(np.uint32))


@pytest.mark.parametrize("xdt", [torch.float16, torch.float32])
def test_every_f16_scale_codes_equal_the_exact_quantizer(cuda, xdt):
    """Identity weights make the K/V the operand values themselves (kv = x exactly), so each head
    vector's absmax can be chosen: every positive finite f16 value once, the other 43 values
    uniform in [-absmax, absmax] in f16. The fused write's codes and scales, and the HIP
    quantizer's on the same K/V, equal the reference expression on the same device (absmax below
    127 * 2^-14 gives a subnormal f16 scale, and quotients past 127 that only clamping brings
    back: absmax 128 * 2^-24 has scale 2^-24 and code 127, not -128). fp16 rows feed the MFMAs
    as they are; fp32 rows (the same values) take the one-pass kernel."""
    heads, d, embed = 8, 44, 352
    amax = torch.arange(1, 0x7C00, dtype=torch.int32).to(torch.int16).view(torch.float16).float()
    nv = amax.numel() + (-amax.numel()) % 8
    amax = torch.cat((amax, torch.ones(nv - amax.numel())))
    g = torch.Generator().manual_seed(5)
    vecs = (torch.rand(nv, d, generator=g) * 2 - 1) * amax[:, None]
    vecs[:, 0] = amax * torch.where(torch.rand(nv, generator=g) < 0.5, -1.0, 1.0)
    vecs = torch.gather(vecs, 1, torch.argsort(torch.rand(nv, d, generator=g), dim=1)).half()
    x = vecs.view(nv // 8, embed).to(cuda)
    w = torch.cat((torch.eye(embed), torch.eye(embed))).to(cuda)
    codes, scales = nori_amd.project_quantize_kv(x.to(xdt), w, heads, d)
    kv = torch.cat((x, x), dim=-1).view(nv // 8, 2, heads, d)
    ref_q, ref_s = torch_quantize(kv)
    bad = (codes != ref_q).any(-1).flatten().nonzero().flatten().cpu()
    if bad.numel():
        v = bad[:4]
        flat = kv.reshape(-1, d).cpu()
        detail = [(float(flat[i].abs().max()), float(scales.flatten()[i]), float(ref_s.flatten()[i]),
                   codes.reshape(-1, d)[i].cpu().tolist(), ref_q.reshape(-1, d)[i].cpu().tolist(),
                   flat[i].tolist()) for i in v.tolist()]
        raise AssertionError(f"{bad.numel()} head vectors differ; first: {detail}")
    assert torch.equal(scales, ref_s)
    hip_q, hip_s = nori_amd.quantize_int8(kv)
    assert torch.equal(hip_q, ref_q) and torch.equal(hip_s.view_as(ref_s), ref_s)


def test_one_pass_equals_the_operand_path_on_the_same_operands(cuda):
    """fp32 rows take the one-pass kernel (no workspace); without the norm its operands are
    f16(x), what fp16 rows feed the two-kernel path as they are, and its MFMA order is the
    same, so codes and scales agree bit for bit (ragged row count, a row slice view)."""
    from nori_amd import _native as nat

    lib = nat.lib()
    f32, f16 = nat.dtype_code(torch.float32), nat.dtype_code(torch.float16)
    assert lib.nori_kv_project_quantize_int8_workspace_bytes(f32, 3, 1000, 352, 1, f16, 44) == 0
    assert lib.nori_kv_project_quantize_int8_workspace_bytes(f32, 3, 1000, 352, 1, f32, 44) > 0
    assert lib.nori_kv_project_quantize_int8_workspace_bytes(f16, 3, 1000, 352, 1, f16, 44) > 0
    assert lib.nori_kv_project_quantize_int8_workspace_bytes(f32, 3, 1000, 392, 1, f16, 44) > 0  # embed > 384
    g = torch.Generator(device=cuda).manual_seed(11)
    x = torch.randn(3, 1000, 352, generator=g, device=cuda)[:, 3:]
    w = torch.randn(704, 352, generator=g, device=cuda) * 352 ** -0.5
    one_q, one_s = nori_amd.project_quantize_kv(x, w, 8, 44)
    op_q, op_s = nori_amd.project_quantize_kv(x.half(), w.half(), 8, 44)
    assert torch.equal(one_q, op_q) and torch.equal(one_s, op_s)


def test_large_row_count(cuda):
    # nori-30m's cross-cache write for one layer at a 64k context: 33 groups x 65536 rows of
    # E = 352 into 2 x 8 heads of 44; compared with the autocast path on a row sample
    g = torch.Generator(device=cuda).manual_seed(5)
    grp, n, embed, heads, d = 33, 65536, 352, 8, 44
    x = torch.randn(1, n, grp, embed, generator=g, device=cuda)
    w = torch.randn(2 * heads * d, embed, generator=g, device=cuda) / embed ** 0.5
    payload = torch.empty((grp, n, 2, heads, d), dtype=torch.int8, device=cuda)
    scale = torch.empty((grp, n, 2, heads, 1), device=cuda)
    nori_amd.project_quantize_kv(
        x.transpose(1, 2), w, heads, d, norm_eps=1e-5,
        out=(payload.view(1, grp, n, 2, heads, d), scale.view(1, grp, n, 2, heads, 1)),
    )
    rows = torch.randint(0, n, (256,), generator=g, device=cuda)
    xs = x[0, rows].transpose(0, 1)  # [grp, 256, E]
    ref_q, ref_s = torch_quantize(autocast_projection(xs, w, heads, d, 1e-5))
    assert_codes_close(payload[:, rows], scale[:, rows], ref_q, ref_s)


def _stack(gold, tag):
    from test_golden_layers import make_stack, weights

    stack = make_stack(gold, tag)
    stack.load_state_dict(weights(gold, tag), strict=True)
    return stack


@pytest.mark.parametrize("tag", ["stack", "stack_mqa"])
@pytest.mark.parametrize("mode", ["plain", "rowchunk", "stream", "hybrid"])
def test_int8_builds_fuse_the_cache_write(cuda, monkeypatch, tag, mode):
    from test_golden_layers import GOLDEN, ROW_CHUNK, check

    with np.load(GOLDEN, allow_pickle=False) as f:
        gold = {k: f[k] for k in f.files}
    stack = _stack(gold, tag).to(cuda)
    calls = []
    real = nori_amd.kv_project.project_quantize_kv

    def counting(*a, **k):
        calls.append(1)
        return real(*a, **k)

    def build(fused):
        x_train = torch.from_numpy(gold[f"{tag}/x_train"]).clone()
        if mode in ("plain", "rowchunk"):
            x_train = x_train.to(cuda)
        kwargs = dict(quantize_kv_cache=True, device=cuda, fused_cache_write=fused)
        if mode != "plain":
            kwargs.update(fit_row_chunk=ROW_CHUNK)
        if mode == "stream":
            kwargs.update(stream_context=True, offload_kv_cache=True)
        elif mode == "hybrid":
            kwargs.update(_hybrid_resident_int8_prefill=True)
        with monkeypatch.context() as m:
            m.setattr(nori_amd.kv_project, "project_quantize_kv", counting)
            with torch.inference_mode(), torch.autocast("cuda", dtype=torch.float16):
                out, caches = stack.build_train_cache(x_train, **kwargs)
                test_out = stack.forward_test_with_cache(torch.from_numpy(gold[f"{tag}/x_test"]).to(cuda), caches)
        return out, caches, test_out

    f_out, f_caches, f_test = build(True)
    assert calls, "fused_cache_write=True did not take the fused cache write"
    calls.clear()
    u_out, u_caches, u_test = build(False)
    assert not calls, "the default int8 build took the fused cache write"
    for fc, uc in zip(f_caches, u_caches):
        fk, uk = fc["seq_kv"], uc["seq_kv"]
        assert type(fk) is type(uk) and isinstance(fk, (ScalableSeqKV, BlockwiseSeqKV))
        if isinstance(fk, ScalableSeqKV):
            fq, fs = fk.device_payload()
            uq, us = uk.device_payload()
        else:
            fq = torch.cat([p for p, _ in fk.iter_payload_blocks()], dim=1)
            fs = torch.cat([s for _, s in fk.iter_payload_blocks()], dim=1)
            uq = torch.cat([p for p, _ in uk.iter_payload_blocks()], dim=1)
            us = torch.cat([s for _, s in uk.iter_payload_blocks()], dim=1)
        assert_codes_close(fq.to(cuda), fs.to(cuda), uq.to(cuda), us.to(cuda), max_frac=1e-2)
    check(f_test, u_test.float().cpu().numpy(), 1e-2)
    sfx = "int8" if mode == "plain" else f"{mode}_int8"
    check(f_test, gold[f"{tag}/test_out_{sfx}"])
    check(f_out, gold[f"{tag}/train_out_{sfx}"])


def test_default_int8_build_codes_equal_the_reference_expression_at_nori30m_dims(cuda, monkeypatch):
    # one nori-30m layer (embed 352, 8 heads of 44, hidden 1056) over 33 tokens x 1,024 context
    # rows: the default int8 build projects the cross cache with F.linear under fp16 autocast and
    # codes it with the HIP quantizer; codes and scales must be torch.equal to the reference
    # expression (kv_cache_scaling.py:29-37) applied by torch on this device to the fp16 K/V of
    # the same operand rows (layer.py:651-683)
    torch.manual_seed(0)
    layer = NL.EncoderBaseLayer(
        nhead=8, embed_dim=352, hid_dim=1056, pre_norm=True, activation="swiglu", layer_arch="smf",
        seq_attn_isolated=True, cross_share_all_kv_heads=False, use_qassmax=True, norm_type="rmsnorm",
        deepnorm_alpha=12 ** -0.5, qass_mode="full",
    ).eval().to(cuda)
    stack = NL.LayerStack([layer]).eval()
    operands = []
    real = NL.MultiheadAttention.project_kv_cache

    def capture(self, x_kv, **kw):
        operands.append((self, x_kv.detach().clone()))
        return real(self, x_kv, **kw)

    monkeypatch.setattr(NL.MultiheadAttention, "project_kv_cache", capture)
    fused_calls = []
    monkeypatch.setattr(nori_amd.kv_project, "project_quantize_kv", lambda *a, **k: fused_calls.append(1))
    x = torch.randn(1, 1024, 33, 352, device=cuda)
    with torch.inference_mode(), torch.autocast("cuda", dtype=torch.float16):
        _, caches = stack.build_train_cache(x, quantize_kv_cache=True, device=cuda)
        assert not fused_calls and len(operands) == 1
        mod, src = operands[0]
        w = mod.qkv_proj_weight[1:].reshape(2 * 8 * 44, 352)
        kv = F.linear(src.reshape(-1, *src.shape[-2:]), w).view(33, 1024, 2, 8, 44)
    assert kv.dtype == torch.float16
    exp_q, exp_s = torch_quantize(kv)
    got_q, got_s = caches[0]["seq_kv"].device_payload()
    assert got_q.shape == exp_q.shape and got_s.shape == exp_s.shape
    assert torch.equal(got_q, exp_q), f"{(got_q != exp_q).sum().item()} codes differ"
    assert torch.equal(got_s, exp_s), f"{(got_s != exp_s).sum().item()} scales differ"
    print(f"[parity] nori-30m default int8 build: {got_q.numel()} codes and {got_s.numel()} scales equal torch's",
          flush=True)
