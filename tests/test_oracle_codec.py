"""Pins the C oracle of the int8 cache codec (oracle/nori_oracle.c) on the CPU.

The oracle restates quantize_int8 / dequantize_int8 (reference
src/synthefy_nori/model/kv_cache_scaling.py:29-41) with torch's per-op rounding. It is
held to checks that would catch a dropped rounding step, a wrong rounding direction, a
transposed axis or a wrong clamp:

* its fp16/bf16 rounding primitives against numpy and torch conversions, exhaustively
  over every 16-bit pattern and on random fp32 values around every rounding boundary;
* its quantizer against torch's own CPU execution of the reference expression, bit for
  bit, for every source dtype;
* both scale modes against an exact-rational restatement (Python Fractions) of the
  same steps;
* hand-computed known answers, including the bf16 double rounding case;
* the invariants the reference's tests state (test_kv_cache_scaling.py:17-22, 60-78).
"""

from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import codec

RNG = np.random.default_rng(1234)


# ----------------------------------------------------------------------------- helpers
def torch_reference_quantize(t: torch.Tensor):
    """The reference expression, executed by torch on the CPU (kv_cache_scaling.py:35-37)."""
    scale = t.abs().amax(dim=-1, keepdim=True).clamp_min(1e-12) / 127.0
    q = torch.clamp(torch.round(t / scale), -127, 127).to(torch.int8)
    return q, scale.to(torch.float32)


def to_oracle_input(t: torch.Tensor) -> tuple[np.ndarray, str]:
    if t.dtype == torch.float32:
        return t.numpy(), "f32"
    if t.dtype == torch.float16:
        return t.numpy(), "f16"
    return t.view(torch.int16).numpy().view(np.uint16), "bf16"


def sample_cache(shape, dtype, outlier_frac=0.02, seed=0):
    g = torch.Generator().manual_seed(seed)
    t = torch.randn(*shape, generator=g)
    d = shape[-1]
    n_out = max(1, round(outlier_frac * d))
    ch = torch.randperm(d, generator=g)[:n_out]
    t[..., ch] *= 8.0
    return t.to(dtype)


def rne(x: Fraction, p: int, emin: int, emax: int) -> Fraction:
    """Round x to nearest even in a binary format with p-bit significands (exact rationals)."""
    if x == 0:
        return Fraction(0)
    sign = -1 if x < 0 else 1
    a = abs(x)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    e = max(e, emin)
    ulp = Fraction(2) ** (e - p + 1)
    n, rem = divmod(a, ulp)
    if rem > ulp / 2 or (rem == ulp / 2 and n % 2 == 1):
        n += 1
    r = n * ulp
    if r >= Fraction(2) ** (emax + 1):
        return Fraction(sign * 10**400)  # overflow marker (never reached by the cases below)
    return sign * r


FMT = {"f32": (24, -126, 127), "f16": (11, -14, 15), "bf16": (8, -126, 127)}


def fraction_quantize(values: list[float], dtype: str, recip: bool) -> tuple[list[int], Fraction]:
    """Exact-rational restatement of the quantizer for one vector (no NaN/inf inputs)."""
    p, emin, emax = FMT[dtype]
    rt = lambda v: rne(v, p, emin, emax)  # noqa: E731
    r32 = lambda v: rne(v, 24, -126, 127)  # noqa: E731
    t = [Fraction(v) for v in values]
    m = max(abs(v) for v in t)
    lo = rt(r32(Fraction(1e-12)))
    if m < lo:
        m = lo
    if recip:
        s = rt(r32(m * r32(Fraction(1) / 127)))
    else:
        s = rt(r32(m / 127))
    codes = []
    for v in t:
        if s == 0:  # fp16 scale underflow: t/0 is +-inf (clamped to +-127) or 0/0 = NaN (code 0)
            codes.append(0 if v == 0 else (127 if v > 0 else -127))
            continue
        q = rt(r32(v / s))
        k = round(q)  # Python rounds half to even
        codes.append(max(-127, min(127, int(k))))
    return codes, s


# ----------------------------------------------------------------------------- rounding
def test_f16_rounding_matches_numpy_on_every_pattern_and_boundary():
    # every fp16 pattern round-trips, and the midpoints between neighbours round to even
    h = np.arange(0, 0x10000, dtype=np.uint32).astype(np.uint16)
    f = h.view(np.float16).astype(np.float32)
    finite = np.isfinite(f)
    assert np.array_equal(codec.f32_to_f16_bits(f[finite]), h[finite])
    with np.errstate(invalid="ignore", over="ignore"):
        mids = (f[:-1].astype(np.float64) + f[1:].astype(np.float64)) / 2
    ok = np.isfinite(mids) & (np.abs(mids) < 65504.0)
    for delta in (-1e-12, 0.0, 1e-12):
        x = (mids[ok] * (1 + delta)).astype(np.float32)
        assert np.array_equal(codec.f32_to_f16_bits(x), x.astype(np.float16).view(np.uint16))
    x = RNG.standard_normal(2_000_000).astype(np.float32) * np.float32(2.0) ** RNG.integers(-30, 20, 2_000_000)
    with np.errstate(over="ignore"):
        expected = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(codec.f32_to_f16_bits(x), expected)


def test_bf16_rounding_matches_torch():
    x = RNG.standard_normal(2_000_000).astype(np.float32) * np.float32(2.0) ** RNG.integers(-120, 120, 2_000_000)
    # add exact bf16 midpoints (ties) and their neighbours
    b = RNG.integers(0, 0x7F7F, 100_000).astype(np.uint32)
    ties = ((b << 16) | 0x8000).view(np.float32)
    x = np.concatenate([x, ties, np.nextafter(ties, np.float32(np.inf)), np.nextafter(ties, np.float32(0))])
    expected = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(codec.f32_to_bf16_bits(x), expected)


# ----------------------------------------------------------------------------- quantize
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("d", [4, 8, 16, 44, 56, 64])
def test_quantize_matches_torch_cpu_expression(dtype, d):
    t = sample_cache((3, 97, 2, 2, d), dtype, seed=d)
    # extra rows: tiny magnitudes, exact ties and a large range
    t[0, 0] = (torch.arange(d, dtype=torch.float32) * 1e-9).to(dtype)
    t[0, 1] = (torch.arange(d, dtype=torch.float32) - d / 2).to(dtype) * 0.5
    t[0, 2] = (torch.randn(d) * 1e4).to(dtype)
    ref_q, ref_s = torch_reference_quantize(t)
    raw, name = to_oracle_input(t)
    q, s = codec.quantize_int8(raw, name, codec.DIV_TRUE)
    assert np.array_equal(q, ref_q.numpy())
    assert np.array_equal(s.view(np.uint32), ref_s.numpy().view(np.uint32))


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("recip", [False, True])
def test_quantize_matches_exact_rational_restatement(dtype, recip):
    rng = np.random.default_rng(7 if recip else 8)
    for trial in range(40):
        d = int(rng.integers(1, 20))
        v = rng.standard_normal(d) * 10.0 ** rng.integers(-6, 4)
        if dtype == "f32":
            raw = v.astype(np.float32)
            vals = [float(x) for x in raw]
        elif dtype == "f16":
            raw = v.astype(np.float16)
            vals = [float(x) for x in raw.astype(np.float32)]
        else:
            raw = codec.f32_to_bf16_bits(v.astype(np.float32))
            vals = [float(x) for x in codec.bf16_bits_to_f32(raw)]
        q, s = codec.quantize_int8(raw[None, :], dtype, codec.DIV_RECIP if recip else codec.DIV_TRUE)
        exp_codes, exp_s = fraction_quantize(vals, dtype, recip)
        assert list(q[0]) == exp_codes, (trial, vals)
        assert Fraction(float(s[0, 0])) == exp_s


def test_known_answers_bf16_double_rounding():
    # amax 1.046875 -> s = bf16(1.046875/127) = 135 * 2^-14; 1.0/s = 121.3630 -> bf16 121.5 -> 122.
    bits = codec.f32_to_bf16_bits(np.array([[1.046875, 1.0]], dtype=np.float32))
    q, s = codec.quantize_int8(bits, "bf16", codec.DIV_TRUE)
    assert q.tolist() == [[127, 122]]
    assert float(s[0, 0]) == 135 * 2.0**-14
    # the other direction: 1.0078125 / s(1.0625) = 120.5256 -> bf16 120.5 -> ties to even 120
    bits = codec.f32_to_bf16_bits(np.array([[1.0625, 1.0078125]], dtype=np.float32))
    q, _ = codec.quantize_int8(bits, "bf16", codec.DIV_TRUE)
    assert q.tolist() == [[127, 120]]
    # fp32 keeps no such rounding: 1.0 / (1.046875/127) = 121.3134 -> 121
    q, _ = codec.quantize_int8(np.array([[1.046875, 1.0]], dtype=np.float32), "f32", codec.DIV_TRUE)
    assert q.tolist() == [[127, 121]]


def test_known_answers_special_vectors():
    # all-zero vector: fp32/bf16 use the 1e-12 floor -> codes 0; fp16's floor is 0 -> 0/0 = NaN -> code 0
    for name, raw in (
        ("f32", np.zeros((1, 4), np.float32)),
        ("bf16", np.zeros((1, 4), np.uint16)),
        ("f16", np.zeros((1, 4), np.float16)),
    ):
        q, s = codec.quantize_int8(raw, name, codec.DIV_TRUE)
        assert q.tolist() == [[0, 0, 0, 0]]
        if name == "f16":
            assert float(s[0, 0]) == 0.0
        else:
            assert float(s[0, 0]) > 0.0
    # scale floor in fp32: 1e-12 / 127
    q, s = codec.quantize_int8(np.array([[1e-15, -1e-15]], np.float32), "f32", codec.DIV_TRUE)
    assert float(s[0, 0]) == float(np.float32(np.float32(1e-12) / np.float32(127.0)))
    # NaN anywhere in a vector -> NaN scale, all codes 0
    q, s = codec.quantize_int8(np.array([[1.0, np.nan, -2.0]], np.float32), "f32", codec.DIV_RECIP)
    assert q.tolist() == [[0, 0, 0]] and np.isnan(s[0, 0])


def test_gpu_scale_mode_differs_from_cpu_only_in_the_scale_rounding():
    # m * fp32(1/127) and m / 127 differ for some amax values; find one and check both modes
    m = np.float32(1.0) + np.arange(1, 50000, dtype=np.float32) * np.float32(2.0**-23)
    div = (m / np.float32(127.0)).astype(np.float32)
    mul = (m * np.float32(1.0 / 127.0)).astype(np.float32)
    idx = np.nonzero(div != mul)[0]
    assert len(idx) > 0
    v = np.array([[m[idx[0]], 0.5]], dtype=np.float32)
    _, s_cpu = codec.quantize_int8(v, "f32", codec.DIV_TRUE)
    _, s_gpu = codec.quantize_int8(v, "f32", codec.DIV_RECIP)
    assert s_cpu[0, 0] == div[idx[0]] and s_gpu[0, 0] == mul[idx[0]]


# ----------------------------------------------------------------------------- invariants
@pytest.mark.parametrize("name", ["f32", "f16", "bf16"])
def test_invariants_absmax_maps_to_127_and_row_slices_are_independent(name):
    t = sample_cache((4, 257, 2, 3, 16), torch.float32, seed=3)
    raw = t.numpy() if name == "f32" else (t.numpy().astype(np.float16) if name == "f16" else codec.f32_to_bf16_bits(t.numpy()))
    q, s = codec.quantize_int8(raw, name, codec.DIV_RECIP)
    assert np.abs(q.astype(np.int32)).max() <= 127
    vals = raw.astype(np.float32) if name != "bf16" else codec.bf16_bits_to_f32(raw)
    arg = np.abs(vals).argmax(axis=-1)
    picked = np.abs(np.take_along_axis(q, arg[..., None], axis=-1).astype(np.int32))
    if name == "bf16":
        # bf16 rounds the scale to 8 bits, so amax/scale can land on 126.75 -> bf16 126.5 -> 126;
        # torch's own bf16 evaluation does the same (about 8% of N(0,1) vectors).
        assert set(np.unique(picked)) <= {126, 127}
    else:
        assert np.all(picked == 127)
    # slice invariance (test_kv_cache_scaling.py:60-78): quantizing row chunks == whole tensor
    parts = [codec.quantize_int8(raw[:, i : i + 64], name, codec.DIV_RECIP) for i in range(0, raw.shape[1], 64)]
    assert np.array_equal(np.concatenate([p[0] for p in parts], axis=1), q)
    assert np.array_equal(np.concatenate([p[1] for p in parts], axis=1), s)


def test_roundtrip_relative_error_below_two_percent():
    # test_kv_cache_scaling.py:17-22
    t = torch.randn(4, 100, 2, 3, 16)
    q, s = codec.quantize_int8(t.numpy(), "f32")
    back = codec.dequantize_int8(q, s, "f32")
    rel = np.abs(back - t.numpy()).max() / np.abs(t.numpy()).max()
    assert rel < 0.02


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_dequantize_matches_torch_cpu_expression(dtype):
    t = sample_cache((2, 33, 2, 2, 44), torch.float32, seed=11)
    q, s = torch_reference_quantize(t)
    expected = (q.to(torch.float32) * s).to(dtype)
    name = {torch.float32: "f32", torch.float16: "f16", torch.bfloat16: "bf16"}[dtype]
    got = codec.dequantize_int8(q.numpy(), s.numpy(), name)
    if dtype == torch.bfloat16:
        assert np.array_equal(got, expected.view(torch.int16).numpy().view(np.uint16))
    else:
        assert np.array_equal(got.view(np.uint16 if dtype == torch.float16 else np.uint32),
                              expected.numpy().view(np.uint16 if dtype == torch.float16 else np.uint32))
