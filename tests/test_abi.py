"""The C-ABI library loads and exports every entry point include/nori_hip.h declares.

CPU only: no kernel is launched. Argument checks that fail before any device work are
exercised too, with the exception types the reference raises for the same mistakes.
"""

from __future__ import annotations

import ctypes
import os
import re

import pytest

from conftest import REPO_ROOT

HEADER = os.path.join(REPO_ROOT, "include", "nori_hip.h")


def declared_symbols() -> list[str]:
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(nori_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_expected_entry_points():
    assert declared_symbols() == sorted(
        [
            "nori_abi_version",
            "nori_last_error",
            "nori_kv_quantize_int8",
            "nori_kv_dequantize_int8",
            "nori_rms_norm",
            "nori_rms_norm_to",
            "nori_residual_add",
            "nori_silu_mul",
            "nori_swiglu_mlp",
            "nori_qass_gate",
            "nori_layer_norm",
            "nori_residual_add_rms_norm",
            "nori_icl_attention",
            "nori_icl_attention_qk",
            "nori_icl_attention_takes_prologue",
            "nori_icl_attention_workspace_size",
            "nori_icl_attention_noalloc",
            "nori_kv_project_quantize_int8",
            "nori_kv_project_quantize_int8_workspace_size",
            "nori_linear_f16",
            "nori_linear_f16_residual_rms_norm",
            "nori_cell_tokens",
            "nori_layer_norm_cells",
            "nori_swiglu_mlp_residual_rms_norm",
            "nori_mfma_f16_probe",
            "nori_mfma_f16_probe_flop",
            "nori_quant_f16_scale_probe",
            "nori_kv_project_quantize_int8_workspace_bytes",
        ]
    )


def test_library_exports_every_declared_symbol():
    from nori_amd import _native

    lib = ctypes.CDLL(_native.library_path())
    for name in declared_symbols():
        assert hasattr(lib, name), name
    assert set(declared_symbols()) == set(_native.SIGNATURES)
    assert _native.lib().nori_abi_version() == _native.ABI_VERSION == 3


def test_argument_errors_map_to_reference_exceptions():
    from nori_amd import _native as nat

    lib = nat.lib()
    # head width 0 -> NORI_ERR_INVALID -> ValueError, before any device call
    st = lib.nori_kv_quantize_int8(None, nat.NORI_BF16, 1, 1, 0, 0, 0, None, 0, 0, None, 0, 0, 1, None)
    assert st == nat.NORI_ERR_INVALID
    assert b"head width" in lib.nori_last_error()
    with pytest.raises(ValueError):
        nat.check(st, "quantize_int8")
    # int8 source is not a float dtype -> NotImplementedError
    st = lib.nori_kv_quantize_int8(None, nat.NORI_I8, 1, 1, 4, 4, 4, None, 0, 4, None, 0, 1, 1, None)
    assert st == nat.NORI_ERR_UNSUPPORTED
    with pytest.raises(NotImplementedError):
        nat.check(st, "quantize_int8")
    # attention: heads not divisible by kv heads / odd head width / empty cache
    args = [None, nat.NORI_BF16, 1, 1, 3, 64, 0, 0, 0, None, nat.NORI_I8, None, 8, 2, 0, 0, 0, 0, 0, 0, 1.0,
            None, nat.NORI_BF16, 0, 0, 0, None, 0, None, 0, None]
    assert lib.nori_icl_attention(*args) == nat.NORI_ERR_INVALID
    args[4], args[13] = 4, 2
    args[5] = 42
    assert lib.nori_icl_attention(*args) == nat.NORI_ERR_UNSUPPORTED
    args[5], args[12] = 64, 0
    assert lib.nori_icl_attention(*args) == nat.NORI_ERR_INVALID
    assert b"empty" in lib.nori_last_error()
    # fused projection + quantize: bad shape, head width not a multiple of 4, unknown dtype
    proj = [None, nat.NORI_F32, 1, 8, 64, 0, 64, 0, 0.0, None, nat.NORI_F32, 64, 2, 16,
            None, 0, 64, None, 0, 4, nat.SCALE_DIV_RECIP, None, 0, None]
    bad = list(proj); bad[13] = 0
    assert lib.nori_kv_project_quantize_int8(*bad) == nat.NORI_ERR_INVALID
    bad = list(proj); bad[13] = 18
    assert lib.nori_kv_project_quantize_int8(*bad) == nat.NORI_ERR_UNSUPPORTED
    assert b"head width" in lib.nori_last_error()
    bad = list(proj); bad[1] = nat.NORI_I8
    assert lib.nori_kv_project_quantize_int8(*bad) == nat.NORI_ERR_UNSUPPORTED
    bad = list(proj); bad[20] = 7
    assert lib.nori_kv_project_quantize_int8(*bad) == nat.NORI_ERR_INVALID
    bad = list(proj); bad[2] = 0
    assert lib.nori_kv_project_quantize_int8(*bad) == nat.NORI_OK  # no rows: nothing to do
    assert lib.nori_kv_project_quantize_int8(*proj) == nat.NORI_ERR_INVALID  # null pointers
    # operand-row workspace: f16 rows padded to 32, none when x is already f16 operands
    assert lib.nori_kv_project_quantize_int8_workspace_size(nat.NORI_F32, 3, 5, 44, 1) == 15 * 64 * 2
    assert lib.nori_kv_project_quantize_int8_workspace_size(nat.NORI_F16, 3, 5, 64, 0) == 0
    assert lib.nori_kv_project_quantize_int8_workspace_size(nat.NORI_F16, 3, 5, 64, 1) == 15 * 64 * 2
    # fused SwiGLU feed-forward: fp16 only, widths 128 / 256 / 352, hidden a multiple of 32
    mlp = [None, nat.NORI_F16, 4, 128, 128, None, None, 256, None, 128, None]
    bad = list(mlp); bad[1] = nat.NORI_BF16
    assert lib.nori_swiglu_mlp(*bad) == nat.NORI_ERR_UNSUPPORTED
    bad = list(mlp); bad[3] = bad[4] = bad[9] = 560
    assert lib.nori_swiglu_mlp(*bad) == nat.NORI_ERR_UNSUPPORTED
    assert b"width 560" in lib.nori_last_error()
    bad = list(mlp); bad[7] = 40
    assert lib.nori_swiglu_mlp(*bad) == nat.NORI_ERR_INVALID
    bad = list(mlp); bad[4] = 100
    assert lib.nori_swiglu_mlp(*bad) == nat.NORI_ERR_INVALID
    bad = list(mlp); bad[2] = 0
    assert lib.nori_swiglu_mlp(*bad) == nat.NORI_OK  # no rows: nothing to do
    assert lib.nori_swiglu_mlp(*mlp) == nat.NORI_ERR_INVALID  # null pointers
    # fused QASS gate: fp16 only, hidden 64, d a multiple of 4 up to 64
    qg = [None, nat.NORI_F16, 4, 10, 56, 560, None, None, None, None, 64, None, None, 560, None]
    bad = list(qg); bad[1] = nat.NORI_F32
    assert lib.nori_qass_gate(*bad) == nat.NORI_ERR_UNSUPPORTED
    bad = list(qg); bad[10] = 32
    assert lib.nori_qass_gate(*bad) == nat.NORI_ERR_UNSUPPORTED
    assert b"hidden width 32" in lib.nori_last_error()
    bad = list(qg); bad[4] = 68
    assert lib.nori_qass_gate(*bad) == nat.NORI_ERR_INVALID
    bad = list(qg); bad[4] = 54
    assert lib.nori_qass_gate(*bad) == nat.NORI_ERR_INVALID
    bad = list(qg); bad[5] = 500
    assert lib.nori_qass_gate(*bad) == nat.NORI_ERR_INVALID
    bad = list(qg); bad[2] = 0
    assert lib.nori_qass_gate(*bad) == nat.NORI_OK  # no rows: nothing to do
    assert lib.nori_qass_gate(*qg) == nat.NORI_ERR_INVALID  # null pointers
    # layer norm: float dtypes only, width a multiple of 4, eps a non-negative number
    ln = [None, nat.NORI_F16, 4, 128, 128, None, None, 1e-5, 0, None, nat.NORI_F32, 128, None]
    bad = list(ln); bad[1] = nat.NORI_I8
    assert lib.nori_layer_norm(*bad) == nat.NORI_ERR_UNSUPPORTED
    bad = list(ln); bad[3] = bad[4] = bad[11] = 126
    assert lib.nori_layer_norm(*bad) == nat.NORI_ERR_INVALID
    bad = list(ln); bad[7] = float("nan")
    assert lib.nori_layer_norm(*bad) == nat.NORI_ERR_INVALID
    bad = list(ln); bad[2] = 0
    assert lib.nori_layer_norm(*bad) == nat.NORI_OK
    assert lib.nori_layer_norm(*ln) == nat.NORI_ERR_INVALID  # null pointers
    # fp16 projection: inner width 128 or 256, output width a multiple of 4, aligned rows
    lin = [None, 1, 1, 4096, 128, 0, 0, 128, None, 128, 64, None, 0, 0, 64, None]
    bad = list(lin); bad[4] = 96
    assert lib.nori_linear_f16(*bad) == nat.NORI_ERR_UNSUPPORTED
    assert b"inner width 96" in lib.nori_last_error()
    bad = list(lin); bad[10] = 62
    assert lib.nori_linear_f16(*bad) == nat.NORI_ERR_UNSUPPORTED
    bad = list(lin); bad[10] = 0
    assert lib.nori_linear_f16(*bad) == nat.NORI_ERR_INVALID
    bad = list(lin); bad[3] = 0
    assert lib.nori_linear_f16(*bad) == nat.NORI_OK  # no rows: nothing to do
    assert lib.nori_linear_f16(*lin) == nat.NORI_ERR_INVALID  # null pointers
    # projection + residual + norm: width 128 or 256 (output width = inner width), aligned rows
    lrn = [None, 1, 1, 4096, 128, 0, 0, 128, None, 128, 0.5, None, 0, 0, 128, 1e-5, None, 0, 0, 128, None]
    bad = list(lrn); bad[4] = 64
    assert lib.nori_linear_f16_residual_rms_norm(*bad) == nat.NORI_ERR_UNSUPPORTED
    assert b"width 64" in lib.nori_last_error()
    bad = list(lrn); bad[4] = -1
    assert lib.nori_linear_f16_residual_rms_norm(*bad) == nat.NORI_ERR_INVALID
    bad = list(lrn); bad[3] = 0
    assert lib.nori_linear_f16_residual_rms_norm(*bad) == nat.NORI_OK  # no rows: nothing to do
    assert lib.nori_linear_f16_residual_rms_norm(*lrn) == nat.NORI_ERR_INVALID  # null pointers
    # SwiGLU + residual + norm: widths 128/128, 256/128, 256/256
    sr = [None, nat.NORI_F16, 64, 128, 128, None, None, 256, 0.3, None, 128, 128, 1e-5, None, 1, 128, 128, None]
    bad = list(sr); bad[11] = 64
    assert lib.nori_swiglu_mlp_residual_rms_norm(*bad) == nat.NORI_ERR_UNSUPPORTED
    bad = list(sr); bad[1] = nat.NORI_BF16
    assert lib.nori_swiglu_mlp_residual_rms_norm(*bad) == nat.NORI_ERR_UNSUPPORTED
    bad = list(sr); bad[7] = 100
    assert lib.nori_swiglu_mlp_residual_rms_norm(*bad) == nat.NORI_ERR_INVALID
    bad = list(sr); bad[2] = 0
    assert lib.nori_swiglu_mlp_residual_rms_norm(*bad) == nat.NORI_OK
    assert lib.nori_swiglu_mlp_residual_rms_norm(*sr) == nat.NORI_ERR_INVALID  # null pointers
    # the cells' last LayerNorm with the positional and target-aware additions
    lc = [None, nat.NORI_F16, 2, 64, 4, 128, 128, None, None, 1e-5, None, None, 32, None, 0.088, None, None]
    bad = list(lc); bad[5] = 96
    assert lib.nori_layer_norm_cells(*bad) == nat.NORI_ERR_UNSUPPORTED
    bad = list(lc); bad[1] = nat.NORI_BF16
    assert lib.nori_layer_norm_cells(*bad) == nat.NORI_ERR_UNSUPPORTED
    bad = list(lc); bad[12] = 65
    assert lib.nori_layer_norm_cells(*bad) == nat.NORI_ERR_INVALID
    bad = list(lc); bad[2] = 0
    assert lib.nori_layer_norm_cells(*bad) == nat.NORI_OK  # no tables: nothing to do
    assert lib.nori_layer_norm_cells(*lc) == nat.NORI_ERR_INVALID  # null pointers
    # cell tokens: 16 or 32 RBF kernels, 96 RBF outputs, 32 PLE bins
    ct = [None, 2, 64, 4, 2, 16, None, None, None, None, None, 1e-5, None, None, 96, None, 32, None, None, None]
    bad = list(ct); bad[5] = 24
    assert lib.nori_cell_tokens(*bad) == nat.NORI_ERR_UNSUPPORTED
    assert b"24 kernels" in lib.nori_last_error()
    bad = list(ct); bad[16] = 16
    assert lib.nori_cell_tokens(*bad) == nat.NORI_ERR_UNSUPPORTED
    bad = list(ct); bad[3] = 0
    assert lib.nori_cell_tokens(*bad) == nat.NORI_ERR_INVALID
    bad = list(ct); bad[2] = 0
    assert lib.nori_cell_tokens(*bad) == nat.NORI_OK  # no rows: nothing to do
    assert lib.nori_cell_tokens(*ct) == nat.NORI_ERR_INVALID  # null pointers
    # the MFMA rate probe (measurement only): operands, a sink and iterations are required
    assert lib.nori_mfma_f16_probe(None, 0, 1, None, 0, None) == nat.NORI_ERR_INVALID
    assert b"mfma_f16_probe" in lib.nori_last_error()
    # the scale probe: no values is no work; values need device pointers
    assert lib.nori_quant_f16_scale_probe(None, 0, None, None, None) == nat.NORI_OK
    assert lib.nori_quant_f16_scale_probe(None, 4, None, None, None) == nat.NORI_ERR_INVALID
    assert lib.nori_quant_f16_scale_probe(None, -1, None, None, None) == nat.NORI_ERR_INVALID
    # empty inputs are a no-op, not an error
    assert lib.nori_kv_quantize_int8(None, nat.NORI_F16, 0, 5, 8, 0, 8, None, 0, 8, None, 0, 1, 1, None) == nat.NORI_OK
    assert lib.nori_rms_norm(None, nat.NORI_F16, 0, 128, 128, None, nat.NORI_F16, 1e-5, None, 128, None) == nat.NORI_OK
    f = lib.nori_rms_norm_to
    assert f(None, nat.NORI_F32, 0, 128, 128, None, nat.NORI_F32, 1e-5, None, nat.NORI_F16, 128, None) == nat.NORI_OK
    # only fp32 rows narrow; an fp16 row is not widened or re-rounded to bf16
    assert f(None, nat.NORI_F16, 0, 128, 128, None, nat.NORI_F16, 1e-5, None, nat.NORI_BF16, 128, None) == nat.NORI_ERR_UNSUPPORTED


def test_operators_refuse_cpu_tensors():
    import torch

    import nori_amd

    t = torch.randn(2, 3, 2, 1, 8)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        nori_amd.quantize_int8(t)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        nori_amd.rms_norm(torch.randn(4, 8), 8)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        nori_amd.icl_attention(torch.randn(2, 3, 1, 8), t)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        nori_amd.project_quantize_kv(torch.randn(5, 32), torch.randn(64, 32), 2, 16)
    from nori_amd.norm import qass_gate

    h16 = lambda *shape: torch.randn(*shape).half()  # noqa: E731
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        qass_gate(h16(1, 8, 2, 56), h16(64, 56), h16(64), h16(56, 64), h16(56), h16(2, 56))
    with pytest.raises(ValueError, match="do not match"):  # the gate's hidden width is 64
        qass_gate(h16(1, 8, 2, 56), h16(32, 56), h16(32), h16(56, 32), h16(56), h16(2, 56))


def test_fused_projection_shape_errors():
    import torch

    import nori_amd

    with pytest.raises(ValueError, match="weight"):
        nori_amd.project_quantize_kv(torch.randn(5, 32), torch.randn(60, 32), 2, 16)
    with pytest.raises(ValueError, match="embed width"):
        nori_amd.project_quantize_kv(torch.randn(5, 48), torch.randn(64, 32), 2, 16)


def test_qk_prologue_only_on_the_short_context_path():
    """nori_icl_attention_qk refuses (NORI_ERR_UNSUPPORTED, nothing launched) the shapes the
    planner sends to the ring MFMA kernel -- for one table, every shape but the short-context
    ones, which attention.short_context() mirrors -- and int8 caches with a key norm; otherwise
    it goes on to the ordinary argument checks (here the null pointers), all before any device
    call. nori_icl_attention_takes_prologue gives the same answer without a call."""
    import ctypes

    from nori_amd import _native as nat
    from nori_amd.attention import short_context

    lib = nat.lib()
    pro = nat.QKPrologue(None, None, nat.NORI_F32, 1e-6, 1.0)
    for nq, nk in ((4, 6), (64, 32), (65, 1), (16, 128), (16, 129), (32, 64), (33, 64), (1, 1)):
        rc = lib.nori_icl_attention_qk(
            None, nat.NORI_F16, 1, nq, 2, 64, 0, 0, 0, None, nat.NORI_F16, None, nk, 2, 0, 0, 128, 0, 0, 0, 0.125,
            None, nat.NORI_F16, 0, 0, 0, None, 0, None, 0, ctypes.addressof(pro), None,
        )
        assert rc == (nat.NORI_ERR_INVALID if short_context(nq, nk) else nat.NORI_ERR_UNSUPPORTED), (nq, nk, rc)
        assert lib.nori_icl_attention_takes_prologue(1, nq, 2, 64, nk, nat.NORI_F16, 0, nat.NORI_F16) == int(
            short_context(nq, nk))
    keyed = nat.QKPrologue(None, 1, nat.NORI_F32, 1e-6, 1.0)  # any non-null gain pointer
    rc = lib.nori_icl_attention_qk(
        None, nat.NORI_F16, 1, 4, 2, 64, 0, 0, 0, None, nat.NORI_I8, None, 6, 2, 0, 0, 128, 0, 0, 0, 0.125,
        None, nat.NORI_F16, 0, 0, 0, None, 0, None, 0, ctypes.addressof(keyed), None,
    )
    assert rc == nat.NORI_ERR_UNSUPPORTED
