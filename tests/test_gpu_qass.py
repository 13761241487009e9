"""The fused QASS gate (nori_qass_gate) on the GPU.

QASSMaxScaling.forward in "full" mode (ref src/synthefy_nori/model/layer.py:316-456) under fp16
autocast: q * base_scale * (1 + tanh(gate_mlp(q))), gate_mlp = Linear(d, 64) -> GELU ->
Linear(64, d). Checked against

* the same module's separate torch ops on the GPU under autocast (the reference's own
  execution): every output within 4 fp16 ulps
  of its own value plus 2 ulps of the gate (2^-10 at 1 + tanh in [1, 2)) times |q * base_scale|:
  the kernel's two GEMMs sum in another order than hipBLASLt's, a hidden activation one ulp off
  moves the gate by about an ulp, and where 1 + tanh(g) nearly cancels (g << 0) that ulp is a
  large part of the output. 99.98 % of the outputs come out bit-identical; the test asks for
  90 %. (torch's own ops on a strided view of the same queries take other GEMM kernels and
  match their contiguous run only to 83 %, so the reference runs on the contiguous copy.)
* the kernel's output for q as a strided view, bit for bit its output for the contiguous copy;
* the module in fp32 on the CPU: within 1e-2 of max |out| (the fp16 chain against fp32);
* head widths 8 / 44 / 56 / 64, 1 and 10 heads, a row count that is not a multiple of the
  kernel's 32-row tiles, q as a strided view into a [rows, 3, heads, d] projection, and that
  the fused path is the one taken.
"""
import math

import pytest
import torch

import nori_amd.layer as layer_mod
from nori_amd.layer import QASSMaxScaling

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)


def _module(heads, d, seed):
    torch.manual_seed(seed)
    m = QASSMaxScaling(num_heads=heads, head_dim=d, qass_mode="full")
    with torch.no_grad():  # the reference zero-initializes the last layers: give the gate some work
        for mlp in (m.base_mlp, m.gate_mlp):
            for lin in (mlp[0], mlp[-1]):
                lin.weight.normal_(0.0, 1.0 / math.sqrt(lin.in_features))
                lin.bias.normal_(0.0, 0.3)
    return m.eval()


def _compare(got, ref, qbs):
    got, ref, qbs = got.double(), ref.double(), qbs.double()
    tol = 4 * 2.0**-11 * ref.abs() + 2 * 2.0**-10 * qbs.abs() + 4 * 2.0**-24
    worst = float(((got - ref).abs() / tol).max())
    same = float((got == ref).double().mean())
    return worst, same


@pytest.mark.parametrize("heads,d", [(10, 56), (1, 64), (4, 44), (2, 8)])
def test_fused_gate_against_the_separate_ops(monkeypatch, heads, d):
    m = _module(heads, d, seed=heads * 100 + d).to(DEV)
    g = torch.Generator().manual_seed(d)
    rows = 1000
    qkv = (torch.randn(rows, 3, heads, d, generator=g) * 2.0).half().to(DEV)
    calls = []
    real = layer_mod.qass_gate
    monkeypatch.setattr(layer_mod, "qass_gate", lambda *a: calls.append(1) or real(*a))
    contiguous = qkv[:, 0].contiguous().view(1, rows, heads, d)
    strided = qkv[:, 0].unsqueeze(0)
    print(f"qass gate heads {heads} d {d} q strides {tuple(strided.stride())}", flush=True)
    with torch.inference_mode(), torch.autocast("cuda", dtype=torch.float16):
        m.fused = True
        got = m(contiguous, 8192)
        got_strided = m(strided, 8192)
        m.fused = False
        ref = m(contiguous, 8192)
        m.qass_mode = "base_only"  # q * base_scale alone, for the error bound
        qbs = m(contiguous, 8192)
        m.qass_mode = "full"
    torch.cuda.synchronize()
    assert len(calls) == 2
    assert got.dtype == torch.float16 and got.shape == contiguous.shape
    worst, same = _compare(got, ref, qbs)
    print(f"  vs separate ops: worst {worst:.2f} of the bound, {same:.4f} bit-identical", flush=True)
    assert worst <= 1.0 and same >= 0.9
    assert torch.equal(got_strided, got)

    cpu = _module(heads, d, seed=heads * 100 + d)
    with torch.no_grad():
        exp = cpu(qkv[:, 0].unsqueeze(0).float().cpu(), 8192)
    err = float((got.float().cpu() - exp).abs().max() / exp.abs().max())
    print(f"  vs fp32 CPU: {err:.3e}", flush=True)
    assert err <= 1e-2


def test_fused_gate_at_the_config4_launch():
    """One config-4 build sub-batch's queries (8.4 M vectors: 102 x 8192 rows, 10 heads of 56):
    every output against the separate ops within the same bound, and the bit-identical share."""
    m = _module(10, 56, seed=7).to(DEV)
    q = torch.randn(102, 8192, 10, 56, device=DEV, dtype=torch.float16) * 2.0
    print("qass gate at [102, 8192, 10, 56]", flush=True)
    with torch.inference_mode(), torch.autocast("cuda", dtype=torch.float16):
        m.fused = True
        got = m(q, 8192)
        m.fused = False
        ref = m(q, 8192)
        m.qass_mode = "base_only"
        qbs = m(q, 8192)
        m.qass_mode = "full"
    torch.cuda.synchronize()
    worst, same = 0.0, 0
    for i in range(0, 102, 17):  # in slices: the float64 bound of the whole tensor is 6 GB per term
        w, sm = _compare(got[i:i + 17], ref[i:i + 17], qbs[i:i + 17])
        worst, same = max(worst, w), same + sm * 17 / 102
    print(f"  vs separate ops: worst {worst:.2f} of the bound, {same:.4f} bit-identical", flush=True)
    assert worst <= 1.0 and same >= 0.9


def test_single_key_and_fp32_queries_keep_the_torch_path(monkeypatch):
    m = _module(2, 32, seed=5).to(DEV)
    monkeypatch.setattr(layer_mod, "qass_gate", lambda *a: pytest.fail("fused gate taken"))
    q = torch.randn(64, 2, 32, device=DEV)
    with torch.inference_mode():
        assert torch.equal(m(q.half(), 1), q.half())  # one key: q unscaled
        out = m(q, 100)  # fp32 queries without autocast: the separate ops
    assert out.dtype == torch.float32
