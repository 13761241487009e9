"""Error figures shared by the parity tests.

``relative_error`` is the measure the prediction bar is stated in: the largest absolute
difference over the largest reference magnitude, max|got - exp| / max|exp|.
"""

from __future__ import annotations

import torch

# Relative error allowed on model predictions (quantiles and point predictions): 1e-3.
PREDICTION_BAR = 1e-3


def relative_error(got, exp) -> float:
    got = torch.as_tensor(got).detach().double().cpu()
    exp = torch.as_tensor(exp).double().cpu()
    scale = exp.abs().max().item()
    return (got - exp).abs().max().item() / (scale if scale > 0 else 1.0)


def check_relative(got, exp, bar: float, what: str) -> float:
    """Assert relative_error(got, exp) <= bar; prints the measured figure either way."""
    rel = relative_error(got, exp)
    print(f"[parity] {what}: relative error {rel:.3e} (bar {bar:.1e})", flush=True)
    assert rel <= bar, f"{what}: relative error {rel:.3e} exceeds {bar:.1e}"
    return rel
