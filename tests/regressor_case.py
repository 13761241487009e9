"""The nori-6m end-to-end case: a seeded random-init nori-6m model and its synthetic table.

Shared by tests/golden/make_regressor_golden.py, which runs the reference's own model on it,
and the tests that hold this package's NoriRegressor to the reference's outputs. The model's
weights are a pure function of a per-parameter (mean, std) table stored with the fixture and
numpy's integer-based random stream (checked by their SHA-256 against the fixture), so no
weights need to be stored.

Table: 1024 context + 256 query rows of 16 float32 features X ~ N(0, 1), target
y = X w + 0.5 sin(X[:, 0]) + 0.1 N(0, 1) with w ~ N(0, 1/16); numpy's default_rng(0).
"""

from __future__ import annotations

import hashlib

import numpy as np
import torch

N_CONTEXT, N_QUERY, N_FEATURES = 1024, 256, 16
QUANTILE_LEVELS = (0.1, 0.5, 0.9)


def table():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((N_CONTEXT + N_QUERY, N_FEATURES)).astype(np.float32)
    w = rng.normal(0.0, 0.25, N_FEATURES)
    y = x.astype(np.float64) @ w + 0.5 * np.sin(x[:, 0].astype(np.float64)) + 0.1 * rng.standard_normal(len(x))
    return x[:N_CONTEXT], y[:N_CONTEXT], x[N_CONTEXT:], y[N_CONTEXT:]


def weight_scales(model) -> dict[str, tuple[float, float]]:
    """(mean, std) of every parameter as the constructor initialized it; std 0 for a constant
    (norm gains, zero biases, the scalar settings). Measured once by the golden recipe and
    stored with the fixture, so the weights below never depend on torch's random streams,
    whose vectorized paths differ from host CPU to host CPU."""
    out = {}
    for name, t in sorted(model.state_dict().items()):
        t = t.detach().double()
        flat = t.reshape(-1)
        if flat.numel() == 1 or bool((flat == flat[0]).all()):
            out[name] = (float(flat[0]), 0.0)
        else:
            out[name] = (float(flat.mean()), float(flat.std()))
    return out


def seeded_model(features_transformer_cls, config: dict, scales: dict[str, tuple[float, float]]):
    """nori-6m with every weight a pure function of ``scales`` and numpy's default_rng(0): each
    random parameter (sorted by name) is mean + std * sqrt(3) * (2u - 1) with u from
    ``Generator.random`` (doubles built from integers: the same bits on every machine), rounded
    once to fp32; constants keep their value. Two adjustments make the predictions depend on
    the inputs at O(1): the zero-initialized QASS output layers get small weights from the same
    stream, and the 999-level head's output layer gets a bias increasing over the levels and
    rows that share one direction (its first row x30 plus each row's own x3), so the collapsed
    mean moves with the input instead of averaging out."""
    model = features_transformer_cls(**config).eval()
    state = model.state_dict()
    rng = np.random.default_rng(0)
    new = {}
    for name in sorted(state):
        mean, std = scales[name]
        shape = tuple(state[name].shape)
        if std == 0.0:
            values = np.full(shape, mean, dtype=np.float64)
        else:
            values = mean + std * np.sqrt(3.0) * (2.0 * rng.random(shape) - 1.0)
        if ".qassmax." in name and name.rsplit(".", 2)[-2] == "2":  # the QASS MLPs' output layers
            values = 0.1 * np.sqrt(3.0) * (2.0 * rng.random(shape) - 1.0)
        new[name] = values
    head = f"reg_y_decoder.{len(model.reg_y_decoder) - 1}"
    n_levels = new[f"{head}.bias"].shape[0]
    new[f"{head}.bias"] = np.array([-2.0 + 4.0 * i / (n_levels - 1) for i in range(n_levels)])
    w = new[f"{head}.weight"]
    new[f"{head}.weight"] = w[:1] * 30.0 + w * 3.0
    model.load_state_dict({k: torch.from_numpy(v.astype(np.float32)) for k, v in new.items()}, strict=True)
    return model


def weights_sha256(model) -> str:
    """SHA-256 over the state dict: names in order, then each tensor's dtype, shape and bytes."""
    h = hashlib.sha256()
    for name, t in sorted(model.state_dict().items()):
        t = t.detach().cpu().contiguous()
        h.update(name.encode())
        h.update(str(t.dtype).encode())
        h.update(str(tuple(t.shape)).encode())
        h.update(t.numpy().tobytes())
    return h.hexdigest()
