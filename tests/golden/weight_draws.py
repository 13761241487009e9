"""Seeded weight draws for golden fixtures whose matrices are too large to store.

A fixture keeps each small tensor as it is and, for a matrix of ``DRAWN_MIN`` elements or more,
only its shape and a scale: the matrix is ``scale * N(0, 1)`` from numpy's PCG64 generator
seeded by the CRC-32 of the state-dict key (numpy's documented stream: the same numpy gives the
same draw on every machine). The fixture's script writes the draws into the reference model
before running it, and the tests rebuild the same state dict from the fixture.
"""

from __future__ import annotations

import zlib

import numpy as np

DRAWN_MIN = 4096


def draw(key: str, shape, scale: float) -> np.ndarray:
    rng = np.random.default_rng(zlib.crc32(key.encode()))
    return (rng.standard_normal(tuple(int(s) for s in shape)) * float(scale)).astype(np.float32)


def pack(state: dict[str, np.ndarray], prefix: str = "") -> tuple[dict[str, np.ndarray], dict[str, np.ndarray]]:
    """Split a state dict into what the fixture stores and the drawn matrices. Returns
    (arrays to store under ``prefix``, the full state dict with the draws in place). Each drawn
    matrix keeps the scale of the tensor it replaces (its standard deviation)."""
    stored: dict[str, np.ndarray] = {}
    full: dict[str, np.ndarray] = {}
    for k, w in state.items():
        w = np.asarray(w)
        if w.dtype == np.float32 and w.size >= DRAWN_MIN:
            scale = np.float32(w.std())
            full[k] = draw(k, w.shape, scale)
            stored[f"{prefix}shape.{k}"] = np.asarray(w.shape, dtype=np.int64)
            stored[f"{prefix}scale.{k}"] = np.asarray(scale)
        else:
            full[k] = w
            stored[f"{prefix}w.{k}"] = w
    return stored, full


def unpack(arrays: dict[str, np.ndarray], prefix: str = "") -> dict[str, np.ndarray]:
    """The state dict a fixture written by ``pack`` describes."""
    state: dict[str, np.ndarray] = {}
    for name, v in arrays.items():
        if not name.startswith(prefix):
            continue
        rest = name[len(prefix):]
        if rest.startswith("w."):
            state[rest[2:]] = v
        elif rest.startswith("shape."):
            k = rest[len("shape."):]
            state[k] = draw(k, v, arrays[f"{prefix}scale.{k}"])
    return state
