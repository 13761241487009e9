"""Exact graph replay of the cached query layers (nori_amd.graphs; the reference's
SYNTHEFY_EXACT_CACHED_CUDAGRAPHS=1 mode, predictor.py:74, 2394-2482).

The nori-6m case's model (tests/regressor_case.py) builds a context cache on its table; its
query rows are then applied eagerly and through the captured HIP graphs of every layer. The
graphs must give the eager outputs bit for bit: on every replay, with eager work and
synchronizations of the program's own between the replays, for fp16 autocast and fp32, int8 and
full-precision caches, and for new query rows of the same shape copied into the captured inputs;
a new cache is captured anew. Through NoriRegressor with the switch on, members run one at a
time (as in the reference's exact mode) and the predictions equal the eager one-at-a-time run.
"""

from __future__ import annotations

import json
import os
import warnings

import numpy as np
import pytest
import torch

import regressor_case as case
from nori_amd import api, graphs
from nori_amd.memory_policy import CacheQuantizedWarning
from nori_amd.transformer import FeaturesTransformer

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "regressor_goldens.npz")


@pytest.fixture(scope="module")
def model(cuda):
    with np.load(GOLDEN, allow_pickle=False) as f:
        scales = json.loads(str(f["case/weight_scales"]))
    return case.seeded_model(FeaturesTransformer, api.NORI_6M_CONFIG, scales).to(cuda)


@pytest.mark.parametrize("amp", [True, False])
@pytest.mark.parametrize("cache_dtype", ["int8", "bf16"])
def test_layer_graphs_replay_the_eager_bits(model, cuda, amp, cache_dtype):
    x_tr, y_tr, x_te, _ = case.table()
    y = torch.from_numpy(((y_tr - y_tr.mean()) / y_tr.std()).astype(np.float32))[None].to(cuda)
    xc = torch.from_numpy(x_tr)[None].to(cuda)
    q1 = torch.from_numpy(x_te)[None].to(cuda)
    q2 = torch.from_numpy(np.random.default_rng(3).standard_normal(x_te.shape).astype(np.float32))[None].to(cuda)
    print(f"graphs: amp {amp}, {cache_dtype} cache", flush=True)
    try:
        with torch.inference_mode(), torch.autocast("cuda", dtype=torch.float16, enabled=amp):
            ctx = model.build_context_cache(xc, y, cache_dtype=cache_dtype)
            eager1 = model.apply_context_cache(q1, ctx)
            eager2 = model.apply_context_cache(q2, ctx)
            replayers = graphs.enable_cached_graphs(model)
            for rep in range(3):
                got = model.apply_context_cache(q1, ctx)
                noise = torch.randn(1 << 20, device=cuda).sum()  # eager work between replays
                torch.cuda.synchronize()
                assert torch.equal(got, eager1), f"replay {rep} differs from the eager run"
                assert torch.isfinite(noise)
            assert torch.equal(model.apply_context_cache(q2, ctx), eager2)
            assert all(r.captures == 1 and r.replays >= 4 for r in replayers)
            # a new cache (another context) is captured anew and matches its own eager run
            ctx2 = model.build_context_cache(xc[:, :512], y[:, :512], cache_dtype=cache_dtype)
            graphs.disable_cached_graphs(model)
            eager3 = model.apply_context_cache(q1, ctx2)
            graphs.enable_cached_graphs(model)
            assert torch.equal(model.apply_context_cache(q1, ctx2), eager3)
            assert torch.equal(model.apply_context_cache(q1, ctx), eager1)
    finally:
        graphs.disable_cached_graphs(model)


def test_regressor_exact_graph_mode_matches_eager_one_at_a_time(model, cuda, monkeypatch):
    x_tr, y_tr, x_te, _ = case.table()
    kwargs = dict(model=model, device=cuda, memory_policy={"cache_dtype": "int8"})
    with warnings.catch_warnings():
        warnings.simplefilter("ignore", CacheQuantizedWarning)
        monkeypatch.setattr(api, "MEMBER_BATCH", 1)
        eager = api.NoriRegressor(**kwargs).fit(x_tr, y_tr).predict(x_te)
        monkeypatch.setattr(api, "MEMBER_BATCH", 4)
        monkeypatch.setenv(graphs.EXACT_CACHED_GRAPHS_ENV, "1")
        reg = api.NoriRegressor(**kwargs).fit(x_tr, y_tr)
        first = reg.predict(x_te)
        second = reg.predict(x_te)
        history = reg.memory_report_["attempt_history"]
        assert all(a["path"] == "cached" and len(a["pipeline_ids"]) == 1 for a in history)
        layers = model.transformer_encoder.layers
        assert all(isinstance(layer.__dict__.get("forward_test_with_cache"), graphs.LayerGraphs) for layer in layers)
        monkeypatch.delenv(graphs.EXACT_CACHED_GRAPHS_ENV)
        reg.predict(x_te[:8])  # switch off: back to the eager layers
        assert not any(isinstance(layer.__dict__.get("forward_test_with_cache"), graphs.LayerGraphs)
                       for layer in layers)
    np.testing.assert_array_equal(first, eager)
    np.testing.assert_array_equal(second, eager)
