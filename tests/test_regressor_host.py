"""Host-side parity of the NoriRegressor surface (no kernel runs here).

* The nori-6m case's weights: this package's seeded build hashes to the SHA-256 the golden
  recipe recorded for the weights it ran the reference with (tests/regressor_case.py).
* The quantile collapse (quantile_dist.py:95-135): equal to the reference's own output on the
  golden quantile bank, and pinned by closed forms -- a constant bank, the identity quantile
  function, invariance to the order of the bank.
* Quantiles read at the head's own levels are the sorted bank's columns; between levels they
  interpolate linearly (api.py:1330-1345).
* The memory-policy ladder: rung, precision, placement, budgets and footprints equal to the
  reference's MemoryPolicy.resolve on the same requests and sizes, refusals included, and
  the report carries every key of the reference's memory_report_.
* fit/predict argument errors, as the reference raises them.
"""

from __future__ import annotations

import json
import math
import os

import numpy as np
import pytest
import torch

import regressor_case as case
from nori_amd import api
from nori_amd.memory_policy import ContextTooLargeError, MemoryPolicy
from nori_amd.transformer import FeaturesTransformer

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "regressor_goldens.npz")


@pytest.fixture(scope="module")
def gold():
    with np.load(GOLDEN, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def test_seeded_nori_6m_weights_are_the_ones_the_reference_ran(gold):
    model = case.seeded_model(FeaturesTransformer, api.NORI_6M_CONFIG, json.loads(str(gold["case/weight_scales"])))
    assert case.weights_sha256(model) == str(gold["case/weights_sha256"])
    assert sum(p.numel() for p in model.parameters()) > 5_000_000  # nori-6m's size


def test_table_is_the_recorded_one(gold):
    x_tr, y_tr, x_te, y_te = case.table()
    for got, key in ((x_tr, "x_train"), (y_tr, "y_train"), (x_te, "x_test"), (y_te, "y_test")):
        assert np.array_equal(got, gold[f"case/{key}"])


def test_quantile_collapse_equals_the_reference_on_its_bank(gold):
    bank = torch.from_numpy(gold["case/bank_norm"]).double()
    taus = torch.from_numpy(gold["case/taus"])
    got = api.quantile_dist_mean(bank, taus).numpy()
    np.testing.assert_allclose(got, gold["case/point_norm"], rtol=0, atol=1e-12)


def test_quantile_collapse_closed_forms():
    taus = torch.tensor([(i + 1) / 1000.0 for i in range(999)], dtype=torch.float64)
    # a constant quantile function is that constant
    assert torch.allclose(api.quantile_dist_mean(torch.full((3, 999), 2.5, dtype=torch.float64), taus),
                          torch.full((3,), 2.5, dtype=torch.float64), rtol=0, atol=1e-12)
    # q(tau) = tau between the outer levels, flat outside: t0^2 + (t1^2 - t0^2) / 2 + (1 - t1) t1
    t0, t1 = 1e-3, 0.999
    exact = t0 * t0 + (t1 * t1 - t0 * t0) / 2 + (1 - t1) * t1
    assert abs(api.quantile_dist_mean(taus[None], taus).item() - exact) < 1e-12
    # the bank is sorted first: any order of the same values gives the same mean
    g = torch.Generator().manual_seed(0)
    q = torch.randn(5, 999, generator=g, dtype=torch.float64)
    perm = torch.randperm(999, generator=g)
    assert torch.allclose(api.quantile_dist_mean(q, taus), api.quantile_dist_mean(q[:, perm], taus), rtol=0, atol=1e-12)
    # half-precision banks integrate in fp32; a single level returns itself
    assert api.quantile_dist_mean(q.half(), taus).dtype == torch.float32
    assert torch.equal(api.quantile_dist_mean(q[:, :1], taus[:1]), q[:, 0])
    with pytest.raises(ValueError):
        api.quantile_dist_mean(q, taus.flip(0))


def test_quantiles_at_the_head_levels_are_bank_columns(gold):
    bank = np.sort(gold["case/bank_norm"].astype(np.float64), axis=1)
    taus = gold["case/taus"]
    got = api._interpolated_quantiles(bank, taus, np.asarray(case.QUANTILE_LEVELS))
    for i, level in enumerate(case.QUANTILE_LEVELS):
        assert np.array_equal(got[i], bank[:, int(round(level * 1000)) - 1])
    mid = api._interpolated_quantiles(bank, taus, np.asarray([0.1005]))[0]
    np.testing.assert_allclose(mid, 0.5 * (bank[:, 99] + bank[:, 100]), rtol=0, atol=1e-12)


def test_memory_ladder_matches_the_reference(gold):
    rows = json.loads(str(gold["ladder/json"]))
    ours_keys = set(MemoryPolicy().as_report())
    for row in rows:
        policy = MemoryPolicy.coerce(row["request"])
        args = dict(est_cache_gb=row["est"], bytes_per_element=row["bpe"], head_dim=row["head_dim"],
                    total_vram_gb=row["vram"], total_ram_gb=row["ram"])
        if "error" in row:
            assert row["error"] == "ContextTooLargeError"
            with pytest.raises(ContextTooLargeError):
                policy.resolve(**args)
            continue
        got = policy.resolve(**args).as_report()
        exp = row["report"]
        for key in ("rung", "cache", "cache_dtype", "offload_to_host", "reuse_context_cache", "context_row_chunk",
                    "stream_context", "allow_quantization"):
            assert got[key] == exp[key], (row["label"], key, got[key], exp[key])
        for key in ("est_cache_gb", "resident_gb", "gpu_budget_absolute_gb", "host_budget_absolute_gb"):
            if exp[key] is None:
                assert got[key] is None, (row["label"], key)
            else:
                assert math.isclose(got[key], exp[key], rel_tol=1e-12), (row["label"], key, got[key], exp[key])
        missing = set(row["report_keys"]) - ours_keys
        assert not missing, f"report lacks the reference's keys {sorted(missing)}"


POLICY_KEYS = ("rung", "cache", "cache_dtype", "offload_to_host", "reuse_context_cache", "context_row_chunk",
               "stream_context", "allow_quantization", "query_chunk", "dropped_context_rows")
GB_KEYS = ("est_cache_gb", "resident_gb", "gpu_budget_absolute_gb", "host_budget_absolute_gb")


def _same_policy(got: dict, exp: dict, label: str) -> None:
    for key in POLICY_KEYS:
        assert got[key] == exp[key], (label, key, got[key], exp[key])
    for key in GB_KEYS:
        if exp[key] is None:
            assert got[key] is None, (label, key)
        else:
            assert math.isclose(got[key], exp[key], rel_tol=1e-12), (label, key, got[key], exp[key])


def test_runtime_fallbacks_and_escalations_match_the_reference(gold):
    # memory_policy.py:1304-1409: the rungs an out-of-memory retry walks from each opening rung,
    # and the records a retry's escalation writes, as the reference computed them
    rows = json.loads(str(gold["ladder/json"]))
    seen = 0
    for row in rows:
        if "error" in row:
            continue
        request = MemoryPolicy.coerce(row["request"])
        resolved = request.resolve(est_cache_gb=row["est"], bytes_per_element=row["bpe"], head_dim=row["head_dim"],
                                   total_vram_gb=row["vram"], total_ram_gb=row["ram"])
        got = request.runtime_fallbacks(resolved, bytes_per_element=row["bpe"], head_dim=row["head_dim"])
        assert [f.rung for f in got] == [f["rung"] for f in row["fallbacks"]], row["label"]
        for g, e in zip(got, row["fallbacks"]):
            _same_policy(g.as_report(), e, row["label"])
        seen += len(got)
        for rung, kwargs, key in (("context_row_chunk", dict(context_row_chunk=512, query_chunk=64), "escalated_chunk"),
                                  ("plain_loop", dict(dropped_context_rows=7), "escalated_plain")):
            if isinstance(row[key], str):
                assert row[key] == "ValueError"
                with pytest.raises(ValueError):
                    resolved.escalated(rung, **kwargs)
            else:
                _same_policy(resolved.escalated(rung, **kwargs).as_report(), row[key], row["label"] + " " + rung)
    assert seen >= 15


def test_fit_row_chunk_retry_ladder_and_attempt_records(gold):
    from nori_amd import memory_policy as M

    assert M.FIT_ROW_CHUNK_RETRY_LADDER == tuple(int(v) for v in gold["ladder/fit_row_chunk_retry"])
    # the retries are the ladder's chunks below the pinned one (predictor.py:1287-1291)
    assert M.fit_row_chunk_attempts(None) == [2048, 1024, 512, 256]
    assert M.fit_row_chunk_attempts(2048) == [1024, 512, 256]
    assert M.fit_row_chunk_attempts(600) == [512, 256]
    assert M.fit_row_chunk_attempts(256) == []
    exp = json.loads(str(gold["ladder/attempt_json"]))
    resolved = MemoryPolicy.coerce({"cache_dtype": "int8"}).resolve(
        est_cache_gb=2.0, bytes_per_element=2, head_dim=64, total_vram_gb=24.0, total_ram_gb=64.0)
    got = M.memory_attempt(resolved, pipeline_ids=[3], path="cached", rung="context_row_chunk", context_row_chunk=512,
                           outcome="oom", reason="oom_retry")
    assert got == exp
    for bad in (dict(outcome="maybe"), dict(reason="why"), dict(rung="nowhere"), dict(context_row_chunk=0)):
        kwargs = dict(pipeline_ids=[0], path="cached", rung="resident_int8", context_row_chunk=None, outcome="oom",
                      reason="resolved")
        kwargs.update(bad)
        with pytest.raises(ValueError):
            M.memory_attempt(resolved, **kwargs)


def test_policy_coercion_and_refusals():
    assert MemoryPolicy.coerce("exact").allow_quantization is False
    assert MemoryPolicy.coerce("max_context").cache_dtype == "int8"
    off = MemoryPolicy.coerce("off")
    assert off.cache is False and off.reuse_context_cache is False
    with pytest.raises(ValueError):
        MemoryPolicy.coerce("fastest")
    with pytest.raises(ValueError):
        MemoryPolicy.coerce({"cache": False, "cache_dtype": "int8"})
    with pytest.raises(ValueError):
        MemoryPolicy.coerce({"rung": "resident_int8"})
    with pytest.raises(ValueError):
        MemoryPolicy.coerce({"no_such_field": 1})
    with pytest.raises(TypeError):
        MemoryPolicy.coerce(3)


def test_fit_and_predict_argument_errors():
    x_tr, y_tr, x_te, _ = case.table()
    reg = api.NoriRegressor(model=object(), device="cpu")
    with pytest.raises(ValueError, match="before predict"):
        reg.predict(x_te)
    with pytest.raises(ValueError, match="same number of rows"):
        reg.fit(x_tr, y_tr[:-1])
    with pytest.raises(ValueError, match="finite"):
        reg.fit(x_tr, np.where(np.arange(len(y_tr)) == 3, np.nan, y_tr))
    with pytest.raises(ValueError, match="one-dimensional"):
        reg.fit(x_tr, np.stack([y_tr, y_tr], 1))
    reg.fit(x_tr, y_tr)
    assert reg.y_mean_ == pytest.approx(float(y_tr.mean())) and reg.n_features_in_ == case.N_FEATURES
    with pytest.raises(ValueError, match="Unknown output_type"):
        reg.predict(x_te, output_type="best")
    with pytest.raises(NotImplementedError):
        reg.predict(x_te, output_type="main")
    with pytest.raises(ValueError, match="requires quantiles"):
        reg.predict(x_te, output_type="quantiles")
    with pytest.raises(ValueError, match="strictly in"):
        reg.predict(x_te, output_type="quantiles", quantiles=[0.0, 0.5])
    with pytest.raises(ValueError, match="only valid"):
        reg.predict(x_te, quantiles=[0.5])
    with pytest.raises(ValueError, match="features"):
        reg.predict(x_te[:, :5])
    with pytest.raises(ValueError, match="memory preset"):
        api.NoriRegressor(model=object(), memory_policy="nope").fit(x_tr, y_tr)


def test_retained_contexts_stay_within_the_byte_budget():
    # predictor.py:2110-2261: retained contexts are bounded by bytes across every slot, the
    # least recently used dropped first; one larger than the whole budget empties the store and
    # is not kept; no budget keeps everything
    sizes = {"a": 40, "b": 30, "c": 20, "d": 50, "huge": 101}
    size_of = sizes.__getitem__
    store: dict = {}
    for slot, name in enumerate("abc"):
        assert api.retain_context(store, slot, ("key", name), 100, size_of)
    assert [e[-1] for e in store.values()] == ["a", "b", "c"]  # 90 of 100
    store[0] = store.pop(0)  # a reuse hit on slot 0 ("a") makes it the most recent
    assert api.retain_context(store, 3, ("key", "d"), 100, size_of)  # needs 50: drops "b", then "c"
    assert [e[-1] for e in store.values()] == ["a", "d"]
    assert api.retain_context(store, 0, ("key", "c"), 100, size_of)  # a slot's new context replaces its old one
    assert sorted(e[-1] for e in store.values()) == ["c", "d"]
    assert not api.retain_context(store, 5, ("key", "huge"), 100, size_of)
    assert store == {}
    for slot, name in enumerate("abcd"):
        assert api.retain_context(store, slot, ("key", name), None, size_of)
    assert len(store) == 4


def test_context_device_bytes_counts_each_device_storage_once():
    # host tensors do not count; views of one storage count once (CPU here: every figure is 0)
    t = torch.zeros(10, 4)
    assert api.context_device_bytes({"kv": t, "views": [t[:5], t[5:]]}) == 0
    assert api.context_device_bytes(object()) == 0


def test_yeo_johnson_pass_falls_back_to_the_plain_prediction(monkeypatch):
    # predictor.py:1934-1957, 1995-2003: a failure inside the augmentation returns the plain
    # prediction instead of ending predict
    reg = api.NoriRegressor(augmentations=("yj",), yj_skew_threshold=0.5)
    point = np.arange(5.0)
    y = np.exp(3.0 * np.random.default_rng(0).standard_normal(200)).astype(np.float32)

    def boom(*a, **k):
        raise RuntimeError("member failed")

    monkeypatch.setattr(reg, "_ensemble_bank", boom)
    out = reg._yeo_johnson_pass(None, None, y, point, None, "mean")
    assert out is point
    # too few finite targets, or a skew below the threshold: the plain prediction, unchanged
    assert reg._yeo_johnson_pass(None, None, y[:5], point, None, "mean") is point
    reg.yj_skew_threshold = 1e9
    assert reg._yeo_johnson_pass(None, None, y, point, None, "mean") is point


def _retry_request():
    return MemoryPolicy(gpu_budget_absolute_gb=1.0, host_budget_absolute_gb=2.0, elements_budget=1_072)


def _resolve(request):
    return request.resolve(est_cache_gb=0.1, bytes_per_element=2, head_dim=4, total_vram_gb=8.0, total_ram_gb=16.0)


def test_runtime_oom_walks_every_allowed_rung_then_bounded_fit_chunks():
    # predictor.py:3142-3400 as the reference's own test drives it
    # (tests/test_inference_pipeline_batching.py:758-794): every budget-feasible precision /
    # placement rung, then the last one with the context-row chunk ladder, each failure recorded
    request = _retry_request()
    resolved = _resolve(request)
    assert resolved.rung == "resident_bf16"
    tried, evicted, history = [], [], []

    def attempt(policy, chunk, hybrid, on_query, state):
        tried.append((policy.cache_dtype, policy.offload_to_host, chunk))
        if (policy.cache_dtype, policy.offload_to_host, chunk) != ("int8", True, 512):
            raise torch.cuda.OutOfMemoryError("synthetic build OOM")
        state["context"] = True
        on_query(300, "success")
        return "bank"

    result, final = api.run_cache_attempts(request, resolved, attempt, bytes_per_element=2, head_dim=4,
                                           history=history, pipeline_id=0, query_chunk=300,
                                           evict=lambda: evicted.append(1))
    expected = [("bf16", False, None), ("int8", False, None), ("bf16", True, None), ("int8", True, None),
                ("int8", True, 2048), ("int8", True, 1024), ("int8", True, 512)]
    assert tried == expected and result == "bank" and len(evicted) == 6
    assert final.rung == "context_row_chunk" and final.context_row_chunk == 512 and final.query_chunk == 300
    assert [a["outcome"] for a in history] == ["oom"] * 6 + ["success"]
    assert [(a["cache_dtype"], a["offload_to_host"], a["context_row_chunk"]) for a in history] == expected
    assert [a["reason"] for a in history] == ["resolved"] + ["oom_retry"] * 6
    assert all(a["dropped_context_rows"] == 0 for a in history)
    assert history[-1]["rung"] == "context_row_chunk" and history[0]["query_chunk"] is None


def test_runtime_oom_records_decode_halvings_and_propagates_when_exhausted():
    request = _retry_request()
    resolved = _resolve(request)
    history = []

    def decode_oom_once(policy, chunk, hybrid, on_query, state):
        # the first rung's build succeeds and its decode halves once (apply_context_cache's
        # callback), then succeeds
        state["context"] = True
        on_query(300, "oom")
        on_query(150, "success")
        return "bank"

    _, final = api.run_cache_attempts(request, resolved, decode_oom_once, bytes_per_element=2, head_dim=4,
                                      history=history, query_chunk=300)
    assert [(a["query_chunk"], a["outcome"], a["reason"]) for a in history] == [
        (300, "oom", "resolved"), (150, "success", "oom_retry")]
    assert final.rung == "resident_bf16" and final.query_chunk == 150

    history = []

    def always_oom(policy, chunk, hybrid, on_query, state):
        raise torch.cuda.OutOfMemoryError("synthetic build OOM")

    with pytest.raises(torch.cuda.OutOfMemoryError):
        api.run_cache_attempts(request, resolved, always_oom, bytes_per_element=2, head_dim=4, history=history)
    assert len(history) == 4 + 4 and all(a["outcome"] == "oom" for a in history)
    assert [a["context_row_chunk"] for a in history[4:]] == [2048, 1024, 512, 256]

    history = []

    def unsupported(policy, chunk, hybrid, on_query, state):
        raise NotImplementedError("no bounded build for serial attention")

    with pytest.raises(NotImplementedError):
        api.run_cache_attempts(request, resolved, unsupported, bytes_per_element=2, head_dim=4, history=history)
    assert [a["outcome"] for a in history] == ["unsupported"]


def test_runtime_oom_retries_a_streamed_context_on_stream_rungs_only():
    request = MemoryPolicy(stream_context=True, host_budget_absolute_gb=2.0)
    resolved = request.resolve(est_cache_gb=0.1, bytes_per_element=2, head_dim=4, total_vram_gb=8.0,
                               total_ram_gb=16.0)
    assert resolved.rung == "stream_bf16" and resolved.context_row_chunk == 2048
    tried, history = [], []

    def attempt(policy, chunk, hybrid, on_query, state):
        tried.append((policy.rung, chunk, hybrid))
        raise torch.cuda.OutOfMemoryError("synthetic build OOM")

    with pytest.raises(torch.cuda.OutOfMemoryError):
        api.run_cache_attempts(request, resolved, attempt, bytes_per_element=2, head_dim=4, history=history)
    # both stream precisions at the resolved cap, then the smaller caps on the last one; never a
    # resident rung, never the hybrid prefill
    assert tried == [("stream_bf16", 2048, False), ("stream_int8", 2048, False), ("stream_int8", 1024, False),
                     ("stream_int8", 512, False), ("stream_int8", 256, False)]
    assert {a["rung"] for a in history} == {"stream_bf16", "stream_int8"}


def test_hybrid_prefill_only_on_the_resident_int8_rung_with_a_chunk():
    request = MemoryPolicy(cache_dtype="int8", gpu_budget_absolute_gb=1.0, host_budget_absolute_gb=2.0,
                           offload_to_host=False)
    resolved = _resolve(request)
    assert resolved.rung == "resident_int8"
    tried = []

    def attempt(policy, chunk, hybrid, on_query, state):
        tried.append((chunk, hybrid))
        if chunk != 1024:
            raise torch.cuda.OutOfMemoryError("synthetic build OOM")
        return "bank"

    api.run_cache_attempts(request, resolved, attempt, bytes_per_element=2, head_dim=4, history=[])
    assert tried == [(None, False), (2048, True), (1024, True)]
