"""NoriRegressor on the GPU against the reference's own nori-6m runs (tests/golden/regressor_goldens.npz,
tests/golden/regressor_autocast_goldens.npz).

The case (tests/regressor_case.py): a seeded random-init nori-6m model, 1024 context + 256
query rows of 16 features, the int8 context cache. The reference ran its context-cache API on
the CPU with the same weights (hash-checked) in fp32, and again under fp16 autocast (its
predictor's own GPU mode, predictor.py:3208-3217); here the whole path runs on the HIP kernels.

* fp32 (mix_precision=False) is held to the prediction bar, max|got - exp| / max|exp| <= 1e-3,
  against the reference's fp32 run.
* fp16 autocast (mix_precision=True, the default) is held to the reference's fp16 autocast run,
  made on the CPU with CUDA autocast's op policy (tests/golden/cuda_autocast_policy.py: CPU
  autocast would leave the encoders' LayerNorm in fp16 and the residual stream with it). Every
  projection and the 999-level head round to fp16 there (the bank's upper levels, ~9 in
  standardized units, to 2^-7), and the reference's own fp16 outputs move by 2.2e-3 (0.1
  quantile), 2.9e-3 (point predictions) and 8.4e-3 (0.9 quantile) when only the order of the
  context rows -- so of its sums -- changes (the golden recipe measures it over three orders and
  stores it). No fp16 run can be held closer than that to another; each output's bar is the
  prediction bar or 1.5 times that spread, whichever is larger (measured here: 2.3e-3 on the
  point predictions, 1.4e-3 to 6.7e-3 on the quantiles). Against the fp32 run, the same factor
  times the reference's own fp16-to-fp32 distance.
Each check prints its figure, and the error relative to the predictions' spread across rows is
printed beside it.
"""

from __future__ import annotations

import json
import os
import warnings

import numpy as np
import pytest
import torch

import regressor_case as case
from nori_amd import api
from nori_amd.memory_policy import CacheQuantizedWarning
from nori_amd.transformer import FeaturesTransformer
from parity import PREDICTION_BAR, check_relative

pytestmark = pytest.mark.gpu

SPREAD_FACTOR = 1.5
# The golden is the reference's context-cache API on the raw columns: a one-member inference
# configuration with no steps (only constant columns dropped; config 1 has none).
RAW = [{}]

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "regressor_goldens.npz")
GOLDEN_AUTOCAST = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "regressor_autocast_goldens.npz")


@pytest.fixture(scope="module")
def gold():
    with np.load(GOLDEN, allow_pickle=False) as f:
        g = {k: f[k] for k in f.files}
    with np.load(GOLDEN_AUTOCAST, allow_pickle=False) as f:
        g.update({f"ac/{k}": f[k] for k in f.files})
    return g


@pytest.fixture(scope="module")
def model(gold):
    m = case.seeded_model(FeaturesTransformer, api.NORI_6M_CONFIG, json.loads(str(gold["case/weight_scales"])))
    assert case.weights_sha256(m) == str(gold["case/weights_sha256"]), "seeded weights differ from the golden run's"
    return m


def spread_note(got, exp, what):
    err = np.abs(np.asarray(got, np.float64) - exp).max()
    print(f"[parity] {what}: max abs {err:.3e} = {err / exp.std():.3e} of the predictions' spread (std {exp.std():.3e})",
          flush=True)


@pytest.mark.parametrize("mix_precision", [True, False])
def test_predictions_match_the_reference(gold, model, cuda, mix_precision):
    tag = "fp16 autocast" if mix_precision else "fp32"
    reg = api.NoriRegressor(model=model, device=cuda, inference_config=RAW, memory_policy="max_context",
                            mix_precision=mix_precision)
    reg.fit(gold["case/x_train"], gold["case/y_train"])
    with warnings.catch_warnings(record=True) as caught:
        warnings.simplefilter("always")
        point = reg.predict(gold["case/x_test"])
    assert any(issubclass(w.category, CacheQuantizedWarning) for w in caught)
    y_mean, y_std = reg.y_mean_, reg.y_std_
    fp32_sorted = np.sort(gold["case/bank_norm"].astype(np.float64), axis=1) * y_std + y_mean
    if mix_precision:
        ac_sorted = np.sort(gold["ac/bank_norm"].astype(np.float64), axis=1) * y_std + y_mean
        # each output against the reference's fp16 run (bar from its own spread over context
        # orders) and its fp32 run (bar from its own fp16-to-fp32 distance)
        goldens = [(ac_sorted, gold["ac/point"], lambda k: max(PREDICTION_BAR, SPREAD_FACTOR * float(gold[f"ac/spread/{k}"])),
                    "reference fp16 autocast run"),
                   (fp32_sorted, gold["case/point"],
                    lambda k: max(PREDICTION_BAR, SPREAD_FACTOR * float(gold[f"ac/vs_fp32/{k}"])), "reference fp32 run")]
    else:
        goldens = [(fp32_sorted, gold["case/point"], lambda k: PREDICTION_BAR, "reference fp32 run")]
    qs = reg.predict(gold["case/x_test"], output_type="quantiles", quantiles=list(case.QUANTILE_LEVELS))
    assert qs.shape == (3, case.N_QUERY)
    full = reg.predict(gold["case/x_test"], output_type="full")
    np.testing.assert_allclose(full["mean"], point, rtol=1e-12, atol=1e-12)
    median = reg.predict(gold["case/x_test"], output_type="median")
    for ref_sorted, ref_point, bar, against in goldens:
        check_relative(point, ref_point, bar("point"), f"nori-6m point predictions ({tag}) vs the {against}")
        spread_note(point, ref_point, f"nori-6m point predictions ({tag}) vs the {against}")
        for i, level in enumerate(case.QUANTILE_LEVELS):
            check_relative(qs[i], ref_sorted[:, int(round(level * 1000)) - 1], bar(f"q{level}"),
                           f"nori-6m quantile {level} ({tag}) vs the {against}")
        check_relative(full["quantiles"], ref_sorted, bar("bank"), f"nori-6m 999-level bank ({tag}) vs the {against}")
        n_levels = ref_sorted.shape[1]
        ref_median = (0.5 * (ref_sorted[:, n_levels // 2 - 1] + ref_sorted[:, n_levels // 2]) if n_levels % 2 == 0
                      else ref_sorted[:, n_levels // 2])
        check_relative(median, ref_median, bar("median"), f"nori-6m median ({tag}) vs the {against}")

    report = reg.memory_report_
    assert report["rung"] == "resident_int8" and report["cache_dtype"] == "int8" and report["cache"] is True
    assert report["context_reused"] is True  # the later calls reused the first call's context


def test_int8_cache_codes_and_context_reuse(gold, model, cuda):
    # fp32, as the reference's CPU run: the K/V the codes come from are then fp32 on both sides
    reg = api.NoriRegressor(model=model, device=cuda, inference_config=RAW, memory_policy={"cache_dtype": "int8"},
                            mix_precision=False)
    reg.fit(gold["case/x_train"], gold["case/y_train"])
    first = reg.predict(gold["case/x_test"])
    assert reg.memory_report_["context_reused"] is False
    second = reg.predict(gold["case/x_test"])
    assert reg.memory_report_["context_reused"] is True
    assert np.array_equal(first, second)
    # layer 0's int8 codes: the K/V of the context's first layer come from the inputs through one
    # norm and one projection; device and host sums differ in order, so a code may sit one step
    # away where a value lies on a rounding boundary
    codes, scales = reg._contexts[0][3].caches[0]["seq_kv"].device_payload()
    d = codes[:, :128].cpu().numpy().astype(np.int32) - gold["case/codes0"].astype(np.int32)
    print(f"[parity] layer-0 int8 codes: {np.mean(d != 0):.2e} differ by one, max {np.abs(d).max()}", flush=True)
    assert np.abs(d).max() <= 1 and np.mean(d != 0) < 0.01
    check_relative(scales[:, :128].cpu(), gold["case/scales0"], 2e-3, "layer-0 int8 scales")
    # a new context (other targets) is encoded again, not served from the retained one
    reg.fit(gold["case/x_train"], gold["case/y_train"] * 2.0)
    reg.predict(gold["case/x_test"][:8])
    assert reg.memory_report_["context_reused"] is False


def test_bf16_rung_and_exact_preset(gold, model, cuda):
    for policy, rung, dtype in ((None, "resident_bf16", "bf16"), ("exact", "resident_bf16", "bf16")):
        reg = api.NoriRegressor(model=model, device=cuda, inference_config=RAW, memory_policy=policy,
                                mix_precision=False)
        reg.fit(gold["case/x_train"], gold["case/y_train"])
        with warnings.catch_warnings():
            warnings.simplefilter("error", CacheQuantizedWarning)  # the full-precision rung does not quantize
            point = reg.predict(gold["case/x_test"])
        assert reg.memory_report_["rung"] == rung and reg.memory_report_["cache_dtype"] == dtype
        # the int8 golden against the full-precision cache: the int8 rounding is inside the bar
        check_relative(point, gold["case/point"], PREDICTION_BAR, f"nori-6m point predictions, {rung} cache")


def test_default_ensemble_members(gold, model, cuda):
    # the reference's default inference configuration: eight members, each with its own
    # features and context cache, banks averaged; every member's context is reused by a second
    # call on the same context, which then returns the same predictions
    reg = api.NoriRegressor(model=model, device=cuda, memory_policy={"cache_dtype": "int8"})
    reg.fit(gold["case/x_train"], gold["case/y_train"])
    with warnings.catch_warnings():
        warnings.simplefilter("ignore", CacheQuantizedWarning)
        first = reg.predict(gold["case/x_test"])
        assert reg.memory_report_["ensemble_members"] == 8 and reg.memory_report_["context_reused"] is False
        second = reg.predict(gold["case/x_test"])
        assert reg.memory_report_["context_reused"] is True
        qs = reg.predict(gold["case/x_test"], output_type="quantiles", quantiles=[0.1, 0.5, 0.9])
    assert np.all(np.isfinite(first)) and np.array_equal(first, second)
    assert np.all(np.diff(qs, axis=0) >= 0)
    # the raw-column member is not the ensemble: the members' features differ from the raw ones
    raw = api.NoriRegressor(model=model, device=cuda, inference_config=RAW, memory_policy={"cache_dtype": "int8"})
    raw.fit(gold["case/x_train"], gold["case/y_train"])
    with warnings.catch_warnings():
        warnings.simplefilter("ignore", CacheQuantizedWarning)
        assert not np.allclose(raw.predict(gold["case/x_test"]), first)


def test_yeo_johnson_pass_on_a_skewed_target(gold, model, cuda):
    # a target with skew above the threshold adds the Yeo-Johnson pass: its point predictions
    # differ from the plain pass's and stay finite; below the threshold nothing changes
    x_tr, x_te = gold["case/x_train"], gold["case/x_test"]
    rng = np.random.default_rng(5)
    y_skewed = np.exp(3.0 * rng.standard_normal(len(x_tr)))
    out = {}
    for aug in ((), ("yj",)):
        reg = api.NoriRegressor(model=model, device=cuda, inference_config=RAW, augmentations=aug,
                                memory_policy={"cache_dtype": "int8"}, mix_precision=False)
        with warnings.catch_warnings():
            warnings.simplefilter("ignore", CacheQuantizedWarning)
            out[aug] = reg.fit(x_tr, y_skewed).predict(x_te)
            if aug:
                plain = reg.fit(x_tr, gold["case/y_train"]).predict(x_te)
                reg.augmentations = ()
                assert np.array_equal(plain, reg.predict(x_te))
    assert np.all(np.isfinite(out[("yj",)])) and not np.allclose(out[()], out[("yj",)])


def test_out_of_memory_on_the_opening_rung_retries_the_next(gold, model, cuda, monkeypatch):
    # predictor.py:3142-3400: a build that runs out of device memory on the opening rung
    # (resident bf16 here) is retried on the next the policy allows (resident int8), and both
    # attempts are in memory_report_["attempt_history"]
    reg = api.NoriRegressor(model=model, device=cuda, inference_config=RAW, mix_precision=False)
    reg.fit(gold["case/x_train"], gold["case/y_train"])
    real = FeaturesTransformer.build_context_cache
    calls = []

    def flaky(self, *a, **k):
        calls.append(k.get("cache_dtype"))
        if len(calls) == 1:
            raise torch.cuda.OutOfMemoryError("synthetic out-of-memory on the first build")
        return real(self, *a, **k)

    monkeypatch.setattr(FeaturesTransformer, "build_context_cache", flaky)
    with warnings.catch_warnings():
        warnings.simplefilter("ignore", CacheQuantizedWarning)
        point = reg.predict(gold["case/x_test"])
    report = reg.memory_report_
    assert calls == ["bf16", "int8"]
    assert [(a["rung"], a["outcome"], a["reason"]) for a in report["attempt_history"]] == [
        ("resident_bf16", "oom", "resolved"), ("resident_int8", "success", "oom_retry")]
    assert report["rung"] == "resident_int8" and report["cache_dtype"] == "int8"
    check_relative(point, gold["case/point"], PREDICTION_BAR, "nori-6m point predictions after the retry (fp32)")


def test_same_shaped_members_are_scored_in_batches(gold, model, cuda, monkeypatch):
    # the default ensemble's two groups of four same-shaped members each run as one batched
    # cache build and apply (predictor.py:2325-2359, 2497-2700); the predictions equal scoring
    # the members one at a time, and a second call reuses both the batched caches and the
    # members' preprocessing fits, giving the same bits
    kwargs = dict(model=model, device=cuda, memory_policy={"cache_dtype": "int8"}, mix_precision=False)
    with warnings.catch_warnings():
        warnings.simplefilter("ignore", CacheQuantizedWarning)
        reg = api.NoriRegressor(**kwargs).fit(gold["case/x_train"], gold["case/y_train"])
        batched = reg.predict(gold["case/x_test"])
        history = reg.memory_report_["attempt_history"]
        assert [a["pipeline_ids"] for a in history if a["path"] == "pipeline_batch"] == [[0, 1, 2, 3], [4, 5, 6, 7]]
        again = reg.predict(gold["case/x_test"])
        assert reg.memory_report_["context_reused"] is True and np.array_equal(batched, again)
        monkeypatch.setattr(api, "MEMBER_BATCH", 1)
        one = api.NoriRegressor(**kwargs).fit(gold["case/x_train"], gold["case/y_train"]).predict(gold["case/x_test"])
    check_relative(batched, one, PREDICTION_BAR, "default ensemble, batched members vs one at a time (fp32)")
