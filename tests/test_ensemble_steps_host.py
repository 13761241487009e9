"""The preprocessing steps outside the default ensemble configuration (nori_amd.ensemble), on the CPU.

The reference's shipped configurations use only the svd_all projection, the quantile-uniform
and adaptive redistributions and ordinal codes; its code also offers the svd_binary /
correlation / mutual-information / extra-trees projections (preprocess.py:1323-1684), the
power, logNormal and quantile_norm_10/_5 redistributions (preprocess.py:970-1222), and one-hot
codes (preprocess.py:686-832). Each is pinned here by what fixes it independently of this code:
the reference's own tests of the SVD fallbacks (tests/test_svd_fallback_visibility.py:30-175,
restated), closed forms and hand-computed matrices, scipy's Yeo-Johnson and Pearson routines,
numpy's SVD, and the sklearn behaviour that decides what the reference's workers become when
they are fitted (``clone`` drops constructor arguments passed through ``**kwargs``).
"""

from __future__ import annotations

import warnings

import numpy as np
import pytest
import torch
from scipy import stats
from sklearn.base import clone
from sklearn.preprocessing import PowerTransformer, QuantileTransformer

from nori_amd import ensemble as en
from nori_amd.degradation import CacheQuantizedWarning, DegradedPipelineWarning, SvdFallbackWarning, strict_pipeline

SVD_BLOCK = {"strategy": "svd_all", "svd_components": 64, "n_features_threshold": 256, "binary_threshold": 1.01}


def _data(n=300, p=400, seed=0):
    g = np.random.default_rng(seed)
    return g.standard_normal((n, p)), g.standard_normal(n)


def _selector(**kw):
    return en.WideTableProjection(**SVD_BLOCK, device="cpu", **kw)


def _break_fit(monkeypatch):
    class Broken(en.DeviceSVD):
        def fit(self, x, y=None):
            raise np.linalg.LinAlgError("synthetic fit failure")

    monkeypatch.setattr(en, "DeviceSVD", Broken)


def _break_transform(step):
    def boom(_x):
        raise np.linalg.LinAlgError("synthetic transform failure")

    step.svd.transform = boom


# ---- the reference's SVD-fallback tests (tests/test_svd_fallback_visibility.py:65-175)
def test_transform_failure_warns_and_zeros():
    x, y = _data()
    step = _selector()
    step.fit(x, [], 0, y=y)
    _break_transform(step)
    with pytest.warns(SvdFallbackWarning, match="all-zero column"):
        out, cat = step.apply(x[:5])
    assert out.shape == (5, 1) and not out.any() and cat == []


def test_transform_failure_is_fatal_under_strict_pipeline():
    x, y = _data()
    step = _selector()
    step.fit(x, [], 0, y=y)
    _break_transform(step)
    with strict_pipeline(), pytest.raises(SvdFallbackWarning, match="all-zero column"):
        step.apply(x[:5])


def test_svd_binary_transform_failure_warns():
    g = np.random.default_rng(1)
    x = (g.random((300, 400)) < 0.3).astype(float)
    step = en.WideTableProjection(strategy="svd_binary", n_features_threshold=256, binary_threshold=0.5,
                                  svd_components=64, device="cpu")
    step.fit(x, [], 0, y=g.standard_normal(300))
    _break_transform(step)
    with pytest.warns(SvdFallbackWarning, match="SVD-projected columns"):
        out, _ = step.apply(x[:5])
    assert out.shape[1] == len(step.keep)


def test_fit_failure_warns_and_passes_through(monkeypatch):
    x, y = _data()
    _break_fit(monkeypatch)
    step = _selector()
    with pytest.warns(SvdFallbackWarning, match="passthrough of all 400 raw columns"):
        step.fit(x, [], 0, y=y)
    assert step.svd is None and step.apply(x[:5])[0].shape[1] == 400


def test_fit_failure_is_fatal_under_strict_pipeline(monkeypatch):
    x, y = _data()
    _break_fit(monkeypatch)
    with strict_pipeline(), pytest.raises(SvdFallbackWarning, match="SVD fit failed"):
        _selector().fit(x, [], 0, y=y)


def test_working_svd_is_silent_even_under_strict_pipeline():
    x, y = _data()
    with warnings.catch_warnings(record=True) as caught:
        warnings.simplefilter("always")
        step = _selector()
        step.fit(x, [], 0, y=y)
        out, _ = step.apply(x[:5])
    assert not [w for w in caught if issubclass(w.category, DegradedPipelineWarning)]
    assert out.shape == (5, 64)
    with strict_pipeline():
        step = _selector()
        step.fit(x, [], 0, y=y)
        assert step.apply(x[:5])[0].shape == (5, 64)


def test_category_tree():
    assert issubclass(SvdFallbackWarning, DegradedPipelineWarning)
    assert issubclass(CacheQuantizedWarning, DegradedPipelineWarning)
    assert issubclass(DegradedPipelineWarning, UserWarning)
    assert not issubclass(SvdFallbackWarning, CacheQuantizedWarning)


def test_strict_pipeline_can_escalate_one_kind_only(monkeypatch):
    x, y = _data()
    _break_fit(monkeypatch)
    with strict_pipeline(CacheQuantizedWarning), pytest.warns(SvdFallbackWarning):
        _selector().fit(x, [], 0, y=y)
    with strict_pipeline(DegradedPipelineWarning), pytest.raises(SvdFallbackWarning):
        _selector().fit(x, [], 0, y=y)


def test_strict_pipeline_restores_filters(monkeypatch):
    x, y = _data()
    _break_fit(monkeypatch)
    before = list(warnings.filters)
    with strict_pipeline(), pytest.raises(SvdFallbackWarning):
        _selector().fit(x, [], 0, y=y)
    assert warnings.filters == before
    with pytest.warns(SvdFallbackWarning):
        _selector().fit(x, [], 0, y=y)


def test_device_solver_failure_falls_back_to_the_library_svd(monkeypatch):
    # the device solver raising hands the fit to sklearn's TruncatedSVD, silently: same subspace
    x, _ = _data(200, 40)

    def no_device(*a, **k):
        raise RuntimeError("device solver unavailable")

    exact = en.DeviceSVD(5, "cpu").fit_transform(x)
    monkeypatch.setattr(torch.linalg, "svd", no_device)
    approx = en.DeviceSVD(5, "cpu", random_state=0, algorithm="arpack").fit_transform(x)
    np.testing.assert_allclose(np.linalg.norm(approx, axis=0), np.linalg.norm(exact, axis=0), rtol=1e-8)


# ---- svd_binary: the binary block's SVD after the other columns
def test_svd_binary_replaces_the_binary_block():
    g = np.random.default_rng(2)
    n = 120
    binary = (g.random((n, 30)) < 0.4).astype(np.float64)
    binary[g.random((n, 30)) < 0.02] = np.nan  # NaNs count as zeros in the block
    other = g.standard_normal((n, 3))
    x = np.hstack([other[:, :1], binary, other[:, 1:]])  # non-binary columns 0, 31, 32
    step = en.WideTableProjection(strategy="svd_binary", n_features_threshold=256, binary_threshold=0.5,
                                  svd_components=64, device="cpu")
    cat = step.fit(x, [0, 5, 32], 3)
    assert cat == [0, 2]  # categorical 0 and 32 are kept (positions 0 and 2); binary 5 is projected away
    out, _ = step.apply(x)
    k = min(64, 30 - 1, n - 1)
    assert out.shape == (n, 3 + k)
    np.testing.assert_array_equal(out[:, :3], other.astype(np.float32))
    block = np.where(np.isnan(binary), 0.0, binary)
    sv = np.linalg.svd(block, compute_uv=False)[:k]
    np.testing.assert_allclose(np.linalg.norm(out[:, 3:].astype(np.float64), axis=0), sv, rtol=1e-5)
    # too few binary columns: the strategy's own gate passes through
    few = np.hstack([g.standard_normal((n, 300)), binary[:, :1]])
    step2 = en.WideTableProjection(strategy="svd_binary", n_features_threshold=256, binary_threshold=0.5,
                                   device="cpu")
    assert step2.fit(few, [1], 3) == [1] and step2.apply(few)[0] is few


# ---- the target-driven projections
def _target_table(n=400, p=150, seed=4):
    g = np.random.default_rng(seed)
    y = g.standard_normal(n)
    x = g.standard_normal((n, p))
    for j, w in zip((7, 40, 99, 120), (3.0, 1.0, 0.5, 0.25)):
        x[:, j] = w * y + g.standard_normal(n)
    x[g.random((n, p)) < 0.01] = np.nan
    x[:, 3] = 1.5  # a constant column scores 0
    return x, y


def test_corr_keeps_the_top_columns_by_pearson():
    x, y = _target_table()
    step = en.WideTableProjection(strategy="corr", top_k=10, n_features_threshold=128, device="cpu")
    cat = step.fit(x, [7, 8], 11, y=y)
    scores = np.zeros(x.shape[1])
    for j in range(x.shape[1]):
        ok = np.isfinite(x[:, j])
        if np.ptp(x[ok, j]) > 0:
            scores[j] = abs(stats.pearsonr(x[ok, j], y[ok]).statistic)
    expected = np.sort(np.argsort(-scores, kind="stable")[:10])
    np.testing.assert_array_equal(step.selected, expected)
    assert {7, 40, 99}.issubset(set(step.selected.tolist()))
    out, _ = step.apply(x)
    np.testing.assert_array_equal(out, x[:, expected])
    assert cat == ([list(expected).index(7)] + ([list(expected).index(8)] if 8 in expected else []))


def test_target_driven_projections_pass_through_without_a_usable_target():
    x, y = _target_table()
    for strategy in ("corr", "mi", "extratrees"):
        step = en.WideTableProjection(strategy=strategy, top_k=10, n_features_threshold=128, device="cpu")
        assert step.fit(x, [2], 0) == [2] and step.apply(x)[0] is x  # no target (the fit on context + queries)
        assert step.fit(x, [2], 0, y=y[:-1]) == [2]  # wrong length
        few = np.full_like(y, np.nan)
        few[:9] = 1.0
        assert step.fit(x, [2], 0, y=few) == [2]  # fewer than max(10, top_k // 4) finite targets
        assert not step.depends_on_rows()
    narrow = x[:, :100]
    step = en.WideTableProjection(strategy="corr", top_k=10, n_features_threshold=128, device="cpu")
    assert step.fit(narrow, [], 0, y=y) == [] and step.apply(narrow)[0] is narrow  # gate closed


@pytest.mark.parametrize("strategy", ["mi", "extratrees"])
def test_nonlinear_scorers_find_the_dependent_columns(strategy):
    # column 5 is the target itself and column 9 its square: mutual information and the forest see
    # both, while |Pearson r| of the square with a symmetric target is about zero
    g = np.random.default_rng(6)
    n, p = 600, 140
    y = g.standard_normal(n)
    x = g.standard_normal((n, p))
    x[:, 5], x[:, 9] = y, y**2
    kw = dict(strategy=strategy, top_k=2, n_features_threshold=128, subsample_rows=500,
              extratrees_n_estimators=20, device="cpu")
    step = en.WideTableProjection(**kw)
    step.fit(x, [], 17, y=y)
    np.testing.assert_array_equal(step.selected, [5, 9])
    again = en.WideTableProjection(**kw)
    again.fit(x, [], 17, y=y)
    np.testing.assert_array_equal(again.selected, step.selected)
    corr = en.WideTableProjection(strategy="corr", top_k=2, n_features_threshold=128, device="cpu")
    corr.fit(x, [], 17, y=y)
    assert 9 not in corr.selected


# ---- what sklearn's clone makes of the reference's kwargs-style workers
def test_kwargs_constructor_arguments_do_not_survive_clone():
    class PowerKw(PowerTransformer):  # the constructor shape of preprocess.py:188
        def __init__(self, var_tolerance=1e-3, max_abs_value=100, **kwargs):
            super().__init__(**kwargs)
            self.var_tolerance, self.max_abs_value = var_tolerance, max_abs_value

    class QuantileKw(QuantileTransformer):  # the constructor shape of preprocess.py:840
        def __init__(self, *, n_quantiles=1000, **kwargs):
            super().__init__(n_quantiles=n_quantiles, **kwargs)

    assert clone(PowerKw(standardize=False)).standardize is True
    q = clone(QuantileKw(output_distribution="normal", n_quantiles=7, random_state=3))
    assert (q.output_distribution, q.random_state, q.subsample) == ("uniform", None, en.QUANTILE_SUBSAMPLE_DEFAULT)


def _redistribute(tag, x, categorical=(), **kw):
    step = en.Redistribute(worker_tags=[tag], device="cpu", **kw)
    step.fit(x, list(categorical), 8)
    return step


def test_power_worker():
    g = np.random.default_rng(9)
    n = 500
    skewed = g.lognormal(0.0, 0.8, n)
    skewed[[3, 70]] = np.nan
    x = np.stack([skewed, np.full(n, 2.5), g.standard_normal(n)], axis=1)
    out = _redistribute("power", x).apply(x)[0]
    ok = np.isfinite(skewed)
    # a transformed column: Yeo-Johnson at the likelihood-maximizing lambda, standardized (scipy)
    z = stats.yeojohnson(skewed[ok], stats.yeojohnson_normmax(skewed[ok]))
    z = (z - z.mean()) / z.std()
    # the NaN rows are filled with the column's mean (0) before the last scaler is fitted
    filled = np.zeros(n)
    filled[ok] = z
    np.testing.assert_allclose(out[ok, 0], z / filled.std(), rtol=0, atol=2e-5)
    assert np.abs(out[~ok, 0]).max() < 1e-9
    # the constant column: its transformed variance is 0, so transform hands back the raw 2.5,
    # and the scaler after it, fitted on the transformed zeros, leaves 2.5
    np.testing.assert_array_equal(out[:, 1], 2.5)
    with pytest.raises(AssertionError):  # not the standardized raw column (what standardize=False would give)
        np.testing.assert_allclose(out[ok, 0], (skewed[ok] - skewed[ok].mean()) / skewed[ok].std(), atol=1e-3)


def test_log_normal_worker_is_a_stateless_shifted_log():
    g = np.random.default_rng(10)
    x = g.standard_normal((50, 3))
    x[4, 1] = np.nan
    step = _redistribute("logNormal", x)
    out = step.apply(x)[0]
    filled = x.copy()
    filled[4, 1] = np.nanmean(x[:, 1])
    np.testing.assert_allclose(out, np.log(filled + abs(filled.min()) + 1e-10), rtol=1e-12)
    assert np.isclose(out.min(), np.log(1e-10))
    # the query matrix is moved by its own smallest entry, not the context's
    q = g.standard_normal((7, 3)) + 5.0
    np.testing.assert_allclose(step.apply(q)[0], np.log(q + q.min() + 1e-10), rtol=1e-12)
    # float32 stays float32 through the worker
    assert _redistribute("logNormal", x.astype(np.float32)).apply(x.astype(np.float32))[0].dtype == np.float32


def test_quantile_norm_tags_are_uniform_uncapped_quantiles():
    g = np.random.default_rng(11)
    x = g.standard_normal((3000, 2))
    for tag, q in (("quantile_norm_10", 300), ("quantile_norm_5", 600)):
        step = _redistribute(tag, x)
        out = step.apply(x)[0]
        fitted = step.worker.named_transformers_[f"feat_transform_{tag}"]
        assert fitted.n_quantiles_ == q  # above the 256 cap of the *_all_data tags
        ref = QuantileTransformer(output_distribution="uniform", n_quantiles=q).fit(x)
        np.testing.assert_allclose(out, ref.transform(x), rtol=0, atol=1e-12)
        assert out.min() >= 0.0 and out.max() <= 1.0


def test_unknown_tags_are_the_identity_and_kdi_needs_its_package():
    x = np.random.default_rng(12).standard_normal((40, 4))
    for tag in ("quantile", None, "something_else"):
        np.testing.assert_array_equal(_redistribute(tag, x).apply(x)[0], x)
    with pytest.raises(NotImplementedError, match="kditransform"):
        _redistribute("kdi_uni", x)


# ---- one-hot codes
def test_onehot_codes():
    x = np.array([[0, 1.5, 5], [1, 2.5, 7], [2, 3.5, 5], [0, 4.5, 7]], dtype=np.float64)
    step = en.CategoryCodes(encoding_strategy="onehot")
    assert step.fit(x, [0, 2], 1) == [0, 1, 2, 3]
    expected = np.array([[1, 0, 0, 0, 1.5], [0, 1, 0, 1, 2.5], [0, 0, 1, 0, 3.5], [1, 0, 0, 1, 4.5]])
    out, cat = step.apply(x)
    np.testing.assert_array_equal(out, expected)
    assert cat == [0, 1, 2, 3]
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")  # sklearn notes the unknown levels
        q, _ = step.apply(np.array([[9, 0.5, 5], [1, 0.25, 6]]))
    np.testing.assert_array_equal(q, [[0, 0, 0, 0, 0.5], [0, 1, 0, 0, 0.25]])


def test_onehot_too_wide_leaves_the_matrix():
    g = np.random.default_rng(13)
    x = np.stack([g.integers(0, 25, 40000).astype(np.float64), g.standard_normal(40000)], axis=1)
    step = en.CategoryCodes(encoding_strategy="onehot")
    assert step.fit(x, [0], 1) == [0]  # 40000 rows x 26 columns >= 10^6 entries
    out, cat = step.apply(x)
    assert out is x and cat == [0]
    with pytest.raises(ValueError):
        en.CategoryCodes(encoding_strategy="binary")


# ---- a member built from these steps
def test_member_with_the_other_steps_runs_and_transforms_new_queries_as_a_refit():
    g = np.random.default_rng(14)
    n, p = 300, 150
    x_tr = g.standard_normal((n, p)).astype(np.float32)
    x_tr[:, 0] = g.integers(0, 3, n)
    y = g.standard_normal(n).astype(np.float32)
    x_tr[:, 10] = y + 0.1 * g.standard_normal(n)
    x_te = g.standard_normal((40, p)).astype(np.float32)
    x_te[:, 0] = g.integers(0, 3, 40)
    config = [{"HighDimFeatureSelector": {"strategy": "corr", "top_k": 12, "n_features_threshold": 128},
               "RebalanceFeatureDistribution": {"worker_tags": ["power"], "original_flag": True},
               "CategoricalFeatureEncoder": {"encoding_strategy": "onehot"},
               "FeatureShuffler": {"mode": "shuffle"}}]
    member = en.build_members(config, 0, "cpu")[0]
    cat0 = en.categorical_columns(x_tr)
    assert cat0 == [0]
    a, b, cat = member.features(x_tr, x_te, cat0, y)
    assert a.shape[0] == n and b.shape == (40, a.shape[1]) and np.isfinite(a).all() and np.isfinite(b).all()
    other = g.standard_normal((9, p)).astype(np.float32)
    other[:, 0] = g.integers(0, 3, 9)
    fresh = en.build_members(config, 0, "cpu")[0]
    _, b2, _ = fresh.features(x_tr, other, cat0, y)
    np.testing.assert_array_equal(member.query_features(other), b2)
