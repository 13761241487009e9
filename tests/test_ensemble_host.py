"""The preprocessing ensemble in front of NoriRegressor (nori_amd.ensemble), on the CPU.

The reference's module (src/synthefy_nori/inference/preprocess.py) cannot be imported here: it
imports ``kditransform``, which this image does not have, so no member's features could be
written as golden vectors from the reference itself. Each step is pinned instead by what fixes
it independently of this code: the default configuration against the SHA-256 digest of the
reference's own configuration file (tests/golden/default_inference_digest.json), the seed draws against
Python's and numpy's generators as the reference calls them, the column operations by closed
forms (which columns a step keeps, which products it forms, what a permutation does), the
distribution steps by the sklearn / scipy routines the reference builds them from, and the
SVD block by the decomposition's own identities. End to end, a member's features are parity
unpinned against the reference.
"""

from __future__ import annotations

import hashlib
import json
import os
import random

import numpy as np
import pytest
from scipy import stats
from sklearn.preprocessing import QuantileTransformer

import regressor_case as case
from nori_amd import ensemble as en

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "default_inference_digest.json")


def test_default_members_are_the_reference_configuration():
    # the digest of the canonical JSON form (sorted keys) of the reference's member list
    with open(GOLDEN) as f:
        gold = json.load(f)
    members = json.loads(json.dumps(list(en.DEFAULT_MEMBERS)))
    assert len(members) == gold["members"]
    assert hashlib.sha256(json.dumps(members, sort_keys=True).encode()).hexdigest() == gold["sha256"]


def test_seed_slots_follow_the_reference_draws():
    members = en.build_members(en.DEFAULT_MEMBERS, 7, "cpu")
    draw = random.Random(7)
    seeds = [draw.randint(0, 10000) for _ in range(8 * en.SEED_SLOTS)]
    for i, m in enumerate(members):
        slots = seeds[i * en.SEED_SLOTS:(i + 1) * en.SEED_SLOTS]
        kinds = [type(s).__name__ for s in m.steps]
        assert kinds == ["WideTableProjection", "FeatureCap", "PairProducts", "DropConstantColumns", "Redistribute",
                         "CategoryCodes", "RowFingerprint", "ColumnOrder"]
        # the projection takes the last slot; the others their position among the rest
        assert m.seeds == [slots[9]] + slots[:7]
    g = np.random.default_rng(7)
    start = g.integers(0, 1000)
    shifts = g.choice(list(range(start, start + 8)), size=8, replace=False)
    assert [m.steps[-1].offset for m in members] == [int(v) for v in shifts]
    with pytest.raises(ValueError):
        en.build_members([], 0, "cpu")


def test_drop_constant_columns():
    x = np.array([[1.0, 2.0, np.nan, 5.0, np.nan], [1.0, 3.0, np.nan, 5.0, 1.0], [1.0, 4.0, np.nan, 6.0, 2.0]])
    step = en.DropConstantColumns()
    cat = step.fit(x, [0, 3, 4], 0)
    out, cat_out = step.apply(x)
    # column 0 constant, column 2 all NaN; column 4 keeps its NaN in row 0 (NaN != NaN)
    np.testing.assert_array_equal(out, x[:, [1, 3, 4]])
    assert cat == cat_out == [1, 2]
    with pytest.raises(ValueError, match="All features are constant"):
        en.DropConstantColumns().fit(np.ones((4, 3)), [], 0)


def test_feature_cap():
    x = np.arange(60.0).reshape(3, 20)
    step = en.FeatureCap(max_features=8)
    cat = step.fit(x, [1, 5, 19], 11)
    keep = np.sort(np.random.default_rng(11).choice(20, size=8, replace=False))
    np.testing.assert_array_equal(step.apply(x)[0], x[:, keep])
    assert cat == sorted(list(keep).index(c) for c in (1, 5, 19) if c in keep)
    small = en.FeatureCap(max_features=50)
    small.fit(x, [], 0)
    np.testing.assert_array_equal(small.apply(x)[0], x)


@pytest.mark.parametrize("p", [1, 3, 4, 9])
def test_pair_products(p):
    g = np.random.default_rng(p)
    x = g.standard_normal((40, p)).astype(np.float32) * np.arange(1, p + 1, dtype=np.float32)
    step = en.PairProducts(max_interaction_features=10)
    step.fit(x, [], 123)
    out, _ = step.apply(x)
    scaled = x / x.std(axis=0)  # StandardScaler without centering: population std
    np.testing.assert_allclose(out[:, :p], scaled, rtol=1e-5)
    count = min(10, p * (p + 1) // 2)
    assert out.shape[1] == p + count
    pairs = list(zip(step.first.tolist(), step.second.tolist()))
    assert all(a <= b for a, b in pairs) and len(set(pairs)) == count
    if count == p * (p + 1) // 2:  # every pair a <= b is taken when there are at most 10
        assert set(pairs) == {(a, b) for a in range(p) for b in range(a, p)}
    for k, (a, b) in enumerate(pairs):
        np.testing.assert_allclose(out[:, p + k], scaled[:, a] * scaled[:, b], rtol=1e-4, atol=1e-6)


def test_column_order():
    x = np.arange(24.0).reshape(2, 12)
    step = en.ColumnOrder(mode="shuffle", offset=5)
    cat = step.fit(x, [0, 7], 99)
    perm = np.random.default_rng(99).permutation(12)
    np.testing.assert_array_equal(step.apply(x)[0], x[:, perm])
    assert cat == sorted(int(np.where(perm == c)[0][0]) for c in (0, 7))
    rot = en.ColumnOrder(mode="rotate", offset=5)
    rot.fit(x, [], 0)
    np.testing.assert_array_equal(rot.apply(x)[0], x[:, np.roll(np.arange(12), 5)])


def test_quantile_member_blocks():
    # original columns, their capped uniform quantile transform, then the SVD of the mean-imputed
    # columns scaled to unit variance
    g = np.random.default_rng(3)
    n, p = 300, 6
    x = g.standard_normal((n, p)) * np.array([1, 2, 3, 4, 5, 6]) + 10
    step = en.Redistribute(worker_tags=["quantile_uniform_all_data"], original_flag=True, svd_tag="svd", device="cpu")
    step.fit(x, [], 42)
    out, cat = step.apply(x)
    k = max(1, min(n // 10 + 1, p // 2))
    assert out.shape == (n, 2 * p + k) and cat == []
    np.testing.assert_array_equal(out[:, :p], x)
    qt = QuantileTransformer(output_distribution="uniform", n_quantiles=min(n // 5, n, 256), subsample=n,
                             random_state=42).fit(x)
    np.testing.assert_allclose(out[:, p:2 * p], qt.transform(x), rtol=0, atol=1e-12)
    assert (out[:, p:2 * p] >= 0).all() and (out[:, p:2 * p] <= 1).all()
    # the SVD block: U * S of the scaled matrix, components orthonormal, each component's
    # largest |U| entry positive
    scaled = np.hstack([x, qt.transform(x)])
    scaled = scaled / scaled.std(axis=0)
    svd = out[:, 2 * p:]
    comps = step.worker.named_steps["svd_worker"].transformer_list[1][1].named_steps["svd"].components_
    np.testing.assert_allclose(comps @ comps.T, np.eye(k), atol=1e-10)
    np.testing.assert_allclose(svd, scaled @ comps.T, rtol=1e-9, atol=1e-9)
    u = svd / np.linalg.norm(svd, axis=0)
    assert all(u[np.argmax(np.abs(u[:, j])), j] > 0 for j in range(k))
    sv = np.linalg.svd(scaled, compute_uv=False)[:k]
    np.testing.assert_allclose(np.linalg.norm(svd, axis=0), sv, rtol=1e-9)
    # a float32 member matrix stays float32 through the scaling, as the reference's
    # float-preserving steps keep it (np.nan_to_num, SimpleImputer, StandardScaler); the SVD is
    # then taken in float64 of those float32 values
    x32 = x.astype(np.float32)
    step32 = en.Redistribute(worker_tags=["quantile_uniform_all_data"], original_flag=True, svd_tag="svd",
                             device="cpu")
    step32.fit(x32, [], 42)
    out32 = step32.apply(x32)[0]
    columns = step32.worker.named_steps["worker"].transform(x32)
    branch = step32.worker.named_steps["svd_worker"].transformer_list[1][1]
    scaled32 = branch.named_steps["save_standard"].transform(columns)
    assert columns.dtype == np.float32 and scaled32.dtype == np.float32
    np.testing.assert_allclose(scaled32, columns / columns.astype(np.float64).std(axis=0), rtol=2e-7, atol=1e-6)
    np.testing.assert_allclose(out32[:, 2 * p:], scaled32.astype(np.float64) @ branch.named_steps["svd"].components_.T,
                               rtol=1e-9, atol=1e-9)


def test_per_column_kinds():
    g = np.random.default_rng(8)
    n = 2500
    cols = {
        "ordinal": g.integers(0, 5, n).astype(float),
        "normal": g.standard_normal(n),
        "positive_heavy_skew": g.pareto(1.5, n),
        "skewed_pos_01": g.beta(0.3, 6.0, n),
        "skewed": g.standard_normal(n) - 10.0 * (g.random(n) < 0.3),
        "other": g.standard_normal(n) + 6.0 * (g.random(n) < 0.5),
    }
    for want, col in cols.items():
        assert en.PerColumnTransform.kind(col) == want, want
    # the fitted transforms: standardized Yeo-Johnson for the negative skewed column, identity
    # for the normal one; fit rows capped at 2000 by a seeded draw
    x = np.stack([cols["normal"], cols["skewed"]], axis=1)
    t = en.PerColumnTransform(random_state=4, n_quantiles=max(n // 10, 2)).fit(x)
    out = t.transform(x)
    np.testing.assert_array_equal(out[:, 0], x[:, 0])
    rows = np.random.default_rng(4).choice(n, size=2000, replace=False)
    lam = stats.yeojohnson(x[rows, 1])[1]
    yj = stats.yeojohnson(x[:, 1], lmbda=lam)
    ref = (yj - stats.yeojohnson(x[rows, 1], lmbda=lam).mean()) / stats.yeojohnson(x[rows, 1], lmbda=lam).std()
    np.testing.assert_allclose(out[:, 1], ref, rtol=1e-3, atol=1e-3)


def test_category_codes():
    g = np.random.default_rng(2)
    n = 400
    levels = np.array([7.0, 3.0, 11.0])
    x = np.stack([g.standard_normal(n), levels[g.integers(0, 3, n)], g.standard_normal(n)], axis=1)
    step = en.CategoryCodes(encoding_strategy="ordinal_strict_feature_shuffled")
    cat = step.fit(x, [1], 17)
    out, cat_out = step.apply(x)
    assert cat == cat_out == [0]
    perm = np.random.default_rng(17).permutation(3)
    code = np.searchsorted(np.sort(levels), x[:, 1])  # OrdinalEncoder: sorted levels
    np.testing.assert_array_equal(out[:, 0], perm[code])
    np.testing.assert_array_equal(out[:, 1:], x[:, [0, 2]])
    # a column whose rarest level has fewer than 10 rows is not encoded
    x2 = x.copy()
    x2[:5, 1] = 99.0
    step2 = en.CategoryCodes(encoding_strategy="ordinal_strict_feature_shuffled")
    assert step2.fit(x2, [1], 17) == []
    np.testing.assert_array_equal(step2.apply(x2)[0], x2)


def test_row_fingerprint():
    g = np.random.default_rng(6)
    x = g.standard_normal((50, 4))
    x[10] = x[3]  # a duplicate context row
    step = en.RowFingerprint()
    step.fit(x, [2], 31)
    salt = int(np.random.default_rng(31).integers(0, 65536))
    out, cat = step.apply(x, is_test=False)
    fp = out[:, -1]
    assert cat == [2] and np.array_equal(out[:, :4], x)
    assert len(np.unique(fp)) == 50 and ((fp >= 0) & (fp < 1)).all()

    def h(row):
        return (int(hashlib.sha256(row.tobytes()).hexdigest(), 16) % 10**12) / 10**12

    assert fp[0] == h(x[0] + salt)
    q, _ = step.apply(x[:5], is_test=True)
    assert q[0, -1] == h(x[0] + salt + salt)  # query rows are salted twice and keep their hash


def test_members_on_config1_table():
    x_tr, y_tr, x_te, _ = case.table()
    y = ((y_tr - y_tr.mean()) / y_tr.std()).astype(np.float32)
    members = en.build_members(en.DEFAULT_MEMBERS, 0, "cpu")
    assert en.categorical_columns(x_tr) == []
    for i, m in enumerate(members):
        a, b, cat = m.features(x_tr, x_te, [], y)
        # 16 columns + 10 products; quantile members keep the originals, add their transform
        # and a 13-column SVD block; adaptive members transform in place; + 1 fingerprint
        assert a.shape == (1024, 66 if i < 4 else 27) and b.shape == (256, a.shape[1]) and cat == []
        assert np.isfinite(a).all() and np.isfinite(b).all()
    raw = en.build_members([{}], 0, "cpu")[0]
    a, b, _ = raw.features(x_tr, x_te, [], y)
    np.testing.assert_array_equal(a, x_tr)
    np.testing.assert_array_equal(b, x_te)


def test_wide_table_projection_gate():
    g = np.random.default_rng(1)
    narrow = g.standard_normal((60, 20))
    step = en.WideTableProjection(strategy="svd_all", n_features_threshold=256, binary_threshold=1.01,
                                  svd_components=512, svd_rows_per_component=3, device="cpu")
    assert step.fit(narrow, [3], 5) == [3]
    assert step.apply(narrow)[0] is narrow
    wide = g.standard_normal((90, 300))
    step.fit(wide, [], 5)
    out, cat = step.apply(wide)
    k = min(512, 299, 89, 90 // 3)
    assert out.shape == (90, k) and cat == []
    sv = np.linalg.svd(wide, compute_uv=False)[:k]
    np.testing.assert_allclose(np.linalg.norm(out, axis=0), sv, rtol=1e-4)


# ---- the reference's own fingerprint tests (tests/test_fingerprint_feature_encoder.py:16-68)
def _float_hash(row: np.ndarray) -> float:
    # float_hash_arr (preprocess.py:1225-1248): SHA-256 of the row's bytes as an integer, modulo
    # 10^12, over 10^12
    return (int(hashlib.sha256(row.tobytes()).hexdigest(), 16) % 10**12) / 10**12


def _fit_fingerprint(x):
    step = en.RowFingerprint()
    step.fit(x, [1], 42)
    return step


def test_fingerprint_context_and_query_use_single_and_double_salt():
    x = np.array([[1.0, 2.0], [3.5, -4.0]], dtype=np.float32)
    step = _fit_fingerprint(x)
    context, context_cat = step.apply(x, is_test=False)
    query, query_cat = step.apply(x.copy(), is_test=True)
    exp_context = np.asarray([_float_hash(row + step.salt) for row in x], dtype=x.dtype)
    exp_query = np.asarray([_float_hash(row + 2 * step.salt) for row in x], dtype=x.dtype)
    np.testing.assert_array_equal(context[:, :-1], x)
    np.testing.assert_array_equal(query[:, :-1], x)
    np.testing.assert_array_equal(context[:, -1], exp_context)
    np.testing.assert_array_equal(query[:, -1], exp_query)
    assert np.all(context[:, -1] != query[:, -1])
    assert context_cat == query_cat == [1]


def test_fingerprint_duplicate_context_rows_are_rehashed_but_query_duplicates_are_not():
    row = np.array([[1.0, 2.0]], dtype=np.float32)
    rows = np.repeat(row, repeats=2, axis=0)
    step = _fit_fingerprint(rows)
    context, _ = step.apply(rows, is_test=False)
    query, _ = step.apply(rows, is_test=True)
    first = _float_hash(row[0] + step.salt)
    second = _float_hash(row[0] + step.salt + 1)  # the duplicate: rehashed as row + salt + 1
    np.testing.assert_array_equal(context[:, -1], np.asarray([first, second], dtype=row.dtype))
    q = _float_hash(row[0] + 2 * step.salt)
    np.testing.assert_array_equal(query[:, -1], np.asarray([q, q], dtype=row.dtype))


def test_fingerprint_unseen_query_uses_the_query_namespace():
    step = _fit_fingerprint(np.array([[1.0, 2.0]], dtype=np.float32))
    query_rows = np.array([[3.0, 4.0]], dtype=np.float32)
    query, _ = step.apply(query_rows, is_test=True)
    np.testing.assert_array_equal(query[:, -1], np.asarray([_float_hash(query_rows[0] + 2 * step.salt)],
                                                           dtype=query_rows.dtype))


# ---- the reference's SVD rank rules (tests/test_preprocess_svd_rank.py:35-102)
def _svd_fit(x, **kw):
    step = en.WideTableProjection(strategy="svd_all", n_features_threshold=256, device="cpu", **kw)
    step.fit(x, [], 0)
    return step


def _svd_rank(step):
    return None if step.svd is None else int(step.svd.components_.shape[0])


def test_short_wide_table_is_reduced_not_rotated():
    x = np.random.default_rng(0).normal(size=(190, 1901))
    k = _svd_rank(_svd_fit(x, svd_components=512, svd_rows_per_component=3))
    assert k is not None and k <= 190 // 3 and k < min(x.shape) - 1


def test_tall_table_still_capped_by_svd_components():
    x = np.random.default_rng(1).normal(size=(6234, 2000))
    assert _svd_rank(_svd_fit(x, svd_components=512, svd_rows_per_component=3)) == 512


def test_default_rows_per_component_keeps_the_previous_rank():
    x = np.random.default_rng(5).normal(size=(300, 400))
    assert _svd_rank(_svd_fit(x, svd_components=256)) == 256


def test_rows_per_component_one_restores_the_previous_rank():
    x = np.random.default_rng(2).normal(size=(190, 1901))
    assert _svd_rank(_svd_fit(x, svd_components=512, svd_rows_per_component=1)) == 189


def test_narrow_table_is_untouched_by_the_gate():
    x = np.random.default_rng(3).normal(size=(5000, 10))
    assert _svd_fit(x, svd_components=512).svd is None


@pytest.mark.parametrize("n", [2, 3, 7])
def test_tiny_row_counts_stay_valid(n):
    x = np.random.default_rng(4).normal(size=(n, 400))
    k = _svd_rank(_svd_fit(x, svd_components=512))
    assert k is None or k >= 1


def test_shipped_configuration_enables_the_rank_rule_and_the_transductive_fit():
    sels = [m["HighDimFeatureSelector"] for m in en.DEFAULT_MEMBERS if "HighDimFeatureSelector" in m]
    assert sels
    for h in sels:
        assert h.get("svd_rows_per_component") == 3 and h.get("svd_components") == 512
        assert h.get("fit_on_test") is True


# ---- the reference's transductive wide-table fit (tests/test_hdf_selector_transductive_fit.py:28-75)
def _shifted_split(seed=0, n_train=400, n_test=100, n_features=40, n_shifted=10, shift=8.0):
    rng = np.random.default_rng(seed)
    x_train = rng.standard_normal((n_train, n_features))
    x_test = rng.standard_normal((n_test, n_features))
    x_test[:, :n_shifted] += shift  # test values far outside the context range
    return x_train.astype(np.float32), x_test.astype(np.float32)


def _selector(**kw):
    return en.WideTableProjection(strategy="svd_all", svd_components=8, n_features_threshold=16, device="cpu", **kw)


def test_transductive_flag_defaults_off_and_is_stored():
    assert _selector().fit_on_test is False
    assert _selector(fit_on_test=True).fit_on_test is True


def test_member_fits_the_projection_on_context_plus_test_only_when_enabled(monkeypatch):
    x_train, x_test = _shifted_split()
    seen = {}
    real_fit = en.WideTableProjection.fit

    def recording_fit(self, x, categorical, seed, y=None):
        seen["rows"] = len(x)
        seen["y"] = y
        return real_fit(self, x, categorical, seed, y=y)

    monkeypatch.setattr(en.WideTableProjection, "fit", recording_fit)
    for flag, rows in ((True, len(x_train) + len(x_test)), (False, len(x_train))):
        seen.clear()
        member = en.Member({"HighDimFeatureSelector": {"strategy": "svd_all", "svd_components": 8,
                                                       "n_features_threshold": 16, "fit_on_test": flag}},
                           list(range(en.SEED_SLOTS)), 0, "cpu")
        member.features(x_train, x_test, [], np.zeros(len(x_train), dtype=np.float32))
        assert seen["rows"] == rows
        if flag:
            assert seen["y"] is None  # labels are never part of the transductive fit


def test_transductive_projection_reconstructs_shifted_test_rows_better():
    x_train, x_test = _shifted_split()
    ctx_only, both = _selector(), _selector()
    ctx_only.fit(x_train, [], 0)
    both.fit(np.vstack([x_train, x_test]), [], 0)
    assert ctx_only.svd is not None and both.svd is not None

    def recon_error(step):
        comps = np.asarray(step.svd.components_, dtype=np.float64)
        x = x_test.astype(np.float64)
        return float(np.mean((x - x @ comps.T @ comps) ** 2))

    assert recon_error(both) < 0.5 * recon_error(ctx_only)


def test_disabled_transductive_flag_is_byte_identical():
    x_train, x_test = _shifted_split()
    a, b = _selector(), _selector(fit_on_test=False)
    a.fit(x_train, [], 0)
    b.fit(x_train, [], 0)
    np.testing.assert_array_equal(a.apply(x_test)[0], b.apply(x_test)[0])


def test_a_fitted_member_transforms_new_query_rows_as_a_fresh_fit_would():
    # every default step is fitted on the context alone (the transductive projection is a
    # pass-through below 257 columns, whatever the rows), so a member fitted once transforms
    # other query rows to exactly what fitting it again with them gives
    x_tr, y_tr, x_te, _ = case.table()
    y = ((y_tr - y_tr.mean()) / y_tr.std()).astype(np.float32)
    other = np.random.default_rng(9).standard_normal((40, x_tr.shape[1])).astype(np.float32)
    for i, (fitted, fresh) in enumerate(zip(en.build_members(en.DEFAULT_MEMBERS, 0, "cpu"),
                                            en.build_members(en.DEFAULT_MEMBERS, 0, "cpu"))):
        a, _, _ = fitted.features(x_tr, x_te, [], y)
        assert fitted.reads_queries is False
        a2, b2, _ = fresh.features(x_tr, other, [], y)
        np.testing.assert_array_equal(a, a2)
        np.testing.assert_array_equal(fitted.query_features(other), b2)
    # an active transductive projection reads the query rows: no reuse
    wide = np.random.default_rng(1).standard_normal((90, 300)).astype(np.float32)
    member = en.Member({"HighDimFeatureSelector": {"strategy": "svd_all", "svd_components": 8,
                                                   "n_features_threshold": 256, "fit_on_test": True}},
                       list(range(en.SEED_SLOTS)), 0, "cpu")
    member.features(wide[:60], wide[60:], [], np.zeros(60, dtype=np.float32))
    assert member.reads_queries is True
    with pytest.raises(RuntimeError):
        member.query_features(wide[60:])
