"""The inference-time preprocessing ensemble in front of ``NoriRegressor``.

The reference scores a table through several members (src/synthefy_nori/inference/predictor.py:
352-418 assembles them, :541-600 fits a member's steps on the context and applies them to both
splits, :2972-3000 runs the members, :3533 averages their quantile banks). Each member reshapes
the feature matrix its own way before the model sees it: a projection of very wide tables, a
cap on the feature count, pairwise products, dropping constant columns, a per-column
redistribution (quantile-uniform, or a transform chosen per column), categorical codes, a row
fingerprint and a column shuffle -- each step seeded from the member's slot of one seed list.

This module restates that for numeric tables, with the reference's configuration format (the
member dictionaries of configs/default_inference.json, whose keys are the step names) and the
same third-party building blocks (sklearn's transformers, scipy's statistics, torch's SVD on
the model's device), so a member's features are the ones the reference would build from the
same inputs and seed. The steps:

=============================  ==============================================================
config key                     here
=============================  ==============================================================
HighDimFeatureSelector         ``WideTableProjection`` (the gate; SVD, correlation, mutual
                               information and extra-trees strategies)
MaxFeatureSubsampler           ``FeatureCap``
PolynomialInteractionGenerator ``PairProducts``
(always)                       ``DropConstantColumns``
MADWinsorizer                  ``MadClip``
RebalanceFeatureDistribution   ``Redistribute`` (+ ``PerColumnTransform`` for "adaptive",
                               ``RevertingPowerTransform`` for "power")
CategoricalFeatureEncoder      ``CategoryCodes`` (ordinal codes or one-hot columns)
FingerprintFeatureEncoder      ``RowFingerprint``
FeatureShuffler                ``ColumnOrder``
=============================  ==============================================================

Each step has ``fit(x, categorical, seed, y=None) -> categorical`` on the context rows and
``apply(x, is_test) -> (x, categorical)`` on either split.
"""

from __future__ import annotations

import copy
import hashlib
import json
import random
import warnings

import numpy as np
import torch
from sklearn.base import BaseEstimator, TransformerMixin
from sklearn.compose import ColumnTransformer
from sklearn.decomposition import TruncatedSVD
from sklearn.ensemble import ExtraTreesRegressor
from sklearn.feature_selection import mutual_info_regression
from sklearn.impute import SimpleImputer
from sklearn.pipeline import FeatureUnion, Pipeline
from sklearn.preprocessing import (
    FunctionTransformer,
    MinMaxScaler,
    OneHotEncoder,
    OrdinalEncoder,
    PowerTransformer,
    QuantileTransformer,
    RobustScaler,
    StandardScaler,
)

from .degradation import SvdFallbackWarning

__all__ = ["DEFAULT_MEMBERS", "Member", "build_members", "categorical_columns", "read_members"]

# configs/default_inference.json: four quantile-uniform members (original columns kept, an SVD
# block appended) and four per-column "adaptive" members, all with the same other steps.
_COMMON = {
    "MaxFeatureSubsampler": {"max_features": 500},
    "PolynomialInteractionGenerator": {"max_interaction_features": 10},
    "CategoricalFeatureEncoder": {"encoding_strategy": "ordinal_strict_feature_shuffled"},
    "FeatureShuffler": {"mode": "shuffle"},
    "FingerprintFeatureEncoder": True,
    "HighDimFeatureSelector": {"strategy": "svd_all", "svd_components": 512, "n_features_threshold": 256,
                               "binary_threshold": 1.01, "svd_rows_per_component": 3, "fit_on_test": True},
}
DEFAULT_MEMBERS: tuple[dict, ...] = tuple(
    [dict(_COMMON, RebalanceFeatureDistribution={"worker_tags": ["quantile_uniform_all_data"], "discrete_flag": False,
                                                 "original_flag": True, "svd_tag": "svd"})] * 4
    + [dict(_COMMON, RebalanceFeatureDistribution={"worker_tags": ["adaptive"], "discrete_flag": False,
                                                   "original_flag": False, "svd_tag": None})] * 4
)

SEED_SLOTS = 10  # seeds per member (predictor.py:219); the wide-table projection takes the last
MIN_ROWS_FOR_CATEGORIES = 100  # predictor.py:216
MIN_UNIQUE_FOR_NUMERIC = 4  # predictor.py:218
QUANTILE_CAP, QUANTILE_SUBSAMPLE_CAP = 256, 10000  # preprocess.py:63-70 (their defaults)
QUANTILE_SUBSAMPLE_DEFAULT = 10000  # sklearn's QuantileTransformer default subsample
ONE_HOT_MAX_ELEMENTS = 1_000_000  # preprocess.py:729-731: a wider one-hot matrix is not built
ADAPTIVE_FIT_ROWS = 2000  # preprocess.py:380-384
_MAX_SEED = int(np.iinfo(np.int32).max)


def read_members(config) -> list[dict]:
    """A member list from a list of dictionaries or a JSON file path (predictor.py:77-94)."""
    if isinstance(config, str):
        with open(config) as f:
            config = json.load(f)
    members = copy.deepcopy(list(config))
    for m in members:
        if (m.get("retrieval_config") or {}).get("use_retrieval"):
            raise ValueError("retrieval inference has been removed; omit retrieval_config and use the full context")
    return members


def _rng(seed) -> tuple[int, np.random.Generator]:
    """(int seed, Generator) of a step's seed, as preprocess.py:461-478 derives them."""
    if seed is None:
        g = np.random.default_rng()
        return int(g.integers(0, _MAX_SEED)), g
    return int(seed), np.random.default_rng(int(seed))


def categorical_columns(x: np.ndarray) -> list[int]:
    """Columns of a numeric context read as categorical: fewer than 4 distinct values, when the
    context has at least 100 rows (predictor.py:616-623)."""
    if x.shape[0] < MIN_ROWS_FOR_CATEGORIES:
        return []
    return [j for j in range(x.shape[1]) if len(np.unique(x[:, j])) < MIN_UNIQUE_FOR_NUMERIC]


# ---------------------------------------------------------------------------------- helpers
def _inf_to_nan(x):
    """Infinities to NaN, in the input's own float type (float32 stays float32)."""
    out = np.array(x, copy=True)
    if out.dtype.kind == "f":
        out[np.isinf(out)] = np.nan
    return out


def _nonfinite_to_nan():
    return FunctionTransformer(func=_inf_to_nan, inverse_func=_identity, check_inverse=False)


def _mean_fill():
    return SimpleImputer(missing_values=np.nan, strategy="mean", keep_empty_features=True)


def _shift_nonnegative(x):
    """The matrix moved up by the magnitude of its smallest entry. Stateless, as the reference's
    step is (preprocess.py:45-46): the query matrix is moved by its own minimum."""
    return x + np.abs(np.nanmin(x))


def _plus_epsilon(x):
    return x + 1e-10


def _identity(x):
    return x


def _capped_quantiles(output: str, n_quantiles: int, seed: int, subsample: int, n_rows: int) -> QuantileTransformer:
    """sklearn's QuantileTransformer with n_quantiles and subsample capped as the reference caps
    them at fit time (preprocess.py:53-70): at most 256 quantiles, the row count, and 10000 rows."""
    return QuantileTransformer(output_distribution=output, n_quantiles=max(2, min(int(n_quantiles), n_rows, QUANTILE_CAP)),
                               subsample=min(int(subsample), QUANTILE_SUBSAMPLE_CAP), random_state=seed)


class DeviceSVD(BaseEstimator, TransformerMixin):
    """The exact truncated SVD of the context (torch.linalg.svd in float64 on the model's
    device), signs fixed so each component's largest-magnitude entry of U is positive (sklearn's
    u-based svd_flip): ``fit_transform`` is U*S, ``transform`` projects on the components
    (preprocess.py:86-156). When the device solver raises (out of memory, no convergence),
    sklearn's TruncatedSVD with ``algorithm`` (default randomized) and ``random_state`` takes
    over, as the reference falls back (preprocess.py:107-112); the projection runs on the GPU
    when the device is one, else in numpy."""

    def __init__(self, n_components: int, device, random_state=None, algorithm=None):
        self.n_components = int(n_components)
        self.device = device
        self.random_state = random_state
        self.algorithm = algorithm

    def fit(self, x, y=None):
        self.fit_transform(x)
        return self

    def fit_transform(self, x, y=None):
        x = np.asarray(x, dtype=np.float64)
        try:
            return self._device_fit(x)
        except Exception:
            svd = TruncatedSVD(n_components=self.n_components, algorithm=self.algorithm or "randomized",
                               random_state=self.random_state)
            out = svd.fit_transform(x)
            self.components_ = svd.components_
            return out

    def _device_fit(self, x):
        xt = torch.from_numpy(x).to(self.device)
        n, p = xt.shape
        k = max(1, min(self.n_components, p, n))
        u, s, vh = torch.linalg.svd(xt, full_matrices=False)
        u, s, vh = u[:, :k], s[:k], vh[:k]
        signs = torch.sign(u[u.abs().argmax(dim=0), torch.arange(k, device=xt.device)])
        signs = torch.where(signs == 0, torch.ones_like(signs), signs)
        self.components_ = (vh * signs[:, None]).cpu().numpy()
        return (u * (s * signs)[None, :]).cpu().numpy()

    def transform(self, x):
        x = np.asarray(x, dtype=np.float64)
        if torch.device(self.device).type == "cuda":
            try:
                xt = torch.from_numpy(x).to(self.device)
                return (xt @ torch.from_numpy(self.components_).to(self.device).T).cpu().numpy()
            except torch.cuda.OutOfMemoryError:
                pass
        return x @ self.components_.T


# ---------------------------------------------------------------------------------- steps
class WideTableProjection:
    """HighDimFeatureSelector (preprocess.py:1323-1684): a pass-through unless the table has
    more than ``n_features_threshold`` columns or at least ``binary_threshold`` of them are
    binary (exactly two distinct finite values); then, by strategy:

    * ``svd_all``: the NaN-zeroed columns replaced by their first
      min(svd_components, p - 1, n - 1, n // svd_rows_per_component) SVD coordinates;
    * ``svd_binary``: when the binary columns are at least ``binary_threshold`` of the table and
      at least two, they are replaced by the first min(svd_components, n_binary - 1, n - 1) SVD
      coordinates of their NaN-zeroed block, placed after the other columns;
    * ``corr`` / ``mi`` / ``extratrees``: the ``top_k`` columns with the largest |Pearson
      correlation| with the target, sklearn's mutual information, or an extra-trees forest's
      impurity importances (the last two on NaN-zeroed rows with a finite target, at most
      ``subsample_rows`` of them drawn without replacement), kept in table order.

    The target-driven strategies pass through when there is no target (the fit on context +
    query rows, ``fit_on_test``, has none), when it has the wrong length or fewer than
    max(10, top_k // 4) finite values, or when the scorer raises; so does any other strategy
    name. An SVD that raises warns with ``SvdFallbackWarning`` and degrades as the reference
    does: at fit, to a pass-through; at transform, to one all-zero column (``svd_all``) or to
    the non-binary columns (``svd_binary``)."""

    def __init__(self, *, strategy="passthrough", top_k=256, n_features_threshold=128, binary_threshold=0.5,
                 svd_components=64, svd_rows_per_component=1, extratrees_n_estimators=100, subsample_rows=5000,
                 fit_on_test=False, device=None):
        self.strategy, self.fit_on_test = strategy, bool(fit_on_test)
        self.top_k = int(top_k)
        self.n_features_threshold, self.binary_threshold = int(n_features_threshold), float(binary_threshold)
        self.svd_components, self.rows_per_component = int(svd_components), max(1, int(svd_rows_per_component))
        self.n_trees, self.subsample_rows = int(extratrees_n_estimators), int(subsample_rows)
        self.device = device
        self.svd, self.selected, self.categorical = None, None, []

    @staticmethod
    def binary_columns(x) -> np.ndarray:
        """Columns with exactly two distinct finite values."""
        return np.array([len(np.unique(c[np.isfinite(c)])) == 2 for c in x.T], dtype=bool)

    @staticmethod
    def correlations(x, y) -> np.ndarray:
        """|Pearson r| of each column with the target over the rows where both are finite; 0 for a
        column with fewer than 3 such rows or a (near-)constant side (preprocess.py:1434-1451)."""
        scores = np.zeros(x.shape[1], dtype=np.float64)
        for j in range(x.shape[1]):
            ok = np.isfinite(x[:, j]) & np.isfinite(y)
            if ok.sum() < 3:
                continue
            a, b = x[ok, j], y[ok]
            if a.std() < 1e-8 or b.std() < 1e-8:
                continue
            r = np.corrcoef(a, b)[0, 1]
            scores[j] = abs(r) if np.isfinite(r) else 0.0
        return scores

    def _passthrough(self, categorical):
        self.svd, self.selected, self.categorical = None, None, list(categorical)
        return list(self.categorical)

    def _degraded(self, stage, exc, fallback):
        warnings.warn(f"HighDimFeatureSelector(strategy={self.strategy!r}): SVD {stage} failed "
                      f"({type(exc).__name__}: {str(exc)[:120]}) -> {fallback}. Predictions are degraded, not "
                      f"the configured pipeline; strict_pipeline() makes this an error.", SvdFallbackWarning,
                      stacklevel=3)

    @staticmethod
    def _remap(kept, categorical):
        position = {int(old): new for new, old in enumerate(kept)}
        return sorted(position[int(c)] for c in categorical if int(c) in position)

    def fit(self, x, categorical, seed, y=None):
        x = np.asarray(x, dtype=np.float64)
        n, p = x.shape
        if self.strategy == "passthrough" or p == 0:
            return self._passthrough(categorical)
        binary = self.binary_columns(x)
        frac = float(binary.mean())
        if not (p > self.n_features_threshold or frac >= self.binary_threshold):
            return self._passthrough(categorical)
        seed_int = int(seed) % 2**31
        if self.strategy in ("svd_all", "svd_binary"):
            if self.strategy == "svd_binary":
                if frac < self.binary_threshold or int(binary.sum()) < 2:
                    return self._passthrough(categorical)
                mask = binary
                k = max(1, min(self.svd_components, int(binary.sum()) - 1, n - 1))
                fallback = f"passthrough of all {p} raw columns ({int(binary.sum())} binary columns left unprojected)"
            else:
                mask = np.ones(p, dtype=bool)
                k = max(1, min(self.svd_components, p - 1, n - 1, n // self.rows_per_component))
                fallback = f"passthrough of all {p} raw columns (no reduction to {k} components)"
            try:
                svd = DeviceSVD(k, self.device, random_state=seed_int)
                svd.fit(np.where(np.isnan(x[:, mask]), 0.0, x[:, mask]))
            except Exception as exc:
                self._degraded("fit", exc, fallback)
                return self._passthrough(categorical)
            self.svd, self.selected, self.mask, self.keep = svd, None, mask, np.where(~mask)[0]
            self.categorical = self._remap(self.keep, categorical) if self.strategy == "svd_binary" else []
            return list(self.categorical)
        if y is None or self.strategy not in ("corr", "mi", "extratrees"):
            return self._passthrough(categorical)
        y = np.asarray(y, dtype=np.float64).ravel()
        if y.size != n:
            return self._passthrough(categorical)
        finite = np.isfinite(y)
        if int(finite.sum()) < max(10, self.top_k // 4):
            return self._passthrough(categorical)
        if self.strategy == "corr":
            scores = self.correlations(x, y)
        else:
            xs, ys = x[finite], y[finite]
            if len(xs) > self.subsample_rows:
                rows = np.random.default_rng(int(seed) % 2**32).choice(len(xs), size=self.subsample_rows, replace=False)
                xs, ys = xs[rows], ys[rows]
            xs = np.where(np.isnan(xs), 0.0, xs)
            try:
                if self.strategy == "mi":
                    scores = mutual_info_regression(xs, ys, random_state=seed_int)
                else:
                    forest = ExtraTreesRegressor(n_estimators=self.n_trees, random_state=seed_int, n_jobs=-1)
                    scores = forest.fit(xs, ys).feature_importances_
            except Exception:
                return self._passthrough(categorical)
        top = max(1, min(self.top_k, p))
        self.svd, self.selected = None, np.sort(np.argsort(-np.asarray(scores), kind="stable")[:top])
        self.categorical = self._remap(self.selected, categorical)
        return list(self.categorical)

    def apply(self, x, is_test=False):
        if self.selected is not None:
            return x[:, self.selected], list(self.categorical)
        if self.svd is None:
            return x, list(self.categorical)
        x = np.asarray(x, dtype=np.float64)
        block = np.where(np.isnan(x[:, self.mask]), 0.0, x[:, self.mask])
        try:
            coords = self.svd.transform(block)
        except Exception as exc:
            if self.strategy == "svd_all":
                self._degraded("transform", exc, f"a single all-zero column for {x.shape[0]} rows "
                                                 f"(all {block.shape[1]} features dropped)")
                return np.zeros((x.shape[0], 1), dtype=np.float32), []
            self._degraded("transform", exc, f"dropping the {block.shape[1]} SVD-projected columns, keeping the "
                                             f"{len(self.keep)} non-binary ones")
            return x[:, self.keep].astype(np.float32), list(self.categorical)
        if self.strategy == "svd_all":
            return coords.astype(np.float32), []
        return np.concatenate([x[:, self.keep], coords], axis=1).astype(np.float32), list(self.categorical)

    def depends_on_rows(self) -> bool:
        """Whether the fit's outcome depends on the rows' values, not only on the column count:
        an active projection does, and so does the gate when binary columns can open it. The
        target-driven strategies pass through on a fit without a target."""
        if self.strategy not in ("svd_all", "svd_binary"):
            return False
        return self.svd is not None or self.binary_threshold <= 1.0


class FeatureCap:
    """MaxFeatureSubsampler (preprocess.py:1685-1731): at most ``max_features`` columns, a sorted
    random subset when there are more."""

    def __init__(self, *, max_features=500):
        if max_features <= 0:
            raise ValueError("max_features must be > 0")
        self.max_features = int(max_features)

    def fit(self, x, categorical, seed, y=None):
        _, g = _rng(seed)
        p = x.shape[1]
        self.keep = np.arange(p) if p <= self.max_features else np.sort(g.choice(p, size=self.max_features, replace=False))
        where = {int(old): new for new, old in enumerate(self.keep.tolist())}
        self.categorical = sorted(where[int(c)] for c in categorical if int(c) in where)
        return self.categorical

    def apply(self, x, is_test=False):
        return x[:, self.keep], self.categorical


class PairProducts:
    """PolynomialInteractionGenerator (preprocess.py:1734-1848): columns divided by their standard
    deviation (StandardScaler without centering), then ``max_interaction_features`` products of
    random column pairs (a <= b, no pair twice) appended."""

    def __init__(self, *, max_interaction_features=None, random_generator=None, disable_above_n_features=None):
        self.max_pairs = int(max_interaction_features) if max_interaction_features else 100
        self.disable_above = None if disable_above_n_features is None else int(disable_above_n_features)

    def fit(self, x, categorical, seed, y=None):
        _, g = _rng(seed)
        self.categorical = list(categorical)
        self.off = x.size == 0 or (self.disable_above is not None and x.shape[1] > self.disable_above)
        if self.off:
            return self.categorical
        p = x.shape[1]
        count = min(self.max_pairs, p * (p + 1) // 2)
        self.scaler = StandardScaler(with_mean=False).fit(x)
        first = g.choice(np.arange(p), size=count, replace=True)
        second = np.full_like(first, -1)
        for i in range(count):
            while second[i] == -1:
                a = first[i]
                taken = second[first == a]
                free = [b for b in range(a, p) if b not in taken]
                if not free:
                    first[i] = g.choice(np.arange(p))
                else:
                    second[i] = g.choice(free)
        self.first, self.second = first, second
        return self.categorical

    def apply(self, x, is_test=False):
        if x.size == 0:
            return x, []
        if self.off:
            return x, self.categorical
        s = self.scaler.transform(x)
        return np.column_stack([s, s[:, self.first] * s[:, self.second]]), self.categorical


class DropConstantColumns:
    """FilterValidFeatures (preprocess.py:482-532): drops the columns whose context values all
    equal the first row's, and all-NaN ones (raises when none is left)."""

    def fit(self, x, categorical, seed, y=None):
        same = (x[0:1, :] == x).mean(axis=0)
        keep = (same < 1.0) & ~np.all(np.isnan(x), axis=0)
        if y is not None and len(x) > len(y):
            n = len(y)
            keep &= ~(np.all(np.isnan(x[:n]), axis=0) | np.all(np.isnan(x[n:]), axis=0))
        if not np.any(keep):
            raise ValueError("All features are constant! Please check your data.")
        self.keep = keep
        self.categorical = [i for i, j in enumerate(np.where(keep)[0]) if j in categorical]
        return self.categorical

    def apply(self, x, is_test=False):
        return x[:, self.keep], self.categorical


class MadClip:
    """MADWinsorizer (preprocess.py:535-623): each non-categorical column clipped to its context
    median +/- n_mad * 1.4826 * MAD (no clip where that scale is below 1e-8), NaN kept."""

    def __init__(self, *, n_mad=6.0, skip_categorical=True, soft_log_clip=False):
        self.n_mad, self.skip_categorical, self.soft = float(n_mad), bool(skip_categorical), bool(soft_log_clip)

    def fit(self, x, categorical, seed, y=None):
        x = np.asarray(x, dtype=np.float64)
        med = np.nanmedian(x, axis=0)
        scale = np.nanmedian(np.abs(x - med), axis=0) * 1.4826
        scale = np.where(scale > 1e-8, scale, np.inf)
        self.lo, self.hi = med - self.n_mad * scale, med + self.n_mad * scale
        self.cat = np.zeros(x.shape[1], dtype=bool)
        if self.skip_categorical and categorical:
            self.cat[[i for i in categorical if 0 <= i < x.shape[1]]] = True
        return categorical

    def apply(self, x, is_test=False):
        x = np.asarray(x, dtype=np.float64)
        if x.shape[1] != len(self.lo):
            return x.astype(np.float32), []
        if self.soft:
            hi_x, lo_x = np.maximum(x - self.hi, 0.0), np.maximum(self.lo - x, 0.0)
            out = np.where(hi_x > 0, self.hi + np.log1p(hi_x), x)
            out = np.where(lo_x > 0, self.lo - np.log1p(lo_x), out)
        else:
            out = np.clip(x, self.lo, self.hi)
        if self.skip_categorical and self.cat.any():
            out[:, self.cat] = x[:, self.cat]
        out = np.where(np.isnan(x), np.nan, out)
        return out.astype(np.float32), list(np.where(self.cat)[0])


class PerColumnTransform(BaseEstimator, TransformerMixin):
    """The "adaptive" redistribution (preprocess.py:239-437): every column gets the transform its
    own distribution calls for, chosen on the whole context column -- identity for columns of
    fewer than 10 distinct values or that look normal (Shapiro statistic > 0.95 on the first
    3000), log1p + standardize for non-negative heavy right tails (Fisher-Pearson skew > 5),
    exp for skewed columns inside [0, 1], min-max to [0.1, 1] + Box-Cox for other skewed
    non-negative ones, Yeo-Johnson for other skewed ones (|median skew| > 1.1), a normal quantile
    transform otherwise -- and fitted on at most 2000 context rows."""

    def __init__(self, *, random_state=None, n_quantiles=100):
        self.random_state, self.n_quantiles = random_state, max(2, int(n_quantiles))

    @staticmethod
    def _median_skew(v):
        v = v[np.isfinite(v)]
        if len(v) < 3:
            return 0.0
        sd = float(np.nanstd(v))
        return 0.0 if sd < 1e-8 else float(3.0 * (np.nanmean(v) - np.nanmedian(v)) / sd)

    @classmethod
    def kind(cls, col) -> str:
        from scipy import stats

        v = col[np.isfinite(col)]
        if len(v) < 3:
            return "identity"
        if len(np.unique(v)) < 10:
            return "ordinal"
        skew = cls._median_skew(v)
        lo, hi = float(np.min(v)), float(np.max(v))
        if lo >= 0:
            try:
                if float(stats.skew(v, bias=False, nan_policy="omit")) > 5.0:
                    return "positive_heavy_skew"
            except Exception:
                pass
        if abs(skew) > 1.1:
            if lo >= 0:
                return "skewed_pos_01" if hi <= 1.0 else "skewed_pos"
            return "skewed"
        try:
            if float(stats.shapiro(v[:3000] if len(v) > 3000 else v).statistic) > 0.95:
                return "normal"
        except Exception:
            pass
        return "other"

    def _transformer(self, kind, n_rows):
        if kind in ("identity", "ordinal", "normal"):
            return FunctionTransformer()
        if kind == "skewed_pos_01":
            return FunctionTransformer(func=np.exp, inverse_func=np.log, check_inverse=False)
        if kind == "positive_heavy_skew":
            return Pipeline([("log1p", FunctionTransformer(func=np.log1p, inverse_func=np.expm1, check_inverse=False)),
                             ("std", StandardScaler())])
        if kind == "skewed_pos":
            return Pipeline([("mm", MinMaxScaler(feature_range=(0.1, 1.0), clip=True)),
                             ("bc", PowerTransformer(method="box-cox", standardize=True))])
        if kind == "skewed":
            return PowerTransformer(method="yeo-johnson", standardize=True)
        return _capped_quantiles("normal", self.n_quantiles, self.random_state, int(1e6), n_rows)

    def fit(self, x, y=None):
        x = np.asarray(x, dtype=np.float64)
        n = x.shape[0]
        fit_rows = x
        if n > ADAPTIVE_FIT_ROWS:
            fit_rows = x[np.random.default_rng(self.random_state).choice(n, size=ADAPTIVE_FIT_ROWS, replace=False)]
        self.kinds, self.transforms = [], []
        for j in range(x.shape[1]):
            kind = self.kind(x[:, j])
            t = self._transformer(kind, fit_rows.shape[0])
            try:
                t.fit(fit_rows[:, j : j + 1])
            except Exception:
                kind, t = "identity", FunctionTransformer().fit(x[:, j : j + 1])
            self.kinds.append(kind)
            self.transforms.append(t)
        return self

    def transform(self, x):
        x = np.asarray(x, dtype=np.float64)
        if x.shape[1] != len(self.transforms):
            raise ValueError(f"fitted on {len(self.transforms)} columns, got {x.shape[1]}")
        out = np.empty_like(x)
        for j, t in enumerate(self.transforms):
            try:
                out[:, j : j + 1] = np.asarray(t.transform(x[:, j : j + 1]), dtype=np.float64)
            except Exception:
                out[:, j] = 0.0
        return np.nan_to_num(out, nan=0.0, posinf=0.0, neginf=0.0)


class RevertingPowerTransform(PowerTransformer):
    """RobustPowerTransformer (preprocess.py:185-236): a per-column Yeo-Johnson transform, each
    column standardized, that hands a column back unchanged when the fit-time output of that
    column has a variance more than ``var_tolerance`` away from 1 or any value above
    ``max_abs_value`` (a constant column, or one with a far outlier). A column whose lambda
    search raises keeps lambda NaN and is left as it is.

    Standardized, although the reference constructs its worker with ``standardize=False``: it
    takes that through ``**kwargs``, which sklearn's ``clone`` cannot see, and ColumnTransformer
    fits a clone, rebuilt with PowerTransformer's default ``standardize=True``. As there, the
    fit returns the transformed (not reverted) columns, so the steps after this one are fitted
    on them while ``transform`` feeds them the reverted columns."""

    def __init__(self, var_tolerance: float = 1e-3, max_abs_value: float = 100.0, *, method="yeo-johnson",
                 standardize=True, copy=True):
        super().__init__(method=method, standardize=standardize, copy=copy)
        self.var_tolerance, self.max_abs_value = var_tolerance, max_abs_value

    def fit(self, x, y=None):
        super().fit(x, y)
        self.revert_ = np.array([], dtype=int)
        return self

    def fit_transform(self, x, y=None):
        z = super().fit_transform(x, y)
        off = np.abs(np.nanvar(z, axis=0) - 1.0) > self.var_tolerance
        large = np.any(z > self.max_abs_value, axis=0)
        self.revert_ = np.flatnonzero(off | large)
        return z

    def transform(self, x):
        z = super().transform(x)
        if len(self.revert_):
            z[:, self.revert_] = np.asarray(x)[:, self.revert_]
        return z

    def _yeo_johnson_optimize(self, x):
        try:
            with warnings.catch_warnings():
                warnings.filterwarnings("ignore", message=r"overflow encountered", category=RuntimeWarning)
                return super()._yeo_johnson_optimize(x)
        except Exception:
            return np.nan

    def _yeo_johnson_transform(self, x, lmbda):
        return x if np.isnan(lmbda) else super()._yeo_johnson_transform(x, lmbda)


class Redistribute:
    """RebalanceFeatureDistribution (preprocess.py:916-1222): the numeric columns through each
    worker transform, next to either all original columns (``original_flag``) or the categorical
    ones, and optionally an SVD block of the result (``svd_tag="svd"``: mean-imputed columns
    scaled to unit variance, min(n // 10 + 1, p // 2) components). Worker tags:

    * quantile_uniform_10 / _5 / _all_data, quantile_norm_all_data: sklearn's quantile transform,
      capped at 256 quantiles and 10000 fitting rows;
    * quantile_norm_10 / _5: what the reference's fitted worker is -- a uniform (not normal)
      quantile transform with min(n // 10 or n // 5, n, 10000) quantiles, unseeded: its QTx takes
      output_distribution and random_state through ``**kwargs``, which sklearn's ``clone`` (the
      ColumnTransformer fits a clone) cannot see;
    * power: ``RevertingPowerTransform`` -> infinities to NaN -> mean fill -> standardize ->
      infinities to NaN -> mean fill;
    * logNormal: infinities to NaN -> mean fill -> shift by the matrix's smallest magnitude ->
      + 1e-10 -> log -> infinities to NaN -> mean fill;
    * adaptive: ``PerColumnTransform``; robust and squash: sklearn's RobustScaler(unit_variance);
    * None and any other name (the reference's fallback, which takes the default "quantile"
      too): the identity.

    The kernel-density-integral tags (kdi*, norm_and_kdi) need the third-party ``kditransform``
    package (the reference's pyproject asks for kditransform>=1.0), which this environment does
    not have; they raise NotImplementedError."""

    def __init__(self, *, worker_tags=None, discrete_flag=False, original_flag=False, svd_tag=None,
                 joined_svd_feature=True, joined_log_normal=True, device=None):
        self.tags = list(worker_tags) if worker_tags is not None else ["quantile"]
        self.discrete_flag, self.original_flag, self.svd_tag = bool(discrete_flag), bool(original_flag), svd_tag
        self.device = device

    def _worker(self, tag, n, seed):
        if tag == "quantile_uniform_10":
            return _capped_quantiles("uniform", max(n // 10, 2), seed, 10_000, n)
        if tag == "quantile_uniform_5":
            return _capped_quantiles("uniform", max(n // 5, 2), seed, 10_000, n)
        if tag == "quantile_uniform_all_data":
            return _capped_quantiles("uniform", max(n // 5, 2), seed, n, n)
        if tag == "quantile_norm_all_data":
            return _capped_quantiles("normal", max(n // 5, 2), seed, n, n)
        if tag in ("quantile_norm_10", "quantile_norm_5"):
            wanted = max(n // (10 if tag.endswith("_10") else 5), 2)
            return QuantileTransformer(output_distribution="uniform", random_state=None,
                                       n_quantiles=max(1, min(wanted, n, QUANTILE_SUBSAMPLE_DEFAULT)),
                                       subsample=QUANTILE_SUBSAMPLE_DEFAULT)
        if tag == "power":
            return Pipeline([("power", RevertingPowerTransform()), ("inf_a", _nonfinite_to_nan()),
                             ("fill_a", _mean_fill()), ("scale", StandardScaler()),
                             ("inf_b", _nonfinite_to_nan()), ("fill_b", _mean_fill())])
        if tag == "logNormal":
            return Pipeline([("inf_a", _nonfinite_to_nan()), ("fill_a", _mean_fill()),
                             ("shift", FunctionTransformer(func=_shift_nonnegative)),
                             ("epsilon", FunctionTransformer(func=_plus_epsilon)),
                             ("log", FunctionTransformer(np.log, validate=False)),
                             ("inf_b", _nonfinite_to_nan()), ("fill_b", _mean_fill())])
        if tag == "adaptive":
            return PerColumnTransform(random_state=seed, n_quantiles=max(n // 10, 2))
        if tag in ("robust", "squash"):
            return RobustScaler(unit_variance=True)
        if isinstance(tag, str) and (tag.startswith("kdi") or tag == "norm_and_kdi"):
            raise NotImplementedError(f"RebalanceFeatureDistribution worker tag {tag!r} needs the kditransform "
                                      "package, which is not installed")
        return FunctionTransformer(_identity)

    def fit(self, x, categorical, seed, y=None):
        static_seed, _ = _rng(seed)
        n, p = x.shape
        cont = [i for i in range(p) if i not in categorical]
        workers = []
        if self.original_flag:
            targets = list(categorical) + cont if self.discrete_flag else cont
            workers.append(("original", "passthrough", list(range(p))))
            self.categorical = list(categorical)
        elif self.discrete_flag:
            targets, self.categorical = list(categorical) + cont, []
        else:
            workers.append(("discrete", "passthrough", list(categorical)))
            targets, self.categorical = cont, list(range(len(categorical)))
        for tag in self.tags:
            workers.append((f"feat_transform_{tag}", self._worker(tag, n, static_seed), targets))
        columns = ColumnTransformer(workers, remainder="drop", sparse_threshold=0.0)
        if self.svd_tag == "svd" and p >= 2:
            scaled = Pipeline([
                ("i2n_pre", _nonfinite_to_nan()),
                ("fill_missing_pre", _mean_fill()),
                ("standard", StandardScaler(with_mean=False)),
                ("i2n_post", _nonfinite_to_nan()),
                ("fill_missing_post", _mean_fill()),
            ])
            svd = Pipeline([("save_standard", scaled),
                            ("svd", DeviceSVD(max(1, min(n // 10 + 1, p // 2)), self.device, random_state=static_seed,
                                              algorithm="arpack"))])
            self.worker = Pipeline([("worker", columns),
                                    ("svd_worker", FeatureUnion([("default", FunctionTransformer(func=_identity)),
                                                                 ("svd", svd)]))])
        else:
            self.worker = columns
        self.worker.fit(x)
        return self.categorical

    def apply(self, x, is_test=False):
        return self.worker.transform(x), self.categorical


class CategoryCodes:
    """CategoricalFeatureEncoder (preprocess.py:686-832): ordinal codes for the categorical
    columns that qualify (the "*feature_shuffled" strategies keep columns whose rarest level
    appears at least 10 times; "strict" also needs fewer than rows / 10 levels), moved to the
    front, with each column's levels relabelled by a seeded permutation for the "_shuffled"
    strategies; "onehot" puts sklearn's one-hot columns of every categorical column first (one
    column for a two-level one, all-zero for a level the context did not have) -- unless that
    matrix would hold a million entries or more on the context rows, when the matrix is left
    as it is; "numeric" / "none" leave the matrix as it is."""

    STRATEGIES = ("ordinal", "ordinal_strict_feature_shuffled", "ordinal_shuffled", "ordinal_feature_shuffled",
                  "onehot", "numeric", "none")

    def __init__(self, *, encoding_strategy="ordinal"):
        if encoding_strategy not in self.STRATEGIES and not str(encoding_strategy).startswith("ordinal"):
            raise ValueError(f"Unsupported encoding strategy: {encoding_strategy}")
        self.strategy = encoding_strategy

    def _qualifies(self, col, strict):
        counts = np.unique(col, return_counts=True)[1] if len(col) else np.array([0])
        if strict:
            return int(counts.min()) >= 10 and len(counts) < len(col) // 10
        return int(counts.min()) >= 10

    def fit(self, x, categorical, seed, y=None):
        self.columns, self.perms = None, None
        if self.strategy in ("numeric", "none"):
            self.categorical = list(categorical)
            return self.categorical
        if self.strategy == "onehot":
            columns = ColumnTransformer([("one_hot_encoder", OneHotEncoder(drop="if_binary", sparse_output=False,
                                                                           handle_unknown="ignore"), list(categorical))],
                                        remainder="passthrough").fit(x)
            width = columns.transform(x).shape[1]
            if x.shape[0] * width >= ONE_HOT_MAX_ELEMENTS:
                self.categorical = list(categorical)
            else:
                self.columns = columns
                self.categorical = list(range(width))[columns.output_indices_["one_hot_encoder"]]
            return list(self.categorical)
        suffix = self.strategy[len("ordinal"):]
        cats = list(categorical)
        if "feature_shuffled" in suffix:
            cats = [j for j in cats if self._qualifies(x[:, j], "strict_feature_shuffled" in suffix)]
        self.columns = ColumnTransformer([("ordinal_encoder", OrdinalEncoder(handle_unknown="use_encoded_value",
                                                                             unknown_value=np.nan), cats)],
                                         remainder="passthrough").fit(x)
        self.categorical = list(range(len(cats)))
        if suffix.endswith("_shuffled"):
            _, g = _rng(seed)
            enc = self.columns.named_transformers_["ordinal_encoder"]
            self.perms = {j: g.permutation(len(enc.categories_[j])) for j in self.categorical}
        return self.categorical

    def apply(self, x, is_test=False):
        if self.columns is None:
            return x, self.categorical
        out = self.columns.transform(x)
        for j, perm in (self.perms or {}).items():
            col = out[:, j]
            ok = ~np.isnan(col)
            col[ok] = perm[col[ok].astype(int)].astype(col.dtype)
        return out, self.categorical


def _row_hash(row: np.ndarray) -> float:
    """SHA-256 of a row's bytes, as an integer modulo 10^12, over 10^12 (preprocess.py:1225-1248)."""
    return (int(hashlib.sha256(row.tobytes()).hexdigest(), 16) % 10**12) / 10**12


class RowFingerprint:
    """FingerprintFeatureEncoder (preprocess.py:1251-1320): a column of row hashes appended. The
    rows are salted with a seeded offset in [0, 65536); context rows whose hash repeats are
    rehashed with +1, +2, ... until unique; query rows are salted twice and keep their first hash."""

    def fit(self, x, categorical, seed, y=None):
        _, g = _rng(seed)
        self.salt = int(g.integers(0, 65536))
        self.categorical = list(categorical)
        return list(categorical)

    def apply(self, x, is_test=False):
        salted = x + self.salt
        fp = np.zeros(x.shape[0], dtype=x.dtype)
        if is_test:
            for i in range(x.shape[0]):
                fp[i] = _row_hash(salted[i] + self.salt)
        else:
            seen = set()
            for i in range(x.shape[0]):
                h, k = _row_hash(salted[i]), 0
                while h in seen:
                    k += 1
                    h = _row_hash(salted[i] + k)
                fp[i] = h
                seen.add(h)
        return np.column_stack([x, fp.reshape(-1, 1)]), self.categorical


class ColumnOrder:
    """FeatureShuffler (preprocess.py:626-683): the columns permuted -- "shuffle" a seeded
    permutation, "rotate" a roll by the member's offset, "latin" both, None the identity."""

    def __init__(self, *, mode="shuffle", offset=0):
        if mode not in ("shuffle", "rotate", "latin", None):
            raise ValueError(f"Unsupported reordering mode: {mode}")
        self.mode, self.offset = mode, int(offset)

    def fit(self, x, categorical, seed, y=None):
        p = x.shape[1]
        idx = np.arange(p)
        if self.mode == "rotate":
            self.order = np.roll(idx, self.offset)
        elif self.mode in ("shuffle", "latin"):
            _, g = _rng(seed)
            self.order = g.permutation(idx)
            if self.mode == "latin":
                self.order = np.roll(self.order, self.offset)
        else:
            self.order = idx
        self.categorical = np.where(np.isin(idx, categorical)[self.order])[0].tolist()
        return self.categorical

    def apply(self, x, is_test=False):
        if len(self.order) != x.shape[1]:
            raise ValueError("The number of features in the input data does not match the training data")
        return x[:, self.order], self.categorical


# ---------------------------------------------------------------------------------- members
class Member:
    """One ensemble member: its steps in the reference's order (predictor.py:378-418) and the
    seed of each (its slot of the seed list: the wide-table projection the last one, every
    other step its position among the rest, predictor.py:558-570)."""

    def __init__(self, config: dict, seeds: list[int], offset: int, device):
        self.steps: list = []
        if "HighDimFeatureSelector" in config:
            self.steps.append(WideTableProjection(**config["HighDimFeatureSelector"], device=device))
        if "MaxFeatureSubsampler" in config:
            self.steps.append(FeatureCap(**config["MaxFeatureSubsampler"]))
        if "PolynomialInteractionGenerator" in config:
            self.steps.append(PairProducts(**config["PolynomialInteractionGenerator"]))
        self.steps.append(DropConstantColumns())
        if "MADWinsorizer" in config:
            self.steps.append(MadClip(**config["MADWinsorizer"]))
        if "RebalanceFeatureDistribution" in config:
            self.steps.append(Redistribute(**config["RebalanceFeatureDistribution"], device=device))
        if "CategoricalFeatureEncoder" in config:
            self.steps.append(CategoryCodes(**config["CategoricalFeatureEncoder"]))
        if config.get("FingerprintFeatureEncoder", False):
            self.steps.append(RowFingerprint())
        if "FeatureShuffler" in config:
            self.steps.append(ColumnOrder(**config["FeatureShuffler"], offset=offset))
        self.seeds = []
        slot = 0
        for step in self.steps:
            if isinstance(step, WideTableProjection):
                self.seeds.append(seeds[SEED_SLOTS - 1])
            else:
                self.seeds.append(seeds[slot])
                slot += 1

    def features(self, x_train: np.ndarray, x_test: np.ndarray, categorical: list[int], y_train: np.ndarray):
        """The member's (context, query) feature matrices: each step fitted on the context
        (the wide-table projection with ``fit_on_test`` on both splits) and applied to both."""
        cat = list(categorical)
        self.reads_queries = False
        for step, seed in zip(self.steps, self.seeds):
            if isinstance(step, WideTableProjection) and step.fit_on_test and len(x_test):
                cat = step.fit(np.vstack([x_train, x_test]), cat, seed)
                self.reads_queries |= step.depends_on_rows()
            else:
                cat = step.fit(x_train, cat, seed, y=y_train)
            x_train, _ = step.apply(x_train, is_test=False)
            x_test, cat = step.apply(x_test, is_test=True)
        self.categorical = cat
        return np.asarray(x_train), np.asarray(x_test), cat

    def query_features(self, x_test: np.ndarray) -> np.ndarray:
        """Other query rows through the steps ``features`` fitted, for a member whose fit did not
        read the query rows (``reads_queries`` False): the same matrix ``features`` would give
        for them, since every other step is fitted on the context alone."""
        if getattr(self, "reads_queries", True):
            raise RuntimeError("this member's fit read its query rows; fit it again with features()")
        for step in self.steps:
            x_test, _ = step.apply(x_test, is_test=True)
        return np.asarray(x_test)


def build_members(config, seed: int, device) -> list[Member]:
    """The members of a configuration and the seeds of their steps, drawn as the reference draws
    them (predictor.py:352-362): Python's random generator seeded with ``seed`` gives 10 seeds
    in [0, 10000] per member, numpy's default_rng(seed) the rotation offsets."""
    members = read_members(config)
    n = len(members)
    if n == 0:
        raise ValueError("the inference configuration has no members")
    draw = random.Random(seed)
    seeds = [draw.randint(0, 10000) for _ in range(n * SEED_SLOTS)]
    g = np.random.default_rng(seed)
    start = g.integers(0, 1000)
    shifts = g.choice(list(range(start, start + n)), size=n, replace=False)
    return [Member(m, seeds[i * SEED_SLOTS:(i + 1) * SEED_SLOTS], int(shifts[i]), device) for i, m in enumerate(members)]
