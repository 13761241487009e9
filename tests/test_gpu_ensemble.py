"""The default preprocessing ensemble on config 1's table with its SVDs on the GPU.

Each of the reference's eight default members (configs/default_inference.json;
preprocess.py:916-1222 for the redistribution step) is run on the nori-6m case's table
(tests/regressor_case.py: 1024 context + 256 query rows, 16 features) with the device SVD on
the GPU, and checked by what fixes it independently of this code:

* feature shapes: quantile members 66 columns (16 + 10 pair products, kept; their uniform
  quantile transform; a 13-column SVD block; the fingerprint), adaptive members 27;
* the quantile block of each quantile member: sklearn's QuantileTransformer with the capped
  settings, fitted on the same context rows, to 1e-12;
* the SVD block: taken from the member's float32 columns scaled in float32 (the closed form to
  float32 rounding); its column norms equal that block's singular values (numpy's LAPACK SVD)
  to 1e-8, the components are orthonormal, and the block is the projection on them;
* the whole member's features: the GPU run equals the CPU run (float64 SVDs) to 1e-9, except
  the row fingerprint, whose hash of a row's bytes changes with any last-bit difference.
"""

from __future__ import annotations

import json
import os

import numpy as np
import pytest
from sklearn.preprocessing import QuantileTransformer

import regressor_case as case
from nori_amd import ensemble as en

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "regressor_goldens.npz")


def _redistribute_io(member, x_tr, x_te, y):
    """Run the member's steps on the context rows up to its redistribution step: (input, output)."""
    cat = []
    for step, seed in zip(member.steps, member.seeds):
        if isinstance(step, en.WideTableProjection) and step.fit_on_test:
            cat = step.fit(np.vstack([x_tr, x_te]), cat, seed)
        else:
            cat = step.fit(x_tr, cat, seed, y=y)
        if isinstance(step, en.Redistribute):
            return x_tr, step.apply(x_tr, is_test=False)[0], step, seed
        x_tr, _ = step.apply(x_tr, is_test=False)
        x_te, cat = step.apply(x_te, is_test=True)
    raise AssertionError("member has no redistribution step")


def test_default_members_on_config1_table(cuda):
    x_tr, y_tr, x_te, _ = case.table()
    y = ((y_tr - y_tr.mean()) / y_tr.std()).astype(np.float32)
    gpu = en.build_members(en.DEFAULT_MEMBERS, 0, cuda)
    cpu = en.build_members(en.DEFAULT_MEMBERS, 0, "cpu")
    for i, (mg, mc) in enumerate(zip(gpu, cpu)):
        a, b, cat = mg.features(x_tr, x_te, [], y)
        print(f"member {i}: features {a.shape} / {b.shape}", flush=True)
        assert a.shape == (1024, 66 if i < 4 else 27) and b.shape == (256, a.shape[1]) and cat == []
        a_cpu, b_cpu, _ = mc.features(x_tr, x_te, [], y)
        # every column but the row fingerprint equals the CPU run's; the fingerprint hashes a row's
        # bytes, so a last-bit difference of the GPU SVD anywhere in a row changes it (the
        # reference's hash on two devices behaves the same): it is held to its own contract, a
        # unique value in [0, 1) per context row
        order = mg.steps[-1].order
        fp = int(np.where(order == len(order) - 1)[0][0])
        rest = [j for j in range(a.shape[1]) if j != fp]
        np.testing.assert_allclose(a[:, rest], a_cpu[:, rest], rtol=1e-9, atol=1e-9)
        np.testing.assert_allclose(b[:, rest], b_cpu[:, rest], rtol=1e-9, atol=1e-9)
        assert len(np.unique(a[:, fp])) == len(a) and ((a[:, fp] >= 0) & (a[:, fp] < 1)).all()
        assert ((b[:, fp] >= 0) & (b[:, fp] < 1)).all()
        if i >= 4:
            continue
        x_in, out, step, seed = _redistribute_io(en.build_members(en.DEFAULT_MEMBERS, 0, cuda)[i], x_tr, x_te, y)
        n, p = x_in.shape
        static_seed, _ = en._rng(seed)
        k = max(1, min(n // 10 + 1, p // 2))  # from the step's input width
        assert out.shape == (n, 2 * p + k)
        np.testing.assert_array_equal(out[:, :p], x_in)
        qt = QuantileTransformer(output_distribution="uniform", n_quantiles=max(2, min(max(n // 5, 2), n, 256)),
                                 subsample=min(n, 10000), random_state=static_seed).fit(x_in)
        np.testing.assert_allclose(out[:, p:2 * p], qt.transform(x_in), rtol=0, atol=1e-12)
        # the block the SVD is taken from: the member's float32 columns scaled to unit variance in
        # float32, as the reference's float-preserving steps leave them (closed form to float32
        # rounding); the SVD identities are checked on that block itself
        columns = step.worker.named_steps["worker"].transform(x_in)
        branch = step.worker.named_steps["svd_worker"].transformer_list[1][1]
        scaled = branch.named_steps["save_standard"].transform(columns)
        assert columns.dtype == np.float32 and scaled.dtype == np.float32
        block = np.hstack([out[:, :p], out[:, p:2 * p]]).astype(np.float64)
        np.testing.assert_allclose(scaled, block / block.std(axis=0), rtol=2e-7, atol=1e-6)
        scaled = scaled.astype(np.float64)
        svd = out[:, 2 * p:]
        sv = np.linalg.svd(scaled, compute_uv=False)[:k]
        # the device solver's float64 singular values against LAPACK's: 1.5e-9 relative measured
        np.testing.assert_allclose(np.linalg.norm(svd, axis=0), sv, rtol=1e-8)
        comps = branch.named_steps["svd"].components_
        np.testing.assert_allclose(comps @ comps.T, np.eye(k), atol=1e-10)
        np.testing.assert_allclose(svd, scaled @ comps.T, rtol=1e-9, atol=1e-9)
        print(f"member {i}: quantile block and {k}-column SVD block pinned", flush=True)


# members built from the steps the shipped configurations do not use: the svd_binary and
# correlation projections, the power / logNormal / quantile_norm_10 redistributions and one-hot
# codes (preprocess.py:686-832, 970-1222, 1323-1684)
OTHER_MEMBERS = [
    {"HighDimFeatureSelector": {"strategy": "corr", "top_k": 10, "n_features_threshold": 12},
     "RebalanceFeatureDistribution": {"worker_tags": ["power"], "original_flag": True},
     "CategoricalFeatureEncoder": {"encoding_strategy": "onehot"}, "FeatureShuffler": {"mode": "shuffle"}},
    {"HighDimFeatureSelector": {"strategy": "svd_binary", "binary_threshold": 0.1, "svd_components": 8},
     "RebalanceFeatureDistribution": {"worker_tags": ["logNormal"], "svd_tag": "svd"},
     "FingerprintFeatureEncoder": True},
    {"RebalanceFeatureDistribution": {"worker_tags": ["quantile_norm_10"], "original_flag": True},
     "CategoricalFeatureEncoder": {"encoding_strategy": "onehot"}, "FeatureShuffler": {"mode": "rotate"}},
]


def _other_table():
    x_tr, y_tr, x_te, _ = case.table()
    x_tr, x_te = x_tr.copy(), x_te.copy()
    # two binary columns and a three-level one, so the binary projection and one-hot codes engage
    for j, levels in ((0, 2), (1, 2), (2, 3)):
        x_tr[:, j] = np.floor(np.abs(x_tr[:, j]) * 7) % levels
        x_te[:, j] = np.floor(np.abs(x_te[:, j]) * 7) % levels
    return x_tr, y_tr, x_te


def test_other_members_features_and_predictions(cuda):
    import warnings

    from nori_amd import api
    from nori_amd.memory_policy import CacheQuantizedWarning
    from nori_amd.transformer import FeaturesTransformer

    x_tr, y_tr, x_te = _other_table()
    y = ((y_tr - y_tr.mean()) / y_tr.std()).astype(np.float32)
    cat = en.categorical_columns(x_tr)
    assert cat == [0, 1, 2]
    for i, (mg, mc) in enumerate(zip(en.build_members(OTHER_MEMBERS, 0, cuda), en.build_members(OTHER_MEMBERS, 0, "cpu"))):
        a, b, _ = mg.features(x_tr, x_te, cat, y)
        a_cpu, b_cpu, _ = mc.features(x_tr, x_te, cat, y)
        print(f"other member {i}: features {a.shape} / {b.shape}", flush=True)
        assert a.shape == a_cpu.shape and np.isfinite(a).all() and np.isfinite(b).all()
        keep = list(range(a.shape[1] - 1)) if i == 1 else list(range(a.shape[1]))  # member 1 ends in the fingerprint
        np.testing.assert_allclose(a[:, keep], a_cpu[:, keep], rtol=1e-9, atol=1e-9)
        np.testing.assert_allclose(b[:, keep], b_cpu[:, keep], rtol=1e-9, atol=1e-9)
    with np.load(GOLDEN, allow_pickle=False) as f:
        scales = json.loads(str(f["case/weight_scales"]))
    model = case.seeded_model(FeaturesTransformer, api.NORI_6M_CONFIG, scales).to(cuda)
    kwargs = dict(model=model, device=cuda, inference_config=OTHER_MEMBERS, memory_policy={"cache_dtype": "int8"},
                  mix_precision=False)
    with warnings.catch_warnings():
        warnings.simplefilter("ignore", CacheQuantizedWarning)
        reg = api.NoriRegressor(**kwargs).fit(x_tr, y_tr)
        point = reg.predict(x_te)
        qs = reg.predict(x_te, output_type="quantiles", quantiles=[0.1, 0.5, 0.9])
        assert reg.memory_report_["ensemble_members"] == 3
    assert point.shape == (len(x_te),) and np.isfinite(point).all() and np.all(np.diff(qs, axis=0) >= 0)
