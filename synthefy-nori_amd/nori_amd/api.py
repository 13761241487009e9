"""``NoriRegressor``: the fit/predict surface of the reference's estimator over this package's
cached path (src/synthefy_nori/api.py:158, 464-620, 862-968, 1122-1151, 1256-1345).

``fit`` validates and stores the context rows and the target's mean and standard deviation;
``predict`` scores query rows against that context through the context cache:

1. the target is standardized with the fitted statistics (api.py:1129);
2. the memory policy picks the cache's precision and placement (``memory_policy.MemoryPolicy``,
   the reference's rung ladder) and ``memory_report_`` records it;
3. ``FeaturesTransformer.build_context_cache`` encodes the context once -- every layer's K/V
   written to the int8 cache by the HIP quantizer on the int8 rungs -- and is kept for later
   calls on the same context (exact byte comparison of the context, as the reference's
   ``_get_or_build_context``, predictor.py:2005-2150, decides reuse);
4. ``apply_context_cache`` scores the query rows (query -> context attention on the HIP
   kernel), under fp16 autocast on a GPU as the reference's predictor runs it
   (predictor.py:3208-3217);
5. the quantile bank becomes the point prediction by the trapezoid mean of its piecewise
   linear quantile function (``quantile_dist_mean``, quantile_dist.py:95-135), its median, or
   quantiles at requested levels (api.py:1256-1345), and is mapped back to the target's units.

The rows go through the preprocessing ensemble of the inference configuration first
(``nori_amd.ensemble``; by default the reference's eight members of
configs/default_inference.json): every member builds its own feature matrices from the context
and query rows, gets its own context cache, and the members' quantile banks are averaged
(predictor.py:2972-3000, 3533) before the collapse. With ``augmentations=("yj",)`` (the
default) a target whose skew exceeds ``yj_skew_threshold`` is also scored in Yeo-Johnson space
and the two point predictions averaged (predictor.py:1880-1990).

What the reference does around this and this surface does not: DataFrame / categorical-string /
text feature handling, multi-target prediction, large-context policies and checkpoint download.
A model comes from a local checkpoint (``model_path``, loaded without unpickling) or as a built
``FeaturesTransformer`` (``model=``).
"""

from __future__ import annotations

import math

import numpy as np
import torch

from . import ensemble, graphs
from .memory_policy import RUNGS, MemoryPolicy, estimate_cache_gb, fit_row_chunk_attempts, memory_attempt, warn_quantized
from .transformer import FeaturesTransformer

__all__ = ["NORI_6M_CONFIG", "NoriRegressor", "build_model", "context_device_bytes", "load_model", "quantile_dist_mean",
           "retain_context"]

# nori-6m, the released base model: configs/model_base.json with the tier-1 training flags of
# scripts/train.sh:146-148 (embed 128, hidden 384, 2 heads, 16 layers, "model v2 lite": SwiGLU,
# RMSNorm pre-norm with deep-norm alpha 16^-1/2, RBF numeric embedding; QASS on, target-aware
# and column-specific y embedding, training/cli.py:1240-1320, 340-352) and the 999-level
# pinball head ((i + 1) / 1000).
NORI_6M_CONFIG = dict(
    preprocess_config_x=dict(num_features=2, nan_handling_enabled=True, normalize_on_train_only=True, normalize_x=True,
                             remove_outliers=False, normalize_by_used_features=True),
    encoder_config_x=dict(num_features=2, embedding_size=128, mask_embedding_size=128, encoder_use_bias=True,
                          numeric_embed_type="RBF",
                          RBF_config=dict(token_embed_dim=16, n_kernels=64, sigma=0.5, use_learn_sigma=False,
                                          use_learn_embeddings=False, use_original_features=False)),
    encoder_config_y=dict(num_inputs=1, embedding_size=128, nan_handling_y_encoder=True, max_num_classes=10),
    decoder_config=dict(num_classes=10, num_reg_quantiles=999, regression_loss="pinball",
                        regression_quantiles=[(i + 1) / 1000.0 for i in range(999)]),
    feature_positional_embedding_type="none", nlayers=16, nhead=2, embed_dim=128, hid_dim=384,
    features_per_group=2, dropout=0.0, pre_norm=True, activation="swiglu", norm_type="rmsnorm",
    deepnorm_alpha=16 ** -0.5, recompute_attn=False, layer_arch="smf", self_share_all_kv_heads=False,
    cross_share_all_kv_heads=False, seq_attn_isolated=True, seq_attn_serial=False, use_qassmax=True,
    qass_mode="full", use_target_aware_embedding=True, use_column_specific_y_aware=True,
)

_CONFIG_KEYS = ("preprocess_config_x", "encoder_config_x", "encoder_config_y", "decoder_config", "nlayers", "nhead",
                "embed_dim", "hid_dim", "feature_positional_embedding_type", "feature_positional_embedding_num_slots",
                "mask_prediction", "features_per_group", "dropout", "pre_norm", "activation", "layer_norm_eps",
                "recompute_attn", "layer_arch", "norm_type", "deepnorm_alpha", "self_share_all_kv_heads",
                "cross_share_all_kv_heads", "seq_attn_isolated", "seq_attn_serial", "use_qassmax", "qass_mode",
                "use_target_aware_embedding", "use_column_specific_y_aware", "use_logn_attention",
                "use_learnable_attn_temperature", "attn_n_ref", "omit_feature_decoder", "two_phase_config")


def build_model(config: dict) -> FeaturesTransformer:
    """A ``FeaturesTransformer`` from an architecture record (utils/loading.py:108-187): the
    fields the constructor takes, unknown ones ignored, the QASS mode "full" when the record
    names none (loading.py:45-68)."""
    kwargs = {k: config[k] for k in _CONFIG_KEYS if k in config}
    if kwargs.get("use_qassmax") and not kwargs.get("qass_mode"):
        kwargs["qass_mode"] = "full"
    if config.get("task_type", "reg") != "reg":
        raise ValueError("only regression checkpoints are supported")
    return FeaturesTransformer(**kwargs)


def load_model(model_path: str) -> FeaturesTransformer:
    """A checkpoint's model (utils/loading.py:206-279), read with ``weights_only=True``: the
    training layout (``model_config`` + ``ema_state_dict`` or ``model_state_dict``) or the
    release layout (``config`` + ``state_dict``); a torch.compile prefix is stripped."""
    blob = torch.load(model_path, map_location="cpu", weights_only=True)
    if "model_config" in blob:
        config, weights = blob["model_config"], blob.get("ema_state_dict") or blob["model_state_dict"]
    elif "state_dict" in blob and "config" in blob:
        config, weights = blob["config"], blob["state_dict"]
    else:
        raise KeyError(f"{model_path}: no model_config/state_dict or config/state_dict entries")
    weights = {k.removeprefix("_orig_mod."): v for k, v in weights.items()}
    model = build_model(dict(config))
    model.load_state_dict(weights)
    return model.eval()


def quantile_dist_mean(q: torch.Tensor, tau: torch.Tensor) -> torch.Tensor:
    """Mean of the distribution whose quantile function runs linearly between the sorted
    predictions ``q[..., k]`` at levels ``tau[k]`` and is flat beyond the outer levels: the
    area under that function (quantile_dist.py:95-135, ``quantile_dist_mean_simple`` with the
    monotone sort). Computed in fp32 for half-precision banks, else in q's dtype."""
    if q.dim() == 0:
        raise ValueError("q must have a quantile axis")
    k = q.shape[-1]
    tau = torch.as_tensor(tau)
    if tau.shape != (k,):
        raise ValueError(f"tau must have shape ({k},), got {tuple(tau.shape)}")
    if not bool(torch.isfinite(tau).all()) or bool((tau <= 0).any()) or bool((tau >= 1).any()) or bool((tau.diff() <= 0).any()):
        raise ValueError("tau must be finite, strictly increasing values in (0, 1)")
    dtype = torch.float32 if q.dtype in (torch.float16, torch.bfloat16) else q.dtype
    q = torch.sort(q.to(dtype), dim=-1).values
    tau = tau.to(device=q.device, dtype=dtype)
    if k == 1:
        return q[..., 0]
    # trapezoids between adjacent levels, plus the flat outer pieces [0, tau_0] and [tau_K-1, 1]
    inner = ((q[..., 1:] + q[..., :-1]) * 0.5 * (tau[1:] - tau[:-1])).sum(dim=-1)
    return tau[0] * q[..., 0] + inner + (1.0 - tau[-1]) * q[..., -1]


def _interpolated_quantiles(bank: np.ndarray, taus: np.ndarray, levels: np.ndarray) -> np.ndarray:
    """[len(levels), rows]: each sorted row's quantile function read at ``levels`` by linear
    interpolation over the level grid (api.py:1330-1345)."""
    grid = np.arange(bank.shape[1], dtype=np.float64)
    out = np.empty((levels.shape[0], bank.shape[0]), dtype=np.float64)
    for i, level in enumerate(levels):
        pos = float(np.interp(level, taus, grid))
        lo = int(math.floor(pos))
        hi = min(lo + 1, bank.shape[1] - 1)
        w = pos - lo
        out[i] = (1.0 - w) * bank[:, lo] + w * bank[:, hi]
    return out


def _numeric_matrix(X, name: str) -> np.ndarray:
    try:
        arr = np.asarray(X, dtype=np.float32)
    except (TypeError, ValueError) as exc:
        raise ValueError(f"{name} must be a numeric matrix") from exc
    if arr.ndim != 2:
        raise ValueError(f"{name} must be two-dimensional [rows, features], got shape {arr.shape}")
    return arr


def context_device_bytes(obj) -> int:
    """Device bytes a retained context holds: the sizes of the distinct GPU storages reachable
    from it (tensors, dicts, lists, tuples and object attributes, 8 levels deep), each storage
    counted once however many views of it the cache keeps (row slices of one payload, a payload
    and its codes/scales views). Host tensors do not count: they are not what runs the GPU out
    of memory. predictor.py:2151-2189 walks a bundle the same way."""
    storages: dict[int, int] = {}
    seen: set[int] = set()

    def walk(o, depth: int) -> None:
        if depth > 8 or id(o) in seen:
            return
        seen.add(id(o))
        if isinstance(o, torch.Tensor):
            if o.device.type == "cuda":
                st = o.untyped_storage()
                storages[st.data_ptr()] = st.nbytes()
            return
        if isinstance(o, dict):
            for v in o.values():
                walk(v, depth + 1)
        elif isinstance(o, (list, tuple, set)):
            for v in o:
                walk(v, depth + 1)
        elif hasattr(o, "__dict__"):
            for v in vars(o).values():
                walk(v, depth + 1)

    try:
        walk(obj, 0)
    except Exception:  # accounting must never break a predict
        return 0
    return sum(storages.values())


def retain_context(contexts: dict, slot, entry, budget: int | None, size_of=context_device_bytes) -> bool:
    """Keep ``entry`` (whose last element is the context) in ``contexts`` under ``slot`` within a
    byte budget across every retained context (predictor.py:2110-2261): with no budget (no
    measurable device memory) it is kept; a context larger than the whole budget empties the
    store and is not kept (reuse is worth nothing if holding it leaves no room to run the
    model); otherwise the least recently used contexts (the dict's insertion order; a reuse hit
    moves its slot to the end) are dropped until the new one fits. Returns whether it was kept."""
    contexts.pop(slot, None)
    if budget is None:
        contexts[slot] = entry
        return True
    incoming = size_of(entry[-1])
    if incoming > budget:
        contexts.clear()
        return False
    total = sum(size_of(e[-1]) for e in contexts.values())
    for old in list(contexts):
        if total + incoming <= budget:
            break
        total -= size_of(contexts.pop(old)[-1])
    contexts[slot] = entry
    return True


def _query_trace(execution: MemoryPolicy, events, *, history: list, pipeline_id, context_row_chunk,
                 reason: str, path: str = "cached") -> MemoryPolicy:
    """One ``attempt_history`` entry per decode event of an attempt (the query-chunk halvings of
    ``apply_context_cache``), returning the policy of the last (predictor.py:1387-1421).
    ``pipeline_id``: the member, or the list of members of a batched attempt."""
    ids = list(pipeline_id) if isinstance(pipeline_id, (list, tuple)) else [pipeline_id]
    final = execution
    for i, (query_chunk, outcome) in enumerate(events):
        final = execution.escalated(execution.rung, dropped_context_rows=0, query_chunk=query_chunk)
        history.append(memory_attempt(final, pipeline_ids=ids, path=path, rung=final.rung,
                                      context_row_chunk=context_row_chunk, query_chunk=query_chunk, outcome=outcome,
                                      reason=reason if i == 0 else "oom_retry"))
    return final


def run_cache_attempts(requested: MemoryPolicy, resolved: MemoryPolicy, attempt, *, bytes_per_element: int,
                       head_dim: int, history: list, pipeline_id: int = 0, query_chunk: int | None = None,
                       evict=lambda: None):
    """The cached path's out-of-memory retries (predictor.py:3142-3400): the opening rung, then
    every budget-feasible precision / placement rung after it (``runtime_fallbacks``), then the
    last of those with the bounded context-row chunk ladder (``fit_row_chunk_attempts``).

    ``attempt(policy, fit_row_chunk, hybrid, on_query_event, state)`` builds (or reuses) the
    context cache for one rung and applies it, calling ``on_query_event(query_chunk, outcome)``
    per decode attempt and setting ``state["context"] = True`` once it holds a context. An
    ``torch.cuda.OutOfMemoryError`` records the attempt, runs ``evict`` (the failed rung's
    retained context), frees torch's cached blocks and moves to the next rung; the last rung's
    error propagates (the reference then falls back to its uncached plain loop, which this
    package does not have; a streamed context never does). A ``NotImplementedError`` is recorded
    as "unsupported" and propagates. Every attempt is appended to ``history`` as the reference's
    ``MemoryAttempt``. Returns (what ``attempt`` returned, the policy of the successful attempt,
    with the rung it reached and its last query chunk)."""
    pinned = requested.context_row_chunk
    initial = resolved.context_row_chunk if resolved.stream_context else pinned
    placements = requested.runtime_fallbacks(resolved, bytes_per_element=bytes_per_element, head_dim=head_dim)
    if not placements:
        raise NotImplementedError(f"memory policy rung {resolved.rung!r} has no cached path to attempt")
    attempts = [(p, initial) for p in placements] + [(placements[-1], c) for c in fit_row_chunk_attempts(initial)]
    for index, (policy, chunk) in enumerate(attempts):
        reason = "resolved" if index == 0 else "oom_retry"
        execution = policy
        if chunk is not None and chunk != initial:
            execution = policy.escalated(policy.rung if policy.stream_context else "context_row_chunk",
                                         context_row_chunk=chunk)
        hybrid = (policy.rung == "resident_int8" and policy.cache_dtype == "int8" and not policy.offload_to_host
                  and not policy.stream_context and chunk is not None)
        events: list = []
        state: dict = {}
        try:
            result = attempt(policy, chunk, hybrid, lambda q, outcome: events.append((q, outcome)), state)
        except NotImplementedError:
            history.append(memory_attempt(policy, pipeline_ids=[pipeline_id], path="cached", rung=policy.rung,
                                          context_row_chunk=chunk, outcome="unsupported", reason=reason))
            evict()
            raise
        except torch.cuda.OutOfMemoryError:
            if events or state.get("context"):
                failed = list(events) or [(query_chunk, "oom")]
                if failed[-1][1] == "success":  # decoded, then ran out of memory afterwards
                    failed[-1] = (failed[-1][0], "oom")
                _query_trace(execution, failed, history=history, pipeline_id=pipeline_id, context_row_chunk=chunk,
                             reason=reason)
            else:
                history.append(memory_attempt(policy, pipeline_ids=[pipeline_id], path="cached", rung=policy.rung,
                                              context_row_chunk=chunk, outcome="oom", reason=reason))
            evict()
            if torch.cuda.is_available():
                torch.cuda.empty_cache()
            if index + 1 < len(attempts):
                continue
            raise
        if not events:
            events.append((query_chunk, "success"))
        final = _query_trace(execution, events, history=history, pipeline_id=pipeline_id, context_row_chunk=chunk,
                             reason=reason)
        return result, final
    raise AssertionError("unreachable: the attempt list is never empty")


# Members scored together in one batched cache build and apply: at most this many, and only
# when their feature matrices are at most this wide (predictor.py:58-67).
MEMBER_BATCH = 4
MEMBER_BATCH_MAX_FEATURES = 256


def _severity(policy: MemoryPolicy) -> tuple:
    """How degraded an outcome is (predictor.py:1307-1331): rung, then dropped rows, then a
    smaller context-row chunk, then a smaller query chunk."""
    rank = RUNGS.index(policy.rung) if policy.rung in RUNGS else -1
    chunk = policy.context_row_chunk
    query = policy.query_chunk
    return (rank, int(policy.dropped_context_rows or 0), -chunk if chunk is not None else float("-inf"),
            -query if query is not None else float("-inf"))


def _device(device) -> torch.device:
    if device is not None:
        return torch.device(device)
    return torch.device("cuda", torch.cuda.current_device()) if torch.cuda.is_available() else torch.device("cpu")


class NoriRegressor:
    """In-context regressor with the reference's ``fit`` / ``predict`` contract (api.py:158-620, 862-968).

    ``model_path``: a local checkpoint; ``model``: a built ``FeaturesTransformer`` (a name such
    as "nori-6m" needs the checkpoint download, which this build does not do). ``device``: a
    ROCm GPU (the kernels have no CPU path). ``inference_config``: the preprocessing ensemble,
    a list of member dictionaries or a JSON path (None: the reference's default eight members;
    ``[{}]`` scores the raw columns, constant ones dropped). ``augmentations``: ``("yj",)`` adds
    the Yeo-Johnson target pass for targets skewed beyond ``yj_skew_threshold``; ``seed`` seeds
    the members' steps. ``quantile_collapse``: "mean" (default) or "median". ``memory_policy``:
    None, a preset ("exact", "max_context", "off"), a dict of ``MemoryPolicy`` fields, or a
    ``MemoryPolicy``. ``mix_precision``: run the cached path under fp16 autocast (the reference
    predictor's GPU default).

    Context caches are kept for reuse across calls, one per member slot, within
    ``context_cache_budget_frac`` (0.25, the reference's share) of the device's memory in all
    (``retain_context``).
    """

    context_cache_budget_frac = 0.25

    def __init__(self, model_path: str | None = None, *, model=None, device=None, inference_config=None,
                 augmentations=("yj",), yj_skew_threshold: float = 10.0, seed: int = 0, quantile_collapse: str = "mean",
                 memory_policy=None, mix_precision: bool = True):
        self.model_path = model_path
        self.model = model
        self.device = device
        self.inference_config = inference_config
        self.augmentations = tuple(augmentations) if augmentations else ()
        self.yj_skew_threshold = float(yj_skew_threshold)
        self.seed = int(seed)
        self.quantile_collapse = quantile_collapse
        self.memory_policy = memory_policy
        self.mix_precision = mix_precision
        self._net = None
        self._contexts = {}  # member slot -> (cache key, x bytes, y bytes, ContextCache)
        self._report = None
        self._attempt_history: list = []
        self._outcome_policy = None
        self._member_fits: dict = {}  # member slot -> (fit key, fitted member, its context features)

    # ------------------------------------------------------------------ sklearn surface
    def get_params(self, deep: bool = True) -> dict:
        return {"model_path": self.model_path, "model": self.model, "device": self.device,
                "inference_config": self.inference_config, "augmentations": self.augmentations,
                "yj_skew_threshold": self.yj_skew_threshold, "seed": self.seed,
                "quantile_collapse": self.quantile_collapse, "memory_policy": self.memory_policy,
                "mix_precision": self.mix_precision}

    def set_params(self, **params) -> "NoriRegressor":
        for k, v in params.items():
            if k not in self.get_params():
                raise ValueError(f"unknown parameter {k!r}")
            setattr(self, k, v)
        return self

    @property
    def memory_report_(self) -> dict | None:
        """What the last ``predict`` did about memory (``MemoryPolicy.as_report()``), or None."""
        return self._report

    # ------------------------------------------------------------------ fit
    def fit(self, X, y) -> "NoriRegressor":
        """Store the context rows and the target's statistics (api.py:464-620): X numeric
        [rows, features], y one finite value per row."""
        MemoryPolicy.coerce(self.memory_policy)  # an incoherent policy fails here, not at predict
        if self.quantile_collapse not in ("mean", "median"):
            raise ValueError(f"quantile_collapse must be 'mean' or 'median', got {self.quantile_collapse!r}")
        x = _numeric_matrix(X, "X")
        try:
            y_arr = np.asarray(y, dtype=np.float64)
        except (TypeError, ValueError) as exc:
            raise ValueError("y must contain only numeric target values") from exc
        if y_arr.ndim != 1:
            raise ValueError(f"y must be one-dimensional for scalar regression, got shape {y_arr.shape}")
        if y_arr.shape[0] != x.shape[0]:
            raise ValueError(f"X and y must contain the same number of rows; got {x.shape[0]} and {y_arr.shape[0]}")
        if not np.all(np.isfinite(y_arr)):
            raise ValueError("y must contain only finite target values")
        self.device_ = _device(self.device)
        self.X_train_ = x
        self.n_features_in_ = x.shape[1]
        self.y_train_ = y_arr
        self.y_mean_ = float(y_arr.mean())
        std = float(y_arr.std())
        self.y_std_ = std if std >= 1e-12 else 1.0
        self._contexts = {}
        self._member_fits = {}
        return self

    # ------------------------------------------------------------------ predict
    def predict(self, X, *, output_type: str = "mean", quantiles: list[float] | None = None):
        """Point predictions ("mean", "median"; "mode" is the median for a quantile head), or
        quantiles at ``quantiles`` levels as [len(quantiles), rows] ("quantiles"), or the whole
        sorted quantile bank with its levels and mean ("full") -- api.py:862-968, 1256-1345."""
        if not hasattr(self, "X_train_"):
            raise ValueError("Call fit(X, y) before predict(X).")
        if output_type not in ("mean", "median", "mode", "quantiles", "full"):
            if output_type == "main":
                raise NotImplementedError("output_type='main' is not supported")
            raise ValueError(f"Unknown output_type={output_type!r}; expected 'mean', 'median', 'mode', 'quantiles' or 'full'.")
        if output_type == "quantiles":
            if not quantiles:
                raise ValueError("output_type='quantiles' requires quantiles=[...] with at least one level in (0, 1).")
            levels = np.asarray(quantiles, dtype=np.float64)
            if np.any((levels <= 0.0) | (levels >= 1.0)):
                raise ValueError("quantiles must lie strictly in (0, 1).")
        elif quantiles is not None:
            raise ValueError("quantiles= is only valid with output_type='quantiles'.")
        x_test = _numeric_matrix(X, "X")
        if x_test.shape[1] != self.n_features_in_:
            raise ValueError(f"X has {x_test.shape[1]} features, the context has {self.n_features_in_}")
        net = self._network()
        # exact graph replay of the cached query layers (predictor.py:2394-2482), on request
        if graphs.cached_graphs_requested():
            graphs.enable_cached_graphs(net)
        else:
            graphs.disable_cached_graphs(net)
        y_norm = ((self.y_train_ - self.y_mean_) / self.y_std_).astype(np.float32)
        # one call's memory outcome: its attempts and its most degraded rung (predictor.py:1333-1351)
        self._attempt_history = []
        self._outcome_policy = None
        bank = self._ensemble_bank(net, x_test, y_norm)  # [rows, K] in standardized target units, fp32
        taus = torch.tensor(net.regression_quantiles, dtype=torch.float64, device=bank.device)
        if output_type in ("mean", "median", "mode"):
            collapse = self.quantile_collapse if output_type == "mean" else "median"
            point = self._collapse(bank, taus, collapse)
            point = self._yeo_johnson_pass(net, x_test, y_norm, point, taus, collapse)
            return point * self.y_std_ + self.y_mean_
        values = np.sort(bank.double().cpu().numpy() * self.y_std_ + self.y_mean_, axis=1)
        grid = taus.cpu().numpy()
        if output_type == "full":
            mean = quantile_dist_mean(torch.from_numpy(values), torch.from_numpy(grid)).numpy()
            return {"quantiles": values, "taus": grid, "mean": mean}
        return _interpolated_quantiles(values, grid, levels)

    # ------------------------------------------------------------------ internals
    @staticmethod
    def _collapse(bank: torch.Tensor, taus: torch.Tensor, collapse: str) -> np.ndarray:
        if collapse == "mean":
            point = quantile_dist_mean(bank.double(), taus)
        else:
            ordered = torch.sort(bank.double(), dim=-1).values
            mid = ordered.shape[-1] // 2
            point = ordered[..., mid] if ordered.shape[-1] % 2 else ordered[..., mid - 1 : mid + 1].mean(-1)
        return point.cpu().numpy()

    def _ensemble_bank(self, net: FeaturesTransformer, x_test: np.ndarray, y_norm: np.ndarray, slot0: int = 0):
        """The mean of the members' quantile banks (predictor.py:2972-3000, 3533): each member's
        features from the context and query rows, scored through that member's context cache.

        Members whose context and query matrices have the same shapes are scored together, up to
        ``MEMBER_BATCH`` at a time and at most ``MEMBER_BATCH_MAX_FEATURES`` features wide, as
        the tables of one batched cache build and apply (predictor.py:2325-2359, 2497-2700) when
        the memory policy keeps the caches resident; the rest, and a batch that runs out of
        device memory, one member at a time (always, when exact graph replay is requested:
        ``SYNTHEFY_EXACT_CACHED_CUDAGRAPHS=1``). A member whose preprocessing fit did not read the
        query rows keeps that fit for later calls on the same context and only transforms the
        new query rows (the fit depends on the context rows, the targets and its seeds alone)."""
        config = ensemble.DEFAULT_MEMBERS if self.inference_config is None else self.inference_config
        members = ensemble.build_members(config, self.seed, self.device_)
        categorical = ensemble.categorical_columns(self.X_train_)
        fit_key = (repr(ensemble.read_members(config)), self.seed, y_norm.tobytes(), str(self.device_))
        feats = []
        for i, member in enumerate(members):
            held = self._member_fits.get(slot0 + i)
            if held is not None and held[0] == fit_key and not held[1].reads_queries:
                x_ctx, x_q = held[2], held[1].query_features(x_test)
            else:
                x_ctx, x_q, _ = member.features(self.X_train_, x_test, categorical, y_norm)
                self._member_fits[slot0 + i] = (fit_key, member, x_ctx)
            feats.append((np.ascontiguousarray(x_ctx, dtype=np.float32), np.ascontiguousarray(x_q, dtype=np.float32)))
        groups: dict = {}
        for i, (x_ctx, x_q) in enumerate(feats):
            groups.setdefault((x_ctx.shape, x_q.shape), []).append(i)
        batches = []
        for idx in groups.values():
            # exact graph replay keeps every member at one table, as the reference's exact mode does
            size = MEMBER_BATCH if feats[idx[0]][0].shape[1] <= MEMBER_BATCH_MAX_FEATURES else 1
            if graphs.cached_graphs_requested():
                size = 1
            batches += [idx[j:j + size] for j in range(0, len(idx), size)]
        banks: list = [None] * len(members)
        reused = True
        quantized = None
        for batch in batches:
            got = None
            if len(batch) > 1:
                got = self._batched_banks(net, [feats[i][0] for i in batch], [feats[i][1] for i in batch], y_norm,
                                          tuple(slot0 + i for i in batch))
            if got is not None:
                out, was_reused, policy = got
                for j, i in enumerate(batch):
                    banks[i] = out[j]
            else:
                for i in batch:
                    banks[i], was_reused, policy = self._quantile_bank(net, feats[i][0], feats[i][1], y_norm, slot0 + i)
            reused &= was_reused
            if policy.cache_dtype == "int8":
                quantized = policy
        total = banks[0]
        for b in banks[1:]:
            total = total + b
        self._report["context_reused"] = reused
        self._report["ensemble_members"] = len(members)
        if quantized is not None:
            warn_quantized(quantized)  # once per predict, as the reference warns once per call
        return total / len(members)

    def _batched_banks(self, net: FeaturesTransformer, xs_ctx: list, xs_q: list, y_norm: np.ndarray, slots: tuple):
        """Several members' banks from one cache build and apply over their feature matrices
        stacked as tables, or None where the batch does not apply: a policy rung other than a
        resident cache without row chunks (the reference batches only those), or a batch that
        runs out of device memory (recorded; its members are then scored one at a time)."""
        dev = self.device_
        if dev.type != "cuda":
            raise RuntimeError("NoriRegressor runs on a ROCm GPU: the nori_amd kernels have no CPU path")
        amp = bool(self.mix_precision)
        n_groups = math.ceil(xs_ctx[0].shape[1] / net.features_per_group) + 1
        policy = self._policy(net, n_groups, 2 if amp else 4, tables=len(slots))
        if (policy.rung not in ("resident_bf16", "resident_int8") or policy.offload_to_host
                or policy.context_row_chunk is not None or policy.stream_context):
            return None
        slot = ("batch",) + slots
        x_ctx = np.stack(xs_ctx)
        y_ctx = np.broadcast_to(y_norm, (len(slots), len(y_norm))).copy()
        build = dict(cache_dtype=policy.cache_dtype, offload_kv_cache=False, fit_row_chunk=None)
        key = (tuple(sorted(build.items())), amp, str(dev))
        events: list = []
        context = None
        try:
            with torch.inference_mode(), torch.autocast("cuda", dtype=torch.float16, enabled=amp):
                context = self._reused_context(slot, key, x_ctx, y_ctx) if policy.reuse_context_cache else None
                reused = context is not None
                if context is None:
                    context = net.build_context_cache(torch.from_numpy(x_ctx).to(dev), torch.from_numpy(y_ctx).to(dev),
                                                      **build)
                    if policy.reuse_context_cache:
                        retain_context(self._contexts, slot, (key, x_ctx.tobytes(), y_ctx.tobytes(), context),
                                       self._context_budget_bytes())
                xq = torch.from_numpy(np.stack(xs_q)).to(dev)
                bank = net.apply_context_cache(xq, context, adaptive_query_chunk=policy.adaptive_query_chunk,
                                               query_chunk_attempt_callback=lambda q, o: events.append((q, o))).float()
        except torch.cuda.OutOfMemoryError:
            self._attempt_history.append(memory_attempt(
                policy, pipeline_ids=list(slots), path="pipeline_batch", rung=policy.rung, context_row_chunk=None,
                query_chunk=events[-1][0] if events else None, outcome="oom", reason="resolved"))
            self._contexts.pop(slot, None)
            del context
            torch.cuda.empty_cache()
            return None
        if not bool(torch.isfinite(bank).all()):
            raise RuntimeError("the model produced non-finite predictions")  # predictor.py:731-765
        final = _query_trace(policy, events or [(int(xs_q[0].shape[0]), "success")], history=self._attempt_history,
                             pipeline_id=list(slots), context_row_chunk=None, reason="resolved",
                             path="pipeline_batch")
        if self._outcome_policy is None or _severity(final) > _severity(self._outcome_policy):
            self._outcome_policy = final
        self._report = self._outcome_policy.as_report()
        self._report["attempt_history"] = list(self._attempt_history)
        return [bank[j] for j in range(len(slots))], reused, final

    def _yeo_johnson_pass(self, net, x_test, y_norm, point, taus, collapse) -> np.ndarray:
        """With "yj" among the augmentations and a target skew (unbiased) of at least
        ``yj_skew_threshold`` in magnitude: the ensemble again on the Yeo-Johnson-transformed
        target, its point prediction clipped to the transformed context range +/- 3 widths and
        mapped back, averaged with the plain one (rows whose inverse is not finite keep the plain
        one) -- predictor.py:1880-1990. The pass is an augmentation: if the skew test or the pass
        itself raises, the plain prediction is returned (predictor.py:1934-1943, 1995-2003), and
        the power transform's warnings are silenced as the reference silences them."""
        if "yj" not in self.augmentations:
            return point
        try:
            from scipy import stats

            y = np.asarray(y_norm, dtype=np.float64)
            y = y[np.isfinite(y)]
            if len(y) < 10:
                return point
            skew = float(stats.skew(y, bias=False))
        except Exception:
            return point
        if not np.isfinite(skew) or abs(skew) < self.yj_skew_threshold:
            return point
        try:
            import warnings

            from sklearn.preprocessing import PowerTransformer

            pt = PowerTransformer(method="yeo-johnson", standardize=True)
            with warnings.catch_warnings():
                warnings.simplefilter("ignore")
                y_yj = pt.fit_transform(np.asarray(y_norm, dtype=np.float64).reshape(-1, 1)).ravel()
            bank = self._ensemble_bank(net, x_test, y_yj.astype(np.float32), slot0=1000)
            p_yj = self._collapse(bank, taus, collapse)
            lo, hi = y_yj.min(), y_yj.max()
            width = (hi - lo) * 3.0 + 1e-6
            with warnings.catch_warnings():
                warnings.simplefilter("ignore")
                back = pt.inverse_transform(np.clip(p_yj, lo - width, hi + width).reshape(-1, 1)).ravel()
            bad = ~np.isfinite(back)
            back[bad] = point[bad]
            return 0.5 * (point + back)
        except Exception as exc:
            print(f"  [YJ] augmentation failed ({type(exc).__name__}: {exc}), "
                  "falling back to identity-only prediction")
            return point

    def _network(self) -> FeaturesTransformer:
        if self._net is None:
            if isinstance(self.model, FeaturesTransformer):
                net = self.model
            elif self.model_path is not None:
                net = load_model(self.model_path)
            elif self.model is not None:
                raise FileNotFoundError(
                    f"model={self.model!r} names a released checkpoint, which this build does not download; "
                    "pass model_path= to a local checkpoint or model= a built FeaturesTransformer"
                )
            else:
                raise ValueError("NoriRegressor needs model_path= or model=")
            if getattr(net, "two_phase_config", None) is not None or not getattr(net, "supports_context_cache", True):
                raise NotImplementedError("this model has no context cache (the two-phase Nori 1.5 encoder)")
            self._net = net.to(self.device_).eval()
        return self._net

    def _policy(self, net: FeaturesTransformer, n_groups: int, compute_bytes: int, tables: int = 1) -> MemoryPolicy:
        policy = MemoryPolicy.coerce(self.memory_policy)
        vram = None
        if self.device_.type == "cuda":
            vram = torch.cuda.get_device_properties(self.device_).total_memory / 1024**3
        est = tables * estimate_cache_gb(n_context_rows=self.X_train_.shape[0], n_groups=n_groups,
                                         nlayers=net.nlayers, embed_dim=net.embed_dim, bytes_per_element=compute_bytes)
        return policy.resolve(est_cache_gb=est, bytes_per_element=compute_bytes,
                              head_dim=net.embed_dim // net.nhead, total_vram_gb=vram)

    def _quantile_bank(self, net: FeaturesTransformer, x_ctx: np.ndarray, x_test: np.ndarray, y_norm: np.ndarray,
                       slot: int) -> tuple[torch.Tensor, bool]:
        """One member's bank: its context cache (built, or the one an earlier call built from the
        same bytes) applied to its query rows, on the rung the memory policy opens with or, after
        an out-of-memory error, the next one the retry ladder allows (``run_cache_attempts``)."""
        dev = self.device_
        if dev.type != "cuda":
            raise RuntimeError("NoriRegressor runs on a ROCm GPU: the nori_amd kernels have no CPU path")
        amp = bool(self.mix_precision)
        n_groups = math.ceil(x_ctx.shape[1] / net.features_per_group) + 1
        compute_bytes = 2 if amp else 4
        requested = MemoryPolicy.coerce(self.memory_policy)
        resolved = self._policy(net, n_groups, compute_bytes)
        if not resolved.cache:
            raise NotImplementedError(
                f"memory policy resolved to rung {resolved.rung!r}: the uncached forward is not part of this build; "
                "allow the cache (the int8 rungs hold about 1.9x more context than bf16)"
            )

        def attempt(policy: MemoryPolicy, fit_row_chunk, hybrid, on_query, state):
            build = dict(cache_dtype=policy.cache_dtype, offload_kv_cache=policy.offload_to_host,
                         fit_row_chunk=fit_row_chunk)
            streaming = policy.stream_context
            if streaming:
                build["stream_context"] = True
            if hybrid:
                build["_hybrid_resident_int8_prefill"] = True
            key = (tuple(sorted(build.items())), amp, str(dev))
            reuse = policy.reuse_context_cache and not streaming
            with torch.inference_mode(), torch.autocast("cuda", dtype=torch.float16, enabled=amp):
                context = self._reused_context(slot, key, x_ctx, y_norm) if reuse else None
                reused = context is not None
                if context is None:
                    home = torch.device("cpu") if streaming else dev
                    xc = torch.from_numpy(x_ctx).to(home)[None]
                    yc = torch.from_numpy(y_norm).to(home)[None]
                    context = net.build_context_cache(xc, yc, **build)
                    if reuse:
                        retain_context(self._contexts, slot, (key, x_ctx.tobytes(), y_norm.tobytes(), context),
                                       self._context_budget_bytes())
                state["context"] = True
                xq = torch.from_numpy(x_test).to(torch.device("cpu") if streaming else dev)[None]
                bank = net.apply_context_cache(xq, context, adaptive_query_chunk=policy.adaptive_query_chunk,
                                               query_chunk_attempt_callback=on_query)[0].float()
            if not bool(torch.isfinite(bank).all()):
                raise RuntimeError("the model produced non-finite predictions")  # predictor.py:731-765
            return bank, reused

        (bank, reused), final = run_cache_attempts(
            requested, resolved, attempt, bytes_per_element=compute_bytes, head_dim=net.embed_dim // net.nhead,
            history=self._attempt_history, pipeline_id=slot, query_chunk=int(x_test.shape[0]),
            evict=lambda: self._contexts.pop(slot, None))
        if self._outcome_policy is None or _severity(final) > _severity(self._outcome_policy):
            self._outcome_policy = final
        self._report = self._outcome_policy.as_report()
        self._report["attempt_history"] = list(self._attempt_history)
        return bank, reused, final

    def _reused_context(self, slot: int, key, x_ctx: np.ndarray, y_norm: np.ndarray):
        """The context a member encoded in an earlier call, when its cache parameters, its context
        features and its targets are byte for byte the ones of this call."""
        held = self._contexts.get(slot)
        if held is None:
            return None
        k, xb, yb, context = held
        if k == key and xb == x_ctx.tobytes() and yb == y_norm.tobytes():
            self._contexts[slot] = self._contexts.pop(slot)  # most recently used: evicted last
            return context
        del self._contexts[slot]
        return None

    def _context_budget_bytes(self) -> int | None:
        """Device bytes all retained contexts may hold together: a minority share of the GPU's
        memory (predictor.py:2191-2216), None off the GPU."""
        if self.device_.type != "cuda":
            return None
        return int(torch.cuda.get_device_properties(self.device_).total_memory * float(self.context_cache_budget_frac))

