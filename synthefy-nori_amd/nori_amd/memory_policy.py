"""Serving-memory policy of the cached regression path: which cache precision and placement a
request opens with, and the report of what ran.

Restates the decision half of ``synthefy_nori.inference.memory_policy``
(src/synthefy_nori/inference/memory_policy.py): the rung ladder (:105-115), the presets
(:917-966), the footprint estimates (:368-406), the budgets (:1073-1083), the precision and
placement candidates (:1085-1137) and ``resolve`` (:1173-1300). It is pure arithmetic: the
cache it chooses is built by ``FeaturesTransformer.build_context_cache``, whose int8 rungs run
the HIP quantizer. The report (``as_report``) carries the reference's ``memory_report_`` keys.
The runtime half is restated too: ``runtime_fallbacks`` (:1304-1375) lists the precision /
placement rungs an out-of-memory retry may step to, ``fit_row_chunk_attempts`` the bounded
prefill retry ladder below them (:175; predictor.py:1287-1291), ``escalated`` (:1377-1409)
records a rung the retry reached, and ``memory_attempt`` one entry of ``attempt_history``
(``MemoryAttempt``, :480-530); ``NoriRegressor`` drives them (predictor.py:3142-3400).
Not restated: the serving-process coercion (``coerce_for_service``) and the element-budget
subsampling, which belong to the reference's control plane.
"""

from __future__ import annotations

import dataclasses
import os
import warnings
from dataclasses import dataclass, field

from .degradation import CacheQuantizedWarning, DegradedPipelineWarning

__all__ = [
    "ATTEMPT_OUTCOMES",
    "ATTEMPT_REASONS",
    "CACHE_DTYPES",
    "FIT_ROW_CHUNK_RETRY_LADDER",
    "MEMORY_PRESETS",
    "RUNGS",
    "CacheQuantizedWarning",
    "ContextTooLargeError",
    "DegradedPipelineWarning",
    "MemoryPolicy",
    "default_stream_context_row_chunk",
    "estimate_cache_gb",
    "fit_row_chunk_attempts",
    "int8_footprint_gb",
    "memory_attempt",
]

MEMORY_PRESETS = ("exact", "max_context", "off")
CACHE_DTYPES = ("bf16", "int8")
# in decreasing memory cost, as the reference orders them (memory_policy.py:105-115)
RUNGS = ("no_cache", "resident_bf16", "resident_int8", "offload_bf16", "offload_int8", "stream_bf16",
         "stream_int8", "context_row_chunk", "plain_loop")
STREAM_RUNGS = ("stream_bf16", "stream_int8")
DEGRADED_RUNGS = ("offload_bf16", "offload_int8", "stream_bf16", "stream_int8", "context_row_chunk", "plain_loop")

# Bounded prefill retries after the last placement rung (memory_policy.py:175): a context-row
# chunk ladder, never below 256 rows, so an out-of-memory build cannot retry forever.
FIT_ROW_CHUNK_RETRY_LADDER = (2048, 1024, 512, 256)
ATTEMPT_OUTCOMES = ("success", "oom", "unsupported")
ATTEMPT_REASONS = ("resolved", "oom_retry", "fallback_after_oom", "fallback_after_unsupported")
DEFAULT_STREAM_CONTEXT_ROW_CHUNK = 2048

GIB = 1024**3
ASSUMED_VRAM_GB = 24.0  # when the device cannot be asked (memory_policy.py: ASSUMED_VRAM_GB)
# staged-row caps of the streamed context by accelerator size (memory_policy.py:157-168, 201-215)
_STREAM_ROW_CHUNKS = ((80.0, 16384), (40.0, 8192), (0.0, 2048))


class ContextTooLargeError(RuntimeError):
    """The context cannot fit without a fallback the policy forbids (memory_policy.py: ContextTooLargeError)."""


def estimate_cache_gb(*, n_context_rows: int, n_groups: int, nlayers: int, embed_dim: int,
                      bytes_per_element: int) -> float:
    """Full-precision K/V cache of every layer, in GiB: a K and a V vector of ``embed_dim`` per
    (layer, token group, context row) (memory_policy.py:368-389)."""
    return nlayers * n_groups * n_context_rows * 2 * embed_dim * bytes_per_element / GIB


def int8_footprint_gb(est_cache_gb: float, *, bytes_per_element: int, head_dim: int) -> float:
    """The same cache as int8 codes plus one fp32 scale per head vector (memory_policy.py:392-406)."""
    return est_cache_gb / max(bytes_per_element, 1) * (1.0 + 4.0 / max(head_dim, 1))


def default_stream_context_row_chunk(total_vram_gb: float | None) -> int:
    vram = ASSUMED_VRAM_GB if total_vram_gb is None else total_vram_gb
    return next(rows for floor, rows in _STREAM_ROW_CHUNKS if vram >= floor)


def fit_row_chunk_attempts(pinned: int | None) -> list[int]:
    """The prefill retry chunks smaller than ``pinned`` (all of them when nothing is pinned); the
    pinned value itself is the attempt that already failed (predictor.py:1287-1291)."""
    return [c for c in FIT_ROW_CHUNK_RETRY_LADDER if pinned is None or c < pinned]


def memory_attempt(policy: "MemoryPolicy", *, pipeline_ids: list[int], path: str, rung: str,
                   context_row_chunk: int | None, outcome: str, reason: str, dropped_context_rows: int = 0,
                   query_chunk: int | None = None) -> dict:
    """One ``attempt_history`` entry, with the fields and checks of the reference's
    ``MemoryAttempt`` (memory_policy.py:480-530)."""
    if outcome not in ATTEMPT_OUTCOMES:
        raise ValueError(f"unknown attempt outcome {outcome!r}")
    if reason not in ATTEMPT_REASONS:
        raise ValueError(f"unknown attempt reason {reason!r}")
    if rung not in RUNGS:
        raise ValueError(f"unknown rung {rung!r}")
    for name, value in (("context_row_chunk", context_row_chunk), ("query_chunk", query_chunk)):
        if value is not None and value <= 0:
            raise ValueError(f"{name} must be positive, got {value!r}")
    if dropped_context_rows < 0:
        raise ValueError("dropped_context_rows must be >= 0")
    return {"pipeline_ids": list(pipeline_ids), "path": path, "rung": rung, "cache_dtype": policy.cache_dtype,
            "offload_to_host": policy.offload_to_host, "context_row_chunk": context_row_chunk,
            "query_chunk": query_chunk, "outcome": outcome, "reason": reason,
            "dropped_context_rows": dropped_context_rows}


def host_ram_gb() -> float:
    """Physical host memory in GiB, or 0.0 when the platform does not say (then nothing offloads)."""
    try:
        return os.sysconf("SC_PAGE_SIZE") * os.sysconf("SC_PHYS_PAGES") / GIB
    except (ValueError, OSError, AttributeError):
        return 0.0


@dataclass(frozen=True)
class MemoryPolicy:
    """Field names, defaults and meanings of the reference's ``MemoryPolicy`` (memory_policy.py:545-720).

    Request fields: ``cache``, ``reuse_context_cache``, ``cache_dtype`` ("bf16" = the
    projected K/V unquantized), ``allow_quantization``, the GPU and host budgets (a fraction
    of the device's total, or an absolute GiB override), ``offload_to_host``,
    ``stream_context``, ``context_row_chunk``, ``adaptive_query_chunk``, ``elements_budget``,
    ``allow_subsample``. Decided fields (set by ``resolve``): ``rung``, ``est_cache_gb``,
    ``resident_gb``, ``query_chunk``, ``dropped_context_rows``, ``attempt_history``.
    """

    cache: bool = True
    reuse_context_cache: bool = True
    cache_dtype: str = "bf16"
    allow_quantization: bool = True
    gpu_budget_frac: float = 0.4
    gpu_budget_absolute_gb: float | None = None
    offload_to_host: bool = True
    host_budget_frac: float = 0.25
    host_budget_absolute_gb: float | None = None
    stream_context: bool = False
    context_row_chunk: int | None = None
    adaptive_query_chunk: bool = True
    elements_budget: int | None = None
    allow_subsample: bool = True
    rung: str | None = None
    est_cache_gb: float | None = None
    resident_gb: float | None = None
    query_chunk: int | None = None
    dropped_context_rows: int = 0
    attempt_history: tuple = field(default_factory=tuple)

    def __post_init__(self):
        if self.cache_dtype not in CACHE_DTYPES:
            raise ValueError(f"cache_dtype must be one of {CACHE_DTYPES}, got {self.cache_dtype!r}")
        for name in ("gpu_budget_frac", "host_budget_frac"):
            value = getattr(self, name)
            if not 0.0 < value <= 1.0:
                raise ValueError(f"{name} must lie in (0, 1], got {value!r}")
        for name in ("gpu_budget_absolute_gb", "host_budget_absolute_gb"):
            value = getattr(self, name)
            if value is not None and value < 0:
                raise ValueError(f"{name} must be >= 0, got {value!r}")
        for name in ("context_row_chunk", "elements_budget", "query_chunk"):
            value = getattr(self, name)
            if value is not None and value <= 0:
                raise ValueError(f"{name} must be positive, got {value!r}")
        if self.rung is not None and self.rung not in RUNGS:
            raise ValueError(f"unknown rung {self.rung!r}")
        if self.rung is None and not self.cache:
            # the cache levers mean nothing without a cache (memory_policy.py: CACHE_ONLY_FIELDS)
            defaults = MemoryPolicy(cache=True)
            asked = [f for f in ("cache_dtype", "allow_quantization", "offload_to_host", "stream_context",
                                 "context_row_chunk", "gpu_budget_frac", "gpu_budget_absolute_gb",
                                 "host_budget_frac", "host_budget_absolute_gb")
                     if getattr(self, f) != getattr(defaults, f)]
            if asked:
                raise ValueError(f"cache=False makes {asked} meaningless; drop them or enable the cache")
        # explicit streaming is host-only and never falls back to the plain loop (memory_policy.py:734-776)
        if self.stream_context and not self.cache:
            raise ValueError("stream_context=True streams the context K/V cache; it needs cache=True")
        if self.stream_context and not self.offload_to_host:
            raise ValueError("stream_context=True keeps the cache in host memory; it needs offload_to_host=True")
        if self.rung in STREAM_RUNGS and not self.stream_context:
            raise ValueError(f"rung={self.rung!r} belongs to an explicitly streamed context (stream_context=True)")

    # ------------------------------------------------------------------ construction
    @classmethod
    def coerce(cls, value) -> "MemoryPolicy":
        """A policy from None (the defaults), a preset name, a dict of fields or a policy
        (memory_policy.py:917-966). Resolved policies and reports are refused as inputs."""
        if isinstance(value, MemoryPolicy):
            if value.rung is not None:
                raise ValueError("memory_policy= was given an already-resolved policy; pass only the fields to set")
            return value
        if value is None:
            return cls()
        if isinstance(value, dict):
            if value.get("rung") is not None:
                raise ValueError("memory_policy= was given a resolved report (it has a rung); pass only fields to set")
            unknown = set(value) - {f.name for f in dataclasses.fields(cls)}
            if unknown:
                raise ValueError(f"unknown memory_policy fields: {sorted(unknown)}")
            return cls(**value)
        if isinstance(value, str):
            if value == "exact":  # never quantize: offload (bit-exact transport) instead
                return cls(allow_quantization=False)
            if value == "max_context":  # start quantized to hold the largest context
                return cls(cache_dtype="int8")
            if value == "off":
                return cls(cache=False, reuse_context_cache=False)
            raise ValueError(f"unknown memory preset {value!r}; expected one of {MEMORY_PRESETS}, a dict, or a MemoryPolicy")
        raise TypeError(f"memory_policy must be a preset name, dict, MemoryPolicy or None, got {type(value).__name__}")

    # ------------------------------------------------------------------ decision
    def gpu_budget(self, total_vram_gb: float) -> float:
        return self.gpu_budget_absolute_gb if self.gpu_budget_absolute_gb is not None else self.gpu_budget_frac * total_vram_gb

    def host_budget(self, total_ram_gb: float) -> float:
        return self.host_budget_absolute_gb if self.host_budget_absolute_gb is not None else self.host_budget_frac * total_ram_gb

    def precisions(self, *, est_cache_gb: float, bytes_per_element: int, head_dim: int) -> list[tuple[str, float]]:
        """Allowed cache precisions with their footprints, most accurate first (memory_policy.py:1085-1102)."""
        int8_gb = int8_footprint_gb(est_cache_gb, bytes_per_element=bytes_per_element, head_dim=head_dim)
        if self.cache_dtype == "int8":
            return [("int8", int8_gb)]
        return [("bf16", est_cache_gb), ("int8", int8_gb)] if self.allow_quantization else [("bf16", est_cache_gb)]

    def placements(self, *, est_cache_gb: float, bytes_per_element: int, head_dim: int, gpu_budget_gb: float,
                   host_budget_gb: float) -> list[tuple[str, str, bool, float]]:
        """Budget-feasible (rung, dtype, offloaded, footprint) in ladder order: every resident
        precision before any offloaded one (memory_policy.py:1104-1137)."""
        options = self.precisions(est_cache_gb=est_cache_gb, bytes_per_element=bytes_per_element, head_dim=head_dim)
        out = [(f"resident_{dt}", dt, False, gb) for dt, gb in options if gb <= gpu_budget_gb]
        if self.offload_to_host:
            out += [(f"offload_{dt}", dt, True, gb) for dt, gb in options if gb <= host_budget_gb]
        return out

    def resolve(self, *, est_cache_gb: float, bytes_per_element: int, head_dim: int,
                total_vram_gb: float | None = None, total_ram_gb: float | None = None,
                cache_eligible: bool = True) -> "MemoryPolicy":
        """The opening rung of one request as a new, resolved policy (memory_policy.py:1173-1300).

        Streaming takes the most accurate precision the host budget holds, or raises
        ``ContextTooLargeError``; without a cache (switched off or not eligible) the rung is
        ``no_cache``; otherwise the first feasible placement, and ``plain_loop`` when none is.
        """
        vram = ASSUMED_VRAM_GB if total_vram_gb is None else total_vram_gb
        ram = host_ram_gb() if total_ram_gb is None else total_ram_gb
        gpu_gb, host_gb = self.gpu_budget(vram), self.host_budget(ram)

        def decided(rung: str, dtype: str, offload: bool, footprint: float, cache: bool, budgets: bool = True):
            streaming = rung in STREAM_RUNGS
            return dataclasses.replace(
                self, cache=cache, cache_dtype=dtype, offload_to_host=offload,
                reuse_context_cache=False if streaming else bool(cache and self.reuse_context_cache),
                gpu_budget_absolute_gb=0.0 if streaming else (gpu_gb if budgets else None),
                host_budget_absolute_gb=host_gb if budgets else None,
                context_row_chunk=(self.context_row_chunk or default_stream_context_row_chunk(vram)) if streaming
                else self.context_row_chunk,
                rung=rung, est_cache_gb=est_cache_gb, resident_gb=footprint,
            )

        if self.stream_context:
            if not cache_eligible:
                raise ValueError("stream_context=True requires a cache-eligible regression path")
            options = self.precisions(est_cache_gb=est_cache_gb, bytes_per_element=bytes_per_element, head_dim=head_dim)
            for dtype, gb in options:
                if gb <= host_gb:
                    return decided(f"stream_{dtype}", dtype, True, gb, cache=True)
            dtype, gb = options[-1]
            raise ContextTooLargeError(
                f"stream_context=True needs a host-resident cache, but even the {dtype} cache ({gb:.1f} GiB) exceeds "
                f"the host budget ({host_gb:.1f} GiB); raise host_budget_frac / host_budget_absolute_gb or allow int8"
            )
        if not self.cache or not cache_eligible:
            return decided("no_cache", self.cache_dtype, False, 0.0, cache=False, budgets=False)
        options = self.placements(est_cache_gb=est_cache_gb, bytes_per_element=bytes_per_element, head_dim=head_dim,
                                  gpu_budget_gb=gpu_gb, host_budget_gb=host_gb)
        if options:
            rung, dtype, offload, gb = options[0]
            return decided(rung, dtype, offload, gb, cache=True)
        dtype, gb = self.precisions(est_cache_gb=est_cache_gb, bytes_per_element=bytes_per_element,
                                    head_dim=head_dim)[-1]
        return decided("plain_loop", dtype, False, gb, cache=False)

    # ------------------------------------------------------------------ runtime retries
    def runtime_fallbacks(self, resolved: "MemoryPolicy", *, bytes_per_element: int,
                          head_dim: int) -> list["MemoryPolicy"]:
        """The precision / placement rungs an out-of-memory retry walks, starting at
        ``resolved``'s own (memory_policy.py:1304-1375): for a streamed context the host-feasible
        stream precisions; for the resident and offloaded rungs the budget-feasible placements,
        recomputed from ``resolved``'s stored estimate and budgets; nothing for the others.
        ``self`` is the request ``resolved`` came from (its reuse and chunk settings carry over)."""
        est = resolved.est_cache_gb or 0.0
        if resolved.rung in STREAM_RUNGS:
            attempts = [
                dataclasses.replace(resolved, cache=True, reuse_context_cache=False, cache_dtype=dtype,
                                    offload_to_host=True, rung=f"stream_{dtype}", resident_gb=gb,
                                    context_row_chunk=resolved.context_row_chunk or DEFAULT_STREAM_CONTEXT_ROW_CHUNK)
                for dtype, gb in self.precisions(est_cache_gb=est, bytes_per_element=bytes_per_element,
                                                 head_dim=head_dim)
                if gb <= (resolved.host_budget_absolute_gb or 0.0)
            ]
            labels = [a.rung for a in attempts]
            return attempts[labels.index(resolved.rung):]
        if resolved.rung not in ("resident_bf16", "resident_int8", "offload_bf16", "offload_int8"):
            return []
        attempts = [
            dataclasses.replace(resolved, cache=True, reuse_context_cache=self.reuse_context_cache, cache_dtype=dtype,
                                offload_to_host=offload, rung=rung, resident_gb=gb,
                                context_row_chunk=self.context_row_chunk)
            for rung, dtype, offload, gb in self.placements(
                est_cache_gb=est, bytes_per_element=bytes_per_element, head_dim=head_dim,
                gpu_budget_gb=resolved.gpu_budget_absolute_gb or 0.0,
                host_budget_gb=resolved.host_budget_absolute_gb or 0.0)
        ]
        labels = [a.rung for a in attempts]
        if resolved.rung not in labels:
            return [resolved]
        return attempts[labels.index(resolved.rung):]

    def escalated(self, rung: str, *, context_row_chunk: int | None = None, dropped_context_rows: int | None = None,
                  query_chunk: int | None = None) -> "MemoryPolicy":
        """A copy recording the rung a retry reached (memory_policy.py:1377-1409); a streamed
        context never leaves the stream rungs, and the plain loop drops the cache."""
        if self.stream_context and rung not in STREAM_RUNGS:
            raise ValueError(f"stream_context=True cannot escalate to rung={rung!r}; it remains on one of "
                             f"{STREAM_RUNGS} or raises instead of silently using plain_loop.")
        updates: dict = {"rung": rung}
        if context_row_chunk is not None:
            updates["context_row_chunk"] = context_row_chunk
        if dropped_context_rows is not None:
            updates["dropped_context_rows"] = dropped_context_rows
        if query_chunk is not None:
            updates["query_chunk"] = query_chunk
        if rung == "plain_loop":
            updates.update(cache=False, reuse_context_cache=False, offload_to_host=False)
        return dataclasses.replace(self, **updates)

    # ------------------------------------------------------------------ report
    @property
    def is_degraded(self) -> bool:
        return self.rung in DEGRADED_RUNGS

    @property
    def is_bit_exact(self) -> bool:
        """No int8 cache and no explicit streaming (the reference's cache-fidelity flag)."""
        return self.cache_dtype != "int8" and self.rung not in STREAM_RUNGS

    def describe(self) -> str:
        return (f"rung={self.rung} cache_dtype={self.cache_dtype} offload={self.offload_to_host} "
                f"est_cache_gb={self.est_cache_gb} resident_gb={self.resident_gb}")

    def as_report(self) -> dict:
        """The ``memory_report_`` dict: every field, with the attempt history as plain dicts."""
        report = dataclasses.asdict(self)
        report["attempt_history"] = [dict(a) for a in self.attempt_history]
        return report

    def with_outcome(self, **updates) -> "MemoryPolicy":
        return dataclasses.replace(self, **updates)


def warn_quantized(policy: MemoryPolicy) -> None:
    """The int8-cache notice of the reference predictor (predictor.py:3286-3305)."""
    warnings.warn(
        f"Nori quantized the context cache to int8: {policy.describe()}. Predictions carry a small numerical "
        "difference from bf16; set memory_policy={'allow_quantization': False} to prevent cache quantization.",
        CacheQuantizedWarning,
        stacklevel=3,
    )
