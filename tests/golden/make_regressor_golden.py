"""Write the golden vectors of the nori-6m end-to-end case and of the memory-policy ladder.

Runs the reference's own code on the CPU in fp32 (in this container only; the product of this
script is the .npz data beside it, never the reference's code):

* the nori-6m case (tests/regressor_case.py): a random-init nori-6m model whose weights are a
  pure function of a stored per-parameter scale table and numpy's integer-based stream is
  built with this package, its state dict loaded strictly into the reference's ``FeaturesTransformer``
  (src/synthefy_nori/model/transformer.py:70-369), and the reference's context-cache API runs
  the table with an int8 cache -- ``build_context_cache(cache_dtype="int8")`` then
  ``apply_context_cache`` (:813-1078) -- on the standardized target, as ``NoriRegressor``'s
  cached path does (api.py:1122-1151; predictor.py:3228-3265). Stored: the table, the scale
  table and the SHA-256 of the weights, the 999-level quantile bank, the reference's point prediction
  (``quantile_dist_mean_simple``, quantile_dist.py:95-135) mapped back to target units, and
  the reference's layer-0 int8 cache codes and scales of the first 128 context rows.
* the ladder: the reference's ``MemoryPolicy.resolve`` (inference/memory_policy.py:1173-1300)
  over presets, fields and cache sizes, with the report keys (``model_dump``).

A second fixture, tests/golden/regressor_autocast_goldens.npz, holds the same case run by the
reference under ``torch.autocast("cpu", dtype=torch.float16)`` with CUDA autocast's op policy
(tests/golden/cuda_autocast_policy.py) -- its predictor's own GPU mode (predictor.py:3208-3217)
-- and its spread: the largest relative change of each output (point
predictions, the 0.1 / 0.5 / 0.9 quantiles, the median, the whole bank) when the same fp16 run
takes the context rows in three other orders (the outputs do not depend on that order except
through the order of the sums), next to its distance from the fp32 run.

Usage: python tests/golden/make_regressor_golden.py
(writes tests/golden/regressor_goldens.npz and tests/golden/regressor_autocast_goldens.npz)
"""

from __future__ import annotations

import json
import os
import sys
import types

import numpy as np
import torch

REFERENCE_SRC = "/root/reference/src"
HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "regressor_goldens.npz")
OUT_AUTOCAST = os.path.join(HERE, "regressor_autocast_goldens.npz")
sys.path[:0] = [os.path.dirname(HERE), os.path.join(os.path.dirname(os.path.dirname(HERE)), "synthefy-nori_amd")]

import regressor_case as case  # noqa: E402
from cuda_autocast_policy import cuda_policy  # noqa: E402

# (label, policy request, est_cache_gb, bytes_per_element, head_dim, vram_gb, ram_gb)
LADDER_CASES = [
    ("default fits", None, 2.0, 2, 64, 24.0, 64.0),
    ("default int8 fallback", None, 12.0, 2, 64, 24.0, 64.0),
    ("default offload", None, 30.0, 2, 64, 24.0, 256.0),
    ("default plain loop", None, 300.0, 2, 64, 24.0, 64.0),
    ("exact offloads", "exact", 12.0, 2, 64, 24.0, 64.0),
    ("max_context", "max_context", 2.0, 2, 64, 24.0, 64.0),
    ("off", "off", 2.0, 2, 64, 24.0, 64.0),
    ("stream bf16", {"stream_context": True}, 2.0, 2, 64, 288.0, 64.0),
    ("stream int8", {"stream_context": True}, 30.0, 2, 44, 288.0, 64.0),
    ("stream explicit chunk", {"stream_context": True, "context_row_chunk": 4096}, 2.0, 4, 56, 24.0, 64.0),
    ("absolute gpu budget", {"gpu_budget_absolute_gb": 1.0}, 1.5, 2, 64, 288.0, 512.0),
    ("no offload", {"offload_to_host": False}, 200.0, 2, 64, 288.0, 512.0),
    ("fp32 footprint", {"cache_dtype": "int8"}, 100.0, 4, 44, 288.0, 64.0),
]


def load_reference():
    for name, sub in (("synthefy_nori", "synthefy_nori"), ("synthefy_nori.model", "synthefy_nori/model"),
                      ("synthefy_nori.inference", "synthefy_nori/inference")):
        mod = types.ModuleType(name)
        mod.__path__ = [os.path.join(REFERENCE_SRC, sub)]
        sys.modules[name] = mod
    import synthefy_nori.inference.memory_policy as mp
    import synthefy_nori.model.layer as layer
    import synthefy_nori.model.quantile_dist as qd
    import synthefy_nori.model.transformer as tr

    return tr, layer, qd, mp


def main():
    tr, layer, qd, mp = load_reference()
    from nori_amd import api, transformer as our_tr

    torch.set_num_threads(8)
    out: dict[str, np.ndarray] = {}

    # ---- the nori-6m case
    torch.manual_seed(0)
    scales = case.weight_scales(api.build_model(api.NORI_6M_CONFIG))
    ours = case.seeded_model(our_tr.FeaturesTransformer, api.NORI_6M_CONFIG, scales)
    ref = tr.FeaturesTransformer(**api.NORI_6M_CONFIG).eval()
    ref.load_state_dict(ours.state_dict(), strict=True)
    for m in ref.modules():
        if isinstance(m, layer.RMSNorm):
            m.use_native = True
    x_tr, y_tr, x_te, y_te = case.table()
    y_mean, y_std = float(y_tr.mean()), float(y_tr.std())
    y_norm = ((y_tr - y_mean) / y_std).astype(np.float32)
    with torch.inference_mode():
        ctx = ref.build_context_cache(torch.from_numpy(x_tr)[None], torch.from_numpy(y_norm)[None], cache_dtype="int8")
        bank = ref.apply_context_cache(torch.from_numpy(x_te)[None], ctx)[0].float()
        taus = torch.tensor(ref.regression_quantiles, dtype=torch.float64)
        point = qd.quantile_dist_mean_simple(bank.double(), taus, enforce_monotone_first=True)
        skv = ctx.caches[0]["seq_kv"]
        codes0, scales0 = skv._q, skv._scale
    out["case/x_train"], out["case/y_train"], out["case/x_test"], out["case/y_test"] = x_tr, y_tr, x_te, y_te
    out["case/weights_sha256"] = np.array(case.weights_sha256(ours))
    out["case/weight_scales"] = np.array(json.dumps(scales))
    out["case/bank_norm"] = bank.numpy()
    out["case/taus"] = taus.numpy()
    out["case/point_norm"] = point.numpy()
    out["case/point"] = point.numpy() * y_std + y_mean
    out["case/codes0"] = codes0[:, :128].numpy()  # layer 0's cache, first 128 context rows
    out["case/scales0"] = scales0[:, :128].numpy()

    # ---- the same case under the reference's fp16 autocast, and its spread over context orders
    def median_of(srt):
        n = srt.shape[1]
        return 0.5 * (srt[:, n // 2 - 1] + srt[:, n // 2]) if n % 2 == 0 else srt[:, n // 2]

    def autocast_run(rows):
        with torch.inference_mode(), torch.autocast("cpu", dtype=torch.float16), cuda_policy():
            c = ref.build_context_cache(torch.from_numpy(x_tr[rows])[None], torch.from_numpy(y_norm[rows])[None],
                                        cache_dtype="int8")
            b = ref.apply_context_cache(torch.from_numpy(x_te)[None], c)[0].float()
        p = qd.quantile_dist_mean_simple(b.double(), taus, enforce_monotone_first=True).numpy() * y_std + y_mean
        srt = np.sort(b.numpy().astype(np.float64), axis=1) * y_std + y_mean
        outs = {"point": p, "bank": srt, "median": median_of(srt)}
        for level in case.QUANTILE_LEVELS:
            outs[f"q{level}"] = srt[:, int(round(level * 1000)) - 1]
        return b.numpy(), outs

    def rel(a, b):
        return float(np.abs(np.asarray(a, np.float64) - b).max() / np.abs(b).max())

    ac: dict[str, np.ndarray] = {}
    bank_ac, outs = autocast_run(np.arange(len(x_tr)))
    ac["bank_norm"] = bank_ac
    ac["point"] = outs["point"]
    fp32_sorted = np.sort(bank.numpy().astype(np.float64), axis=1) * y_std + y_mean
    fp32_outs = {"point": out["case/point"], "bank": fp32_sorted, "median": median_of(fp32_sorted)}
    for level in case.QUANTILE_LEVELS:
        fp32_outs[f"q{level}"] = fp32_sorted[:, int(round(level * 1000)) - 1]
    spread = {k: 0.0 for k in outs}
    for seed in range(3):
        _, outs_p = autocast_run(np.random.default_rng(300 + seed).permutation(len(x_tr)))
        for k in outs:
            spread[k] = max(spread[k], rel(outs_p[k], outs[k]))
    for k in outs:
        ac[f"spread/{k}"] = np.array(spread[k])
        ac[f"vs_fp32/{k}"] = np.array(rel(outs[k], fp32_outs[k]))
    np.savez_compressed(OUT_AUTOCAST, **ac)
    print("fp16 autocast: spread over context orders " + ", ".join(f"{k} {v:.2e}" for k, v in spread.items()))

    # ---- the ladder
    rows = []
    for label, request, est, bpe, hd, vram, ram in LADDER_CASES:
        row = {"label": label, "request": request, "est": est, "bpe": bpe, "head_dim": hd, "vram": vram, "ram": ram}
        try:
            resolved = mp.MemoryPolicy.coerce(request).resolve(
                est_cache_gb=est, bytes_per_element=bpe, head_dim=hd, total_vram_gb=vram, total_ram_gb=ram
            )
        except Exception as exc:  # the refusal is the recorded outcome
            row["error"] = type(exc).__name__
        else:
            dump = resolved.model_dump()
            row["report"] = {k: dump[k] for k in dump if k != "attempt_history"}
            row["report_keys"] = sorted(dump)
            # the runtime out-of-memory retries from that opening rung (memory_policy.py:1304-1375)
            fallbacks = mp.MemoryPolicy.coerce(request).runtime_fallbacks(resolved, bytes_per_element=bpe, head_dim=hd)
            row["fallbacks"] = [{k: v for k, v in f.model_dump().items() if k != "attempt_history"} for f in fallbacks]
            # a retry's escalation records (memory_policy.py:1377-1409)
            try:
                esc = resolved.escalated("context_row_chunk", context_row_chunk=512, query_chunk=64)
                row["escalated_chunk"] = {k: v for k, v in esc.model_dump().items() if k != "attempt_history"}
            except Exception as exc:
                row["escalated_chunk"] = type(exc).__name__
            try:
                esc = resolved.escalated("plain_loop", dropped_context_rows=7)
                row["escalated_plain"] = {k: v for k, v in esc.model_dump().items() if k != "attempt_history"}
            except Exception as exc:
                row["escalated_plain"] = type(exc).__name__
        rows.append(row)
    out["ladder/json"] = np.array(json.dumps(rows))
    out["ladder/fit_row_chunk_retry"] = np.array(mp.FIT_ROW_CHUNK_RETRY_LADDER, dtype=np.int64)
    # one attempt_history entry as the reference's MemoryAttempt writes it (memory_policy.py:480-530)
    resolved = mp.MemoryPolicy.coerce({"cache_dtype": "int8"}).resolve(
        est_cache_gb=2.0, bytes_per_element=2, head_dim=64, total_vram_gb=24.0, total_ram_gb=64.0)
    attempt = mp.MemoryAttempt(pipeline_ids=[3], path="cached", rung="context_row_chunk",
                               cache_dtype=resolved.cache_dtype, offload_to_host=resolved.offload_to_host,
                               context_row_chunk=512, query_chunk=None, outcome="oom", reason="oom_retry",
                               dropped_context_rows=0).model_dump()
    out["ladder/attempt_json"] = np.array(json.dumps(attempt))
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT}: point predictions {out['case/point'][:4]}, ladder {[r.get('report', {}).get('rung', r.get('error')) for r in rows]}")


if __name__ == "__main__":
    main()
