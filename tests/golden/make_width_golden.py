"""Write golden vectors for the model-level cases at head widths 44 and 56 (tests/width_cases.py).

Runs the reference's own modules (src/synthefy_nori/model/layer.py: ``EncoderBaseLayer``,
``LayerStack`` build_train_cache / forward_test_with_cache, :1771-1967, 2058-2108;
transformer.py: ``FeaturesTransformer`` build_context_cache / apply_context_cache, :813-1078) on
the CPU, twice per case:

* in fp32, with a full-precision and an int8 cache;
* under ``torch.autocast("cpu", dtype=torch.float16)`` with CUDA autocast's op policy
  (tests/golden/cuda_autocast_policy.py) and an int8 cache -- the reference's own fp16
  autocast run, the mode its predictor uses on a GPU (predictor.py:3208-3217) -- and
  again with the context rows in three other orders. The outputs do not depend on the order of
  the context rows, except through the order of the sums; the largest relative change over the
  three orders is stored as ``spread_*``: how far the reference's own fp16 run moves when only
  its summation order changes.

The weights are ``width_cases.seeded_state`` of the reference constructor's (mean, std) per
parameter; the fixture (tests/golden/width_goldens.npz) holds that table, the weights' SHA-256
and the outputs; the inputs are regenerated from their seeds. Only this container holds the
reference (at /root/reference), whose package ``__init__`` files are skipped as in
make_golden.py.

Usage: python tests/golden/make_width_golden.py   (writes tests/golden/width_goldens.npz)
"""

from __future__ import annotations

import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "width_goldens.npz")
sys.path[:0] = [HERE, os.path.dirname(HERE)]

import regressor_case as case  # noqa: E402
import width_cases as wc  # noqa: E402
from cuda_autocast_policy import cuda_policy  # noqa: E402
from make_golden import load_reference  # noqa: E402

CPU = torch.device("cpu")


def f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def stack_case(L, idx: int, tag: str, out: dict) -> None:
    c = wc.STACKS[tag]
    torch.manual_seed(40 + idx)
    layers = [L.EncoderBaseLayer(**wc.layer_kwargs(c)).eval() for _ in range(c["layers"])]
    for layer in layers:
        for m in layer.modules():
            if isinstance(m, L.RMSNorm):
                m.use_native = True  # the serving setting (utils/loading.py:272-277)
    stack = L.LayerStack(layers).eval()
    scales = case.weight_scales(stack)
    stack.load_state_dict(wc.seeded_state(stack.state_dict(), scales, 40 + idx), strict=True)
    x_train, x_test = (torch.from_numpy(a) for a in wc.stack_inputs(tag))

    def run(xt, quant, autocast):
        with torch.inference_mode(), torch.autocast("cpu", dtype=torch.float16, enabled=autocast), cuda_policy():
            tr_out, caches = stack.build_train_cache(xt.clone(), quantize_kv_cache=quant, device=CPU)
            te_out = stack.forward_test_with_cache(x_test.clone(), caches)
        return f32(tr_out), f32(te_out), caches

    # the context rows' outputs are stored for every ROW_STEP-th row and layer 0's codes for the
    # first CODE_ROWS rows (the fixture stays small; the GPU run computes every row)
    for quant in (False, True):
        sfx = "int8" if quant else "fp"
        tr, te, caches = run(x_train, quant, False)
        out[f"{tag}/train_out_{sfx}"], out[f"{tag}/test_out_{sfx}"] = tr[:, ::wc.ROW_STEP], te[:, ::wc.QUERY_STEP]
        if quant:
            out[f"{tag}/codes0"] = caches[0]["seq_kv"]._q[:, : wc.CODE_ROWS].numpy()
    tr, te, caches = run(x_train, True, True)
    out[f"{tag}/train_out_int8_ac"], out[f"{tag}/test_out_int8_ac"] = tr[:, ::wc.ROW_STEP], te[:, ::wc.QUERY_STEP]
    out[f"{tag}/codes0_ac"] = caches[0]["seq_kv"]._q[:, : wc.CODE_ROWS].numpy()
    s_tr = s_te = 0.0
    for perm in wc.permutations(x_train.shape[1]):
        tr_p, te_p, _ = run(x_train[:, perm], True, True)
        s_tr = max(s_tr, wc.relative(tr_p, tr[:, perm]))
        s_te = max(s_te, wc.relative(te_p, te))
    out[f"{tag}/spread_train_out_int8_ac"] = np.array(s_tr)
    out[f"{tag}/spread_test_out_int8_ac"] = np.array(s_te)
    out[f"{tag}/weight_scales"] = np.array(json.dumps(scales))
    out[f"{tag}/weights_sha256"] = np.array(case.weights_sha256(stack))
    print(f"{tag}: fp16 autocast vs fp32 {wc.relative(te[:, ::wc.QUERY_STEP], out[f'{tag}/test_out_int8']):.3e}, "
          f"spread over context orders {s_te:.3e} (test rows), {s_tr:.3e} (context rows)", flush=True)


def model_case(L, T, idx: int, tag: str, out: dict) -> None:
    c = wc.MODELS[tag]
    torch.manual_seed(50 + idx)
    model = T.FeaturesTransformer(**wc.model_config(c)).eval()
    for m in model.modules():
        if isinstance(m, L.RMSNorm):
            m.use_native = True
    scales = case.weight_scales(model)
    model.load_state_dict(wc.seeded_state(model.state_dict(), scales, 50 + idx, wc.head_name(model)), strict=True)
    x_np, y_np = wc.model_table(tag)
    x, y = torch.from_numpy(x_np), torch.from_numpy(y_np)
    n_ctx = c["n_ctx"]

    def run(xc, yc, cache_dtype, autocast):
        with torch.inference_mode(), torch.autocast("cpu", dtype=torch.float16, enabled=autocast), cuda_policy():
            ctx = model.build_context_cache(xc, yc, cache_dtype=cache_dtype)
            return f32(model.apply_context_cache(x[:, n_ctx:], ctx))

    for cache_dtype in ("bf16", "int8"):
        out[f"{tag}/pred_{cache_dtype}"] = run(x[:, :n_ctx], y, cache_dtype, False)
    pred_ac = run(x[:, :n_ctx], y, "int8", True)
    out[f"{tag}/pred_int8_ac"] = pred_ac
    spread = 0.0
    for perm in wc.permutations(n_ctx):
        spread = max(spread, wc.relative(run(x[:, :n_ctx][:, perm], y[:, perm], "int8", True), pred_ac))
    out[f"{tag}/spread_pred_int8_ac"] = np.array(spread)
    out[f"{tag}/weight_scales"] = np.array(json.dumps(scales))
    out[f"{tag}/weights_sha256"] = np.array(case.weights_sha256(model))
    print(f"{tag}: fp16 autocast vs fp32 {wc.relative(pred_ac, out[f'{tag}/pred_int8']):.3e}, "
          f"spread over context orders {spread:.3e}", flush=True)


def main():
    L, _ = load_reference()
    import synthefy_nori.model.transformer as T

    torch.set_num_threads(8)
    out: dict[str, np.ndarray] = {}
    for idx, tag in enumerate(wc.STACKS):
        stack_case(L, idx, tag, out)
    for idx, tag in enumerate(wc.MODELS):
        model_case(L, T, idx, tag, out)
    np.savez_compressed(OUT, **out)
    total = sum(v.nbytes for v in out.values())
    print(f"wrote {OUT}: {len(out)} arrays, {total / 1e6:.2f} MB uncompressed")


if __name__ == "__main__":
    main()
