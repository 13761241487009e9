"""Write golden vectors for the cached sequence-attention layer path.

Runs the reference's own model code (synthefy_nori.model.layer and .kv_cache_scaling,
src/synthefy_nori/model/layer.py:459-1162, 1164-1967, 2058-2108) on the CPU in fp32, on
reduced random-init modules built with nori-6m's layer flags (smf arch, pre-norm RMSNorm,
SwiGLU, deepnorm alpha, isolated sequence attentions, QASS "full"), and stores their
weights, inputs and outputs as arrays. Nothing else pins these functions: they compose
projections, QASS, attention, norms and MLPs whose composition has no closed form.

Only this container holds the reference (at /root/reference); the committed product of this
script is the .npz data beside it, never the reference's code. The package's parent
``__init__`` files are skipped (they pull in the product API's optional dependencies): the
model modules import only torch, numpy and einops.

Usage: python tests/golden/make_golden.py   (writes tests/golden/layer_cache_goldens.npz)
"""

from __future__ import annotations

import os
import sys
import types

import numpy as np
import torch

REFERENCE_SRC = "/root/reference/src"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "layer_cache_goldens.npz")


def load_reference():
    for name, sub in (("synthefy_nori", "synthefy_nori"), ("synthefy_nori.model", "synthefy_nori/model")):
        mod = types.ModuleType(name)
        mod.__path__ = [os.path.join(REFERENCE_SRC, sub)]
        sys.modules[name] = mod
    import synthefy_nori.model.kv_cache_scaling as kv_mod
    import synthefy_nori.model.layer as layer_mod

    return layer_mod, kv_mod


def perturb_qass(attn, gen):
    """QASS initializes its last layers to zero (q * log n); give them small weights so the
    learned base and gate terms are exercised."""
    if attn.qassmax is None:
        return
    for mlp in (attn.qassmax.base_mlp, attn.qassmax.gate_mlp):
        if mlp is None:
            continue
        with torch.no_grad():
            mlp[-1].weight.copy_(torch.randn(mlp[-1].weight.shape, generator=gen) * 0.1)
            mlp[-1].bias.copy_(torch.randn(mlp[-1].bias.shape, generator=gen) * 0.1)


def row_slices(t, widths):
    start = 0
    for w in widths:
        yield t[:, start : start + w]
        start += w


def main():
    L, K = load_reference()
    torch.set_num_threads(4)
    out: dict[str, np.ndarray] = {}

    def put(prefix, name, t):
        out[f"{prefix}/{name}"] = t.detach().cpu().numpy()

    # ---------------------------------------------------------------- a6 / a7: one attention
    for tag, copy_first in (("mha", False), ("mqa", True)):
        torch.manual_seed(10)
        E, H = 32, 2
        attn = L.MultiheadAttention(E, H, qkv_combined=False, use_qassmax=True, qass_mode="full").eval()
        gen = torch.Generator().manual_seed(11)
        perturb_qass(attn, gen)
        x_ctx = torch.randn(2, 3, 100, E, generator=gen)  # [B, G, N, E] (rows/features transposed)
        x_q = torch.randn(2, 3, 37, E, generator=gen)
        with torch.inference_mode():
            cache = attn.project_kv_cache(x_ctx, copy_first_head_kv=copy_first)
            dense = attn.forward_with_kv_cache(x_q, cache)[0]
            scal = K.ScalableSeqKV(cache["kv"], cache["batch"], cache["groups"], quantize=True, device=torch.device("cpu"))
            int8 = attn.forward_with_kv_cache(x_q, scal)[0]
            bw = K.BlockwiseSeqKV.from_row_slices(
                row_slices(cache["kv"], (64, 1, 35)), cache["batch"], cache["groups"], quantize=True,
                device=torch.device("cpu"), dtype=cache["kv"].dtype, offload=True,
            )
            blockwise = attn.forward_with_kv_cache(x_q, bw)[0]
        p = f"attn_{tag}"
        for k, v in attn.state_dict().items():
            put(p, "w." + k, v)
        put(p, "x_ctx", x_ctx)
        put(p, "x_q", x_q)
        put(p, "kv", cache["kv"])
        put(p, "codes", scal._q)
        put(p, "scales", scal._scale)
        put(p, "out_dense", dense)
        put(p, "out_int8", int8)
        put(p, "out_blockwise_int8", blockwise)

    # ---------------------------------------------------------------- a12 / a13: a two-layer stack
    for tag, cross_share in (("stack", False), ("stack_mqa", True)):
        torch.manual_seed(20)
        E, H, HID, NL = 32, 2, 48, 2
        layers = [
            L.EncoderBaseLayer(
                nhead=H, embed_dim=E, hid_dim=HID, pre_norm=True, activation="swiglu", layer_arch="smf",
                seq_attn_isolated=True, cross_share_all_kv_heads=cross_share, use_qassmax=True,
                norm_type="rmsnorm", deepnorm_alpha=NL ** -0.5, qass_mode="full",
            ).eval()
            for _ in range(NL)
        ]
        gen = torch.Generator().manual_seed(21)
        for layer in layers:
            for attn in layer.sequence_attentions:
                perturb_qass(attn, gen)
            for m in layer.modules():
                if isinstance(m, L.RMSNorm):
                    m.use_native = True  # the serving setting (utils/loading.py:272-277)
        stack = L.LayerStack(layers).eval()
        x_train = torch.randn(2, 100, 3, E, generator=gen)  # [B, N, G, E]
        x_test = torch.randn(2, 29, 3, E, generator=gen)
        p = tag
        with torch.inference_mode():
            for quant in (False, True):
                xt = x_train.clone()
                xt_out, caches = stack.build_train_cache(xt, quantize_kv_cache=quant, device=torch.device("cpu"))
                y = stack.forward_test_with_cache(x_test.clone(), caches)
                sfx = "int8" if quant else "fp"
                put(p, f"train_out_{sfx}", xt_out)
                put(p, f"test_out_{sfx}", y)
                for i, c in enumerate(caches):
                    skv = c["seq_kv"]
                    if quant:
                        put(p, f"codes{i}", skv._q)
                        put(p, f"scales{i}", skv._scale)
        for k, v in stack.state_dict().items():
            put(p, "w." + k, v)
        put(p, "x_train", x_train)
        put(p, "x_test", x_test)
        out[f"{p}/config"] = np.array([E, H, HID, NL, int(cross_share)], dtype=np.int64)

    np.savez_compressed(OUT, **out)
    total = sum(v.nbytes for v in out.values())
    print(f"wrote {OUT}: {len(out)} arrays, {total / 1e6:.2f} MB uncompressed")


if __name__ == "__main__":
    main()
