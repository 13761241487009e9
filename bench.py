"""Benchmark of the Nori ICL hot path on one MI355X.

Workload (the long-context configuration the headline metric is quoted on): nori-30m
block dims -- 12 layers, embed 352, 8 heads of width 44 -- one table whose 64 features
give 33 feature-group tokens, a 65,536-row context and 4 query batches of 1,024 rows.

One step is the whole ICL stage of that job, with inputs resident in HBM:
  * cache build: every layer's full-precision (fp16, the GPU autocast dtype) context
    K/V [33, 65536, 2, 8, 44] is quantized to the int8 cache (HIP codec);
  * 4 query batches x 12 layers of the cached sequence-attention sublayer
    (layer.py:1945-1953 with forward_with_kv_cache :685-745): RMSNorm of the query
    tokens (HIP), Q projection (hipBLASLt GEMM), query -> context attention over the
    int8 cache (HIP, int8 K/V dequantized in registers), output projection and the
    deepnorm residual.
value = query rows per second of the step (4,096 rows per step).

The JSON line also carries the roofline of the dominant kernel (attention, bound by
dense fp16/bf16 MFMA at 2.5 PFLOP/s), measured with HIP events on the launch stream
around each attention call (its kernel and, when the context is split, the merge of
the partials), the same for the quantize kernel against 8 TB/s of HBM, the HBM traffic
per launch measured by rocprofv3 counters (profiles/traffic_nori30m_64k.md, when
present), the fused context-cache write (RMSNorm -> K/V projection -> int8 codes) of one
layer against the unfused sequence it replaces, one layer's prefill self-attention over the
fp16 context K/V, the same configuration through the model-level context-cache API
(build once, 4 query batches), the kernel-level legs of the nori-6m block and the nori-100m
layer, config 4 end to end (a nori-100m-dims model over 32 tables of 8192 context + 2048 query
rows, built and applied 8 tables at a time), the many-small-tables path (512 tables through a nori-1-5-sized two-phase model), the
context-side RMSNorm against HBM bandwidth, config 1 (NoriRegressor fit/predict on a nori-6m
table of 1024 + 256 rows with an int8 cache), and the CPU baseline: the same step as the
reference runs it on the CPU -- fp32 torch on every host core, through oracle.sublayer (the
reference's quantizer expression, and the cached sequence-attention sublayer with the
online-softmax scan of layer.py:777-839 over the GPU-built int8 codes) -- timed on a bounded
sample of token groups and extrapolated.
"""

from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "synthefy-nori_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK = 8.0e12  # B/s
MFMA_BF16_PEAK = 2.5e15  # FLOP/s, dense
TRAFFIC_SUMMARY = os.path.join(ROOT, "profiles", "traffic_nori30m_64k.md")

# nori-30m block dims and the 64k-row context configuration
LAYERS, EMBED, HEADS, HEAD_DIM = 12, 352, 8, 44
GROUPS = 33  # ceil(64 features / 2 per group) + 1 target token
CONTEXT_ROWS = 65536
QUERY_BATCHES, QUERY_ROWS = 4, 1024
DEEPNORM_ALPHA = LAYERS ** -0.5


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=3)
    p.add_argument("--warmup", type=int, default=1)
    p.add_argument("--layers", type=int, default=LAYERS, help=argparse.SUPPRESS)
    p.add_argument("--cpu-baseline", choices=["on", "off"], default="on")
    p.add_argument("--cpu-sample-groups", type=int, default=8,
                   help="token groups (of 33) of one layer in the CPU baseline's timed sample")
    p.add_argument(
        "--streamed", action="store_true",
        help="measure the host-streamed long-context path instead: one layer's int8 cache in pinned host "
        "blocks, one 1024-row query batch, block copies overlapped with attention vs serialized",
    )
    p.add_argument(
        "--probe-traffic", action="store_true",
        help="run a 1 GiB device copy (counter calibration), one quantize, one attention and one dequantize "
        "launch of the workload twice, untimed, for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE passes",
    )
    p.add_argument(
        "--other-configs", action="store_true",
        help="measure only the kernel-level legs of configs 2 (nori-6m block) and 4 (nori-100m layer)",
    )
    p.add_argument(
        "--small-tables", action="store_true",
        help="measure only the many-small-tables path: a nori-1-5-shaped two-phase model over 512 tables of "
        "256 context + 64 query rows",
    )
    p.add_argument(
        "--config1", action="store_true",
        help="measure only config 1: NoriRegressor fit/predict on a nori-6m table of 1024 context + 256 query rows",
    )
    p.add_argument(
        "--config4", action="store_true",
        help="measure only config 4 end to end: a nori-100m-dims model over 32 tables of 8192 context + 2048 query "
        "rows, built and applied 8 tables at a time through the context-cache API",
    )
    p.add_argument(
        "--model", action="store_true",
        help="measure only the model-level context-cache API end to end (build once, 4 query batches)",
    )
    p.add_argument(
        "--prefill", action="store_true",
        help="measure only one layer's prefill self-attention (65536 x 65536, fp16 K/V)",
    )
    p.add_argument(
        "--mfma-ceiling", action="store_true",
        help="measure only the dense f16 MFMA rate under the power limit (random vs all-zero operands) and the "
        "workload's attention launch on its real cache vs an all-zero cache",
    )
    p.add_argument(
        "--cache-write", action="store_true",
        help="measure only the fused context-cache write of one layer against the unfused sequence "
        "(also the command its rocprofv3 trace and counters are taken with)",
    )
    return p.parse_args()


def probe_traffic(torch, dev):
    import nori_amd
    from nori_amd.kv_cache_scaling import _dequantize_into, _quantize_into

    a = torch.empty(1 << 30, dtype=torch.uint8, device=dev).fill_(1)
    b = torch.empty_like(a)
    g = torch.Generator(device=dev).manual_seed(2)
    kv = torch.randn((GROUPS, CONTEXT_ROWS, 2, HEADS, HEAD_DIM), generator=g, device=dev, dtype=torch.float16)
    codes = torch.empty(kv.shape, dtype=torch.int8, device=dev)
    scales = torch.empty(kv.shape[:-1] + (1,), dtype=torch.float32, device=dev)
    q = torch.randn((GROUPS, QUERY_ROWS, HEADS, HEAD_DIM), generator=g, device=dev, dtype=torch.float16)
    out = torch.empty_like(kv)
    for _ in range(2):
        b.copy_(a)
        _quantize_into(kv, codes, scales)
        nori_amd.icl_attention(q, codes, scales)
        _dequantize_into(codes, scales, out)
    torch.cuda.synchronize()
    print("traffic probe: 2 x (1 GiB copy, quantize, attention, dequantize) done", flush=True)


def streamed(torch, dev, args, block_rows=8192):
    """Host-streamed long-context attention (BlockwiseSeqKV offloaded, layer.py:841-934): the
    PCIe-inclusive rate. The layer's int8 cache lives in pinned host blocks of block_rows rows;
    each query batch stages every block to the device. Prints one JSON line."""
    import nori_amd
    from nori_amd import attention as attn
    from nori_amd.kv_cache_scaling import BlockwiseSeqKV

    g = torch.Generator(device=dev).manual_seed(2)
    kv = torch.randn((GROUPS, CONTEXT_ROWS, 2, HEADS, HEAD_DIM), generator=g, device=dev, dtype=torch.float16)
    cache = BlockwiseSeqKV.from_row_slices(
        (kv[:, a : a + block_rows] for a in range(0, CONTEXT_ROWS, block_rows)), 1, GROUPS, quantize=True,
        device=dev, dtype=kv.dtype, offload=True,
    )
    del kv
    q = torch.randn((GROUPS, QUERY_ROWS, HEADS, HEAD_DIM), generator=g, device=dev, dtype=torch.float16)
    host_bytes = cache.host_bytes()

    def serialized():
        out = torch.zeros((GROUPS, QUERY_ROWS, HEADS, HEAD_DIM), dtype=torch.float32, device=dev)
        lse = torch.full((GROUPS, HEADS, QUERY_ROWS), float("-inf"), dtype=torch.float32, device=dev)
        for payload, scales in cache.iter_payload_blocks():
            nori_amd.icl_attention(q, payload, scales, out=out, lse=lse, merge=True)
        return out

    def overlapped():
        return attn.compute_attention_blockwise(q, cache)

    results = {}
    for name, fn in (("serialized", serialized), ("overlapped", overlapped)):
        fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            fn()
        torch.cuda.synchronize()
        sec = (time.perf_counter() - t0) / args.steps
        results[name] = {
            "ms_per_query_batch": round(sec * 1e3, 3),
            "query_rows_per_s": round(QUERY_ROWS / sec, 1),
            "h2d_GBps": round(host_bytes / sec / 1e9, 2),
        }
    print(json.dumps({
        "streamed": {
            "workload": f"one nori-30m layer, {CONTEXT_ROWS}-row int8 context in pinned host blocks of {block_rows} "
            f"rows, {QUERY_ROWS} query rows x {GROUPS} token groups x {HEADS} heads",
            "host_bytes_per_query_batch": host_bytes,
            **results,
        }
    }), flush=True)


def build_workload(torch, layers, dev):
    g = torch.Generator(device=dev).manual_seed(2)
    kv_shape = (GROUPS, CONTEXT_ROWS, 2, HEADS, HEAD_DIM)
    kv = [torch.randn(kv_shape, generator=g, device=dev, dtype=torch.float16) for _ in range(layers)]
    codes = [torch.empty(kv_shape, dtype=torch.int8, device=dev) for _ in range(layers)]
    scales = [torch.empty(kv_shape[:-1] + (1,), dtype=torch.float32, device=dev) for _ in range(layers)]
    wq = [(torch.randn(HEADS * HEAD_DIM, EMBED, generator=g, device=dev) * EMBED ** -0.5).half() for _ in range(layers)]
    wo = [(torch.randn(HEADS, HEAD_DIM, EMBED, generator=g, device=dev) * 0.02).half() for _ in range(layers)]
    queries = [torch.randn(GROUPS, QUERY_ROWS, EMBED, generator=g, device=dev, dtype=torch.float16) for _ in range(QUERY_BATCHES)]
    return kv, codes, scales, wq, wo, queries


def cache_write(torch, dev, codes, scales, reps=5):
    """One layer's cross-cache write at this workload, from the layer's fp32 context rows
    [1, 65536, 33, 352]: the fused path (nori_amd.project_quantize_kv: one pass from the fp32
    rows, or the operand-row pass + projection/quantizer kernel where the one pass does not
    apply) against the unfused one it replaces (HIP RMSNorm, torch's
    fp16-autocast F.linear, HIP quantizer), each timed with HIP events on the launch stream.
    Both write `codes` / `scales` [33, 65536, 2, 8, 44]."""
    import nori_amd
    from nori_amd.kv_cache_scaling import _quantize_into

    g = torch.Generator(device=dev).manual_seed(3)
    x = torch.randn(1, CONTEXT_ROWS, GROUPS, EMBED, generator=g, device=dev)
    w = torch.randn(2 * HEADS * HEAD_DIM, EMBED, generator=g, device=dev) * EMBED ** -0.5
    xt = x.transpose(1, 2)
    out = (codes.view(1, GROUPS, CONTEXT_ROWS, 2, HEADS, HEAD_DIM), scales.view(1, GROUPS, CONTEXT_ROWS, 2, HEADS, 1))
    stream = torch.cuda.current_stream(dev)

    def fused():
        nori_amd.project_quantize_kv(xt, w, HEADS, HEAD_DIM, norm_eps=1e-5, out=out)

    def unfused():
        xn = nori_amd.rms_norm(x, EMBED, None, 1e-5)
        with torch.autocast("cuda", dtype=torch.float16):
            kv = torch.nn.functional.linear(xn.transpose(1, 2).reshape(GROUPS, CONTEXT_ROWS, EMBED), w)
        _quantize_into(kv.view(GROUPS, CONTEXT_ROWS, 2, HEADS, HEAD_DIM), codes, scales)

    def avg_ms(fn):
        fn()
        ev = []
        for _ in range(reps):
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            fn()
            e1.record(stream)
            ev.append((e0, e1))
        torch.cuda.synchronize()
        return sum(a.elapsed_time(b) for a, b in ev) / reps

    fused_ms, unfused_ms = avg_ms(fused), avg_ms(unfused)
    rows = GROUPS * CONTEXT_ROWS
    n_kv = rows * 2 * HEADS * HEAD_DIM
    # one pass (no workspace) from the fp32 rows, or the operand-row pass + projection kernel
    one_pass = nori_amd._native.lib().nori_kv_project_quantize_int8_workspace_bytes(
        nori_amd._native.dtype_code(torch.float32), GROUPS, CONTEXT_ROWS, EMBED, 1,
        nori_amd._native.dtype_code(torch.float16), HEAD_DIM) == 0
    # algorithmic HBM bytes: x read, codes + scales written (and for the two-kernel path the
    # f16 operand rows written and read)
    fused_bytes = rows * EMBED * 4 + n_kv + 4 * rows * 2 * HEADS + (0 if one_pass else 2 * rows * EMBED * 2)
    del x, xt
    return {
        "what": "one layer's int8 cross-cache write from fp32 context rows: RMSNorm -> K/V projection "
        "(fp16 operands, fp32 sums) -> exact int8 quantizer, 33 x 65536 rows, embed 352 -> 2 x 8 x 44",
        "fused_path": "one pass from the fp32 rows (kv_rows_kernel)" if one_pass
        else "operand-row pass + projection/quantizer kernel",
        "fused_ms": round(fused_ms, 4),
        "unfused_ms": round(unfused_ms, 4),
        "speedup": round(unfused_ms / fused_ms, 3),
        "fused_algorithmic_bytes": fused_bytes,
        "fused_GBps": round(fused_bytes / fused_ms / 1e6, 1),
        "fused_TFLOPs": round(2.0 * rows * EMBED * 2 * HEADS * HEAD_DIM / fused_ms / 1e9, 1),
    }


def mfma_ceiling(torch, dev, codes, scales, att_flop, iters=4096, reps=3):
    """The dense f16 MFMA rate the GPU sustains under its power limit, on random and on all-zero
    operands (nori_mfma_f16_probe: nothing but v_mfma_f32_32x32x16_f16, four wavefronts per SIMD),
    and the workload's attention launch over its real int8 cache against the same launch over an
    all-zero cache: the kernel's time depends on its data the way the MFMA rate does."""
    import ctypes

    import nori_amd
    from nori_amd import _native as nat

    g = torch.Generator(device=dev).manual_seed(11)
    n_vec = 1 << 20  # 16-byte vectors of f16 pairs: sign and mantissa random, |v| in [0.25, 4)
    mant = torch.randint(0, 1 << 10, (n_vec * 8,), generator=g, device=dev, dtype=torch.int32)
    expo = torch.randint(13, 16, (n_vec * 8,), generator=g, device=dev, dtype=torch.int32)
    sign = torch.randint(0, 2, (n_vec * 8,), generator=g, device=dev, dtype=torch.int32)
    rnd = ((sign << 15) | (expo << 10) | mant).to(torch.int16)
    zero = torch.zeros_like(rnd)
    sink = torch.empty(1 << 20, dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream(dev)
    lib = nat.lib()
    flop = lib.nori_mfma_f16_probe_flop(iters)

    def probe_rate(ops):
        def call():
            nat.check(lib.nori_mfma_f16_probe(ctypes.c_void_p(ops.data_ptr()), n_vec, iters,
                                              ctypes.c_void_p(sink.data_ptr()), sink.numel(),
                                              nat.stream_of(dev)), "mfma_f16_probe")
        call()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            call()
        e1.record(stream)
        torch.cuda.synchronize()
        return flop * reps / (e0.elapsed_time(e1) / 1e3)

    rate_rnd, rate_zero = probe_rate(rnd), probe_rate(zero)
    q = torch.randn((GROUPS, QUERY_ROWS, HEADS, HEAD_DIM), generator=g, device=dev, dtype=torch.float16)
    out = torch.empty_like(q)
    ws = torch.empty(max(nori_amd.attention.workspace_bytes(GROUPS, QUERY_ROWS, HEADS, HEAD_DIM, CONTEXT_ROWS), 1),
                     dtype=torch.uint8, device=dev)

    def attn_ms(c):
        nori_amd.icl_attention(q, c, scales, out=out, workspace=ws)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(10):
            nori_amd.icl_attention(q, c, scales, out=out, workspace=ws)
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / 10

    ms_real, ms_zero = attn_ms(codes), attn_ms(torch.zeros_like(codes))
    return {
        "what": "dense f16 MFMA rate under the power limit (v_mfma_f32_32x32x16_f16 only, 4 wavefronts per SIMD, "
        "8 operand register sets per wavefront) on random operands (|v| in [0.25, 4), random sign and mantissa) "
        "and on all-zero operands; the bench's attention launch on its N(0,1) int8 cache and on an all-zero cache",
        "mfma_f16_random_TFLOPs": round(rate_rnd / 1e12, 1),
        "mfma_f16_zero_TFLOPs": round(rate_zero / 1e12, 1),
        "random_frac_of_peak": round(rate_rnd / MFMA_BF16_PEAK, 4),
        "attention_ms_real_cache": round(ms_real, 4),
        "attention_ms_zero_cache": round(ms_zero, 4),
        "attention_frac_of_random_ceiling": round(att_flop / (ms_real / 1e3) / rate_rnd, 4),
    }


def prefill_attention(torch, dev, kv16, reps=2):
    """The context self-attention of one layer's prefill (layer.py:1884-1888): all 65,536 context
    rows attend to the layer's full-precision (fp16) context K/V [33, 65536, 2, 8, 44] with the
    fp16-cache variant of the attention kernel. HIP events around each call."""
    import nori_amd
    from nori_amd import attention as attn

    g = torch.Generator(device=dev).manual_seed(4)
    q = torch.randn(GROUPS, CONTEXT_ROWS, HEADS, HEAD_DIM, generator=g, device=dev, dtype=torch.float16)
    out = torch.empty_like(q)
    ws = torch.empty(max(attn.workspace_bytes(GROUPS, CONTEXT_ROWS, HEADS, HEAD_DIM, CONTEXT_ROWS), 1),
                     dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream(dev)
    nori_amd.icl_attention(q, kv16, out=out, workspace=ws)
    ev = []
    for _ in range(reps):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        nori_amd.icl_attention(q, kv16, out=out, workspace=ws)
        e1.record(stream)
        ev.append((e0, e1))
    torch.cuda.synchronize()
    ms = sum(a.elapsed_time(b) for a, b in ev) / reps
    flop = 4.0 * GROUPS * HEADS * CONTEXT_ROWS * CONTEXT_ROWS * HEAD_DIM
    del q, out, ws
    return {
        "what": "one layer's prefill self-attention: 33 x 65536 context rows x 8 heads attending to "
        "the layer's fp16 context K/V (65536 rows), icl_attention_kernel<48, f16 cache, fold, 16 waves>",
        "avg_launch_ms": round(ms, 3),
        "achieved": round(flop / (ms * 1e-3) / 1e12, 1),
        "unit": "TFLOP/s",
        "frac": round(flop / (ms * 1e-3) / MFMA_BF16_PEAK, 4),
        "work_per_launch": f"{flop:.4e} FLOP = 4*33*8*65536*65536*44",
    }


def model_config(layers=LAYERS, embed=EMBED, heads=HEADS, hid=4 * EMBED, quantiles=(0.1, 0.5, 0.9), rbf=(8, 16)):
    """A random-init model at the given block dims (by default this workload's: 12 layers, embed
    352, 8 heads; 2 features per group, SwiGLU, RMSNorm pre-norm, QASS, target-aware
    embedding), with the encoders of the reference's configuration files."""
    return dict(
        preprocess_config_x=dict(
            num_features=2, nan_handling_enabled=True, normalize_on_train_only=True, normalize_x=True,
            remove_outliers=True, normalize_by_used_features=True,
        ),
        encoder_config_x=dict(
            num_features=2, embedding_size=embed, mask_embedding_size=embed, encoder_use_bias=True,
            numeric_embed_type="RBF",
            RBF_config=dict(token_embed_dim=rbf[0], n_kernels=rbf[1], sigma=0.5, use_learn_sigma=False,
                            use_learn_embeddings=False, use_original_features=False),
        ),
        encoder_config_y=dict(num_inputs=1, embedding_size=embed, nan_handling_y_encoder=True, max_num_classes=10),
        decoder_config=dict(num_classes=10, num_reg_quantiles=len(quantiles), regression_loss="pinball",
                            regression_quantiles=list(quantiles)),
        nlayers=layers, nhead=heads, embed_dim=embed, hid_dim=hid,
        features_per_group=2, dropout=0.0,
        pre_norm=True, activation="swiglu", norm_type="rmsnorm", deepnorm_alpha=layers ** -0.5, layer_arch="smf",
        feature_positional_embedding_type="none", seq_attn_isolated=True, cross_share_all_kv_heads=False,
        use_qassmax=True, qass_mode="full", use_target_aware_embedding=True, use_column_specific_y_aware=True,
    )


def end_to_end(torch, dev, batches=QUERY_BATCHES):
    """The long-context configuration through the model-level context-cache API: a 65,536-row
    context of 64 float32 features (5 % NaN) with a nonlinear target, cached once as int8
    (FeaturesTransformer.build_context_cache), then 4 query batches of 1,024 rows
    (apply_context_cache), under the fp16 autocast of GPU inference. Wall clock around each
    phase with the device synchronized."""
    import nori_amd

    g = torch.Generator().manual_seed(7)
    n_feat = 64
    x = torch.randn(1, CONTEXT_ROWS + batches * QUERY_ROWS, n_feat, generator=g)
    x[torch.rand(x.shape, generator=g) < 0.05] = float("nan")
    xf = torch.nan_to_num(x)
    pair = xf[..., 0::2] * xf[..., 1::2]
    y = pair.sum(-1) / n_feat ** 0.5 + 0.1 * torch.randn(x.shape[:2], generator=g)
    x, y = x.to(dev), y.to(dev)
    model = nori_amd.FeaturesTransformer(**model_config()).eval().to(dev)
    with torch.inference_mode(), torch.autocast("cuda", dtype=torch.float16):
        # both build paths once on 1024 rows (library and kernel set-up out of the timed builds);
        # then the opt-in fused cache write (projection + quantizer in one kernel), timed and
        # freed; then the default build, whose int8 codes are bit-exact to the reference
        # expression, which the query batches use
        for fused in (True, False):
            warm = model.build_context_cache(x[:, :1024], y[:, :1024], cache_dtype="int8", fused_cache_write=fused)
            del warm
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ctx = model.build_context_cache(x[:, :CONTEXT_ROWS], y[:, :CONTEXT_ROWS], cache_dtype="int8",
                                        fused_cache_write=True)
        torch.cuda.synchronize()
        t_build_fused = time.perf_counter() - t0
        del ctx
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ctx = model.build_context_cache(x[:, :CONTEXT_ROWS], y[:, :CONTEXT_ROWS], cache_dtype="int8")
        torch.cuda.synchronize()
        t_build = time.perf_counter() - t0
        # one warm batch, then the timed batches
        model.apply_context_cache(x[:, CONTEXT_ROWS:CONTEXT_ROWS + QUERY_ROWS], ctx, row_chunk_size=QUERY_ROWS)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(batches):
            lo = CONTEXT_ROWS + i * QUERY_ROWS
            pred = model.apply_context_cache(x[:, lo:lo + QUERY_ROWS], ctx, row_chunk_size=QUERY_ROWS)
        torch.cuda.synchronize()
        t_apply = time.perf_counter() - t0
    finite = bool(torch.isfinite(pred).all())
    del ctx, model, x, y
    return {
        "what": "model-level context-cache API at this workload: random-init 12-layer embed-352 model, "
        "65536-row context of 64 features (5 % NaN) cached once as int8, 4 query batches of 1024 rows, "
        "fp16 autocast; build_context_cache_s is the default build (library GEMM, then the exact quantizer: "
        "codes bit-exact to the reference expression), build_context_cache_fused_write_s the opt-in fused "
        "cache write",
        "build_context_cache_s": round(t_build, 3),
        "build_context_cache_fused_write_s": round(t_build_fused, 3),
        "apply_query_rows_per_s": round(batches * QUERY_ROWS / t_apply, 1),
        "apply_ms_per_batch": round(t_apply * 1e3 / batches, 2),
        "predictions_finite": finite,
    }


# The batched configuration at nori-100m block dims (assumed: 16 layers, embed 560, 10 heads of
# 56, hidden 1680): 32 tables of 8192 context + 2048 query rows and 100 features, 80 Gaussian
# and 20 categorical codes; the tables go through the context-cache API 8 at a time (the
# 16-layer int8 cache of all 32 tables is about 257 GB, beside the build's transients).
CONFIG4 = dict(tables=32, context=8192, queries=2048, numeric=80, categorical=20, sub_batch=8)


def config4_table(np):
    """Config 4's synthetic tables (numpy default_rng(3)): per table, 80 N(0, 1) features and 20
    categorical columns with k ~ U{2..50} levels each and uniform codes (as floats, after the
    numeric ones); y = X_num a + t_3 with a ~ N(0, 1/80) and Student-t noise of 3 degrees of
    freedom."""
    c = CONFIG4
    rng = np.random.default_rng(3)
    rows = c["context"] + c["queries"]
    xn = rng.standard_normal((c["tables"], rows, c["numeric"])).astype(np.float32)
    levels = rng.integers(2, 51, size=(c["tables"], 1, c["categorical"]))
    xc = np.floor(rng.random((c["tables"], rows, c["categorical"])) * levels).astype(np.float32)
    a = rng.normal(0.0, c["numeric"] ** -0.5, size=(c["tables"], c["numeric"], 1))
    y = (xn.astype(np.float64) @ a)[..., 0] + rng.standard_t(3, size=(c["tables"], rows))
    return np.concatenate([xn, xc], axis=-1), y.astype(np.float32)


def config4_model(torch, dev):
    """Config 4 end to end through the model-level context-cache API: a random-init model at
    nori-100m block dims with the 999-level quantile head, 32 tables built and applied 8 at a
    time (build_context_cache(cache_dtype="int8"), then apply_context_cache over the tables'
    2048 query rows in chunks of 1024), under fp16 autocast; the point prediction is the
    quantile bank's trapezoid mean. Wall clock with the device synchronized, after one warm
    sub-batch of a single 1024-row table."""
    import numpy as np

    import nori_amd
    from nori_amd.api import quantile_dist_mean

    c = CONFIG4
    levels = [(i + 1) / 1000.0 for i in range(999)]
    x_np, y_np = config4_table(np)
    x, y = torch.from_numpy(x_np).to(dev), torch.from_numpy(y_np).to(dev)
    torch.manual_seed(3)
    model = nori_amd.FeaturesTransformer(**model_config(layers=16, embed=560, heads=10, hid=1680, quantiles=levels,
                                                        rbf=(16, 64))).eval().to(dev)
    params = sum(p.numel() for p in model.parameters())
    tau = torch.tensor(levels, device=dev)
    n_ctx, tb = c["context"], c["sub_batch"]
    with torch.inference_mode(), torch.autocast("cuda", dtype=torch.float16):
        warm = model.build_context_cache(x[:1, :1024], y[:1, :1024], cache_dtype="int8")
        model.apply_context_cache(x[:1, n_ctx:n_ctx + 256], warm, row_chunk_size=256)
        del warm
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats(dev)
        t_build = t_apply = 0.0
        points = []
        for t0 in range(0, c["tables"], tb):
            torch.cuda.synchronize()
            s0 = time.perf_counter()
            ctx = model.build_context_cache(x[t0:t0 + tb, :n_ctx], y[t0:t0 + tb, :n_ctx], cache_dtype="int8")
            torch.cuda.synchronize()
            s1 = time.perf_counter()
            bank = model.apply_context_cache(x[t0:t0 + tb, n_ctx:], ctx, row_chunk_size=1024)
            points.append(quantile_dist_mean(bank, tau))
            torch.cuda.synchronize()
            s2 = time.perf_counter()
            t_build += s1 - s0
            t_apply += s2 - s1
            del ctx, bank
            print(f"config 4: tables {t0}-{t0 + tb - 1} built in {s1 - s0:.2f} s, applied in {s2 - s1:.2f} s",
                  file=sys.stderr, flush=True)
    pred = torch.cat(points)
    finite = bool(torch.isfinite(pred).all())
    peak = torch.cuda.max_memory_allocated(dev)
    del model, x, y, pred, points
    q_rows = c["tables"] * c["queries"]
    return {
        "what": "config 4 end to end: random-init nori-100m-dims model (16 layers, embed 560, 10 heads of 56, "
        f"hidden 1680, 999 quantiles; {params / 1e6:.1f} M parameters), 32 tables x (8192 context + 2048 query rows) "
        "x 100 features (80 Gaussian, 20 categorical codes with 2-50 levels), Student-t (df 3) target; "
        "int8 context cache built and applied 8 tables at a time, fp16 autocast, point prediction by the "
        "quantile bank's trapezoid mean",
        "total_s": round(t_build + t_apply, 3),
        "build_context_cache_s": round(t_build, 3),
        "apply_s": round(t_apply, 3),
        "query_rows_per_s": round(q_rows / (t_build + t_apply), 1),
        "apply_query_rows_per_s": round(q_rows / t_apply, 1),
        "tables_per_s": round(c["tables"] / (t_build + t_apply), 3),
        "peak_allocated_gb": round(peak / 2 ** 30, 1),
        "predictions_finite": finite,
    }


# A random-init two-phase model of about Nori 1.5's size (20.8 M parameters; its dims are not in
# the reference's sources): 128-wide cells with 2 heads of 64, 12 cell layers, 2 target tokens,
# 6 row layers of width 256 with 4 heads of 64, PLE cells of 32 bins, 999 quantiles.
SMALL_TABLES = dict(tables=512, context=256, queries=64, features=8, reps=5)


def two_phase_config():
    return dict(
        preprocess_config_x=dict(
            num_features=2, nan_handling_enabled=True, normalize_on_train_only=True, normalize_x=True,
            remove_outliers=False, normalize_by_used_features=True, prompt_quantile_ple_bins=32,
        ),
        encoder_config_x=dict(
            num_features=2, embedding_size=128, mask_embedding_size=128, encoder_use_bias=True, numeric_embed_type="RBF",
            RBF_config=dict(token_embed_dim=8, n_kernels=16, sigma=0.5, use_learn_sigma=False,
                            use_learn_embeddings=False, use_original_features=False),
            prompt_quantile_ple_bins=32,
        ),
        encoder_config_y=dict(num_inputs=1, embedding_size=128, nan_handling_y_encoder=True, max_num_classes=10),
        decoder_config=dict(num_reg_quantiles=999, regression_loss="pinball"),
        nlayers=12, nhead=2, embed_dim=128, hid_dim=384, features_per_group=2, dropout=0.0, pre_norm=True,
        activation="swiglu", norm_type="rmsnorm", deepnorm_alpha=18 ** -0.5, feature_positional_embedding_type="subortho",
        use_target_aware_embedding=True, use_column_specific_y_aware=True, use_qassmax=True, qass_mode="log_only",
        omit_feature_decoder=True, two_phase_config=dict(target_tokens=2, row_layers=6, row_heads=4, row_hidden_dim=1024),
    )


def small_tables(torch, dev):
    """The many-small-tables path: 512 independent tables of 256 context + 64 query rows x 8
    float32 features X ~ U(-3, 3), y a random degree-2 polynomial of X + 0.05 N(0, 1), through
    the two-phase model's forward (context and query rows together, as Nori 1.5 runs it) under
    the fp16 autocast of GPU inference; quantiles 0.05 / 0.5 / 0.95 taken from the 999-level
    head. Wall clock over `reps` forwards with the device synchronized, after one warm-up."""
    import nori_amd

    c = SMALL_TABLES
    g = torch.Generator().manual_seed(4)
    rows = c["context"] + c["queries"]
    x = torch.rand(c["tables"], rows, c["features"], generator=g) * 6.0 - 3.0
    quad = torch.randn(c["tables"], c["features"], c["features"], generator=g) / c["features"]
    lin = torch.randn(c["tables"], c["features"], generator=g) / c["features"] ** 0.5
    y = torch.einsum("bnf,bfg,bng->bn", x, quad, x) + (x * lin[:, None]).sum(-1)
    y = y + 0.05 * torch.randn(y.shape, generator=g)
    x, y = x.to(dev), y[:, : c["context"]].to(dev)
    model = nori_amd.FeaturesTransformer(**two_phase_config()).eval().to(dev)
    n_params = sum(p.numel() for p in model.parameters())
    pick = torch.tensor([49, 499, 949], device=dev)  # levels 0.05, 0.5, 0.95 of (i + 1) / 1000

    def forward():
        return model(x=x, y=y, eval_pos=c["context"], task_type="reg").index_select(-1, pick)

    with torch.inference_mode(), torch.autocast("cuda", dtype=torch.float16):
        out = forward()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(c["reps"]):
            out = forward()
        torch.cuda.synchronize()
        dt = (time.perf_counter() - t0) / c["reps"]
    assert out.shape == (c["tables"], c["queries"], 3) and bool(torch.isfinite(out).all())
    return {
        "what": "config 5: many small tables, a nori-1-5-shaped two-phase model "
        f"({n_params / 1e6:.1f} M parameters, random init): {c['tables']} tables x ({c['context']} context + "
        f"{c['queries']} query rows) x {c['features']} features, fp16 autocast, quantiles 0.05/0.5/0.95",
        "ms_per_forward": round(dt * 1e3, 3),
        "query_rows_per_s": round(c["tables"] * c["queries"] / dt, 1),
        "tables_per_s": round(c["tables"] / dt, 1),
    }


def other_configs(torch, dev):
    """Kernel-level legs of the other cached configurations, each timed with HIP events:
    config 2, the isolated ICL block at nori-6m dims (1 table, G = 9 tokens, 4096 context rows,
    1024 queries, H = 2, D = 64, bf16 with 3 channels x8), and config 4, one layer of the batched
    pipeline at nori-100m dims (32 tables x G = 51 tokens, 8192 context rows, 2048 queries,
    H = 10, D = 56, fp16). Quantize and attention separately."""
    import nori_amd
    from nori_amd import attention as attn
    from nori_amd.kv_cache_scaling import _quantize_into

    stream = torch.cuda.current_stream(dev)

    def avg_ms(fn, reps):
        fn()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    def leg(name, bg, nk, nq, heads, d, dtype, reps_q, reps_a, outliers):
        g = torch.Generator(device=dev).manual_seed(1)
        kv = torch.randn(bg, nk, 2, heads, d, generator=g, device=dev, dtype=dtype)
        q = torch.randn(bg, nq, heads, d, generator=g, device=dev, dtype=dtype)
        if outliers:
            ch = torch.randperm(heads * d, generator=torch.Generator().manual_seed(1))[:outliers]
            kv.view(bg, nk, 2, heads * d)[..., ch] *= 8
            q.view(bg, nq, heads * d)[..., ch] *= 8
        codes = torch.empty(kv.shape, dtype=torch.int8, device=dev)
        scales = torch.empty(kv.shape[:-1] + (1,), dtype=torch.float32, device=dev)
        ws = torch.empty(max(attn.workspace_bytes(bg, nq, heads, d, nk), 1), dtype=torch.uint8, device=dev)
        out = torch.empty_like(q)
        q_ms = avg_ms(lambda: _quantize_into(kv, codes, scales), reps_q)
        a_ms = avg_ms(lambda: nori_amd.icl_attention(q, codes, scales, out=out, workspace=ws), reps_a)
        n = kv.numel()
        qbytes = n * (kv.element_size() + 1) + 4 * n // d
        flop = 4.0 * bg * heads * nq * nk * d
        return {
            "what": name,
            "quantize_ms": round(q_ms, 4),
            "quantize_GBps": round(qbytes / (q_ms * 1e-3) / 1e9, 1),
            "quantize_frac": round(qbytes / (q_ms * 1e-3) / HBM_PEAK, 4),
            "attention_ms": round(a_ms, 4),
            "attention_TFLOPs": round(flop / (a_ms * 1e-3) / 1e12, 1),
            "attention_frac": round(flop / (a_ms * 1e-3) / MFMA_BF16_PEAK, 4),
        }

    c2 = leg("config 2: isolated ICL block, nori-6m dims: BG 9, 4096 context rows, 1024 queries, H 2, D 64, "
             "bf16 with 3 channels x8", 9, 4096, 1024, 2, 64, torch.bfloat16, 200, 50, 3)
    c4 = leg("config 4: one layer of the batched pipeline, nori-100m dims: BG 32 x 51, 8192 context rows, "
             "2048 queries, H 10, D 56, fp16", 32 * 51, 8192, 2048, 10, 56, torch.float16, 3, 2, 0)
    return {"config2": c2, "config4": c4}


def measured_traffic():
    """HBM bytes per launch of the attention and quantize kernels from the committed
    rocprofv3 FETCH_SIZE/WRITE_SIZE summary (scaled by the copy-kernel calibration), or None."""
    try:
        text = open(TRAFFIC_SUMMARY).read()
    except OSError:
        return None, None, None
    found = {}
    for name in ("attention", "quantize", "dequantize"):
        m = re.search(rf"^traffic_bytes_{name}\s*=\s*([0-9.eE+]+)", text, re.M)
        found[name] = float(m.group(1)) if m else None
    return found["attention"], found["quantize"], found["dequantize"]


def main():
    args = parse_args()
    if args.gpus != 1:
        print(
            "bench.py measures one MI355X: the Nori ICL path shards by table/token group or by "
            "context rows without changing the per-GPU kernel, and this build runs on a single GPU. "
            "Run with --gpus 1.",
            file=sys.stderr,
        )
        sys.exit(2)
    import torch

    import nori_amd
    from nori_amd import attention as attn
    from nori_amd.kv_cache_scaling import _dequantize_into, _quantize_into

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if args.probe_traffic:
        probe_traffic(torch, dev)
        return
    if args.other_configs:
        print(json.dumps(other_configs(torch, dev)), flush=True)
        return
    if args.model:
        print(json.dumps(end_to_end(torch, dev)), flush=True)
        return
    if args.config4:
        print(json.dumps(config4_model(torch, dev)), flush=True)
        return
    if args.small_tables:
        print(json.dumps(small_tables(torch, dev)), flush=True)
        return
    if args.config1:
        print(json.dumps(config1(torch, dev)), flush=True)
        return
    if args.prefill:
        shape = (GROUPS, CONTEXT_ROWS, 2, HEADS, HEAD_DIM)
        kv16 = torch.randn(shape, generator=torch.Generator(device=dev).manual_seed(2), device=dev, dtype=torch.float16)
        print(json.dumps(prefill_attention(torch, dev, kv16)), flush=True)
        return
    if args.mfma_ceiling:
        shape = (GROUPS, CONTEXT_ROWS, 2, HEADS, HEAD_DIM)
        kv16 = torch.randn(shape, generator=torch.Generator(device=dev).manual_seed(2), device=dev, dtype=torch.float16)
        codes = torch.empty(shape, dtype=torch.int8, device=dev)
        scales = torch.empty(shape[:-1] + (1,), dtype=torch.float32, device=dev)
        _quantize_into(kv16, codes, scales)
        del kv16
        print(json.dumps(mfma_ceiling(torch, dev, codes, scales,
                                      4.0 * GROUPS * HEADS * QUERY_ROWS * CONTEXT_ROWS * HEAD_DIM)), flush=True)
        return
    if args.cache_write:
        shape = (GROUPS, CONTEXT_ROWS, 2, HEADS, HEAD_DIM)
        codes = torch.empty(shape, dtype=torch.int8, device=dev)
        scales = torch.empty(shape[:-1] + (1,), dtype=torch.float32, device=dev)
        print(json.dumps(cache_write(torch, dev, codes, scales)), flush=True)
        return
    if args.streamed:
        streamed(torch, dev, args)
        return
    layers = args.layers
    kv, codes, scales, wq, wo, queries = build_workload(torch, layers, dev)
    ws_bytes = attn.workspace_bytes(GROUPS, QUERY_ROWS, HEADS, HEAD_DIM, CONTEXT_ROWS)
    workspace = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream(dev)

    def timed(fn, sink, on=None):
        on = stream if on is None else on
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(on)
        r = fn()
        e1.record(on)
        sink.append((e0, e1))
        return r

    # Streams (all at the default priority). The cache build runs on `side`, and each layer's
    # attentions wait only for that layer's codes: the HBM-bound quantizations of layers 1..11
    # overlap the MFMA-bound attention of the layers before them. The query batches, which are
    # independent, run on a stream each; their attentions stay one at a time (each waits for
    # the previous one, so every timed launch has the GPU to itself and they share the
    # workspace), while the other batches' norms, projections and residual adds fill the gaps.
    side = torch.cuda.Stream(dev)
    bstreams = [stream] + [torch.cuda.Stream(dev) for _ in range(len(queries) - 1)]

    def step(record):
        qsink, asink = ([], []) if record else (None, None)
        for s_ in [side] + bstreams[1:]:
            s_.wait_stream(stream)  # inputs written; the previous step's attention has read the codes
        ready = []
        with torch.cuda.stream(side):
            for layer in range(layers):
                _quantize_into(kv[layer], codes[layer], scales[layer])
                ev = torch.cuda.Event()
                ev.record(side)
                ready.append(ev)
        xs = list(queries)
        last = None
        for layer in range(layers):
            for bi, st in enumerate(bstreams):
                with torch.cuda.stream(st):
                    st.wait_event(ready[layer])
                    xn = nori_amd.rms_norm(xs[bi], EMBED, None, 1e-5)
                    q = torch.nn.functional.linear(xn, wq[layer]).view(GROUPS, QUERY_ROWS, HEADS, HEAD_DIM)
                    if last is not None:
                        st.wait_event(last)
                    f = lambda q=q, layer=layer: nori_amd.icl_attention(q, codes[layer], scales[layer], workspace=workspace)  # noqa: E731
                    o = timed(f, asink, st) if record else f()
                    last = torch.cuda.Event()
                    last.record(st)
                    xs[bi] = xs[bi] + DEEPNORM_ALPHA * torch.einsum("...hd,hds->...s", o, wo[layer])
        for s_ in [side] + bstreams[1:]:
            stream.wait_stream(s_)
        return xs, qsink, asink

    for _ in range(args.warmup):
        step(False)
    torch.cuda.synchronize()
    events_q, events_a = [], []
    t0 = time.perf_counter()
    for _ in range(args.steps):
        _, qs, as_ = step(True)
        events_q += qs
        events_a += as_
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    attn_ms = [a.elapsed_time(b) for a, b in events_a]
    # the quantizer's roofline from launches of its own (in the step it shares the GPU with
    # the attention): each layer once, HIP events around each launch
    q_events = []
    for layer in range(layers):
        f = lambda layer=layer: _quantize_into(kv[layer], codes[layer], scales[layer])  # noqa: E731
        timed(f, q_events)
    torch.cuda.synchronize()
    quant_ms = [a.elapsed_time(b) for a, b in q_events]

    # dequantization (the full-precision read of a ScalableSeqKV, kv_cache_scaling.py:40-41,
    # 78-90) is not on the step's path -- attention reads the codes -- so it is timed on its
    # own, outside the step: one layer's cache back to fp16, HIP events around each launch
    dq_out = torch.empty_like(kv[0])
    dq_events = []
    for i in range(6):
        f = lambda: _dequantize_into(codes[0], scales[0], dq_out)  # noqa: E731
        timed(f, dq_events) if i else f()
    torch.cuda.synchronize()
    dequant_ms = [a.elapsed_time(b) for a, b in dq_events]
    del dq_out
    ceiling = mfma_ceiling(torch, dev, codes[0], scales[0],
                           4.0 * GROUPS * HEADS * QUERY_ROWS * CONTEXT_ROWS * HEAD_DIM)
    write = cache_write(torch, dev, codes[0], scales[0])
    prefill = prefill_attention(torch, dev, kv[0])
    model_e2e = end_to_end(torch, dev)
    kv0 = [kv[0]]
    del kv
    others = other_configs(torch, dev)
    c4 = config4_model(torch, dev)
    tables = small_tables(torch, dev)
    norm_leg = rmsnorm_leg(torch, dev)
    c1 = config1(torch, dev)

    rows_per_step = QUERY_BATCHES * QUERY_ROWS
    ms_per_step = elapsed * 1e3 / args.steps
    value = rows_per_step * args.steps / elapsed

    attn_flop = 4.0 * GROUPS * HEADS * QUERY_ROWS * CONTEXT_ROWS * HEAD_DIM  # per launch, unpadded D
    attn_avg_s = sum(attn_ms) / len(attn_ms) / 1e3
    attn_achieved = attn_flop / attn_avg_s
    n_elem = GROUPS * CONTEXT_ROWS * 2 * HEADS * HEAD_DIM
    quant_bytes = n_elem * (2 + 1) + 4 * n_elem // HEAD_DIM  # fp16 in, int8 + fp32 scale out
    quant_avg_s = sum(quant_ms) / len(quant_ms) / 1e3
    quant_achieved = quant_bytes / quant_avg_s
    dequant_avg_s = sum(dequant_ms) / len(dequant_ms) / 1e3
    dequant_achieved = quant_bytes / dequant_avg_s  # int8 + fp32 scale in, fp16 out: the same bytes
    attn_traffic, quant_traffic, dequant_traffic = measured_traffic()

    line = {
        "metric": "query rows/s @ 64k-row int8 ctx; attn % MFMA peak; quant kernel % HBM BW",
        "value": round(value, 2),
        "unit": "query rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 MFMA (int8 K/V codes, fp32 softmax/accumulate)",
        "data": "synthetic: random-init nori-30m block weights, N(0,1) fp16 context K/V and query tokens",
        "config": {
            "workload": "nori-30m ICL stage: int8 cache build for 12 layers over a 65536-row context "
            "+ 4 query batches x 1024 rows x 12 cached attention sublayers",
            "layers": layers, "embed": EMBED, "heads": HEADS, "head_dim": HEAD_DIM,
            "token_groups": GROUPS, "context_rows": CONTEXT_ROWS,
            "query_rows_per_step": rows_per_step, "cache": "int8 per-vector absmax (resident)",
        },
        "roofline": {
            "kernel": "icl_attention_kernel<48, int8, fold, 16 waves> (+ combine_splits_kernel)",
            "bound": "mfma",
            "achieved": round(attn_achieved / 1e12, 2),
            "peak": MFMA_BF16_PEAK / 1e12,
            "unit": "TFLOP/s",
            "frac": round(attn_achieved / MFMA_BF16_PEAK, 4),
            "traffic": attn_traffic,
            "work_per_launch": f"{attn_flop:.4e} FLOP = 4*33*8*1024*65536*44",
            "avg_launch_ms": round(attn_avg_s * 1e3, 4),
            "launches": len(attn_ms),
        },
        "quant_roofline": {
            "kernel": "quantize_wave_kernel<f16, 44>",
            "bound": "hbm",
            "achieved": round(quant_achieved / 1e9, 1),
            "peak": HBM_PEAK / 1e9,
            "unit": "GB/s",
            "frac": round(quant_achieved / HBM_PEAK, 4),
            "traffic": quant_traffic,
            "work_per_launch": f"{quant_bytes:.4e} B = n*(2+1) + 4*n/44, n = 33*65536*2*8*44",
            "avg_launch_ms": round(quant_avg_s * 1e3, 4),
            "launches": len(quant_ms),
        },
        "dequant_roofline": {
            "kernel": "dequantize kernel, int8 + fp32 scale -> fp16",
            "bound": "hbm",
            "achieved": round(dequant_achieved / 1e9, 1),
            "peak": HBM_PEAK / 1e9,
            "unit": "GB/s",
            "frac": round(dequant_achieved / HBM_PEAK, 4),
            "traffic": dequant_traffic,
            "work_per_launch": f"{quant_bytes:.4e} B = n*(1+2) + 4*n/44, n = 33*65536*2*8*44",
            "avg_launch_ms": round(dequant_avg_s * 1e3, 4),
            "launches": len(dequant_ms),
        },
    }
    line["mfma_ceiling"] = ceiling
    line["cache_write"] = write
    line["prefill_attention"] = prefill
    line["end_to_end"] = model_e2e
    line["other_configs"] = others
    line["config4_end_to_end"] = c4
    line["small_tables"] = tables
    line["rmsnorm_roofline"] = norm_leg
    line["config1"] = c1
    if args.cpu_baseline == "on":
        line["cpu_baseline"] = cpu_baseline(torch, kv0, codes, scales, wq, wo, queries, layers, args.cpu_sample_groups)
    print(json.dumps(line), flush=True)


def cpu_model() -> str:
    """The host CPU's model name (what lscpu reports), from /proc/cpuinfo."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.lower().startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform

    return platform.processor() or "unknown"


def cpu_baseline(torch, kv, codes, scales, wq, wo, queries, layers, groups):
    """The same step on the host CPU, as the reference runs it there: fp32 torch on every core
    (predictor.py:318-321 turns mixed precision off on the CPU), through oracle.sublayer -- the
    quantizer as the reference's expression (kv_cache_scaling.py:29-37) on the fp32 cache, and
    per query batch the cached sequence-attention step (RMSNorm, Q projection, the online-softmax
    scan over the dequantized int8 cache in 32768-row blocks, layer.py:777-839, output
    projection, residual) over the codes the GPU built (bit-exact, so moved to the host as they
    are).

    Sample (about 10-20 s on a 16-core host): ``groups`` of the 33 token groups of one layer --
    their quantize and one 1024-row query batch; the step scales linearly in groups, layers and
    batches: 12 layers x 33/groups x (quantize + 4 batches), reported as extrapolated.
    """
    from oracle import sublayer as osl

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    src = kv[0][:groups].float().cpu()
    osl.quantize_int8(src[:1, :1024])  # first-call set-up outside the timing
    t0 = time.perf_counter()
    osl.quantize_int8(src)
    t_quant = time.perf_counter() - t0
    del src
    x = queries[0][:groups].float().cpu()
    w_q, w_o = wq[0].float().cpu(), wo[0].float().cpu()
    c, s = codes[0][:groups].cpu(), scales[0][:groups].cpu()
    t0 = time.perf_counter()
    osl.sequence_attention_step(x, w_q, w_o, c, s, heads=HEADS, head_dim=HEAD_DIM, alpha=DEEPNORM_ALPHA)
    t_batch = time.perf_counter() - t0
    seconds_per_step = layers * (GROUPS / groups) * (t_quant + QUERY_BATCHES * t_batch)
    return {
        "value": round(QUERY_BATCHES * QUERY_ROWS / seconds_per_step, 4),
        "unit": "query rows/s",
        "cores": cores,
        "cpu_model": cpu_model(),
        "kind": "port",
        "extrapolated": True,
        "seconds_per_step": round(seconds_per_step, 2),
        "sample": f"oracle.sublayer, fp32 torch, {cores} threads: quantize of {groups} of {GROUPS} token groups of one "
        f"layer's fp32 K/V ({t_quant:.2f} s) and one {QUERY_ROWS}-row query batch through that layer's cached "
        f"sequence attention over the GPU-built int8 codes of the same {groups} groups ({t_batch:.2f} s); "
        f"extrapolated linearly to {layers} layers x {GROUPS} groups x (quantize + {QUERY_BATCHES} batches)",
    }


def rmsnorm_leg(torch, dev, reps=6):
    """The context-side RMSNorm of one layer at this workload (33 x 65536 rows of 352 fp32, no
    weight, eps 1e-5) writing the fp16 projection operand, as the whole-context build does:
    HIP events around each launch."""
    import nori_amd

    g = torch.Generator(device=dev).manual_seed(6)
    x = torch.randn(GROUPS * CONTEXT_ROWS, EMBED, generator=g, device=dev)
    out = torch.empty(x.shape, dtype=torch.float16, device=dev)
    stream = torch.cuda.current_stream(dev)
    nori_amd.rms_norm(x, EMBED, None, 1e-5, out=out)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        nori_amd.rms_norm(x, EMBED, None, 1e-5, out=out)
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    nbytes = x.numel() * (4 + 2)
    return {
        "kernel": "rms_norm (fp32 in, fp16 out)", "bound": "hbm",
        "achieved": round(nbytes / (ms * 1e-3) / 1e9, 1), "peak": HBM_PEAK / 1e9, "unit": "GB/s",
        "frac": round(nbytes / (ms * 1e-3) / HBM_PEAK, 4), "avg_launch_ms": round(ms, 4),
        "work_per_launch": f"{nbytes:.4e} B = n*(4+2), n = 33*65536*352",
    }


# config 1: the reference's CPU end-to-end case on its NoriRegressor surface, run here on the
# GPU: a random-init nori-6m model, one table of 1024 context + 256 query rows x 16 features
CONFIG1 = dict(context=1024, queries=256, features=16, quantiles=(0.1, 0.5, 0.9), reps=3)


def config1(torch, dev):
    """NoriRegressor fit/predict on config 1's table (seed 0: X ~ N(0, 1), w ~ N(0, 1/16),
    y = X.w + 0.5 sin(X[:, 0]) + 0.1 N(0, 1)) with an int8 context cache (memory_policy
    {"cache_dtype": "int8"}; fp16 autocast), through the default eight-member preprocessing
    ensemble as the reference's estimator runs it, and through one member on the raw columns.
    The first predict builds the members' context caches, later ones reuse them (every predict
    fits the members' preprocessing steps again, as the reference does); wall clock with the
    device synchronized."""
    import numpy as np

    from nori_amd import api
    from nori_amd.transformer import FeaturesTransformer

    c = CONFIG1
    rng = np.random.default_rng(0)
    x = rng.standard_normal((c["context"] + c["queries"], c["features"])).astype(np.float32)
    w = rng.normal(0.0, 0.25, c["features"])
    y = x.astype(np.float64) @ w + 0.5 * np.sin(x[:, 0].astype(np.float64)) + 0.1 * rng.standard_normal(len(x))
    torch.manual_seed(0)
    model = FeaturesTransformer(**api.NORI_6M_CONFIG)
    xc, yc, xq = x[: c["context"]], y[: c["context"]], x[c["context"]:]
    out = {}
    for name, config in (("ensemble", None), ("raw_member", [{}])):
        reg = api.NoriRegressor(model=model, device=dev, inference_config=config, memory_policy={"cache_dtype": "int8"})
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        reg.fit(xc, yc)
        point = reg.predict(xq)
        torch.cuda.synchronize()
        t_first = time.perf_counter() - t0
        t0 = time.perf_counter()
        for _ in range(c["reps"]):
            point = reg.predict(xq)
            qs = reg.predict(xq, output_type="quantiles", quantiles=list(c["quantiles"]))
        torch.cuda.synchronize()
        t_again = (time.perf_counter() - t0) / c["reps"]
        report = reg.memory_report_
        assert np.isfinite(point).all() and np.isfinite(qs).all() and qs.shape == (3, c["queries"])
        out[name] = {
            "members": int(report["ensemble_members"]),
            "fit_and_first_predict_s": round(t_first, 4),
            "predict_point_and_quantiles_s": round(t_again, 4),
            "query_rows_per_s": round(c["queries"] / t_again, 1),
            "context_reused": bool(report["context_reused"]),
        }
    return {
        "what": "config 1: NoriRegressor fit/predict, random-init nori-6m, 1 table of 1024 context + 256 query rows "
        "x 16 features, int8 context cache, point + quantiles 0.1/0.5/0.9, fp16 autocast; the default "
        "eight-member preprocessing ensemble (4 quantile-uniform + 4 per-column members, 66 / 27 features each) "
        "and one member on the raw columns",
        "path": f"memory_policy {{'cache_dtype': 'int8'}} -> rung {report['rung']} (cache {report['cache_dtype']}, "
        "build_context_cache + apply_context_cache per member, dense ScalableSeqKV)",
        **out["ensemble"],
        "raw_member": out["raw_member"],
    }


if __name__ == "__main__":
    main()
