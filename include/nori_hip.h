/*
 * nori_hip.h -- C ABI of libnori_hip.so, the MI355X (gfx950) kernels of Nori's
 * in-context-learning (ICL) hot path: the int8 context K/V cache codec, RMSNorm, and
 * query-row -> context attention over the cached K/V.
 *
 * The reference (Synthefy/synthefy-nori) has no FFI: its operators are Python
 * callables over torch tensors. Each entry point below replaces one of them; the
 * comment names the reference function (file:line, relative to the reference repo
 * root) whose semantics it implements. The Python drop-ins that keep the reference's
 * names and signatures call these through ctypes (synthefy-nori_amd/nori_amd/_native.py).
 *
 * Conventions
 *   - Plain C types only. Device buffers are raw device pointers owned by the
 *     caller; the library allocates nothing unless a function says otherwise.
 *   - `stream` is a hipStream_t passed as void*; NULL is the legacy default stream.
 *     Work is enqueued on it; no entry point synchronises the host.
 *   - Strides are in ELEMENTS of the buffer they describe; the innermost (head_dim)
 *     axis is always contiguous.
 *   - Every entry point returns a nori_status. On failure, nori_last_error() returns
 *     a thread-local message describing the first problem found.
 */
#ifndef NORI_HIP_H
#define NORI_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    NORI_OK = 0,
    NORI_ERR_INVALID = 1,      /* bad shape/stride/pointer: the reference raises ValueError   */
    NORI_ERR_RUNTIME = 2,      /* HIP launch/runtime failure: RuntimeError                      */
    NORI_ERR_UNSUPPORTED = 3,  /* combination not implemented: NotImplementedError              */
    NORI_ERR_OUT_OF_MEMORY = 4 /* hipErrorOutOfMemory: torch.cuda.OutOfMemoryError upstream     */
} nori_status;

typedef enum {
    NORI_F32 = 0,
    NORI_F16 = 1,
    NORI_BF16 = 2,
    NORI_I8 = 3
} nori_dtype;

/* How `amax / 127.0` is evaluated when the scale is formed (see nori_kv_quantize_int8). */
typedef enum {
    NORI_SCALE_DIV_TRUE = 0,  /* IEEE division: torch's CPU kernel                          */
    NORI_SCALE_DIV_RECIP = 1  /* multiply by fp32 1/127: torch's ROCm/CUDA kernel            */
} nori_scale_div;

/* Flags of nori_icl_attention. */
#define NORI_ATTN_MERGE 1u /* merge into running (out fp32, lse) instead of overwriting them */

/* Version of this ABI (bumped on any signature change; 2: nori_icl_attention_takes_prologue takes
 * the query dtype; nori_linear_f16, nori_linear_f16_residual_rms_norm, nori_cell_tokens,
 * nori_layer_norm_cells, nori_swiglu_mlp_residual_rms_norm and the MFMA probe added; 3:
 * nori_quant_f16_scale_probe and nori_kv_project_quantize_int8_workspace_bytes added). */
#define NORI_ABI_VERSION 3
int nori_abi_version(void);

/* Thread-local description of the last failure on this thread ("" if none). */
const char* nori_last_error(void);

/*
 * Symmetric per-vector absmax int8 quantization of K/V head vectors.
 * Replaces quantize_int8 (src/synthefy_nori/model/kv_cache_scaling.py:29-37):
 *     scale = t.abs().amax(-1, keepdim=True).clamp_min(1e-12) / 127.0
 *     codes = clamp(round(t / scale), -127, 127).to(int8);  scales = scale.to(float32)
 * evaluated with torch's per-op rounding in the source dtype, so codes and scales are
 * bit-identical to the torch expression on the device `scale_div` names.
 *
 * Vectors are addressed two-level, so a slice written into preallocated storage
 * (BlockwiseSeqKV.from_row_slices, kv_cache_scaling.py:253-303) needs no copy:
 *   vector (o, i), o < n_outer, i < n_inner, has its d elements at
 *     src    + o*src_outer_stride    + i*src_inner_stride      (src_dtype)
 *     codes  + o*codes_outer_stride  + i*codes_inner_stride    (int8)
 *   and its scale at scales + o*scales_outer_stride + i*scales_inner_stride (fp32).
 * For a contiguous [BG, N, 2, Hkv, D] cache: n_outer = 1, n_inner = BG*N*2*Hkv,
 * inner strides d / d / 1.
 * src_dtype: NORI_F32, NORI_F16 or NORI_BF16. NaN inside a vector yields code 0.
 */
int nori_kv_quantize_int8(const void* src, int src_dtype, int64_t n_outer, int64_t n_inner, int32_t d,
                          int64_t src_outer_stride, int64_t src_inner_stride, int8_t* codes,
                          int64_t codes_outer_stride, int64_t codes_inner_stride, float* scales,
                          int64_t scales_outer_stride, int64_t scales_inner_stride, int32_t scale_div,
                          void* stream);

/*
 * Dequantization: dst = (float(codes) * scale) rounded to dst_dtype.
 * Replaces dequantize_int8 (kv_cache_scaling.py:40-41). Same two-level addressing
 * as nori_kv_quantize_int8, with dst in place of src.
 */
int nori_kv_dequantize_int8(const int8_t* codes, const float* scales, int64_t n_outer, int64_t n_inner,
                            int32_t d, int64_t codes_outer_stride, int64_t codes_inner_stride,
                            int64_t scales_outer_stride, int64_t scales_inner_stride, void* dst,
                            int dst_dtype, int64_t dst_outer_stride, int64_t dst_inner_stride,
                            void* stream);

/*
 * RMSNorm over rows of `cols` elements: y = x * rsqrt(mean(x^2) + eps) (* weight).
 * Replaces RMSNorm.forward (src/synthefy_nori/model/layer.py:251-258), native
 * (F.rms_norm) variant: statistic and product in fp32, one rounding to `dtype`.
 * weight may be NULL (elementwise_affine=False, the layer norms of layer.py:1346-1349);
 * otherwise it has `cols` elements of `weight_dtype`. y may be x (in place, same row stride):
 * the per-head key norm of the two-phase attentions (layer.py:497-500) normalizes the K half
 * of a projected [.., 2, H, D] K/V tensor in place, one head (rows at stride 2*H*D) a call.
 */
int nori_rms_norm(const void* x, int dtype, int64_t rows, int32_t cols, int64_t x_row_stride,
                  const void* weight, int weight_dtype, float eps, void* y, int64_t y_row_stride,
                  void* stream);

/*
 * nori_rms_norm with the result written as `y_dtype`: fp32 rows may be written as fp16 or
 * bf16 (any other pair is NORI_ERR_UNSUPPORTED). The value is the fp32 norm rounded once to
 * y_dtype -- bit for bit what an autocast projection's input cast makes of the norm's fp32
 * output (RMSNorm under torch.autocast, layer.py:251-258, followed by F.linear), so a norm
 * that feeds a projection hands it its operand directly instead of an fp32 copy to cast.
 */
int nori_rms_norm_to(const void* x, int dtype, int64_t rows, int32_t cols, int64_t x_row_stride,
                     const void* weight, int weight_dtype, float eps, void* y, int y_dtype,
                     int64_t y_row_stride, void* stream);

/*
 * Query-row -> context attention over a K/V cache:
 *     out[b, i, h, :] = softmax_j(scale * q[b, i, h, :] . k[b, j, hk, :]) @ v[b, j, hk, :]
 * with hk = h / (heads / kv_heads) (MQA/GQA broadcast, layer.py:640-649, 956).
 * Replaces the dense cached attention (MultiheadAttention.compute_attention_by_torch,
 * layer.py:936-1049), the CPU blockwise online softmax (layer.py:747-839) and the
 * GPU per-block flex + LSE merge (layer.py:841-934, _flex_attention_with_lse :132-182).
 *
 * q      : [bg, nq, heads, d] at q + b*q_bg_stride + i*q_row_stride + h*q_head_stride.
 * kv     : the cache as the reference lays it out, [bg, nk, 2, kv_heads, d]:
 *          K of (b, j, hk) at kv + b*kv_bg_stride + j*kv_row_stride + hk*d,
 *          V at the same place + kv_half_stride.
 *          kv_dtype NORI_I8: int8 codes with fp32 scales at
 *            kv_scales + b*sc_bg_stride + j*sc_row_stride + hk (+ sc_half_stride for V),
 *            dequantized in-kernel (kv_cache_scaling.py:40-41);
 *          NORI_F16 / NORI_BF16 / NORI_F32: full-precision cache, kv_scales ignored.
 * scale  : logit scale (1/sqrt(d) when the reference passes none, layer.py:798, 857).
 * out    : [bg, nq, heads, d] addressed like q, in out_dtype.
 * lse    : optional natural-log log-sum-exp of the scaled logits, fp32, [bg, heads, nq]
 *          contiguous (the flex LSE, layer.py:87-93, 123).
 * flags  : NORI_ATTN_MERGE: `out` (must be NORI_F32) and `lse` (required) hold a
 *          running normalized output and LSE from earlier key blocks; this call merges
 *          its keys into them exactly as layer.py:914-920 does (start from lse = -inf,
 *          out = 0).
 * workspace / workspace_bytes: device scratch for the split-context schedule; size from
 *          nori_icl_attention_workspace_size(). May be NULL/0, which disables splitting.
 * Requires d % 4 == 0, 4 <= d <= 128, heads % kv_heads == 0, nk >= 1.
 */
int nori_icl_attention(const void* q, int q_dtype, int64_t bg, int64_t nq, int32_t heads, int32_t d,
                       int64_t q_bg_stride, int64_t q_row_stride, int64_t q_head_stride, const void* kv,
                       int kv_dtype, const float* kv_scales, int64_t nk, int32_t kv_heads,
                       int64_t kv_bg_stride, int64_t kv_row_stride, int64_t kv_half_stride,
                       int64_t sc_bg_stride, int64_t sc_row_stride, int64_t sc_half_stride, float scale,
                       void* out, int out_dtype, int64_t out_bg_stride, int64_t out_row_stride,
                       int64_t out_head_stride, float* lse, uint32_t flags, void* workspace,
                       int64_t workspace_bytes, void* stream);

/*
 * Deep-norm residual update out[i] = x[i] + alpha * u[i] over n elements, x and out fp32, u
 * of u_dtype (NORI_F32 / NORI_F16 / NORI_BF16), rounded as torch evaluates `x + alpha * u`
 * for those dtypes: the product in fp32 rounded to u_dtype, then the fp32 sum. Replaces the
 * two passes of the two-phase encoder's residual updates (two_phase.py:198, 209, 220-225,
 * 264, 271-272). out may be x.
 */
int nori_residual_add(const float* x, const void* u, int u_dtype, float alpha, int64_t n, float* out,
                      void* stream);

/*
 * A deep-norm residual update and the RMSNorm (no weight) that reads its result, in one pass:
 * x_out = x + alpha * u exactly as nori_residual_add forms it (x, x_out fp32 [rows, cols],
 * contiguous; x_out may be x; u's rows contiguous, or -- u_rows = {d1, d2, s0, s1, s2} -- row
 * r = (i0 * d1 + i1) * d2 + i2 of u at element i0 * s0 + i1 * s1 + i2 * s2, e.g. a transposed
 * [batch, groups, rows] update of a [batch, rows, groups] stream; u_rows NULL for contiguous
 * rows), then y = x_out * rsqrt(mean(x_out^2) + eps) exactly as
 * nori_rms_norm_to forms it from fp32 rows, written as y_dtype (NORI_F32, or NORI_F16 /
 * NORI_BF16: the projection operand an autocast F.linear makes of it). Row r of y starts at
 * element (r / y_group) * y_group_stride + (r % y_group) * y_row_stride, so the rows of several
 * streams can be interleaved into one token buffer. The two-phase encoder's residual updates
 * followed by the pre-norm of the next sublayer (two_phase.py:198-225, 264-272 with
 * layer.py:251-253), bit for bit the two separate calls. Rows of more than 1024 elements, cols
 * not a multiple of 4 and unaligned operands return NORI_ERR_UNSUPPORTED before any device work.
 */
int nori_residual_add_rms_norm(const float* x, const void* u, int u_dtype, const int64_t* u_rows, float alpha,
                               int64_t rows, int32_t cols, float eps, float* x_out, void* y, int y_dtype,
                               int64_t y_group, int64_t y_group_stride, int64_t y_row_stride, void* stream);

/*
 * LayerNorm over rows of `cols` elements: y = (x - mean) * rsqrt(var + eps) * weight + bias,
 * then max(y, 0) when `relu` is non-zero, written as `y_dtype`. Replaces the nn.LayerNorm
 * calls of the cell encoder under the dtype rules of fp16 autocast (the RBF numeric
 * embedding's norm, src/synthefy_nori/model/encoders.py:118-276, and the fusion MLP
 * Linear -> LayerNorm -> ReLU -> Linear -> LayerNorm, :432-585): statistics in fp32 (mean,
 * biased variance), fp32 weight and bias (either may be NULL), the fp32 result rounded once
 * to y_dtype -- the fp16 operand an autocast F.linear makes of it, or fp32. cols is a
 * multiple of 4; rows at x_row_stride / y_row_stride elements (multiples of 4), x and y
 * aligned to 4 elements.
 */
int nori_layer_norm(const void* x, int x_dtype, int64_t rows, int32_t cols, int64_t x_row_stride, const float* weight,
                    const float* bias, float eps, int relu, void* y, int y_dtype, int64_t y_row_stride, void* stream);

/*
 * SwiGLU gate over the [gate | up] output of one fused projection (gate and up weights stacked,
 * so the operand is read once): out[r, j] = T(T(silu(gu[r, j])) * gu[r, hidden + j]) with
 * silu(x) = x / (1 + exp(-x)) in fp32 and T the rounding to `dtype` (NORI_F32 / NORI_F16 /
 * NORI_BF16) -- torch's F.silu(gate) * up in that dtype, the middle of SwiGLUMLP.forward
 * (src/synthefy_nori/model/layer.py:261-274). Rows at row_stride (>= 2 * hidden) elements in,
 * out_row_stride (>= hidden) out.
 */
int nori_silu_mul(const void* gu, int dtype, int64_t rows, int32_t hidden, int64_t row_stride, void* out,
                  int64_t out_row_stride, void* stream);

/*
 * The whole SwiGLU feed-forward sublayer in one kernel, for fp16 rows (the fp16-autocast
 * SwiGLUMLP.forward, src/synthefy_nori/model/layer.py:261-274, without biases):
 *     y[r] = T(T(T(silu(T(x[r] Wg^T))) * T(x[r] Wu^T)) Wd^T)
 * with T the rounding to fp16 and fp32 sums. x: [rows, width] at x_row_stride elements;
 * w_gate_up: [2 * hidden, width] contiguous, the gate rows then the up rows; w_down:
 * [width, hidden] contiguous; y: [rows, width] at y_row_stride. width (the sublayer's in and
 * out features) is 128, 256 or 352; hidden is the gate/up width padded to a multiple of 32
 * with zero gate/up rows and zero down columns. Strides are multiples of 8 and the four
 * pointers 16-byte aligned. The projections sum in their own order (a value may differ from
 * the unfused GEMMs by one fp16 ulp) and silu uses the hardware exp2 and reciprocal; the
 * hidden activations never leave the CU. Other widths or dtypes: NORI_ERR_UNSUPPORTED
 * (the caller keeps the unfused projections and nori_silu_mul).
 */
int nori_swiglu_mlp(const void* x, int dtype, int64_t rows, int32_t width, int64_t x_row_stride,
                    const void* w_gate_up, const void* w_down, int32_t hidden, void* y, int64_t y_row_stride,
                    void* stream);

/*
 * nori_swiglu_mlp followed by the deep-norm residual update of an fp32 stream and the next
 * sublayer's RMSNorm without weight, in one kernel (reference model/two_phase.py:209,
 * 220-225, 271-272 with layer.py:251-253 and 261-274): per row r, u = the MLP's fp16 output
 * (never written), stream[r] = stream[r] + fp16(fp32(u) * alpha) in place, and each group of
 * norm_width columns k is normalized, fp16(s * rsqrt(mean(s^2) + eps)), into output group
 * q = r * (width / norm_width) + k at element (q / y_group) * y_group_stride +
 * (q % y_group) * y_row_stride of y (fp16). Bit for bit nori_swiglu_mlp then
 * nori_residual_add_rms_norm. Built for width 128 (norm_width 128) and 256 (norm_width 128
 * or 256); stream rows stream_row_stride apart, 16-byte aligned; y 8-byte aligned.
 */
int nori_swiglu_mlp_residual_rms_norm(const void* x, int dtype, int64_t rows, int32_t width, int64_t x_row_stride,
                                      const void* w_gate_up, const void* w_down, int32_t hidden, float alpha,
                                      float* stream_rows, int64_t stream_row_stride, int32_t norm_width, float eps,
                                      void* y, int64_t y_group, int64_t y_group_stride, int64_t y_row_stride,
                                      void* stream);

/*
 * QASS "full" query scaling in one pass (replaces QASSMaxScaling.forward's gate branch,
 * src/synthefy_nori/model/layer.py:316-456, as it runs under fp16 autocast):
 *     out[r, h] = T(T(q[r, h] * base_scale[h]) * T(1 + T(tanh(T(T(gelu(T(q[r, h] W1^T + b1))) W2^T + b2)))))
 * with T the rounding to fp16, fp32 sums and gelu the erf form. q: [rows, heads, d] fp16 with
 * rows q_row_stride elements apart and heads contiguous; w1: [hidden, d], b1: [hidden], w2:
 * [d, hidden], b2: [d], base_scale: [heads, d] (log n * (1 + tanh(base_mlp(log n))), formed by
 * the caller), all fp16 and contiguous; out like q at out_row_stride. hidden is 64; d a
 * multiple of 4 up to 64; strides multiples of 4; q, base_scale and out 8-byte aligned. The two
 * GEMMs sum in their own order (a value may differ from the separate ops by one fp16 ulp).
 * Other shapes or dtypes: NORI_ERR_UNSUPPORTED (the caller keeps the separate ops).
 */
int nori_qass_gate(const void* q, int dtype, int64_t rows, int32_t heads, int32_t d, int64_t q_row_stride,
                   const void* w1, const void* b1, const void* w2, const void* b2, int32_t hidden,
                   const void* base_scale, void* out, int64_t out_row_stride, void* stream);

/*
 * What the two-phase encoder's attentions do to q and k between the projection and the
 * attention (layer.py:1122-1134 with qk_norm and QASS "log_only", layer.py:433-456), applied
 * by nori_icl_attention_qk to each query row and key row as it is loaded:
 *     q := T(T(q * rsqrt(mean(q^2) + eps)) * q_weight)   when q_weight is not NULL
 *     q := T(q * q_mult)                                  when q_mult != 1
 *     k := T(T(k * rsqrt(mean(k^2) + eps)) * k_weight)   when k_weight is not NULL
 * (means over the head's d elements in fp32, T = rounding to the q or cache dtype), the
 * values the per-head RMSNorm (eps 1e-6, elementwise gain) and the fp16 multiply by
 * fp16(log n) produce when run as separate passes.
 */
typedef struct {
    const void* q_weight; /* [d] query norm gain, or NULL: no query norm */
    const void* k_weight; /* [d] key norm gain, or NULL: no key norm */
    int weight_dtype;     /* nori_dtype of both gains */
    float eps;
    float q_mult;         /* 1.0f: no multiply */
} nori_qk_prologue;

/*
 * nori_icl_attention with the q/k prologue above fused into the loads. Has no counterpart in
 * the reference as one call (it replaces the RMSNorm passes over q and K, the q multiply and
 * the attention of MultiheadAttention.forward, layer.py:1062-1162). Taken where the
 * short-context kernel runs (few queries over few keys: the in-row attentions of the
 * two-phase encoder, full-precision caches) and on resident-context launches (fp16 queries
 * over contexts of up to 256 keys read by many queries: its column and row attentions; a key
 * norm there needs an fp16 cache); nori_icl_attention_takes_prologue says which. Elsewhere it returns
 * NORI_ERR_UNSUPPORTED having done nothing, and the caller runs the separate passes.
 */
int nori_icl_attention_qk(const void* q, int q_dtype, int64_t bg, int64_t nq, int32_t heads, int32_t d,
                          int64_t q_bg_stride, int64_t q_row_stride, int64_t q_head_stride, const void* kv,
                          int kv_dtype, const float* kv_scales, int64_t nk, int32_t kv_heads,
                          int64_t kv_bg_stride, int64_t kv_row_stride, int64_t kv_half_stride,
                          int64_t sc_bg_stride, int64_t sc_row_stride, int64_t sc_half_stride, float scale,
                          void* out, int out_dtype, int64_t out_bg_stride, int64_t out_row_stride,
                          int64_t out_head_stride, float* lse, uint32_t flags, void* workspace,
                          int64_t workspace_bytes, const nori_qk_prologue* prologue, void* stream);

/*
 * Fused context-cache write: K/V projection of context rows straight into the int8 cache.
 * Replaces MultiheadAttention.project_kv_cache (src/synthefy_nori/model/layer.py:651-683)
 * followed by quantize_int8 (kv_cache_scaling.py:29-37) on the GPU's autocast path, with the
 * layer's RMSNorm (layer.py:251-253, without an elementwise weight) optionally applied first:
 *     xn = norm ? T(x * rsqrt(mean(x^2) + eps)) : x          (T = x_dtype)
 *     kv[r, j*d + e] = f16( f16(xn[r]) . f16(weight[j*d + e]) )  (fp32 accumulation)
 *     codes, scales = quantize_int8(kv) with T = fp16 and the scale formed per `scale_div`
 * Rows sit on a two-level grid, row (o, i) for o < n_outer, i < n_inner (a row slice of a
 * [BG, N, ...] cache, or activations read group by group, in one call):
 * x      : embed elements at x + o*x_outer_stride + i*x_row_stride (elements), x_dtype
 *          NORI_F32 / NORI_F16 / NORI_BF16;
 * weight : [2*kv_heads*d, embed] at weight + k*w_row_stride (K heads, then V heads: the
 *          reference's qkv_proj_weight[1:] viewed as [2*H*D, E], or its first head for a
 *          shared-head cache);
 * codes  : [2, kv_heads, d] int8 at codes + o*codes_outer_stride + i*codes_row_stride (bytes);
 * scales : [2, kv_heads] fp32 at scales + o*scales_outer_stride + i*scales_row_stride (floats).
 * Rows of x and weight must be 16-byte aligned and a whole number of 16-byte chunks; code
 * rows 4-byte aligned; d a multiple of 4 up to 128; embed at most 1024. The fp16 K/V are never
 * written.
 * workspace: see nori_kv_project_quantize_int8_workspace_bytes. fp32 x with fp16 weight rows,
 * embed a multiple of 8 up to 384 and d up to 64 (nori-30m: 352, 44) take one pass with no
 * workspace (each row read and normalized once, every head in one workgroup); other cases
 * write the f16 operand rows to the workspace first.
 * The projection's fp32 sums run in MFMA order, not the library GEMM's, so a K/V value can
 * differ from torch's fp16 F.linear in its last bit and its code by one.
 */
int nori_kv_project_quantize_int8(const void* x, int x_dtype, int64_t n_outer, int64_t n_inner, int32_t embed,
                                  int64_t x_outer_stride, int64_t x_row_stride, int32_t norm, float eps,
                                  const void* weight, int weight_dtype, int64_t w_row_stride, int32_t kv_heads,
                                  int32_t d, int8_t* codes, int64_t codes_outer_stride, int64_t codes_row_stride,
                                  float* scales, int64_t scales_outer_stride, int64_t scales_row_stride,
                                  int32_t scale_div, void* workspace, int64_t workspace_bytes, void* stream);

/* Bytes of (16-byte aligned) workspace nori_kv_project_quantize_int8 needs: the f16 operand
 * rows, n_outer*n_inner rows of embed rounded up to 32 -- 0 when x is used as it is (fp16, no
 * norm, embed a multiple of 32). Written and read within the call's stream order. */
int64_t nori_kv_project_quantize_int8_workspace_size(int x_dtype, int64_t n_outer, int64_t n_inner, int32_t embed,
                                                     int32_t norm);
/* The workspace one nori_kv_project_quantize_int8 call with these arguments needs: 0 where it
 * takes the one pass (fp32 x, fp16 weight, embed a multiple of 8 up to 384, d up to 64), else
 * nori_kv_project_quantize_int8_workspace_size. */
int64_t nori_kv_project_quantize_int8_workspace_bytes(int x_dtype, int64_t n_outer, int64_t n_inner, int32_t embed,
                                                      int32_t norm, int weight_dtype, int32_t d);

/*
 * 1 when nori_icl_attention_qk takes a prologue for these sizes, cache dtype and query dtype
 * (with a key norm when with_key_norm is nonzero), 0 when it would return
 * NORI_ERR_UNSUPPORTED. Has no counterpart in the reference: it answers, for the caller
 * choosing between the fused prologue and the separate norm passes of
 * MultiheadAttention.forward (layer.py:1122-1134), the launch planner's question without
 * device work.
 */
int32_t nori_icl_attention_takes_prologue(int64_t bg, int64_t nq, int32_t heads, int32_t d, int64_t nk,
                                          int32_t kv_dtype, int32_t with_key_norm, int32_t q_dtype);

/* Bytes of workspace nori_icl_attention uses for these sizes (0 when it never splits). */
int64_t nori_icl_attention_workspace_size(int64_t bg, int64_t nq, int32_t heads, int32_t d, int64_t nk);

/* Bytes of split-context scratch the library holds per device for nori_icl_attention_noalloc. */
#define NORI_NOALLOC_SCRATCH_BYTES (32LL << 20)

/*
 * nori_icl_attention without a workspace argument, allocating nothing: no hipMalloc, no
 * hipFree, no allocating library call. Has no counterpart in the reference; it is for callers
 * that cannot allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid allocation). Arguments mean what they mean for nori_icl_attention.
 * The split-context partials go to a scratch array of NORI_NOALLOC_SCRATCH_BYTES that the
 * library holds on every device it runs on until the process ends; its address is looked up
 * on the first call on a device. Sizes whose partials need more scratch than that
 * (nori_icl_attention_workspace_size) return NORI_ERR_UNSUPPORTED before any device work.
 * Every call on a device shares that device's scratch: calls that overlap on one device (on
 * different streams, or from different threads) race and must be ordered by the caller.
 */
int nori_icl_attention_noalloc(const void* q, int q_dtype, int64_t bg, int64_t nq, int32_t heads, int32_t d,
                               int64_t q_bg_stride, int64_t q_row_stride, int64_t q_head_stride, const void* kv,
                               int kv_dtype, const float* kv_scales, int64_t nk, int32_t kv_heads,
                               int64_t kv_bg_stride, int64_t kv_row_stride, int64_t kv_half_stride,
                               int64_t sc_bg_stride, int64_t sc_row_stride, int64_t sc_half_stride, float scale,
                               void* out, int out_dtype, int64_t out_bg_stride, int64_t out_row_stride,
                               int64_t out_head_stride, float* lse, uint32_t flags, void* stream);

/*
 * y = x W^T in fp16: the F.linear of the attention projections under the GPU's fp16 autocast
 * (reference model/layer.py:651-683 for the K/V projection, 1114-1160 for the Q, K/V and
 * output projections; model/two_phase.py:53-55, 122-138 for the two-phase attentions): fp32
 * sums of fp16 products, one rounding to fp16 (the library GEMM's result up to the order of
 * its fp32 sums). x holds n_outer * n_mid * n_inner rows of k fp16 elements, row (o, j, i) at
 * element offset o * x_outer_stride + j * x_mid_stride + i * x_row_stride; weight holds n rows
 * of k elements, w_row_stride apart; output row (o, j, i) is written at o * y_outer_stride +
 * j * y_mid_stride + i * y_row_stride. k is 128 or 256 and n a multiple of 4; x and weight
 * rows 16-byte aligned, output rows 8-byte aligned. Built for tall operands (HBM-bound: each x
 * row read once, each output row written once).
 */
int nori_linear_f16(const void* x, int64_t n_outer, int64_t n_mid, int64_t n_inner, int32_t k,
                    int64_t x_outer_stride, int64_t x_mid_stride, int64_t x_row_stride, const void* weight,
                    int64_t w_row_stride, int32_t n, void* y, int64_t y_outer_stride, int64_t y_mid_stride,
                    int64_t y_row_stride, void* stream);

/*
 * The output projection of an attention sublayer, the deep-norm residual update and the next
 * sublayer's RMSNorm in one pass (reference model/two_phase.py:198, 209, 220-225, 264, 271-272:
 * `x = x + alpha * out_proj(attn)` then `norm(x)` with an RMSNorm without weight,
 * model/layer.py:251-253, whose result the next projection takes as fp16 under autocast):
 *   u = fp16(a W^T) (as nori_linear_f16), x = x + fp16(fp32(u) * alpha) in fp32 (in place),
 *   y = fp16(x * rsqrt(mean(x^2) + eps)).
 * Bit for bit nori_linear_f16 followed by nori_residual_add_rms_norm (fp16 update and output).
 * a: n_outer * n_mid * n_inner rows of k fp16 elements on the three-level grid of
 * nori_linear_f16; weight: k rows of k elements (output width = k), w_row_stride apart; x: the
 * fp32 stream rows and y: the fp16 output rows, on the same grid with their own strides. k is
 * 128 or 256; a and weight rows 16-byte aligned, x rows 16-byte aligned, y rows 8-byte
 * aligned; a, x and y must not overlap.
 */
int nori_linear_f16_residual_rms_norm(const void* a, int64_t n_outer, int64_t n_mid, int64_t n_inner, int32_t k,
                                      int64_t a_outer_stride, int64_t a_mid_stride, int64_t a_row_stride,
                                      const void* weight, int64_t w_row_stride, float alpha, float* x,
                                      int64_t x_outer_stride, int64_t x_mid_stride, int64_t x_row_stride, float eps,
                                      void* y, int64_t y_outer_stride, int64_t y_mid_stride, int64_t y_row_stride,
                                      void* stream);

/*
 * The cell encoder's last LayerNorm followed by the two additions of the two-phase forward
 * (reference model/transformer.py:370-562: the feature positional embedding of the cell's
 * group, then the target-aware row bias, :1080-1132), over cells x [tables, rows, groups,
 * cols] (fp16 or fp32 rows x_row_stride apart; the fusion network's last Linear output):
 *   v = LayerNorm(x) * weight + bias                       (as nori_layer_norm, fp32)
 *   v = v + pos[group]                                     (pos fp32 [groups][cols], or NULL)
 *   rb = ctx[table][row] for row < eval_pos, else 0         (ctx fp32 [tables][eval_pos][cols])
 *   with alpha: gate = sigmoid(sum(v * rb) * inv_sqrt_e),
 *               v = (v + (1 - alpha) rb) + alpha (rb * gate)
 *   without alpha: v = v + rb;  no ctx: no row bias.
 * y: fp32 [tables * rows * groups][cols], contiguous. cols 64, 128 or 256. Each op rounds as
 * torch's does; the norm's statistics and the gate's dot product are summed in the kernel's
 * order.
 */
int nori_layer_norm_cells(const void* x, int x_dtype, int64_t tables, int64_t rows, int64_t groups, int32_t cols,
                          int64_t x_row_stride, const float* weight, const float* bias, float eps, const float* pos,
                          const float* ctx, int64_t eval_pos, const float* alpha, float inv_sqrt_e, float* y,
                          void* stream);

/*
 * The fp16 cell tokens of the two-phase model's cell embedding under fp16 autocast: what
 * MaskEmbEncoder.forward (reference model/encoders.py:432-585) hands its fusion network's
 * first Linear, from the cell values x [tables, rows, groups, features] (fp32): per value the
 * scientific-notation RBF embedding (encoders.py:118-276: float64 mantissa/exponent split and
 * Gaussian kernels, the gate of the sign/exponent embeddings, LayerNorm, output Linear) in
 * channels [0, n_rbf), the prompt-quantile PLE coordinates (encoders.py:309-429) in
 * [n_rbf, n_rbf + n_bins), or the mask embedding where x is NaN. gate_table: fp16
 * [40][2][n_kernels], sigmoid(gamma) then tanh(beta) of the gate MLP for the row
 * 20 (x < 0) + 10 (exponent < 0) + exponent digit; centers [n_kernels], sigma [1], ln_weight,
 * ln_bias [n_kernels] fp32 (may be NULL: 1, 0); w_out fp16 [n_rbf][n_kernels], b_out fp16
 * [n_rbf] (may be NULL); edges fp32 [tables][groups][features][n_bins + 1]; mask_embedding
 * fp32 [n_rbf + n_bins] (NULL: NaN cells keep the embedding of 0); out fp16
 * [tables * rows * groups * features][n_rbf + n_bins]. Built for n_kernels 16 or 32,
 * n_rbf 96, n_bins 32. The LayerNorm's and the output projection's fp32 sums are in the
 * kernel's order; every other op rounds as torch's does.
 */
int nori_cell_tokens(const float* x, int64_t tables, int64_t rows, int32_t groups, int32_t features,
                     int32_t n_kernels, const float* centers, const float* sigma, const void* gate_table,
                     const float* ln_weight, const float* ln_bias, float ln_eps, const void* w_out, const void* b_out,
                     int32_t n_rbf, const float* edges, int32_t n_bins, const float* mask_embedding, void* out,
                     void* stream);

/* ---- measurement (no counterpart in the reference) ----
 *
 * The dense f16 MFMA rate this GPU sustains on given operand data. Under a dense MFMA load
 * the engine clock is set by the power limit, and an MFMA's power depends on its operand
 * bits, so the achievable rate depends on the data (bench.py times random against all-zero
 * operands beside the attention kernel's figures). nori_mfma_f16_probe runs nothing but
 * v_mfma_f32_32x32x16_f16 for `iters` iterations of eight MFMAs per wavefront, four
 * wavefronts per SIMD on every CU, each wavefront cycling through eight operand register sets
 * read from `operands` (n_vec 16-byte vectors of f16 pairs, indexed modulo n_vec); `sink`
 * (sink_len floats) takes the accumulators so nothing is optimized away.
 * nori_mfma_f16_probe_flop gives the FLOP one call performs on the current device (-1 when it
 * cannot be queried).
 */
int nori_mfma_f16_probe(const void* operands, int64_t n_vec, int32_t iters, float* sink, int64_t sink_len,
                        void* stream);
int64_t nori_mfma_f16_probe_flop(int64_t iters);

/* The scale and reciprocal the fused cache write (nori_kv_project_quantize_int8) derives from an
 * f16 head vector's absmax, without a division: s = f16(|absmax| * RN(1/127)) and
 * y = rcp(s) refined by one Newton step, for n f16 absmax values (their sign is ignored) into
 * s[n] and y[n] (fp32). A check hook with no counterpart in the reference: it lets a test hold
 * s to f16(|absmax| / 127) (quantize_int8, src/synthefy_nori/model/kv_cache_scaling.py:29-37)
 * and y to the correctly rounded 1/s over every f16 value, the premise of the fused write's
 * exact quotients. n at most 2^30. */
int nori_quant_f16_scale_probe(const uint16_t* absmax, int64_t n, float* s, float* y, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NORI_HIP_H */
