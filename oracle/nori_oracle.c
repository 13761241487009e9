/*
 * CPU oracle for the int8 context-cache codec and RMSNorm.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker the HIP kernels are compared
 * against; it is never part of the product path. Only tests/, the smoke check in
 * __graft_entry__.py and the cpu_baseline leg of bench.py may load it.
 *
 * What it restates (reference file:line, paths relative to the reference repo root):
 *
 *   quantize_int8   src/synthefy_nori/model/kv_cache_scaling.py:29-37
 *       scale = t.abs().amax(-1, keepdim=True).clamp_min(1e-12) / 127.0
 *       q     = clamp(round(t / scale), -127, 127).to(int8);  scale.to(float32)
 *   dequantize_int8 src/synthefy_nori/model/kv_cache_scaling.py:40-41
 *       (q.float() * scale).to(dtype)
 *
 * Torch evaluates every one of those ops in the tensor's own dtype T: each op is
 * computed in fp32 ("opmath") and its result rounded to T before the next op reads
 * it. For T = bf16 that means t/scale is rounded to bf16 BEFORE round() sees it, so
 * 101.3 -> 101.5 -> 102 is part of the specification. The oracle therefore rounds
 * to T after every op, exactly where torch does.
 *
 * One step differs by device. `m / 127.0` divides by a Python scalar: torch's CPU
 * kernel performs a true IEEE division, while its ROCm/CUDA kernel multiplies by the
 * host-computed fp32 reciprocal 1.0f/127.0f (aten BinaryDivTrueKernel, CPU-scalar
 * branch). `div_mode` selects which of the two the oracle reproduces:
 *   ORACLE_DIV_TRUE  (0)  torch on CPU
 *   ORACLE_DIV_RECIP (1)  torch on a GPU
 *
 * NaN inside a vector propagates through amax to the scale and every quotient; the
 * int8 conversion of NaN is implementation-defined in C. The oracle returns code 0
 * for it, which is what the GPU's float->int conversion produces.
 *
 * Parity pins for this file live in tests/test_oracle_codec.py: exhaustive f16/bf16
 * rounding against numpy and bit twiddling, torch's own CPU execution of the reference
 * expression on random tensors of every dtype, hand-computed known answers (including
 * the bf16 double-rounding case) and the invariants the reference's tests state.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

enum { ORACLE_F32 = 0, ORACLE_F16 = 1, ORACLE_BF16 = 2 };
enum { ORACLE_DIV_TRUE = 0, ORACLE_DIV_RECIP = 1 };

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* fp32 -> bf16 bits, round to nearest even; NaN stays a (quiet) NaN. */
uint16_t oracle_f32_to_bf16(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float oracle_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* fp32 -> IEEE binary16 bits, round to nearest even, with subnormals and overflow. */
uint16_t oracle_f32_to_f16(float f) {
    uint32_t u = f2u(f);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t a = u & 0x7fffffffu;
    if (a >= 0x7f800000u) return (uint16_t)(sign | (a > 0x7f800000u ? 0x7e00u : 0x7c00u));
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to inf */
    if (a < 0x38800000u) {                                    /* below 2^-14: subnormal */
        /* |f| * 2^24 is exact in fp32; rintf rounds half to even in the default mode. */
        float m = rintf(u2f(a) * 16777216.0f);
        return (uint16_t)(sign | (uint16_t)m);
    }
    uint32_t h = (((a >> 23) - 112u) << 10) | ((a & 0x7fffffu) >> 13);
    uint32_t rb = a & 0x1fffu;
    if (rb > 0x1000u || (rb == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

float oracle_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0x1f) return u2f(sign | 0x7f800000u | (m << 13) | (m ? 0x00400000u : 0u));
    if (e == 0) return (h & 0x8000u) ? -ldexpf((float)m, -24) : ldexpf((float)m, -24);
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

/* Round an fp32 value to dtype T and return it as fp32 again. */
static inline float round_to(float f, int dtype) {
    switch (dtype) {
        case ORACLE_F16: return oracle_f16_to_f32(oracle_f32_to_f16(f));
        case ORACLE_BF16: return oracle_bf16_to_f32(oracle_f32_to_bf16(f));
        default: return f;
    }
}

static inline float load_as_f32(const void* src, int dtype, int64_t i) {
    switch (dtype) {
        case ORACLE_F16: return oracle_f16_to_f32(((const uint16_t*)src)[i]);
        case ORACLE_BF16: return oracle_bf16_to_f32(((const uint16_t*)src)[i]);
        default: return ((const float*)src)[i];
    }
}

static inline void store_from_f32(void* dst, int dtype, int64_t i, float v) {
    switch (dtype) {
        case ORACLE_F16: ((uint16_t*)dst)[i] = oracle_f32_to_f16(v); break;
        case ORACLE_BF16: ((uint16_t*)dst)[i] = oracle_f32_to_bf16(v); break;
        default: ((float*)dst)[i] = v; break;
    }
}

/* clamp_min's floor 1e-12 converted to T the way c10::Scalar::to<T>() does it
 * (double -> float -> T). In fp16 it underflows to 0. */
static inline float clamp_floor(int dtype) { return round_to((float)1e-12, dtype); }

/* Quantize one vector of d elements.  kv_cache_scaling.py:35-37. */
static void quantize_vector(const void* src, int dtype, int64_t base, int d, int div_mode,
                            int8_t* codes, float* scale_out) {
    /* t.abs().amax(-1): exact in T; NaN propagates. */
    float m = 0.0f;
    int has_nan = 0;
    for (int i = 0; i < d; ++i) {
        float a = fabsf(load_as_f32(src, dtype, base + i));
        if (a != a) has_nan = 1;
        else if (a > m) m = a;
    }
    if (has_nan) m = NAN;
    /* .clamp_min(1e-12): max(m, floor) in T, NaN stays NaN. */
    float lo = clamp_floor(dtype);
    if (!(m != m) && m < lo) m = lo;
    /* / 127.0 */
    float s;
    if (div_mode == ORACLE_DIV_RECIP) {
        const float inv127 = 1.0f / 127.0f; /* computed in fp32 on the host by torch */
        s = round_to(m * inv127, dtype);
    } else {
        s = round_to(m / 127.0f, dtype);
    }
    for (int i = 0; i < d; ++i) {
        float t = load_as_f32(src, dtype, base + i);
        float r = round_to(t / s, dtype);         /* t / scale, rounded to T */
        float k = nearbyintf(r);                    /* torch.round: half to even, exact in T */
        int8_t c;
        if (k != k) c = 0;                          /* NaN: see header */
        else if (k > 127.0f) c = 127;
        else if (k < -127.0f) c = -127;
        else c = (int8_t)k;
        codes[base + i] = c;
    }
    *scale_out = s; /* scale.to(float32): exact */
}

/* Quantize n_vec contiguous vectors of d elements of dtype `dtype`.
 * codes: n_vec*d int8; scales: n_vec fp32. */
void oracle_quantize_int8(const void* src, int dtype, int64_t n_vec, int d, int div_mode,
                          int8_t* codes, float* scales) {
    for (int64_t v = 0; v < n_vec; ++v)
        quantize_vector(src, dtype, v * (int64_t)d, d, div_mode, codes, &scales[v]);
}

/* (q.float() * scale).to(dtype).  kv_cache_scaling.py:40-41. */
void oracle_dequantize_int8(const int8_t* codes, const float* scales, int64_t n_vec, int d,
                            void* dst, int dtype) {
    for (int64_t v = 0; v < n_vec; ++v) {
        float s = scales[v];
        for (int i = 0; i < d; ++i) {
            int64_t j = v * (int64_t)d + i;
            store_from_f32(dst, dtype, j, (float)codes[j] * s);
        }
    }
}

/* Round-trip helpers so the Python side can pin the rounding primitives directly. */
void oracle_round_f32_array(const float* x, int64_t n, int dtype, float* y) {
    for (int64_t i = 0; i < n; ++i) y[i] = round_to(x[i], dtype);
}

void oracle_f32_to_f16_array(const float* x, int64_t n, uint16_t* y) {
    for (int64_t i = 0; i < n; ++i) y[i] = oracle_f32_to_f16(x[i]);
}

void oracle_f32_to_bf16_array(const float* x, int64_t n, uint16_t* y) {
    for (int64_t i = 0; i < n; ++i) y[i] = oracle_f32_to_bf16(x[i]);
}

/*
 * RMSNorm, layer.py:233-258: y = x * rsqrt(mean(x^2) + eps) (* w).
 * The oracle evaluates the statistic and the product in double and rounds once to
 * the output dtype; the kernels are held to a stated ulp tolerance against it (torch's
 * own native and decomposed variants differ by 1 bf16 ulp, predictor.py:247-250).
 */
void oracle_rms_norm(const void* x, const void* w, int dtype, int64_t rows, int cols,
                     double eps, void* y) {
    for (int64_t r = 0; r < rows; ++r) {
        double acc = 0.0;
        for (int c = 0; c < cols; ++c) {
            double v = (double)load_as_f32(x, dtype, r * cols + c);
            acc += v * v;
        }
        double inv = 1.0 / sqrt(acc / (double)cols + eps);
        for (int c = 0; c < cols; ++c) {
            double v = (double)load_as_f32(x, dtype, r * cols + c) * inv;
            if (w) v *= (double)load_as_f32(w, dtype, c);
            store_from_f32(y, dtype, r * cols + c, (float)v);
        }
    }
}
