// LayerNorm over rows for gfx950: y = (x - mean) * rsqrt(var + eps) (* w + b), optionally
// followed by a ReLU, written in the dtype of the op that consumes it.
//
// Semantics: torch.nn.functional.layer_norm as the cell encoder's modules run it (the RBF
// numeric embedding's norm and the fusion MLP's two norms, src/synthefy_nori/model/
// encoders.py:118-276, 432-585): statistics in fp32 (mean, biased variance), the affine
// parameters in fp32. Under fp16 autocast torch runs layer_norm in fp32 and the following
// F.linear rounds its input to fp16; the kernel writes that fp16 operand directly (one
// rounding of the same fp32 value), or fp32 where an fp32 op follows. The statistics are
// summed in a different order than torch's Welford loop, so values can differ from torch's
// in the last fp32 bit.
//
// Schedule. HBM-bound: each row is read once and written once. Rows whose length is 4 times
// a power of two up to 256 are owned by a group of cols/4 lanes, 4 consecutive elements a
// lane (a 128-wide row: 32 lanes, two rows a wavefront); the group reduces with lane
// shuffles. Other widths (a multiple of 4) take one wavefront per row, looping over the row.
#include <algorithm>
#include <type_traits>

#include "nori_common.h"

#pragma clang fp contract(off)

namespace {

using namespace nori;

constexpr int kThreads = 256;

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <int DT>
__device__ __forceinline__ void load4(const void* p, int64_t i, float (&v)[4]) {
    if constexpr (DT == NORI_F32) {
        const f32x4 c = *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(p) + i);
        v[0] = c[0]; v[1] = c[1]; v[2] = c[2]; v[3] = c[3];
    } else {
        const u32x2 c = *reinterpret_cast<const u32x2*>(reinterpret_cast<const uint16_t*>(p) + i);
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const uint16_t lo = (uint16_t)(c[k] & 0xffff), hi = (uint16_t)(c[k] >> 16);
            v[2 * k] = DT == NORI_F16 ? f16_to_f32(lo) : bf16_to_f32(lo);
            v[2 * k + 1] = DT == NORI_F16 ? f16_to_f32(hi) : bf16_to_f32(hi);
        }
    }
}

template <int DT>
__device__ __forceinline__ void store4(void* p, int64_t i, const float (&v)[4]) {
    if constexpr (DT == NORI_F32) {
        *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(p) + i) = f32x4{v[0], v[1], v[2], v[3]};
    } else {
        u32x2 c;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const uint32_t lo = DT == NORI_F16 ? f32_to_f16(v[2 * k]) : f32_to_bf16(v[2 * k]);
            const uint32_t hi = DT == NORI_F16 ? f32_to_f16(v[2 * k + 1]) : f32_to_bf16(v[2 * k + 1]);
            c[k] = lo | (hi << 16);
        }
        *reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(p) + i) = c;
    }
}

// sum over the G lanes of a group (G a power of two, groups aligned in the wavefront)
template <int G>
__device__ __forceinline__ float group_sum(float s) {
#pragma unroll
    for (int off = G / 2; off > 0; off >>= 1) s += __shfl_xor(s, off, G);
    return s;
}

// (v - mean) * rstd (* w + b), then the ReLU
__device__ __forceinline__ void finish(float (&v)[4], float mean, float rstd, const float* w, const float* b, int c0,
                                       bool relu) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        float o = (v[k] - mean) * rstd;
        if (w) o = o * w[c0 + k];
        if (b) o = o + b[c0 + k];
        v[k] = relu ? (o < 0.0f ? 0.0f : o) : o;  // NaN passes through, as torch.relu keeps it
    }
}

template <int XDT, int YDT, int G>
__global__ void __launch_bounds__(kThreads)
layer_norm_group_kernel(const void* x, int64_t rows, int cols, int64_t xs, const float* w, const float* b, float eps,
                        int relu, void* y, int64_t ys) {
    const int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    const int64_t row = t / G;
    const int c0 = 4 * (int)(t % G);
    const bool ok = row < rows;  // every lane joins the shuffles
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    if (ok) load4<XDT>(x, row * xs + c0, v);
    const float inv_n = 1.0f / (float)cols;
    const float mean = group_sum<G>((v[0] + v[1]) + (v[2] + v[3])) * inv_n;
    float d2 = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) d2 += (v[k] - mean) * (v[k] - mean);
    const float var = group_sum<G>(d2) * inv_n;
    const float rstd = rsqrtf(var + eps);
    finish(v, mean, rstd, w, b, c0, relu != 0);
    if (ok) store4<YDT>(y, row * ys + c0, v);
}

// one wavefront per row of any width that is a multiple of 4
template <int XDT, int YDT>
__global__ void __launch_bounds__(kThreads)
layer_norm_row_kernel(const void* x, int64_t rows, int cols, int64_t xs, const float* w, const float* b, float eps,
                      int relu, void* y, int64_t ys) {
    const int64_t row = (int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;  // whole wavefronts
    const float inv_n = 1.0f / (float)cols;
    float s = 0.f;
    for (int c = 4 * lane; c < cols; c += 256) {
        float v[4];
        load4<XDT>(x, row * xs + c, v);
        s += (v[0] + v[1]) + (v[2] + v[3]);
    }
    const float mean = group_sum<64>(s) * inv_n;
    float d2 = 0.f;
    for (int c = 4 * lane; c < cols; c += 256) {
        float v[4];
        load4<XDT>(x, row * xs + c, v);
#pragma unroll
        for (int k = 0; k < 4; ++k) d2 += (v[k] - mean) * (v[k] - mean);
    }
    const float rstd = rsqrtf(group_sum<64>(d2) * inv_n + eps);
    for (int c = 4 * lane; c < cols; c += 256) {
        float v[4];
        load4<XDT>(x, row * xs + c, v);
        finish(v, mean, rstd, w, b, c, relu != 0);
        store4<YDT>(y, row * ys + c, v);
    }
}

// The cell encoder's last LayerNorm with the two additions that follow it in the two-phase
// forward: the feature positional embedding of the cell's group and the target-aware row
// bias (transformer.py apply_feature_positional_embeddings / apply_target_aware_embedding).
// A group of G lanes owns a row (b, s, g) as in layer_norm_group_kernel (same arithmetic
// for the norm); rows are walked in a grid-stride loop.
struct CellsArgs {
    const void* x;
    int64_t rows, rows_per_table, groups, xs;  // rows = tables * rows_per_table * groups
    const float* w;
    const float* b;
    float eps;
    const float* pos;    // [groups][cols] or null
    const float* ctx;    // [tables][eval_pos][cols] or null
    int64_t eval_pos;
    const float* alpha;  // device scalar (the gated mix) or null (plain row bias)
    float inv_sqrt_e;
    float* y;
};

template <int XDT, int G>
__global__ void __launch_bounds__(kThreads) layer_norm_cells_kernel(const CellsArgs a) {
    constexpr int cols = 4 * G;
    const int c0 = 4 * (threadIdx.x % G);
    const float inv_n = 1.0f / (float)cols;
    const float alpha = a.alpha ? *a.alpha : 0.0f;
    const float one_minus = 1.0f - alpha;
    float w[4], bb[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        w[k] = a.w ? a.w[c0 + k] : 1.0f;
        bb[k] = a.b ? a.b[c0 + k] : 0.0f;
    }
    const int64_t per = kThreads / G;
    const int64_t first = (int64_t)blockIdx.x * per + threadIdx.x / G, step = (int64_t)gridDim.x * per;
    const int64_t iters = (a.rows + step - 1) / step;  // the same for every lane: the shuffles stay uniform
    for (int64_t it = 0; it < iters; ++it) {
        const int64_t row = first + it * step;
        const bool ok = row < a.rows;
        float v[4] = {0.f, 0.f, 0.f, 0.f};
        if (ok) load4<XDT>(a.x, row * a.xs + c0, v);
        const float mean = group_sum<G>((v[0] + v[1]) + (v[2] + v[3])) * inv_n;
        float d2 = 0.f;
#pragma unroll
        for (int k = 0; k < 4; ++k) d2 += (v[k] - mean) * (v[k] - mean);
        const float rstd = rsqrtf(group_sum<G>(d2) * inv_n + a.eps);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            float o = (v[k] - mean) * rstd;
            o = o * w[k];
            v[k] = o + bb[k];
        }
        const int64_t rr = ok ? row : 0;
        const int64_t g = rr % a.groups, ts = rr / a.groups;  // (table, row) of the cell
        const int64_t t = ts / a.rows_per_table, s = ts % a.rows_per_table;
        if (a.pos) {
#pragma unroll
            for (int k = 0; k < 4; ++k) v[k] = v[k] + a.pos[g * cols + c0 + k];
        }
        if (a.ctx) {
            float rb[4] = {0.f, 0.f, 0.f, 0.f};
            if (s < a.eval_pos) {
                const f32x4 c = *reinterpret_cast<const f32x4*>(a.ctx + (t * a.eval_pos + s) * cols + c0);
                rb[0] = c[0]; rb[1] = c[1]; rb[2] = c[2]; rb[3] = c[3];
            }
            if (a.alpha) {
                float dot = 0.f;
#pragma unroll
                for (int k = 0; k < 4; ++k) dot += v[k] * rb[k];
                const float z = group_sum<G>(dot) * a.inv_sqrt_e;
                const float gate = 1.0f / (1.0f + expf(-z));
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const float lhs = v[k] + one_minus * rb[k];
                    v[k] = lhs + alpha * (rb[k] * gate);
                }
            } else {
#pragma unroll
                for (int k = 0; k < 4; ++k) v[k] = v[k] + rb[k];
            }
        }
        if (ok) *reinterpret_cast<f32x4*>(a.y + row * cols + c0) = f32x4{v[0], v[1], v[2], v[3]};
    }
}

template <int XDT, int YDT>
void launch(const void* x, int64_t rows, int cols, int64_t xs, const float* w, const float* b, float eps, int relu,
            void* y, int64_t ys, hipStream_t stream) {
    const int g = cols / 4;
    auto grouped = [&](auto G_) {
        constexpr int G = decltype(G_)::value;
        const dim3 grid((unsigned)((rows * G + kThreads - 1) / kThreads));
        hipLaunchKernelGGL((layer_norm_group_kernel<XDT, YDT, G>), grid, dim3(kThreads), 0, stream, x, rows, cols, xs, w, b,
                           eps, relu, y, ys);
    };
    switch (g) {
        case 1: grouped(std::integral_constant<int, 1>{}); return;
        case 2: grouped(std::integral_constant<int, 2>{}); return;
        case 4: grouped(std::integral_constant<int, 4>{}); return;
        case 8: grouped(std::integral_constant<int, 8>{}); return;
        case 16: grouped(std::integral_constant<int, 16>{}); return;
        case 32: grouped(std::integral_constant<int, 32>{}); return;
        case 64: grouped(std::integral_constant<int, 64>{}); return;
        default: break;
    }
    const dim3 grid((unsigned)((rows + kThreads / 64 - 1) / (kThreads / 64)));
    hipLaunchKernelGGL((layer_norm_row_kernel<XDT, YDT>), grid, dim3(kThreads), 0, stream, x, rows, cols, xs, w, b, eps,
                       relu, y, ys);
}

}  // namespace

extern "C" int nori_layer_norm(const void* x, int x_dtype, int64_t rows, int32_t cols, int64_t x_row_stride,
                               const float* weight, const float* bias, float eps, int relu, void* y, int y_dtype,
                               int64_t y_row_stride, void* stream_v) {
    clear_error();
    auto is_float = [](int dt) { return dt == NORI_F32 || dt == NORI_F16 || dt == NORI_BF16; };
    if (!is_float(x_dtype) || !is_float(y_dtype))
        return fail(NORI_ERR_UNSUPPORTED, "layer_norm: unsupported dtypes %s -> %s", dtype_name(x_dtype), dtype_name(y_dtype));
    if (rows < 0 || cols <= 0 || cols % 4 != 0)
        return fail(NORI_ERR_INVALID, "layer_norm: bad shape (%lld rows of %d; the width must be a multiple of 4)",
                    (long long)rows, cols);
    if (x_row_stride < cols || y_row_stride < cols || x_row_stride % 4 != 0 || y_row_stride % 4 != 0)
        return fail(NORI_ERR_INVALID, "layer_norm: row strides (%lld, %lld) must be multiples of 4 and at least %d",
                    (long long)x_row_stride, (long long)y_row_stride, cols);
    if (!(eps >= 0.0f)) return fail(NORI_ERR_INVALID, "layer_norm: eps must be a non-negative number");
    if (rows == 0) return NORI_OK;
    if (!x || !y) return fail(NORI_ERR_INVALID, "layer_norm: null pointer");
    if ((uintptr_t)x % (4 * dtype_size(x_dtype)) || (uintptr_t)y % (4 * dtype_size(y_dtype)))
        return fail(NORI_ERR_INVALID, "layer_norm: x and y must be aligned to 4 elements");
    if (rows > (int64_t)0x7fffffff * kThreads / 64) return fail(NORI_ERR_UNSUPPORTED, "layer_norm: too many rows");
    hipStream_t stream = (hipStream_t)stream_v;
    NORI_DISPATCH_FLOAT(x_dtype, XDT, {
        NORI_DISPATCH_FLOAT(y_dtype, YDT, {
            launch<XDT, YDT>(x, rows, cols, x_row_stride, weight, bias, eps, relu, y, y_row_stride, stream);
        });
    });
    return launch_status("layer_norm");
}

extern "C" int nori_layer_norm_cells(const void* x, int x_dtype, int64_t tables, int64_t rows, int64_t groups,
                                     int32_t cols, int64_t x_row_stride, const float* weight, const float* bias,
                                     float eps, const float* pos, const float* ctx, int64_t eval_pos,
                                     const float* alpha, float inv_sqrt_e, float* y, void* stream_v) {
    clear_error();
    if (x_dtype != NORI_F32 && x_dtype != NORI_F16)
        return fail(NORI_ERR_UNSUPPORTED, "layer_norm_cells: unsupported input dtype %s", dtype_name(x_dtype));
    if (tables < 0 || rows < 0 || groups <= 0 || eval_pos < 0 || eval_pos > rows)
        return fail(NORI_ERR_INVALID, "layer_norm_cells: bad shape %lld x %lld x %lld, eval_pos %lld",
                    (long long)tables, (long long)rows, (long long)groups, (long long)eval_pos);
    if (cols != 64 && cols != 128 && cols != 256)
        return fail(NORI_ERR_UNSUPPORTED, "layer_norm_cells: width %d (64, 128 or 256 are built)", cols);
    if (!(eps >= 0.0f)) return fail(NORI_ERR_INVALID, "layer_norm_cells: eps must be a non-negative number");
    if (tables == 0 || rows == 0) return NORI_OK;
    if (!x || !y) return fail(NORI_ERR_INVALID, "layer_norm_cells: null pointer");
    if (x_row_stride < cols || x_row_stride % 4 || (uintptr_t)x % (4 * dtype_size(x_dtype)) || (uintptr_t)y % 16 ||
        (ctx && (uintptr_t)ctx % 16))
        return fail(NORI_ERR_INVALID, "layer_norm_cells: rows must be aligned to 4 elements (y and ctx to 16 bytes)");
    CellsArgs a;
    a.x = x;
    a.rows = tables * rows * groups;
    a.rows_per_table = rows;
    a.groups = groups;
    a.xs = x_row_stride;
    a.w = weight;
    a.b = bias;
    a.eps = eps;
    a.pos = pos;
    a.ctx = ctx;
    a.eval_pos = eval_pos;
    a.alpha = alpha;
    a.inv_sqrt_e = inv_sqrt_e;
    a.y = y;
    const int g = cols / 4;
    const int64_t need = (a.rows * g + kThreads - 1) / kThreads;
    const unsigned grid = (unsigned)std::min<int64_t>(need, (int64_t)device_cus() * 16);
    hipStream_t stream = (hipStream_t)stream_v;
    auto go = [&](auto G_) {
        constexpr int G = decltype(G_)::value;
        if (x_dtype == NORI_F16)
            hipLaunchKernelGGL((layer_norm_cells_kernel<NORI_F16, G>), dim3(grid), dim3(kThreads), 0, stream, a);
        else
            hipLaunchKernelGGL((layer_norm_cells_kernel<NORI_F32, G>), dim3(grid), dim3(kThreads), 0, stream, a);
    };
    if (g == 16) go(std::integral_constant<int, 16>{});
    else if (g == 32) go(std::integral_constant<int, 32>{});
    else go(std::integral_constant<int, 64>{});
    return launch_status("layer_norm_cells");
}
