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
