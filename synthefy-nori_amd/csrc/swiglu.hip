// SwiGLU gate of the feed-forward sublayers: out = silu(g) * u for the [gate | up] output of
// one fused projection (SwiGLUMLP.forward, src/synthefy_nori/model/layer.py:261-274, whose
// gate and up projections read the same operand). Rounded as torch rounds the two ops in the
// projection's dtype T: silu in fp32 (x / (1 + exp(-x))) rounded to T, the product of the two
// T values in fp32 rounded to T. One pass reading 2h and writing h elements per row, instead
// of silu's read and write and the product's two reads and one write.
#include <math.h>

#include "nori_common.h"

// each op rounds separately, as torch's do
#pragma clang fp contract(off)

namespace {

using namespace nori;

constexpr int kThreads = 256;

template <int DT>
__device__ __forceinline__ float gate(float g, float u) {
    const float s = round_to<DT>(g / (1.0f + expf(-g)));
    return s * u;
}

// W elements of one row per thread (hidden % W == 0, rows and pointers 16-byte aligned: W = 8
// for 16-bit types, 4 for fp32): one 16-byte load of g and of u, one 16-byte store. The row
// is found by a 32-bit division (the launch keeps rows * hidden / W below 2^31).
template <int DT>
__global__ void __launch_bounds__(kThreads)
silu_mul_vec_kernel(const void* gu, int64_t rows, int32_t hidden, int64_t row_stride, void* out, int64_t out_stride) {
    constexpr int W = DT == NORI_F32 ? 4 : 8;
    const uint32_t per_row = (uint32_t)hidden / W;
    const uint32_t i = blockIdx.x * kThreads + threadIdx.x;
    if ((int64_t)i >= rows * per_row) return;
    const uint32_t r = i / per_row;
    const int c = W * (int)(i - r * per_row);
    const int64_t g0 = (int64_t)r * row_stride + c, u0 = g0 + hidden, o0 = (int64_t)r * out_stride + c;
    if constexpr (DT == NORI_F32) {
        const f32x4 g = *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(gu) + g0);
        const f32x4 u = *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(gu) + u0);
        f32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = gate<DT>(g[e], u[e]);
        *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(out) + o0) = o;
    } else {
        const uint4 gw = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(gu) + g0);
        const uint4 uw = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(gu) + u0);
        const uint32_t gh[4] = {gw.x, gw.y, gw.z, gw.w}, uh[4] = {uw.x, uw.y, uw.z, uw.w};
        uint32_t oh[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint16_t gb = (uint16_t)(gh[e >> 1] >> (16 * (e & 1)));
            const uint16_t ub = (uint16_t)(uh[e >> 1] >> (16 * (e & 1)));
            const float g = DT == NORI_F16 ? f16_to_f32(gb) : bf16_to_f32(gb);
            const float u = DT == NORI_F16 ? f16_to_f32(ub) : bf16_to_f32(ub);
            const float o = gate<DT>(g, u);
            const uint32_t ob = DT == NORI_F16 ? f32_to_f16(o) : f32_to_bf16(o);
            oh[e >> 1] |= ob << (16 * (e & 1));
        }
        *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(out) + o0) = uint4{oh[0], oh[1], oh[2], oh[3]};
    }
}

// Any width and alignment: a block covers whole rows, a thread walks its row's elements.
template <int DT>
__global__ void __launch_bounds__(kThreads)
silu_mul_kernel(const void* gu, int64_t rows, int32_t hidden, int64_t row_stride, void* out, int64_t out_stride) {
    const int64_t r = blockIdx.x;
    if (r >= rows) return;
    for (int c = threadIdx.x; c < hidden; c += kThreads) {
        const float g = load_elem<DT>(gu, r * row_stride + c);
        const float u = load_elem<DT>(gu, r * row_stride + hidden + c);
        store_elem<DT>(out, r * out_stride + c, gate<DT>(g, u));
    }
}

}  // namespace

extern "C" int nori_silu_mul(const void* gu, int dtype, int64_t rows, int32_t hidden, int64_t row_stride, void* out,
                             int64_t out_row_stride, void* stream_v) {
    clear_error();
    if (rows < 0 || hidden <= 0)
        return fail(NORI_ERR_INVALID, "silu_mul: bad shape (%lld rows of %d)", (long long)rows, hidden);
    if (dtype != NORI_F32 && dtype != NORI_F16 && dtype != NORI_BF16)
        return fail(NORI_ERR_UNSUPPORTED, "silu_mul: unsupported dtype %s", dtype_name(dtype));
    if (row_stride < 2 * (int64_t)hidden || out_row_stride < hidden)
        return fail(NORI_ERR_INVALID, "silu_mul: row strides (%lld, %lld) below the row widths (%d, %d)",
                    (long long)row_stride, (long long)out_row_stride, 2 * hidden, hidden);
    if (rows == 0) return NORI_OK;
    if (!gu || !out) return fail(NORI_ERR_INVALID, "silu_mul: null pointer");
    hipStream_t stream = (hipStream_t)stream_v;
    const int w = dtype == NORI_F32 ? 4 : 8;
    const bool vec = hidden % w == 0 && row_stride % w == 0 && out_row_stride % w == 0 && (uintptr_t)gu % 16 == 0 &&
                     (uintptr_t)out % 16 == 0 && rows * (hidden / w) < 0x7fffffffLL;
    if (!vec && rows > 0x7fffffffLL) return fail(NORI_ERR_UNSUPPORTED, "silu_mul: too many rows");
    const dim3 grid(vec ? (unsigned)((rows * (hidden / w) + kThreads - 1) / kThreads) : (unsigned)rows);
    NORI_DISPATCH_FLOAT(dtype, DT, {
        if (vec) hipLaunchKernelGGL(silu_mul_vec_kernel<DT>, grid, dim3(kThreads), 0, stream, gu, rows, hidden, row_stride, out, out_row_stride);
        else hipLaunchKernelGGL(silu_mul_kernel<DT>, grid, dim3(kThreads), 0, stream, gu, rows, hidden, row_stride, out, out_row_stride);
    });
    return launch_status("silu_mul");
}
