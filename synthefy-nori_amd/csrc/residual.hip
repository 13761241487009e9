// Deep-norm residual update out = x + alpha * u for an fp32 residual stream x and a sublayer
// output u (fp16, bf16 or fp32), with torch's rounding of the expression `x + alpha * u`
// (src/synthefy_nori/model/two_phase.py:198, 209, 220-225, 264, 271-272): the
// product is formed in fp32 and rounded to u's dtype, then added to x in fp32. One pass
// reading x and u and writing out, instead of a pass for the product and one for the sum.
#include "nori_common.h"

// each op rounds separately, as torch's do
#pragma clang fp contract(off)

namespace {

using namespace nori;

constexpr int kThreads = 256;

template <int UT>
__device__ __forceinline__ float scaled(float u, float alpha) {
    return round_to<UT>(u * alpha);
}

// 4 elements per thread: one 16-byte load of x, a 16- or 8-byte load of u, one 16-byte store.
template <int UT>
__global__ void __launch_bounds__(kThreads)
residual_add_vec_kernel(const float* x, const void* u, float alpha, int64_t n4, float* out) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= n4) return;
    const f32x4 xv = reinterpret_cast<const f32x4*>(x)[i];
    float uv[4];
    if constexpr (UT == NORI_F32) {
        const f32x4 w = reinterpret_cast<const f32x4*>(u)[i];
#pragma unroll
        for (int e = 0; e < 4; ++e) uv[e] = w[e];
    } else {
        const uint2 w = reinterpret_cast<const uint2*>(u)[i];
        const uint32_t h[2] = {w.x, w.y};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint16_t b = (uint16_t)(h[e >> 1] >> (16 * (e & 1)));
            uv[e] = UT == NORI_F16 ? f16_to_f32(b) : bf16_to_f32(b);
        }
    }
    f32x4 r;
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = xv[e] + scaled<UT>(uv[e], alpha);
    reinterpret_cast<f32x4*>(out)[i] = r;
}

// Any alignment and length: one element per thread.
template <int UT>
__global__ void __launch_bounds__(kThreads)
residual_add_kernel(const float* x, const void* u, float alpha, int64_t n, float* out) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= n) return;
    out[i] = x[i] + scaled<UT>(load_elem<UT>(u, i), alpha);
}

template <int UT>
int launch(const float* x, const void* u, float alpha, int64_t n, float* out, hipStream_t stream) {
    const int us = UT == NORI_F32 ? 4 : 2;
    const bool vec = n % 4 == 0 && (uintptr_t)x % 16 == 0 && (uintptr_t)out % 16 == 0 && (uintptr_t)u % (4 * us) == 0;
    const int64_t items = vec ? n / 4 : n;
    const int64_t blocks = (items + kThreads - 1) / kThreads;
    if (blocks > 0x7fffffffLL) return fail(NORI_ERR_UNSUPPORTED, "residual_add: %lld elements exceed one launch", (long long)n);
    if (vec)
        hipLaunchKernelGGL((residual_add_vec_kernel<UT>), dim3((unsigned)blocks), dim3(kThreads), 0, stream, x, u, alpha, items, out);
    else
        hipLaunchKernelGGL((residual_add_kernel<UT>), dim3((unsigned)blocks), dim3(kThreads), 0, stream, x, u, alpha, items, out);
    return launch_status("residual_add");
}

}  // namespace

extern "C" int nori_residual_add(const float* x, const void* u, int u_dtype, float alpha, int64_t n, float* out,
                                 void* stream_v) {
    clear_error();
    if (n < 0) return fail(NORI_ERR_INVALID, "residual_add: negative length %lld", (long long)n);
    if (u_dtype != NORI_F32 && u_dtype != NORI_F16 && u_dtype != NORI_BF16)
        return fail(NORI_ERR_UNSUPPORTED, "residual_add: unsupported update dtype %s", dtype_name(u_dtype));
    if (n == 0) return NORI_OK;
    if (!x || !u || !out) return fail(NORI_ERR_INVALID, "residual_add: null pointer");
    hipStream_t stream = (hipStream_t)stream_v;
    if (u_dtype == NORI_F16) return launch<NORI_F16>(x, u, alpha, n, out, stream);
    if (u_dtype == NORI_BF16) return launch<NORI_BF16>(x, u, alpha, n, out, stream);
    return launch<NORI_F32>(x, u, alpha, n, out, stream);
}
