// RMSNorm for gfx950: y = x * rsqrt(mean(x^2) + eps) (* w), rows of `cols` elements.
//
// Semantics: RMSNorm.forward with use_native=True, i.e. torch.nn.functional.rms_norm
// (src/synthefy_nori/model/layer.py:251-253): the mean of squares and the product are
// formed in fp32 and the result is rounded once to the input dtype (then multiplied by
// the weight when one is given).
//
// Schedule. HBM-bound: each row is read once and written once. A group of G lanes
// (G = the power of two covering the row's 16-byte chunks, at most 64) owns one row:
// every lane loads 16-byte chunks, accumulates x^2 in fp32, the group reduces with
// lane shuffles, and the same registers are scaled and stored. A 128-wide bf16 row
// is 16 chunks, so one wavefront normalizes 4 rows per pass. Rows whose length or
// alignment does not allow 16-byte chunks use an element-wise kernel.
#include "nori_common.h"

// torch rounds the result of every op separately; no multiply-add is fused here unless
// the source writes fmaf. (Narrowing conversions are kept apart by pin_f32.)
#pragma clang fp contract(off)

namespace {

using namespace nori;

constexpr int kThreads = 256;
constexpr int kMaxChunksPerLane = 4;  // rows up to 64*4 chunks = 4 KiB on the chunked path

template <int DT>
__device__ __forceinline__ void unpack_chunk(const uint4& c, float* f) {
    if constexpr (DT == NORI_F32) {
        f[0] = __uint_as_float(c.x); f[1] = __uint_as_float(c.y);
        f[2] = __uint_as_float(c.z); f[3] = __uint_as_float(c.w);
    } else {
        const uint32_t w[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            if constexpr (DT == NORI_F16) {
                f[2 * k] = f16_to_f32((uint16_t)(w[k] & 0xffff));
                f[2 * k + 1] = f16_to_f32((uint16_t)(w[k] >> 16));
            } else {
                f[2 * k] = __uint_as_float(w[k] << 16);
                f[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
            }
        }
    }
}

template <int DT>
__device__ __forceinline__ uint4 pack_chunk(const float* f) {
    uint4 c;
    if constexpr (DT == NORI_F32) {
        c.x = __float_as_uint(f[0]); c.y = __float_as_uint(f[1]);
        c.z = __float_as_uint(f[2]); c.w = __float_as_uint(f[3]);
    } else {
        uint32_t w[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            uint32_t lo, hi;
            if constexpr (DT == NORI_F16) { lo = f32_to_f16(f[2 * k]); hi = f32_to_f16(f[2 * k + 1]); }
            else { lo = f32_to_bf16(f[2 * k]); hi = f32_to_bf16(f[2 * k + 1]); }
            w[k] = lo | (hi << 16);
        }
        c.x = w[0]; c.y = w[1]; c.z = w[2]; c.w = w[3];
    }
    return c;
}

// The EPC outputs of one chunk, rounded to DT (the norm's result dtype) and stored as OT: a
// 16-byte store when OT is DT, 8 bytes for an fp32 row written as fp16/bf16 (the cast an
// autocast projection applies to the fp32 result, bit for bit).
template <int DT, int OT, int EPC>
__device__ __forceinline__ void store_chunk(uint8_t* p, const float* o) {
    if constexpr (OT == DT) {
        *reinterpret_cast<uint4*>(p) = pack_chunk<DT>(o);
    } else {
        static_assert(DT == NORI_F32 && EPC == 4, "narrowing stores are from fp32 rows");
        uint2 c;
        uint16_t h[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) h[e] = OT == NORI_F16 ? f32_to_f16(o[e]) : f32_to_bf16(o[e]);
        c.x = h[0] | ((uint32_t)h[1] << 16);
        c.y = h[2] | ((uint32_t)h[3] << 16);
        *reinterpret_cast<uint2*>(p) = c;
    }
}

// G lanes per row; rows_per_block = kThreads / G. A row's lanes load all of it before the
// reduction and store after it, so y may be x (in place; no restrict qualifiers).
template <int DT, int WDT, int OT, int G>
__global__ void __launch_bounds__(kThreads)
rms_norm_chunked_kernel(const uint8_t* x, int64_t rows, int cols, int64_t x_row_bytes,
                        const void* w, float eps, uint8_t* y, int64_t y_row_bytes) {
    constexpr int EPC = 16 / (DT == NORI_F32 ? 4 : 2);  // elements per 16-byte chunk
    constexpr int OUT_CHUNK = EPC * (OT == NORI_F32 ? 4 : 2);  // bytes of one chunk's outputs
    const int lane_in_row = threadIdx.x % G;
    const int64_t row = (int64_t)blockIdx.x * (kThreads / G) + threadIdx.x / G;
    const int nchunks = cols / EPC;
    const bool active = row < rows;
    float v[kMaxChunksPerLane][EPC];
    float acc = 0.0f;
#pragma unroll
    for (int k = 0; k < kMaxChunksPerLane; ++k) {
        const int ch = lane_in_row + k * G;
        if (active && ch < nchunks) {
            const uint4 c = *reinterpret_cast<const uint4*>(x + row * x_row_bytes + (int64_t)ch * 16);
            unpack_chunk<DT>(c, v[k]);
#pragma unroll
            for (int e = 0; e < EPC; ++e) acc = fmaf(v[k][e], v[k][e], acc);
        }
    }
#pragma unroll
    for (int off = G / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off, G);
    const float inv = rsqrtf(acc / (float)cols + eps);
#pragma unroll
    for (int k = 0; k < kMaxChunksPerLane; ++k) {
        const int ch = lane_in_row + k * G;
        if (active && ch < nchunks) {
            float o[EPC];
#pragma unroll
            for (int e = 0; e < EPC; ++e) {
                o[e] = round_to<DT>(v[k][e] * inv);
                if (w) o[e] = o[e] * load_elem<WDT>(w, (int64_t)ch * EPC + e);
            }
            store_chunk<DT, OT, EPC>(y + row * y_row_bytes + (int64_t)ch * OUT_CHUNK, o);
        }
    }
}

// One wavefront per row, element-wise loads: any width and alignment. Each element is read
// and then written by the same lane, so y may be x.
template <int DT, int WDT, int OT>
__global__ void __launch_bounds__(kThreads)
rms_norm_elementwise_kernel(const void* x, int64_t rows, int cols, int64_t x_row_stride,
                            const void* w, float eps, void* y, int64_t y_row_stride) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * (kThreads / 64) + threadIdx.x / 64;
    if (row >= rows) return;
    float acc = 0.0f;
    for (int c = lane; c < cols; c += 64) {
        const float v = load_elem<DT>(x, row * x_row_stride + c);
        acc = fmaf(v, v, acc);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
    const float inv = rsqrtf(acc / (float)cols + eps);
    for (int c = lane; c < cols; c += 64) {
        float o = round_to<DT>(load_elem<DT>(x, row * x_row_stride + c) * inv);
        if (w) o = o * load_elem<WDT>(w, c);
        store_elem<OT>(y, row * y_row_stride + c, round_to<DT>(o));
    }
}

// The deep-norm residual update and the RMSNorm that reads its result, in one pass over an fp32
// residual stream of rows x cols: xo = x + RN_UT(alpha * u) (nori_residual_add's rounding), then
// y = rms_norm(xo) written as OT. The statistic is formed by the same G lanes, chunk order and
// shuffles as rms_norm_chunked_kernel<NORI_F32, *, OT, G>, so y equals that kernel run on xo, bit
// for bit. Row r of y starts at byte (r / y_group) * y_group_bytes + (r % y_group) * y_row_bytes
// (rows of a token buffer that interleaves several streams). Row r of u, with r = (i0 * u_d1 + i1) *
// u_d2 + i2, starts at element i0 * u_s0 + i1 * u_s1 + i2 * u_s2 (a transposed update, e.g. a
// column attention's [batch, groups, rows] output added to a [batch, rows, groups] stream).
// xo may be x.
struct UpdateRows {
    int64_t d1, d2, s0, s1, s2;  // row r -> (r / (d1 d2), (r / d2) % d1, r % d2) at these strides
};

template <int UT, int OT, int G>
__global__ void __launch_bounds__(kThreads)
residual_rms_norm_kernel(const float* x, const void* u, UpdateRows ur, float alpha, int64_t rows, int cols, float eps,
                         float* xo, uint8_t* y, int64_t y_group, int64_t y_group_bytes, int64_t y_row_bytes) {
    constexpr int EPC = 4;
    constexpr int OUT_CHUNK = EPC * (OT == NORI_F32 ? 4 : 2);
    const int lane_in_row = threadIdx.x % G;
    const int64_t row = (int64_t)blockIdx.x * (kThreads / G) + threadIdx.x / G;
    const int nchunks = cols / EPC;
    const bool active = row < rows;
    float v[kMaxChunksPerLane][EPC];
    float acc = 0.0f;
    int64_t u_row = 0;
    if (active) {
        const int64_t t = row / ur.d2;
        u_row = (t / ur.d1) * ur.s0 + (t % ur.d1) * ur.s1 + (row % ur.d2) * ur.s2;
    }
#pragma unroll
    for (int k = 0; k < kMaxChunksPerLane; ++k) {
        const int ch = lane_in_row + k * G;
        if (active && ch < nchunks) {
            const int64_t at = row * cols + (int64_t)ch * EPC;
            const int64_t u_at = u_row + (int64_t)ch * EPC;
            const f32x4 xv = *reinterpret_cast<const f32x4*>(x + at);
            float uv[EPC];
            if constexpr (UT == NORI_F32) {
                const f32x4 w = *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(u) + u_at);
#pragma unroll
                for (int e = 0; e < EPC; ++e) uv[e] = w[e];
            } else {
                const uint2 w = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(u) + u_at);
                const uint32_t h[2] = {w.x, w.y};
#pragma unroll
                for (int e = 0; e < EPC; ++e) {
                    const uint16_t b = (uint16_t)(h[e >> 1] >> (16 * (e & 1)));
                    uv[e] = UT == NORI_F16 ? f16_to_f32(b) : bf16_to_f32(b);
                }
            }
            f32x4 r;
#pragma unroll
            for (int e = 0; e < EPC; ++e) {
                v[k][e] = xv[e] + round_to<UT>(uv[e] * alpha);
                r[e] = v[k][e];
            }
            *reinterpret_cast<f32x4*>(xo + at) = r;
#pragma unroll
            for (int e = 0; e < EPC; ++e) acc = fmaf(v[k][e], v[k][e], acc);
        }
    }
#pragma unroll
    for (int off = G / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off, G);
    const float inv = rsqrtf(acc / (float)cols + eps);
    const int64_t y_at = active ? (row / y_group) * y_group_bytes + (row % y_group) * y_row_bytes : 0;
#pragma unroll
    for (int k = 0; k < kMaxChunksPerLane; ++k) {
        const int ch = lane_in_row + k * G;
        if (active && ch < nchunks) {
            float o[EPC];
#pragma unroll
            for (int e = 0; e < EPC; ++e) o[e] = v[k][e] * inv;
            store_chunk<NORI_F32, OT, EPC>(y + y_at + (int64_t)ch * OUT_CHUNK, o);
        }
    }
}

template <int DT, int WDT, int OT>
int launch(const void* x, int64_t rows, int cols, int64_t xs, const void* w, float eps, void* y, int64_t ys,
           hipStream_t stream) {
    constexpr int es = (DT == NORI_F32) ? 4 : 2;
    constexpr int os = (OT == NORI_F32) ? 4 : 2;
    constexpr int EPC = 16 / es;
    constexpr int OUT_CHUNK = EPC * os;
    const bool aligned = ((uintptr_t)x % 16 == 0) && ((uintptr_t)y % OUT_CHUNK == 0) && ((xs * es) % 16 == 0) &&
                         ((ys * os) % OUT_CHUNK == 0) && (cols % EPC == 0);
    const int nchunks = cols / EPC;
    if (aligned && nchunks <= 64 * kMaxChunksPerLane) {
        int g = 1;
        while (g < nchunks && g < 64) g <<= 1;
        const int rows_per_block = kThreads / g;
        const unsigned grid = (unsigned)((rows + rows_per_block - 1) / rows_per_block);
#define NORI_RMS_CASE(GV)                                                                                     \
    case GV:                                                                                                   \
        hipLaunchKernelGGL((rms_norm_chunked_kernel<DT, WDT, OT, GV>), dim3(grid), dim3(kThreads), 0, stream,   \
                           (const uint8_t*)x, rows, cols, xs * es, w, eps, (uint8_t*)y, ys * os);              \
        break;
        switch (g) {
            NORI_RMS_CASE(1) NORI_RMS_CASE(2) NORI_RMS_CASE(4) NORI_RMS_CASE(8)
            NORI_RMS_CASE(16) NORI_RMS_CASE(32) NORI_RMS_CASE(64)
        }
#undef NORI_RMS_CASE
    } else {
        const unsigned grid = (unsigned)((rows + (kThreads / 64) - 1) / (kThreads / 64));
        hipLaunchKernelGGL((rms_norm_elementwise_kernel<DT, WDT, OT>), dim3(grid), dim3(kThreads), 0, stream, x, rows,
                           cols, xs, w, eps, y, ys);
    }
    return launch_status("rms_norm");
}

}  // namespace

extern "C" int nori_rms_norm_to(const void* x, int dtype, int64_t rows, int32_t cols, int64_t x_row_stride,
                                const void* weight, int weight_dtype, float eps, void* y, int y_dtype,
                                int64_t y_row_stride, void* stream_v) {
    clear_error();
    if (y_dtype != dtype && !(dtype == NORI_F32 && (y_dtype == NORI_F16 || y_dtype == NORI_BF16)))
        return fail(NORI_ERR_UNSUPPORTED, "rms_norm: %s rows cannot be written as %s (fp32 rows may be written as "
                    "fp16 or bf16)", dtype_name(dtype), dtype_name(y_dtype));
    if (rows < 0 || cols <= 0) return fail(NORI_ERR_INVALID, "rms_norm: bad shape rows=%lld cols=%d", (long long)rows, cols);
    if (dtype != NORI_F32 && dtype != NORI_F16 && dtype != NORI_BF16)
        return fail(NORI_ERR_UNSUPPORTED, "rms_norm: unsupported dtype %s", dtype_name(dtype));
    if (weight && weight_dtype != NORI_F32 && weight_dtype != NORI_F16 && weight_dtype != NORI_BF16)
        return fail(NORI_ERR_UNSUPPORTED, "rms_norm: unsupported weight dtype %s", dtype_name(weight_dtype));
    if (rows == 0) return NORI_OK;
    if (!x || !y) return fail(NORI_ERR_INVALID, "rms_norm: null pointer");
    if (!weight) weight_dtype = dtype;
    hipStream_t stream = (hipStream_t)stream_v;
    int st = NORI_OK;
    if (y_dtype == dtype) {
        NORI_DISPATCH_FLOAT(dtype, DT,
            NORI_DISPATCH_FLOAT(weight_dtype, WDT,
                st = launch<DT, WDT, DT>(x, rows, cols, x_row_stride, weight, eps, y, y_row_stride, stream)));
    } else if (y_dtype == NORI_F16) {
        NORI_DISPATCH_FLOAT(weight_dtype, WDT,
            st = launch<NORI_F32, WDT, NORI_F16>(x, rows, cols, x_row_stride, weight, eps, y, y_row_stride, stream));
    } else {
        NORI_DISPATCH_FLOAT(weight_dtype, WDT,
            st = launch<NORI_F32, WDT, NORI_BF16>(x, rows, cols, x_row_stride, weight, eps, y, y_row_stride, stream));
    }
    return st;
}

extern "C" int nori_rms_norm(const void* x, int dtype, int64_t rows, int32_t cols, int64_t x_row_stride,
                             const void* weight, int weight_dtype, float eps, void* y, int64_t y_row_stride,
                             void* stream_v) {
    return nori_rms_norm_to(x, dtype, rows, cols, x_row_stride, weight, weight_dtype, eps, y, dtype, y_row_stride,
                            stream_v);
}

namespace {

template <int UT, int OT>
int launch_residual(const float* x, const void* u, const UpdateRows& ur, float alpha, int64_t rows, int cols, float eps,
                    float* xo, void* y, int64_t y_group, int64_t y_group_bytes, int64_t y_row_bytes, hipStream_t stream) {
    const int nchunks = cols / 4;
    int g = 1;
    while (g < nchunks && g < 64) g <<= 1;
    const int rows_per_block = kThreads / g;
    const unsigned grid = (unsigned)((rows + rows_per_block - 1) / rows_per_block);
#define NORI_RES_CASE(GV)                                                                                         \
    case GV:                                                                                                       \
        hipLaunchKernelGGL((residual_rms_norm_kernel<UT, OT, GV>), dim3(grid), dim3(kThreads), 0, stream, x, u, ur, \
                           alpha, rows, cols, eps, xo, (uint8_t*)y, y_group, y_group_bytes, y_row_bytes);          \
        break;
    switch (g) {
        NORI_RES_CASE(1) NORI_RES_CASE(2) NORI_RES_CASE(4) NORI_RES_CASE(8)
        NORI_RES_CASE(16) NORI_RES_CASE(32) NORI_RES_CASE(64)
    }
#undef NORI_RES_CASE
    return launch_status("residual_add_rms_norm");
}

}  // namespace

extern "C" int nori_residual_add_rms_norm(const float* x, const void* u, int u_dtype, const int64_t* u_rows,
                                          float alpha, int64_t rows, int32_t cols, float eps, float* x_out, void* y,
                                          int y_dtype, int64_t y_group, int64_t y_group_stride, int64_t y_row_stride,
                                          void* stream_v) {
    clear_error();
    if (rows < 0 || cols <= 0 || y_group <= 0)
        return fail(NORI_ERR_INVALID, "residual_add_rms_norm: bad shape rows=%lld cols=%d y_group=%lld",
                    (long long)rows, cols, (long long)y_group);
    // the update's rows: contiguous unless u_rows = {d1, d2, s0, s1, s2} says otherwise
    UpdateRows ur{1, 1, cols, 0, 0};
    if (u_rows) {
        ur = UpdateRows{u_rows[0], u_rows[1], u_rows[2], u_rows[3], u_rows[4]};
        if (ur.d1 <= 0 || ur.d2 <= 0 || rows % (ur.d1 * ur.d2) != 0)
            return fail(NORI_ERR_INVALID, "residual_add_rms_norm: update rows (%lld x %lld) do not tile %lld rows",
                        (long long)ur.d1, (long long)ur.d2, (long long)rows);
    }
    if (u_dtype != NORI_F32 && u_dtype != NORI_F16 && u_dtype != NORI_BF16)
        return fail(NORI_ERR_UNSUPPORTED, "residual_add_rms_norm: unsupported update dtype %s", dtype_name(u_dtype));
    if (y_dtype != NORI_F32 && y_dtype != NORI_F16 && y_dtype != NORI_BF16)
        return fail(NORI_ERR_UNSUPPORTED, "residual_add_rms_norm: unsupported output dtype %s", dtype_name(y_dtype));
    if (rows == 0) return NORI_OK;
    if (!x || !u || !x_out || !y) return fail(NORI_ERR_INVALID, "residual_add_rms_norm: null pointer");
    const int us = u_dtype == NORI_F32 ? 4 : 2, os = y_dtype == NORI_F32 ? 4 : 2, out_chunk = 4 * os;
    const bool fits = cols % 4 == 0 && cols / 4 <= 64 * kMaxChunksPerLane && (uintptr_t)x % 16 == 0 &&
                      (uintptr_t)x_out % 16 == 0 && (uintptr_t)u % (4 * us) == 0 && (uintptr_t)y % out_chunk == 0 &&
                      (y_row_stride * os) % out_chunk == 0 && (y_group_stride * os) % out_chunk == 0 &&
                      (ur.s0 * us) % (4 * us) == 0 && (ur.s1 * us) % (4 * us) == 0 && (ur.s2 * us) % (4 * us) == 0;
    if (!fits)
        return fail(NORI_ERR_UNSUPPORTED, "residual_add_rms_norm: rows of %d elements at these alignments take the "
                    "separate residual_add and rms_norm", cols);
    hipStream_t stream = (hipStream_t)stream_v;
    const int64_t gb = y_group_stride * os, rb = y_row_stride * os;
    if (u_dtype == NORI_F16) {
        if (y_dtype == NORI_F16) return launch_residual<NORI_F16, NORI_F16>(x, u, ur, alpha, rows, cols, eps, x_out, y, y_group, gb, rb, stream);
        if (y_dtype == NORI_BF16) return launch_residual<NORI_F16, NORI_BF16>(x, u, ur, alpha, rows, cols, eps, x_out, y, y_group, gb, rb, stream);
        return launch_residual<NORI_F16, NORI_F32>(x, u, ur, alpha, rows, cols, eps, x_out, y, y_group, gb, rb, stream);
    }
    if (u_dtype == NORI_BF16) {
        if (y_dtype == NORI_F16) return launch_residual<NORI_BF16, NORI_F16>(x, u, ur, alpha, rows, cols, eps, x_out, y, y_group, gb, rb, stream);
        if (y_dtype == NORI_BF16) return launch_residual<NORI_BF16, NORI_BF16>(x, u, ur, alpha, rows, cols, eps, x_out, y, y_group, gb, rb, stream);
        return launch_residual<NORI_BF16, NORI_F32>(x, u, ur, alpha, rows, cols, eps, x_out, y, y_group, gb, rb, stream);
    }
    if (y_dtype == NORI_F16) return launch_residual<NORI_F32, NORI_F16>(x, u, ur, alpha, rows, cols, eps, x_out, y, y_group, gb, rb, stream);
    if (y_dtype == NORI_BF16) return launch_residual<NORI_F32, NORI_BF16>(x, u, ur, alpha, rows, cols, eps, x_out, y, y_group, gb, rb, stream);
    return launch_residual<NORI_F32, NORI_F32>(x, u, ur, alpha, rows, cols, eps, x_out, y, y_group, gb, rb, stream);
}
