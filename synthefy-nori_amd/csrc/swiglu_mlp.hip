// Fused SwiGLU feed-forward sublayer on the MFMA units:
//     y = (silu(x Wg^T) * (x Wu^T)) Wd^T
// for fp16 rows (SwiGLUMLP.forward, src/synthefy_nori/model/layer.py:261-274, under fp16
// autocast). The unfused sequence writes the [rows, 2h] gate|up projection to HBM, reads it
// back for the gate and writes [rows, h], and the down projection reads that again; here the
// hidden activations of a row tile never leave the CU.
//
// Workgroup: NW wavefronts of 32 rows each. Per chunk of 32 hidden units:
//   1. up:   G^T, U^T [32 hidden x 32 rows] = W{g,u}[chunk] . X^T on v_mfma_f32_32x32x16_f16
//            (A: weight rows staged in LDS; B: the wavefront's X fragments, held in registers
//            for the whole kernel);
//   2. gate: a = f16(f16(silu(f16(g))) * f16(u)) in registers; one v_permlane32_swap per word
//            pair turns the C layout into the B operand of step 3;
//   3. down: Y^T [width x 32 rows] += Wd[:, chunk] . a^T, accumulated over every chunk.
// The weight chunks (gate and up rows [64, width], down columns [width, 32]) go global -> LDS
// directly (global_load_lds_dwordx4: no staging registers, no LDS write instructions) into a
// double-buffered ring, the next chunk's loads in flight while the current chunk computes; one
// barrier per chunk. The weight chunks stream through every workgroup: at width 256 the
// staging costs about a third of the kernel's time (measured by leaving it out), the gate's
// VALU work about an eighth.
//
// nori_swiglu_mlp_residual_rms_norm ends the kernel with the deep-norm residual update of an
// fp32 stream and the next sublayer's RMSNorm (no weight) instead of writing y: per row
// x = x + f16(f16(y) * alpha) in place, then f16(x * rsqrt(mean(x^2) + eps)) over norm
// groups of NW columns (the whole row, or 128-column tokens of a wider row) -- bit for bit
// nori_swiglu_mlp followed by nori_residual_add_rms_norm: the sum of squares runs in that
// kernel's order (an fma chain over each 4-column chunk, then pairwise over the chunk index
// bits from the highest; a lane here holds every chunk of its half-row, chunk 8 t + 2 j + hh).
//
// Rounding: the projections sum in fp32 and round to fp16 as hipBLASLt's fp16 GEMMs do, but in
// their own order, so a value can differ from the unfused sequence's by one fp16 ulp where the
// fp32 sum sits at a rounding boundary. silu(g) = g * rcp(1 + 2^(-g log2 e)) with the hardware
// exp2 and reciprocal, within a few fp32 ulp of torch's g / (1 + exp(-g)) before its rounding
// to fp16; the product of two fp16 values is exact in fp32, so f16(s * u) is one packed fp16
// multiply.
#include "nori_common.h"

// the residual epilogue rounds every op separately, as torch does
#pragma clang fp contract(off)

namespace {

using namespace nori;

constexpr int HC = 32;  // hidden units per chunk
constexpr float kLog2eF = 1.4426950408889634f;

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

// Wavefronts per workgroup: eight (two per SIMD) at width 128, whose Y^T accumulators
// (width / 2 registers), X fragments (width / 4) and chunk G^T, U^T (32) leave the compiler
// room in 256 registers; four above (at width 256 an eight-wavefront build spills and runs
// 4-6 % slower).
constexpr int waves_for(int e) { return e <= 128 ? 8 : 4; }

template <int E>
struct MlpGeom {
    static_assert(E % 32 == 0, "width is a multiple of 32");
    static constexpr int NW = waves_for(E);
    static constexpr int THREADS = 64 * NW;
    static constexpr int KS = E / 16;  // k-steps of the up projection
    static constexpr int OT = E / 32;  // 32-row tiles of Y^T
    // A chunk in LDS, in 16-byte granules: gate rows 0-31 then up rows 0-31, each E/8 granules
    // and one of padding (the 16 lanes of a b128 read then land on distinct banks), then the
    // down rows [E, 32 hidden], 4 granules and one of padding each.
    static constexpr int GROW = E / 8 + 1;
    static constexpr int NG = 2 * HC * GROW;
    static constexpr int NDG = E * 5;
    static constexpr int LOADS = (NG + NDG + 63) / 64;  // wavefront loads of 64 granules
    static constexpr int BUF = LOADS * 64 * 8;           // f16 per ring buffer
};

__device__ __forceinline__ uint32_t pack_f16(float a, float b) {
    const f16x2 h = f16x2{(_Float16)pin_f32(a), (_Float16)pin_f32(b)};
    return __builtin_bit_cast(uint32_t, h);
}

// The gate of two hidden units: f16(f16(silu(f16(g))) * f16(u)) as one packed word.
__device__ __forceinline__ uint32_t gate_pair(float g0, float g1, float u0, float u1) {
    const f16x2 gh = f16x2{(_Float16)g0, (_Float16)g1};
    const f16x2 uh = f16x2{(_Float16)u0, (_Float16)u1};
    const float a = (float)gh[0], b = (float)gh[1];
    const float s0 = a * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(a * -kLog2eF));
    const float s1 = b * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(b * -kLog2eF));
    const f16x2 sh = f16x2{(_Float16)s0, (_Float16)s1};
    return __builtin_bit_cast(uint32_t, sh * uh);
}

// The residual epilogue's operands (NW > 0): the fp32 stream (row r at xs + r * xs_row, updated
// in place) and the normalized output, norm group q = r * (E / NW) + k at
// (q / y_group) * y_group_stride + (q % y_group) * y_row_stride elements from y.
struct ResEpi {
    float* xs;
    int64_t xs_row;
    float alpha, eps;
    int64_t y_group, y_group_stride, y_row_stride;
};

// NW: 0 writes y = the MLP's output (rows ys apart); else the residual epilogue with norm
// groups of NW columns.
template <int E, int NW>
__global__ void __launch_bounds__(MlpGeom<E>::THREADS)
swiglu_mlp_kernel(const uint16_t* __restrict__ x, int64_t rows, int64_t xs, const uint16_t* __restrict__ wgu,
                  const uint16_t* __restrict__ wd, int hp, uint16_t* __restrict__ y, int64_t ys, const ResEpi ep) {
    using G = MlpGeom<E>;
    __shared__ __attribute__((aligned(16))) _Float16 ring[2 * G::BUF];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
    const int64_t r0 = (int64_t)blockIdx.x * (G::NW * 32) + wave * 32;
    const int nch = hp / HC;

    // ---- staging: wavefront load i (i = wave, wave + NW, ...) fills granules [64i, 64i + 64)
    // of a buffer, lane l granule 64i + l; padding granules (and the tail past the chunk) load
    // a valid weight granule that nothing reads
    auto fetch = [&](int h0, int b) {
#pragma unroll
        for (int k = 0; k < (G::LOADS + G::NW - 1) / G::NW; ++k) {
            const int i = wave + k * G::NW;
            if (i >= G::LOADS) break;  // uniform over the wavefront
            const int q = 64 * i + lane;
            const uint16_t* src;
            if (q < G::NG) {
                const int row = q / G::GROW, cp = min(q % G::GROW, E / 8 - 1);
                src = wgu + ((int64_t)(row / HC) * hp + h0 + row % HC) * E + 8 * cp;
            } else {
                const int qd = min(q - G::NG, G::NDG - 1), e = qd / 5, cp = min(qd % 5, 3);
                src = wd + (int64_t)e * hp + h0 + 8 * cp;
            }
            __builtin_amdgcn_global_load_lds(src, (lds_void*)(ring + b * G::BUF + 512 * i), 16, 0, 0);
        }
    };

    // ---- X fragments (B operand of the up projection): lane holds x[row][16s + 8hh + 0..7]
    f16x8 xf[G::KS];
    {
        const int64_t row = r0 + l32;
        const bool ok = row < rows;
#pragma unroll
        for (int s = 0; s < G::KS; ++s) {
            u32x4 v = u32x4{0u, 0u, 0u, 0u};
            if (ok) v = *reinterpret_cast<const u32x4*>(x + row * xs + 16 * s + 8 * hh);
            xf[s] = __builtin_bit_cast(f16x8, v);
        }
    }

    f32x16 yt[G::OT];
#pragma unroll
    for (int t = 0; t < G::OT; ++t) yt[t] = f32x16{};

    fetch(0, 0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();

    for (int c = 0; c < nch; ++c) {
        const int cur = c & 1;
        // the next chunk into the other buffer, whose last reads were in chunk c-1 (before the
        // previous barrier); it lands while this chunk computes
        if (c + 1 < nch) fetch(HC * (c + 1), cur ^ 1);
        const _Float16* Gc = ring + cur * G::BUF;
        const _Float16* Dc = Gc + 8 * G::NG;

        // 1. G^T and U^T of the chunk
        f32x16 gt = f32x16{}, ut = f32x16{};
#pragma unroll
        for (int s = 0; s < G::KS; ++s) {
            const f16x8 ag = *reinterpret_cast<const f16x8*>(Gc + 8 * (l32 * G::GROW + 2 * s + hh));
            const f16x8 au = *reinterpret_cast<const f16x8*>(Gc + 8 * ((HC + l32) * G::GROW + 2 * s + hh));
            gt = __builtin_amdgcn_mfma_f32_32x32x16_f16(ag, xf[s], gt, 0, 0, 0);
            ut = __builtin_amdgcn_mfma_f32_32x32x16_f16(au, xf[s], ut, 0, 0, 0);
        }

        // 2. the gate, as words w[j][p] = hidden 8j + 4hh + 2p + {0, 1} of row l32, then the
        //    B operands of the down projection: k-step ks holds hidden 16ks + 8hh + 0..7
        uint32_t w[4][2];
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                const int i0 = 4 * j + 2 * p;
                w[j][p] = gate_pair(gt[i0], gt[i0 + 1], ut[i0], ut[i0 + 1]);
            }
        f16x8 af[2];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            // lanes 0-31 keep their words of hidden 16ks + 0..3 and take 4..7 from lane +32;
            // lanes 32-63 keep 16ks + 12..15 and take 8..11 from lane -32
            const auto s0 = __builtin_amdgcn_permlane32_swap(w[2 * ks][0], w[2 * ks + 1][0], false, false);
            const auto s1 = __builtin_amdgcn_permlane32_swap(w[2 * ks][1], w[2 * ks + 1][1], false, false);
            af[ks] = __builtin_bit_cast(f16x8, u32x4{s0[0], s1[0], s0[1], s1[1]});
        }

        // 3. Y^T += Wd[:, chunk] a^T
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int t = 0; t < G::OT; ++t) {
                const f16x8 ad = *reinterpret_cast<const f16x8*>(Dc + 8 * ((32 * t + l32) * 5 + 2 * ks + hh));
                yt[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ad, af[ks], yt[t], 0, 0, 0);
            }

        if (c + 1 < nch) {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wavefront's loads are in LDS
            __syncthreads();
        }
    }

    // ---- y[row][e .. e+3] from Y^T: element 4j + i of tile t is e = 32t + 8j + 4hh + i
    const int64_t row = r0 + l32;
    if constexpr (NW > 0) {
        static_assert(E % NW == 0 && NW % 32 == 0, "norm groups of whole tiles");
        constexpr int TT = NW / 32;  // tiles per norm group
        const bool ok = row < rows;
        float* xr = ep.xs + (ok ? row : 0) * ep.xs_row;
        float part[G::OT][4];
#pragma unroll
        for (int t = 0; t < G::OT; ++t)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int e = 32 * t + 8 * j + 4 * hh;
                const f32x4 xv = ok ? *reinterpret_cast<const f32x4*>(xr + e) : f32x4{0.f, 0.f, 0.f, 0.f};
                float p = 0.f;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float u = round_to<NORI_F16>(yt[t][4 * j + i]);
                    const float v = xv[i] + round_to<NORI_F16>(u * ep.alpha);
                    yt[t][4 * j + i] = v;
                    p = fmaf(v, v, p);
                }
                if (ok) *reinterpret_cast<f32x4*>(xr + e) = f32x4{yt[t][4 * j], yt[t][4 * j + 1], yt[t][4 * j + 2], yt[t][4 * j + 3]};
                part[t][j] = p;
            }
#pragma unroll
        for (int k = 0; k < E / NW; ++k) {
            // chunk 8 t' + 2 j + hh of the group (t' = t - k TT): pairs over (t', j) from the
            // highest bit in the lane, then over hh (lane bit 5)
            float q[4 * TT];
#pragma unroll
            for (int t = 0; t < TT; ++t)
#pragma unroll
                for (int j = 0; j < 4; ++j) q[4 * t + j] = part[k * TT + t][j];
#pragma unroll
            for (int st = 2 * TT; st >= 1; st >>= 1) {
#pragma unroll
                for (int i = 0; i < st; ++i) q[i] = q[i] + q[i + st];
            }
            float tot = q[0];
            tot = tot + __shfl_xor(tot, 32);
            const float inv = rsqrtf(tot / (float)NW + ep.eps);
            if (ok) {
                const int64_t qr = row * (E / NW) + k;
                uint16_t* yr = y + (qr / ep.y_group) * ep.y_group_stride + (qr % ep.y_group) * ep.y_row_stride;
#pragma unroll
                for (int t = 0; t < TT; ++t)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const f32x16& v = yt[k * TT + t];
                        uint16_t h[4];
#pragma unroll
                        for (int i = 0; i < 4; ++i) h[i] = f32_to_f16(v[4 * j + i] * inv);
                        *reinterpret_cast<u32x2*>(yr + 32 * t + 8 * j + 4 * hh) =
                            u32x2{h[0] | ((uint32_t)h[1] << 16), h[2] | ((uint32_t)h[3] << 16)};
                    }
            }
        }
    } else if (row < rows) {
        uint16_t* yr = y + row * ys;
#pragma unroll
        for (int t = 0; t < G::OT; ++t)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int e = 32 * t + 8 * j + 4 * hh;
                const f32x16& v = yt[t];
                *reinterpret_cast<u32x2*>(yr + e) = u32x2{pack_f16(v[4 * j], v[4 * j + 1]), pack_f16(v[4 * j + 2], v[4 * j + 3])};
            }
    }
}

template <int E, int NW = 0>
void launch(const uint16_t* x, int64_t rows, int64_t xs, const uint16_t* wgu, const uint16_t* wd, int hp, uint16_t* y,
            int64_t ys, hipStream_t stream, const ResEpi& ep = ResEpi{}) {
    using G = MlpGeom<E>;
    const int64_t per = G::NW * 32;
    const dim3 grid((unsigned)((rows + per - 1) / per));
    hipLaunchKernelGGL((swiglu_mlp_kernel<E, NW>), grid, dim3(G::THREADS), 0, stream, x, rows, xs, wgu, wd, hp, y, ys,
                       ep);
}

}  // namespace

extern "C" int nori_swiglu_mlp(const void* x, int dtype, int64_t rows, int32_t width, int64_t x_row_stride,
                               const void* w_gate_up, const void* w_down, int32_t hidden, void* y, int64_t y_row_stride,
                               void* stream_v) {
    clear_error();
    if (dtype != NORI_F16) return fail(NORI_ERR_UNSUPPORTED, "swiglu_mlp: unsupported dtype %s (float16 only)", dtype_name(dtype));
    if (width != 128 && width != 256 && width != 352)
        return fail(NORI_ERR_UNSUPPORTED, "swiglu_mlp: no kernel for width %d (128, 256 or 352)", width);
    if (rows < 0 || rows > 0x7fffffffLL || hidden <= 0 || hidden % 32 != 0)
        return fail(NORI_ERR_INVALID, "swiglu_mlp: bad shape (%lld rows, hidden %d: a positive multiple of 32)",
                    (long long)rows, hidden);
    if (x_row_stride < width || y_row_stride < width || x_row_stride % 8 != 0 || y_row_stride % 8 != 0)
        return fail(NORI_ERR_INVALID, "swiglu_mlp: row strides (%lld, %lld) must be multiples of 8 and at least %d",
                    (long long)x_row_stride, (long long)y_row_stride, width);
    if (rows == 0) return NORI_OK;
    if (!x || !w_gate_up || !w_down || !y) return fail(NORI_ERR_INVALID, "swiglu_mlp: null pointer");
    if ((uintptr_t)x % 16 || (uintptr_t)w_gate_up % 16 || (uintptr_t)w_down % 16 || (uintptr_t)y % 16)
        return fail(NORI_ERR_INVALID, "swiglu_mlp: x, the weights and y must be 16-byte aligned");
    hipStream_t stream = (hipStream_t)stream_v;
    auto xp = reinterpret_cast<const uint16_t*>(x);
    auto gp = reinterpret_cast<const uint16_t*>(w_gate_up);
    auto dp = reinterpret_cast<const uint16_t*>(w_down);
    auto yp = reinterpret_cast<uint16_t*>(y);
    switch (width) {
        case 128: launch<128>(xp, rows, x_row_stride, gp, dp, hidden, yp, y_row_stride, stream); break;
        case 256: launch<256>(xp, rows, x_row_stride, gp, dp, hidden, yp, y_row_stride, stream); break;
        default: launch<352>(xp, rows, x_row_stride, gp, dp, hidden, yp, y_row_stride, stream); break;
    }
    return launch_status("swiglu_mlp");
}

extern "C" int nori_swiglu_mlp_residual_rms_norm(const void* x, int dtype, int64_t rows, int32_t width,
                                                 int64_t x_row_stride, const void* w_gate_up, const void* w_down,
                                                 int32_t hidden, float alpha, float* stream_rows,
                                                 int64_t stream_row_stride, int32_t norm_width, float eps, void* y,
                                                 int64_t y_group, int64_t y_group_stride, int64_t y_row_stride,
                                                 void* stream_v) {
    clear_error();
    if (dtype != NORI_F16)
        return fail(NORI_ERR_UNSUPPORTED, "swiglu_mlp_residual_rms_norm: unsupported dtype %s (float16 only)", dtype_name(dtype));
    if (!((width == 128 && norm_width == 128) || (width == 256 && (norm_width == 128 || norm_width == 256))))
        return fail(NORI_ERR_UNSUPPORTED, "swiglu_mlp_residual_rms_norm: width %d with norm width %d (128/128, 256/128 "
                    "and 256/256 are built)", width, norm_width);
    if (rows < 0 || rows > 0x7fffffffLL || hidden <= 0 || hidden % 32 != 0 || y_group <= 0)
        return fail(NORI_ERR_INVALID, "swiglu_mlp_residual_rms_norm: bad shape (%lld rows, hidden %d, y_group %lld)",
                    (long long)rows, hidden, (long long)y_group);
    if (x_row_stride < width || x_row_stride % 8 || stream_row_stride < width || stream_row_stride % 4 ||
        y_group_stride % 4 || y_row_stride % 4)
        return fail(NORI_ERR_INVALID, "swiglu_mlp_residual_rms_norm: row strides must be multiples of 8 (x) or 4");
    if (rows == 0) return NORI_OK;
    if (!x || !w_gate_up || !w_down || !stream_rows || !y)
        return fail(NORI_ERR_INVALID, "swiglu_mlp_residual_rms_norm: null pointer");
    if ((uintptr_t)x % 16 || (uintptr_t)w_gate_up % 16 || (uintptr_t)w_down % 16 || (uintptr_t)stream_rows % 16 ||
        (uintptr_t)y % 8)
        return fail(NORI_ERR_INVALID, "swiglu_mlp_residual_rms_norm: x, the weights and the stream must be 16-byte "
                    "aligned, y 8-byte aligned");
    const ResEpi ep{stream_rows, stream_row_stride, alpha, eps, y_group, y_group_stride, y_row_stride};
    hipStream_t stream = (hipStream_t)stream_v;
    auto xp = reinterpret_cast<const uint16_t*>(x);
    auto gp = reinterpret_cast<const uint16_t*>(w_gate_up);
    auto dp = reinterpret_cast<const uint16_t*>(w_down);
    auto yp = reinterpret_cast<uint16_t*>(y);
    if (width == 128) launch<128, 128>(xp, rows, x_row_stride, gp, dp, hidden, yp, 0, stream, ep);
    else if (norm_width == 128) launch<256, 128>(xp, rows, x_row_stride, gp, dp, hidden, yp, 0, stream, ep);
    else launch<256, 256>(xp, rows, x_row_stride, gp, dp, hidden, yp, 0, stream, ep);
    return launch_status("swiglu_mlp_residual_rms_norm");
}
