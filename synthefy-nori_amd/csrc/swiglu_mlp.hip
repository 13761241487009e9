// Fused SwiGLU feed-forward sublayer on the MFMA units:
//     y = (silu(x Wg^T) * (x Wu^T)) Wd^T
// for fp16 rows (SwiGLUMLP.forward, src/synthefy_nori/model/layer.py:261-274, under fp16
// autocast). The unfused sequence writes the [rows, 2h] gate|up projection to HBM, reads it
// back for the gate and writes [rows, h], and the down projection reads that again; here the
// hidden activations of a row tile never leave the CU.
//
// Workgroup: 4 wavefronts; a wavefront owns 32 * RT rows. Per chunk of 32 hidden units:
//   1. up:   G^T, U^T [32 hidden x 32 rows] = W{g,u}[chunk] . X^T on v_mfma_f32_32x32x16_f16
//            (A: weight rows staged in LDS; B: the wavefront's X fragments, held in registers
//            for the whole kernel);
//   2. gate: a = f16(f16(silu(f16(g))) * f16(u)) in registers; one v_permlane32_swap per word
//            pair turns the C layout into the B operand of step 3;
//   3. down: Y^T [width x 32 rows] += Wd[:, chunk] . a^T, accumulated over every chunk.
// The weight chunks (gate and up rows [64, width], down columns [width, 32]) are staged into a
// double-buffered LDS ring by the whole workgroup, the next chunk's global loads in flight
// while the current chunk computes; one barrier per chunk.
//
// Rounding: the projections sum in fp32 and round to fp16 as hipBLASLt's fp16 GEMMs do, but in
// their own order, so a value can differ from the unfused sequence's by one fp16 ulp where the
// fp32 sum sits at a rounding boundary. The gate uses the hardware exp2 and reciprocal
// (silu(g) = g * rcp(1 + 2^(-g log2 e))), within a few fp32 ulp of torch's g / (1 + exp(-g))
// before the rounding to fp16.
#include "nori_common.h"

namespace {

using namespace nori;

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int HC = 32;  // hidden units per chunk
constexpr float kLog2eF = 1.4426950408889634f;

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int E>
struct MlpGeom {
    static_assert(E % 32 == 0, "width is a multiple of 32");
    static constexpr int KS = E / 16;         // k-steps of the up projection
    static constexpr int OT = E / 32;         // 32-row tiles of Y^T
    static constexpr int GPITCH = E + 8;      // f16 per staged gate/up row (+16 B: the 16 lanes of a
                                              // b128 read land on distinct banks)
    static constexpr int DPITCH = HC + 8;     // f16 per staged down row (80 B, likewise)
    static constexpr int GBUF = 2 * HC * GPITCH;  // gate rows 0-31, then up rows 0-31
    static constexpr int DBUF = E * DPITCH;
    static constexpr int GPIECES = 2 * HC * E / 8;  // 16-byte pieces of a chunk
    static constexpr int DPIECES = E * HC / 8;
    static constexpr int PIECES = GPIECES + DPIECES;
    static constexpr int PPT = (PIECES + kThreads - 1) / kThreads;  // pieces per thread
};

// Rows per wavefront (32 * RT): two row tiles share each weight fragment where the registers
// allow it (width 128).
constexpr int row_tiles(int e) { return e <= 128 ? 2 : 1; }

__device__ __forceinline__ float round_f16(float v) { return (float)(_Float16)pin_f32(v); }

// f16(f16(silu(g)) * u) for g, u already fp16 values
__device__ __forceinline__ float gate_value(float g, float u) {
    const float s = round_f16(g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-g * kLog2eF)));
    return s * u;
}

__device__ __forceinline__ uint32_t pack_f16(float a, float b) {
    const f16x2 h = f16x2{(_Float16)pin_f32(a), (_Float16)pin_f32(b)};
    return __builtin_bit_cast(uint32_t, h);
}

template <int E, int RT>
__global__ void __launch_bounds__(kThreads, 1)
swiglu_mlp_kernel(const uint16_t* __restrict__ x, int64_t rows, int64_t xs, const uint16_t* __restrict__ wgu,
                  const uint16_t* __restrict__ wd, int hp, uint16_t* __restrict__ y, int64_t ys) {
    using G = MlpGeom<E>;
    __shared__ __attribute__((aligned(16))) _Float16 Gs[2 * G::GBUF];
    __shared__ __attribute__((aligned(16))) _Float16 Ds[2 * G::DBUF];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
    const int64_t r0 = (int64_t)blockIdx.x * (kWaves * 32 * RT) + wave * 32 * RT;
    const int nch = (hp + HC - 1) / HC;

    // ---- staging plan: piece p = tid + i * kThreads of a chunk whose first hidden unit is h0
    auto fetch = [&](int h0, u32x4 (&buf)[G::PPT]) {
#pragma unroll
        for (int i = 0; i < G::PPT; ++i) {
            const int p = tid + i * kThreads;
            u32x4 v = u32x4{0u, 0u, 0u, 0u};
            if (p < G::GPIECES) {
                const int row = p / (E / 8), cp = p % (E / 8);
                const int h = h0 + row % HC;
                if (h < hp) v = *reinterpret_cast<const u32x4*>(wgu + ((int64_t)(row / HC) * hp + h) * E + 8 * cp);
            } else if (p < G::PIECES) {
                const int q = p - G::GPIECES, e = q / (HC / 8), cp = q % (HC / 8);
                const int h = h0 + 8 * cp;  // hp is a multiple of 8: a piece is valid whole or not at all
                if (h < hp) v = *reinterpret_cast<const u32x4*>(wd + (int64_t)e * hp + h);
            }
            buf[i] = v;
        }
    };
    auto store = [&](int b, const u32x4 (&buf)[G::PPT]) {
#pragma unroll
        for (int i = 0; i < G::PPT; ++i) {
            const int p = tid + i * kThreads;
            if (p < G::GPIECES) {
                const int row = p / (E / 8), cp = p % (E / 8);
                *reinterpret_cast<u32x4*>(&Gs[b * G::GBUF + row * G::GPITCH + 8 * cp]) = buf[i];
            } else if (p < G::PIECES) {
                const int q = p - G::GPIECES, e = q / (HC / 8), cp = q % (HC / 8);
                *reinterpret_cast<u32x4*>(&Ds[b * G::DBUF + e * G::DPITCH + 8 * cp]) = buf[i];
            }
        }
    };

    // ---- X fragments (B operand of the up projection): lane holds x[row][16s + 8hh + 0..7]
    f16x8 xf[RT][G::KS];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        const int64_t row = r0 + 32 * rt + l32;
        const bool ok = row < rows;
#pragma unroll
        for (int s = 0; s < G::KS; ++s) {
            u32x4 v = u32x4{0u, 0u, 0u, 0u};
            if (ok) v = *reinterpret_cast<const u32x4*>(x + row * xs + 16 * s + 8 * hh);
            xf[rt][s] = __builtin_bit_cast(f16x8, v);
        }
    }

    f32x16 yt[RT][G::OT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int t = 0; t < G::OT; ++t) yt[rt][t] = f32x16{};

    u32x4 buf[G::PPT];
    fetch(0, buf);
    store(0, buf);
    __syncthreads();

    for (int c = 0; c < nch; ++c) {
        const int cur = c & 1;
        if (c + 1 < nch) fetch(HC * (c + 1), buf);  // lands while this chunk computes
        const _Float16* Gc = Gs + cur * G::GBUF;
        const _Float16* Dc = Ds + cur * G::DBUF;

        // 1. G^T and U^T of the chunk
        f32x16 gt[RT], ut[RT];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) gt[rt] = ut[rt] = f32x16{};
#pragma unroll
        for (int s = 0; s < G::KS; ++s) {
            const f16x8 ag = *reinterpret_cast<const f16x8*>(Gc + l32 * G::GPITCH + 16 * s + 8 * hh);
            const f16x8 au = *reinterpret_cast<const f16x8*>(Gc + (HC + l32) * G::GPITCH + 16 * s + 8 * hh);
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                gt[rt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ag, xf[rt][s], gt[rt], 0, 0, 0);
                ut[rt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(au, xf[rt][s], ut[rt], 0, 0, 0);
            }
        }

        // 2. the gate, as words w[j][p] = hidden 8j + 4hh + 2p + {0, 1} of row l32, then the
        //    B operands of the down projection: k-step ks holds hidden 16ks + 8hh + 0..7
        f16x8 af[RT][2];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            uint32_t w[4][2];
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int p = 0; p < 2; ++p) {
                    const int i0 = 4 * j + 2 * p;
                    const float v0 = gate_value(round_f16(gt[rt][i0]), round_f16(ut[rt][i0]));
                    const float v1 = gate_value(round_f16(gt[rt][i0 + 1]), round_f16(ut[rt][i0 + 1]));
                    w[j][p] = pack_f16(v0, v1);
                }
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                // lanes 0-31 keep their words of hidden 16ks + 0..3 and take 4..7 from lane +32;
                // lanes 32-63 keep 16ks + 12..15 and take 8..11 from lane -32
                const auto s0 = __builtin_amdgcn_permlane32_swap(w[2 * ks][0], w[2 * ks + 1][0], false, false);
                const auto s1 = __builtin_amdgcn_permlane32_swap(w[2 * ks][1], w[2 * ks + 1][1], false, false);
                af[rt][ks] = __builtin_bit_cast(f16x8, u32x4{s0[0], s1[0], s0[1], s1[1]});
            }
        }

        // 3. Y^T += Wd[:, chunk] a^T
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int t = 0; t < G::OT; ++t) {
                const f16x8 ad = *reinterpret_cast<const f16x8*>(Dc + (32 * t + l32) * G::DPITCH + 16 * ks + 8 * hh);
#pragma unroll
                for (int rt = 0; rt < RT; ++rt)
                    yt[rt][t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ad, af[rt][ks], yt[rt][t], 0, 0, 0);
            }

        // the next chunk into the other buffer, whose last reads were in chunk c-1 (before the
        // previous barrier)
        if (c + 1 < nch) {
            store(cur ^ 1, buf);
            __syncthreads();
        }
    }

    // ---- y[row][e .. e+3] from Y^T: element 4j + i of tile t is e = 32t + 8j + 4hh + i
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        const int64_t row = r0 + 32 * rt + l32;
        if (row >= rows) continue;
        uint16_t* yr = y + row * ys;
#pragma unroll
        for (int t = 0; t < G::OT; ++t)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int e = 32 * t + 8 * j + 4 * hh;
                const f32x16& v = yt[rt][t];
                *reinterpret_cast<u32x2*>(yr + e) = u32x2{pack_f16(v[4 * j], v[4 * j + 1]), pack_f16(v[4 * j + 2], v[4 * j + 3])};
            }
    }
}

template <int E>
void launch(const uint16_t* x, int64_t rows, int64_t xs, const uint16_t* wgu, const uint16_t* wd, int hp, uint16_t* y,
            int64_t ys, hipStream_t stream) {
    constexpr int RT = row_tiles(E);
    const int64_t per = kWaves * 32 * RT;
    const dim3 grid((unsigned)((rows + per - 1) / per));
    hipLaunchKernelGGL((swiglu_mlp_kernel<E, RT>), grid, dim3(kThreads), 0, stream, x, rows, xs, wgu, wd, hp, y, ys);
}

}  // namespace

extern "C" int nori_swiglu_mlp(const void* x, int dtype, int64_t rows, int32_t width, int64_t x_row_stride,
                               const void* w_gate_up, const void* w_down, int32_t hidden, void* y, int64_t y_row_stride,
                               void* stream_v) {
    clear_error();
    if (dtype != NORI_F16) return fail(NORI_ERR_UNSUPPORTED, "swiglu_mlp: unsupported dtype %s (float16 only)", dtype_name(dtype));
    if (width != 128 && width != 256 && width != 352)
        return fail(NORI_ERR_UNSUPPORTED, "swiglu_mlp: no kernel for width %d (128, 256 or 352)", width);
    if (rows < 0 || rows > 0x7fffffffLL || hidden <= 0 || hidden % 8 != 0)
        return fail(NORI_ERR_INVALID, "swiglu_mlp: bad shape (%lld rows, hidden %d: a positive multiple of 8)",
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
