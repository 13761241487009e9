// QASS "full" query scaling in one pass on the MFMA units: for each query head vector q (d
// wide, fp16),
//     out = q * base_scale[h] * (1 + tanh(W2 gelu(W1 q + b1) + b2))
// as QASSMaxScaling.forward computes it under fp16 autocast (src/synthefy_nori/model/
// layer.py:316-456: the gate MLP Linear(d, 64) -> GELU -> Linear(64, d), then the two
// multiplies), rounded where torch's separate ops round: each linear's fp32 sum plus its bias
// rounded to fp16, GELU (erf form) and tanh evaluated in fp32 and rounded, 1 + t rounded, the
// two products rounded in turn. base_scale = log n * (1 + tanh(base_mlp(log n))) is one
// [heads, d] vector per call, formed by the caller. The separate ops make seven passes over
// the queries (two GEMMs, GELU, tanh, add, two multiplies, about 15 GB per 8.4 M vectors of
// 56); this kernel reads each query once and writes it once.
//
// Schedule. A wavefront takes 32 rows of one head at a time. The first GEMM runs transposed,
// H^T [64 hidden x 32 rows] = W1 [64 x d] Q^T, on v_mfma_f32_32x32x16_f16 with W1 (from LDS)
// as the A operand and the query rows (from global) as B. The second also runs transposed,
// G^T [d x 32 rows] = W2 [d x 64] H^T, and its B operand is the first's output registers
// after the bias, GELU and fp16 rounding, with no data movement: both GEMMs enumerate the
// k index of a 16-wide step in the order slot m of lane half hh <-> 4 hh + m % 4 + 8 (m / 4)
// (the rows a lane holds of a 32 x 32 result), the LDS copies of W1 and W2 are stored in that
// order, and the query elements a lane loads for the first GEMM are exactly the ones its
// second-GEMM results belong to. So the epilogue multiplies each result by the query value
// already in the lane's registers and writes 4 consecutive elements per 8-byte store.
#include <math.h>

#include "nori_common.h"

// each op rounds separately, as torch's do
#pragma clang fp contract(off)

namespace {

using namespace nori;

constexpr int kWaves = 4;
constexpr int kHid = 64;    // the gate MLP's hidden width (QASSMaxScaling's hidden_dim)
constexpr int kPitch = 72;  // f16 per LDS weight row (144 bytes: rows start on different banks)
constexpr float kSqrtHalf = 0.70710678118654752440f;

typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) _Float16 lds_f16;
typedef __attribute__((address_space(3))) f16x8 lds_f16x8;

// k index, within a 16-wide step, of slot m (0..7) of lane half hh: the order both GEMMs use
__host__ __device__ constexpr int kperm(int hh, int m) { return 4 * hh + (m & 3) + 8 * (m >> 2); }

__device__ __forceinline__ float r16(float v) { return round_to<NORI_F16>(v); }

__device__ __forceinline__ f16x8 join(u32x2_t lo, u32x2_t hi) {
    return __builtin_bit_cast(f16x8, u32x4_t{lo[0], lo[1], hi[0], hi[1]});
}

__device__ __forceinline__ float half_at(u32x2_t w, int i) {
    return f16_to_f32((uint16_t)(w[i >> 1] >> (16 * (i & 1))));
}

// torch's GELU (approximate='none') on an fp16 value, in fp32, rounded to fp16
__device__ __forceinline__ float gelu16(float x) { return r16(x * 0.5f * (1.0f + erff(x * kSqrtHalf))); }

template <int KS1, int NT2>  // k-steps of the first GEMM (ceil(d / 16)), 32-row tiles of the second (ceil(d / 32))
__global__ void __launch_bounds__(64 * kWaves, 4)
qass_gate_kernel(const uint16_t* q, int64_t rows, int heads, int d, int64_t qs, const uint16_t* w1,
                 const uint16_t* b1, const uint16_t* w2, const uint16_t* b2, const uint16_t* bs, uint16_t* out,
                 int64_t os, int64_t ntiles) {
    __shared__ __attribute__((aligned(16))) _Float16 w1s[kHid * kPitch];  // [hidden][k order], zeros past d
    __shared__ __attribute__((aligned(16))) _Float16 w2s[64 * kPitch];    // [output][k order], zero rows past d
    __shared__ __attribute__((aligned(16))) float b1s[kHid];
    __shared__ __attribute__((aligned(16))) float b2s[64];
    const int tid = threadIdx.x;
    for (int i = tid; i < 64 * 64; i += 64 * kWaves) {
        const int j = i >> 6, p = i & 63;
        const int c = 16 * (p >> 4) + kperm((p >> 3) & 1, p & 7);  // source column of LDS column p
        w1s[j * kPitch + p] = __builtin_bit_cast(_Float16, c < d ? w1[j * d + c] : (uint16_t)0);
        w2s[j * kPitch + p] = __builtin_bit_cast(_Float16, j < d ? w2[j * kHid + c] : (uint16_t)0);
    }
    if (tid < 64) {
        b1s[tid] = f16_to_f32(b1[tid]);
        b2s[tid] = tid < d ? f16_to_f32(b2[tid]) : 0.0f;
    }
    __syncthreads();

    const int wave = tid >> 6, lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
    const lds_f16* w1l = (const lds_f16*)w1s + l32 * kPitch + 8 * hh;
    const lds_f16* w2l = (const lds_f16*)w2s + l32 * kPitch + 8 * hh;
    for (int64_t tile = (int64_t)blockIdx.x * kWaves + wave; tile < ntiles; tile += (int64_t)gridDim.x * kWaves) {
        const int h = (int)(tile % heads);
        const int64_t r = (tile / heads) * 32 + l32;  // this lane's row
        const bool live = r < rows;
        const uint16_t* qr = q + (live ? r : rows - 1) * qs + (int64_t)h * d;

        // the lane's query elements: step s, half e holds q[16 s + 4 hh + 8 e + 0..3] (zeros
        // past d; the address clamped inside the row)
        u32x2_t qw[KS1][2];
#pragma unroll
        for (int s = 0; s < KS1; ++s)
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const int c = 16 * s + 4 * hh + 8 * e;
                const u32x2_t v = *reinterpret_cast<const u32x2_t*>(qr + min(c, d - 4));
                qw[s][e] = c < d ? v : u32x2_t{0u, 0u};
            }

        // H^T = W1 Q^T: acc1[t][4 g + i] is hidden unit 32 t + 8 g + 4 hh + i of row l32
        f32x16 acc1[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            acc1[t] = f32x16{};
#pragma unroll
            for (int s = 0; s < KS1; ++s) {
                const f16x8 a = *reinterpret_cast<const lds_f16x8*>(w1l + 32 * t * kPitch + 16 * s);
                acc1[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, join(qw[s][0], qw[s][1]), acc1[t], 0, 0, 0);
            }
        }
        // bias, GELU, fp16: hw[t][g] holds hidden units 32 t + 8 g + 4 hh + 0..3
        u32x2_t hw[2][4];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const f32x4 bb = *reinterpret_cast<const f32x4*>(&b1s[32 * t + 8 * g + 4 * hh]);
                float y[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) y[i] = gelu16(r16(acc1[t][4 * g + i] + bb[i]));
                hw[t][g] = u32x2_t{(uint32_t)f32_to_f16(y[0]) | ((uint32_t)f32_to_f16(y[1]) << 16),
                                   (uint32_t)f32_to_f16(y[2]) | ((uint32_t)f32_to_f16(y[3]) << 16)};
            }

        // G^T = W2 H^T: step s of the hidden units takes hw[s / 2][2 (s % 2) + 0..1] as its B
        // operand; acc2[t][4 g + i] is output 32 t + 8 g + 4 hh + i of row l32
        f32x16 acc2[NT2];
#pragma unroll
        for (int t = 0; t < NT2; ++t) {
            acc2[t] = f32x16{};
#pragma unroll
            for (int s = 0; s < kHid / 16; ++s) {
                const f16x8 a = *reinterpret_cast<const lds_f16x8*>(w2l + 32 * t * kPitch + 16 * s);
                acc2[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, join(hw[s >> 1][2 * (s & 1)], hw[s >> 1][2 * (s & 1) + 1]),
                                                                 acc2[t], 0, 0, 0);
            }
        }

        // out = (q * base_scale) * (1 + tanh(g + b2)); output o = 32 t + 8 g + 4 hh + i uses
        // the query element in qw[2 t + g / 2][g % 2], lane slot i
        if (live) {
            uint16_t* orow = out + r * os + (int64_t)h * d;
            const uint16_t* bsr = bs + (int64_t)h * d;
#pragma unroll
            for (int t = 0; t < NT2; ++t)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int o = 32 * t + 8 * g + 4 * hh;
                    if (o >= d) continue;
                    const u32x2_t qv = qw[2 * t + (g >> 1)][g & 1];
                    const u32x2_t sv = *reinterpret_cast<const u32x2_t*>(bsr + o);
                    const f32x4 bb = *reinterpret_cast<const f32x4*>(&b2s[o]);
                    uint32_t ob[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float gs = r16(1.0f + r16(tanhf(r16(acc2[t][4 * g + i] + bb[i]))));
                        ob[i] = f32_to_f16(r16(half_at(qv, i) * half_at(sv, i)) * gs);
                    }
                    *reinterpret_cast<u32x2_t*>(orow + o) = u32x2_t{ob[0] | (ob[1] << 16), ob[2] | (ob[3] << 16)};
                }
        }
    }
}

template <int KS1, int NT2>
void launch(const uint16_t* q, int64_t rows, int heads, int d, int64_t qs, const uint16_t* w1, const uint16_t* b1,
            const uint16_t* w2, const uint16_t* b2, const uint16_t* bs, uint16_t* out, int64_t os, hipStream_t stream) {
    const int64_t ntiles = (rows + 31) / 32 * heads;
    const int64_t grid = std::min<int64_t>((ntiles + kWaves - 1) / kWaves, 16384);
    hipLaunchKernelGGL((qass_gate_kernel<KS1, NT2>), dim3((unsigned)grid), dim3(64 * kWaves), 0, stream, q, rows,
                       heads, d, qs, w1, b1, w2, b2, bs, out, os, ntiles);
}

}  // namespace

extern "C" int nori_qass_gate(const void* q, int dtype, int64_t rows, int32_t heads, int32_t d, int64_t q_row_stride,
                              const void* w1, const void* b1, const void* w2, const void* b2, int32_t hidden,
                              const void* base_scale, void* out, int64_t out_row_stride, void* stream_v) {
    clear_error();
    if (dtype != NORI_F16) return fail(NORI_ERR_UNSUPPORTED, "qass_gate: %s queries (float16 only)", dtype_name(dtype));
    if (hidden != kHid) return fail(NORI_ERR_UNSUPPORTED, "qass_gate: gate hidden width %d (64 only)", hidden);
    if (rows < 0 || heads <= 0 || d < 4 || d > 64 || d % 4)
        return fail(NORI_ERR_INVALID, "qass_gate: bad shape (%lld rows, %d heads of %d; d a multiple of 4 up to 64)",
                    (long long)rows, heads, d);
    if (q_row_stride < (int64_t)heads * d || out_row_stride < (int64_t)heads * d || q_row_stride % 4 ||
        out_row_stride % 4)
        return fail(NORI_ERR_INVALID, "qass_gate: row strides (%lld, %lld) must be multiples of 4 and at least %d",
                    (long long)q_row_stride, (long long)out_row_stride, heads * d);
    if (rows == 0) return NORI_OK;
    if (!q || !w1 || !b1 || !w2 || !b2 || !base_scale || !out) return fail(NORI_ERR_INVALID, "qass_gate: null pointer");
    if ((uintptr_t)q % 8 || (uintptr_t)out % 8 || (uintptr_t)base_scale % 8)
        return fail(NORI_ERR_INVALID, "qass_gate: q, base_scale and out must be 8-byte aligned");
    if ((rows + 31) / 32 * heads > ((int64_t)1 << 40)) return fail(NORI_ERR_UNSUPPORTED, "qass_gate: too many rows");
    const auto* qh = reinterpret_cast<const uint16_t*>(q);
    const auto* w1h = reinterpret_cast<const uint16_t*>(w1);
    const auto* b1h = reinterpret_cast<const uint16_t*>(b1);
    const auto* w2h = reinterpret_cast<const uint16_t*>(w2);
    const auto* b2h = reinterpret_cast<const uint16_t*>(b2);
    const auto* bsh = reinterpret_cast<const uint16_t*>(base_scale);
    auto* oh = reinterpret_cast<uint16_t*>(out);
    hipStream_t stream = (hipStream_t)stream_v;
    const int ks1 = (d + 15) / 16;
    switch (ks1) {
        case 1: launch<1, 1>(qh, rows, heads, d, q_row_stride, w1h, b1h, w2h, b2h, bsh, oh, out_row_stride, stream); break;
        case 2: launch<2, 1>(qh, rows, heads, d, q_row_stride, w1h, b1h, w2h, b2h, bsh, oh, out_row_stride, stream); break;
        case 3: launch<3, 2>(qh, rows, heads, d, q_row_stride, w1h, b1h, w2h, b2h, bsh, oh, out_row_stride, stream); break;
        default: launch<4, 2>(qh, rows, heads, d, q_row_stride, w1h, b1h, w2h, b2h, bsh, oh, out_row_stride, stream); break;
    }
    return launch_status("qass_gate");
}
