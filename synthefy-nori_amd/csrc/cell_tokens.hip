// Cell tokens of the two-phase encoder's cell embedding for gfx950, under fp16 autocast:
// MaskEmbEncoder.forward with the scientific-notation RBF embedding and prompt-quantile PLE
// coordinates (src/synthefy_nori/model/encoders.py:118-276 RBFembedding, :309-429 PLE
// encode, :432-585 MaskEmbEncoder), from the cell values to the fp16 operand of the fusion
// network's first Linear. Per value x of a (table, row, group, feature) cell:
//   x0 = 0 if x is NaN else x                                   (masked_fill)
//   |x0| = m 10^e, e = clamp(floor(log10 |x0|), -9, 9), m = |x0| / 10^e   (float64)
//   rbf_k = f32(exp(-((m - c_k)^2) / f32(2 sigma^2)))           (float64, 16 or 32 centers)
//   pre_k = f32(rbf_k * sigmoid(gamma_k)) + tanh(beta_k)         (gamma, beta: the gate MLP of
//           the sign, exponent-sign and exponent-digit embeddings, one of 40 rows of a table)
//   rbf token = f16(LayerNorm(pre) * w + b) W_out^T + b_out       (fp16, fp32 sums)
//   ple_i = clamp((x0 - e_i) / (e_{i+1} - e_i), 0, 1), 0 for a bin of zero width or a
//           non-finite x0 (edges of the cell's (table, group, feature) column), in fp16
//   token = [rbf token | ple], or the mask embedding (fp16) where x is NaN.
// Every op rounds as the reference's torch ops do (double math through the same device
// library functions torch's kernels call: log10, pow, exp; correctly rounded divisions), with
// two exceptions of order only: the LayerNorm statistics are summed in the order of
// nori_layer_norm, and the output projection's fp32 sums in the MFMA's order.
//
// Schedule. A wavefront takes 32 consecutive values per step: lanes 0-31 split one value
// each into (m, e, table row); groups of NK / 4 lanes then take a value each (4 kernels and
// NB / (NK / 4) bins a lane), form pre, its LayerNorm and the PLE coordinates; the normalized
// rows go through the wavefront's LDS slice into two MFMA tiles (16 tokens) per 16 outputs
// with W_out held in registers; the finished 32 tokens (8 KiB, contiguous in the output)
// leave through LDS as 16-byte stores.
#include <math.h>

#include <algorithm>
#include <type_traits>

#include "nori_common.h"

// torch rounds every op separately
#pragma clang fp contract(off)

namespace {

using namespace nori;

constexpr int kWaves = 4;
constexpr int kVals = 32;  // values per wavefront step

struct CellArgs {
    const float* x;
    int64_t n, per_table;  // values; values per table (rows x groups x features)
    int64_t gf;            // groups x features
    const float* centers;
    const float* sigma;
    const _Float16* table;  // [40][2][NK]: sigmoid(gamma), tanh(beta)
    const float* ln_w;
    const float* ln_b;
    float ln_eps;
    const _Float16* w_out;  // [n_rbf][NK]
    const _Float16* b_out;  // [n_rbf] or null
    const float* edges;     // [tables][groups][features][n_bins + 1]
    const float* mask_emb;  // [n_rbf + n_bins] or null
    _Float16* out;          // [n][n_rbf + n_bins]
    int64_t steps;          // wavefront steps of kVals values
};

__device__ __forceinline__ float clamp01(float c) { return c != c ? c : fminf(fmaxf(c, 0.0f), 1.0f); }

__device__ __forceinline__ uint2 pack4(const uint16_t (&h)[4]) {
    return uint2{h[0] | ((uint32_t)h[1] << 16), h[2] | ((uint32_t)h[3] << 16)};
}

template <int NK>
struct TokGeom {
    static constexpr int G = NK / 4;        // lanes per value (4 kernels a lane)
    static constexpr int VPP = 64 / G;      // values per pass
    static constexpr int LNP = NK + 8;      // f16 pitch of a staged LayerNorm row
};

template <int NK, int NRBF, int NB>
constexpr size_t token_lds() {
    return (size_t)kWaves * kVals * ((NRBF + NB + 8) + TokGeom<NK>::LNP) * sizeof(_Float16);
}

template <int NK, int NRBF, int NB>
__global__ void __launch_bounds__(kWaves * 64) cell_token_kernel(const CellArgs a) {
    using T = TokGeom<NK>;
    constexpr int E = NRBF + NB, OP = E + 8, NO = NRBF / 16, BPL = NB / T::G;  // bins per lane
    static_assert((NK == 16 || NK == 32) && NRBF % 16 == 0 && BPL % 4 == 0 && E % 8 == 0, "token layout");
    extern __shared__ __attribute__((aligned(16))) _Float16 lds[];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    _Float16* ot = lds + wave * kVals * (OP + T::LNP);  // [kVals][OP] tokens
    _Float16* lt = ot + kVals * OP;                     // [kVals][LNP] normalized rows
    const int grp = lane / T::G, gi = lane % T::G;      // G lanes per value
    const int n16 = lane & 15, g4 = lane >> 4;          // MFMA lane coordinates

    // W_out rows as the MFMA A operand: lane (n16, g4) holds row 16 o + n16, k = (NK / 4) g4 ..
    typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
    using wvec = typename std::conditional<NK == 32, f16x8, f16x4>::type;
    constexpr int KL = NK / 4;  // k elements a lane holds
    wvec wf[NO];
#pragma unroll
    for (int o = 0; o < NO; ++o) wf[o] = *reinterpret_cast<const wvec*>(a.w_out + (16 * o + n16) * NK + KL * g4);
    float bo[NO][4];
#pragma unroll
    for (int o = 0; o < NO; ++o)
#pragma unroll
        for (int e = 0; e < 4; ++e) bo[o][e] = a.b_out ? (float)a.b_out[16 * o + 4 * g4 + e] : 0.0f;
    double cen[4];
    float lw[4], lb[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        cen[e] = (double)a.centers[4 * gi + e];
        lw[e] = a.ln_w ? a.ln_w[4 * gi + e] : 1.0f;
        lb[e] = a.ln_b ? a.ln_b[4 * gi + e] : 0.0f;
    }
    const float sg = *a.sigma;
    const double den = (double)(2.0f * (sg * sg));
    const float inv_n = 1.0f / (float)NK;

    const int64_t wave_id = (int64_t)blockIdx.x * kWaves + wave, nwaves = (int64_t)gridDim.x * kWaves;
    for (int64_t step = wave_id; step < a.steps; step += nwaves) {
        const int64_t v0 = step * kVals;
        // ---- lanes 0..31: value v0 + lane into (m, e, table row, edge row)
        double m = 0.0;
        int row = 0, miss = 0;
        float x0 = 0.0f;
        int64_t eoff = 0;
        {
            const int64_t v = v0 + (lane & 31);
            const bool ok = v < a.n;
            const float xv = ok ? a.x[v] : 0.0f;
            miss = xv != xv;
            x0 = miss ? 0.0f : xv;
            const double xw = (double)x0, mag = fabs(xw);
            const bool zero = mag == 0.0;
            double ef = floor(log10(zero ? 1.0 : mag));
            ef = ef != ef ? ef : fmin(fmax(ef, -9.0), 9.0);
            const int64_t ei = (int64_t)ef;
            const double mm = mag / pow(10.0, (double)ei);
            m = zero ? 0.0 : mm;
            const int64_t ae = ei < 0 ? -ei : ei;
            row = (xw < 0.0 ? 20 : 0) + (ei < 0 ? 10 : 0) + (int)(ae % 10);
            const int64_t vv = ok ? v : 0;
            eoff = ((vv / a.per_table) * a.gf + vv % a.gf) * (NB + 1);  // (table, group, feature) column
        }
        // ---- G lanes per value: value VPP p + grp
#pragma unroll
        for (int p = 0; p < kVals / T::VPP; ++p) {
            const int src = T::VPP * p + grp;
            const double mv = __shfl(m, src);
            const int tr = __shfl(row, src);
            const float xv = __shfl(x0, src);
            const int64_t eo = __shfl(eoff, src);
            const _Float16* tb = a.table + tr * (2 * NK) + 4 * gi;
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const double d = mv - cen[e];
                const double t = -(d * d);
                const float rbf = (float)exp(t / den);
                const float pre = rbf * (float)tb[e];
                v[e] = pre + (float)tb[NK + e];
            }
            // LayerNorm over the value's NK kernels (nori_layer_norm's order)
            float s = (v[0] + v[1]) + (v[2] + v[3]);
#pragma unroll
            for (int off = T::G / 2; off > 0; off >>= 1) s += __shfl_xor(s, off, T::G);
            const float mean = s * inv_n;
            float d2 = 0.f;
#pragma unroll
            for (int e = 0; e < 4; ++e) d2 += (v[e] - mean) * (v[e] - mean);
#pragma unroll
            for (int off = T::G / 2; off > 0; off >>= 1) d2 += __shfl_xor(d2, off, T::G);
            const float rstd = rsqrtf(d2 * inv_n + a.ln_eps);
            uint16_t h[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float o = (v[e] - mean) * rstd;
                o = o * lw[e];
                o = o + lb[e];
                h[e] = f32_to_f16(o);
            }
            *reinterpret_cast<uint2*>(lt + src * T::LNP + 4 * gi) = pack4(h);
            // PLE coordinates of bins BPL gi .. + BPL - 1
            const bool fin = isfinite(xv);
#pragma unroll
            for (int c4 = 0; c4 < BPL / 4; ++c4) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int k = BPL * gi + 4 * c4 + e;
                    const float lo = a.edges[eo + k], hi = a.edges[eo + k + 1];
                    const float w = hi - lo;
                    const bool open = w > 0.0f;
                    const float c = clamp01((xv - lo) / (open ? w : 1.0f));
                    h[e] = f32_to_f16(fin && open ? c : 0.0f);
                }
                *reinterpret_cast<uint2*>(ot + src * OP + NRBF + BPL * gi + 4 * c4) = pack4(h);
            }
        }
        // ---- out_layer: tokens 16 t + n16, outputs 16 o + 4 g4 .. + 3
#pragma unroll
        for (int t = 0; t < kVals / 16; ++t) {
            const wvec xb = *reinterpret_cast<const wvec*>(lt + (16 * t + n16) * T::LNP + KL * g4);
#pragma unroll
            for (int o = 0; o < NO; ++o) {
                f32x4 acc;
                if constexpr (NK == 32)
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(wf[o], xb, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                else
                    acc = __builtin_amdgcn_mfma_f32_16x16x16f16(wf[o], xb, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                uint16_t h[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) h[e] = f32_to_f16(acc[e] + bo[o][e]);
                *reinterpret_cast<uint2*>(ot + (16 * t + n16) * OP + 16 * o + 4 * g4) = pack4(h);
            }
        }
        // ---- the step's tokens, 16 bytes a lane (E / 8 lanes per token)
        constexpr int LPT = E / 8, TPS = 64 / LPT;
        static_assert(64 % LPT == 0 && kVals % TPS == 0, "token stores");
#pragma unroll
        for (int st = 0; st < kVals / TPS; ++st) {
            const int tk = st * TPS + lane / LPT, ch = lane % LPT;
            const int64_t v = v0 + tk;
            const int mt = __shfl(miss, tk);
            uint4 q = *reinterpret_cast<const uint4*>(ot + tk * OP + 8 * ch);
            if (mt && a.mask_emb) {
                uint16_t h[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) h[e] = f32_to_f16(a.mask_emb[8 * ch + e]);
                q = uint4{h[0] | ((uint32_t)h[1] << 16), h[2] | ((uint32_t)h[3] << 16), h[4] | ((uint32_t)h[5] << 16),
                          h[6] | ((uint32_t)h[7] << 16)};
            }
            if (v < a.n) *reinterpret_cast<uint4*>(a.out + v * E + 8 * ch) = q;
        }
    }
}

template <int NK, int NRBF, int NB>
int launch_tokens(const CellArgs& a, hipStream_t stream) {
    constexpr size_t lds = token_lds<NK, NRBF, NB>();
    static_assert(lds <= 64 * 1024, "one workgroup's LDS");
    const int per_cu = (int)(160 * 1024 / lds);
    const int64_t grid = std::min<int64_t>((a.steps + kWaves - 1) / kWaves, (int64_t)device_cus() * per_cu);
    hipLaunchKernelGGL((cell_token_kernel<NK, NRBF, NB>), dim3((unsigned)grid), dim3(kWaves * 64), lds, stream, a);
    return launch_status("cell_tokens");
}

}  // namespace

extern "C" int nori_cell_tokens(const float* x, int64_t tables, int64_t rows, int32_t groups, int32_t features,
                                int32_t n_kernels, const float* centers, const float* sigma, const void* gate_table,
                                const float* ln_weight, const float* ln_bias, float ln_eps, const void* w_out,
                                const void* b_out, int32_t n_rbf, const float* edges, int32_t n_bins,
                                const float* mask_embedding, void* out, void* stream) {
    clear_error();
    if (tables < 0 || rows < 0 || groups <= 0 || features <= 0)
        return fail(NORI_ERR_INVALID, "cell_tokens: bad shape %lld x %lld x %d x %d", (long long)tables, (long long)rows,
                    groups, features);
    if ((n_kernels != 16 && n_kernels != 32) || n_rbf != 96 || n_bins != 32)
        return fail(NORI_ERR_UNSUPPORTED,
                    "cell_tokens: %d kernels, %d RBF outputs and %d PLE bins (16 or 32, 96 and 32 are built)", n_kernels,
                    n_rbf, n_bins);
    if (tables == 0 || rows == 0) return NORI_OK;
    if (rows > INT64_MAX / 256 / ((int64_t)groups * features) || tables > INT64_MAX / 256 / (rows * groups * features))
        return fail(NORI_ERR_INVALID, "cell_tokens: too many values");
    if (!x || !centers || !sigma || !gate_table || !w_out || !edges || !out)
        return fail(NORI_ERR_INVALID, "cell_tokens: null pointer");
    if ((uintptr_t)w_out % 16 || (uintptr_t)out % 16)
        return fail(NORI_ERR_INVALID, "cell_tokens: w_out and out must be 16-byte aligned");
    CellArgs a;
    a.x = x;
    a.per_table = rows * groups * features;
    a.n = tables * a.per_table;
    a.gf = (int64_t)groups * features;
    a.centers = centers;
    a.sigma = sigma;
    a.table = reinterpret_cast<const _Float16*>(gate_table);
    a.ln_w = ln_weight;
    a.ln_b = ln_bias;
    a.ln_eps = ln_eps;
    a.w_out = reinterpret_cast<const _Float16*>(w_out);
    a.b_out = reinterpret_cast<const _Float16*>(b_out);
    a.edges = edges;
    a.mask_emb = mask_embedding;
    a.out = reinterpret_cast<_Float16*>(out);
    a.steps = (a.n + kVals - 1) / kVals;
    hipStream_t s = (hipStream_t)stream;
    return n_kernels == 16 ? launch_tokens<16, 96, 32>(a, s) : launch_tokens<32, 96, 32>(a, s);
}
