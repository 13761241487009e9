// Tall-skinny fp16 projection y = x W^T for gfx950: the F.linear of the attention projections
// under fp16 autocast (layer.py projections; reference layer.py:651-683, 1114-1160), for row
// counts in the hundreds of thousands and inner widths of 128 or 256.
//
// Semantics. y[r, c] = f16(sum_k f16(x[r, k]) * f16(W[c, k])) with fp32 sums: what the
// library GEMM computes for fp16 operands under autocast, up to the order of the fp32 sums.
//
// Shapes. These GEMMs are HBM-bound (K = 128 or 256: every output element costs 2 bytes of
// write against 2K FLOP), so the kernel is built for bandwidth: each x row is read from HBM
// once and each output row written once.
//   * A workgroup of 8 wavefronts owns a block of 256 rows and a chunk of NC output columns
//     (128 for K = 128, 64 for K = 256); the chunk's weight rows are staged in LDS as f16
//     (zero rows past n).
//   * Each wavefront holds its 32 rows of x as v_mfma_f32_16x16x32_f16 B operands (lane
//     n + 16*(k/8) holds row n, elements 8*(k/8)..+8 of every 32-wide step) and computes the
//     transposed product W x^T tile by tile: each lane ends with four consecutive output
//     columns of one row. 64 columns at a time are staged in the wavefront's LDS slice and
//     stored row by row, 16 bytes per lane and 128 contiguous bytes per row (written straight
//     from the MFMA layout, a store instruction touched 16 rows in 32-byte pieces and the
//     kernel ran 10-20 % slower at N = 128-256).
//   * Rows are addressed on a three-level grid, row r = (o * n_mid + j) * n_inner + i (strides
//     x_outer, x_mid, x_row and y_outer, y_mid, y_row), so strided views (a token subset of
//     each row, a slice of a stacked output, the [table, group, row] transpose of a
//     [table, row, group] cell buffer) are read and written in place.
//   * Workgroups are numbered so that the column chunks of one row block are consecutive on
//     one XCD (the hardware deals workgroup i to XCD i % 8): the x block is read from HBM once
//     and served to the other chunks by that XCD's L2.
//
// nori_linear_f16_residual_rms_norm fuses the output projection of an attention sublayer with
// the deep-norm residual update of an fp32 stream and the next sublayer's RMSNorm (no weight)
// into the operand dtype (two_phase.py:198, 209, 220-225, 264, 271-272; layer.py:251-253):
//   u = f16(a W^T),  x = x + f16(u * alpha),  y = f16(x * rsqrt(mean(x^2) + eps)),
// each op rounded as torch rounds it. The output width equals the inner width (128 or 256),
// so a wavefront holds whole rows of u in its accumulators: x is read and written once, y
// written once, and u never reaches memory. The mean of squares is summed in the order of
// the separate residual + norm kernel (nori_residual_add_rms_norm: an fma chain over each
// 4-element chunk, then pairwise over the chunk index bits from the highest), so x and y are
// bit for bit what F.linear-equivalent u through that kernel gives.
//   * Persistent workgroups: W is staged in LDS once (128 x 136 or 256 x 264 f16) and each
//     workgroup walks 128-row blocks, 16 rows per wavefront; a wavefront issues a block's
//     stream loads and the next block's operand loads before the block's MFMAs.
//   * The epilogue moves u through LDS into a row layout (16 lanes on 64 consecutive columns
//     of a row), so the stream is read and written in whole 256-byte row pieces.
#include <algorithm>

#include "nori_common.h"

// the residual update and the norm round every op separately, as torch does
#pragma clang fp contract(off)

namespace {

using namespace nori;

constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr int kNR = 2;                    // 16-row tiles per wavefront
constexpr int kRows = kWaves * kNR * 16;  // rows per workgroup

struct LinArgs {
    const _Float16* x; int64_t rows, n_mid, n_inner, x_outer, x_mid, x_row;
    const _Float16* w; int64_t w_row;
    int n;
    _Float16* y; int64_t y_outer, y_mid, y_row;
    int nchunks;
    int64_t grid;
};

// element offsets of row r in x and y on the three-level row grid
__device__ __forceinline__ void row_offsets(const LinArgs& a, int64_t r, int64_t& xo, int64_t& yo) {
    const int64_t oj = r / a.n_inner, i = r - oj * a.n_inner;
    const int64_t o = oj / a.n_mid, j = oj - o * a.n_mid;
    xo = o * a.x_outer + j * a.x_mid + i * a.x_row;
    yo = o * a.y_outer + j * a.y_mid + i * a.y_row;
}

__device__ __forceinline__ uint32_t pack_f16_rn(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, f16x2{(_Float16)lo, (_Float16)hi});
}

template <int KS, int NC>
__global__ void __launch_bounds__(kThreads) linear_f16_kernel(const LinArgs a) {
    constexpr int PITCH = 32 * KS + 8;  // f16 per staged W row: +16 bytes spreads the 16-row reads over the banks
    constexpr int GC = 64;              // output columns staged per wavefront between stores
    constexpr int SP = GC + 8;          // f16 per staged output row
    __shared__ __attribute__((aligned(16))) _Float16 wt[NC * PITCH];
    __shared__ __attribute__((aligned(16))) _Float16 ot[kWaves * kNR * 16 * SP];

    const int64_t wg = blockIdx.x;
    const int64_t xcd = wg % 8, local = wg / 8, per = a.grid / 8, extra = a.grid % 8;
    const int64_t t = xcd * per + (xcd < extra ? xcd : extra) + local;
    const int chunk = (int)(t % a.nchunks);
    const int64_t rb = t / a.nchunks;
    const int c0 = chunk * NC;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4;

    f16x8 xf[kNR][KS];
#pragma unroll
    for (int nt = 0; nt < kNR; ++nt) {
        const int64_t row = rb * kRows + wave * (kNR * 16) + nt * 16 + (lane & 15);
        int64_t xo, yo;
        row_offsets(a, row < a.rows ? row : a.rows - 1, xo, yo);
        const _Float16* xrow = a.x + xo + 8 * g;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) xf[nt][ks] = *reinterpret_cast<const f16x8*>(xrow + 32 * ks);
    }
    // rows this lane stores from the staged tile: 8 rows per pass, 8 lanes per row
    int64_t soff[4];
    bool svalid[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        const int64_t row = rb * kRows + wave * (kNR * 16) + 8 * p + (lane >> 3);
        svalid[p] = row < a.rows;
        int64_t xo;
        row_offsets(a, svalid[p] ? row : a.rows - 1, xo, soff[p]);
    }

    for (int e = tid; e < NC * KS * 4; e += kThreads) {
        const int r = e / (KS * 4), q = e % (KS * 4);
        uint4 v = {0u, 0u, 0u, 0u};
        if (c0 + r < a.n) v = *reinterpret_cast<const uint4*>(a.w + (int64_t)(c0 + r) * a.w_row + 8 * q);
        *reinterpret_cast<uint4*>(wt + r * PITCH + 8 * q) = v;
    }
    __syncthreads();

    const _Float16* wa = wt + (lane & 15) * PITCH + 8 * g;
    _Float16* my = ot + wave * (kNR * 16) * SP;
    const int ncols = min(NC, a.n - c0);
    for (int gc = 0; gc < ncols; gc += GC) {
#pragma unroll
        for (int mm = 0; mm < GC / 16; ++mm) {
            const int m = gc / 16 + mm;
            f32x4 acc[kNR];
#pragma unroll
            for (int nt = 0; nt < kNR; ++nt) acc[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const f16x8 av = *reinterpret_cast<const f16x8*>(wa + 16 * m * PITCH + 32 * ks);
#pragma unroll
                for (int nt = 0; nt < kNR; ++nt) acc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, xf[nt][ks], acc[nt], 0, 0, 0);
            }
#pragma unroll
            for (int nt = 0; nt < kNR; ++nt)
                *reinterpret_cast<uint2*>(my + (nt * 16 + (lane & 15)) * SP + 16 * mm + 4 * g) =
                    uint2{pack_f16_rn(acc[nt][0], acc[nt][1]), pack_f16_rn(acc[nt][2], acc[nt][3])};
        }
        // the wavefront's 32 rows x 64 columns, row by row: 16 bytes per lane, 128 per row
        const int col = c0 + gc + 8 * (lane & 7);
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const uint4 v = *reinterpret_cast<const uint4*>(my + (8 * p + (lane >> 3)) * SP + 8 * (lane & 7));
            if (svalid[p]) {
                if (col + 8 <= a.n) *reinterpret_cast<uint4*>(a.y + soff[p] + col) = v;
                else if (col + 4 <= a.n) *reinterpret_cast<uint2*>(a.y + soff[p] + col) = uint2{v.x, v.y};
            }
        }
    }
}

template <int KS, int NC>
int launch(LinArgs a, hipStream_t stream) {
    a.nchunks = (a.n + NC - 1) / NC;
    a.grid = (a.rows + kRows - 1) / kRows * a.nchunks;
    if (a.grid > 0x7fffffffLL) return fail(NORI_ERR_UNSUPPORTED, "linear_f16: %lld rows exceed one launch", (long long)a.rows);
    hipLaunchKernelGGL((linear_f16_kernel<KS, NC>), dim3((unsigned)a.grid), dim3(kThreads), 0, stream, a);
    return launch_status("linear_f16");
}

// ---------------------------------------------------------------- projection + residual + norm

struct ResArgs {
    const _Float16* a; int64_t rows, n_mid, n_inner, a_outer, a_mid, a_row;
    const _Float16* w; int64_t w_row;
    float* x; int64_t x_outer, x_mid, x_row;
    _Float16* y; int64_t y_outer, y_mid, y_row;
    float alpha, eps;
    int64_t nblocks;
};

struct RowIndex { int64_t o, j, i; };

// row r of the three-level grid, r = (o * n_mid + j) * n_inner + i (32-bit divisions when the
// grid fits them: a 64-bit division is about a hundred instructions)
__device__ __forceinline__ RowIndex split_row(int64_t r, int64_t n_mid, int64_t n_inner, bool narrow) {
    if (narrow) {
        const uint32_t r32 = (uint32_t)r, ni = (uint32_t)n_inner, nm = (uint32_t)n_mid;
        const uint32_t oj = r32 / ni, o = oj / nm;
        return {(int64_t)o, (int64_t)(oj - o * nm), (int64_t)(r32 - oj * ni)};
    }
    const int64_t oj = r / n_inner, i = r - oj * n_inner;
    const int64_t o = oj / n_mid, j = oj - o * n_mid;
    return {o, j, i};
}

// K = N = 32 KS; one 16-row tile per wavefront and block; W in dynamic LDS (K rows of K + 8
// f16), then each wavefront's 16 x 72 f16 slice for u. Per block a wavefront issues its
// stream loads and the next block's operand loads before its MFMAs, so both are in flight
// while it computes. The epilogue runs row by row, 64 columns at a time: u of four column
// tiles goes through the wavefront's LDS slice, and 16 lanes take a row's 64 columns (4
// consecutive elements each), so stream rows move 256 contiguous bytes per row and
// instruction and output rows 128. Lane l handles tile rows 4 p + l / 16 (p = 0..3) at
// columns 64 q + 4 (l % 16) for every chunk q: its chunk index in the row is 16 q + l % 16.
template <int KS, int WAVES>
__global__ void __launch_bounds__(WAVES * 64, KS == 4 ? 4 : 2) linear_residual_norm_kernel(const ResArgs a) {
    constexpr int K = 32 * KS, PITCH = K + 8;
    constexpr int kBlockRows = WAVES * 16;
    constexpr int NCH = K / 64, UP = 64 + 8;  // 64-column chunks; pitch of a staged u row
    extern __shared__ __attribute__((aligned(16))) _Float16 wt[];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4;
    const int c4 = 4 * (lane & 15);
    const bool narrow = a.rows <= 0x7fffffffLL;

    for (int e = tid; e < K * (K / 8); e += WAVES * 64) {
        const int r = e / (K / 8), q = e % (K / 8);
        *reinterpret_cast<uint4*>(wt + r * PITCH + 8 * q) =
            *reinterpret_cast<const uint4*>(a.w + (int64_t)r * a.w_row + 8 * q);
    }
    const _Float16* wa = wt + (lane & 15) * PITCH + 8 * g;
    _Float16* ut = wt + K * PITCH + wave * 16 * UP;

    auto operand_row = [&](int64_t blk) {
        const int64_t row = blk * kBlockRows + wave * 16 + (lane & 15);
        const RowIndex ri = split_row(row < a.rows ? row : a.rows - 1, a.n_mid, a.n_inner, narrow);
        return a.a + ri.o * a.a_outer + ri.j * a.a_mid + ri.i * a.a_row + 8 * g;
    };
    f16x8 xf[KS];
    int64_t blk = blockIdx.x;
    {
        const _Float16* ar = operand_row(blk);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) xf[ks] = *reinterpret_cast<const f16x8*>(ar + 32 * ks);
    }
    __syncthreads();

    for (; blk < a.nblocks; blk += gridDim.x) {
        // lane r < 16 computes tile row r's stream and output offsets; the passes take them
        // from there
        const int64_t row0 = blk * kBlockRows + wave * 16;
        const RowIndex ri = split_row(row0 + (lane & 15) < a.rows ? row0 + (lane & 15) : a.rows - 1, a.n_mid,
                                      a.n_inner, narrow);
        const int64_t xo = ri.o * a.x_outer + ri.j * a.x_mid + ri.i * a.x_row;
        const int64_t yo = ri.o * a.y_outer + ri.j * a.y_mid + ri.i * a.y_row;
        f32x4 v[4][NCH];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const int rr = 4 * p + (lane >> 4);
            const int64_t xop = __shfl(xo, rr) + c4;
#pragma unroll
            for (int q = 0; q < NCH; ++q)
                v[p][q] = row0 + rr < a.rows ? *reinterpret_cast<const f32x4*>(a.x + xop + 64 * q)
                                             : f32x4{0.f, 0.f, 0.f, 0.f};
        }
        // the next block's operand rows (the last block re-reads its own: in bounds, unused)
        f16x8 xn[KS];
        {
            const int64_t nb = blk + gridDim.x;
            const _Float16* ar = operand_row(nb < a.nblocks ? nb : blk);
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) xn[ks] = *reinterpret_cast<const f16x8*>(ar + 32 * ks);
        }
        float part[4][NCH];
#pragma unroll
        for (int q = 0; q < NCH; ++q) {
            f32x4 acc[4];
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                acc[m] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
                    const f16x8 av = *reinterpret_cast<const f16x8*>(wa + 16 * (4 * q + m) * PITCH + 32 * ks);
                    acc[m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, xf[ks], acc[m], 0, 0, 0);
                }
            }
            // u = fp16(acc): row lane & 15, columns 16 m + 4 g of this chunk
#pragma unroll
            for (int m = 0; m < 4; ++m)
                *reinterpret_cast<uint2*>(ut + (lane & 15) * UP + 16 * m + 4 * g) =
                    uint2{pack_f16_rn(acc[m][0], acc[m][1]), pack_f16_rn(acc[m][2], acc[m][3])};
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const int rr = 4 * p + (lane >> 4);
                const uint2 uw = *reinterpret_cast<const uint2*>(ut + rr * UP + c4);
                const uint32_t hw[2] = {uw.x, uw.y};
                float pp = 0.f;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float u = f16_to_f32((uint16_t)(hw[e >> 1] >> (16 * (e & 1))));
                    v[p][q][e] = v[p][q][e] + round_to<NORI_F16>(u * a.alpha);
                    pp = fmaf(v[p][q][e], v[p][q][e], pp);
                }
                part[p][q] = pp;
                const int64_t xop = __shfl(xo, rr) + c4 + 64 * q;
                if (row0 + rr < a.rows) *reinterpret_cast<f32x4*>(a.x + xop) = v[p][q];
            }
        }
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            // pairs over the chunk index bits from the highest: q's in the lane, then l % 16's
#pragma unroll
            for (int st = NCH / 2; st >= 1; st >>= 1) {
#pragma unroll
                for (int q = 0; q < st; ++q) part[p][q] = part[p][q] + part[p][q + st];
            }
            float tot = part[p][0];
#pragma unroll
            for (int off = 8; off > 0; off >>= 1) tot = tot + __shfl_xor(tot, off);
            const float inv = rsqrtf(tot / (float)K + a.eps);
            const int rr = 4 * p + (lane >> 4);
            const int64_t yop = __shfl(yo, rr) + c4;
            if (row0 + rr < a.rows) {
#pragma unroll
                for (int q = 0; q < NCH; ++q) {
                    uint16_t h[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) h[e] = f32_to_f16(v[p][q][e] * inv);
                    *reinterpret_cast<uint2*>(a.y + yop + 64 * q) =
                        uint2{h[0] | ((uint32_t)h[1] << 16), h[2] | ((uint32_t)h[3] << 16)};
                }
            }
        }
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) xf[ks] = xn[ks];
    }
}

template <int KS, int WAVES>
int launch_residual(ResArgs a, hipStream_t stream) {
    constexpr int K = 32 * KS;
    constexpr size_t lds = ((size_t)K * (K + 8) + (size_t)WAVES * 16 * 72) * sizeof(_Float16);
    constexpr int kBlockRows = WAVES * 16;
    static_assert(lds <= 160 * 1024, "W must fit one workgroup's LDS");
    if (hipFuncSetAttribute((const void*)linear_residual_norm_kernel<KS, WAVES>,
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
        return fail(NORI_ERR_RUNTIME, "linear_f16_residual_rms_norm: cannot reserve %zu bytes of LDS", lds);
    a.nblocks = (a.rows + kBlockRows - 1) / kBlockRows;
    // resident workgroups per CU: LDS-bound, and at most 16 wavefronts per CU
    const int per_cu = std::max(1, (int)std::min<size_t>(160 * 1024 / lds, 16 / WAVES));
    const int64_t grid = std::min<int64_t>(a.nblocks, (int64_t)device_cus() * per_cu);
    hipLaunchKernelGGL((linear_residual_norm_kernel<KS, WAVES>), dim3((unsigned)grid), dim3(WAVES * 64), lds,
                       stream, a);
    return launch_status("linear_f16_residual_rms_norm");
}

}  // namespace

extern "C" int nori_linear_f16(const void* x, int64_t n_outer, int64_t n_mid, int64_t n_inner, int32_t k,
                               int64_t x_outer_stride, int64_t x_mid_stride, int64_t x_row_stride, const void* weight,
                               int64_t w_row_stride, int32_t n, void* y, int64_t y_outer_stride, int64_t y_mid_stride,
                               int64_t y_row_stride, void* stream) {
    clear_error();
    if (n_outer < 0 || n_mid < 0 || n_inner < 0 || k <= 0 || n <= 0)
        return fail(NORI_ERR_INVALID, "linear_f16: bad shape n_outer=%lld n_mid=%lld n_inner=%lld k=%d n=%d",
                    (long long)n_outer, (long long)n_mid, (long long)n_inner, k, n);
    if (k != 128 && k != 256) return fail(NORI_ERR_UNSUPPORTED, "linear_f16: inner width %d is not 128 or 256", k);
    if (n % 4) return fail(NORI_ERR_UNSUPPORTED, "linear_f16: output width %d is not a multiple of 4", n);
    if (n_outer == 0 || n_mid == 0 || n_inner == 0) return NORI_OK;
    if (n_inner > INT64_MAX / n_mid || n_mid * n_inner > INT64_MAX / n_outer)
        return fail(NORI_ERR_INVALID, "linear_f16: %lld x %lld x %lld rows overflow", (long long)n_outer,
                    (long long)n_mid, (long long)n_inner);
    if (!x || !weight || !y) return fail(NORI_ERR_INVALID, "linear_f16: null pointer");
    // 16-byte x and W row chunks, 8-byte output pieces
    if ((uintptr_t)x % 16 || x_row_stride % 8 || x_mid_stride % 8 || x_outer_stride % 8 || (uintptr_t)weight % 16 ||
        w_row_stride % 8 || w_row_stride < k || (uintptr_t)y % 8 || y_row_stride % 4 || y_mid_stride % 4 ||
        y_outer_stride % 4)
        return fail(NORI_ERR_UNSUPPORTED,
                    "linear_f16: x and weight rows must be 16-byte aligned, output rows 8-byte aligned");
    LinArgs a;
    a.x = reinterpret_cast<const _Float16*>(x);
    a.rows = n_outer * n_mid * n_inner;
    a.n_mid = n_mid;
    a.n_inner = n_inner;
    a.x_outer = x_outer_stride;
    a.x_mid = x_mid_stride;
    a.x_row = x_row_stride;
    a.w = reinterpret_cast<const _Float16*>(weight);
    a.w_row = w_row_stride;
    a.n = n;
    a.y = reinterpret_cast<_Float16*>(y);
    a.y_outer = y_outer_stride;
    a.y_mid = y_mid_stride;
    a.y_row = y_row_stride;
    hipStream_t s = (hipStream_t)stream;
    return k == 128 ? launch<4, 128>(a, s) : launch<8, 64>(a, s);
}

extern "C" int nori_linear_f16_residual_rms_norm(const void* a, int64_t n_outer, int64_t n_mid, int64_t n_inner,
                                                 int32_t k, int64_t a_outer_stride, int64_t a_mid_stride,
                                                 int64_t a_row_stride, const void* weight, int64_t w_row_stride,
                                                 float alpha, float* x, int64_t x_outer_stride, int64_t x_mid_stride,
                                                 int64_t x_row_stride, float eps, void* y, int64_t y_outer_stride,
                                                 int64_t y_mid_stride, int64_t y_row_stride, void* stream) {
    clear_error();
    if (n_outer < 0 || n_mid < 0 || n_inner < 0 || k <= 0)
        return fail(NORI_ERR_INVALID, "linear_f16_residual_rms_norm: bad shape n_outer=%lld n_mid=%lld n_inner=%lld k=%d",
                    (long long)n_outer, (long long)n_mid, (long long)n_inner, k);
    if (k != 128 && k != 256)
        return fail(NORI_ERR_UNSUPPORTED, "linear_f16_residual_rms_norm: width %d is not 128 or 256", k);
    if (n_outer == 0 || n_mid == 0 || n_inner == 0) return NORI_OK;
    if (n_inner > INT64_MAX / n_mid || n_mid * n_inner > INT64_MAX / n_outer)
        return fail(NORI_ERR_INVALID, "linear_f16_residual_rms_norm: %lld x %lld x %lld rows overflow",
                    (long long)n_outer, (long long)n_mid, (long long)n_inner);
    if (!a || !weight || !x || !y) return fail(NORI_ERR_INVALID, "linear_f16_residual_rms_norm: null pointer");
    // 16-byte operand and weight chunks, 16-byte pieces of x, 8-byte pieces of y
    if ((uintptr_t)a % 16 || a_row_stride % 8 || a_mid_stride % 8 || a_outer_stride % 8 || (uintptr_t)weight % 16 ||
        w_row_stride % 8 || w_row_stride < k || (uintptr_t)x % 16 || x_row_stride % 4 || x_mid_stride % 4 ||
        x_outer_stride % 4 || (uintptr_t)y % 8 || y_row_stride % 4 || y_mid_stride % 4 || y_outer_stride % 4)
        return fail(NORI_ERR_UNSUPPORTED, "linear_f16_residual_rms_norm: operand and weight rows must be 16-byte "
                    "aligned, stream rows 16-byte aligned, output rows 8-byte aligned");
    ResArgs r;
    r.a = reinterpret_cast<const _Float16*>(a);
    r.rows = n_outer * n_mid * n_inner;
    r.n_mid = n_mid;
    r.n_inner = n_inner;
    r.a_outer = a_outer_stride;
    r.a_mid = a_mid_stride;
    r.a_row = a_row_stride;
    r.w = reinterpret_cast<const _Float16*>(weight);
    r.w_row = w_row_stride;
    r.x = x;
    r.x_outer = x_outer_stride;
    r.x_mid = x_mid_stride;
    r.x_row = x_row_stride;
    r.y = reinterpret_cast<_Float16*>(y);
    r.y_outer = y_outer_stride;
    r.y_mid = y_mid_stride;
    r.y_row = y_row_stride;
    r.alpha = alpha;
    r.eps = eps;
    hipStream_t s = (hipStream_t)stream;
    return k == 128 ? launch_residual<4, 8>(r, s) : launch_residual<8, 8>(r, s);
}
