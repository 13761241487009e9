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
#include "nori_common.h"

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
