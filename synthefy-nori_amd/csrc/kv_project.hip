// Fused context-cache write for gfx950: (RMSNorm ->) K/V projection -> int8 quantization.
//
// Semantics. For every context row x (embed elements) and every cache head vector j (the
// rows [j*d, j*d + d) of the projection weight W [2*kv_heads*d, embed], K heads then V heads,
// the order of project_kv_cache, src/synthefy_nori/model/layer.py:651-683):
//   xn  = norm ? T(x * rsqrt(mean(x^2) + eps)) : x       (RMSNorm, layer.py:251-253; T = x dtype)
//   kv  = f16(f16(xn) . f16(W_j)^T)                       (the fp16 projection of the GPU's
//                                                          autocast path: f16 operands, fp32
//                                                          accumulation, one rounding)
//   codes, scale = quantize_int8(kv)  in f16             (kv_cache_scaling.py:29-37, exact)
// The fp16 K/V never exist in memory: each projected head vector is rounded and quantized in
// registers.
//
// Two kernels.
// * operand rows (unless x is already f16 operands: f16, no norm, embed a multiple of 32):
//   one wavefront per row normalizes it and writes f16(xn) to a workspace row padded with
//   zeros to a multiple of 32 -- the cast the autocast path makes before its GEMM, with the
//   norm folded in.
// * projection + quantizer: persistent workgroups of 8 wavefronts, two per CU. A workgroup
//   owns a group of `hg` cache heads: their weight rows, each head padded with zero rows to
//   16 * MT, stay in LDS as f16 for the whole launch. It walks blocks of 8 * 16 * NR rows
//   (NR = 1); each wavefront loads its 16 * NR operand rows straight into v_mfma_f32_16x16x32_f16 B
//   operands (lane n + 16*(k/8) holds row n, elements 8*(k/8)..+8 of every 32-wide step).
//   Per head, the MFMAs compute the transposed projection W_j . x^T, whose result layout gives
//   every lane four consecutive K/V columns of one row: the head's absmax is a per-lane max and
//   two shuffles, and the four codes leave as one 32-bit store. Workgroups are numbered so the
//   head groups of one row block sit on one XCD and share its L2 for the operand rows.
#include <math.h>

#include <algorithm>

#include "nori_common.h"
#include "quant_common.h"

#pragma clang fp contract(off)

namespace {

using namespace nori;
using namespace nori::quant;

constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr int kWgPerCu = 2;  // resident workgroups per CU when the weight tile fits half the LDS
constexpr size_t kLds = 160 * 1024;
constexpr int kPrepWaves = 4;

// Rows are addressed on a two-level grid, row r = o * n_inner + i (o < n_outer, i < n_inner).
struct Grid {
    int64_t rows, n_inner;
};

__device__ __forceinline__ uint4 load16(const void* base, int64_t byte_off) {
    return *reinterpret_cast<const uint4*>(reinterpret_cast<const uint8_t*>(base) + byte_off);
}

// the elements of one raw 16-byte chunk of dtype DT as f32 (4 for fp32, 8 for 16-bit types)
template <int DT>
__device__ __forceinline__ void unpack(const uint4 v, float* f) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        if constexpr (DT == NORI_F32) {
            f[k] = __uint_as_float(w[k]);
        } else if constexpr (DT == NORI_F16) {
            f[2 * k] = f16_to_f32((uint16_t)(w[k] & 0xffff));
            f[2 * k + 1] = f16_to_f32((uint16_t)(w[k] >> 16));
        } else {
            f[2 * k] = __uint_as_float(w[k] << 16);
            f[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
        }
    }
}

template <int DT> constexpr int chunk_elems() { return DT == NORI_F32 ? 4 : 8; }

// ------------------------------------------------------------------ operand rows
struct PrepArgs {
    const void* x; Grid grid; int embed; int64_t x_outer, x_row;  // x strides in elements
    int norm; float eps;
    _Float16* ws; int pitch;  // workspace rows of `pitch` f16 (32 * steps), dense
};

// One wavefront per row, kPrepRows rows at a time (their loads in flight together), rows in
// contiguous runs per wavefront. Lane l holds 16-byte chunks l, l + 64, ... (at most 4: embed
// <= 1024); the statistic is a wavefront reduction.
constexpr int kPrepRows = 4;

template <int DT>
__global__ void __launch_bounds__(kPrepWaves * 64) prep_rows_kernel(const PrepArgs a) {
    constexpr int EPC = chunk_elems<DT>();
    constexpr int ES = DT == NORI_F32 ? 4 : 2;
    const int lane = threadIdx.x & 63;
    const int64_t nw = (int64_t)gridDim.x * kPrepWaves;
    const int64_t w = (int64_t)blockIdx.x * kPrepWaves + (threadIdx.x >> 6);
    const int64_t per = (a.grid.rows + nw - 1) / nw;
    const int64_t r_begin = w * per, r_end = std::min<int64_t>(a.grid.rows, r_begin + per);
    if (r_begin >= r_end) return;
    int64_t o = r_begin / a.grid.n_inner, i = r_begin - o * a.grid.n_inner;
    const int nch = a.embed / EPC;
    for (int64_t r0 = r_begin; r0 < r_end; r0 += kPrepRows) {
        uint4 v[kPrepRows][4];
#pragma unroll
        for (int q = 0; q < kPrepRows; ++q) {
            const bool row_in = r0 + q < r_end;
            const int64_t base = (o * a.x_outer + i * a.x_row) * ES;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int c = lane + 64 * j;
                v[q][j] = row_in && c < nch ? load16(a.x, base + (int64_t)c * 16) : uint4{0u, 0u, 0u, 0u};
            }
            if (++i == a.grid.n_inner) { i = 0; ++o; }
        }
        float inv[kPrepRows];
#pragma unroll
        for (int q = 0; q < kPrepRows; ++q) {
            inv[q] = 1.0f;
            if (a.norm) {
                float acc = 0.0f;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    float f[EPC];
                    unpack<DT>(v[q][j], f);
#pragma unroll
                    for (int e = 0; e < EPC; ++e) acc = fmaf(f[e], f[e], acc);
                }
#pragma unroll
                for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off);
                inv[q] = rsqrtf(acc / (float)a.embed + a.eps);
            }
        }
#pragma unroll
        for (int q = 0; q < kPrepRows; ++q) {
            if (r0 + q >= r_end) break;
            _Float16* dst = a.ws + (r0 + q) * a.pitch;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int c = lane + 64 * j;
                if (c < nch) {
                    float f[EPC];
                    unpack<DT>(v[q][j], f);
                    _Float16 h[EPC];
#pragma unroll
                    for (int e = 0; e < EPC; ++e)
                        h[e] = (_Float16)pin_f32(a.norm ? round_to<DT>(f[e] * inv[q]) : f[e]);
                    if constexpr (EPC == 8) {
                        *reinterpret_cast<f16x8*>(dst + c * EPC) = f16x8{h[0], h[1], h[2], h[3], h[4], h[5], h[6], h[7]};
                    } else {
                        *reinterpret_cast<uint2*>(dst + c * EPC) =
                            uint2{(uint32_t)__builtin_bit_cast(uint16_t, h[0]) | ((uint32_t)__builtin_bit_cast(uint16_t, h[1]) << 16),
                                  (uint32_t)__builtin_bit_cast(uint16_t, h[2]) | ((uint32_t)__builtin_bit_cast(uint16_t, h[3]) << 16)};
                    }
                }
            }
            // zeros from embed to the padded width, in 4-element pieces (embed is a multiple of 4)
            for (int u = a.embed / 4 + lane; u < a.pitch / 4; u += 64) *reinterpret_cast<uint2*>(dst + 4 * u) = uint2{0u, 0u};
        }
    }
}

// ------------------------------------------------------------------ projection + quantizer
struct ProjArgs {
    const _Float16* xs; Grid grid; int64_t xs_outer, xs_row;  // f16 operand rows (elements)
    const void* w; int wdt; int64_t w_stride;  // W [2*kv_heads*d, embed], row stride in elements
    int embed;
    int nheads;  // 2 * kv_heads cache head vectors per row
    int d, dp;   // head width, padded with zero rows to the kernel's 16 * MT
    int hg;      // heads per group (the last group may hold fewer)
    int ngroups;
    int ksteps;  // operand steps of 32 elements in a row (its f16 row holds zeros past embed)
    int xp;      // LDS pitch of the weight rows (f16 elements): 32 * KS + 8
    int8_t* codes; int64_t codes_outer, codes_row;    // codes: nheads*d bytes per row
    float* scales; int64_t scales_outer, scales_row;  // scales: nheads floats per row
    int scale_div;
    int bm;           // rows per block
    int64_t nblocks;  // row blocks
    int streams;      // workgroups per head group
};

// Weight rows c < hg*dp of the group (zero rows in each head's padding and past the last head)
// into the LDS tile as f16, zero-padded to the pitch. Loaded once per workgroup, eight 16-byte
// chunks per thread in flight at a time.
template <int WDT>
__device__ __forceinline__ void load_weights(const ProjArgs& a, _Float16* wt, int head0, int ghe, int tid) {
    constexpr int EPC = chunk_elems<WDT>();
    constexpr int ES = WDT == NORI_F32 ? 4 : 2;
    constexpr int kRowThreads = 4;
    const int lr = tid / kRowThreads, lq = tid % kRowThreads;
    const int nch = a.embed / EPC, pch = (a.xp - 8) / EPC;
    for (int c = lr; c < a.hg * a.dp; c += kThreads / kRowThreads) {
        const int hh = c / a.dp, e = c % a.dp;
        const bool valid = hh < ghe && e < a.d;
        const int64_t base = ((int64_t)(head0 + hh) * a.d + e) * a.w_stride * ES;
        for (int j0 = lq; j0 < pch; j0 += kRowThreads * 8) {
            uint4 v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int j = j0 + kRowThreads * u;
                v[u] = (valid && j < nch) ? load16(a.w, base + (int64_t)j * 16) : uint4{0u, 0u, 0u, 0u};
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int j = j0 + kRowThreads * u;
                if (j < pch) {
                    float f[EPC];
                    unpack<WDT>(v[u], f);
                    _Float16* dst = wt + c * a.xp + j * EPC;
#pragma unroll
                    for (int q = 0; q < EPC; ++q) dst[q] = (_Float16)f[q];
                }
            }
        }
    }
}

// Row r0 + off on the two-level grid, given (o0, i0) of r0; off < 256.
__device__ __forceinline__ void row_coords(int64_t o0, int64_t i0, int off, int64_t n_inner, int64_t& o,
                                           int64_t& i) {
    i = i0 + off;
    o = o0;
    if (n_inner >= 256) {
        if (i >= n_inner) { i -= n_inner; ++o; }
    } else {
        const uint32_t q = (uint32_t)i / (uint32_t)n_inner;  // i < n_inner + 256 < 512
        o += q;
        i -= (int64_t)q * n_inner;
    }
}

template <int NR, int KS, int MT>
__global__ void __launch_bounds__(kThreads, 2) kv_project_quantize_kernel(const ProjArgs a) {
    extern __shared__ __attribute__((aligned(16))) _Float16 wt[];  // [hg*dp][xp]

    // work: XCD-aware numbering, the head groups of a stream consecutive within one XCD
    const int nwg = (int)gridDim.x;
    const int wg = (int)blockIdx.x;
    const int t = (wg % 8) * (nwg / 8) + min(wg % 8, nwg % 8) + wg / 8;
    const int group = t % a.ngroups;
    const int stream = t / a.ngroups;
    const int head0 = group * a.hg;
    const int ghe = min(a.hg, a.nheads - head0);  // heads in this group

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int g = lane >> 4;  // result lanes hold columns 4g..4g+3 of each 16-column tile

    if (a.wdt == NORI_F32) load_weights<NORI_F32>(a, wt, head0, ghe, tid);
    else if (a.wdt == NORI_F16) load_weights<NORI_F16>(a, wt, head0, ghe, tid);
    else load_weights<NORI_BF16>(a, wt, head0, ghe, tid);
    __syncthreads();

    const _Float16* wa = wt + (lane & 15) * a.xp + 8 * g;  // A operand rows of tile 0 of head 0
    // columns of the last tile past d are the heads' zero padding rows: left out of the absmax
    bool pad_ok[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) pad_ok[q] = 16 * (MT - 1) + 4 * g + q < a.d;

    // ---- operand rows of block rb for this wavefront -> B operands; their code and scale row
    // offsets. Lanes of rows past the last read the last row and store nothing.
    auto load_rows = [&](int64_t rb, f16x8 (&xf)[NR][KS], int64_t (&c_off)[NR], int64_t (&s_off)[NR]) {
        const int64_t r0 = rb * a.bm;
        const int64_t o0 = r0 / a.grid.n_inner, i0 = r0 - o0 * a.grid.n_inner;
#pragma unroll
        for (int nt = 0; nt < NR; ++nt) {
            const int off0 = (wave * NR + nt) * 16 + (lane & 15);
            const bool valid = r0 + off0 < a.grid.rows;
            int64_t o, i;
            row_coords(o0, i0, valid ? off0 : (int)(a.grid.rows - 1 - r0), a.grid.n_inner, o, i);
            const _Float16* xrow = a.xs + o * a.xs_outer + i * a.xs_row + 8 * g;
            c_off[nt] = valid ? o * a.codes_outer + i * a.codes_row : -1;
            s_off[nt] = valid ? o * a.scales_outer + i * a.scales_row : -1;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks)
                xf[nt][ks] = ks < a.ksteps ? *reinterpret_cast<const f16x8*>(xrow + 32 * ks) : f16x8{};
        }
    };

    // ---- every head of the group on one block's operand rows
    auto do_heads = [&](const f16x8 (&xf)[NR][KS], const int64_t (&c_off)[NR], const int64_t (&s_off)[NR]) {
        for (int hh = 0; hh < ghe; ++hh) {
            // ---- projection of the head: MT column tiles x NR row tiles
            f32x4 acc[MT][NR];
#pragma unroll
            for (int m = 0; m < MT; ++m)
#pragma unroll
                for (int nt = 0; nt < NR; ++nt) acc[m][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
            const _Float16* wh = wa + hh * a.dp * a.xp;
            // all KS steps and MT tiles: past `ksteps`, and in each head's padding rows, the
            // operands are zero, so the MFMA chain has no branch
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    const f16x8 av = *reinterpret_cast<const f16x8*>(wh + 16 * m * a.xp + 32 * ks);
#pragma unroll
                    for (int nt = 0; nt < NR; ++nt)
                        acc[m][nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, xf[nt][ks], acc[m][nt], 0, 0, 0);
                }
            }
            // operand reads two steps ahead of the MFMAs that use them
            __builtin_amdgcn_sched_group_barrier(0x100, 2 * MT, 0);
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                __builtin_amdgcn_sched_group_barrier(0x008, MT * NR, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, MT, 0);
            }

            // ---- quantize: lane holds columns 16m + 4g + [0, 4) of row (lane & 15)
#pragma unroll
            for (int nt = 0; nt < NR; ++nt) {
                uint16_t hv[MT][4];
                uint32_t key = 0;
#pragma unroll
                for (int m = 0; m < MT; ++m) {
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        hv[m][q] = f32_to_f16(acc[m][nt][q]);
                        const uint32_t k = abs_key<NORI_F16>(hv[m][q]);
                        key = max(key, m < MT - 1 || pad_ok[q] ? k : 0u);
                    }
                }
                // the row's 4 lanes (lane ^ 16, lane ^ 32): lane swaps on the VALU
                {
                    const auto s16 = __builtin_amdgcn_permlane16_swap(key, key, false, false);
                    key = max(s16[0], s16[1]);
                    const auto s32 = __builtin_amdgcn_permlane32_swap(key, key, false, false);
                    key = max(s32[0], s32[1]);
                }
                const VectorScale vs = make_scale_f16_fast(key);  // both scale_div modes
                uint32_t words[MT];
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    float q[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        // t * RN(1/s): with a normal fp16 scale its code is the quotient's
                        q[i] = f16_to_f32(hv[m][i]) * vs.y;
                    }
                    words[m] = pack_codes_fast<NORI_F16>(q);
                }
                // scales outside the fast quotient's range (zero, subnormal or huge vectors, NaN):
                // recode exactly, on a wave-uniform branch that is almost never taken
                if (__builtin_expect(__builtin_amdgcn_ballot_w64(!vs.fast) != 0, 0)) {
                    if (!vs.fast) {
#pragma unroll
                        for (int m = 0; m < MT; ++m)
                            words[m] = pack4(code_of<NORI_F16>(f16_to_f32(hv[m][0]), vs), code_of<NORI_F16>(f16_to_f32(hv[m][1]), vs),
                                             code_of<NORI_F16>(f16_to_f32(hv[m][2]), vs), code_of<NORI_F16>(f16_to_f32(hv[m][3]), vs));
                    }
                }
                if (c_off[nt] >= 0) {
                    int8_t* crow = a.codes + c_off[nt] + (int64_t)(head0 + hh) * a.d;
#pragma unroll
                    for (int m = 0; m < MT; ++m)
                        if (16 * m + 4 * g < a.d) *reinterpret_cast<uint32_t*>(crow + 16 * m + 4 * g) = words[m];
                    if (g == 0) a.scales[s_off[nt] + head0 + hh] = vs.s;
                }
            }
        }
    };

    // blocks stream, stream + streams, ...: the next block's operand rows load while this
    // block's heads compute (two register sets, used in turn)
    int64_t rb = stream;
    if (rb >= a.nblocks) return;
    f16x8 xa[NR][KS], xb[NR][KS];
    int64_t ca[NR], sa[NR], cb[NR], sb[NR];
    load_rows(rb, xa, ca, sa);
    for (;;) {
        int64_t nb = rb + a.streams;
        if (nb < a.nblocks) load_rows(nb, xb, cb, sb);
        do_heads(xa, ca, sa);
        if (nb >= a.nblocks) break;
        rb = nb;
        nb = rb + a.streams;
        if (nb < a.nblocks) load_rows(nb, xa, ca, sa);
        do_heads(xb, cb, sb);
        if (nb >= a.nblocks) break;
        rb = nb;
    }
}

template <int NR, int KS, int MT>
int launch_with(const ProjArgs& a, size_t lds, hipStream_t stream) {
    const dim3 grid((unsigned)(a.streams * a.ngroups));
    if (hipFuncSetAttribute((const void*)kv_project_quantize_kernel<NR, KS, MT>,
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
        return fail(NORI_ERR_RUNTIME, "kv_project_quantize_int8: cannot reserve %zu bytes of LDS", lds);
    hipLaunchKernelGGL((kv_project_quantize_kernel<NR, KS, MT>), grid, dim3(kThreads), lds, stream, a);
    return launch_status("kv_project_quantize_int8");
}

template <int NR, int KS>
int launch_mt(const ProjArgs& a, size_t lds, hipStream_t stream) {
    switch (a.dp / 16) {
        case 1: return launch_with<NR, KS, 1>(a, lds, stream);
        case 2: return launch_with<NR, KS, 2>(a, lds, stream);
        case 3: return launch_with<NR, KS, 3>(a, lds, stream);
        case 4: return launch_with<NR, KS, 4>(a, lds, stream);
        case 6: return launch_with<NR, KS, 6>(a, lds, stream);
        default: return launch_with<NR, KS, 8>(a, lds, stream);
    }
}

// column tiles per head the kernel is built for (a head padded with zero rows up to them)
int padded_tiles(int d) {
    const int mt = (d + 15) / 16;
    return mt <= 4 ? mt : (mt <= 6 ? 6 : 8);
}

// operand steps the kernel holds in registers (KS >= ksteps; the steps past ksteps are zero)
int padded_steps(int ksteps) {
    for (int k : {4, 8, 11, 12, 16, 24}) if (ksteps <= k) return k;
    return 32;
}

// 16 rows per wavefront (one row tile: eight wavefronts, four per SIMD across the two
// workgroups of a CU, hide the per-head chain better than four wavefronts of two tiles)
int launch(ProjArgs& a, int kpad, size_t lds, hipStream_t stream) {
    a.bm = kWaves * 16;
    a.nblocks = (a.grid.rows + a.bm - 1) / a.bm;
    const int64_t slots = (int64_t)device_cus() * (lds <= kLds / kWgPerCu ? kWgPerCu : 1);
    a.streams = (int)std::max<int64_t>(1, std::min<int64_t>(a.nblocks, slots / a.ngroups));
    switch (kpad) {
        case 4: return launch_mt<1, 4>(a, lds, stream);
        case 8: return launch_mt<1, 8>(a, lds, stream);
        case 11: return launch_mt<1, 11>(a, lds, stream);
        case 12: return launch_mt<1, 12>(a, lds, stream);
        case 16: return launch_mt<1, 16>(a, lds, stream);
        case 24: return launch_mt<1, 24>(a, lds, stream);
        default: return launch_mt<1, 32>(a, lds, stream);
    }
}

// x feeds the MFMAs as it is: f16, no norm, whole 32-element steps
bool direct_operands(int x_dtype, int32_t embed, int32_t norm) {
    return x_dtype == NORI_F16 && !norm && embed % 32 == 0;
}

// ------------------------------------------------------------------ one pass from fp32 rows
// Every head of a row block in one workgroup: each fp32 row is read and normalized once, in
// the registers that feed the MFMAs, and the f16 weights stream through LDS one head at a time
// (two tile buffers: the next head's tile loads while this head computes, one barrier per
// head). The barrier would keep every wave of the CU in the same phase -- all multiplying,
// then all quantizing -- so half the waves (one of the two on each SIMD) run half a head
// behind: each quantizes head h - 1 before multiplying head h, and the MFMA and quantizer work
// of the two halves overlap. No
// operand-row pass and no workspace; each 704-byte code row is written by one workgroup.
struct RowsArgs {
    const float* x; Grid grid; int64_t x_outer, x_row;  // fp32 rows (elements)
    int norm; float eps;
    const _Float16* w; int64_t w_stride;  // f16 W [nheads * d, embed] (row stride in elements)
    int embed, nheads, d;
    int8_t* codes; int64_t codes_outer, codes_row;
    float* scales; int64_t scales_outer, scales_row;
    int64_t nblocks;  // blocks of kWaves * 16 rows
};

template <int KS, int MT>
__global__ void __launch_bounds__(kThreads, 2) kv_rows_kernel(const RowsArgs a) {
    constexpr int XP = 32 * KS + 8;  // LDS pitch of a weight row (f16): +16 bytes spreads the 16-row reads
    constexpr int DP = 16 * MT;      // weight rows per head tile, zero past d
    constexpr int CPR = 4 * KS;      // 16-byte chunks of a padded weight row
    constexpr int TILE = DP * XP;    // f16 per tile buffer
    constexpr int WCH = (DP * CPR + kThreads - 1) / kThreads;  // chunks per thread per tile
    extern __shared__ __attribute__((aligned(16))) _Float16 wt[];  // [2][DP][XP]

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int g = lane >> 4;  // result lanes hold columns 4g..4g+3 of each 16-column tile

    // this thread's 16-byte chunks of a head tile: their weight offset within a head's rows (-1:
    // zero padding past d or past embed) and their LDS offset, the same for every head
    int64_t w_off[WCH];
    int l_off[WCH];
#pragma unroll
    for (int u = 0; u < WCH; ++u) {
        const int c = tid + kThreads * u;
        const int row = c / CPR, col = c - row * CPR;
        w_off[u] = c < DP * CPR && row < a.d && col * 8 < a.embed ? (int64_t)row * a.w_stride + col * 8 : -1;
        l_off[u] = c < DP * CPR ? row * XP + col * 8 : -1;
    }
    const int64_t head_stride = (int64_t)a.d * a.w_stride;
    // head h's weight rows, f16, zero past d and past embed, as 16-byte chunks of this thread
    auto load_tile = [&](int h, uint4 (&wr)[WCH]) {
        const _Float16* wh = a.w + h * head_stride;
#pragma unroll
        for (int u = 0; u < WCH; ++u)
            wr[u] = w_off[u] >= 0 ? *reinterpret_cast<const uint4*>(wh + w_off[u]) : uint4{0u, 0u, 0u, 0u};
    };
    auto store_tile = [&](int buf, const uint4 (&wr)[WCH]) {
#pragma unroll
        for (int u = 0; u < WCH; ++u)
            if (l_off[u] >= 0) *reinterpret_cast<uint4*>(wt + buf * TILE + l_off[u]) = wr[u];
    };

    int64_t rb = blockIdx.x;
    if (rb >= a.nblocks) return;  // whole workgroup
    uint4 wr[WCH];
    load_tile(0, wr);
    store_tile(0, wr);
    __syncthreads();
    int buf = 0;  // the buffer holding the current head's tile

    const _Float16* wa = wt + (lane & 15) * XP + 8 * g;  // A operand rows of tile 0
    bool pad_ok[4];  // columns of the last tile past d are zero padding: left out of the absmax
#pragma unroll
    for (int q = 0; q < 4; ++q) pad_ok[q] = 16 * (MT - 1) + 4 * g + q < a.d;

    // quantize + store one head's 16 rows: lane holds columns 16m + 4g + [0, 4) of row (lane & 15)
    auto quant = [&](const f32x4 (&acc)[MT], int hd, int64_t c_off, int64_t s_off) {
        uint16_t hv[MT][4];
        uint32_t key = 0;
#pragma unroll
        for (int m = 0; m < MT; ++m) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                hv[m][q] = f32_to_f16(acc[m][q]);
                const uint32_t k = abs_key<NORI_F16>(hv[m][q]);
                key = max(key, m < MT - 1 || pad_ok[q] ? k : 0u);
            }
        }
        {
            const auto s16 = __builtin_amdgcn_permlane16_swap(key, key, false, false);
            key = max(s16[0], s16[1]);
            const auto s32 = __builtin_amdgcn_permlane32_swap(key, key, false, false);
            key = max(s32[0], s32[1]);
        }
        const VectorScale vs = make_scale_f16_fast(key);  // both scale_div modes
        uint32_t words[MT];
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            float q[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                // t * RN(1/s): with a normal fp16 scale its code is the quotient's
                q[e] = f16_to_f32(hv[m][e]) * vs.y;
            }
            words[m] = pack_codes_fast<NORI_F16>(q);
        }
        // scales outside the fast quotient's range: recode exactly, on a wave-uniform branch
        if (__builtin_expect(__builtin_amdgcn_ballot_w64(!vs.fast) != 0, 0)) {
            if (!vs.fast) {
#pragma unroll
                for (int m = 0; m < MT; ++m)
                words[m] = pack4(code_of<NORI_F16>(f16_to_f32(hv[m][0]), vs), code_of<NORI_F16>(f16_to_f32(hv[m][1]), vs),
                             code_of<NORI_F16>(f16_to_f32(hv[m][2]), vs), code_of<NORI_F16>(f16_to_f32(hv[m][3]), vs));
            }
        }
        if (c_off >= 0) {
            int8_t* crow = a.codes + c_off + (int64_t)hd * a.d;
#pragma unroll
            for (int m = 0; m < MT; ++m)
                if (16 * m + 4 * g < a.d) *reinterpret_cast<uint32_t*>(crow + 16 * m + 4 * g) = words[m];
            if (g == 0) a.scales[s_off + hd] = vs.s;
        }
    };
    // half the waves run half a head behind: they quantize head h - 1 while the others multiply head h
    // (waves 4-7: wave w shares a SIMD with wave w ^ 4, so each SIMD holds one of each)
    const bool lag = (wave >> 2) & 1;
    f32x4 prev[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) prev[m] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (; rb < a.nblocks; rb += gridDim.x) {
        // ---- this wavefront's 16 rows: lane n + 16 g holds row n's elements 32 ks + 8 g + [0, 8)
        const int64_t r = rb * (kWaves * 16) + wave * 16 + (lane & 15);
        const bool valid = r < a.grid.rows;
        const int64_t rr = valid ? r : a.grid.rows - 1;  // rows past the last read the last, store nothing
        const int64_t o = rr / a.grid.n_inner, i = rr - o * a.grid.n_inner;
        const float* xrow = a.x + o * a.x_outer + i * a.x_row + 8 * g;
        const int64_t c_off = valid ? o * a.codes_outer + i * a.codes_row : -1;
        const int64_t s_off = valid ? o * a.scales_outer + i * a.scales_row : -1;
        f16x8 xf[KS];
        {
            f32x4 v[KS][2];
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const bool in = 32 * ks + 8 * g < a.embed;  // embed is a multiple of 8
                v[ks][0] = in ? *reinterpret_cast<const f32x4*>(xrow + 32 * ks) : f32x4{0.f, 0.f, 0.f, 0.f};
                v[ks][1] = in ? *reinterpret_cast<const f32x4*>(xrow + 32 * ks + 4) : f32x4{0.f, 0.f, 0.f, 0.f};
            }
            float inv = 1.0f;
            if (a.norm) {
                float ss = 0.0f;
#pragma unroll
                for (int ks = 0; ks < KS; ++ks)
#pragma unroll
                    for (int h = 0; h < 2; ++h)
#pragma unroll
                        for (int e = 0; e < 4; ++e) ss = fmaf(v[ks][h][e], v[ks][h][e], ss);
                // the row's four lanes (lane ^ 16, lane ^ 32)
                const auto s16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(ss), __float_as_uint(ss), false, false);
                ss = __uint_as_float(s16[0]) + __uint_as_float(s16[1]);
                const auto s32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(ss), __float_as_uint(ss), false, false);
                ss = __uint_as_float(s32[0]) + __uint_as_float(s32[1]);
                inv = rsqrtf(ss / (float)a.embed + a.eps);
            }
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                f16x8 h;
#pragma unroll
                for (int e = 0; e < 8; ++e) h[e] = (_Float16)pin_f32(v[ks][e >> 2][e & 3] * inv);
                xf[ks] = h;
            }
        }

        for (int hd = 0; hd < a.nheads; ++hd) {
            // the next tile: this block's next head, or the next block's first
            const bool more = hd + 1 < a.nheads || rb + gridDim.x < a.nblocks;
            if (more) load_tile(hd + 1 < a.nheads ? hd + 1 : 0, wr);

            if (lag && hd > 0) quant(prev, hd - 1, c_off, s_off);
            f32x4 acc[MT];
#pragma unroll
            for (int m = 0; m < MT; ++m) acc[m] = f32x4{0.f, 0.f, 0.f, 0.f};
            const _Float16* wh = wa + buf * TILE;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    const f16x8 av = *reinterpret_cast<const f16x8*>(wh + 16 * m * XP + 32 * ks);
                    acc[m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, xf[ks], acc[m], 0, 0, 0);
                }
            }

            if (!lag) quant(acc, hd, c_off, s_off);
            else {
#pragma unroll
                for (int m = 0; m < MT; ++m) prev[m] = acc[m];
            }

            if (more) store_tile(buf ^ 1, wr);
            __syncthreads();  // the next tile is in place; every wave is done with this one
            buf ^= 1;
        }
        if (lag) quant(prev, a.nheads - 1, c_off, s_off);
    }
}

template <int KS, int MT>
int launch_rows_with(const RowsArgs& a, hipStream_t stream) {
    const size_t lds = (size_t)2 * 16 * MT * (32 * KS + 8) * 2;
    if (hipFuncSetAttribute((const void*)kv_rows_kernel<KS, MT>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) !=
        hipSuccess)
        return fail(NORI_ERR_RUNTIME, "kv_project_quantize_int8: cannot reserve %zu bytes of LDS", lds);
    // one round of resident workgroups (registers hold one per CU at nori-30m's shape), each
    // walking its share of the row blocks
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kv_rows_kernel<KS, MT>, kThreads, lds) != hipSuccess ||
        per_cu < 1)
        per_cu = 1;
    const int64_t slots = (int64_t)device_cus() * per_cu;
    const dim3 grid((unsigned)std::min<int64_t>(a.nblocks, slots));
    hipLaunchKernelGGL((kv_rows_kernel<KS, MT>), grid, dim3(kThreads), lds, stream, a);
    return launch_status("kv_project_quantize_int8 (one pass)");
}

// The one-pass kernel takes fp32 rows with f16 weights, embed a multiple of 8 up to 384 (the
// row's fp32 values are held in registers while the norm is taken) and two head tiles within
// half the LDS (two workgroups per CU).
bool one_pass(int x_dtype, int weight_dtype, int32_t embed, int32_t d) {
    if (x_dtype != NORI_F32 || weight_dtype != NORI_F16 || embed % 8 || embed > 384 || d > 64) return false;
    const int kpad = padded_steps((embed + 31) / 32);
    const int mt = padded_tiles(d);
    return (size_t)2 * 16 * mt * (32 * kpad + 8) * 2 <= kLds / kWgPerCu;
}

int launch_rows(RowsArgs& a, hipStream_t stream) {
    a.nblocks = (a.grid.rows + kWaves * 16 - 1) / (kWaves * 16);
    const int kpad = padded_steps((a.embed + 31) / 32);
    const int mt = padded_tiles(a.d);
#define NORI_ROWS_MT(KS_)                                          \
    switch (mt) {                                                  \
        case 1: return launch_rows_with<KS_, 1>(a, stream);        \
        case 2: return launch_rows_with<KS_, 2>(a, stream);        \
        case 3: return launch_rows_with<KS_, 3>(a, stream);        \
        default: return launch_rows_with<KS_, 4>(a, stream);       \
    }
    switch (kpad) {
        case 4: NORI_ROWS_MT(4)
        case 8: NORI_ROWS_MT(8)
        case 11: NORI_ROWS_MT(11)
        default: NORI_ROWS_MT(12)
    }
#undef NORI_ROWS_MT
}


}  // namespace

extern "C" int64_t nori_kv_project_quantize_int8_workspace_size(int x_dtype, int64_t n_outer, int64_t n_inner,
                                                               int32_t embed, int32_t norm) {
    if (n_outer <= 0 || n_inner <= 0 || embed <= 0 || direct_operands(x_dtype, embed, norm)) return 0;
    if (n_inner > INT64_MAX / n_outer) return 0;
    return n_outer * n_inner * (int64_t)((embed + 31) / 32 * 32) * 2;
}

extern "C" int64_t nori_kv_project_quantize_int8_workspace_bytes(int x_dtype, int64_t n_outer, int64_t n_inner,
                                                                int32_t embed, int32_t norm, int weight_dtype,
                                                                int32_t d) {
    if (one_pass(x_dtype, weight_dtype, embed, d)) return 0;
    return nori_kv_project_quantize_int8_workspace_size(x_dtype, n_outer, n_inner, embed, norm);
}

extern "C" int nori_kv_project_quantize_int8(const void* x, int x_dtype, int64_t n_outer, int64_t n_inner,
                                            int32_t embed, int64_t x_outer_stride, int64_t x_row_stride, int32_t norm,
                                            float eps, const void* weight, int weight_dtype, int64_t w_row_stride,
                                            int32_t kv_heads, int32_t d, int8_t* codes, int64_t codes_outer_stride,
                                            int64_t codes_row_stride, float* scales, int64_t scales_outer_stride,
                                            int64_t scales_row_stride, int32_t scale_div, void* workspace,
                                            int64_t workspace_bytes, void* stream_v) {
    clear_error();
    if (n_outer < 0 || n_inner < 0 || embed <= 0 || kv_heads <= 0 || d <= 0)
        return fail(NORI_ERR_INVALID, "kv_project_quantize_int8: bad shape n_outer=%lld n_inner=%lld embed=%d kv_heads=%d d=%d",
                    (long long)n_outer, (long long)n_inner, embed, kv_heads, d);
    if (x_dtype != NORI_F32 && x_dtype != NORI_F16 && x_dtype != NORI_BF16)
        return fail(NORI_ERR_UNSUPPORTED, "kv_project_quantize_int8: unsupported input dtype %s", dtype_name(x_dtype));
    if (weight_dtype != NORI_F32 && weight_dtype != NORI_F16 && weight_dtype != NORI_BF16)
        return fail(NORI_ERR_UNSUPPORTED, "kv_project_quantize_int8: unsupported weight dtype %s",
                    dtype_name(weight_dtype));
    if (scale_div != NORI_SCALE_DIV_TRUE && scale_div != NORI_SCALE_DIV_RECIP)
        return fail(NORI_ERR_INVALID, "kv_project_quantize_int8: unknown scale_div %d", scale_div);
    if (d % 4 || d > 128)
        return fail(NORI_ERR_UNSUPPORTED, "kv_project_quantize_int8: head width %d is not a multiple of 4 up to 128", d);
    // an operand row is held in registers: at most 32 steps of 32 elements
    if (embed > 1024)
        return fail(NORI_ERR_UNSUPPORTED, "kv_project_quantize_int8: embed %d exceeds 1024", embed);
    if (n_outer == 0 || n_inner == 0) return NORI_OK;
    if (n_inner > INT64_MAX / n_outer)
        return fail(NORI_ERR_INVALID, "kv_project_quantize_int8: %lld x %lld rows overflow", (long long)n_outer,
                    (long long)n_inner);
    if (!x || !weight || !codes || !scales) return fail(NORI_ERR_INVALID, "kv_project_quantize_int8: null pointer");
    // 16-byte row chunks of x and W, 4-byte code words
    const int xes = dtype_size(x_dtype), wes = dtype_size(weight_dtype);
    if (embed % (16 / xes) || embed % (16 / wes) || (uintptr_t)x % 16 || (x_row_stride * xes) % 16 ||
        (x_outer_stride * xes) % 16 || (uintptr_t)weight % 16 || (w_row_stride * wes) % 16)
        return fail(NORI_ERR_UNSUPPORTED,
                    "kv_project_quantize_int8: x and weight rows must be 16-byte aligned whole 16-byte chunks");
    if ((uintptr_t)codes % 4 || codes_row_stride % 4 || codes_outer_stride % 4)
        return fail(NORI_ERR_UNSUPPORTED, "kv_project_quantize_int8: code rows must be 4-byte aligned");
    const Grid grid{n_outer * n_inner, n_inner};
    hipStream_t stream = (hipStream_t)stream_v;
    if (one_pass(x_dtype, weight_dtype, embed, d)) {
        RowsArgs r;
        r.x = reinterpret_cast<const float*>(x); r.grid = grid; r.x_outer = x_outer_stride; r.x_row = x_row_stride;
        r.norm = norm; r.eps = eps;
        r.w = reinterpret_cast<const _Float16*>(weight); r.w_stride = w_row_stride;
        r.embed = embed; r.nheads = 2 * kv_heads; r.d = d;
        r.codes = codes; r.codes_outer = codes_outer_stride; r.codes_row = codes_row_stride;
        r.scales = scales; r.scales_outer = scales_outer_stride; r.scales_row = scales_row_stride;
        return launch_rows(r, stream);
    }
    const int64_t ws_need = nori_kv_project_quantize_int8_workspace_size(x_dtype, n_outer, n_inner, embed, norm);
    if (ws_need > 0 && (!workspace || workspace_bytes < ws_need || (uintptr_t)workspace % 16))
        return fail(NORI_ERR_INVALID, "kv_project_quantize_int8: needs a 16-byte aligned workspace of %lld bytes",
                    (long long)ws_need);

    const int ksteps = (embed + 31) / 32;

    ProjArgs a;
    a.grid = grid;
    if (ws_need > 0) {
        PrepArgs p;
        p.x = x; p.grid = grid; p.embed = embed; p.x_outer = x_outer_stride; p.x_row = x_row_stride;
        p.norm = norm; p.eps = eps;
        p.ws = reinterpret_cast<_Float16*>(workspace); p.pitch = 32 * ksteps;
        const int64_t waves = std::min<int64_t>((grid.rows + kPrepRows - 1) / kPrepRows, (int64_t)device_cus() * 16);
        const dim3 pgrid((unsigned)((waves + kPrepWaves - 1) / kPrepWaves));
        NORI_DISPATCH_FLOAT(x_dtype, XDT,
                            hipLaunchKernelGGL((prep_rows_kernel<XDT>), pgrid, dim3(kPrepWaves * 64), 0, stream, p));
        const int st = launch_status("kv_project_quantize_int8 (operand rows)");
        if (st != NORI_OK) return st;
        a.xs = p.ws; a.xs_outer = n_inner * (int64_t)p.pitch; a.xs_row = p.pitch;
    } else {
        a.xs = reinterpret_cast<const _Float16*>(x); a.xs_outer = x_outer_stride; a.xs_row = x_row_stride;
    }
    a.w = weight; a.wdt = weight_dtype; a.w_stride = w_row_stride;
    a.embed = embed;
    a.nheads = 2 * kv_heads; a.d = d; a.dp = 16 * padded_tiles(d);
    a.ksteps = ksteps;
    const int kpad = padded_steps(ksteps);
    a.xp = 32 * kpad + 8;  // +16 bytes per row: the 16-byte operand reads of 16 rows spread over the banks
    a.codes = codes; a.codes_outer = codes_outer_stride; a.codes_row = codes_row_stride;
    a.scales = scales; a.scales_outer = scales_outer_stride; a.scales_row = scales_row_stride;
    a.scale_div = scale_div;
    // heads per group: as many as fit half the LDS (two workgroups per CU), else the whole LDS,
    // then spread evenly over the groups
    const size_t head_bytes = (size_t)a.dp * a.xp * 2;
    if (head_bytes > kLds)
        return fail(NORI_ERR_UNSUPPORTED, "kv_project_quantize_int8: embed %d x head width %d exceeds the LDS", embed, d);
    const size_t budget = head_bytes <= kLds / kWgPerCu ? kLds / kWgPerCu : kLds;
    const int hg_max = std::min<int>(a.nheads, (int)(budget / head_bytes));
    a.ngroups = (a.nheads + hg_max - 1) / hg_max;
    a.hg = (a.nheads + a.ngroups - 1) / a.ngroups;
    return launch(a, kpad, (size_t)a.hg * head_bytes, stream);
}

namespace {

__global__ void __launch_bounds__(256) f16_scale_probe_kernel(const uint16_t* absmax, int64_t n, float* s, float* y) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const VectorScale vs = make_scale_f16_fast(abs_key<NORI_F16>(absmax[i]));
    s[i] = vs.s;
    y[i] = vs.y;
}

}  // namespace

extern "C" int nori_quant_f16_scale_probe(const uint16_t* absmax, int64_t n, float* s, float* y, void* stream) {
    clear_error();
    if (n < 0 || n > ((int64_t)1 << 30))
        return fail(NORI_ERR_INVALID, "quant_f16_scale_probe: n=%lld outside [0, 2^30]", (long long)n);
    if (n == 0) return NORI_OK;
    if (!absmax || !s || !y) return fail(NORI_ERR_INVALID, "quant_f16_scale_probe: null pointer");
    hipLaunchKernelGGL(f16_scale_probe_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       absmax, n, s, y);
    return launch_status("quant_f16_scale_probe");
}
