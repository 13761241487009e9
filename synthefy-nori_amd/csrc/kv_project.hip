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
// so the fp16 K/V of the layer never exist in HBM: the projection is rounded in LDS and
// quantized there.
//
// Schedule. Persistent workgroups of 4 wavefronts. A workgroup owns a group of `hg` cache
// heads: their weight rows, each padded to a multiple of 16 with zero rows, stay in LDS as f16
// for the whole launch; it walks row blocks of 64 context rows. Per block, the x tile is
// loaded (and normalized) into LDS as f16; each wavefront projects 16 rows onto the group's
// heads with v_mfma_f32_16x16x32_f16 (the embed width in steps of 32), rounds its 16 x (hg*dp)
// results to f16 into its own LDS tile, and quantizes its 16*hg head vectors from there
// (lanes split each vector; the absmax is exchanged with lane shuffles), staging the codes in
// LDS for coalesced stores. Workgroups are numbered so the head groups of one row block sit
// on one XCD and share its L2 for the x rows.
#include <math.h>

#include <algorithm>

#include "nori_common.h"
#include "quant_common.h"

#pragma clang fp contract(off)

namespace {

using namespace nori;
using namespace nori::quant;

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kBM = 64;             // context rows per block (16 per wavefront)
constexpr int kRowThreads = kThreads / kBM;  // threads that load one x row

// Rows are addressed on a two-level grid, row r = o * n_inner + i (o < n_outer, i < n_inner):
// x at o * x_outer + i * x_row elements, codes at o * codes_outer + i * codes_row bytes, scales at
// o * scales_outer + i * scales_row floats -- so a slice of rows of a [BG, N, ...] cache, or the
// rows of a [N, G, E] activation read group by group, is one launch.
struct ProjArgs {
    const void* x; int64_t rows, n_inner; int embed; int64_t x_outer, x_row;  // x rows of embed elements
    int norm; float eps;
    const void* w; int64_t w_stride;                            // W [2*kv_heads*d, embed]
    int nheads;  // 2 * kv_heads cache head vectors per row
    int d, dp;   // head width, padded to 16
    int hg;      // heads per group (the last group may hold fewer)
    int ngroups;
    int ep, xp;  // embed padded to 32, LDS row pitch of the x and W tiles (f16 elements)
    int8_t* codes; int64_t codes_outer, codes_row;  // codes: nheads*d bytes per row
    float* scales; int64_t scales_outer, scales_row;  // scales: nheads floats per row
    int scale_div;
    int64_t nblocks;  // row blocks
    int streams;      // workgroups per head group
};

// elements of one 16-byte chunk of dtype DT, as f32
template <int DT>
__device__ __forceinline__ void load_chunk(const void* base, int64_t elem, float* f) {
    if constexpr (DT == NORI_F32) {
        const float4 v = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(base) + elem);
        f[0] = v.x; f[1] = v.y; f[2] = v.z; f[3] = v.w;
    } else {
        const uint4 v = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(base) + elem);
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
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

// The row of `embed` elements at element offset `base` into an LDS row of f16, zero-padded to
// `ep` (all zeros when !valid), optionally RMS-normalized (rounded to DT first, as RMSNorm
// returns DT). The kRowThreads threads of a row split its 16-byte chunks and reduce the
// statistic together.
template <int DT>
__device__ __forceinline__ void load_row(const void* src, int64_t base, bool valid, int embed, int ep, bool norm,
                                         float eps, _Float16* dst, int q) {
    constexpr int EPC = DT == NORI_F32 ? 4 : 8;  // elements per 16-byte chunk
    const int nchunks = embed / EPC;
    float acc = 0.0f;
    if (norm) {
        for (int c = q; c < nchunks; c += kRowThreads) {
            float f[EPC];
            if (valid) load_chunk<DT>(src, base + (int64_t)c * EPC, f);
            else for (int e = 0; e < EPC; ++e) f[e] = 0.0f;
#pragma unroll
            for (int e = 0; e < EPC; ++e) acc = fmaf(f[e], f[e], acc);
        }
#pragma unroll
        for (int off = kRowThreads / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off, kRowThreads);
    }
    const float inv = norm ? rsqrtf(acc / (float)embed + eps) : 1.0f;
    for (int c = q; c < ep / EPC; c += kRowThreads) {
        float f[EPC];
        if (valid && c < nchunks) load_chunk<DT>(src, base + (int64_t)c * EPC, f);
        else for (int e = 0; e < EPC; ++e) f[e] = 0.0f;
        _Float16 h[EPC];
#pragma unroll
        for (int e = 0; e < EPC; ++e) h[e] = (_Float16)pin_f32(norm ? round_to<DT>(f[e] * inv) : f[e]);
        if constexpr (EPC == 8) {
            *reinterpret_cast<f16x8*>(dst + c * EPC) = f16x8{h[0], h[1], h[2], h[3], h[4], h[5], h[6], h[7]};
        } else {
            *reinterpret_cast<f16x2*>(dst + c * EPC) = f16x2{h[0], h[1]};
            *reinterpret_cast<f16x2*>(dst + c * EPC + 2) = f16x2{h[2], h[3]};
        }
    }
}

template <int XDT, int WDT, int NT>
__global__ void __launch_bounds__(kThreads) kv_project_quantize_kernel(const ProjArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    __shared__ int64_t row_x[kBM], row_c[kBM], row_s[kBM];  // this block's row offsets (-1: past the end)
    // LDS: x tile [kBM][xp] f16 | W group [hg*dp][xp] f16 | per-wave f16 results [kBM][hg*dp] |
    //      per-wave codes [kBM][hg*d]
    const int gc = a.hg * a.dp;  // group columns (padded)
    _Float16* xt = reinterpret_cast<_Float16*>(smem);
    _Float16* wt = xt + kBM * a.xp;
    _Float16* kvt = wt + gc * a.xp;
    int8_t* ct = reinterpret_cast<int8_t*>(kvt + kBM * gc);

    // work: XCD-aware numbering, the head groups of a stream consecutive within one XCD
    const int nwg = (int)gridDim.x;
    const int wg = (int)blockIdx.x;
    const int t = (wg % 8) * (nwg / 8) + min(wg % 8, nwg % 8) + wg / 8;
    const int group = t % a.ngroups;
    const int stream = t / a.ngroups;
    const int head0 = group * a.hg;
    const int ghe = min(a.hg, a.nheads - head0);  // heads in this group

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int lr = tid / kRowThreads, lq = tid % kRowThreads;

    // weight rows of the group, zero rows in the padding of each head and past the last head
    for (int c = lr; c < gc; c += kBM) {
        const int hh = c / a.dp, e = c % a.dp;
        const bool valid = hh < ghe && e < a.d;
        load_row<WDT>(a.w, ((int64_t)(head0 + hh) * a.d + e) * a.w_stride, valid, a.embed, a.ep, false, 0.0f,
                      wt + c * a.xp, lq);
    }

    _Float16* kv_w = kvt + wave * 16 * gc;  // this wavefront's 16 rows of results
    int8_t* ct_w = ct + wave * 16 * (a.hg * a.d);
    const int ksteps = a.ep / 32;
    for (int64_t rb = stream; rb < a.nblocks; rb += a.streams) {
        const int64_t r0 = rb * kBM;
        __syncthreads();  // the previous block's tiles and offsets are no longer read; W is loaded
        if (tid < kBM) {
            const int64_t r = r0 + tid;
            const int64_t o = r / a.n_inner, i = r - o * a.n_inner;
            const bool in = r < a.rows;
            row_x[tid] = in ? o * a.x_outer + i * a.x_row : -1;
            row_c[tid] = in ? o * a.codes_outer + i * a.codes_row : -1;
            row_s[tid] = in ? o * a.scales_outer + i * a.scales_row : -1;
        }
        __syncthreads();
        const int64_t xoff = row_x[lr];
        load_row<XDT>(a.x, xoff, xoff >= 0, a.embed, a.ep, a.norm != 0, a.eps, xt + lr * a.xp, lq);
        __syncthreads();

        // ---- projection: 16 rows x gc columns per wavefront
        f32x4 acc[NT];
#pragma unroll
        for (int n = 0; n < NT; ++n) acc[n] = f32x4{0.f, 0.f, 0.f, 0.f};
        const _Float16* xa = xt + (wave * 16 + (lane & 15)) * a.xp + 8 * (lane >> 4);
        const _Float16* wb = wt + (lane & 15) * a.xp + 8 * (lane >> 4);
        for (int ks = 0; ks < ksteps; ++ks) {
            const f16x8 av = *reinterpret_cast<const f16x8*>(xa + 32 * ks);
#pragma unroll
            for (int n = 0; n < NT; ++n) {
                if (16 * n < gc) {
                    const f16x8 bv = *reinterpret_cast<const f16x8*>(wb + 16 * n * a.xp + 32 * ks);
                    acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, acc[n], 0, 0, 0);
                }
            }
        }
        // f16 results: lane holds column 16n + lane%16 of rows 4*(lane/16) + i
#pragma unroll
        for (int n = 0; n < NT; ++n) {
            if (16 * n < gc) {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    kv_w[(4 * (lane >> 4) + i) * gc + 16 * n + (lane & 15)] = (_Float16)pin_f32(acc[n][i]);
            }
        }
        __syncthreads();  // results visible across the lanes that quantize them

        // ---- quantize the wavefront's 16 * ghe head vectors: lpv lanes per vector
        const int nvec = 16 * ghe;
        const int lpv = nvec >= 64 ? 1 : (nvec >= 32 ? 2 : (nvec >= 16 ? 4 : 4));
        const int epl = (a.d + lpv - 1) / lpv;  // elements per lane
        for (int v0 = 0; v0 < nvec; v0 += 64 / lpv) {
            const int v = v0 + lane / lpv, part = lane % lpv;
            const bool on = v < nvec;
            const int row = on ? v % 16 : 0, hh = on ? v / 16 : 0;
            const int e0 = part * epl, e1 = min(a.d, e0 + epl);
            const uint16_t* src = reinterpret_cast<const uint16_t*>(kv_w) + row * gc + hh * a.dp;
            uint32_t key = 0;
            if (on)
                for (int e = e0; e < e1; ++e) key = max(key, abs_key<NORI_F16>(src[e]));
            for (int off = 1; off < lpv; off <<= 1) key = max(key, (uint32_t)__shfl_xor((int)key, off, 64));
            const VectorScale vs = make_scale<NORI_F16>(key, a.scale_div);
            if (on) {
                for (int e = e0; e < e1; ++e)
                    ct_w[row * (a.hg * a.d) + hh * a.d + e] = (int8_t)code_of<NORI_F16>(f16_to_f32(src[e]), vs);
                const int64_t soff = row_s[wave * 16 + row];
                if (part == 0 && soff >= 0) a.scales[soff + head0 + hh] = vs.s;
            }
        }
        __syncthreads();  // staged codes visible across the lanes that store them
        // ---- codes out: each row's ghe*d bytes at its group offset, in 4-byte words
        const int rwords = ghe * a.d / 4;
        for (int i = lane; i < 16 * rwords; i += 64) {
            const int row = i / rwords, wd = i % rwords;
            const int64_t coff = row_c[wave * 16 + row];
            if (coff >= 0)
                *reinterpret_cast<uint32_t*>(a.codes + coff + (int64_t)head0 * a.d + 4 * wd) =
                    *reinterpret_cast<const uint32_t*>(ct_w + row * (a.hg * a.d) + 4 * wd);
        }
    }
}

int device_cus() {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) return 256;
    return cus;
}

size_t lds_bytes(int hg, int dp, int d, int xp) {
    return (size_t)(kBM * xp + hg * dp * xp + kBM * hg * dp) * 2 + (size_t)kBM * hg * d;
}

constexpr size_t kLdsLimit = 160 * 1024 - 3 * kBM * sizeof(int64_t);  // dynamic LDS beside the row offsets

template <int XDT, int WDT>
int launch(const ProjArgs& a, size_t lds, hipStream_t stream) {
    const int nt = a.hg * a.dp / 16;
    const dim3 grid((unsigned)(a.streams * a.ngroups));
#define NORI_PROJ_NT(N)                                                                                          \
    if (nt <= N) {                                                                                              \
        if (hipFuncSetAttribute((const void*)kv_project_quantize_kernel<XDT, WDT, N>,                           \
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)             \
            return fail(NORI_ERR_RUNTIME, "kv_project_quantize_int8: cannot reserve %zu bytes of LDS", lds);     \
        hipLaunchKernelGGL((kv_project_quantize_kernel<XDT, WDT, N>), grid, dim3(kThreads), lds, stream, a);   \
        return launch_status("kv_project_quantize_int8");                                                       \
    }
    NORI_PROJ_NT(4) NORI_PROJ_NT(8) NORI_PROJ_NT(16)
#undef NORI_PROJ_NT
    return fail(NORI_ERR_UNSUPPORTED, "kv_project_quantize_int8: %d column tiles per group", nt);
}

}  // namespace

extern "C" int nori_kv_project_quantize_int8(const void* x, int x_dtype, int64_t n_outer, int64_t n_inner,
                                            int32_t embed, int64_t x_outer_stride, int64_t x_row_stride, int32_t norm,
                                            float eps, const void* weight, int weight_dtype, int64_t w_row_stride,
                                            int32_t kv_heads, int32_t d, int8_t* codes, int64_t codes_outer_stride,
                                            int64_t codes_row_stride, float* scales, int64_t scales_outer_stride,
                                            int64_t scales_row_stride, int32_t scale_div, void* stream_v) {
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
    if (d % 4 || d > 256)
        return fail(NORI_ERR_UNSUPPORTED, "kv_project_quantize_int8: head width %d is not a multiple of 4 up to 256", d);
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

    ProjArgs a;
    a.x = x; a.rows = n_outer * n_inner; a.n_inner = n_inner; a.embed = embed;
    a.x_outer = x_outer_stride; a.x_row = x_row_stride;
    a.norm = norm; a.eps = eps;
    a.w = weight; a.w_stride = w_row_stride;
    a.nheads = 2 * kv_heads; a.d = d; a.dp = (d + 15) / 16 * 16;
    a.ep = (embed + 31) / 32 * 32;
    a.xp = a.ep + 8;  // +16 bytes per row: the 16-byte operand reads of 16 rows spread over the banks
    a.codes = codes; a.codes_outer = codes_outer_stride; a.codes_row = codes_row_stride;
    a.scales = scales; a.scales_outer = scales_outer_stride; a.scales_row = scales_row_stride;
    a.scale_div = scale_div;
    // heads per group: as many as fit the LDS with the x tile (at most 16 column tiles)
    int hg = 1;
    while (hg < a.nheads && (hg + 1) * a.dp <= 256 && lds_bytes(hg + 1, a.dp, d, a.xp) <= kLdsLimit) ++hg;
    if (lds_bytes(hg, a.dp, d, a.xp) > kLdsLimit)
        return fail(NORI_ERR_UNSUPPORTED, "kv_project_quantize_int8: embed %d x head width %d exceeds the LDS", embed, d);
    a.hg = hg;
    a.ngroups = (a.nheads + hg - 1) / hg;
    a.nblocks = (a.rows + kBM - 1) / kBM;
    const int64_t slots = device_cus();
    a.streams = (int)std::max<int64_t>(1, std::min<int64_t>(a.nblocks, slots / a.ngroups));
    const size_t lds = lds_bytes(hg, a.dp, d, a.xp);
    hipStream_t stream = (hipStream_t)stream_v;
    int st = NORI_OK;
    NORI_DISPATCH_FLOAT(x_dtype, XDT, NORI_DISPATCH_FLOAT(weight_dtype, WDT, st = launch<XDT, WDT>(a, lds, stream)));
    return st;
}
