// int8 context K/V cache codec for gfx950: quantize and dequantize head vectors.
//
// Semantics (bit-exact): quantize_int8 / dequantize_int8,
// src/synthefy_nori/model/kv_cache_scaling.py:29-41, evaluated the way torch does it,
// i.e. every op computed in fp32 and its result rounded to the source dtype T:
//   m = amax|t|                (exact; NaN propagates)
//   m = max(m, T(1e-12))       (clamp_min; T(1e-12) is 0 in fp16)
//   s = T(m / 127)             (CPU: IEEE division; ROCm: m * fp32(1/127))
//   c = clamp(rint(T(t / s)), -127, 127)   (t/s is an IEEE fp32 quotient, then T-rounded)
//   scale = float(s)
// Dequantize: T(float(c) * scale).
//
// Schedule. HBM-bound streaming: a workgroup stages a tile of up to 256 vectors that
// are contiguous in memory into LDS with 128-bit loads (any head width: a 44-element
// bf16 vector is 88 bytes and not 16-byte aligned on its own, but 256 of them are),
// each thread then codes one vector out of LDS, the codes go back through LDS and
// leave with 128-bit stores. Vectors that are not contiguous, or too long for the
// tile, take a one-thread-per-vector kernel reading global memory directly.
//
// The per-element quotient t/s uses one IEEE reciprocal per vector and Markstein's
// correction q = fma(fma(-q0, s, t), y, q0), q0 = t*y, y = RN(1/s). For 2^-96 <= s <= 2^96
// it returns the correctly rounded quotient wherever |t/s| >= 1/4 (below that the code is
// 0 whichever quotient is used); checked for every fp16 and bf16 (t, s) pair and for
// random fp32 pairs on the CPU by tests/exact_quotient_check.c. Other vectors (zero,
// tiny, huge, infinite or NaN scale) divide exactly.
#include <algorithm>

#include "nori_common.h"
#include "quant_common.h"

// torch rounds the result of every op separately; no multiply-add is fused here unless
// the source writes fmaf. (Narrowing conversions are kept apart by pin_f32.)
#pragma clang fp contract(off)

namespace {

using namespace nori;
using namespace nori::quant;

constexpr int kTileThreads = 256;
constexpr int kMaxTileVectorBytes = 128;  // keeps the tile under 48 KiB of LDS; longer vectors use the direct kernel

// Cooperative global -> LDS copy of `nbytes` (a multiple of `elem` bytes).
__device__ __forceinline__ void copy_in(uint8_t* __restrict__ lds, const uint8_t* __restrict__ g, int nbytes,
                                        int elem) {
    const int tid = threadIdx.x;
    int done = 0;
    if ((((uintptr_t)g) & 15) == 0) {
        const int n16 = nbytes >> 4;
        for (int i = tid; i < n16; i += kTileThreads)
            reinterpret_cast<uint4*>(lds)[i] = reinterpret_cast<const uint4*>(g)[i];
        done = n16 << 4;
    }
    if (elem == 4) {
        for (int i = (done >> 2) + tid; i < (nbytes >> 2); i += kTileThreads)
            reinterpret_cast<uint32_t*>(lds)[i] = reinterpret_cast<const uint32_t*>(g)[i];
    } else {
        for (int i = (done >> 1) + tid; i < (nbytes >> 1); i += kTileThreads)
            reinterpret_cast<uint16_t*>(lds)[i] = reinterpret_cast<const uint16_t*>(g)[i];
    }
}

// Cooperative LDS -> global copy of `nbytes` bytes (any count, any alignment >= 1).
__device__ __forceinline__ void copy_out(uint8_t* __restrict__ g, const uint8_t* __restrict__ lds, int nbytes) {
    const int tid = threadIdx.x;
    int done = 0;
    if ((((uintptr_t)g) & 15) == 0) {
        const int n16 = nbytes >> 4;
        for (int i = tid; i < n16; i += kTileThreads)
            reinterpret_cast<uint4*>(g)[i] = reinterpret_cast<const uint4*>(lds)[i];
        done = n16 << 4;
    }
    for (int i = done + tid; i < nbytes; i += kTileThreads) g[i] = lds[i];
}

// ------------------------------------------------------------------ quantize
template <int DT>
__global__ void __launch_bounds__(kTileThreads)
quantize_tile_kernel(const uint8_t* __restrict__ src, int64_t n_inner, int d, int64_t src_outer_bytes,
                     int8_t* __restrict__ codes, int64_t codes_outer, float* __restrict__ scales,
                     int64_t scales_outer, int64_t tiles_per_outer, int scale_div) {
    using S = typename Storage<DT>::T;
    constexpr int es = sizeof(S);
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int64_t tile = blockIdx.x;
    const int64_t o = tile / tiles_per_outer;
    const int64_t v0 = (tile - o * tiles_per_outer) * kTileThreads;
    const int nv = (int)min<int64_t>(kTileThreads, n_inner - v0);
    const int vec_bytes = d * es;
    uint8_t* lds_src = lds;
    uint8_t* lds_codes = lds + ((kTileThreads * vec_bytes + 15) & ~15);

    copy_in(lds_src, src + o * src_outer_bytes + v0 * vec_bytes, nv * vec_bytes, es);
    __syncthreads();

    const int v = threadIdx.x;
    if (v < nv) {
        const S* x = reinterpret_cast<const S*>(lds_src) + (int64_t)v * d;
        uint32_t mk = 0;
        for (int i = 0; i < d; ++i) mk = max(mk, abs_key<DT>(x[i]));
        const VectorScale vs = make_scale<DT>(mk, scale_div);
        uint8_t* c = lds_codes + v * d;
        int i = 0;
        if ((d & 3) == 0) {
            for (; i < d; i += 4) {
                const uint32_t w = pack4(code_of<DT>(bits_to_f32<DT>(x[i]), vs), code_of<DT>(bits_to_f32<DT>(x[i + 1]), vs),
                                         code_of<DT>(bits_to_f32<DT>(x[i + 2]), vs), code_of<DT>(bits_to_f32<DT>(x[i + 3]), vs));
                *reinterpret_cast<uint32_t*>(c + i) = w;
            }
        }
        for (; i < d; ++i) c[i] = (uint8_t)(int8_t)code_of<DT>(bits_to_f32<DT>(x[i]), vs);
        scales[o * scales_outer + v0 + v] = vs.s;
    }
    __syncthreads();
    copy_out(reinterpret_cast<uint8_t*>(codes + o * codes_outer + v0 * d), lds_codes, nv * d);
}

template <int DT>
__global__ void __launch_bounds__(kTileThreads)
quantize_direct_kernel(const void* __restrict__ src_v, int64_t n_outer, int64_t n_inner, int d,
                       int64_t src_outer, int64_t src_inner, int8_t* __restrict__ codes, int64_t codes_outer,
                       int64_t codes_inner, float* __restrict__ scales, int64_t scales_outer,
                       int64_t scales_inner, int scale_div) {
    using S = typename Storage<DT>::T;
    const S* src = reinterpret_cast<const S*>(src_v);
    const int64_t idx = (int64_t)blockIdx.x * kTileThreads + threadIdx.x;
    if (idx >= n_outer * n_inner) return;
    const int64_t o = idx / n_inner, i = idx - o * n_inner;
    const S* x = src + o * src_outer + i * src_inner;
    uint32_t mk = 0;
    for (int e = 0; e < d; ++e) mk = max(mk, abs_key<DT>(x[e]));
    const VectorScale vs = make_scale<DT>(mk, scale_div);
    int8_t* c = codes + o * codes_outer + i * codes_inner;
    for (int e = 0; e < d; ++e) c[e] = (int8_t)code_of<DT>(bits_to_f32<DT>(x[e]), vs);
    scales[o * scales_outer + i * scales_inner] = vs.s;
}

// ------------------------------------------------------------------ quantize, wave path
// One wavefront codes 64 consecutive head vectors (a "chunk") of one outer index: it pulls
// the chunk's bytes with coalesced 16-byte loads into its own LDS region, each lane then
// reads its vector with 8/16-byte LDS reads, codes it in registers (width D known at
// compile time, so nothing is indexed dynamically), writes the codes back to the region
// and the wave stores them with 16-byte stores. No workgroup barrier: the region is
// private to the wave and LDS operations of a wave complete in order.
//
// Fast-path codes: with q the exact quotient RN(t/s) (Markstein, above; for fp16, whose fast
// scales are normal, the product RN(t * RN(1/s)), which has the same code), the code is
// rint(RN_T(q)). For fp16 that is one packed add: RN16(q) + 1536 in fp16 rounds to an
// integer half-to-even (the fp16 spacing in [1024, 2048) is 1), and the low byte of
// 1536 + k is k in two's complement. fp32 and bf16 do the same with 1.5 * 2^23 in fp32.
// |t| <= amax bounds |t/s| by 127 * (1 + 2^-11) for fp16 and fp32 sources, so only bf16
// (scale rounded to 8 bits) needs the clamp; vectors outside the fast domain (zero, tiny,
// huge, inf, NaN) take code_of().
//
// Lanes exchange data through the region, which the compiler would otherwise treat as
// private to each lane and reorder freely: wave_sync() orders the phases.
constexpr int kChunk = 64;
constexpr int kWaveWaves = 4;

// Orders LDS accesses of the lanes of one wavefront: a compiler fence scoped to the wave
// (the hardware already executes a wave's LDS operations in order).
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

template <int DT>
__device__ __forceinline__ float elem_of(const uint32_t* x, int e) {
    if constexpr (DT == NORI_F32) return __uint_as_float(x[e]);
    else {
        const uint32_t w = x[e >> 1];
        const uint16_t b = (e & 1) ? (uint16_t)(w >> 16) : (uint16_t)(w & 0xffffu);
        return bits_to_f32<DT>(b);
    }
}

template <int DT, int D>
__global__ void __launch_bounds__(kWaveWaves * 64)
quantize_wave_kernel(const uint8_t* __restrict__ src, int64_t n_outer, int64_t n_inner, int64_t src_outer_bytes,
                     uint8_t* __restrict__ codes, int64_t codes_outer, float* __restrict__ scales, int64_t scales_outer,
                     int64_t chunks_per_outer, int scale_div) {
    using S = typename Storage<DT>::T;
    constexpr int es = sizeof(S);
    constexpr int VB = D * es;            // bytes per source vector (a multiple of 8)
    constexpr int XW = VB / 4;            // source dwords per vector
    constexpr int CB = kChunk * VB;       // source bytes per chunk (a multiple of 16)
    constexpr int WPL = (CB / 16 + 63) / 64;  // 16-byte words per lane
    constexpr int OB = kChunk * D;        // code bytes per chunk (a multiple of 16)
    constexpr int OPL = (OB / 16 + 63) / 64;
    static_assert(D % 4 == 0 && VB % 8 == 0 && CB % 16 == 0 && OB % 16 == 0, "vector width");
    __shared__ __attribute__((aligned(16))) uint8_t lds[kWaveWaves][CB];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    uint8_t* region = lds[wave];
    const int64_t total = n_outer * chunks_per_outer;

    for (int64_t ch = (int64_t)blockIdx.x * kWaveWaves + wave; ch < total; ch += (int64_t)gridDim.x * kWaveWaves) {
        const int64_t o = ch / chunks_per_outer;
        const int64_t v0 = (ch - o * chunks_per_outer) * kChunk;
        const int nv = (int)min<int64_t>(kChunk, n_inner - v0);
        const uint8_t* g = src + o * src_outer_bytes + v0 * VB;
        const int nbytes = nv * VB;

        // ---- chunk -> LDS (whole 16-byte words; the last word of a ragged tail per element)
        u32x4v w[WPL];
#pragma unroll
        for (int k = 0; k < WPL; ++k) {
            const int idx = lane + 64 * k;
            if (16 * idx + 16 <= nbytes) {
                w[k] = *reinterpret_cast<const u32x4v*>(g + 16 * idx);
            } else {
                w[k] = u32x4v{0u, 0u, 0u, 0u};
                if (16 * idx < nbytes) {
                    S tmp[16 / es];
#pragma unroll
                    for (int e = 0; e < 16 / es; ++e)
                        tmp[e] = (16 * idx + e * es < nbytes) ? reinterpret_cast<const S*>(g + 16 * idx)[e] : (S)0;
                    w[k] = __builtin_bit_cast(u32x4v, tmp);
                }
            }
        }
#pragma unroll
        for (int k = 0; k < WPL; ++k) {
            const int idx = lane + 64 * k;
            if (16 * idx < CB) *reinterpret_cast<u32x4v*>(region + 16 * idx) = w[k];
        }
        wave_sync();

        // ---- this lane's vector
        uint32_t x[XW];
#pragma unroll
        for (int j = 0; j < XW; j += 2) {
            const u32x2v v = *reinterpret_cast<const u32x2v*>(region + lane * VB + 4 * j);
            x[j] = v.x;
            x[j + 1] = v.y;
        }
        uint32_t mk;
        if constexpr (DT == NORI_F32) {
            mk = 0;
#pragma unroll
            for (int j = 0; j < XW; ++j) mk = max(mk, x[j] & 0x7fffffffu);
        } else {
            u16x2 m2 = {0, 0};
#pragma unroll
            for (int j = 0; j < XW; ++j) m2 = __builtin_elementwise_max(m2, __builtin_bit_cast(u16x2, x[j] & 0x7fff7fffu));
            mk = max((uint32_t)m2.x, (uint32_t)m2.y);
        }
        const VectorScale vs = make_scale<DT>(mk, scale_div);
        uint32_t c[D / 4];
        if (vs.fast) {
#pragma unroll
            for (int j = 0; j < D / 4; ++j) {
                float q[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float t = elem_of<DT>(x, 4 * j + i);
                    const float q0 = t * vs.y;
                    if constexpr (DT == NORI_F16) {
                        q[i] = q0;  // a normal fp16 scale: the product's code is the quotient's
                    } else {
                        q[i] = fmaf(fmaf(-q0, vs.s, t), vs.y, q0);  // the correctly rounded t/s (Markstein)
                    }
                }
                c[j] = pack_codes_fast<DT>(q);
            }
        } else {
#pragma unroll
            for (int j = 0; j < D / 4; ++j)
                c[j] = pack4(code_of<DT>(elem_of<DT>(x, 4 * j), vs), code_of<DT>(elem_of<DT>(x, 4 * j + 1), vs),
                             code_of<DT>(elem_of<DT>(x, 4 * j + 2), vs), code_of<DT>(elem_of<DT>(x, 4 * j + 3), vs));
        }

        // ---- codes -> LDS, once every lane has read its vector
        wave_sync();
#pragma unroll
        for (int j = 0; j < D / 4; ++j) *reinterpret_cast<uint32_t*>(region + lane * D + 4 * j) = c[j];
        wave_sync();
        if (lane < nv) scales[o * scales_outer + v0 + lane] = vs.s;
        uint8_t* gc = codes + o * codes_outer + v0 * D;
        const int cbytes = nv * D;
#pragma unroll
        for (int k = 0; k < OPL; ++k) {
            const int idx = lane + 64 * k;
            if (16 * idx >= OB) continue;
            const u32x4v cw = *reinterpret_cast<const u32x4v*>(region + 16 * idx);
            if (16 * idx + 16 <= cbytes) {
                *reinterpret_cast<u32x4v*>(gc + 16 * idx) = cw;
            } else if (16 * idx < cbytes) {
                const uint8_t* cb = reinterpret_cast<const uint8_t*>(&cw);
                for (int e = 0; e < 16 && 16 * idx + e < cbytes; ++e) gc[16 * idx + e] = cb[e];
            }
        }
        wave_sync();  // the next chunk overwrites the region
    }
}

// Launches the wave path when the width has an instantiation and the layout allows 16-byte
// transfers; returns false otherwise (the caller then uses the tile or direct kernel).
template <int DT>
bool launch_quantize_wave(const void* src, int64_t n_outer, int64_t n_inner, int d, int64_t src_outer_bytes,
                          int8_t* codes, int64_t codes_outer, float* scales, int64_t scales_outer, int scale_div,
                          hipStream_t stream) {
    if ((uintptr_t)src % 16 || (uintptr_t)codes % 16 || (n_outer > 1 && (src_outer_bytes % 16 || codes_outer % 16)))
        return false;
    // four waves' chunks must fit the 64 KiB of LDS a workgroup may address
    if ((int64_t)kWaveWaves * kChunk * d * dtype_size(DT) > 65536) return false;
    const int64_t cpo = (n_inner + kChunk - 1) / kChunk;
    const int64_t chunks = cpo * n_outer;
    // enough waves to keep HBM busy, few enough that each walks several chunks
    const int64_t grid = std::max<int64_t>(1, std::min<int64_t>((chunks + kWaveWaves - 1) / kWaveWaves, (int64_t)device_cus() * 8));
#define NORI_QW(DV)                                                                                           \
    case DV:                                                                                                  \
        hipLaunchKernelGGL((quantize_wave_kernel<DT, DV>), dim3((unsigned)grid), dim3(kWaveWaves * 64), 0, stream, \
                           (const uint8_t*)src, n_outer, n_inner, src_outer_bytes, (uint8_t*)codes, codes_outer,   \
                           scales, scales_outer, cpo, scale_div);                                              \
        return true;
    switch (d) {
        NORI_QW(16) NORI_QW(32) NORI_QW(44) NORI_QW(48) NORI_QW(56) NORI_QW(64)
        default: break;
    }
    if constexpr (DT != NORI_F32) {
        switch (d) {
            NORI_QW(96) NORI_QW(128)
            default: break;
        }
    }
    return false;
#undef NORI_QW
}

// ------------------------------------------------------------------ dequantize
template <int DT>
__global__ void __launch_bounds__(kTileThreads)
dequant_tile_kernel(const int8_t* __restrict__ codes, int64_t n_inner, int d, int64_t codes_outer,
                    const float* __restrict__ scales, int64_t scales_outer, uint8_t* __restrict__ dst,
                    int64_t dst_outer_bytes, int64_t tiles_per_outer) {
    using S = typename Storage<DT>::T;
    constexpr int es = sizeof(S);
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int64_t tile = blockIdx.x;
    const int64_t o = tile / tiles_per_outer;
    const int64_t v0 = (tile - o * tiles_per_outer) * kTileThreads;
    const int nv = (int)min<int64_t>(kTileThreads, n_inner - v0);
    uint8_t* lds_codes = lds;
    uint8_t* lds_out = lds + ((kTileThreads * d + 15) & ~15);

    const uint8_t* gc = reinterpret_cast<const uint8_t*>(codes + o * codes_outer + v0 * d);
    {
        // codes: 16-byte chunks when aligned, bytes otherwise
        const int nbytes = nv * d;
        int done = 0;
        if ((((uintptr_t)gc) & 15) == 0) {
            const int n16 = nbytes >> 4;
            for (int i = threadIdx.x; i < n16; i += kTileThreads)
                reinterpret_cast<uint4*>(lds_codes)[i] = reinterpret_cast<const uint4*>(gc)[i];
            done = n16 << 4;
        }
        for (int i = done + threadIdx.x; i < nbytes; i += kTileThreads) lds_codes[i] = gc[i];
    }
    __syncthreads();
    const int v = threadIdx.x;
    if (v < nv) {
        const float s = scales[o * scales_outer + v0 + v];
        const int8_t* c = reinterpret_cast<const int8_t*>(lds_codes) + v * d;
        S* y = reinterpret_cast<S*>(lds_out) + (int64_t)v * d;
        for (int i = 0; i < d; ++i) {
            const float f = (float)c[i] * s;
            if constexpr (DT == NORI_F32) y[i] = __float_as_uint(f);
            else if constexpr (DT == NORI_F16) y[i] = f32_to_f16(f);
            else y[i] = f32_to_bf16(f);
        }
    }
    __syncthreads();
    copy_out(dst + o * dst_outer_bytes + v0 * d * es, lds_out, nv * d * es);
}

// Contiguous slabs of vectors (head width d >= 16): thread t of a slab converts the 16 codes
// [16t, 16t + 16) -- one 16-byte load -- which belong to at most two vectors, so it needs at
// most two scales, and writes 16 output elements with 16-byte stores. The product is formed in
// fp32 and rounded once to the output dtype: (q.float() * scale).to(dtype).
template <int DT>
__global__ void __launch_bounds__(kTileThreads)
dequant_flat_kernel(const int8_t* __restrict__ codes, int64_t n_outer, int64_t n_inner, int d, int64_t codes_outer,
                    const float* __restrict__ scales, int64_t scales_outer, uint8_t* __restrict__ dst,
                    int64_t dst_outer_bytes, int64_t chunks_per_outer) {
    using S = typename Storage<DT>::T;
    constexpr int es = sizeof(S);
    const int64_t gid = (int64_t)blockIdx.x * kTileThreads + threadIdx.x;
    const int64_t o = gid / chunks_per_outer;
    const int64_t t = gid - o * chunks_per_outer;
    const int64_t n_elem = n_inner * d;
    const int64_t e0 = 16 * t;
    if (o >= n_outer || e0 >= n_elem) return;
    const int8_t* c = codes + o * codes_outer;
    const float* sc = scales + o * scales_outer;
    S* y = reinterpret_cast<S*>(dst + o * dst_outer_bytes);
    const int64_t v0 = e0 / d;
    const int split = (int)min<int64_t>(16, (v0 + 1) * d - e0);  // elements of vector v0 in the chunk
    const float s0 = sc[v0];
    if (e0 + 16 <= n_elem) {
        const float s1 = split < 16 ? sc[v0 + 1] : s0;
        const uint4 w = *reinterpret_cast<const uint4*>(c + e0);
        const uint32_t words[4] = {w.x, w.y, w.z, w.w};
        S out[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int code = (int)(int8_t)(words[i >> 2] >> (8 * (i & 3)));
            const float f = (float)code * (i < split ? s0 : s1);
            if constexpr (DT == NORI_F32) out[i] = __float_as_uint(f);
            else if constexpr (DT == NORI_F16) out[i] = f32_to_f16(f);
            else out[i] = f32_to_bf16(f);
        }
        uint4* yo = reinterpret_cast<uint4*>(y + e0);
#pragma unroll
        for (int k = 0; k < 16 * es / 16; ++k) yo[k] = reinterpret_cast<const uint4*>(out)[k];
    } else {
        // the slab's last, partial chunk
        for (int64_t e = e0; e < n_elem; ++e) {
            const float f = (float)c[e] * sc[e / d];
            if constexpr (DT == NORI_F32) y[e] = __float_as_uint(f);
            else if constexpr (DT == NORI_F16) y[e] = f32_to_f16(f);
            else y[e] = f32_to_bf16(f);
        }
    }
}

template <int DT>
__global__ void __launch_bounds__(kTileThreads)
dequant_direct_kernel(const int8_t* __restrict__ codes, int64_t n_outer, int64_t n_inner, int d,
                      int64_t codes_outer, int64_t codes_inner, const float* __restrict__ scales,
                      int64_t scales_outer, int64_t scales_inner, void* __restrict__ dst_v, int64_t dst_outer,
                      int64_t dst_inner) {
    using S = typename Storage<DT>::T;
    S* dst = reinterpret_cast<S*>(dst_v);
    const int64_t idx = (int64_t)blockIdx.x * kTileThreads + threadIdx.x;
    if (idx >= n_outer * n_inner) return;
    const int64_t o = idx / n_inner, i = idx - o * n_inner;
    const float s = scales[o * scales_outer + i * scales_inner];
    const int8_t* c = codes + o * codes_outer + i * codes_inner;
    S* y = dst + o * dst_outer + i * dst_inner;
    for (int e = 0; e < d; ++e) {
        const float f = (float)c[e] * s;
        if constexpr (DT == NORI_F32) y[e] = __float_as_uint(f);
        else if constexpr (DT == NORI_F16) y[e] = f32_to_f16(f);
        else y[e] = f32_to_bf16(f);
    }
}

int check_common(int64_t n_outer, int64_t n_inner, int32_t d) {
    if (n_outer < 0 || n_inner < 0) return fail(NORI_ERR_INVALID, "negative vector count (%lld x %lld)", (long long)n_outer, (long long)n_inner);
    if (d <= 0) return fail(NORI_ERR_INVALID, "head width must be positive, got %d", d);
    return NORI_OK;
}

}  // namespace

extern "C" int nori_kv_quantize_int8(const void* src, int src_dtype, int64_t n_outer, int64_t n_inner, int32_t d,
                                     int64_t src_outer_stride, int64_t src_inner_stride, int8_t* codes,
                                     int64_t codes_outer_stride, int64_t codes_inner_stride, float* scales,
                                     int64_t scales_outer_stride, int64_t scales_inner_stride, int32_t scale_div,
                                     void* stream_v) {
    clear_error();
    if (int st = check_common(n_outer, n_inner, d)) return st;
    if (src_dtype != NORI_F32 && src_dtype != NORI_F16 && src_dtype != NORI_BF16)
        return fail(NORI_ERR_UNSUPPORTED, "quantize_int8: unsupported source dtype %s", dtype_name(src_dtype));
    if (scale_div != NORI_SCALE_DIV_TRUE && scale_div != NORI_SCALE_DIV_RECIP)
        return fail(NORI_ERR_INVALID, "quantize_int8: unknown scale_div %d", scale_div);
    if (n_outer == 0 || n_inner == 0) return NORI_OK;
    if (!src || !codes || !scales) return fail(NORI_ERR_INVALID, "quantize_int8: null pointer");
    hipStream_t stream = (hipStream_t)stream_v;
    const int es = dtype_size(src_dtype);
    const bool contiguous = src_inner_stride == d && codes_inner_stride == d && scales_inner_stride == 1;
    if (contiguous) {
        bool done = false;
        NORI_DISPATCH_FLOAT(src_dtype, DT,
            done = launch_quantize_wave<DT>(src, n_outer, n_inner, d, src_outer_stride * es, codes, codes_outer_stride,
                                            scales, scales_outer_stride, scale_div, stream));
        if (done) return launch_status("quantize_int8");
    }
    const bool tiled = contiguous && d * es <= kMaxTileVectorBytes;
    if (tiled) {
        const int64_t tiles_per_outer = (n_inner + kTileThreads - 1) / kTileThreads;
        const int64_t grid = tiles_per_outer * n_outer;
        const size_t lds = ((size_t)kTileThreads * d * es + 15) / 16 * 16 + (size_t)kTileThreads * d;
        NORI_DISPATCH_FLOAT(src_dtype, DT,
            hipLaunchKernelGGL(quantize_tile_kernel<DT>, dim3((unsigned)grid), dim3(kTileThreads), lds, stream,
                               (const uint8_t*)src, n_inner, d, src_outer_stride * es, codes, codes_outer_stride,
                               scales, scales_outer_stride, tiles_per_outer, scale_div));
    } else {
        const int64_t total = n_outer * n_inner;
        const int64_t grid = (total + kTileThreads - 1) / kTileThreads;
        NORI_DISPATCH_FLOAT(src_dtype, DT,
            hipLaunchKernelGGL(quantize_direct_kernel<DT>, dim3((unsigned)grid), dim3(kTileThreads), 0, stream, src,
                               n_outer, n_inner, d, src_outer_stride, src_inner_stride, codes, codes_outer_stride,
                               codes_inner_stride, scales, scales_outer_stride, scales_inner_stride, scale_div));
    }
    return launch_status("quantize_int8");
}

extern "C" int nori_kv_dequantize_int8(const int8_t* codes, const float* scales, int64_t n_outer, int64_t n_inner,
                                       int32_t d, int64_t codes_outer_stride, int64_t codes_inner_stride,
                                       int64_t scales_outer_stride, int64_t scales_inner_stride, void* dst,
                                       int dst_dtype, int64_t dst_outer_stride, int64_t dst_inner_stride,
                                       void* stream_v) {
    clear_error();
    if (int st = check_common(n_outer, n_inner, d)) return st;
    if (dst_dtype != NORI_F32 && dst_dtype != NORI_F16 && dst_dtype != NORI_BF16)
        return fail(NORI_ERR_UNSUPPORTED, "dequantize_int8: unsupported output dtype %s", dtype_name(dst_dtype));
    if (n_outer == 0 || n_inner == 0) return NORI_OK;
    if (!codes || !scales || !dst) return fail(NORI_ERR_INVALID, "dequantize_int8: null pointer");
    hipStream_t stream = (hipStream_t)stream_v;
    const int es = dtype_size(dst_dtype);
    const bool contiguous = dst_inner_stride == d && codes_inner_stride == d && scales_inner_stride == 1;
    // 16-byte code loads and output stores from slab bases
    const bool flat = contiguous && d >= 16 && ((uintptr_t)codes % 16) == 0 && (codes_outer_stride % 16) == 0 &&
                      ((uintptr_t)dst % 16) == 0 && ((dst_outer_stride * es) % 16) == 0;
    if (flat) {
        const int64_t chunks_per_outer = (n_inner * d + 15) / 16;
        const int64_t blocks = (chunks_per_outer * n_outer + kTileThreads - 1) / kTileThreads;
        if (blocks > 0x7fffffffLL) return fail(NORI_ERR_UNSUPPORTED, "dequantize_int8: cache too large for one launch");
        NORI_DISPATCH_FLOAT(dst_dtype, DT,
            hipLaunchKernelGGL(dequant_flat_kernel<DT>, dim3((unsigned)blocks), dim3(kTileThreads), 0, stream, codes,
                               n_outer, n_inner, d, codes_outer_stride, scales, scales_outer_stride, (uint8_t*)dst,
                               dst_outer_stride * es, chunks_per_outer));
        return launch_status("dequantize_int8");
    }
    const bool tiled = contiguous && d * es <= kMaxTileVectorBytes;
    if (tiled) {
        const int64_t tiles_per_outer = (n_inner + kTileThreads - 1) / kTileThreads;
        const int64_t grid = tiles_per_outer * n_outer;
        const size_t lds = ((size_t)kTileThreads * d + 15) / 16 * 16 + (size_t)kTileThreads * d * es;
        NORI_DISPATCH_FLOAT(dst_dtype, DT,
            hipLaunchKernelGGL(dequant_tile_kernel<DT>, dim3((unsigned)grid), dim3(kTileThreads), lds, stream, codes,
                               n_inner, d, codes_outer_stride, scales, scales_outer_stride, (uint8_t*)dst,
                               dst_outer_stride * es, tiles_per_outer));
    } else {
        const int64_t total = n_outer * n_inner;
        const int64_t grid = (total + kTileThreads - 1) / kTileThreads;
        NORI_DISPATCH_FLOAT(dst_dtype, DT,
            hipLaunchKernelGGL(dequant_direct_kernel<DT>, dim3((unsigned)grid), dim3(kTileThreads), 0, stream, codes,
                               n_outer, n_inner, d, codes_outer_stride, codes_inner_stride, scales,
                               scales_outer_stride, scales_inner_stride, dst, dst_outer_stride, dst_inner_stride));
    }
    return launch_status("dequantize_int8");
}
