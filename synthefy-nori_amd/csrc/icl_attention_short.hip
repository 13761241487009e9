// Query-row -> context attention for short contexts and few queries (the in-row attentions of
// the two-phase encoder: a cell over its row's few cells and target tokens, a row over its own
// cells). Chosen by the planner in icl_attention.hip when the MFMA kernel's fixed cost per
// (b, h) unit -- a 64-query tile, a 64-key staged block, the pipeline fill -- would dwarf the
// work. Same arguments and results as that kernel (dense output, LSE, running-output merge).
//
// One group of G lanes per (b, h, query) row, G = d/4 rounded up to a power of two: a lane holds
// 4 head elements of the query, its partial logit per key is summed over the group with DPP
// (all within a 16-lane row; a 32-lane group adds one swizzle), and the online softmax runs in
// fp32 on the VALU, key by key, from K/V rows loaded 4 elements per lane (16-, 8- or 4-byte
// loads). The rows of one (b, h) are consecutive, so the groups of a wavefront read the same
// K/V rows. Values are computed in fp32 from the exact cache values (codes x scales for int8).
// With a prologue the per-head q/k RMS norms (and the q multiply) run on the rows as loaded,
// rounded as the separate passes round them: the group holds a whole row, so the mean of
// squares is one more group sum.
#include <math.h>

#include "icl_attention_kernel.h"

namespace {

using namespace nori;
using namespace nori::attn;

constexpr int kThreads = 256;

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Sum over the G lanes of a group (G a power of two up to 32); every lane gets the sum.
template <int G>
__device__ __forceinline__ float group_sum(float v) {
    if constexpr (G >= 2) v += dpp<0xb1>(v);   // quad_perm [1, 0, 3, 2]: lane ^ 1
    if constexpr (G >= 4) v += dpp<0x4e>(v);   // quad_perm [2, 3, 0, 1]: lane ^ 2
    if constexpr (G >= 8) v += dpp<0x141>(v);  // row_half_mirror: the other quad of 8
    if constexpr (G >= 16) v += dpp<0x140>(v); // row_mirror: the other 8 of 16
    if constexpr (G >= 32) v += __shfl_xor(v, 16);
    return v;
}

// 4 consecutive cache elements as loaded (one 16-, 8- or 4-byte load), and as fp32 values
// (int8: the codes).
template <int KVT> struct Raw4 { u32x2 w; };
template <> struct Raw4<NORI_F32> { f32x4 w; };
template <> struct Raw4<NORI_I8> { uint32_t w; };

template <int KVT>
__device__ __forceinline__ Raw4<KVT> load_raw4(const void* p, int64_t i) {
    Raw4<KVT> r;
    if constexpr (KVT == NORI_F32) r.w = *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(p) + i);
    else if constexpr (KVT == NORI_I8) r.w = *reinterpret_cast<const uint32_t*>(reinterpret_cast<const int8_t*>(p) + i);
    else r.w = *reinterpret_cast<const u32x2*>(reinterpret_cast<const uint16_t*>(p) + i);
    return r;
}

template <int KVT>
__device__ __forceinline__ f32x4 to_f32x4(const Raw4<KVT>& raw) {
    f32x4 r;
    if constexpr (KVT == NORI_F32) {
        r = raw.w;
    } else if constexpr (KVT == NORI_I8) {
#pragma unroll
        for (int e = 0; e < 4; ++e) r[e] = (float)(int8_t)(raw.w >> (8 * e));
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint16_t h = (uint16_t)(raw.w[e >> 1] >> (16 * (e & 1)));
            r[e] = KVT == NORI_F16 ? f16_to_f32(h) : bf16_to_f32(h);
        }
    }
    return r;
}

// Keys whose K/V rows are loaded together and share one rescale: 4 for contexts of more than
// 8 keys (33 x 33: 14 % faster than key by key), 1 for the in-row attentions of a few keys,
// where the extra registers cost more occupancy than the overlapped loads gain.
constexpr int chunk_for(int64_t nk) { return nk > 8 ? 4 : 1; }

// Rounding to a runtime dtype (the query's), as torch rounds each op's result.
__device__ __forceinline__ float round_dt(float v, int dt) {
    if (dt == NORI_F16) return round_to<NORI_F16>(v);
    if (dt == NORI_BF16) return round_to<NORI_BF16>(v);
    return v;
}

// T(T(v * rsqrt(mean(v^2) + eps)) * w) over the group's row (4 elements per lane; lanes past
// the row hold zeros), with T rounding to dtype dt: the RMSNorm pass of the reference.
template <int G>
__device__ __forceinline__ void norm_row(f32x4& v, const f32x4& w, int d, float eps, int dt) {
    const float ss = group_sum<G>(v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3]);
    const float inv = rsqrtf(ss / (float)d + eps);
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = round_dt(round_dt(v[e] * inv, dt) * w[e], dt);
}

template <int KVT, int G, int kChunk>
__global__ void __launch_bounds__(kThreads) icl_attention_short_kernel(const Args a, int64_t rows, const Prologue pro) {
    const int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    int64_t row = t / G;  // (b, h, query) with the query fastest
    const bool valid = row < rows;
    if (!valid) row = rows - 1;  // keep every lane of the group active through the reductions
    const int sub = (int)(threadIdx.x % G);
    const int64_t qi = row % a.nq;
    const int64_t bh = row / a.nq;
    const int h = (int)(bh % a.heads);
    const int64_t b = bh / a.heads;
    const int hk = h / a.hgroup;
    const int c0 = 4 * sub;
    const bool live = c0 < a.d;  // d % 4 == 0: a lane's 4 elements are all in or all out

    f32x4 q = {0.f, 0.f, 0.f, 0.f}, kw = {1.f, 1.f, 1.f, 1.f};
    if (live) {
        const int64_t qb = b * a.q_bg + qi * a.q_row + (int64_t)h * a.q_head + c0;
        if (a.flags & kQVec4) {  // 16-bit, 4-element aligned: one 8-byte load
            const u32x2 w = *reinterpret_cast<const u32x2*>(reinterpret_cast<const uint16_t*>(a.q) + qb);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint16_t x = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
                q[e] = a.q_dtype == NORI_BF16 ? bf16_to_f32(x) : f16_to_f32(x);
            }
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) q[e] = load_as_f32(a.q, a.q_dtype, qb + e);
        }
    }
    if (pro.qw) {
        f32x4 qw = {0.f, 0.f, 0.f, 0.f};
        if (live)
#pragma unroll
            for (int e = 0; e < 4; ++e) qw[e] = load_as_f32(pro.qw, pro.wdt, c0 + e);
        norm_row<G>(q, qw, a.d, pro.eps, a.q_dtype);
    }
    if (pro.qmult != 1.f)
#pragma unroll
        for (int e = 0; e < 4; ++e) q[e] = round_dt(q[e] * pro.qmult, a.q_dtype);
#pragma unroll
    for (int e = 0; e < 4; ++e) q[e] *= a.scale_log2;
    const bool knorm = pro.kw != nullptr;
    if (knorm && live)
#pragma unroll
        for (int e = 0; e < 4; ++e) kw[e] = load_as_f32(pro.kw, pro.wdt, c0 + e);
    const int64_t kbase = b * a.kv_bg + (int64_t)hk * a.d + c0;
    const int64_t sbase = b * a.sc_bg + hk;
    float m = -INFINITY, l = 0.f;
    f32x4 o = {0.f, 0.f, 0.f, 0.f};
    // Keys in chunks of kChunk: all of a chunk's K/V rows are loaded before the first is used
    // (the loads overlap instead of one latency per key), then its logits, one rescale of the
    // running sums to the chunk's max, and one exponential per key. The chunk length is
    // uniform over the wavefront.
#pragma unroll 2
    for (int64_t j0 = 0; j0 < a.nk; j0 += kChunk) {
        const int nj = (int)min((int64_t)kChunk, a.nk - j0);
        Raw4<KVT> rk[kChunk], rv[kChunk];
        float ks[kChunk], vsc[kChunk];
#pragma unroll
        for (int u = 0; u < kChunk; ++u) {
            ks[u] = 1.f;
            vsc[u] = 1.f;
            if (u < nj) {
                const int64_t j = j0 + u;
                if (live) {
                    rk[u] = load_raw4<KVT>(a.kv, kbase + j * a.kv_row);
                    rv[u] = load_raw4<KVT>(a.kv, kbase + j * a.kv_row + a.kv_half);
                } else {
                    rk[u] = Raw4<KVT>{};
                    rv[u] = Raw4<KVT>{};
                }
                if constexpr (KVT == NORI_I8) {
                    ks[u] = a.kvs[sbase + j * a.sc_row];
                    vsc[u] = a.kvs[sbase + j * a.sc_row + a.sc_half];
                }
            }
        }
        float s[kChunk];
        float m_new = m;
#pragma unroll
        for (int u = 0; u < kChunk; ++u) {
            s[u] = -INFINITY;
            if (u < nj) {
                f32x4 k = to_f32x4<KVT>(rk[u]);
                if constexpr (KVT != NORI_I8) {
                    if (knorm) norm_row<G>(k, kw, a.d, pro.eps, KVT);
                }
                s[u] = group_sum<G>(q[0] * k[0] + q[1] * k[1] + q[2] * k[2] + q[3] * k[3]) * ks[u];
                m_new = fmaxf(m_new, s[u]);
            }
        }
        const float alpha = __builtin_amdgcn_exp2f(m - m_new);
        l *= alpha;
        o *= alpha;
#pragma unroll
        for (int u = 0; u < kChunk; ++u) {
            if (u < nj) {
                const float p = __builtin_amdgcn_exp2f(s[u] - m_new);
                l += p;
                o += (p * vsc[u]) * to_f32x4<KVT>(rv[u]);
            }
        }
        m = m_new;
    }
    if (!valid) return;
    const float inv = 1.0f / l;
    const float lse_part = (m + __log2f(l)) * kLn2;
    const bool merge = a.flags & NORI_ATTN_MERGE;
    float w_old = 0.f, w_new = 1.f, lse_out = lse_part;
    if (merge) merge_weights(a.lse[row], lse_part, w_old, w_new, lse_out);
    if (live && (a.flags & kOutVec4)) {  // 16-bit output, no merge: one 8-byte store
        const int64_t ob = b * a.o_bg + qi * a.o_row + (int64_t)h * a.o_head + c0;
        const bool bf = a.out_dtype == NORI_BF16;
        uint32_t w[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const float v0 = o[2 * i] * inv, v1 = o[2 * i + 1] * inv;
            w[i] = (uint32_t)(bf ? f32_to_bf16(v0) : f32_to_f16(v0)) | ((uint32_t)(bf ? f32_to_bf16(v1) : f32_to_f16(v1)) << 16);
        }
        *reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(a.out) + ob) = u32x2{w[0], w[1]};
    } else if (live) {
        const int64_t ob = b * a.o_bg + qi * a.o_row + (int64_t)h * a.o_head + c0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float r = o[e] * inv;
            if (merge) r = reinterpret_cast<const float*>(a.out)[ob + e] * w_old + r * w_new;
            store_from_f32(a.out, a.out_dtype, ob + e, r);
        }
    }
    if (a.lse && sub == 0) a.lse[row] = lse_out;
}

template <int KVT, int KC>
int launch_chunked(const Args& a, const Prologue& pro, hipStream_t stream) {
    const int quads = (a.d + 3) / 4;
    const int64_t rows = a.bg * a.heads * a.nq;
    int g = 1;
    while (g < quads) g *= 2;
    const int64_t threads = rows * g;
    if ((threads + kThreads - 1) / kThreads > 0x7fffffffLL)
        return fail(NORI_ERR_UNSUPPORTED, "icl_attention: %lld query rows exceed one launch", (long long)rows);
    const dim3 grid((unsigned)((threads + kThreads - 1) / kThreads)), block(kThreads);
    switch (g) {
        case 1: hipLaunchKernelGGL((icl_attention_short_kernel<KVT, 1, KC>), grid, block, 0, stream, a, rows, pro); break;
        case 2: hipLaunchKernelGGL((icl_attention_short_kernel<KVT, 2, KC>), grid, block, 0, stream, a, rows, pro); break;
        case 4: hipLaunchKernelGGL((icl_attention_short_kernel<KVT, 4, KC>), grid, block, 0, stream, a, rows, pro); break;
        case 8: hipLaunchKernelGGL((icl_attention_short_kernel<KVT, 8, KC>), grid, block, 0, stream, a, rows, pro); break;
        case 16: hipLaunchKernelGGL((icl_attention_short_kernel<KVT, 16, KC>), grid, block, 0, stream, a, rows, pro); break;
        default: hipLaunchKernelGGL((icl_attention_short_kernel<KVT, 32, KC>), grid, block, 0, stream, a, rows, pro); break;
    }
    return NORI_OK;
}

template <int KVT>
int launch_group(const Args& a, const Prologue& pro, hipStream_t stream) {
    return chunk_for(a.nk) == 4 ? launch_chunked<KVT, 4>(a, pro, stream) : launch_chunked<KVT, 1>(a, pro, stream);
}

}  // namespace

namespace nori {
namespace attn {

int launch_short(int kv_dtype, const Args& a, const Prologue& pro, hipStream_t stream) {
    switch (kv_dtype) {
        case NORI_I8: return launch_group<NORI_I8>(a, pro, stream);
        case NORI_F16: return launch_group<NORI_F16>(a, pro, stream);
        case NORI_BF16: return launch_group<NORI_BF16>(a, pro, stream);
        default: return launch_group<NORI_F32>(a, pro, stream);
    }
}

}  // namespace attn
}  // namespace nori
