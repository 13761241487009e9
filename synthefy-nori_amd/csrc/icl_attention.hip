// Query-row -> context attention over an int8 (or full-precision) K/V cache, gfx950.
//
// Semantics: softmax(scale * q k^T) v per (table-group b, head h), K/V head
// hk = h / (heads / kv_heads); natural-log LSE of the scaled logits. This is the dense
// cached attention (layer.py:936-1049), the CPU online-softmax scan (layer.py:777-839) and
// the GPU flex block + exact LSE merge (layer.py:841-934) of the reference, with the
// int8 dequantization (kv_cache_scaling.py:40-41) folded into the tile loads.
//
// Schedule (one workgroup = 8 wavefronts = 256 query rows of one (b, h), one context range):
//   * Q rows live in registers as f16 MFMA operands for the whole scan.
//   * The context is scanned in blocks of 64 rows. All 512 threads stage a block into LDS:
//       K: int8 codes -> exact f16 integers (v_perm builds 1024+u, v_pk_add subtracts 1152);
//          the per-row K scale is kept as an fp32 factor and applied to the logits, so K
//          itself is exact in the MFMA;
//       V: int8 codes -> f16 codes -> times the row's V scale (v_pk_mul_f16), stored
//          transposed ([d][row]) with rows permuted inside each 16-row group so the
//          probabilities leave the logit MFMA already in the operand order of the PV MFMA.
//   * Per wavefront and block: S^T = K Q^T (v_mfma_f32_32x32x16_f16), logits
//     x = fma(s, kscale*scale*log2e, -m), online softmax in base 2 with lazy rescaling
//     (the running max only moves when a block exceeds it by 2^8), P packed to f16,
//     row sums by v_dot2 on the packed P, O^T += V^T P^T (v_mfma_f32_32x32x16_f16).
//   * Small grids split the context across workgroups; partial (O, LSE) pairs are merged
//     exactly by a second kernel (the same identity as layer.py:915-920).
//   * Workgroups are renumbered so the query tiles that share one (b, h) context land on
//     the same XCD (blocks are dealt round-robin over the 8 XCDs), keeping K/V re-reads in
//     that XCD's L2.
#include <math.h>

#include <algorithm>

#include "nori_common.h"

namespace {

using namespace nori;

constexpr int KB = 64;               // context rows per LDS block
constexpr int WAVES = 8;             // wavefronts per workgroup
constexpr int QPW = 32;              // query rows per wavefront
constexpr int QTILE = WAVES * QPW;   // query rows per workgroup
constexpr int THREADS = WAVES * 64;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kRescaleSlack = 8.0f;  // log2 units a block may exceed the running max by

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <int DP>
struct Geometry {
    static_assert(DP % 16 == 0 && DP >= 16 && DP <= 128, "padded head width");
    static constexpr int DV = (DP + 31) / 32 * 32;  // PV output rows (MFMA M granule)
    static constexpr int KSTEPS = DP / 16;          // logit MFMA k-steps
    static constexpr int VTILES = DV / 32;
    static constexpr int DQMAX = DP / 4;            // 4-wide quads per padded head vector
    static constexpr int KPITCH = DP + 8;           // f16 elements per K row in LDS (+16 B)
    static constexpr int VPITCH = KB + 8;           // f16 elements per V^T row in LDS (+16 B)
    static constexpr int UNITS = 2 * 16 * DQMAX;    // staging units: (K|V, row quad, d quad)
};

// 4 int8 codes -> two f16x2 holding the same integers (exact).
__device__ __forceinline__ void codes_to_f16(uint32_t w, uint32_t& lo, uint32_t& hi) {
    const uint32_t u = w ^ 0x80808080u;  // c + 128 in [1, 255]
    const uint32_t a = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);  // f16 1024+u0, 1024+u1
    const uint32_t b = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);  // f16 1024+u2, 1024+u3
    const f16x2 bias = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    lo = __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, a) + bias);
    hi = __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, b) + bias);
}

__device__ __forceinline__ uint32_t pack_f16(float a, float b) {
    return __builtin_bit_cast(uint32_t, f16x2{(_Float16)a, (_Float16)b});
}

template <int KVT>
__device__ __forceinline__ void load_quad_f16(const void* base, int64_t off, uint32_t& lo, uint32_t& hi) {
    if constexpr (KVT == NORI_F16) {
        const u32x2 v = *reinterpret_cast<const u32x2*>(reinterpret_cast<const uint16_t*>(base) + off);
        lo = v.x; hi = v.y;
    } else if constexpr (KVT == NORI_BF16) {
        const u32x2 v = *reinterpret_cast<const u32x2*>(reinterpret_cast<const uint16_t*>(base) + off);
        lo = pack_f16(__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xffff0000u));
        hi = pack_f16(__uint_as_float(v.y << 16), __uint_as_float(v.y & 0xffff0000u));
    } else {
        const u32x4 v = *reinterpret_cast<const u32x4*>(reinterpret_cast<const float*>(base) + off);
        lo = pack_f16(__uint_as_float(v.x), __uint_as_float(v.y));
        hi = pack_f16(__uint_as_float(v.z), __uint_as_float(v.w));
    }
}

__device__ __forceinline__ float load_as_f32(const void* p, int dt, int64_t i) {
    if (dt == NORI_F32) return reinterpret_cast<const float*>(p)[i];
    if (dt == NORI_F16) return f16_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
    return bf16_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
}

__device__ __forceinline__ void store_from_f32(void* p, int dt, int64_t i, float v) {
    if (dt == NORI_F32) reinterpret_cast<float*>(p)[i] = v;
    else if (dt == NORI_F16) reinterpret_cast<uint16_t*>(p)[i] = f32_to_f16(v);
    else reinterpret_cast<uint16_t*>(p)[i] = f32_to_bf16(v);
}

struct AttnArgs {
    const void* q; int q_dtype; int64_t nq; int heads; int d;
    int64_t q_bg, q_row, q_head;
    const void* kv; const float* kvs; int64_t nk; int hgroup;
    int64_t kv_bg, kv_row, kv_half, sc_bg, sc_row, sc_half;
    float scale_log2;  // scale * log2(e)
    void* out; int out_dtype; int64_t o_bg, o_row, o_head;
    float* lse; uint32_t flags;
    int64_t bg; int nqt; int nsplit; int64_t keys_per_split;
    float* part_o; float* part_lse;  // [nsplit][bg][heads][nq][d], [nsplit][bg][heads][nq]
    int64_t nblocks;
};

// Merge a normalized partial (o, lse) into the running fp32 output/LSE (layer.py:915-920).
__device__ __forceinline__ void merge_weights(float lse_old, float lse_new_part, float& w_old, float& w_new,
                                              float& lse_out) {
    const float mx = fmaxf(lse_old, lse_new_part);
    if (mx == -INFINITY) { w_old = 0.f; w_new = 0.f; lse_out = -INFINITY; return; }
    lse_out = mx + log1pf(expf(-fabsf(lse_old - lse_new_part)));
    w_old = expf(lse_old - lse_out);
    w_new = expf(lse_new_part - lse_out);
}

template <int DP, int KVT>
__global__ void __launch_bounds__(THREADS)
icl_attention_kernel(const AttnArgs a) {
    using G = Geometry<DP>;
    __shared__ __attribute__((aligned(16))) _Float16 Ks[KB * G::KPITCH];
    __shared__ __attribute__((aligned(16))) _Float16 Vt[G::DV * G::VPITCH];
    __shared__ __attribute__((aligned(16))) float kfac[KB];

    // ---- XCD-aware renumbering: the 8 XCDs receive blocks round-robin; give each XCD a
    // contiguous range of work items so neighbouring query tiles share an L2.
    const int64_t nb = a.nblocks;
    const int64_t xcd = blockIdx.x % 8, local = blockIdx.x / 8;
    const int64_t per = nb / 8, extra = nb % 8;
    const int64_t work = xcd * per + min<int64_t>(xcd, extra) + local;
    const int qt = (int)(work % a.nqt);
    int64_t rest = work / a.nqt;
    const int split = (int)(rest % a.nsplit);
    rest /= a.nsplit;
    const int h = (int)(rest % a.heads);
    const int64_t b = rest / a.heads;
    const int hk = h / a.hgroup;

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
    const int64_t qi = (int64_t)qt * QTILE + wave * QPW + l32;
    const int64_t k_begin = (int64_t)split * a.keys_per_split;
    const int64_t k_end = min<int64_t>(a.nk, k_begin + a.keys_per_split);
    const int d = a.d;
    const int dq_valid = d >> 2;

    // ---- Q fragment (B operand of S^T = K Q^T): lane holds q[qi][16ks + 8hh + 0..7]
    f16x8 qf[G::KSTEPS];
    {
        const bool qok = qi < a.nq;
        const int64_t qbase = b * a.q_bg + qi * a.q_row + (int64_t)h * a.q_head;
#pragma unroll
        for (int ks = 0; ks < G::KSTEPS; ++ks) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int dd = 16 * ks + 8 * hh + j;
                qf[ks][j] = (qok && dd < d) ? (_Float16)load_as_f32(a.q, a.q_dtype, qbase + dd) : (_Float16)0.0f;
            }
        }
    }
    // V^T rows beyond the padded logit width are never staged; keep them zero.
    for (int i = tid; i < (G::DV - DP) * G::VPITCH; i += THREADS) Vt[DP * G::VPITCH + i] = (_Float16)0.0f;

    f32x16 o[G::VTILES];
#pragma unroll
    for (int vt = 0; vt < G::VTILES; ++vt) o[vt] = f32x16{};
    float m_run = 0.0f;  // running max (log2 units), valid after the first block
    float l_run = 0.0f;  // this lane's share of the running denominator
    bool first = true;

    const char* kv_b = reinterpret_cast<const char*>(a.kv);
    const int kv_es = (KVT == NORI_F32) ? 4 : (KVT == NORI_I8 ? 1 : 2);

    for (int64_t kb = k_begin; kb < k_end; kb += KB) {
        __syncthreads();  // the previous block's LDS is no longer read
        // ---------------- stage K and V of rows [kb, kb+64) into LDS
        for (int u = tid; u < G::UNITS; u += THREADS) {
            const int kvsel = u / (16 * G::DQMAX);
            const int rem = u - kvsel * (16 * G::DQMAX);
            const int rq = rem / G::DQMAX;   // row quad 0..15
            const int dq = rem - rq * G::DQMAX;
            uint32_t lo[4], hi[4];
            float sc[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int64_t row = kb + 4 * rq + i;
                const bool ok = dq < dq_valid && row < k_end;
                const int64_t eoff = b * a.kv_bg + row * a.kv_row + kvsel * a.kv_half + (int64_t)hk * d + 4 * dq;
                if constexpr (KVT == NORI_I8) {
                    const uint32_t w = ok ? *reinterpret_cast<const uint32_t*>(kv_b + eoff) : 0u;
                    codes_to_f16(w, lo[i], hi[i]);
                    sc[i] = ok ? a.kvs[b * a.sc_bg + row * a.sc_row + kvsel * a.sc_half + hk] : 0.0f;
                } else {
                    if (ok) load_quad_f16<KVT>(a.kv, eoff, lo[i], hi[i]);
                    else { lo[i] = 0u; hi[i] = 0u; }
                    sc[i] = 1.0f;
                }
            }
            (void)kv_es;
            if (kvsel == 0) {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    *reinterpret_cast<u32x2*>(&Ks[(4 * rq + i) * G::KPITCH + 4 * dq]) = u32x2{lo[i], hi[i]};
                if (dq == 0) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) kfac[4 * rq + i] = (KVT == NORI_I8 ? sc[i] : 1.0f) * a.scale_log2;
                }
            } else {
                if constexpr (KVT == NORI_I8) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const f16x2 s2 = {(_Float16)sc[i], (_Float16)sc[i]};
                        lo[i] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, lo[i]) * s2);
                        hi[i] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, hi[i]) * s2);
                    }
                }
                // transpose the 4x4 (row, d) block: dword pairs (row0,row1), (row2,row3) per d
                const int pos = 16 * (rq >> 2) + 4 * ((rq & 3) == 1 ? 2 : ((rq & 3) == 2 ? 1 : (rq & 3)));
                const uint32_t d0a = __builtin_amdgcn_perm(lo[1], lo[0], 0x05040100u);
                const uint32_t d0b = __builtin_amdgcn_perm(lo[3], lo[2], 0x05040100u);
                const uint32_t d1a = __builtin_amdgcn_perm(lo[1], lo[0], 0x07060302u);
                const uint32_t d1b = __builtin_amdgcn_perm(lo[3], lo[2], 0x07060302u);
                const uint32_t d2a = __builtin_amdgcn_perm(hi[1], hi[0], 0x05040100u);
                const uint32_t d2b = __builtin_amdgcn_perm(hi[3], hi[2], 0x05040100u);
                const uint32_t d3a = __builtin_amdgcn_perm(hi[1], hi[0], 0x07060302u);
                const uint32_t d3b = __builtin_amdgcn_perm(hi[3], hi[2], 0x07060302u);
                *reinterpret_cast<u32x2*>(&Vt[(4 * dq + 0) * G::VPITCH + pos]) = u32x2{d0a, d0b};
                *reinterpret_cast<u32x2*>(&Vt[(4 * dq + 1) * G::VPITCH + pos]) = u32x2{d1a, d1b};
                *reinterpret_cast<u32x2*>(&Vt[(4 * dq + 2) * G::VPITCH + pos]) = u32x2{d2a, d2b};
                *reinterpret_cast<u32x2*>(&Vt[(4 * dq + 3) * G::VPITCH + pos]) = u32x2{d3a, d3b};
            }
        }
        __syncthreads();

        // ---------------- logits S^T[32 rows x 32 queries] for the two 32-row halves
        f32x16 s[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            s[t] = f32x16{};
#pragma unroll
            for (int ks = 0; ks < G::KSTEPS; ++ks) {
                const f16x8 kf = *reinterpret_cast<const f16x8*>(&Ks[(32 * t + l32) * G::KPITCH + 16 * ks + 8 * hh]);
                s[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[ks], s[t], 0, 0, 0);
            }
        }
        // lane holds rows 32t + 8g + 4hh + i (g, i in 0..3) for query qi
        const bool partial = kb + KB > k_end;
        float x[2][16];
        float bm = -INFINITY;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const f32x4 f = *reinterpret_cast<const f32x4*>(&kfac[32 * t + 8 * g + 4 * hh]);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float v = first ? s[t][4 * g + i] * f[i] : fmaf(s[t][4 * g + i], f[i], -m_run);
                    if (partial && kb + 32 * t + 8 * g + 4 * hh + i >= k_end) v = -INFINITY;
                    x[t][4 * g + i] = v;
                }
            }
        }
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 16; r += 2) bm = __builtin_fmaxf(bm, __builtin_fmaxf(x[t][r], x[t][r + 1]));
        bm = fmaxf(bm, __shfl_xor(bm, 32));
        if (first) {
            // x holds absolute logits; anchor the running max on this block
            m_run = bm;
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r) x[t][r] -= m_run;
            first = false;
        } else if (__any(bm > kRescaleSlack)) {
            // x is relative to m_run; move the max up where a block overshoots
            const float shift = fmaxf(bm, 0.0f);
            const float alpha = __builtin_amdgcn_exp2f(-shift);
            m_run += shift;
            l_run *= alpha;
#pragma unroll
            for (int vt = 0; vt < G::VTILES; ++vt)
#pragma unroll
                for (int r = 0; r < 16; ++r) o[vt][r] *= alpha;
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r) x[t][r] -= shift;
        }
        // ---------------- probabilities, row sums, PV
        f16x8 pf[4];
        const f16x2 ones = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
#pragma unroll
            for (int j = 0; j < 8; j += 2) {
                const float p0 = __builtin_amdgcn_exp2f(x[c >> 1][8 * (c & 1) + j]);
                const float p1 = __builtin_amdgcn_exp2f(x[c >> 1][8 * (c & 1) + j + 1]);
                const f16x2 pp = __builtin_bit_cast(f16x2, __builtin_amdgcn_cvt_pkrtz(p0, p1));
                l_run = __builtin_amdgcn_fdot2(pp, ones, l_run, false);
                pf[c][j] = pp[0];
                pf[c][j + 1] = pp[1];
            }
        }
#pragma unroll
        for (int vt = 0; vt < G::VTILES; ++vt) {
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const f16x8 vf = *reinterpret_cast<const f16x8*>(&Vt[(32 * vt + l32) * G::VPITCH + 16 * c + 8 * hh]);
                o[vt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pf[c], o[vt], 0, 0, 0);
            }
        }
    }

    // ---------------- epilogue
    const float l_tot = l_run + __shfl_xor(l_run, 32);
    if (qi >= a.nq) return;
    const float inv = 1.0f / l_tot;
    const float lse_part = (m_run + __log2f(l_tot)) * kLn2;
    if (a.nsplit > 1) {
        const int64_t prow = ((split * a.bg + b) * a.heads + h) * a.nq + qi;
        float* po = a.part_o + prow * d;
#pragma unroll
        for (int vt = 0; vt < G::VTILES; ++vt)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int d0 = 32 * vt + 8 * g + 4 * hh;
                if (d0 < d)
                    *reinterpret_cast<f32x4*>(po + d0) =
                        f32x4{o[vt][4 * g] * inv, o[vt][4 * g + 1] * inv, o[vt][4 * g + 2] * inv, o[vt][4 * g + 3] * inv};
            }
        if (hh == 0) a.part_lse[prow] = lse_part;
        return;
    }
    const int64_t obase = b * a.o_bg + qi * a.o_row + (int64_t)h * a.o_head;
    const int64_t lse_idx = (b * a.heads + h) * a.nq + qi;
    float w_old = 0.f, w_new = 1.f, lse_out = lse_part;
    if (a.flags & NORI_ATTN_MERGE) merge_weights(a.lse[lse_idx], lse_part, w_old, w_new, lse_out);
#pragma unroll
    for (int vt = 0; vt < G::VTILES; ++vt)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int d0 = 32 * vt + 8 * g + 4 * hh;
            if (d0 < d) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float v = o[vt][4 * g + i] * inv;
                    if (a.flags & NORI_ATTN_MERGE) {
                        const float old = reinterpret_cast<const float*>(a.out)[obase + d0 + i];
                        v = old * w_old + v * w_new;
                    }
                    store_from_f32(a.out, a.out_dtype, obase + d0 + i, v);
                }
            }
        }
    if (a.lse && hh == 0) a.lse[lse_idx] = lse_out;
}

// Merge nsplit partial (O, LSE) pairs per (b, h, query) -- and the running output when
// merging -- into the final output. One thread per (b, h, query).
__global__ void __launch_bounds__(256)
combine_splits_kernel(const AttnArgs a) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t rows = a.bg * a.heads * a.nq;
    if (idx >= rows) return;
    const int64_t qi = idx % a.nq;
    const int64_t bh = idx / a.nq;
    const int h = (int)(bh % a.heads);
    const int64_t b = bh / a.heads;
    const int d = a.d;
    float mx = -INFINITY;
    for (int s = 0; s < a.nsplit; ++s) mx = fmaxf(mx, a.part_lse[s * rows + idx]);
    float sum = 0.f;
    for (int s = 0; s < a.nsplit; ++s) sum += expf(a.part_lse[s * rows + idx] - mx);
    const float lse_part = mx + logf(sum);
    float w_old = 0.f, w_new = 1.f, lse_out = lse_part;
    if (a.flags & NORI_ATTN_MERGE) merge_weights(a.lse[idx], lse_part, w_old, w_new, lse_out);
    const int64_t obase = b * a.o_bg + qi * a.o_row + (int64_t)h * a.o_head;
    for (int dd = 0; dd < d; ++dd) {
        float v = 0.f;
        for (int s = 0; s < a.nsplit; ++s)
            v += expf(a.part_lse[s * rows + idx] - lse_part) * a.part_o[(s * rows + idx) * d + dd];
        if (a.flags & NORI_ATTN_MERGE) v = reinterpret_cast<const float*>(a.out)[obase + dd] * w_old + v * w_new;
        store_from_f32(a.out, a.out_dtype, obase + dd, v);
    }
    if (a.lse) a.lse[idx] = lse_out;
}

int device_cu_count() {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) return 256;
    return cus;
}

int choose_splits(int64_t bg, int64_t nq, int heads, int64_t nk, int cus) {
    const int64_t nqt = (nq + QTILE - 1) / QTILE;
    const int64_t base = bg * heads * nqt;
    const int64_t target = 2 * (int64_t)cus;
    if (base >= target) return 1;
    int64_t want = (target + base - 1) / base;
    const int64_t max_by_keys = nk / (4 * KB);  // keep at least 4 blocks per split
    want = std::min<int64_t>(want, std::max<int64_t>(1, max_by_keys));
    return (int)std::max<int64_t>(1, std::min<int64_t>(want, 64));
}

template <int DP>
int launch_dp(int kv_dtype, const AttnArgs& args, hipStream_t stream) {
    const dim3 grid((unsigned)args.nblocks), block(THREADS);
    switch (kv_dtype) {
        case NORI_I8: hipLaunchKernelGGL((icl_attention_kernel<DP, NORI_I8>), grid, block, 0, stream, args); break;
        case NORI_F16: hipLaunchKernelGGL((icl_attention_kernel<DP, NORI_F16>), grid, block, 0, stream, args); break;
        case NORI_BF16: hipLaunchKernelGGL((icl_attention_kernel<DP, NORI_BF16>), grid, block, 0, stream, args); break;
        case NORI_F32: hipLaunchKernelGGL((icl_attention_kernel<DP, NORI_F32>), grid, block, 0, stream, args); break;
        default: return fail(NORI_ERR_UNSUPPORTED, "icl_attention: unsupported cache dtype %s", dtype_name(kv_dtype));
    }
    return NORI_OK;
}

}  // namespace

extern "C" int64_t nori_icl_attention_workspace_size(int64_t bg, int64_t nq, int32_t heads, int32_t d, int64_t nk) {
    if (bg <= 0 || nq <= 0 || heads <= 0 || d <= 0 || nk <= 0) return 0;
    const int ns = choose_splits(bg, nq, heads, nk, device_cu_count());
    if (ns <= 1) return 0;
    return (int64_t)ns * bg * heads * nq * (d + 1) * (int64_t)sizeof(float);
}

extern "C" int nori_icl_attention(const void* q, int q_dtype, int64_t bg, int64_t nq, int32_t heads, int32_t d,
                                  int64_t q_bg_stride, int64_t q_row_stride, int64_t q_head_stride, const void* kv,
                                  int kv_dtype, const float* kv_scales, int64_t nk, int32_t kv_heads,
                                  int64_t kv_bg_stride, int64_t kv_row_stride, int64_t kv_half_stride,
                                  int64_t sc_bg_stride, int64_t sc_row_stride, int64_t sc_half_stride, float scale,
                                  void* out, int out_dtype, int64_t out_bg_stride, int64_t out_row_stride,
                                  int64_t out_head_stride, float* lse, uint32_t flags, void* workspace,
                                  int64_t workspace_bytes, void* stream_v) {
    clear_error();
    if (bg < 0 || nq < 0) return fail(NORI_ERR_INVALID, "icl_attention: negative batch (%lld) or query count (%lld)", (long long)bg, (long long)nq);
    if (heads <= 0 || kv_heads <= 0 || heads % kv_heads)
        return fail(NORI_ERR_INVALID, "icl_attention: query heads %d cannot attend to %d K/V heads", heads, kv_heads);
    if (d < 4 || d > 128 || d % 4)
        return fail(NORI_ERR_UNSUPPORTED, "icl_attention: head width %d is not a multiple of 4 in [4, 128]", d);
    if (nk <= 0) return fail(NORI_ERR_INVALID, "icl_attention: empty K/V cache");
    if (q_dtype != NORI_F32 && q_dtype != NORI_F16 && q_dtype != NORI_BF16)
        return fail(NORI_ERR_UNSUPPORTED, "icl_attention: unsupported query dtype %s", dtype_name(q_dtype));
    if (out_dtype != NORI_F32 && out_dtype != NORI_F16 && out_dtype != NORI_BF16)
        return fail(NORI_ERR_UNSUPPORTED, "icl_attention: unsupported output dtype %s", dtype_name(out_dtype));
    if ((flags & NORI_ATTN_MERGE) && (out_dtype != NORI_F32 || !lse))
        return fail(NORI_ERR_INVALID, "icl_attention: merging needs an fp32 running output and an LSE buffer");
    if (kv_dtype == NORI_I8 && !kv_scales) return fail(NORI_ERR_INVALID, "icl_attention: int8 cache without scales");
    if (bg == 0 || nq == 0) return NORI_OK;
    if (!q || !kv || !out) return fail(NORI_ERR_INVALID, "icl_attention: null pointer");
    if (kv_dtype == NORI_I8 && (((uintptr_t)kv) % 4 || kv_row_stride % 4 || kv_bg_stride % 4 || kv_half_stride % 4))
        return fail(NORI_ERR_UNSUPPORTED, "icl_attention: int8 cache rows must be 4-byte aligned");

    AttnArgs args;
    args.q = q; args.q_dtype = q_dtype; args.nq = nq; args.heads = heads; args.d = d;
    args.q_bg = q_bg_stride; args.q_row = q_row_stride; args.q_head = q_head_stride;
    args.kv = kv; args.kvs = kv_scales; args.nk = nk; args.hgroup = heads / kv_heads;
    args.kv_bg = kv_bg_stride; args.kv_row = kv_row_stride; args.kv_half = kv_half_stride;
    args.sc_bg = sc_bg_stride; args.sc_row = sc_row_stride; args.sc_half = sc_half_stride;
    args.scale_log2 = scale * kLog2e;
    args.out = out; args.out_dtype = out_dtype; args.o_bg = out_bg_stride; args.o_row = out_row_stride;
    args.o_head = out_head_stride; args.lse = lse; args.flags = flags;
    args.bg = bg;
    args.nqt = (int)((nq + QTILE - 1) / QTILE);
    int ns = choose_splits(bg, nq, heads, nk, device_cu_count());
    const int64_t need = (int64_t)ns * bg * heads * nq * (d + 1) * (int64_t)sizeof(float);
    if (ns > 1 && (!workspace || workspace_bytes < need)) ns = 1;
    int64_t kps = (nk + ns - 1) / ns;
    kps = (kps + KB - 1) / KB * KB;
    ns = (int)((nk + kps - 1) / kps);
    args.nsplit = ns;
    args.keys_per_split = kps;
    args.part_o = ns > 1 ? reinterpret_cast<float*>(workspace) : nullptr;
    args.part_lse = ns > 1 ? reinterpret_cast<float*>(workspace) + (int64_t)ns * bg * heads * nq * d : nullptr;
    args.nblocks = bg * heads * (int64_t)args.nqt * ns;
    if (args.nblocks > 0x7fffffffLL) return fail(NORI_ERR_UNSUPPORTED, "icl_attention: grid too large");

    hipStream_t stream = (hipStream_t)stream_v;
    const int dp = (d + 15) / 16 * 16;
    int st;
    switch (dp) {
        case 16: st = launch_dp<16>(kv_dtype, args, stream); break;
        case 32: st = launch_dp<32>(kv_dtype, args, stream); break;
        case 48: st = launch_dp<48>(kv_dtype, args, stream); break;
        case 64: st = launch_dp<64>(kv_dtype, args, stream); break;
        case 80: st = launch_dp<80>(kv_dtype, args, stream); break;
        case 96: st = launch_dp<96>(kv_dtype, args, stream); break;
        case 112: st = launch_dp<112>(kv_dtype, args, stream); break;
        default: st = launch_dp<128>(kv_dtype, args, stream); break;
    }
    if (st != NORI_OK) return st;
    if ((st = launch_status("icl_attention")) != NORI_OK) return st;
    if (ns > 1) {
        const int64_t rows = bg * heads * nq;
        hipLaunchKernelGGL(combine_splits_kernel, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, stream, args);
        return launch_status("icl_attention combine");
    }
    return NORI_OK;
}
