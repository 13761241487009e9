// Query-row -> context attention kernel for gfx950 (device template; the host entry point
// and the launch dispatch live in icl_attention.hip, the explicit instantiations in
// icl_attention_<cache dtype>.hip).
//
// Semantics: out[b, i, h] = softmax_j(scale * q[b, i, h] . k[b, j, hk]) @ v[b, j, hk] with
// hk = h / (heads / kv_heads), plus the natural-log LSE of the scaled logits: the dense cached
// attention (layer.py:936-1049), the CPU online-softmax scan (layer.py:777-839) and the GPU
// flex block + exact LSE merge (layer.py:841-934) of the reference, with the int8
// dequantization of kv_cache_scaling.py:40-41 folded into the tile loads.
//
// Schedule. A workgroup of NW wavefronts owns NW*32 query rows of one (b, h) and one
// context range, scanned in blocks of 64 keys.
//   * Q lives in registers as f16 MFMA operands for the whole scan.
//   * K/V blocks are software pipelined: while the wavefronts compute on block i from one
//     LDS buffer, each thread holds its share of block i+1's raw cache words (issued before
//     the compute, consumed after it) and converts them into the other buffer, so one
//     barrier per block separates the two and the HBM latency hides under the MFMA work.
//       K: int8 codes -> exact f16 integers (v_perm builds 1024+u, one packed add removes
//          the bias); the row's scale times scale*log2(e) goes to an fp32 table, so the
//          logit MFMA is exact in the codes and the scale is applied in fp32.
//       V: exact f16 codes times the f16 row scale (one packed multiply, RN): the fp16
//          value the reference's dequantization produces; stored transposed ([d][key]) with keys
//          permuted inside each 16-key group so the probabilities leave the logit MFMA in
//          the operand order of the PV MFMA (no cross-lane moves).
//   * Per wavefront and block: S^T = K Q^T (v_mfma_f32_32x32x16_f16, 32 keys x 32 queries per
//     tile), x = s*kfac - m (one fma), online softmax in base 2 with lazy rescaling (the
//     running max only moves when a block exceeds it by 2^8), P rounded to f16, and
//     O^T += V^T P^T (v_mfma_f32_32x32x16_f16).
//   * The softmax denominator comes out of the PV MFMA: when the head width leaves a padding
//     row in the last 32-row tile of V^T, that row holds ones and accumulates sum_j p_j for
//     free; only head widths that are multiples of 32 sum P on the VALU.
//   * Workgroups are renumbered so that the query tiles and heads that read the same cache
//     rows are dealt to the same XCD (the hardware deals workgroups round-robin over the 8
//     XCDs), so each cache line comes from HBM once per XCD and is then served by its L2.
#pragma once

#include <math.h>

#include "nori_common.h"

namespace nori {
namespace attn {

// Context rows (keys) per block, the unit of staging and of the one barrier per block:
// 128 for 16-wave workgroups (a barrier over 16 wavefronts is the costlier one), 64 otherwise.
constexpr int block_keys(int nw) { return nw == 16 ? 128 : 64; }
constexpr int QPW = 32;  // query rows per wavefront
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kRescaleSlack = 8.0f;  // log2 units a block may exceed the running max by

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct Args {
    const void* q; int q_dtype; int64_t nq; int heads; int d;
    int64_t q_bg, q_row, q_head;
    const void* kv; const float* kvs; int64_t nk; int hgroup;
    int64_t kv_bg, kv_row, kv_half, sc_bg, sc_row, sc_half;
    float scale_log2;  // logit scale * log2(e)
    void* out; int out_dtype; int64_t o_bg, o_row, o_head;
    float* lse; uint32_t flags;
    // Work items are (b, h, query tile) units, numbered with the query tile fastest. Units
    // [0, n_whole) scan the whole context; each of the tail units [n_whole, nunits) is split
    // into nsplit ranges of keys_per_split keys whose partial (O, LSE) pairs a second kernel
    // merges. grid = n_whole + (nunits - n_whole) * nsplit workgroups.
    int64_t bg; int nqt; int qrows; int nsplit; int64_t keys_per_split;
    int64_t nunits, n_whole, grid;
    float* part_o; float* part_lse;  // [nsplit][tail unit][qrows][d], [nsplit][tail unit][qrows]
};

// 4 int8 codes -> two f16x2 holding the same integers (exact): v_perm builds the f16 bit
// patterns of 1024 + (c + 128), one packed add subtracts 1152.
__device__ __forceinline__ void codes_to_f16(uint32_t w, uint32_t& lo, uint32_t& hi) {
    const uint32_t u = w ^ 0x80808080u;
    const uint32_t a = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
    const uint32_t b = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
    const f16x2 bias = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    lo = __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, a) + bias);
    hi = __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, b) + bias);
}

// 4 int8 codes times a row scale -> two f16x2: exact f16 code integers times the scale
// rounded to f16, one packed multiply (RN). For caches built from fp16 or bf16 tensors the
// scale is an fp16/bf16 value, exactly representable in f16, so this is the value of
// (q.float() * scale).to(float16), the reference's fp16 dequantization, bit for bit; an
// fp32-built cache picks up one extra f16 rounding of its scale (2^-11 relative).
__device__ __forceinline__ void codes_scaled_to_f16(uint32_t w, float s, uint32_t& lo, uint32_t& hi) {
    codes_to_f16(w, lo, hi);
    const _Float16 sh = (_Float16)s;
    const f16x2 s2 = {sh, sh};
    lo = __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, lo) * s2);
    hi = __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, hi) * s2);
}

// Max of 16 values as a depth-3 tree of v_max3_f32, without the NaN-quieting copies the
// compiler puts in front of fmaxf operands (the inputs are MFMA results; NaN inputs give NaN
// outputs either way), in one asm block (the compiler follows every asm statement with a
// hazard nop; one block pays it once).
__device__ __forceinline__ float max16f(const float (&x)[16]) {
    float r, t0, t1, t2, t3;
    asm("v_max3_f32 %1, %5, %6, %7\n\t"
        "v_max3_f32 %2, %8, %9, %10\n\t"
        "v_max3_f32 %3, %11, %12, %13\n\t"
        "v_max3_f32 %4, %14, %15, %16\n\t"
        "v_max3_f32 %0, %17, %18, %19\n\t"
        "v_max3_f32 %1, %1, %2, %20\n\t"
        "v_max3_f32 %0, %0, %3, %4\n\t"
        "v_max_f32 %0, %0, %1"
        : "=&v"(r), "=&v"(t0), "=&v"(t1), "=&v"(t2), "=&v"(t3)
        : "v"(x[0]), "v"(x[1]), "v"(x[2]), "v"(x[3]), "v"(x[4]), "v"(x[5]), "v"(x[6]), "v"(x[7]), "v"(x[8]),
          "v"(x[9]), "v"(x[10]), "v"(x[11]), "v"(x[12]), "v"(x[13]), "v"(x[14]), "v"(x[15]));
    return r;
}

__device__ __forceinline__ float max2f(float a, float b) {
    float r;
    asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

// Value of lane l ^ 32 (the other half-wave), via v_permlane32_swap (no LDS round trip).
__device__ __forceinline__ float other_half(float v) {
    // the swap trades lanes 32-63 of the first operand with lanes 0-31 of the second: r[0]
    // holds lanes 0-31 of v in both halves, r[1] lanes 32-63. fi=true reads the partner lane
    // even where the compiler has masked it off (a select around the call may do that).
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), true, false);
    return __uint_as_float((__lane_id() < 32) ? r[1] : r[0]);
}

__device__ __forceinline__ uint32_t pack_f16(float a, float b) {
    return __builtin_bit_cast(uint32_t, f16x2{(_Float16)a, (_Float16)b});
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

// Merge a normalized partial (o, lse) into the running fp32 output/LSE (layer.py:915-920).
__device__ __forceinline__ void merge_weights(float lse_old, float lse_part, float& w_old, float& w_new,
                                              float& lse_out) {
    const float mx = fmaxf(lse_old, lse_part);
    if (mx == -INFINITY) { w_old = 0.f; w_new = 0.f; lse_out = -INFINITY; return; }
    lse_out = mx + log1pf(expf(-fabsf(lse_old - lse_part)));
    w_old = expf(lse_old - lse_out);
    w_new = expf(lse_part - lse_out);
}

// Raw cache words of one staging unit (4 key rows x 4 head elements of K or V).
template <int KVT> struct Raw;
template <> struct Raw<NORI_I8> { uint32_t w[4]; float s[4]; };
template <> struct Raw<NORI_F16> { u32x2 w[4]; };
template <> struct Raw<NORI_BF16> { u32x2 w[4]; };
template <> struct Raw<NORI_F32> { u32x4 w[4]; };

// How a kernel forms the logits and the softmax denominator for head width d, padded width DP.
enum Mode : int {
    // d < DP. K column d holds ones and the Q fragment carries -m (the running max) there,
    // so the logit MFMA returns s - m in log2 units with no VALU work: Q is prescaled by
    // scale*log2(e) and K rows are dequantized with their scales, the f16 value of the
    // reference's dequantization. The padding row of V^T holds ones and sums P.
    kFold = 0,
    // d = DP < DV: x = s * kfac - m on the VALU from exact f16 K codes and an fp32 per-key
    // factor (scale * scale*log2(e)); the padding row of V^T sums P.
    kOnes = 1,
    // d = DP = DV: as kOnes, with the denominator summed on the VALU.
    kValu = 2,
};

constexpr int mode_for(int d) { return d % 16 != 0 ? kFold : (d % 32 != 0 ? kOnes : kValu); }

template <int DP, bool ONES, int NW>
struct Geometry {
    static_assert(DP % 16 == 0 && DP >= 16 && DP <= 128, "padded head width");
    static constexpr int KB = block_keys(NW);
    static constexpr int SPB = KB / 32;             // 32-key steps per block
    static constexpr int DV = (DP + 31) / 32 * 32;  // PV output rows (MFMA M granule)
    static constexpr int KSTEPS = DP / 16;          // logit MFMA k-steps
    static constexpr int VTILES = DV / 32;
    static constexpr int DQMAX = DP / 4;            // 4-element quads per padded head vector
    static constexpr int KPITCH = DP + 8;           // f16 per K row in LDS (+16 B: conflict-free b128 reads)
    static constexpr int VPITCH = KB + 8;           // f16 per V^T row in LDS
    static constexpr int KBUF = KB * KPITCH;
    static constexpr int VBUF = DV * VPITCH;
    // LDS buffers in the K/V ring: three let a block be staged while the previous block's V
    // and the next block's K are both being read (one barrier per block); wide heads, whose
    // buffers are large, use two and a second barrier. The budget keeps two 8-wave
    // workgroups on a CU (a 16-wave workgroup has the CU to itself).
    static constexpr int BUF_BYTES = (KBUF + VBUF) * 2 + KB * 4;
    static constexpr int NBUF = 3 * BUF_BYTES <= (NW == 16 ? 120 : 64) * 1024 ? 3 : 2;
};

// Shapes with a 16-wave workgroup: narrow heads, where 32 query rows per wavefront fit in
// 128 VGPRs (4 wavefronts per SIMD) with the pipelined logits in flight.
constexpr bool has_16_waves(int dp, int mode) { return dp <= 32 || (dp == 48 && mode == kFold); }

// Register budget: narrow heads keep 4 wavefronts per SIMD (two 8-wave workgroups per CU).
template <int DP, int NW>
struct WavesPerEU { static constexpr int value = (NW == 16 || (NW == 8 && DP <= 48)) ? 4 : 1; };

template <int DP, int KVT, int MODE, int NW>
__global__ void __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(WavesPerEU<DP, NW>::value)))
icl_attention_kernel(const Args a) {
    constexpr bool ONES = MODE != kValu;
    constexpr bool FOLD = MODE == kFold;
    using G = Geometry<DP, ONES, NW>;
    constexpr int KB = G::KB;
    constexpr int THREADS = NW * 64;
    constexpr int UNITS = 2 * (KB / 4) * G::DQMAX;
    constexpr int NU = (UNITS + THREADS - 1) / THREADS;  // staging units per thread (upper bound)
    __shared__ __attribute__((aligned(16))) _Float16 Ks[G::NBUF * G::KBUF];
    __shared__ __attribute__((aligned(16))) _Float16 Vt[G::NBUF * G::VBUF];
    __shared__ __attribute__((aligned(16))) float kfac[FOLD ? 4 : G::NBUF * KB];

    // ---- work item, XCD-aware: the hardware deals workgroup i to XCD i % 8; within each phase
    // (whole units, then tail ranges) give each XCD a contiguous range of items, so the
    // workgroups an XCD runs together read the same cache rows (the query tiles of one
    // (b, h), and with a split context the same key range of both tiles).
    int64_t unit;
    int split = -1;  // context range of a tail unit; -1 for a whole unit
    {
        const bool tail = (int64_t)blockIdx.x >= a.n_whole;
        const int64_t base = tail ? a.n_whole : 0;
        const int64_t n = tail ? a.grid - a.n_whole : a.n_whole;
        const int64_t g = (int64_t)blockIdx.x - base;
        const int64_t xcd = g % 8, local = g / 8, per = n / 8, extra = n % 8;
        const int64_t t = xcd * per + min<int64_t>(xcd, extra) + local;
        if (!tail) {
            unit = t;
        } else {
            unit = a.n_whole + t / a.nsplit;
            split = (int)(t % a.nsplit);
        }
    }
    const int qt = (int)(unit % a.nqt);
    const int h = (int)((unit / a.nqt) % a.heads);
    const int64_t b = unit / a.nqt / a.heads;
    const int hk = h / a.hgroup;

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
    const int64_t qi = (int64_t)qt * (NW * QPW) + wave * QPW + l32;
    const int64_t k_begin = split < 0 ? 0 : (int64_t)split * a.keys_per_split;
    const int64_t k_end = split < 0 ? a.nk : min<int64_t>(a.nk, k_begin + a.keys_per_split);
    const int nblk = (int)((k_end - k_begin + KB - 1) / KB);
    const int d = a.d;
    const int dqv = d >> 2;

    // ---- constant LDS: K columns [d, DP) and V^T rows [d, DV) of every buffer are never
    // staged; they stay zero, except K column d when the logit offset is folded into the
    // MFMA (d is a multiple of 4, so it opens quad d/4) and the ones row (last V^T row)
    // that sums P.
    for (int row = tid; row < G::NBUF * KB; row += THREADS)
        for (int dq = dqv; dq < G::DQMAX; ++dq)
            *reinterpret_cast<u32x2*>(&Ks[(row / KB) * G::KBUF + (row % KB) * G::KPITCH + 4 * dq]) =
                u32x2{(FOLD && dq == dqv) ? 0x3c00u : 0u, 0u};
    for (int e = tid; e < G::NBUF * G::DV * KB; e += THREADS) {
        const int row = (e / KB) % G::DV;  // compile-time divisors
        if (row >= d)
            Vt[(e / (G::DV * KB)) * G::VBUF + row * G::VPITCH + e % KB] =
                (ONES && row == G::DV - 1) ? (_Float16)1.0f : (_Float16)0.0f;
    }

    // ---- Q fragment (B operand of S^T = K Q^T): lane holds q[qi][16ks + 8hh + 0..7], times
    // scale*log2(e) when the logit offset is folded (element d then carries -m, 0 until the
    // first step sets it); the dtype branch is uniform and taken once, outside the loops
    f16x8 qf[G::KSTEPS];
    {
        const float qmul = FOLD ? a.scale_log2 : 1.0f;
        const bool qok = qi < a.nq;
        const int64_t qbase = b * a.q_bg + qi * a.q_row + (int64_t)h * a.q_head;
        auto fill = [&](auto load) {
#pragma unroll
            for (int ks = 0; ks < G::KSTEPS; ++ks) {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int dd = 16 * ks + 8 * hh + j;
                    qf[ks][j] = (qok && dd < d) ? (_Float16)(load(qbase + dd) * qmul) : (_Float16)0.0f;
                }
            }
        };
        if (a.q_dtype == NORI_F16) fill([&](int64_t i) { return f16_to_f32(reinterpret_cast<const uint16_t*>(a.q)[i]); });
        else if (a.q_dtype == NORI_BF16) fill([&](int64_t i) { return bf16_to_f32(reinterpret_cast<const uint16_t*>(a.q)[i]); });
        else fill([&](int64_t i) { return reinterpret_cast<const float*>(a.q)[i]; });
    }

    // ---- staging plan of this thread: unit u covers rows 4rq..4rq+3 and elements 4dq..4dq+3
    // of K (kvsel 0; consecutive threads take consecutive dq, so loads are contiguous) or of V
    // (kvsel 1; consecutive threads take consecutive rq, so the transposed LDS writes of a
    // wavefront land in distinct banks). Loads go through one buffer descriptor per block
    // based at the block's first row (a row holds K then V of every head, so valid rows end
    // at nvalid*row_bytes): per-lane offsets are 32-bit and rows past the end of the context
    // range fall outside the descriptor and read as zero. The same holds for the scales.
    constexpr int kv_es = (KVT == NORI_F32) ? 4 : (KVT == NORI_I8 ? 1 : 2);
    const uint32_t row_bytes = (uint32_t)(a.kv_row * kv_es);
    const uint32_t srow_bytes = (uint32_t)(a.sc_row * 4);
    uint32_t u_off[NU], u_soff[NU], u_lds[NU];
    bool u_v[NU], u_on[NU], u_dq0[NU];
#pragma unroll
    for (int u = 0; u < NU; ++u) {
        const int idx = tid + u * THREADS;
        const int nk_units = (KB / 4) * dqv;
        int rq, dq;
        u_on[u] = idx < 2 * nk_units;
        u_v[u] = idx >= nk_units;
        if (!u_v[u]) { rq = idx / dqv; dq = idx - rq * dqv; }
        else { const int v = idx - nk_units; rq = v % (KB / 4); dq = v / (KB / 4); }
        if (!u_on[u]) { rq = 0; dq = 0; }
        u_dq0[u] = dq == 0;
        u_off[u] = 4 * rq * row_bytes + (uint32_t)(((u_v[u] ? a.kv_half : 0) + hk * d + 4 * dq) * kv_es);
        u_soff[u] = 4 * rq * srow_bytes + (uint32_t)(((u_v[u] ? a.sc_half : 0) + hk) * 4);
        // LDS element offset of the unit's first write in a buffer
        if (!u_v[u]) u_lds[u] = (uint32_t)(4 * rq * G::KPITCH + 4 * dq);
        else u_lds[u] = (uint32_t)(4 * dq * G::VPITCH + 16 * (rq >> 2) + 4 * (((rq & 1) << 1) | ((rq >> 1) & 1)));
    }
    const char* kv_bg_base = reinterpret_cast<const char*>(a.kv) + b * a.kv_bg * kv_es;
    const char* sc_bg_base = reinterpret_cast<const char*>(a.kvs) + b * a.sc_bg * 4;

    auto load_block = [&](int64_t kb, Raw<KVT> (&raw)[NU]) {
        const uint32_t nvalid = (uint32_t)min<int64_t>(KB, k_end - kb);
        const __amdgpu_buffer_rsrc_t rkv = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(kv_bg_base + kb * a.kv_row * kv_es), 0, (int)(nvalid * row_bytes), 0x00020000);
        __amdgpu_buffer_rsrc_t rsc = rkv;
        if constexpr (KVT == NORI_I8)
            rsc = __builtin_amdgcn_make_buffer_rsrc((void*)(sc_bg_base + kb * a.sc_row * 4), 0, (int)(nvalid * srow_bytes),
                                                    0x00020000);
#pragma unroll
        for (int u = 0; u < NU; ++u) {
            if (!u_on[u]) continue;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t off = u_off[u] + i * row_bytes;
                if constexpr (KVT == NORI_I8) {
                    raw[u].w[i] = __builtin_amdgcn_raw_buffer_load_b32(rkv, off, 0, 0);
                    raw[u].s[i] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rsc, u_soff[u] + i * srow_bytes, 0, 0));
                } else if constexpr (KVT == NORI_F32) {
                    raw[u].w[i] = __builtin_amdgcn_raw_buffer_load_b128(rkv, off, 0, 0);
                } else {
                    raw[u].w[i] = __builtin_amdgcn_raw_buffer_load_b64(rkv, off, 0, 0);
                }
            }
        }
    };

    auto store_block = [&](int bufsel, const Raw<KVT> (&raw)[NU]) {
        _Float16* Kd = Ks + bufsel * G::KBUF;
        _Float16* Vd = Vt + bufsel * G::VBUF;
        float* kf = kfac + bufsel * KB;
#pragma unroll
        for (int u = 0; u < NU; ++u) {
            if (!u_on[u]) continue;
            uint32_t lo[4], hi[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if constexpr (KVT == NORI_I8) {
                    if (!FOLD && !u_v[u]) codes_to_f16(raw[u].w[i], lo[i], hi[i]);
                    else codes_scaled_to_f16(raw[u].w[i], raw[u].s[i], lo[i], hi[i]);
                } else if constexpr (KVT == NORI_F16) {
                    lo[i] = raw[u].w[i].x; hi[i] = raw[u].w[i].y;
                } else if constexpr (KVT == NORI_BF16) {
                    const u32x2 v = raw[u].w[i];
                    lo[i] = pack_f16(__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xffff0000u));
                    hi[i] = pack_f16(__uint_as_float(v.y << 16), __uint_as_float(v.y & 0xffff0000u));
                } else {
                    const u32x4 v = raw[u].w[i];
                    lo[i] = pack_f16(__uint_as_float(v.x), __uint_as_float(v.y));
                    hi[i] = pack_f16(__uint_as_float(v.z), __uint_as_float(v.w));
                }
            }
            if (!u_v[u]) {
                _Float16* dst = Kd + u_lds[u];
#pragma unroll
                for (int i = 0; i < 4; ++i) *reinterpret_cast<u32x2*>(dst + i * G::KPITCH) = u32x2{lo[i], hi[i]};
                if (!FOLD && u_dq0[u]) {
                    const int r0 = (int)(u_lds[u] / G::KPITCH);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        float f = a.scale_log2;
                        if constexpr (KVT == NORI_I8) f = raw[u].s[i] * a.scale_log2;
                        kf[r0 + i] = f;
                    }
                }
            } else {
                // transpose the 4x4 (row, d) block; rows of a 16-key group go to columns with
                // bits 2 and 3 of the key index swapped (the PV operand order)
                _Float16* dst = Vd + u_lds[u];
                *reinterpret_cast<u32x2*>(dst + 0 * G::VPITCH) =
                    u32x2{__builtin_amdgcn_perm(lo[1], lo[0], 0x05040100u), __builtin_amdgcn_perm(lo[3], lo[2], 0x05040100u)};
                *reinterpret_cast<u32x2*>(dst + 1 * G::VPITCH) =
                    u32x2{__builtin_amdgcn_perm(lo[1], lo[0], 0x07060302u), __builtin_amdgcn_perm(lo[3], lo[2], 0x07060302u)};
                *reinterpret_cast<u32x2*>(dst + 2 * G::VPITCH) =
                    u32x2{__builtin_amdgcn_perm(hi[1], hi[0], 0x05040100u), __builtin_amdgcn_perm(hi[3], hi[2], 0x05040100u)};
                *reinterpret_cast<u32x2*>(dst + 3 * G::VPITCH) =
                    u32x2{__builtin_amdgcn_perm(hi[1], hi[0], 0x07060302u), __builtin_amdgcn_perm(hi[3], hi[2], 0x07060302u)};
            }
        }
    };

    f32x16 o[G::VTILES];
#pragma unroll
    for (int vt = 0; vt < G::VTILES; ++vt) o[vt] = f32x16{};
    float m_run = 0.0f;  // running max (log2 units)
    float l_run = 0.0f;  // this lane's share of the denominator (VALU-summed head widths only)

    // S^T[32 keys x 32 queries] of the 32 K rows at Kh (lane: keys 8g + 4hh + i, query qi)
    auto logits = [&](const _Float16* Kh) {
        f32x16 acc = f32x16{};
#pragma unroll
        for (int ks = 0; ks < G::KSTEPS; ++ks) {
            const f16x8 kfr = *reinterpret_cast<const f16x8*>(&Kh[l32 * G::KPITCH + 16 * ks + 8 * hh]);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kfr, qf[ks], acc, 0, 0, 0);
        }
        return acc;
    };

    // Online softmax of one 32-key step whose first key is kstep (logits s, per-key factors
    // kf[0..32), V^T columns Vh[.][0..32)), then O^T += V^T P^T. s_next holds the following
    // step's logits, already in flight; with the offset folded into the MFMA they carry the
    // running max they were issued with and follow it when it moves.
    auto softmax_pv = [&](const f32x16& s, f32x16& s_next, const float* kf, const _Float16* Vh, int64_t kstep,
                          bool first) {
        float x[16];
        if constexpr (FOLD) {
#pragma unroll
            for (int r = 0; r < 16; ++r) x[r] = s[r];
        } else {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const f32x4 f = *reinterpret_cast<const f32x4*>(&kf[8 * g + 4 * hh]);
#pragma unroll
                for (int i = 0; i < 4; ++i) x[4 * g + i] = fmaf(s[4 * g + i], f[i], -m_run);
            }
        }
        if (kstep + 32 > k_end) {  // the last step of a context range may be partial
#pragma unroll
            for (int g = 0; g < 4; ++g)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (kstep + 8 * g + 4 * hh + i >= k_end) x[4 * g + i] = -INFINITY;
        }
        float bm = max16f(x);
        {
            // both halves of the swap together hold lanes l and l ^ 32 in every lane
            const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(bm), __float_as_uint(bm), true, false);
            bm = max2f(__uint_as_float(r[0]), __uint_as_float(r[1]));
        }
        if (first || __any(bm > kRescaleSlack)) {
            // anchor the running max on the first step (its first key is valid for every
            // query); afterwards move it up where a step overshoots it (rare: the max settles
            // within the first few blocks). A folded max is an f16 value (the Q fragment
            // carries it), so the shift is the exact difference of two f16 values.
            float shift = first ? bm : fmaxf(bm, 0.0f);
            if constexpr (FOLD) shift = (float)(_Float16)(m_run + shift) - m_run;
            if (!first) {
                const float alpha = __builtin_amdgcn_exp2f(-shift);
                l_run *= alpha;
#pragma unroll
                for (int vt = 0; vt < G::VTILES; ++vt)
#pragma unroll
                    for (int r = 0; r < 16; ++r) o[vt][r] *= alpha;
            }
            m_run += shift;
#pragma unroll
            for (int r = 0; r < 16; ++r) x[r] -= shift;
            if constexpr (FOLD) {
#pragma unroll
                for (int r = 0; r < 16; ++r) s_next[r] -= shift;
#pragma unroll
                for (int ks = 0; ks < G::KSTEPS; ++ks)
#pragma unroll
                    for (int j = 0; j < 8; ++j)
                        if (16 * ks + 8 * hh + j == d) qf[ks][j] = (_Float16)(-m_run);
            }
        }
        // probabilities (f16, RN); pf[c] holds keys 16c + 8hh + 0..7 in the PV operand order
        f16x8 pf[2];
#pragma unroll
        for (int c = 0; c < 2; ++c) {
#pragma unroll
            for (int j = 0; j < 8; j += 2) {
                const float p0 = __builtin_amdgcn_exp2f(x[8 * c + j]);
                const float p1 = __builtin_amdgcn_exp2f(x[8 * c + j + 1]);
                const f16x2 pp = f16x2{(_Float16)p0, (_Float16)p1};
                if constexpr (!ONES) {
                    const f16x2 ones = {(_Float16)1.0f, (_Float16)1.0f};
                    l_run = __builtin_amdgcn_fdot2(pp, ones, l_run, false);
                }
                pf[c][j] = pp[0];
                pf[c][j + 1] = pp[1];
            }
        }
#pragma unroll
        for (int vt = 0; vt < G::VTILES; ++vt) {
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const f16x8 vf = *reinterpret_cast<const f16x8*>(&Vh[(32 * vt + l32) * G::VPITCH + 16 * c + 8 * hh]);
                o[vt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pf[c], o[vt], 0, 0, 0);
            }
        }
    };

    // Software pipeline over 32-key steps: each step issues the logit MFMAs of the following
    // step before its own softmax, so every wavefront always holds MFMA work that is
    // independent of the VALU work in front of it. Blocks are staged into the LDS ring ahead
    // of use from raw words loaded one block before that.
    //   * three buffers: block i+2 is staged while block i is computed (after its first
    //     step) and one barrier closes each block, so the staging overlaps the compute of
    //     the other wavefronts;
    //   * two buffers (wide heads): block i+1 is staged before the last step of block i,
    //     fenced by a barrier on each side.
    Raw<KVT> raw[NU];
    load_block(k_begin, raw);
    store_block(0, raw);
    constexpr int AHEAD = G::NBUF >= 3 ? 2 : 1;
    if constexpr (AHEAD == 2) {
        if (nblk > 1) {
            load_block(k_begin + KB, raw);
            store_block(1, raw);
        }
    }
    if (nblk > AHEAD) load_block(k_begin + AHEAD * KB, raw);
    __syncthreads();
    f32x16 s_cur = logits(Ks);

    for (int blk = 0; blk < nblk; ++blk) {
        const int64_t kb = k_begin + (int64_t)blk * KB;
        const int cur = blk % G::NBUF, nxt = (blk + 1) % G::NBUF;
        const _Float16* Kc = Ks + cur * G::KBUF;
        const _Float16* Vc = Vt + cur * G::VBUF;
        const float* kf = kfac + (FOLD ? 0 : cur * KB);
#pragma unroll
        for (int st = 0; st < G::SPB; ++st) {
            if constexpr (AHEAD == 1) {
                if (st == G::SPB - 1) {
                    __syncthreads();  // every wavefront is done with block blk-1, the target buffer
                    if (blk + 1 < nblk) {
                        store_block(nxt, raw);
                        if (blk + 2 < nblk) load_block(kb + 2 * KB, raw);  // lands during the next block
                    }
                    __syncthreads();
                }
            }
            // logits of the following step in flight: the next 32 rows of this block, or the
            // first 32 rows of the next block (a stale buffer after the last block, unused)
            f32x16 s_next = logits(st + 1 < G::SPB ? Kc + 32 * (st + 1) * G::KPITCH : Ks + nxt * G::KBUF);
            softmax_pv(s_cur, s_next, kf + (FOLD ? 0 : 32 * st), Vc + 32 * st, kb + 32 * st, blk == 0 && st == 0);
            s_cur = s_next;
            if constexpr (AHEAD == 2) {
                if (st == 0 && blk + 2 < nblk) {
                    store_block((blk + 2) % G::NBUF, raw);
                    if (blk + 3 < nblk) load_block(kb + 3 * KB, raw);  // lands during the next block
                }
            }
        }
        if constexpr (AHEAD == 2) __syncthreads();
    }

    // ---------------- epilogue
    float l_tot;
    if constexpr (ONES) {
        // O^T row DV-1 (tile VTILES-1, g = 3, i = 3) sits in the upper half-wave
        const float mine = o[G::VTILES - 1][15];
        const float theirs = other_half(mine);
        l_tot = hh ? mine : theirs;
    } else {
        l_tot = l_run + other_half(l_run);
    }
    if (qi >= a.nq) return;
    const float inv = 1.0f / l_tot;
    const float lse_part = (m_run + __log2f(l_tot)) * kLn2;
    if (split >= 0) {
        const int64_t prow = (split * (a.nunits - a.n_whole) + (unit - a.n_whole)) * a.qrows + (qi - (int64_t)qt * a.qrows);
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
    const bool merge = a.flags & NORI_ATTN_MERGE;
    float w_old = 0.f, w_new = 1.f, lse_out = lse_part;
    if (merge) merge_weights(a.lse[lse_idx], lse_part, w_old, w_new, lse_out);
#pragma unroll
    for (int vt = 0; vt < G::VTILES; ++vt)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int d0 = 32 * vt + 8 * g + 4 * hh;
            if (d0 < d) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float v = o[vt][4 * g + i] * inv;
                    if (merge) v = reinterpret_cast<const float*>(a.out)[obase + d0 + i] * w_old + v * w_new;
                    store_from_f32(a.out, a.out_dtype, obase + d0 + i, v);
                }
            }
        }
    if (a.lse && hh == 0) a.lse[lse_idx] = lse_out;
}

// Launches the kernel instantiation for (cache dtype KVT, dp, mode, nw) over a.grid
// workgroups. Each icl_attention_<dtype>.hip instantiates one KVT (parallel builds).
template <int KVT, int DP, int MODE>
int launch_shape(int nw, const Args& a, hipStream_t stream) {
    const dim3 grid((unsigned)a.grid);
    if constexpr (has_16_waves(DP, MODE)) {
        if (nw == 16) {
            hipLaunchKernelGGL((icl_attention_kernel<DP, KVT, MODE, 16>), grid, dim3(16 * 64), 0, stream, a);
            return NORI_OK;
        }
    }
    if (nw == 8) hipLaunchKernelGGL((icl_attention_kernel<DP, KVT, MODE, 8>), grid, dim3(8 * 64), 0, stream, a);
    else hipLaunchKernelGGL((icl_attention_kernel<DP, KVT, MODE, 2>), grid, dim3(2 * 64), 0, stream, a);
    return NORI_OK;
}

// Padded head width DP has two kernels: kFold for d < DP, and kOnes (DP % 32 = 16) or kValu
// (DP % 32 = 0) for d = DP.
template <int KVT>
int launch_dtype(int dp, int mode, int nw, const Args& a, hipStream_t stream) {
    const bool fold = mode == kFold;
    switch (dp) {
        case 16: return fold ? launch_shape<KVT, 16, kFold>(nw, a, stream) : launch_shape<KVT, 16, kOnes>(nw, a, stream);
        case 32: return fold ? launch_shape<KVT, 32, kFold>(nw, a, stream) : launch_shape<KVT, 32, kValu>(nw, a, stream);
        case 48: return fold ? launch_shape<KVT, 48, kFold>(nw, a, stream) : launch_shape<KVT, 48, kOnes>(nw, a, stream);
        case 64: return fold ? launch_shape<KVT, 64, kFold>(nw, a, stream) : launch_shape<KVT, 64, kValu>(nw, a, stream);
        case 80: return fold ? launch_shape<KVT, 80, kFold>(nw, a, stream) : launch_shape<KVT, 80, kOnes>(nw, a, stream);
        case 96: return fold ? launch_shape<KVT, 96, kFold>(nw, a, stream) : launch_shape<KVT, 96, kValu>(nw, a, stream);
        case 112: return fold ? launch_shape<KVT, 112, kFold>(nw, a, stream) : launch_shape<KVT, 112, kOnes>(nw, a, stream);
        case 128: return fold ? launch_shape<KVT, 128, kFold>(nw, a, stream) : launch_shape<KVT, 128, kValu>(nw, a, stream);
        default: return fail(NORI_ERR_UNSUPPORTED, "icl_attention: no kernel for padded head width %d", dp);
    }
}

int launch_i8(int dp, int mode, int nw, const Args& a, hipStream_t stream);
int launch_f16(int dp, int mode, int nw, const Args& a, hipStream_t stream);
int launch_bf16(int dp, int mode, int nw, const Args& a, hipStream_t stream);
int launch_f32(int dp, int mode, int nw, const Args& a, hipStream_t stream);

inline int launch_kvt(int kv_dtype, int dp, int mode, int nw, const Args& a, hipStream_t stream) {
    switch (kv_dtype) {
        case NORI_I8: return launch_i8(dp, mode, nw, a, stream);
        case NORI_F16: return launch_f16(dp, mode, nw, a, stream);
        case NORI_BF16: return launch_bf16(dp, mode, nw, a, stream);
        case NORI_F32: return launch_f32(dp, mode, nw, a, stream);
        default: return fail(NORI_ERR_UNSUPPORTED, "icl_attention: unsupported cache dtype %s", dtype_name(kv_dtype));
    }
}

// Workgroups of the int8-cache kernel for (dp, mode, nw) that fit on one CU at once.
int resident_workgroups(int dp, int mode, int nw);

}  // namespace attn
}  // namespace nori
