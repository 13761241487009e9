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
// context range, scanned in blocks of KB keys.
//   * Q lives in registers as f16 MFMA operands for the whole scan.
//   * K/V blocks are staged into an LDS ring, both row-major ([key][d], f16), two blocks
//     ahead of use, from raw cache words loaded one block before that. A staging lane owns 16
//     consecutive elements of one row of K or V: one 16-byte load of int8 codes, an exact
//     int8 -> f16 conversion (v_perm builds 1024+u, one packed add removes the bias), the row
//     scale applied by one packed multiply, and two 16-byte LDS writes. The (chunk, K|V) of a
//     lane is uniform over its wavefront, and the staging wavefronts are spread evenly over
//     the four SIMDs.
//   * Per wavefront and 32-key step: S^T = K Q^T (v_mfma_f32_32x32x16_f16, 32 keys x 32
//     queries), online softmax in base 2 with lazy rescaling (the running max only moves when
//     a step exceeds it by 2^8), P rounded to f16, then O^T += V^T P^T on
//     v_mfma_f32_16x16x32_f16 (16 head elements x 16 queries per tile, so V pads only to the
//     next multiple of 16). Four v_permlane16_swap turn the probabilities of the logit tile
//     into the two 16-query B operands; V^T operands come straight from the row-major V tile
//     through ds_read_b64_tr_b16, whose per-lane row addresses put the keys in the order the
//     swapped probabilities hold them.
//   * When the head width is not a multiple of 16 the padding carries the rest of the
//     softmax: K column d holds ones and the Q fragment -m (the running max), so the logit
//     MFMA returns s - m in log2 units, and the last V column holds ones, so the PV MFMA
//     accumulates the denominator sum_j p_j in its last output row.
//   * Workgroups are renumbered so that the query tiles and heads that read the same cache
//     rows are dealt to the same XCD (the hardware deals workgroups round-robin over the 8
//     XCDs), so each cache line comes from HBM once per XCD and is then served by its L2.
#pragma once

#include <math.h>

#include "nori_common.h"

namespace nori {
namespace attn {

// Resident-context workgroups: 10 wavefronts (320 query rows of one (b, h)) that stage the
// unit's whole context, at most kResidentKeys rows, into LDS once, behind one barrier, and then
// scan it with no further staging. For contexts this short the ring's per-block load latency
// and barriers dominate: the 256-key column attention of many small tables spends 90 % of a
// wavefront's life waiting in the ring kernel. The scan's arithmetic is the ring kernel's.
constexpr int kResidentKeys = 256;
constexpr bool resident(int nw) { return nw == 10; }

// Context rows (keys) per block, the unit of staging and of the one barrier per block:
// 128 for 16-wave workgroups (a barrier over 16 wavefronts is the costlier one), the whole
// context for resident workgroups, 64 otherwise.
constexpr int block_keys(int nw) { return nw == 16 ? 128 : (resident(nw) ? kResidentKeys : 64); }
constexpr int QPW = 32;  // query rows per wavefront
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kRescaleSlack = 8.0f;  // log2 units a step may exceed the running max by

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
// LDS (address space 3) views: constant offsets from an LDS pointer fold into the DS
// instructions' offset field, so a step's operand reads share one address register
typedef __attribute__((address_space(3))) _Float16 lds_f16;
typedef __attribute__((address_space(3))) f16x8 lds_f16x8;
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// An LDS pointer the optimizer cannot take apart: the per-block operand bases pass through
// this, so every read of a step is base + constant (without it, loop strength reduction
// rebuilds each read's address from separate per-read terms on the VALU).
__device__ __forceinline__ const lds_f16* opaque_lds(const lds_f16* p) {
    uint32_t a = (uint32_t)(uintptr_t)p;
    asm("" : "+v"(a));
    return (const lds_f16*)(uintptr_t)a;
}

// ds_read_b64_tr_b16 at an LDS address (8-byte aligned)
__device__ __forceinline__ f16x4 read_tr16(const lds_f16* p) {
    return __builtin_bit_cast(f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)p));
}

// Layout facts the host has checked, passed in the high bits of Args::flags (the C ABI's
// flags use the low bits): 16-bit queries whose pointer, row, head and batch strides are
// multiples of 8 elements with d a multiple of 8 (16-byte fragment loads) or of 4 elements
// (8-byte loads), and a 16-bit output with 4-element aligned pointer and strides written
// without a merge (8-byte stores).
constexpr uint32_t kQVec8 = 1u << 31;
constexpr uint32_t kQVec4 = 1u << 30;
constexpr uint32_t kOutVec4 = 1u << 29;

struct Args {
    const void* q; int q_dtype; int64_t nq; int heads; int d;
    int64_t q_bg, q_row, q_head;
    const void* kv; const float* kvs; int64_t nk; int hgroup;
    int64_t kv_bg, kv_row, kv_half, sc_bg, sc_row, sc_half;
    float scale_log2;  // logit scale * log2(e)
    void* out; int out_dtype; int64_t o_bg, o_row, o_head;
    float* lse; uint32_t flags;
    // The q/k prologue of resident-context launches (null gains: none): the per-head RMS norms
    // of the query rows and of the staged key rows with their gains (dtype pwdt) and eps, then
    // the query multiply pqmult, each step rounded to its operand's dtype.
    const void* pqw = nullptr; const void* pkw = nullptr; int pwdt = NORI_F32; float peps = 0.f; float pqmult = 1.f;
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

// Two f16x2 words times an f16 scale, one packed multiply each (RN). For caches built from
// fp16 or bf16 tensors the scale is an fp16/bf16 value, exactly representable in f16, so
// code * scale is the value of (q.float() * scale).to(float16), the reference's fp16
// dequantization, bit for bit; an fp32-built cache picks up one extra f16 rounding of its
// scale (2^-11 relative).
__device__ __forceinline__ uint32_t scale_f16x2(uint32_t w, _Float16 s) {
    const f16x2 s2 = {s, s};
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, w) * s2);
}

// Max of 16 values as a depth-3 tree of v_max3_f32, without the NaN-quieting copies the
// compiler puts in front of fmaxf operands (the inputs are MFMA results; NaN inputs give NaN
// outputs either way), in one asm block (the compiler follows every asm statement with a
// hazard nop; one block pays it once). The compiler pads no wait states in front of an asm
// block for MFMA results it reads, so its inputs must be MFMA results issued well before
// (here: one pipeline step earlier).
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

// Value of lane `src` (all lanes active).
__device__ __forceinline__ float lane_value(float v, int src) {
    return __int_as_float(__builtin_amdgcn_ds_bpermute(src << 2, __float_as_int(v)));
}

__device__ __forceinline__ uint32_t pack_f16(float a, float b) {
    return __builtin_bit_cast(uint32_t, f16x2{(_Float16)a, (_Float16)b});
}

// v rounded to a runtime dtype, as torch rounds an op's result in that dtype
__device__ __forceinline__ float round_to_dtype(float v, int dt) {
    if (dt == NORI_F16) return round_to<NORI_F16>(v);
    if (dt == NORI_BF16) return round_to<NORI_BF16>(v);
    return v;
}

// sum over the 4 lanes of a quad (DPP quad permutations), every lane gets it
__device__ __forceinline__ float quad_sum(float v) {
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xb1, 0xf, 0xf, false));  // lane ^ 1
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4e, 0xf, 0xf, false));  // lane ^ 2
    return v;
}

// w[a][b] = element idx(a, b) of the gain vector p (dtype dt; d elements; indices at or past d
// read element d - 1), converted to fp32 behind one dtype branch: the per-element branches of
// load_as_f32 in unrolled loops cost more than the loads
template <int A, int B, typename Idx>
__device__ __forceinline__ void gains_of(const void* p, int dt, int d, Idx idx, float (&w)[A][B]) {
    auto fill = [&](auto load) {
#pragma unroll
        for (int a = 0; a < A; ++a)
#pragma unroll
            for (int b = 0; b < B; ++b) w[a][b] = load(min(idx(a, b), d - 1));
    };
    if (dt == NORI_F32) fill([&](int i) { return reinterpret_cast<const float*>(p)[i]; });
    else if (dt == NORI_F16) fill([&](int i) { return f16_to_f32(reinterpret_cast<const uint16_t*>(p)[i]); });
    else fill([&](int i) { return bf16_to_f32(reinterpret_cast<const uint16_t*>(p)[i]); });
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

constexpr int elem_size(int kvt) { return kvt == NORI_F32 ? 4 : (kvt == NORI_I8 ? 1 : 2); }

// Raw cache words of one staging unit: 16 consecutive elements of one row of K or V (and,
// for int8 codes, the row's scale).
template <int KVT>
struct Raw {
    uint32_t w[4 * elem_size(KVT)];
    float s;
};

// nbytes (a multiple of 4, at most 4 * NWORDS, uniform over the wavefront) raw bytes at byte
// offset `off` of a buffer, in 16/12/8/4-byte loads; the words past nbytes are zero.
template <int NWORDS>
__device__ __forceinline__ void load_words(__amdgpu_buffer_rsrc_t r, uint32_t off, int nbytes, uint32_t (&w)[NWORDS]) {
#pragma unroll
    for (int p = 0; p < NWORDS / 4; ++p) {
        const int left = nbytes - 16 * p;
        const uint32_t o = off + 16 * p;
        if (left >= 16) {
            const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, o, 0, 0);
            w[4 * p] = v.x; w[4 * p + 1] = v.y; w[4 * p + 2] = v.z; w[4 * p + 3] = v.w;
        } else if (left == 12) {
            const u32x3 v = __builtin_amdgcn_raw_buffer_load_b96(r, o, 0, 0);
            w[4 * p] = v.x; w[4 * p + 1] = v.y; w[4 * p + 2] = v.z; w[4 * p + 3] = 0u;
        } else if (left == 8) {
            const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, o, 0, 0);
            w[4 * p] = v.x; w[4 * p + 1] = v.y; w[4 * p + 2] = 0u; w[4 * p + 3] = 0u;
        } else if (left == 4) {
            w[4 * p] = __builtin_amdgcn_raw_buffer_load_b32(r, o, 0, 0);
            w[4 * p + 1] = 0u; w[4 * p + 2] = 0u; w[4 * p + 3] = 0u;
        } else {
            w[4 * p] = 0u; w[4 * p + 1] = 0u; w[4 * p + 2] = 0u; w[4 * p + 3] = 0u;
        }
    }
}

// How a kernel forms the logits and the softmax denominator for head width d, padded width DP.
enum Mode : int {
    // d < DP (d not a multiple of 16). K column d holds ones and the Q fragment carries -m
    // (the running max) there, so the logit MFMA returns s - m in log2 units with no VALU
    // work: Q is prescaled by scale*log2(e) and K rows are dequantized with their scales, the
    // f16 value of the reference's dequantization. The last V column holds ones and sums P.
    kFold = 0,
    // d = DP: x = s * kfac - m on the VALU from exact f16 K codes and an fp32 per-key factor
    // (scale * scale*log2(e)); the denominator is summed on the VALU.
    kValu = 1,
};

constexpr int mode_for(int d) { return d % 16 != 0 ? kFold : kValu; }

template <int DP, int NW>
struct Geometry {
    static_assert(DP % 16 == 0 && DP >= 16 && DP <= 128, "padded head width");
    static constexpr int KB = block_keys(NW);
    static constexpr int SPB = KB / 32;        // 32-key steps per block
    static constexpr int KSTEPS = DP / 16;     // logit MFMA k-steps
    static constexpr int VT = DP / 16;         // 16-row tiles of O^T (PV output)
    static constexpr int KPITCH = DP + 8;      // f16 per K row in LDS (+16 B: conflict-free b128 reads)
    // f16 per V row: the transposed reads of a 16-lane group take 32 bytes from each of 4
    // rows, which land in distinct banks when the row stride is an odd multiple of 32 bytes
    static constexpr int VPITCH = DP % 32 == 0 ? DP + 16 : DP;
    // A transposed read serves 32 lanes at a time from the 64 banks (256 bytes): lanes 0-15
    // read rows 0-3 (+4: 4-7) of a 32-row step and lanes 16-31 rows 16-19 (20-23), and
    // 16 * VPITCH bytes is a multiple of 256, so rows 16-31 of every step sit 128 bytes
    // further on (4 * VPITCH bytes is 128 modulo 256: they take the banks of rows 4-7).
    static constexpr int VSTEP = 32 * VPITCH + 64;  // f16 per 32-row step of a V buffer
    static constexpr int KBUF = KB * KPITCH;
    static constexpr int VBUF = (KB / 32) * VSTEP;
    // f16 offset of row r of a V buffer
    static constexpr __host__ __device__ int vrow(int r) { return (r >> 5) * VSTEP + (r & 31) * VPITCH + ((r & 16) ? 64 : 0); }
    // LDS buffers in the K/V ring: three let a block be staged while the previous block's V
    // and the next block's K are both being read (one barrier per block); wide heads, whose
    // buffers are large, use two and a second barrier. The budget keeps two 8-wave or three
    // 5-wave workgroups on a CU (a 16-wave workgroup has the CU to itself). A resident
    // workgroup holds one buffer, the whole context (two fit on a CU at head widths up to 64).
    static constexpr int BUF_BYTES = (KBUF + VBUF) * 2 + KB * 4;
    static constexpr int NBUF =
        resident(NW) ? 1 : (3 * BUF_BYTES <= (NW == 16 ? 120 : (NW == 5 ? 52 : 72)) * 1024 ? 3 : 2);
};

// Shapes with a 16-wave workgroup: narrow heads, where 32 query rows per wavefront fit in
// 128 VGPRs (4 wavefronts per SIMD) with the pipelined logits in flight. (A 64-wide head in
// the VALU mode needs more and spills.)
constexpr bool has_16_waves(int dp, int mode) { return dp <= 32 || ((dp == 48 || dp == 64) && mode == kFold); }

// Shapes with a 5-wave workgroup (160 query rows; three per CU): heads up to 64 wide, for query
// counts that 160-row tiles cover with less padding than 256- or 512-row ones (320 rows: two
// exact tiles instead of two 256-row tiles).
constexpr bool has_5_waves(int dp) { return dp <= 64; }

// Shapes with a resident-context workgroup (10 wavefronts, two per CU): heads up to 64 wide,
// whose 256-key K and V buffers (80 KB) leave room for a second workgroup.
constexpr bool has_resident(int dp) { return dp <= 64; }

// Register budget: heads up to 64 wide keep 4 wavefronts per SIMD (two 8-wave workgroups per
// CU). Without the bound the 64-wide 8-wave fold kernel takes 135 VGPRs and only one workgroup
// fits; with it, it (and the 48-wide VALU-mode kernel) spills 6 registers to scratch and still
// runs faster (nori-100m layer shape on 8-wave workgroups: 94.4 ms unbounded, 80.7 ms bounded).
template <int DP, int NW>
struct WavesPerEU {
    // two resident 10-wave workgroups per CU: five wavefronts per SIMD
    static constexpr int value = resident(NW) ? 5 : ((NW == 16 || ((NW == 8 || NW == 5) && DP <= 64)) ? 4 : 1);
};

template <int DP, int KVT, int MODE, int NW>
__global__ void __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(WavesPerEU<DP, NW>::value)))
icl_attention_kernel(const Args a) {
    constexpr bool FOLD = MODE == kFold;
    using G = Geometry<DP, NW>;
    constexpr int KB = G::KB;
    constexpr int THREADS = NW * 64;
    constexpr int ES = elem_size(KVT);
    constexpr int NU = (2 * KB * (DP / 16) + THREADS - 1) / THREADS;  // staging units per thread (upper bound)
    __shared__ __attribute__((aligned(16))) _Float16 Ks[G::NBUF * G::KBUF];
    __shared__ __attribute__((aligned(16))) _Float16 Vs[G::NBUF * G::VBUF];
    __shared__ __attribute__((aligned(16))) float kfac[(FOLD || KVT != NORI_I8) ? 4 : G::NBUF * KB];

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
    // keys in this context range (< 2^31, checked on the host), kept in a scalar register so
    // the per-step "partial step" test is a scalar branch
    const int klen = __builtin_amdgcn_readfirstlane((int)(k_end - k_begin));
    const int nblk = (klen + KB - 1) / KB;
    const int d = a.d;

    // ---- constant LDS: K columns [d, DP) and V columns [d, DP) of every buffer are never
    // staged; they stay zero, except, when the logit offset and the denominator are folded
    // into the MFMAs, K column d (ones: d is a multiple of 4, so it opens quad d/4) and the
    // last V column (ones).
    for (int e = tid; e < G::NBUF * KB * (DP / 4); e += THREADS) {
        const int row = e / (DP / 4), col = 4 * (e % (DP / 4));  // compile-time divisors
        if (col >= d) {
            *reinterpret_cast<u32x2*>(&Ks[(row / KB) * G::KBUF + (row % KB) * G::KPITCH + col]) =
                u32x2{(FOLD && col == d) ? 0x3c00u : 0u, 0u};
            *reinterpret_cast<u32x2*>(&Vs[(row / KB) * G::VBUF + G::vrow(row % KB) + col]) =
                u32x2{0u, (FOLD && col == DP - 4) ? 0x3c000000u : 0u};
        }
    }

    // ---- Q fragment (B operand of S^T = K Q^T): lane holds q[qi][16ks + 8hh + 0..7], times
    // scale*log2(e) when the logit offset is folded (element d then carries -m, 0 until the
    // first step sets it); the dtype branch is uniform and taken once, outside the loops
    f16x8 qf[G::KSTEPS];
    {
        const float qmul = FOLD ? a.scale_log2 : 1.0f;
        const bool qok = qi < a.nq;
        // Every element is loaded, at an index clamped into a valid row (the last query for the
        // padding rows of a tile, element d - 1 past the head), and the value is selected away:
        // with no branch around a load, the fragment's loads issue back to back and share one
        // wait instead of costing one memory round trip each.
        const int64_t qbase = b * a.q_bg + min<int64_t>(qi, a.nq - 1) * a.q_row + (int64_t)h * a.q_head;
        float qv[G::KSTEPS][8];
        // Resident-context launches take fp16 queries only (the launch planner sends the others
        // to the ring kernels): a workgroup there runs its code once, so the query dtypes it
        // does not take would only cost it instruction fetches.
        if (a.flags & kQVec8) {
            // one 16-byte load per 8-element chunk (a chunk past the head is zero)
            const uint16_t* q16 = reinterpret_cast<const uint16_t*>(a.q);
            const bool bf = !resident(NW) && a.q_dtype == NORI_BF16;
#pragma unroll
            for (int ks = 0; ks < G::KSTEPS; ++ks) {
                const int dd = 16 * ks + 8 * hh;
                const u32x4 w = *reinterpret_cast<const u32x4*>(q16 + qbase + min(dd, d - 8));
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const uint16_t e = (uint16_t)(w[j >> 1] >> (16 * (j & 1)));
                    qv[ks][j] = dd < d ? (bf ? bf16_to_f32(e) : f16_to_f32(e)) : 0.0f;
                }
            }
        } else {
            auto fill = [&](auto load) {
#pragma unroll
                for (int ks = 0; ks < G::KSTEPS; ++ks) {
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const int dd = 16 * ks + 8 * hh + j;
                        const float v = load(qbase + min(dd, d - 1));
                        qv[ks][j] = dd < d ? v : 0.0f;
                    }
                }
            };
            if (resident(NW) || a.q_dtype == NORI_F16) fill([&](int64_t i) { return f16_to_f32(reinterpret_cast<const uint16_t*>(a.q)[i]); });
            else if (a.q_dtype == NORI_BF16) fill([&](int64_t i) { return bf16_to_f32(reinterpret_cast<const uint16_t*>(a.q)[i]); });
            else fill([&](int64_t i) { return reinterpret_cast<const float*>(a.q)[i]; });
        }
        if constexpr (resident(NW)) {
            if (a.pqw) {
                // the query row's RMS norm with its gain, T(T(q * rsqrt(mean(q^2) + eps)) * w),
                // then T(q * qmult), T rounding to fp16 (the query dtype) as the separate passes
                // do; the row's other half is in lane ^ 32
                float ss = 0.0f;
#pragma unroll
                for (int ks = 0; ks < G::KSTEPS; ++ks)
#pragma unroll
                    for (int j = 0; j < 8; ++j) ss = fmaf(qv[ks][j], qv[ks][j], ss);
                ss += other_half(ss);
                const float inv = rsqrtf(ss / (float)d + a.peps);
                // the gains of this lane's elements behind one dtype branch (per-element dtype
                // branches in these unrolled loops cost a short-lived workgroup more than its
                // arithmetic does), then the fp16 roundings
                float wq[G::KSTEPS][8];
                gains_of(a.pqw, a.pwdt, d, [&](int ks, int j) { return 16 * ks + 8 * hh + j; }, wq);
#pragma unroll
                for (int ks = 0; ks < G::KSTEPS; ++ks)
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        if (16 * ks + 8 * hh + j < d) {
                            float v = round_to<NORI_F16>(round_to<NORI_F16>(qv[ks][j] * inv) * wq[ks][j]);
                            if (a.pqmult != 1.0f) v = round_to<NORI_F16>(v * a.pqmult);
                            qv[ks][j] = v;
                        }
                    }
            }
        }
#pragma unroll
        for (int ks = 0; ks < G::KSTEPS; ++ks)
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int dd = 16 * ks + 8 * hh + j;
                qf[ks][j] = (qok && dd < d) ? (_Float16)(qv[ks][j] * qmul) : (_Float16)0.0f;
            }
    }

    // ---- staging plan of this thread. Unit idx = tid + u * THREADS covers elements
    // [16c, 16c + n) of row idx % KB of K (half 0) or V (half 1), with (c, half) = idx / KB
    // split as c = group / 2, half = group % 2: KB is a multiple of 64, so (c, half) -- and the
    // load width n = min(16, d - 16c) -- are uniform over a wavefront. Loads go through one
    // buffer descriptor per block based at the block's first row (a row holds K then V of every
    // head, so valid rows end at nvalid*row_bytes): per-lane offsets are 32-bit and rows past
    // the end of the context range fall outside the descriptor and read as zero. The same
    // holds for the scales.
    const uint32_t row_bytes = (uint32_t)(a.kv_row * ES);
    const uint32_t srow_bytes = (uint32_t)(a.sc_row * 4);
    const int nch = (d + 15) >> 4;  // 16-element chunks per head vector
    const int wave_first = __builtin_amdgcn_readfirstlane(wave * 64);
    uint32_t u_off[NU], u_soff[NU], u_lds[NU];
    int u_nel[NU];  // elements of the unit (0: no unit), uniform over the wavefront
    bool u_v[NU], u_c0[NU];
#pragma unroll
    for (int u = 0; u < NU; ++u) {
        const int first = wave_first + u * THREADS;  // unit of lane 0
        const int group = first / KB;                // uniform
        const int row = first % KB + lane;
        const int half = group & 1, c = group >> 1;
        u_nel[u] = c < nch ? min(16, d - 16 * c) : 0;
        u_v[u] = half != 0;
        u_c0[u] = c == 0;
        u_off[u] = row * row_bytes + (uint32_t)(((half ? a.kv_half : 0) + hk * d + 16 * c) * ES);
        u_soff[u] = row * srow_bytes + (uint32_t)(((half ? a.sc_half : 0) + hk) * 4);
        u_lds[u] = (uint32_t)((half ? G::vrow(row) : row * G::KPITCH) + 16 * c);
    }
    const char* kv_bg_base = reinterpret_cast<const char*>(a.kv) + b * a.kv_bg * ES;
    const char* sc_bg_base = reinterpret_cast<const char*>(a.kvs) + b * a.sc_bg * 4;

    auto load_block = [&](int64_t kb, Raw<KVT> (&raw)[NU]) {
        const uint32_t nvalid = (uint32_t)min<int64_t>(KB, k_end - kb);
        const __amdgpu_buffer_rsrc_t rkv = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(kv_bg_base + kb * a.kv_row * ES), 0, (int)(nvalid * row_bytes), 0x00020000);
        __amdgpu_buffer_rsrc_t rsc = rkv;
        if constexpr (KVT == NORI_I8)
            rsc = __builtin_amdgcn_make_buffer_rsrc((void*)(sc_bg_base + kb * a.sc_row * 4), 0, (int)(nvalid * srow_bytes),
                                                    0x00020000);
#pragma unroll
        for (int u = 0; u < NU; ++u) {
            if (u_nel[u] == 0) continue;
            load_words(rkv, u_off[u], u_nel[u] * ES, raw[u].w);
            if constexpr (KVT == NORI_I8) raw[u].s = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rsc, u_soff[u], 0, 0));
        }
    };

    auto store_block = [&](int bufsel, const Raw<KVT> (&raw)[NU]) {
#pragma unroll
        for (int u = 0; u < NU; ++u) {
            const int n = u_nel[u];
            if (n == 0) continue;
            // 16 f16 of the unit, as 8 words
            uint32_t f[8];
            if constexpr (KVT == NORI_I8) {
                const bool scaled = FOLD || u_v[u];
                const _Float16 sh = (_Float16)raw[u].s;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    codes_to_f16(raw[u].w[i], f[2 * i], f[2 * i + 1]);
                    if (scaled) {
                        f[2 * i] = scale_f16x2(f[2 * i], sh);
                        f[2 * i + 1] = scale_f16x2(f[2 * i + 1], sh);
                    }
                }
                if (!FOLD && !u_v[u] && u_c0[u]) kfac[bufsel * KB + (int)(u_lds[u] / G::KPITCH)] = raw[u].s * a.scale_log2;
            } else if constexpr (KVT == NORI_F16) {
#pragma unroll
                for (int i = 0; i < 8; ++i) f[i] = raw[u].w[i];
            } else if constexpr (KVT == NORI_BF16) {
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const uint32_t v = raw[u].w[i];
                    f[i] = pack_f16(__uint_as_float(v << 16), __uint_as_float(v & 0xffff0000u));
                }
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i) f[i] = pack_f16(__uint_as_float(raw[u].w[2 * i]), __uint_as_float(raw[u].w[2 * i + 1]));
            }
            _Float16* dst = (u_v[u] ? Vs + bufsel * G::VBUF : Ks + bufsel * G::KBUF) + u_lds[u];
            // n f16 (a multiple of 4, uniform over the wavefront): 16-byte and 8-byte writes
            if (n >= 8) *reinterpret_cast<u32x4*>(dst) = u32x4{f[0], f[1], f[2], f[3]};
            else *reinterpret_cast<u32x2*>(dst) = u32x2{f[0], f[1]};
            if (n == 16) *reinterpret_cast<u32x4*>(dst + 8) = u32x4{f[4], f[5], f[6], f[7]};
            else if (n == 12) *reinterpret_cast<u32x2*>(dst + 8) = u32x2{f[4], f[5]};
        }
    };

    // O^T accumulators: tile (t, qb) holds rows 16t + 4*(lane/16) + 0..3 of query 16qb + lane%16
    f32x4 o[G::VT][2];
#pragma unroll
    for (int t = 0; t < G::VT; ++t) o[t][0] = o[t][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run = 0.0f;  // running max (log2 units) of query l32
    float l_run = 0.0f;  // this lane's share of the denominator (VALU-summed head widths only)

    // S^T[32 keys x 32 queries] of the 32 K rows whose first row is at this lane's Kl - its own
    // row offset (lane: keys 8g + 4hh + i, query qi)
    const int k_lane = l32 * G::KPITCH + 8 * hh;  // this lane's A-operand element in a 32-row step
    // PREFETCH (the shapes whose register budget has room) holds the K operands of the step
    // after next in registers across a step, so the logit MFMAs never wait on LDS, and reads a
    // step's V operands before its softmax.
    constexpr bool PREFETCH = (DP <= 48 && !(KVT == NORI_F32 && NW == 8)) || WavesPerEU<DP, NW>::value == 1;
    // K operands of one 32-key step (the A operands of its logit MFMAs) at this lane's Kl
    auto read_k = [&](const lds_f16* Kl, f16x8 (&kfr)[G::KSTEPS]) {
#pragma unroll
        for (int ks = 0; ks < G::KSTEPS; ++ks) kfr[ks] = *reinterpret_cast<const lds_f16x8*>(Kl + 16 * ks);
    };
    auto logits = [&](const f16x8 (&kfr)[G::KSTEPS]) {
        f32x16 acc = f32x16{};
#pragma unroll
        for (int ks = 0; ks < G::KSTEPS; ++ks) acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kfr[ks], qf[ks], acc, 0, 0, 0);
        return acc;
    };

    // Row offset (in f16 elements, within a 32-key step of a V buffer) of this lane's
    // transposed V^T reads. ds_read_b64_tr_b16 gives lane i of each 16-lane group g element
    // i % 4 of the 8 bytes read by lanes 16g + i/4 + 4j (j = 0..3), so a lane reading 4
    // consecutive head elements of key row R(g, t) makes lane i receive V[keys][16T + i]: the
    // A operand of the 16x16x32 PV MFMA, with its k-slot 8g + j holding key
    // sigma(g, j) = 16(g%2) + 4(g/2) + 8(j/4) + j%4 -- the key the swapped probability
    // registers hold in that slot. The second read (slots 4..7) is 8 key rows further.
    const int vg = lane >> 4, vt = lane & 15;
    const int v_lane = G::vrow(16 * (vg & 1) + 4 * (vg >> 1) + (vt >> 2)) + 4 * (vt & 3);
    const lds_f16* const KsL = (const lds_f16*)Ks;
    const lds_f16* const VsL = (const lds_f16*)Vs;
    auto read_v = [&](const lds_f16* Vl, f16x8 (&vf)[G::VT]) {
#pragma unroll
        for (int t = 0; t < G::VT; ++t) {
            const f16x4 lo = read_tr16(Vl + 16 * t);
            const f16x4 hi = read_tr16(Vl + 8 * G::VPITCH + 16 * t);
            vf[t] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        }
    };

    // Probabilities of keys 2t, 2t + 1 of a step's 16 (f16, RN) from their base-2 logit
    // offsets, as one word (keys 8(t/2) + 4hh + 2(t%2) + 0..1); lsum takes their sum
    // (VALU-summed head widths).
    auto prob_pair = [&](const float (&x)[16], int t, float& lsum) {
        const f16x2 pp = f16x2{(_Float16)__builtin_amdgcn_exp2f(x[2 * t]), (_Float16)__builtin_amdgcn_exp2f(x[2 * t + 1])};
        if constexpr (!FOLD) {
            const f16x2 ones = {(_Float16)1.0f, (_Float16)1.0f};
            lsum = __builtin_amdgcn_fdot2(pp, ones, lsum, false);
        }
        return __builtin_bit_cast(uint32_t, pp);
    };
    // The B operands of the two 16-query blocks from a step's 8 probability words: swapping
    // words t and t + 4 between 16-lane rows gives block 0 (queries 0-15) and block 1
    // (queries 16-31) their 32 keys each.
    auto b_operands = [&](const uint32_t (&pw)[8], f16x8& p0, f16x8& p1) {
        u32x4 pa, pb;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const auto r = __builtin_amdgcn_permlane16_swap(pw[t], pw[t + 4], false, false);
            pa[t] = r[0];
            pb[t] = r[1];
        }
        p0 = __builtin_bit_cast(f16x8, pa);
        p1 = __builtin_bit_cast(f16x8, pb);
    };

    // One 32-key step whose first key is kstep (relative to the range start): s holds its
    // logits S (issued one step earlier), kfr the K operands of the following step, kf its
    // per-key factors (int8 VALU mode) and Vl this lane's V operand address in the step. On
    // return s holds the following step's logits and O^T has taken V^T P^T.
    //   * With PREFETCH, one straight run issues the following step's logit MFMAs and,
    //     between them, this step's softmax on the VALU (the lane max, the 16 exponentials,
    //     the f16 conversions and the swaps into B operands), so a wavefront's VALU work runs
    //     while its own MFMAs do. The probabilities are formed against the current running max
    //     before it is known whether the step moves it; a step that does (rare once the max
    //     settles, always the first) forms them again after the rescale. Otherwise (fewer
    //     registers) the logit MFMAs are issued first and the softmax follows the rescale test.
    //   * The PV MFMAs follow; the block staging and the K operand reads of the step after
    //     next are issued behind them.
    //   * check = false (uniform over the workgroup) leaves out the lane max and the rescale
    //     test: the optimistic scan of the folded kernels (see the block loop).
    auto step = [&](bool check, f32x16& s, f16x8 (&kfr)[G::KSTEPS], const lds_f16* Kl, const float* kf, const lds_f16* Vl,
                    int kstep, bool first) {
        // V operands: read first where the register budget allows (PREFETCH shapes), so their
        // LDS latency passes under the softmax, else after it
        f16x8 vf[G::VT];
        if constexpr (PREFETCH) read_v(Vl, vf);
        float x[16];
        if constexpr (FOLD) {
#pragma unroll
            for (int r = 0; r < 16; ++r) x[r] = s[r];
        } else {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                f32x4 f;
                if constexpr (KVT == NORI_I8) f = *reinterpret_cast<const f32x4*>(&kf[8 * g + 4 * hh]);
                else f = f32x4{a.scale_log2, a.scale_log2, a.scale_log2, a.scale_log2};
#pragma unroll
                for (int i = 0; i < 4; ++i) x[4 * g + i] = fmaf(s[4 * g + i], f[i], -m_run);
            }
        }
        if (kstep + 32 > klen) {  // the last step of a context range may be partial
#pragma unroll
            for (int g = 0; g < 4; ++g)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (kstep + 8 * g + 4 * hh + i >= klen) x[4 * g + i] = -INFINITY;
        }
        // ---- the straight run: following step's logits on the MFMAs, this step's softmax on
        // the VALU
        // With PREFETCH, logit MFMA ks is followed by its share of the probabilities, each
        // segment fenced off so the wavefront issues them while that MFMA runs (the next MFMA
        // waits for its result). The lane's max over its 16 keys decides whether any query of the
        // wavefront must move its running max (max16f reads logits issued one step earlier, long
        // complete); the folded kernels take it after the straight run, in checked steps only.
        f32x16 s_next = f32x16{};
        float bm = 0.0f, l_step = 0.0f;
        uint32_t pw[8];
        f16x8 p0, p1;
#pragma unroll
        for (int ks = 0; ks < G::KSTEPS; ++ks) {
            // without PREFETCH each K operand is read just before its MFMA (fewer live registers)
            const f16x8 kop = PREFETCH ? kfr[ks] : *reinterpret_cast<const lds_f16x8*>(Kl + 16 * ks);
            s_next = __builtin_amdgcn_mfma_f32_32x32x16_f16(kop, qf[ks], s_next, 0, 0, 0);
            if (ks == 0) {
                if constexpr (PREFETCH) __builtin_amdgcn_sched_barrier(0);
                if constexpr (!FOLD) bm = max16f(x);
            }
            if constexpr (PREFETCH) {
#pragma unroll
                for (int t = 8 * ks / G::KSTEPS; t < 8 * (ks + 1) / G::KSTEPS; ++t) pw[t] = prob_pair(x, t, l_step);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        if constexpr (PREFETCH) b_operands(pw, p0, p1);
        bool moves = false;
        if (check) {
            if constexpr (FOLD) bm = max16f(x);
            moves = first || __any(bm > kRescaleSlack);
        }
        if (moves) {
            {
                // both halves of the swap together hold lanes l and l ^ 32 in every lane
                const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(bm), __float_as_uint(bm), true, false);
                bm = max2f(__uint_as_float(r[0]), __uint_as_float(r[1]));
            }
            // anchor the running max on the first step (its first key is valid for every
            // query); afterwards move it up where a step overshoots it (rare: the max settles
            // within the first few blocks). A folded max is an f16 value (the Q fragment
            // carries it), so the shift is the exact difference of two f16 values.
            float shift = first ? bm : fmaxf(bm, 0.0f);
            if constexpr (FOLD) shift = (float)(_Float16)(m_run + shift) - m_run;
            if (!first) {
                const float alpha = __builtin_amdgcn_exp2f(-shift);
                l_run *= alpha;
                // alpha of query lane%16 (query block 0) and 16 + lane%16 (block 1)
                const auto ab = __builtin_amdgcn_permlane16_swap(__float_as_uint(alpha), __float_as_uint(alpha), false, false);
                const float a0 = __uint_as_float(ab[0]), a1 = __uint_as_float(ab[1]);
#pragma unroll
                for (int t = 0; t < G::VT; ++t) {
                    o[t][0] *= a0;
                    o[t][1] *= a1;
                }
            }
            m_run += shift;
#pragma unroll
            for (int r = 0; r < 16; ++r) x[r] -= shift;
            if constexpr (FOLD) {
                // the following step's logits were issued with the old max
#pragma unroll
                for (int r = 0; r < 16; ++r) s_next[r] -= shift;
#pragma unroll
                for (int ks = 0; ks < G::KSTEPS; ++ks)
#pragma unroll
                    for (int j = 0; j < 8; ++j)
                        if (16 * ks + 8 * hh + j == d) qf[ks][j] = (_Float16)(-m_run);
            }
            if constexpr (PREFETCH) {  // formed against the old max: again
                l_step = 0.0f;
#pragma unroll
                for (int t = 0; t < 8; ++t) pw[t] = prob_pair(x, t, l_step);
                b_operands(pw, p0, p1);
            }
        }
        if constexpr (!PREFETCH) {
#pragma unroll
            for (int t = 0; t < 8; ++t) pw[t] = prob_pair(x, t, l_step);
            b_operands(pw, p0, p1);
        }
        if constexpr (!FOLD) l_run += l_step;
        if constexpr (!PREFETCH) read_v(Vl, vf);
#pragma unroll
        for (int t = 0; t < G::VT; ++t) {
            o[t][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf[t], p0, o[t][0], 0, 0, 0);
            o[t][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf[t], p1, o[t][1], 0, 0, 0);
        }
        s = s_next;
    };

    // Software pipeline over 32-key steps: each step issues the logit MFMAs of the following
    // step, whose K operands were read one step (or, with PREFETCH, two steps) earlier. Blocks
    // are staged into the LDS ring ahead of use from raw words loaded one block before that.
    //   * three buffers: block i+2 is staged while block i is computed (after its first
    //     step) and one barrier closes each block, so the staging overlaps the compute of
    //     the other wavefronts;
    //   * two buffers (wide heads): block i+1 is staged before the second-to-last step of
    //     block i, fenced by a barrier on each side, so the K operands of its first step can
    //     be read during the last step of block i.
    // The folded kernels scan optimistically: every block after the first skips the per-step
    // rescale test and keeps the running max the first block anchored. Probabilities then stay
    // finite in f16 while no logit exceeds that max by 16 (log2 units); one that does turns into
    // inf, and the denominator the PV MFMA sums in its last row becomes inf or NaN (no rescale
    // runs in such a scan, so nothing multiplies it back). Each wavefront tests its denominators
    // after the scan; if any is not finite, the workgroup scans its context range again with the
    // test on every step (pass 1, the lazy-rescale scan). The two scans do the same arithmetic
    // otherwise. (The VALU-mode kernels scan once with the test on: at DP 64 the second pass's
    // live state spills inside their loop and costs more than the test.)
    if constexpr (resident(NW)) {
        // the whole context range (klen <= KB keys, checked on the host) in one staged buffer,
        // then one checked 32-key step after another; rows past klen are staged as zeros and
        // masked out of the partial last step
        {
            Raw<KVT> raw[NU];
            load_block(k_begin, raw);
            store_block(0, raw);
        }
        __syncthreads();
        if constexpr (KVT == NORI_F16) {
            if (a.pkw) {
                // each staged key row's RMS norm with its gain, rounded to f16 (the cache dtype)
                // as the separate pass rounds it: 4 lanes per row, DP / 4 elements each
                constexpr int EPL = DP / 4;
                const int part = tid & 3;
                float wk[EPL / 4][4];  // this lane's gains, the same for every row it normalizes
                gains_of(a.pkw, a.pwdt, d, [&](int e, int i) { return part * EPL + 4 * e + i; }, wk);
                for (int r = tid >> 2; r < klen; r += THREADS / 4) {
                    _Float16* row = Ks + r * G::KPITCH + part * EPL;
                    float v[EPL];
                    float ss = 0.0f;
#pragma unroll
                    for (int e = 0; e < EPL; e += 4) {
                        const f16x4 x = *reinterpret_cast<const f16x4*>(row + e);
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            v[e + i] = part * EPL + e + i < d ? (float)x[i] : 0.0f;
                            ss = fmaf(v[e + i], v[e + i], ss);
                        }
                    }
                    ss = quad_sum(ss);
                    const float inv = rsqrtf(ss / (float)d + a.peps);
#pragma unroll
                    for (int e = 0; e < EPL; e += 4) {
                        if (part * EPL + e < d) {  // d is a multiple of 4
                            f16x4 x;
#pragma unroll
                            for (int i = 0; i < 4; ++i)
                                x[i] = (_Float16)round_to<NORI_F16>(round_to<NORI_F16>(v[e + i] * inv) * wk[e / 4][i]);
                            *reinterpret_cast<f16x4*>(row + e) = x;
                        }
                    }
                }
                __syncthreads();
            }
        }
        const int nsteps = (klen + 31) >> 5;
        const lds_f16* Kr = opaque_lds(KsL + k_lane);
        const lds_f16* Vr = opaque_lds(VsL + v_lane);
        f16x8 kfr[G::KSTEPS];
        read_k(Kr, kfr);
        f32x16 s_cur = logits(kfr);
        read_k(Kr + 32 * min(1, G::SPB - 1) * G::KPITCH, kfr);  // the K operands of step 1
        for (int st = 0; st < nsteps; ++st) {
            // the following step's K rows (a valid buffer row past the last step, unused)
            const int nx = min(st + 1, G::SPB - 1);
            step(true, s_cur, kfr, Kr + 32 * nx * G::KPITCH, kfac + ((FOLD || KVT != NORI_I8) ? 0 : 32 * st),
                 Vr + st * G::VSTEP, 32 * st, st == 0);
            if constexpr (PREFETCH) read_k(Kr + 32 * min(st + 2, G::SPB - 1) * G::KPITCH, kfr);
        }
    } else {
    __shared__ int rescan;
    if (tid == 0) rescan = 0;  // ordered before its readers by the barriers of the scan
    constexpr int PASSES = FOLD ? 2 : 1;
    for (int pass = 0; pass < PASSES; ++pass) {
    const bool checked_scan = !FOLD || pass == 1;
    if (pass == 1) {
#pragma unroll
        for (int t = 0; t < G::VT; ++t) o[t][0] = o[t][1] = f32x4{0.f, 0.f, 0.f, 0.f};
        m_run = 0.0f;
        l_run = 0.0f;
#pragma unroll
        for (int ks = 0; ks < G::KSTEPS; ++ks)
#pragma unroll
            for (int j = 0; j < 8; ++j)
                if (16 * ks + 8 * hh + j == d) qf[ks][j] = (_Float16)0.0f;
    }
    Raw<KVT> raw[NU];
    load_block(k_begin, raw);
    store_block(0, raw);
    constexpr int AHEAD = G::NBUF >= 3 ? 2 : 1;
    static_assert(G::SPB >= 2, "a block spans at least two steps");
    if constexpr (AHEAD == 2) {
        if (nblk > 1) {
            load_block(k_begin + KB, raw);
            store_block(1, raw);
        }
    }
    if (nblk > AHEAD) load_block(k_begin + AHEAD * KB, raw);
    __syncthreads();
    f16x8 kfr[G::KSTEPS];
    read_k(KsL + k_lane, kfr);
    f32x16 s_cur = logits(kfr);
    read_k(KsL + k_lane + 32 * G::KPITCH, kfr);  // the K operands of step 1

    for (int blk = 0; blk < nblk; ++blk) {
        const int64_t kb = k_begin + (int64_t)blk * KB;
        const int cur = blk % G::NBUF, nxt = (blk + 1) % G::NBUF;
        // this lane's operand addresses in the current and next buffers; every step of the
        // block reads at constant offsets from them
        const lds_f16* Kc = opaque_lds(KsL + cur * G::KBUF + k_lane);
        const lds_f16* Kn = opaque_lds(KsL + nxt * G::KBUF + k_lane);
        const lds_f16* Vc = opaque_lds(VsL + cur * G::VBUF + v_lane);
        const float* kf = kfac + ((FOLD || KVT != NORI_I8) ? 0 : cur * KB);
#pragma unroll
        for (int st = 0; st < G::SPB; ++st) {
            if constexpr (AHEAD == 1) {
                if (st == G::SPB - 2) {
                    __syncthreads();  // every wavefront is done with block blk-1, the target buffer
                    if (blk + 1 < nblk) {
                        store_block(nxt, raw);
                        if (blk + 2 < nblk) load_block(kb + 2 * KB, raw);  // lands during the next block
                    }
                    __syncthreads();
                }
            }
            step(checked_scan || blk == 0, s_cur, kfr, st + 1 < G::SPB ? Kc + 32 * (st + 1) * G::KPITCH : Kn,
                 kf + ((FOLD || KVT != NORI_I8) ? 0 : 32 * st), Vc + st * G::VSTEP, blk * KB + 32 * st,
                 blk == 0 && st == 0);
            // K operands of the step after next: this block's rows, or the next block's (a
            // stale buffer after the last block, unused)
            if constexpr (PREFETCH)
                read_k(st + 2 < G::SPB ? Kc + 32 * (st + 2) * G::KPITCH : Kn + 32 * (st + 2 - G::SPB) * G::KPITCH, kfr);
            if constexpr (AHEAD == 2) {
                if (st == 0 && blk + 2 < nblk) {
                    store_block((blk + 2) % G::NBUF, raw);
                    if (blk + 3 < nblk) load_block(kb + 3 * KB, raw);  // lands during the next block
                }
            }
        }
        if constexpr (AHEAD == 2) __syncthreads();
    }
    if (checked_scan) break;
    {
        // the denominators sit in O^T row DP-1: tile VT-1, element 3 of lanes 48-63
        const bool bad = lane >= 48 && !(__builtin_isfinite(o[G::VT - 1][0][3]) && __builtin_isfinite(o[G::VT - 1][1][3]));
        if (__any(bad) && lane == 0) rescan = 1;
    }
    __syncthreads();  // every flag written; every read of the ring done before pass 1 restages it
    if (!rescan) break;
    }
    }  // ring scan

    // ---------------- epilogue: per query, its denominator and running max in the O^T layout
    // (lane holds query 16qb + lane%16)
    float l_q[2], m_q[2];
    if constexpr (FOLD) {
        // the ones column sums P into O^T row DP-1: tile VT-1, element 3 of lanes 48-63
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) l_q[qb] = lane_value(o[G::VT - 1][qb][3], 48 + (lane & 15));
    } else {
        const float l_tot = l_run + other_half(l_run);
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) l_q[qb] = lane_value(l_tot, 16 * qb + (lane & 15));
    }
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) m_q[qb] = lane_value(m_run, 16 * qb + (lane & 15));
    const bool merge = a.flags & NORI_ATTN_MERGE;
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
        const int64_t qo = (int64_t)qt * (NW * QPW) + wave * QPW + 16 * qb + (lane & 15);
        if (qo >= a.nq) continue;
        const float inv = 1.0f / l_q[qb];
        const float lse_part = (m_q[qb] + __log2f(l_q[qb])) * kLn2;
        if (split >= 0) {
            const int64_t prow =
                (split * (a.nunits - a.n_whole) + (unit - a.n_whole)) * a.qrows + (qo - (int64_t)qt * a.qrows);
            float* po = a.part_o + prow * d;
#pragma unroll
            for (int t = 0; t < G::VT; ++t) {
                const int d0 = 16 * t + 4 * (lane >> 4);
                if (d0 < d) *reinterpret_cast<f32x4*>(po + d0) = o[t][qb] * inv;
            }
            if ((lane >> 4) == 0) a.part_lse[prow] = lse_part;
            continue;
        }
        const int64_t obase = b * a.o_bg + qo * a.o_row + (int64_t)h * a.o_head;
        const int64_t lse_idx = (b * a.heads + h) * a.nq + qo;
        float w_old = 0.f, w_new = 1.f, lse_out = lse_part;
        if (merge) merge_weights(a.lse[lse_idx], lse_part, w_old, w_new, lse_out);
        if (a.flags & kOutVec4) {
            // the lane's 4 consecutive head elements in one 8-byte store
            const bool bf = a.out_dtype == NORI_BF16;
#pragma unroll
            for (int t = 0; t < G::VT; ++t) {
                const int d0 = 16 * t + 4 * (lane >> 4);
                if (d0 < d) {
                    uint32_t w[2];
#pragma unroll
                    for (int i = 0; i < 2; ++i) {
                        const float v0 = o[t][qb][2 * i] * inv, v1 = o[t][qb][2 * i + 1] * inv;
                        const uint32_t h0 = bf ? f32_to_bf16(v0) : f32_to_f16(v0);
                        const uint32_t h1 = bf ? f32_to_bf16(v1) : f32_to_f16(v1);
                        w[i] = h0 | (h1 << 16);
                    }
                    *reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(a.out) + obase + d0) = u32x2{w[0], w[1]};
                }
            }
            if (a.lse && (lane >> 4) == 0) a.lse[lse_idx] = lse_out;
            continue;
        }
#pragma unroll
        for (int t = 0; t < G::VT; ++t) {
            const int d0 = 16 * t + 4 * (lane >> 4);
            if (d0 < d) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float v = o[t][qb][i] * inv;
                    if (merge) v = reinterpret_cast<const float*>(a.out)[obase + d0 + i] * w_old + v * w_new;
                    store_from_f32(a.out, a.out_dtype, obase + d0 + i, v);
                }
            }
        }
        if (a.lse && (lane >> 4) == 0) a.lse[lse_idx] = lse_out;
    }
}

// Per-row q/k transforms applied as the short-context kernel loads them (the C ABI's
// nori_qk_prologue): per-head RMS norms with gains, and a multiply of the normed q.
struct Prologue {
    const void* qw = nullptr;  // [d] query norm gain or null
    const void* kw = nullptr;  // [d] key norm gain or null
    int wdt = NORI_F32;
    float eps = 0.f;
    float qmult = 1.f;
};

// The short-context kernel (icl_attention_short.hip): one launch over every (b, h, query) row.
int launch_short(int kv_dtype, const Args& a, const Prologue& pro, hipStream_t stream);

// The few-token MFMA kernel (icl_attention_tile.hip): a wavefront per (b, h, 32-query tile)
// over the unit's whole context; tile_shape() says which calls it takes.
bool tile_shape(int q_dtype, int kv_dtype, int64_t nq, int64_t nk, int d, uint32_t flags);
int launch_tile(Args a, hipStream_t stream);

// Few queries attending to few keys: the VALU kernel, whose cost grows with nq * nk, beats the
// MFMA kernel's fixed cost per (b, h) unit (a 64-query tile over a staged 64-key block).
constexpr bool short_context(int64_t nq, int64_t nk) { return nq <= 64 && nk <= 128 && nq * nk <= 2048; }

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
    if constexpr (has_5_waves(DP)) {
        if (nw == 5) {
            hipLaunchKernelGGL((icl_attention_kernel<DP, KVT, MODE, 5>), grid, dim3(5 * 64), 0, stream, a);
            return NORI_OK;
        }
    }
    if constexpr (has_resident(DP)) {
        if (nw == 10) {
            hipLaunchKernelGGL((icl_attention_kernel<DP, KVT, MODE, 10>), grid, dim3(10 * 64), 0, stream, a);
            return NORI_OK;
        }
    }
    if (nw == 8) hipLaunchKernelGGL((icl_attention_kernel<DP, KVT, MODE, 8>), grid, dim3(8 * 64), 0, stream, a);
    else hipLaunchKernelGGL((icl_attention_kernel<DP, KVT, MODE, 2>), grid, dim3(2 * 64), 0, stream, a);
    return NORI_OK;
}

// Padded head width DP has two kernels: kFold for d < DP and kValu for d = DP.
template <int KVT>
int launch_dtype(int dp, int mode, int nw, const Args& a, hipStream_t stream) {
    const bool fold = mode == kFold;
    switch (dp) {
        case 16: return fold ? launch_shape<KVT, 16, kFold>(nw, a, stream) : launch_shape<KVT, 16, kValu>(nw, a, stream);
        case 32: return fold ? launch_shape<KVT, 32, kFold>(nw, a, stream) : launch_shape<KVT, 32, kValu>(nw, a, stream);
        case 48: return fold ? launch_shape<KVT, 48, kFold>(nw, a, stream) : launch_shape<KVT, 48, kValu>(nw, a, stream);
        case 64: return fold ? launch_shape<KVT, 64, kFold>(nw, a, stream) : launch_shape<KVT, 64, kValu>(nw, a, stream);
        case 80: return fold ? launch_shape<KVT, 80, kFold>(nw, a, stream) : launch_shape<KVT, 80, kValu>(nw, a, stream);
        case 96: return fold ? launch_shape<KVT, 96, kFold>(nw, a, stream) : launch_shape<KVT, 96, kValu>(nw, a, stream);
        case 112: return fold ? launch_shape<KVT, 112, kFold>(nw, a, stream) : launch_shape<KVT, 112, kValu>(nw, a, stream);
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
