// Host entry points of query-row -> context attention (nori_icl_attention): argument
// checks, the context-split plan, and the kernel that merges split partials. The kernel
// itself is icl_attention_kernel.h.
#include <math.h>

#include <algorithm>
#include <mutex>

#include "icl_attention_kernel.h"

namespace {

using namespace nori;
using namespace nori::attn;

// Merges the nsplit partial (O, LSE) pairs of every tail unit's rows -- and the running
// output when merging -- into the final output. A row's head vector is spread over LPR lanes
// (one 4-element quad each, LPR >= d/4), 256 / LPR rows per workgroup. When merging, every lane
// of a row reads the row's running LSE before the row's first lane overwrites it: the barrier
// between the two keeps a lane from reading the new value (the lanes of a row all sit in one
// workgroup, not always in one wavefront).
template <int LPR>
__global__ void __launch_bounds__(256)
combine_splits_kernel(const Args a) {
    const int dqv = a.d >> 2;
    const int64_t ntail = a.nunits - a.n_whole;
    const int64_t prows = ntail * a.qrows;  // partial rows per context range
    const int dq = (int)(threadIdx.x % LPR);
    const int64_t prow = (int64_t)blockIdx.x * (256 / LPR) + threadIdx.x / LPR;
    const int64_t unit = a.n_whole + prow / a.qrows;
    const int qt = (int)(unit % a.nqt);
    const int h = (int)((unit / a.nqt) % a.heads);
    const int64_t b = unit / a.nqt / a.heads;
    const int64_t qi = (int64_t)qt * a.qrows + prow % a.qrows;
    const bool active = prow < prows && dq < dqv && qi < a.nq;
    const bool merge = a.flags & NORI_ATTN_MERGE;
    const int64_t row = (b * a.heads + h) * a.nq + qi;
    float lse_part = -INFINITY;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    float w_old = 0.f, w_new = 1.f, lse_out = 0.f;
    if (active) {
        float mx = -INFINITY;
        for (int s = 0; s < a.nsplit; ++s) mx = fmaxf(mx, a.part_lse[s * prows + prow]);
        float sum = 0.f;
        for (int s = 0; s < a.nsplit; ++s) sum += expf(a.part_lse[s * prows + prow] - mx);
        lse_part = mx + logf(sum);
        for (int s = 0; s < a.nsplit; ++s) {
            const float w = expf(a.part_lse[s * prows + prow] - lse_part);
            const f32x4 v = *reinterpret_cast<const f32x4*>(a.part_o + (s * prows + prow) * a.d + 4 * dq);
            acc += w * v;
        }
        lse_out = lse_part;
        if (merge) merge_weights(a.lse[row], lse_part, w_old, w_new, lse_out);
    }
    if (merge) __syncthreads();  // every lane has read its row's running LSE
    if (!active) return;
    const int64_t obase = b * a.o_bg + qi * a.o_row + (int64_t)h * a.o_head + 4 * dq;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float v = acc[i];
        if (merge) v = reinterpret_cast<const float*>(a.out)[obase + i] * w_old + v * w_new;
        store_from_f32(a.out, a.out_dtype, obase + i, v);
    }
    if (a.lse && dq == 0) a.lse[row] = lse_out;
}

struct Plan {
    bool short_ctx;  // the VALU kernel for few queries over few keys (no tiles, no split)
    int dp;          // head width padded to the logit MFMA granule (16)
    int mode;        // how logits and the denominator are formed (attn::Mode)
    int nw;          // wavefronts per workgroup (32 query rows each)
    int nqt;         // query tiles per (b, h)
    int64_t nunits;  // (b, h, query tile) work units
    int64_t n_whole; // units that scan the whole context in one workgroup
    int nsplit;      // context ranges per tail unit (1: no split)
    int64_t kps;     // keys per context range (a multiple of the block)
};

// Chooses the tile shape and the schedule. Units fill the resident workgroup slots of the
// device round after round; only the units of the last, partly filled round (the tail) are
// split, into context ranges that spread them over the slots the full rounds leave idle, and a
// second kernel merges their partials. A split is taken when the rounds it saves outweigh
// the partials' HBM traffic.
Plan make_plan(int64_t bg, int64_t nq, int heads, int d, int64_t nk, int q_dtype) {
    Plan p;
    p.short_ctx = short_context(nq, nk);
    p.dp = (d + 15) / 16 * 16;
    p.mode = mode_for(d);
    p.nw = (nq > 256 && has_16_waves(p.dp, p.mode)) ? 16 : (nq > 96 ? 8 : 2);
    auto padded = [&](int nw) { return (nq + nw * QPW - 1) / (nw * QPW) * nw * QPW; };
    // a 160-row tile where it covers the queries with fewer padded rows (320 queries: two
    // exact tiles instead of two 256-row ones)
    if (p.nw != 2 && has_5_waves(p.dp)) {
        if (padded(5) * 5 < padded(p.nw) * 4) p.nw = 5;
    }
    // resident-context workgroups for fp16 queries and contexts of up to 256 keys read by more
    // than 160 queries per (b, h), where their 320-row tiles pad the queries no more than the
    // ring's tiles and there are at least two units per CU: each unit stages its whole context
    // once (320 x 256 keys, 2048 (b, h) units, d 64: 308 -> 274 us)
    if (!p.short_ctx && q_dtype == NORI_F16 && nk <= kResidentKeys && nq > 5 * QPW && has_resident(p.dp) &&
        padded(10) <= padded(p.nw)) {
        const int nqt = (int)((nq + 10 * QPW - 1) / (10 * QPW));
        if (bg * heads * (int64_t)nqt >= 2 * (int64_t)device_cus()) {
            p.nw = 10;
            p.nqt = nqt;
            p.nunits = bg * heads * (int64_t)nqt;
            p.n_whole = p.nunits;
            p.nsplit = 1;
            p.kps = kResidentKeys;
            return p;
        }
    }
    p.nqt = (int)((nq + p.nw * QPW - 1) / (p.nw * QPW));
    p.nunits = bg * heads * (int64_t)p.nqt;
    const int KB = block_keys(p.nw);
    const int64_t nkb = (nk + KB - 1) / KB;
    const int64_t slots = (int64_t)device_cus() * std::max(1, resident_workgroups(p.dp, p.mode, p.nw));
    const int64_t full = p.nunits / slots, tail = p.nunits % slots;
    // seconds per block of one workgroup at ~40 % of the dense MFMA peak shared by all slots
    const double t_blk = (double)p.nw * QPW * KB * p.dp * 4.0 / (1.0e15 / (double)slots);
    // write + read of one context range's partials of the tail units
    const double t_partial = (double)tail * p.nw * QPW * (d + 1) * 8.0 / 5.0e12;
    p.n_whole = p.nunits;
    p.nsplit = 1;
    p.kps = nkb * KB;
    if (tail == 0 || p.short_ctx) return p;
    double best = (double)(full + 1) * nkb * t_blk;
    const int64_t max_split = std::max<int64_t>(1, std::min<int64_t>(64, nkb / 4));
    for (int64_t ns = 2; ns <= max_split; ++ns) {
        const int64_t blocks = (nkb + ns - 1) / ns;
        const int64_t ns_eff = (nkb + blocks - 1) / blocks;
        const int64_t tail_rounds = (tail * ns_eff + slots - 1) / slots;
        const double cost = (double)(full * nkb + tail_rounds * blocks) * t_blk + ns_eff * t_partial + 5e-6;
        if (cost < best * 0.995) {
            best = cost;
            p.n_whole = full * slots;
            p.nsplit = (int)ns_eff;
            p.kps = blocks * KB;
        }
    }
    return p;
}

// Whether a launch of this shape runs the q/k prologue: the short-context kernel always, a
// resident-context launch when the key norm (if any) applies to an f16 cache.
bool takes_prologue(int64_t bg, int64_t nq, int heads, int d, int64_t nk, int kv_dtype, const void* k_weight,
                    int q_dtype) {
    if (short_context(nq, nk)) return true;
    return make_plan(bg, nq, heads, d, nk, q_dtype).nw == 10 && (!k_weight || kv_dtype == NORI_F16);
}

int64_t workspace_bytes(const Plan& p, int d) {
    if (p.nsplit <= 1) return 0;
    return (int64_t)p.nsplit * (p.nunits - p.n_whole) * p.nw * QPW * (d + 1) * (int64_t)sizeof(float);
}

}  // namespace

extern "C" int32_t nori_icl_attention_takes_prologue(int64_t bg, int64_t nq, int32_t heads, int32_t d, int64_t nk,
                                                     int32_t kv_dtype, int32_t with_key_norm, int32_t q_dtype) {
    if (bg <= 0 || nq <= 0 || heads <= 0 || d < 4 || d > 128 || d % 4 || nk <= 0) return 0;
    static const char one = 0;
    return takes_prologue(bg, nq, heads, d, nk, kv_dtype, with_key_norm ? &one : nullptr, q_dtype) ? 1 : 0;
}

extern "C" int64_t nori_icl_attention_workspace_size(int64_t bg, int64_t nq, int32_t heads, int32_t d, int64_t nk) {
    if (bg <= 0 || nq <= 0 || heads <= 0 || d < 4 || d > 128 || d % 4 || nk <= 0) return 0;
    // the ring kernels' plan: resident-context launches (fp16 queries) never split, so this
    // bounds the workspace whatever the query dtype
    return workspace_bytes(make_plan(bg, nq, heads, d, nk, NORI_F32), d);
}

namespace {

// Both entry points: checks, plan, launch. `pro` (may be null) is the q/k prologue, which
// only the short-context kernel applies.
int run_attention(const void* q, int q_dtype, int64_t bg, int64_t nq, int32_t heads, int32_t d,
                  int64_t q_bg_stride, int64_t q_row_stride, int64_t q_head_stride, const void* kv, int kv_dtype,
                  const float* kv_scales, int64_t nk, int32_t kv_heads, int64_t kv_bg_stride, int64_t kv_row_stride,
                  int64_t kv_half_stride, int64_t sc_bg_stride, int64_t sc_row_stride, int64_t sc_half_stride,
                  float scale, void* out, int out_dtype, int64_t out_bg_stride, int64_t out_row_stride,
                  int64_t out_head_stride, float* lse, uint32_t flags, void* workspace,
                  int64_t workspace_bytes_given, const nori_qk_prologue* pro, void* stream_v) {
    clear_error();
    Prologue prologue;
    if (pro) {
        if ((pro->q_weight || pro->k_weight) && pro->weight_dtype != NORI_F32 && pro->weight_dtype != NORI_F16 &&
            pro->weight_dtype != NORI_BF16)
            return fail(NORI_ERR_UNSUPPORTED, "icl_attention: unsupported norm gain dtype %s",
                        dtype_name(pro->weight_dtype));
        if (pro->k_weight && kv_dtype == NORI_I8)
            return fail(NORI_ERR_UNSUPPORTED, "icl_attention: a key norm applies to full-precision caches only");
        if (!(pro->eps >= 0.f) || !(pro->q_mult == pro->q_mult))
            return fail(NORI_ERR_INVALID, "icl_attention: prologue eps must be >= 0 and q_mult a number");
        prologue.qw = pro->q_weight;
        prologue.kw = pro->k_weight;
        prologue.wdt = pro->weight_dtype;
        prologue.eps = pro->eps;
        prologue.qmult = pro->q_mult;
        if (bg > 0 && nq > 0 && heads > 0 && d >= 4 && nk > 0 &&
            !takes_prologue(bg, nq, heads, d, nk, kv_dtype, pro->k_weight, q_dtype))
            return fail(NORI_ERR_UNSUPPORTED,
                        "icl_attention: the q/k prologue runs only on the short-context kernel (few queries over few "
                        "keys) and on resident-context launches (%lld x %lld here)",
                        (long long)nq, (long long)nk);
    }
    if (bg < 0 || nq < 0)
        return fail(NORI_ERR_INVALID, "icl_attention: negative batch (%lld) or query count (%lld)", (long long)bg, (long long)nq);
    if (heads <= 0 || kv_heads <= 0 || heads % kv_heads)
        return fail(NORI_ERR_INVALID, "icl_attention: query heads %d cannot attend to %d K/V heads", heads, kv_heads);
    if (d < 4 || d > 128 || d % 4)
        return fail(NORI_ERR_UNSUPPORTED, "icl_attention: head width %d is not a multiple of 4 in [4, 128]", d);
    if (nk <= 0) return fail(NORI_ERR_INVALID, "icl_attention: empty K/V cache");
    if (nk > 2147483647LL - 1024)
        return fail(NORI_ERR_UNSUPPORTED, "icl_attention: %lld context rows exceed the 2^31 - 1024 rows of one launch",
                    (long long)nk);
    if (q_dtype != NORI_F32 && q_dtype != NORI_F16 && q_dtype != NORI_BF16)
        return fail(NORI_ERR_UNSUPPORTED, "icl_attention: unsupported query dtype %s", dtype_name(q_dtype));
    if (out_dtype != NORI_F32 && out_dtype != NORI_F16 && out_dtype != NORI_BF16)
        return fail(NORI_ERR_UNSUPPORTED, "icl_attention: unsupported output dtype %s", dtype_name(out_dtype));
    if (kv_dtype != NORI_I8 && kv_dtype != NORI_F16 && kv_dtype != NORI_BF16 && kv_dtype != NORI_F32)
        return fail(NORI_ERR_UNSUPPORTED, "icl_attention: unsupported cache dtype %s", dtype_name(kv_dtype));
    if (flags & ~NORI_ATTN_MERGE) return fail(NORI_ERR_INVALID, "icl_attention: unknown flags 0x%x", flags);
    if ((flags & NORI_ATTN_MERGE) && (out_dtype != NORI_F32 || !lse))
        return fail(NORI_ERR_INVALID, "icl_attention: merging needs an fp32 running output and an LSE buffer");
    if (kv_dtype == NORI_I8 && !kv_scales) return fail(NORI_ERR_INVALID, "icl_attention: int8 cache without scales");
    if (bg == 0 || nq == 0) return NORI_OK;
    if (!q || !kv || !out) return fail(NORI_ERR_INVALID, "icl_attention: null pointer");
    // cache rows are read 4 elements at a time, through 32-bit offsets within a block of up
    // to 128 rows, and a row must hold its K then V heads (the [.., N, 2, Hkv, D] cache layout)
    const int es = dtype_size(kv_dtype);
    if (((uintptr_t)kv) % (4 * es) || kv_row_stride % 4 || kv_bg_stride % 4 || kv_half_stride % 4)
        return fail(NORI_ERR_UNSUPPORTED, "icl_attention: cache rows must start on 4-element boundaries");
    if (kv_half_stride < (int64_t)kv_heads * d || kv_row_stride < kv_half_stride + (int64_t)kv_heads * d ||
        (double)kResidentKeys * kv_row_stride * es >= 2147483647.0)
        return fail(NORI_ERR_UNSUPPORTED,
                    "icl_attention: cache rows must be [K heads | V heads] within one row stride of < 8 MiB");
    if (kv_dtype == NORI_I8 && (sc_half_stride < kv_heads || sc_row_stride < sc_half_stride + kv_heads))
        return fail(NORI_ERR_UNSUPPORTED, "icl_attention: scale rows must be [K heads | V heads] within one row stride");

    const Plan plan = make_plan(bg, nq, heads, d, nk, q_dtype);
    Args args;
    args.q = q; args.q_dtype = q_dtype; args.nq = nq; args.heads = heads; args.d = d;
    args.q_bg = q_bg_stride; args.q_row = q_row_stride; args.q_head = q_head_stride;
    args.kv = kv; args.kvs = kv_scales; args.nk = nk; args.hgroup = heads / kv_heads;
    args.kv_bg = kv_bg_stride; args.kv_row = kv_row_stride; args.kv_half = kv_half_stride;
    args.sc_bg = sc_bg_stride; args.sc_row = sc_row_stride; args.sc_half = sc_half_stride;
    args.scale_log2 = scale * kLog2e;
    args.out = out; args.out_dtype = out_dtype; args.o_bg = out_bg_stride; args.o_row = out_row_stride;
    args.o_head = out_head_stride; args.lse = lse; args.flags = flags;
    args.bg = bg;
    if (pro && plan.nw == 10 && !plan.short_ctx) {
        args.pqw = prologue.qw;
        args.pkw = prologue.kw;
        args.pwdt = prologue.wdt;
        args.peps = prologue.eps;
        args.pqmult = prologue.qmult;
    }
    args.nqt = plan.nqt;
    args.qrows = plan.nw * QPW;
    args.nunits = plan.nunits;
    args.n_whole = plan.n_whole;
    args.nsplit = plan.nsplit;
    args.keys_per_split = plan.kps;
    const int64_t need = workspace_bytes(plan, d);
    if (need > 0 && (!workspace || workspace_bytes_given < need)) {
        // no (or too little) scratch: every unit scans the whole context
        args.n_whole = plan.nunits;
        args.nsplit = 1;
    }
    args.grid = args.n_whole + (args.nunits - args.n_whole) * args.nsplit;
    const int64_t prows = (args.nunits - args.n_whole) * args.qrows;
    args.part_o = args.nsplit > 1 ? reinterpret_cast<float*>(workspace) : nullptr;
    args.part_lse = args.nsplit > 1 ? reinterpret_cast<float*>(workspace) + (int64_t)args.nsplit * prows * d : nullptr;
    if (args.grid * plan.nw * 64 > 0xffffffffLL) return fail(NORI_ERR_UNSUPPORTED, "icl_attention: grid too large");

    hipStream_t stream = (hipStream_t)stream_v;
    // few-token MFMA kernel from 8 queries up (8 x 10 tokens, 2 heads of 64: 0.69 against 0.84 ms
    // on the short-context kernel, which stays ahead at 4 queries and fewer: 0.36 against 0.68).
    // It reads queries 4 elements (8 bytes) at a time, so their rows and heads must start on
    // 4-element boundaries; other query views take the kernels below, which read them one
    // element at a time.
    const bool q_vec4 = (uintptr_t)q % 8 == 0 && q_bg_stride % 4 == 0 && q_row_stride % 4 == 0 && q_head_stride % 4 == 0;
    const bool q16 = q_dtype == NORI_F16 || q_dtype == NORI_BF16;
    if (q16 && q_vec4) args.flags |= kQVec4;
    if (q16 && d % 8 == 0 && (uintptr_t)q % 16 == 0 && q_bg_stride % 8 == 0 && q_row_stride % 8 == 0 &&
        q_head_stride % 8 == 0)
        args.flags |= kQVec8;
    if ((out_dtype == NORI_F16 || out_dtype == NORI_BF16) && !(flags & NORI_ATTN_MERGE) && (uintptr_t)out % 8 == 0 &&
        out_bg_stride % 4 == 0 && out_row_stride % 4 == 0 && out_head_stride % 4 == 0)
        args.flags |= kOutVec4;
    if (tile_shape(q_dtype, kv_dtype, nq, nk, d, flags) && q_vec4 && !pro && (!plan.short_ctx || nq >= 8)) {
        const int st = launch_tile(args, stream);
        return st != NORI_OK ? st : launch_status("icl_attention tile");
    }
    if (plan.short_ctx) {
        const int st = launch_short(kv_dtype, args, prologue, stream);
        return st != NORI_OK ? st : launch_status("icl_attention short");
    }
    int st = launch_kvt(kv_dtype, plan.dp, plan.mode, plan.nw, args, stream);
    if (st != NORI_OK) return st;
    if ((st = launch_status("icl_attention")) != NORI_OK) return st;
    if (args.nsplit > 1) {
        if (d <= 64)
            hipLaunchKernelGGL(combine_splits_kernel<16>, dim3((unsigned)((prows + 15) / 16)), dim3(256), 0, stream, args);
        else
            hipLaunchKernelGGL(combine_splits_kernel<32>, dim3((unsigned)((prows + 7) / 8)), dim3(256), 0, stream, args);
        return launch_status("icl_attention combine");
    }
    return NORI_OK;
}

}  // namespace

extern "C" int nori_icl_attention(const void* q, int q_dtype, int64_t bg, int64_t nq, int32_t heads, int32_t d,
                                  int64_t q_bg_stride, int64_t q_row_stride, int64_t q_head_stride, const void* kv,
                                  int kv_dtype, const float* kv_scales, int64_t nk, int32_t kv_heads,
                                  int64_t kv_bg_stride, int64_t kv_row_stride, int64_t kv_half_stride,
                                  int64_t sc_bg_stride, int64_t sc_row_stride, int64_t sc_half_stride, float scale,
                                  void* out, int out_dtype, int64_t out_bg_stride, int64_t out_row_stride,
                                  int64_t out_head_stride, float* lse, uint32_t flags, void* workspace,
                                  int64_t workspace_bytes_given, void* stream_v) {
    return run_attention(q, q_dtype, bg, nq, heads, d, q_bg_stride, q_row_stride, q_head_stride, kv, kv_dtype,
                         kv_scales, nk, kv_heads, kv_bg_stride, kv_row_stride, kv_half_stride, sc_bg_stride,
                         sc_row_stride, sc_half_stride, scale, out, out_dtype, out_bg_stride, out_row_stride,
                         out_head_stride, lse, flags, workspace, workspace_bytes_given, nullptr, stream_v);
}

extern "C" int nori_icl_attention_qk(const void* q, int q_dtype, int64_t bg, int64_t nq, int32_t heads, int32_t d,
                                     int64_t q_bg_stride, int64_t q_row_stride, int64_t q_head_stride, const void* kv,
                                     int kv_dtype, const float* kv_scales, int64_t nk, int32_t kv_heads,
                                     int64_t kv_bg_stride, int64_t kv_row_stride, int64_t kv_half_stride,
                                     int64_t sc_bg_stride, int64_t sc_row_stride, int64_t sc_half_stride, float scale,
                                     void* out, int out_dtype, int64_t out_bg_stride, int64_t out_row_stride,
                                     int64_t out_head_stride, float* lse, uint32_t flags, void* workspace,
                                     int64_t workspace_bytes_given, const nori_qk_prologue* prologue, void* stream_v) {
    if (!prologue) {
        clear_error();
        return fail(NORI_ERR_INVALID, "icl_attention_qk: null prologue");
    }
    return run_attention(q, q_dtype, bg, nq, heads, d, q_bg_stride, q_row_stride, q_head_stride, kv, kv_dtype,
                         kv_scales, nk, kv_heads, kv_bg_stride, kv_row_stride, kv_half_stride, sc_bg_stride,
                         sc_row_stride, sc_half_stride, scale, out, out_dtype, out_bg_stride, out_row_stride,
                         out_head_stride, lse, flags, workspace, workspace_bytes_given, prologue, stream_v);
}

namespace {

// Scratch of nori_icl_attention_noalloc: the split-context partials (O and LSE of the tail
// units' context ranges) live in this array instead of a caller's workspace. Every device the
// library runs on holds its own copy, from module load until the process ends. Nothing in it
// has to start at zero: every partial the merge kernel reads is written by the attention
// kernel of the same call first.
static __device__ __align__(256) unsigned char scratch[NORI_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex scratch_mu;
void* scratch_addr[kMaxDevices] = {};  // device address of `scratch` per device

// The address of the current device's copy of `scratch`, looked up once per device with that
// device current. The host-side name `scratch` is only a handle for the lookup: kernels and
// copies take the returned address.
int device_scratch(void** addr) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
        return fail(NORI_ERR_RUNTIME, "icl_attention_noalloc: no current HIP device");
    std::lock_guard<std::mutex> lock(scratch_mu);
    if (!scratch_addr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return fail(NORI_ERR_RUNTIME, "icl_attention_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s",
                        dev, hipGetErrorString(e));
        scratch_addr[dev] = p;
    }
    *addr = scratch_addr[dev];
    return NORI_OK;
}

}  // namespace

extern "C" int nori_icl_attention_noalloc(const void* q, int q_dtype, int64_t bg, int64_t nq, int32_t heads,
                                          int32_t d, int64_t q_bg_stride, int64_t q_row_stride,
                                          int64_t q_head_stride, const void* kv, int kv_dtype,
                                          const float* kv_scales, int64_t nk, int32_t kv_heads,
                                          int64_t kv_bg_stride, int64_t kv_row_stride, int64_t kv_half_stride,
                                          int64_t sc_bg_stride, int64_t sc_row_stride, int64_t sc_half_stride,
                                          float scale, void* out, int out_dtype, int64_t out_bg_stride,
                                          int64_t out_row_stride, int64_t out_head_stride, float* lse,
                                          uint32_t flags, void* stream_v) {
    clear_error();
    // the size check comes first and touches no device state
    const int64_t need = nori_icl_attention_workspace_size(bg, nq, heads, d, nk);
    if (need > NORI_NOALLOC_SCRATCH_BYTES)
        return fail(NORI_ERR_UNSUPPORTED,
                    "icl_attention_noalloc: these sizes need %lld bytes of split-context scratch, more than the "
                    "%lld bytes the library holds per device; call nori_icl_attention with a workspace",
                    (long long)need, (long long)NORI_NOALLOC_SCRATCH_BYTES);
    void* ws = nullptr;
    const int st = device_scratch(&ws);
    if (st != NORI_OK) return st;
    return run_attention(q, q_dtype, bg, nq, heads, d, q_bg_stride, q_row_stride, q_head_stride, kv, kv_dtype,
                         kv_scales, nk, kv_heads, kv_bg_stride, kv_row_stride, kv_half_stride, sc_bg_stride,
                         sc_row_stride, sc_half_stride, scale, out, out_dtype, out_bg_stride, out_row_stride,
                         out_head_stride, lse, flags, ws, NORI_NOALLOC_SCRATCH_BYTES, nullptr, stream_v);
}
