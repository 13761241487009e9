// Exact per-op rounding of the int8 cache quantizer, shared by the codec kernels
// (kv_codec.hip) and the fused projection + quantize kernel (kv_project.hip).
//
// quantize_int8 (src/synthefy_nori/model/kv_cache_scaling.py:29-37) as torch evaluates it:
// every op computed in fp32 and its result rounded to the cache dtype T:
//   m = amax|t|, m = max(m, T(1e-12)), s = T(m / 127), c = clamp(rint(T(t / s)), -127, 127).
// The per-element quotient uses one IEEE reciprocal per vector and Markstein's correction
// q = fma(fma(-q0, s, t), y, q0), q0 = t*y, y = RN(1/s): for 2^-96 <= s <= 2^96 it returns the
// correctly rounded quotient wherever |t/s| >= 1/4 (below that the code is 0 whichever
// quotient is used); checked for every fp16 and bf16 (t, s) pair and for random fp32 pairs on
// the CPU by tests/exact_quotient_check.c. Other vectors divide exactly.
//
// A translation unit including this header must keep fp contraction off (the quotient's
// fmas are written out; no other multiply-add may be fused).
#pragma once

#include "nori_common.h"

namespace nori {
namespace quant {

template <int DT> struct Storage;
template <> struct Storage<NORI_F32> { using T = uint32_t; };
template <> struct Storage<NORI_F16> { using T = uint16_t; };
template <> struct Storage<NORI_BF16> { using T = uint16_t; };

template <int DT>
__device__ __forceinline__ float bits_to_f32(typename Storage<DT>::T b) {
    if constexpr (DT == NORI_F32) return __uint_as_float(b);
    else if constexpr (DT == NORI_F16) return f16_to_f32(b);
    else return bf16_to_f32(b);
}

// |x| as an unsigned key whose integer order is the float order with NaN on top, so an
// integer max is a NaN-propagating absmax (torch's amax propagates NaN).
template <int DT>
__device__ __forceinline__ uint32_t abs_key(typename Storage<DT>::T b) {
    if constexpr (DT == NORI_F32) return b & 0x7fffffffu;
    else return (uint32_t)b & 0x7fffu;
}

// For an fp16 source with a normal scale the code of the plain product RN(t * y) already equals
// the code of RN(t/s) for every element a vector can hold (an exhaustive check over the
// (s, t) pairs: tests/exact_quotient_check.c), so the fp16 kernels skip Markstein's correction.
// Scales the fast quotient and packing take. Outside [2^-96, 2^96] the residual fma(-q0, s, t)
// may be subnormal and inexact. An f16 scale must also be normal (>= 2^-14): a subnormal one is
// rounded with a relative error up to 1/2, so |t/s| can pass 127 (absmax 190 * 2^-24 gives
// s = 2^-24 and quotients up to 190), and only the exact path clamps.
template <int DT>
__device__ __forceinline__ bool fast_scale(float s) {
    return s >= (DT == NORI_F16 ? 0x1p-14f : 0x1p-96f) && s <= 0x1p96f;
}

struct VectorScale {
    float s;     // scale in T, widened to fp32
    float y;     // RN(1/s)
    bool fast;   // Markstein quotient valid for this vector
};

template <int DT>
__device__ __forceinline__ VectorScale make_scale(uint32_t max_key, int scale_div) {
    const float m = bits_to_f32<DT>((typename Storage<DT>::T)max_key);
    const float floor_t = round_to<DT>((float)1e-12);  // clamp_min(1e-12) in T
    const float m2 = (m != m) ? m : fmaxf(m, floor_t);
    float s;
    if (scale_div == NORI_SCALE_DIV_RECIP) s = round_to<DT>(m2 * (1.0f / 127.0f));
    else s = round_to<DT>(m2 / 127.0f);
    VectorScale vs;
    vs.s = s;
    vs.y = 1.0f / s;
    vs.fast = fast_scale<DT>(s);
    return vs;
}

// The scale of an f16 vector from its absmax key, without a division: f16(m * RN(1/127)) equals
// f16(m / 127) for every f16 m (an exhaustive check over the f16 values: the exact quotient m/127
// is never within the products' rounding error of an f16 rounding boundary), so both scale_div
// modes give it; y = RN(1/s) from the hardware reciprocal and one Newton step (equal to the
// correctly rounded reciprocal for every positive f16 s: nori_quant_f16_scale_probe).
__device__ __forceinline__ VectorScale make_scale_f16_fast(uint32_t max_key) {
    const float m = bits_to_f32<NORI_F16>((uint16_t)max_key);
    VectorScale vs;
    vs.s = round_to<NORI_F16>(m * (1.0f / 127.0f));
    const float y0 = __builtin_amdgcn_rcpf(vs.s);
    vs.y = fmaf(fmaf(-vs.s, y0, 1.0f), y0, y0);
    vs.fast = fast_scale<NORI_F16>(vs.s);
    return vs;
}

// Code of one element of a vector whose scale has vs.fast (then `t` is finite: |t| <= amax < inf).
template <int DT>
__device__ __forceinline__ int code_fast(float t, const VectorScale& vs) {
    const float q0 = t * vs.y;
    const float r = fmaf(-q0, vs.s, t);
    const float q = fmaf(r, vs.y, q0);
    const float k = rintf(round_to<DT>(q));
    return (int)__builtin_amdgcn_fmed3f(k, -127.0f, 127.0f);
}

// Code of one element.
template <int DT>
__device__ __forceinline__ int code_of(float t, const VectorScale& vs) {
    if (vs.fast) return code_fast<DT>(t, vs);
    const float k = rintf(round_to<DT>(t / vs.s));
    if (k != k) return 0;  // NaN -> 0, the GPU's float->int conversion of NaN
    return (int)fminf(fmaxf(k, -127.0f), 127.0f);
}

// Codes of four correctly rounded quotients q = t/s of a fast-domain vector, packed into one
// word (element 0 in the low byte): rint(RN_T(q)) without a float -> int conversion. For fp16,
// adding 1536 in fp16 rounds to an integer (the spacing in [1024, 2048) is 1, ties to even)
// and leaves the code in the low byte of the result; |t| <= amax bounds |q| by 127 * (1 + 2^-11)
// for fp16 (normal scales: fast_scale) and fp32 sources, so only bf16 (scale rounded to 8 bits)
// needs a clamp.
template <int DT>
__device__ __forceinline__ uint32_t pack_codes_fast(const float (&q)[4]) {
    if constexpr (DT == NORI_F16) {
        const f16x2 magic = {(_Float16)1536.0f, (_Float16)1536.0f};
        const f16x2 h01 = f16x2{(_Float16)pin_f32(q[0]), (_Float16)pin_f32(q[1])} + magic;
        const f16x2 h23 = f16x2{(_Float16)pin_f32(q[2]), (_Float16)pin_f32(q[3])} + magic;
        return __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, h23), __builtin_bit_cast(uint32_t, h01), 0x06040200u);
    } else {
        // bf16 rounding of q can reach 127.5 (its spacing there is 0.5), which rounds to 128:
        // clamp in the shifted domain, where every value is an exact integer
        constexpr float kMagic = 12582912.0f;
        uint32_t k[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float v = round_to<DT>(q[i]) + kMagic;
            if constexpr (DT == NORI_BF16) v = __builtin_amdgcn_fmed3f(v, kMagic - 127.0f, kMagic + 127.0f);
            k[i] = __float_as_uint(v);
        }
        return (k[0] & 0xffu) | ((k[1] & 0xffu) << 8) | ((k[2] & 0xffu) << 16) | (k[3] << 24);
    }
}

__device__ __forceinline__ uint32_t pack4(int a, int b, int c, int d) {
    return (uint32_t)(a & 0xff) | ((uint32_t)(b & 0xff) << 8) | ((uint32_t)(c & 0xff) << 16) |
           ((uint32_t)(d & 0xff) << 24);
}

}  // namespace quant
}  // namespace nori
