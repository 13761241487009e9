/*
 * Exhaustive CPU check of the quotient recipe the int8 quantize kernel uses
 * (synthefy-nori_amd/csrc/kv_codec.hip, code_of): with y = RN(1/s),
 *     q0 = RN(t*y);  r = fma(-q0, s, t);  q = fma(r, y, q0)
 * must equal the IEEE quotient RN(t/s) -- and so give the same int8 code -- for every
 * element t and scale s of a 16-bit source, whenever 2^-96 <= s <= 2^96 (the kernel's
 * fast-path domain; outside it the residual r can fall into the subnormal range and
 * lose bits, so the kernel divides exactly there).
 *
 * For T in {bf16, fp16} it enumerates every positive finite T value s with normal
 * s and 1/s, and every finite T value t with |t| <= 130*s (the amax element maps to
 * about 127, so no element of a vector exceeds that), both signs, and compares
 *     code = clamp(rint(RN_T(q)), -127, 127)
 * between the two quotients. fp32 sources are checked on random pairs.
 * Prints "<dtype> pairs=<n> code_mismatch=<k> quotient_mismatch=<j>" per dtype, where
 * quotient_mismatch counts pairs with |t/s| >= 1/4 whose two quotients differ in any bit.
 * For fp16 it also checks the plain product: with a normal fp16 scale (s >= 2^-14, the fp16
 * kernels' fast domain) the code of RN(t*y) alone must equal the code of RN(t/s)
 * ("product_mismatch=<m>"), so the fp16 kernels may skip the correction.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

static float bf16_round(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return f;
    u += 0x7fffu + ((u >> 16) & 1u);
    return u2f(u & 0xffff0000u);
}

static float f16_bits_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0x1f) return u2f(sign | 0x7f800000u | (m << 13));
    if (e == 0) { float v = ldexpf((float)m, -24); return sign ? -v : v; }
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

static uint16_t f32_to_f16_bits(float f) {
    uint32_t u = f2u(f);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t a = u & 0x7fffffffu;
    if (a >= 0x7f800000u) return (uint16_t)(sign | (a > 0x7f800000u ? 0x7e00u : 0x7c00u));
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
    if (a < 0x38800000u) return (uint16_t)(sign | (uint16_t)rintf(u2f(a) * 16777216.0f));
    uint32_t h = (((a >> 23) - 112u) << 10) | ((a & 0x7fffffu) >> 13);
    uint32_t rb = a & 0x1fffu;
    if (rb > 0x1000u || (rb == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

static float f16_round(float f) { return f16_bits_to_f32(f32_to_f16_bits(f)); }

static int code_from(float q, int dt) {
    float r = dt == 1 ? f16_round(q) : (dt == 2 ? bf16_round(q) : q);
    float k = rintf(r);
    if (k > 127.f) k = 127.f;
    if (k < -127.f) k = -127.f;
    return (int)k;
}

static long long product_mismatch = 0;

static void check_pair(float t, float s, float y, int dt, long long* pairs, long long* cm, long long* qm) {
    volatile float tv = t, sv = s;
    float exact = tv / sv;
    float q0 = t * y;
    float r = fmaf(-q0, s, t);
    float q = fmaf(r, y, q0);
    (*pairs)++;
    /* Where |t/s| < 1/4 the residual may be subnormal and inexact; the code is 0 either
     * way there, which the code comparison below still checks. For |t/s| >= 1/2 and
     * s >= 2^-96 the residual is a multiple of 2^-143 and exact. */
    if (fabsf(exact) >= 0.25f && f2u(q) != f2u(exact)) (*qm)++;
    if (code_from(q, dt) != code_from(exact, dt)) (*cm)++;
    if (dt == 1 && s >= 0x1p-14f && code_from(q0, dt) != code_from(exact, dt)) product_mismatch++;
}

/* The kernel's fast-path predicate (kv_codec.hip, make_scale). */
static int fast_domain(float s) { return s >= 0x1p-96f && s <= 0x1p96f; }

static void run16(int dt) {
    long long pairs = 0, cm = 0, qm = 0;
    for (uint32_t sb = 1; sb < 0x7f80u; ++sb) {
        float s = dt == 2 ? u2f(sb << 16) : f16_bits_to_f32((uint16_t)sb);
        if (dt == 1 && sb >= 0x7c00u) break;
        if (!isfinite(s) || s <= 0.f) continue;
        volatile float one = 1.0f;
        float y = one / s;
        (void)y;
        if (!fast_domain(s)) continue;
        float lim = 130.0f * s;
        uint32_t tmax = dt == 2 ? 0x7f80u : 0x7c00u;
        for (uint32_t tb = 0; tb < tmax; ++tb) {
            float t = dt == 2 ? u2f(tb << 16) : f16_bits_to_f32((uint16_t)tb);
            if (t > lim) break;
            check_pair(t, s, y, dt, &pairs, &cm, &qm);
            if (t != 0.f) check_pair(-t, s, y, dt, &pairs, &cm, &qm);
        }
    }
    printf("%s pairs=%lld code_mismatch=%lld quotient_mismatch=%lld\n", dt == 2 ? "bf16" : "f16", pairs, cm, qm);
    if (dt == 1) printf("f16 product_mismatch=%lld\n", product_mismatch);
}

static uint64_t rng = 0x9e3779b97f4a7c15ull;
static uint32_t next32(void) {
    rng ^= rng << 13; rng ^= rng >> 7; rng ^= rng << 17;
    return (uint32_t)(rng >> 32);
}

static void run32(long long n) {
    long long pairs = 0, cm = 0, qm = 0;
    for (long long i = 0; i < n; ++i) {
        /* scale: random fp32 inside the fast-path domain */
        uint32_t e = 31 + next32() % 193u; /* 2^-96 .. 2^96 */
        float s = u2f((e << 23) | (next32() & 0x7fffffu));
        volatile float one = 1.0f;
        float y = one / s;
        if (!fast_domain(s)) continue;
        /* element: t = s * u, u uniform in [-128, 128], then perturbed in its last bits */
        float u = ((float)(next32() & 0xffffffu) / 16777216.0f) * 256.0f - 128.0f;
        float t = u2f(f2u(s * u) ^ (next32() & 0xffu));
        if (!isfinite(t)) continue;
        check_pair(t, s, y, 0, &pairs, &cm, &qm);
    }
    printf("f32 pairs=%lld code_mismatch=%lld quotient_mismatch=%lld\n", pairs, cm, qm);
}

int main(int argc, char** argv) {
    long long n32 = argc > 1 ? atoll(argv[1]) : 20000000LL;
    run16(2);
    run16(1);
    run32(n32);
    return 0;
}
