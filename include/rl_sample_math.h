/*
 * rl_sample_math.h - arithmetic that must be bit-identical on the host C
 * side and the gfx950 device side of the sampler.
 *
 *  - Philox4x32-10 counter-based RNG (Salmon, Moraes, Dror, Shaw, "Parallel
 *    random numbers: as easy as 1, 2, 3", SC'11): round multipliers
 *    0xD2511F53 / 0xCD9E8D57, Weyl key increments 0x9E3779B9 / 0xBB67AE85.
 *  - rl_expf_cw: e^x by Cody-Waite range reduction (Cody & Waite, "Software
 *    Manual for the Elementary Functions", 1980): x = n ln2 + r with
 *    ln2 split into a 9-bit head and a tail so n*ln2_hi is exact, then the
 *    degree-7 Taylor polynomial of e^r on |r| <= ln2/2 in Horner form with
 *    explicit fused multiply-adds, then scaling by 2^n through the exponent
 *    field. Every step is a correctly rounded IEEE-754 binary32 operation
 *    (fmaf, *, +, floorf, int<->float conversion), so gcc and hipcc produce
 *    the same bits as long as neither contracts or reassociates; this header
 *    switches contraction off for the functions it defines.
 *  - the order-preserving u32 key of a float and the 24-bit sampling weight.
 */
#pragma once

#include <stdint.h>
#include <math.h>

#if defined(__HIPCC__)
#define RL_HD __host__ __device__ __forceinline__
#else
#define RL_HD static inline
#endif

#if defined(__clang__)
#define RL_FP_CONTRACT_OFF _Pragma("clang fp contract(off)")
#else
#define RL_FP_CONTRACT_OFF
#endif

#define RL_PHILOX_M0 0xD2511F53u
#define RL_PHILOX_M1 0xCD9E8D57u
#define RL_PHILOX_W0 0x9E3779B9u
#define RL_PHILOX_W1 0xBB67AE85u

/* out[0..3] = Philox4x32-10(ctr[0..3], key[0..1]) */
RL_HD void
rl_philox4x32_10(const uint32_t ctr_in[4], const uint32_t key_in[2], uint32_t out[4])
{
    uint32_t c0 = ctr_in[0], c1 = ctr_in[1], c2 = ctr_in[2], c3 = ctr_in[3];
    uint32_t k0 = key_in[0], k1 = key_in[1];
    for (int round = 0; round < 10; ++round) {
        const uint64_t p0 = (uint64_t)RL_PHILOX_M0 * (uint64_t)c0;
        const uint64_t p1 = (uint64_t)RL_PHILOX_M1 * (uint64_t)c2;
        const uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
        const uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
        c0 = hi1 ^ c1 ^ k0;
        c1 = lo1;
        c2 = hi0 ^ c3 ^ k1;
        c3 = lo0;
        k0 += RL_PHILOX_W0;
        k1 += RL_PHILOX_W1;
    }
    out[0] = c0;
    out[1] = c1;
    out[2] = c2;
    out[3] = c3;
}

/* The 64-bit uniform draw of one sampling event: key = seed, counter =
 * (step, row). */
RL_HD uint64_t
rl_sample_draw64(uint64_t seed, uint64_t step, uint32_t row)
{
    uint32_t ctr[4], key[2], out[4];
    ctr[0] = (uint32_t)step;
    ctr[1] = (uint32_t)(step >> 32);
    ctr[2] = row;
    ctr[3] = 0u;
    key[0] = (uint32_t)seed;
    key[1] = (uint32_t)(seed >> 32);
    rl_philox4x32_10(ctr, key, out);
    return (uint64_t)out[0] | ((uint64_t)out[1] << 32);
}

/* floor(a * b / 2^64) without 128-bit types (schoolbook on 32-bit limbs). */
RL_HD uint64_t
rl_mulhi_u64(uint64_t a, uint64_t b)
{
    const uint64_t a_lo = (uint32_t)a, a_hi = a >> 32;
    const uint64_t b_lo = (uint32_t)b, b_hi = b >> 32;
    const uint64_t ll = a_lo * b_lo;
    const uint64_t lh = a_lo * b_hi;
    const uint64_t hl = a_hi * b_lo;
    const uint64_t hh = a_hi * b_hi;
    const uint64_t mid = (ll >> 32) + (uint32_t)lh + (uint32_t)hl;
    return hh + (lh >> 32) + (hl >> 32) + (mid >> 32);
}

#define RL_EXP_LOG2E 1.44269504088896341f
#define RL_EXP_LN2_HI 0.693359375f      /* 355/512: 9 significant bits */
#define RL_EXP_LN2_LO -2.12194440e-4f   /* ln2 - 355/512 */

RL_HD float
rl_expf_cw(float x)
{
    RL_FP_CONTRACT_OFF
    if (!(x >= -87.0f))      /* below 2^-125.5, and NaN */
        return 0.0f;
    if (x > 88.0f)
        return INFINITY;
    const float n = floorf(x * RL_EXP_LOG2E + 0.5f);
    float r = fmaf(-n, RL_EXP_LN2_HI, x);
    r = fmaf(-n, RL_EXP_LN2_LO, r);
    float p = 1.0f / 5040.0f;
    p = fmaf(p, r, 1.0f / 720.0f);
    p = fmaf(p, r, 1.0f / 120.0f);
    p = fmaf(p, r, 1.0f / 24.0f);
    p = fmaf(p, r, 1.0f / 6.0f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    const int e = (int)n + 127;   /* n in [-126, 127] here */
    union {
        uint32_t u;
        float f;
    } scale;
    scale.u = (uint32_t)e << 23;
    return p * scale.f;
}

/* Sampling weight of a logit that sits `d` = x - max(x) <= 0 below the row
 * maximum: floor(e^d * 2^24), in [0, 2^24]. */
RL_HD uint32_t
rl_sample_weight(float d)
{
    return (uint32_t)(rl_expf_cw(d) * 16777216.0f);
}

/* rl_sample_weight without branches, for d <= 0 (and NaN): the same
 * operations in the same order on max(d, -87), then 0 selected for
 * !(d >= -87). Equal to rl_sample_weight(d) bit for bit on that domain; the
 * sampler kernels use it in their per-element loops. */
RL_HD uint32_t
rl_sample_weight_nb(float d)
{
    RL_FP_CONTRACT_OFF
    const float x = d >= -87.0f ? d : -87.0f;
    const float n = floorf(x * RL_EXP_LOG2E + 0.5f);
    float r = fmaf(-n, RL_EXP_LN2_HI, x);
    r = fmaf(-n, RL_EXP_LN2_LO, r);
    float p = 1.0f / 5040.0f;
    p = fmaf(p, r, 1.0f / 720.0f);
    p = fmaf(p, r, 1.0f / 120.0f);
    p = fmaf(p, r, 1.0f / 24.0f);
    p = fmaf(p, r, 1.0f / 6.0f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    union {
        uint32_t u;
        float f;
    } scale;
    scale.u = (uint32_t)((int)n + 127) << 23;
    const uint32_t w = (uint32_t)(p * scale.f * 16777216.0f);
    return d >= -87.0f ? w : 0u;
}

/* rl_sample_weight_nb with fewer operations, for d <= 0, -inf and NaN: the
 * same range reduction and polynomial on max(d, -87) (NaN gives -87), then
 * one multiply by 2^(n+24) in place of 2^n and 2^24, and no final select.
 * Equal bit for bit: 2^n p is normal whenever the weight is nonzero, so the
 * two scalings round alike, and d <= -87 weighs 0 either way. *f receives the
 * float before the truncation, e^d 2^24 to about an ulp (about 2^-102 for
 * d <= -87): the terms of the row's log-sum-exp. */
RL_HD uint32_t
rl_sample_weight_f(float d, float *f)
{
    RL_FP_CONTRACT_OFF
    const float x = fmaxf(d, -87.0f);
    const float n = floorf(x * RL_EXP_LOG2E + 0.5f);
    float r = fmaf(-n, RL_EXP_LN2_HI, x);
    r = fmaf(-n, RL_EXP_LN2_LO, r);
    float p = 1.0f / 5040.0f;
    p = fmaf(p, r, 1.0f / 720.0f);
    p = fmaf(p, r, 1.0f / 120.0f);
    p = fmaf(p, r, 1.0f / 24.0f);
    p = fmaf(p, r, 1.0f / 6.0f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    union {
        uint32_t u;
        float f;
    } scale;
    scale.u = (uint32_t)((int)n + 151) << 23; /* n >= -126 here */
    *f = p * scale.f;
    return (uint32_t)*f;
}

/* Order-preserving u32 key of a non-NaN float; -0 and +0 share a key. */
RL_HD uint32_t
rl_float_key(float x)
{
    union {
        float f;
        uint32_t u;
    } v;
    v.f = (x == 0.0f) ? 0.0f : x;
    return (v.u & 0x80000000u) ? ~v.u : (v.u | 0x80000000u);
}

RL_HD float
rl_key_float(uint32_t k)
{
    union {
        float f;
        uint32_t u;
    } v;
    v.u = (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k;
    return v.f;
}

/* ceil(p * W) in double: the nucleus threshold on the integer weights. */
RL_HD uint64_t
rl_topp_threshold(float p, uint64_t w_total)
{
    const double t = ceil((double)p * (double)w_total);
    return (uint64_t)t;
}
