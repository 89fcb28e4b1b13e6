/* hmoe_rng.h - counter-based synthetic data generator shared by the host (C oracle, packers) and the device (HIP
 * generators), so that the seeded weights and inputs of the MoE layer are bit-identical wherever they are made.
 *
 * Every value is a pure function of (key, index). Keys are derived from (seed, layer, kind, expert) with splitmix64
 * finalisers (Steele, Lea, Flood, "Fast splittable pseudorandom number generators", OOPSLA 2014). Normal deviates use
 * the Box-Muller transform with a natural log and a cosine written here from their series (atanh series for log,
 * Taylor series for sin/cos after an exact quadrant reduction), evaluated with explicit fmaf and correctly rounded
 * division and square root only, so host and device produce the same float bits. Compile users with
 * -ffp-contract=off (gcc) / -ffp-contract=off -fhip-fp32-correctly-rounded-divide-sqrt (hipcc).
 *
 * Conversions to bf16 and f16 round to nearest even.
 */
#ifndef HMOE_RNG_H
#define HMOE_RNG_H

#include <stdint.h>

#if defined(__HIPCC__)
#define HMOE_HD static inline __host__ __device__
#else
#define HMOE_HD static inline
#endif

/* tensor kinds of the synthetic layer (the key's `kind` field) */
enum {
    HMOE_KIND_X = 0,        /* MoE input rows, N(0, 1) -> bf16 */
    HMOE_KIND_ROUTER = 1,   /* router weight W_g [E][H], N(0, 0.02) fp32 */
    HMOE_KIND_BIAS = 2,     /* selection bias [E], N(0, sigma) fp32 */
    HMOE_KIND_GATE_Q = 3,   /* int4 codes of gate [I][H] */
    HMOE_KIND_UP_Q = 4,     /* int4 codes of up [I][H] */
    HMOE_KIND_DOWN_Q = 5,   /* int4 codes of down [H][I] */
    HMOE_KIND_GATE_S = 6,   /* bf16 |N(0, 0.004)| group-128 scales of gate [I][H/128] */
    HMOE_KIND_UP_S = 7,
    HMOE_KIND_DOWN_S = 8,
    HMOE_KIND_SH_GATE = 9,  /* shared expert gate [I][H], bf16 N(0, 0.02) */
    HMOE_KIND_SH_UP = 10,
    HMOE_KIND_SH_DOWN = 11, /* shared expert down [H][I] */
    HMOE_KIND_PARTIAL = 12, /* caller partial-sum buffer, N(0, 0.1) fp32 */
    HMOE_KIND_NORM_W = 13,  /* RMSNorm weight, 1 + N(0, 0.02) fp32 */
    HMOE_KIND_PERM = 14     /* seeded permutations (popularity order) */
};

HMOE_HD uint64_t hmoe_mix64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

/* key of one tensor of the synthetic layer */
HMOE_HD uint64_t hmoe_key(uint64_t seed, uint32_t layer, uint32_t kind, uint32_t expert)
{
    uint64_t k = hmoe_mix64(seed ^ 0x6a09e667f3bcc909ull);
    k = hmoe_mix64(k ^ ((uint64_t) layer * 0x9e3779b97f4a7c15ull));
    k = hmoe_mix64(k ^ ((uint64_t) kind * 0xc2b2ae3d27d4eb4full));
    return hmoe_mix64(k ^ ((uint64_t) expert * 0x165667b19e3779f9ull));
}

/* 64 random bits of element `idx` of the tensor with key `key` */
HMOE_HD uint64_t hmoe_bits(uint64_t key, uint64_t idx)
{
    return hmoe_mix64(key + (idx + 1ull) * 0x9e3779b97f4a7c15ull);
}

HMOE_HD uint32_t hmoe_f2u(float f) { union { float f; uint32_t u; } v; v.f = f; return v.u; }
HMOE_HD float hmoe_u2f(uint32_t u) { union { float f; uint32_t u; } v; v.u = u; return v.f; }

/* natural log of u in (0, 1], u a normal float: u = m 2^e with m in [sqrt(1/2), sqrt(2)), log m = 2 atanh(t),
 * t = (m - 1) / (m + 1), |t| <= 0.1716, series to t^9 (truncation < 1e-9 relative) */
HMOE_HD float hmoe_logf(float u)
{
    const uint32_t b = hmoe_f2u(u);
    int e = (int) (b >> 23) - 127;
    float m = hmoe_u2f((b & 0x007fffffu) | 0x3f800000u);
    if (m > 1.41421356f) { m = m * 0.5f; e = e + 1; }
    const float t = (m - 1.0f) / (m + 1.0f);
    const float t2 = t * t;
    float p = __builtin_fmaf(t2, 0.111111111f, 0.142857143f);
    p = __builtin_fmaf(t2, p, 0.2f);
    p = __builtin_fmaf(t2, p, 0.333333333f);
    p = __builtin_fmaf(t2, p, 1.0f);
    return __builtin_fmaf((float) e, 0.693147181f, (t + t) * p);
}

/* cos(2 pi j / 2^24) for j in [0, 2^24): exact quadrant split, then Taylor series of sin / cos on [0, pi/2)
 * (truncation < 6e-9) */
HMOE_HD float hmoe_cos2pi24(uint32_t j)
{
    const uint32_t q = (j >> 22) & 3u;
    const float th = (float) (j & 0x3fffffu) * 3.7450702e-07f;     /* (2 pi / 2^24) * frac, in [0, pi/2) */
    const float t2 = th * th;
    float c = __builtin_fmaf(t2, 2.0876757e-09f, -2.7557319e-07f);  /* 1/12!, -1/10! */
    c = __builtin_fmaf(t2, c, 2.4801587e-05f);                      /* 1/8! */
    c = __builtin_fmaf(t2, c, -1.3888889e-03f);                     /* -1/6! */
    c = __builtin_fmaf(t2, c, 4.1666667e-02f);                      /* 1/4! */
    c = __builtin_fmaf(t2, c, -0.5f);
    c = __builtin_fmaf(t2, c, 1.0f);
    float s = __builtin_fmaf(t2, 1.6059044e-10f, -2.5052108e-08f);  /* 1/13!, -1/11! */
    s = __builtin_fmaf(t2, s, 2.7557319e-06f);                      /* 1/9! */
    s = __builtin_fmaf(t2, s, -1.9841270e-04f);                     /* -1/7! */
    s = __builtin_fmaf(t2, s, 8.3333333e-03f);                      /* 1/5! */
    s = __builtin_fmaf(t2, s, -1.6666667e-01f);                     /* -1/3! */
    s = __builtin_fmaf(t2 * th, s, th);
    return q == 0u ? c : q == 1u ? -s : q == 2u ? -c : s;
}

/* standard normal deviate of element idx (Box-Muller, cosine branch) */
HMOE_HD float hmoe_normal(uint64_t key, uint64_t idx)
{
    const uint64_t h = hmoe_bits(key, idx);
    const float u1 = (float) ((h >> 40) + 1ull) * 5.9604644775390625e-08f;    /* (0, 1] */
    const float r = __builtin_sqrtf(-2.0f * hmoe_logf(u1));
    return r * hmoe_cos2pi24((uint32_t) (h & 0xffffffull));
}

/* int4 code (q + 8, q uniform in [-8, 7]) of element k of row n of an [N][K] matrix: one 64-bit draw per 16 codes */
HMOE_HD uint32_t hmoe_code(uint64_t key, int64_t n, int64_t K, int64_t k)
{
    const uint64_t flat = (uint64_t) (n * K + k);
    return (uint32_t) (hmoe_bits(key, flat >> 4) >> (4u * (uint32_t) (flat & 15u))) & 15u;
}

/* fp32 -> bf16, round to nearest even (NaN kept quiet) */
HMOE_HD uint16_t hmoe_f2bf(float f)
{
    uint32_t u = hmoe_f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t) ((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t) (u >> 16);
}

HMOE_HD float hmoe_bf2f(uint16_t b) { return hmoe_u2f((uint32_t) b << 16); }

/* fp32 -> f16, round to nearest even, with subnormals, overflow to inf, NaN kept */
HMOE_HD uint16_t hmoe_f2h(float f)
{
    const uint32_t u = hmoe_f2u(f);
    const uint32_t sign = (u >> 16) & 0x8000u;
    const uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint16_t) (sign | 0x7e00u);
    if (a >= 0x477ff000u) return (uint16_t) (sign | 0x7c00u);          /* >= 65520 rounds to inf */
    if (a >= 0x38800000u)                                               /* normal f16 range (>= 2^-14) */
    {
        const uint32_t m = a + 0xfffu + ((a >> 13) & 1u);               /* round at bit 13 */
        return (uint16_t) (sign | ((m - 0x38000000u) >> 13));
    }
    if (a < 0x33000000u) return (uint16_t) sign;                        /* < 2^-25 rounds to zero */
    /* subnormal f16: value = a * 2^24 units of 2^-24 */
    const uint32_t e = a >> 23;                                         /* biased exponent, 102..112 */
    const uint32_t mant = (a & 0x7fffffu) | 0x800000u;
    const uint32_t shift = 126u - e;                                    /* 14..24 */
    const uint32_t q = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1u);
    const uint32_t r = q + ((rem > half || (rem == half && (q & 1u))) ? 1u : 0u);
    return (uint16_t) (sign | r);
}

HMOE_HD float hmoe_h2f(uint16_t h)
{
    const uint32_t sign = ((uint32_t) h & 0x8000u) << 16;
    const uint32_t e = ((uint32_t) h >> 10) & 31u, m = (uint32_t) h & 1023u;
    if (e == 31u) return hmoe_u2f(sign | 0x7f800000u | (m << 13));
    if (e == 0u) { const float v = (float) m * 5.9604644775390625e-08f; return sign ? -v : v; }
    return hmoe_u2f(sign | ((e + 112u) << 23) | (m << 13));
}

/* e^x for the router sigmoid, written from the series so host and device agree bit for bit: x clamped to
 * [-87, 88], n = floor(x log2 e + 1/2), r = x - n ln 2 (two-constant Cody-Waite split), e^r by its Taylor series to
 * r^8 (|r| <= 0.35: truncation < 3e-9), times 2^n assembled in the exponent field */
HMOE_HD float hmoe_expf(float x)
{
    x = x > 88.0f ? 88.0f : (x < -87.0f ? -87.0f : x);
    const float n = __builtin_floorf(x * 1.44269504f + 0.5f);
    float r = __builtin_fmaf(-n, 0.693145752f, x);
    r = __builtin_fmaf(-n, 1.42860677e-06f, r);
    float p = __builtin_fmaf(r, 2.48015873e-05f, 1.98412698e-04f);   /* 1/8!, 1/7! */
    p = __builtin_fmaf(r, p, 1.38888889e-03f);                      /* 1/6! */
    p = __builtin_fmaf(r, p, 8.33333333e-03f);                      /* 1/5! */
    p = __builtin_fmaf(r, p, 4.16666667e-02f);                      /* 1/4! */
    p = __builtin_fmaf(r, p, 1.66666667e-01f);                      /* 1/3! */
    p = __builtin_fmaf(r, p, 0.5f);
    p = __builtin_fmaf(r, p, 1.0f);
    p = __builtin_fmaf(r, p, 1.0f);
    return p * hmoe_u2f((uint32_t) ((int) n + 127) << 23);
}

/* sigmoid of a router logit, as the fused router computes it: 1 / (1 + e^-l) (exl3_router.py:96) */
HMOE_HD float hmoe_sigmoid(float l) { return 1.0f / (1.0f + hmoe_expf(-l)); }

/* order-preserving unsigned key of a float (exl3_router.py:97-98, nr4_kernel.cuh:64) */
HMOE_HD uint32_t hmoe_okey(float v)
{
    const uint32_t u = hmoe_f2u(v);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

#endif /* HMOE_RNG_H */
