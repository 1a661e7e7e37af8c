/* TEST INFRASTRUCTURE — part of the CPU oracle. Only tests/, the smoke check
 * and bench.py's cpu_baseline leg may load it; the product never does.
 *
 * Deterministic single-precision exp and log used by the oracle.
 *
 * The reference builds with --use_fast_math (tinygs/CMakeLists.txt:198-202),
 * so its expf/logf are approximate and not reproducible off NVIDIA hardware.
 * The build fixes one definition that the CPU oracle and the GPU kernels
 * both evaluate with the same IEEE-754 operations in the same order
 * (round-to-nearest add/mul/fma, correctly rounded division, exact ldexp),
 * so binning decisions that depend on exp/log are bit-identical.
 *
 * Method: Cody & Waite argument reduction (W. J. Cody, W. Waite, "Software
 * Manual for the Elementary Functions", 1980), followed by
 *   exp: degree-7 Taylor polynomial of e^r on |r| <= ln2/2 (Horner, fmaf);
 *        truncation error (ln2/2)^8/8! < 5.3e-9 relative.
 *   log: log(m) = 2*atanh(s), s = (m-1)/(m+1), m in [sqrt(1/2), sqrt(2));
 *        odd series up to s^9; truncation error < 1e-9 relative.
 * Accuracy is checked in tests against libm's double-precision exp/log.
 *
 * The product carries its own copy (tinygs_amd/csrc/detmath.h); a test checks
 * both copies agree bit for bit over a sweep of inputs.
 */
#ifndef ORACLE_DETMATH_H
#define ORACLE_DETMATH_H

#include <math.h>
#include <stdint.h>
#include <string.h>

static inline float orc_bits_to_float(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t orc_float_to_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* e^x for float x. Inputs above 88.7228394 give +inf, below -103.972 give 0. */
static inline float orc_expf(float x) {
    if (x != x) return x;
    if (x > 88.72283935546875f) return INFINITY;
    if (x < -103.97208404541015625f) return 0.0f;
    const float k = rintf(x * 1.44269502162933349609375f);          /* round(x / ln2) */
    float r = fmaf(k, -0.693145751953125f, x);                        /* ln2 high part, 15 bits */
    r = fmaf(k, -1.428606765330187045037746429443359375e-06f, r);    /* ln2 low part */
    float p = 1.98412698412698412698e-04f;                            /* 1/7! */
    p = fmaf(p, r, 1.38888888888888888889e-03f);                      /* 1/6! */
    p = fmaf(p, r, 8.33333333333333333333e-03f);                      /* 1/5! */
    p = fmaf(p, r, 4.16666666666666666667e-02f);                      /* 1/4! */
    p = fmaf(p, r, 1.66666666666666666667e-01f);                      /* 1/3! */
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return ldexpf(p, (int)k);
}

/* 2^x for -150 <= x <= 0 (the blend forward's alpha = o 2^(-sigma'), sigma'
 * in log2 units): k = rint(x), r = x - k in [-1/2, 1/2] (exact), 2^r by the
 * degree-5 minimax polynomial of relative error 7.5e-8 (Remez exchange,
 * E. Remez 1934), coefficients rounded to float (Horner, fmaf); exact ldexp. */
static inline float orc_exp2_core(float x) {
    const float k = rintf(x);
    const float r = x - k;
    float p = 0x1.5c08e6p-10f;
    p = fmaf(p, r, 0x1.3d0c52p-7f);
    p = fmaf(p, r, 0x1.c6b6e4p-5f);
    p = fmaf(p, r, 0x1.ebf918p-3f);
    p = fmaf(p, r, 0x1.62e428p-1f);
    p = fmaf(p, r, 0x1.000002p+0f);
    return ldexpf(p, (int)k);
}

/* natural log for float x > 0; x == 0 gives -inf, x < 0 or NaN gives NaN. */
static inline float orc_logf(float x) {
    if (!(x > 0.0f)) return (x == 0.0f) ? -INFINITY : NAN;
    if (x == INFINITY) return x;
    uint32_t u = orc_float_to_bits(x);
    int e = 0;
    if (u < 0x00800000u) {              /* subnormal: scale up by 2^23 */
        x = x * 8388608.0f;
        u = orc_float_to_bits(x);
        e = -23;
    }
    e += (int)((u >> 23) & 0xffu) - 127;
    float m = orc_bits_to_float((u & 0x007fffffu) | 0x3f800000u);  /* [1, 2) */
    if (m > 1.41421353816986083984375f) { m = m * 0.5f; e += 1; }  /* [sqrt(1/2), sqrt(2)] */
    const float f = m - 1.0f;
    const float s = f / (m + 1.0f);
    const float s2 = s * s;
    float p = 1.11111111111111111111e-01f;                          /* 1/9 */
    p = fmaf(p, s2, 1.42857142857142857143e-01f);                   /* 1/7 */
    p = fmaf(p, s2, 2.00000000000000000000e-01f);                   /* 1/5 */
    p = fmaf(p, s2, 3.33333333333333333333e-01f);                   /* 1/3 */
    const float t = s2 * p;                                          /* s^2/3 + s^4/5 + ... */
    /* log(m) = 2s + 2s*t = f - (f - 2s) + 2s*t; evaluate as 2*(s + s*t). */
    const float logm = 2.0f * fmaf(s, t, s);
    const float ef = (float)e;
    return fmaf(ef, 0.693145751953125f, fmaf(ef, 1.428606765330187045037746429443359375e-06f, logm));
}

/* IEEE float -> binary16 bits, round to nearest even (used for fp16 staging). */
static inline uint16_t orc_float_to_half_bits(float f) {
    uint32_t x = orc_float_to_bits(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t absx = x & 0x7fffffffu;
    if (absx >= 0x7f800000u) {                       /* inf / nan */
        return (uint16_t)(sign | 0x7c00u | (absx > 0x7f800000u ? 0x200u : 0u));
    }
    if (absx >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);  /* rounds to >= 65520 -> inf */
    if (absx < 0x38800000u) {                        /* result subnormal or zero */
        if (absx < 0x33000000u) return (uint16_t)sign;   /* < 2^-25: rounds to 0 */
        uint32_t mant = (absx & 0x007fffffu) | 0x00800000u;
        int shift = 126 - (int)(absx >> 23);          /* 14 + (113 - exp) */
        uint32_t half_mant = mant >> (shift);
        uint32_t rem = mant & ((1u << shift) - 1u);
        uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (half_mant & 1u))) half_mant += 1u;
        return (uint16_t)(sign | half_mant);
    }
    uint32_t r = absx - 0x38000000u;                 /* rebias exponent 127 -> 15 */
    uint32_t half = r >> 13;
    uint32_t rem = r & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (half & 1u))) half += 1u;
    return (uint16_t)(sign | half);
}

static inline float orc_half_bits_to_float(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = ((uint32_t)h >> 10) & 0x1fu;
    uint32_t m = (uint32_t)h & 0x3ffu;
    if (e == 0) {
        if (m == 0) return orc_bits_to_float(sign);
        float v = (float)m * 5.9604644775390625e-08f;   /* m * 2^-24 exactly */
        return sign ? -v : v;
    }
    if (e == 31) return orc_bits_to_float(sign | 0x7f800000u | (m << 13));
    return orc_bits_to_float(sign | ((e + 112u) << 23) | (m << 13));
}

static inline float orc_round_half(float f) { return orc_half_bits_to_float(orc_float_to_half_bits(f)); }

#endif
