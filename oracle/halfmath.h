/* TEST INFRASTRUCTURE — the oracle's canonical half-precision arithmetic
 * (IEEE binary16 values held as their 16-bit patterns), the same definitions
 * as the kernels' tinygs_amd/csrc/halfmath.h:
 *   oh_rn     float -> half, round to nearest even
 *   oh_rd     float -> half, toward -inf (RN, then one step down if RN rounded up)
 *   add/sub/mul/div   correctly rounded: the float operation on the exact
 *             float values of two halves, rounded to half (innocuous double
 *             rounding, 24 >= 2 * 11 + 2; Figueroa 1995)
 *   oh_fma    correctly rounded a * b + c: the product is exact in double,
 *             the sum's rounding error is recovered exactly by TwoSum
 *             (Knuth, TAOCP vol. 2, 4.2.2), and the final rounding to half
 *             takes the error's sign into account at halfway points
 *   oh_exp2   correctly rounded 2^x: double exp2 of the half, rounded to half
 *   oh_min    IEEE minNum (a NaN operand yields the other);  oh_relu x > 0 ? x : +0;
 *             oh_sat clamp to [0,1] (NaN -> 0)
 *   oh_from_fixed  the correctly rounded half of S * 2^-24, S an integer (an
 *             exact sum of half values: every finite half is a multiple of 2^-24)
 */
#pragma once

#include <math.h>
#include <stdint.h>

#include "detmath.h"

typedef uint16_t oh16;

static inline float oh_f(oh16 a) { return orc_half_bits_to_float(a); }
static inline oh16 oh_rn(float x) { return orc_float_to_half_bits(x); }

static inline oh16 oh_step_down(oh16 b) {
    if (b & 0x8000u) return (oh16)(b + 1u);
    return b == 0u ? (oh16)0x8001u : (oh16)(b - 1u);
}
static inline oh16 oh_rd(float x) {
    const oh16 r = oh_rn(x);
    return oh_f(r) > x ? oh_step_down(r) : r;
}

/* Round v + e to half, where e is a tiny error whose sign alone matters
 * (err_sign < 0, 0 or > 0; |e| far below half precision). */
static inline oh16 oh_round_double(double v, int err_sign) {
    if (v != v) return (oh16)0x7e00u;
    const uint16_t sign = v < 0 ? 0x8000u : 0u;
    double a = fabs(v);
    if (sign) err_sign = -err_sign;   /* now relative to |v| */
    if (a == 0.0) {
        if (err_sign == 0) return sign;
        /* a tiny nonzero value rounds to zero of its own sign */
        return err_sign > 0 ? sign : (oh16)(sign ^ 0x8000u);
    }
    int e;
    frexp(a, &e);          /* a = m 2^e, m in [0.5, 1) */
    int qe = e - 1 - 10;   /* quantum of the half binade */
    if (qe < -24) qe = -24;
    const double q = ldexp(1.0, qe);
    const double m = a / q;            /* exact: q is a power of two */
    double fl = floor(m);
    const double frac = m - fl;
    /* below / above the halfway point the error cannot cross it (|e| is below
     * half a double ulp of v); at it, the error's sign decides, else even */
    int up;
    if (frac > 0.5) up = 1;
    else if (frac < 0.5) up = 0;
    else up = err_sign > 0 ? 1 : (err_sign < 0 ? 0 : (int)((int64_t)fl & 1));
    const double r = (fl + up) * q;
    if (r >= 65520.0 || r > 65504.0) return (oh16)(sign | 0x7c00u);
    return (oh16)(sign | orc_float_to_half_bits((float)r));
}

static inline oh16 oh_add(oh16 a, oh16 b) { return oh_rn(oh_f(a) + oh_f(b)); }
static inline oh16 oh_sub(oh16 a, oh16 b) { return oh_rn(oh_f(a) - oh_f(b)); }
static inline oh16 oh_mul(oh16 a, oh16 b) { return oh_rn(oh_f(a) * oh_f(b)); }
static inline oh16 oh_div(oh16 a, oh16 b) { return oh_rn(oh_f(a) / oh_f(b)); }
static inline oh16 oh_neg(oh16 a) { return (oh16)(a ^ 0x8000u); }
static inline oh16 oh_abs(oh16 a) { return (oh16)(a & 0x7fffu); }

static inline oh16 oh_fma(oh16 a, oh16 b, oh16 c) {
    const double fa = oh_f(a), fb = oh_f(b), fc = oh_f(c);
    if (fa != fa || fb != fb || fc != fc) return (oh16)0x7e00u;
    if (isinf(fa) || isinf(fb) || isinf(fc)) {
        const double r = fa * fb + fc;   /* inf / NaN propagation */
        return r != r ? (oh16)0x7e00u : (r > 0 ? (oh16)0x7c00u : (oh16)0xfc00u);
    }
    const double p = fa * fb;            /* exact: 11 x 11 bits */
    const double s = p + fc;
    const double bb = s - p;
    const double err = (p - (s - bb)) + (fc - bb);   /* TwoSum: p + fc = s + err exactly */
    if (s == 0.0 && err == 0.0) {
        /* exact zero: IEEE sign rules (x + -x = +0; -0 + -0 = -0) */
        const int neg_p = (signbit(p) != 0), neg_c = (signbit(fc) != 0);
        return (neg_p && neg_c) ? (oh16)0x8000u : (oh16)0u;
    }
    return oh_round_double(s, err > 0 ? 1 : (err < 0 ? -1 : 0));
}

static inline oh16 oh_exp2(oh16 x) {
    const double fx = oh_f(x);
    if (fx != fx) return (oh16)0x7e00u;
    return oh_round_double(exp2(fx), 0);
}

static inline int oh_lt(oh16 a, oh16 b) { return oh_f(a) < oh_f(b); }
static inline int oh_isnan(oh16 a) { return (a & 0x7fffu) > 0x7c00u; }
/* IEEE minNum: a NaN operand yields the other one (the blend never compares
 * two zeros, so the order of -0 and +0 is not needed) */
static inline oh16 oh_min(oh16 a, oh16 b) {
    if (oh_isnan(a)) return b;
    if (oh_isnan(b)) return a;
    return oh_lt(b, a) ? b : a;
}
static inline oh16 oh_relu(oh16 x) { return oh_f(x) > 0.0f ? x : (oh16)0u; }
static inline oh16 oh_sat(oh16 x) {
    const float f = oh_f(x);
    return f > 0.0f ? (f < 1.0f ? x : (oh16)0x3c00u) : (oh16)0u;
}

/* Correctly rounded (to nearest even) half of S * 2^-24, by integer shifts:
 * the same steps as the kernels' half_of_fixed. */
static inline oh16 oh_from_fixed(int64_t S) {
    if (S == 0) return 0u;
    const uint16_t sign = S < 0 ? 0x8000u : 0u;
    const uint64_t a = S < 0 ? (uint64_t)0 - (uint64_t)S : (uint64_t)S;
    if (a >= ((uint64_t)65520u << 24)) return (oh16)(sign | 0x7c00u);   /* rounds to infinity */
    int msb = 63;
    while (!((a >> msb) & 1u)) --msb;
    uint64_t q = a;
    int shift = 0;
    if (msb > 10) {
        shift = msb - 10;
        q = a >> shift;
        const uint64_t rem = a - (q << shift), half = (uint64_t)1 << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) ++q;
    }
    const float v = ldexpf((float)q, shift - 24);   /* exact: q < 2^12 */
    return (oh16)(sign | oh_rn(v));
}
