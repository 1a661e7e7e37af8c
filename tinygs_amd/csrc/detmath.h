// Deterministic single-precision exp / log for the FastGS kernels.
//
// The reference compiles with --use_fast_math (tinygs/CMakeLists.txt:198-202),
// so its expf/logf results are not reproducible. Tile assignment, per-pixel
// contributor counts and the 1/255 alpha cut depend on these functions, so
// the build fixes one definition evaluated with IEEE-754 operations only:
// round-to-nearest add/mul/fma, rint, exact ldexp. The same operations in
// the same order give the same bits on the CPU and on gfx950, provided the
// translation unit is compiled with -ffp-contract=off.
//
// Method: Cody & Waite argument reduction (W. J. Cody, W. Waite, "Software
// Manual for the Elementary Functions", 1980) followed by
//   exp: degree-7 Taylor polynomial of e^r, |r| <= ln2/2 (Horner form);
//        truncation error (ln2/2)^8/8! < 5.3e-9 relative, <= 2 ulp overall.
//   log: log(m) = 2 atanh(s), s = (m-1)/(m+1), m in [sqrt(1/2), sqrt(2)],
//        odd series to s^9; <= 2 ulp overall.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define TGS_HD __host__ __device__ __forceinline__

namespace tgs {

TGS_HD uint32_t f2u(float f) { return __builtin_bit_cast(uint32_t, f); }
TGS_HD float u2f(uint32_t u) { return __builtin_bit_cast(float, u); }

// e^x. Inputs above 88.7228394 give +inf, below -103.972 give 0, NaN passes.
TGS_HD float det_expf(float x) {
    if (x != x) return x;
    if (x > 88.72283935546875f) return __builtin_inff();
    if (x < -103.97208404541015625f) return 0.0f;
    const float k = __builtin_rintf(x * 1.44269502162933349609375f);
    float r = __builtin_fmaf(k, -0.693145751953125f, x);
    r = __builtin_fmaf(k, -1.428606765330187045037746429443359375e-06f, r);
    float p = 1.98412698412698412698e-04f;
    p = __builtin_fmaf(p, r, 1.38888888888888888889e-03f);
    p = __builtin_fmaf(p, r, 8.33333333333333333333e-03f);
    p = __builtin_fmaf(p, r, 4.16666666666666666667e-02f);
    p = __builtin_fmaf(p, r, 1.66666666666666666667e-01f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    return __builtin_ldexpf(p, (int)k);
}

// e^x for -104 <= x <= 0 without range checks; same bits as det_expf for
// x >= -103.97208 and 0 below it (k = -150 there and p < 1).
TGS_HD float det_expf_core(float x) {
    const float k = __builtin_rintf(x * 1.44269502162933349609375f);
    float r = __builtin_fmaf(k, -0.693145751953125f, x);
    r = __builtin_fmaf(k, -1.428606765330187045037746429443359375e-06f, r);
    float p = 1.98412698412698412698e-04f;
    p = __builtin_fmaf(p, r, 1.38888888888888888889e-03f);
    p = __builtin_fmaf(p, r, 8.33333333333333333333e-03f);
    p = __builtin_fmaf(p, r, 4.16666666666666666667e-02f);
    p = __builtin_fmaf(p, r, 1.66666666666666666667e-01f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    return __builtin_ldexpf(p, (int)k);
}

// 2^x for -150 <= x <= 0: the blend forward's alpha = o 2^(-sigma'), with
// sigma' = sigma log2(e) evaluated from a conic prescaled by log2(e).
// k = rint(x), r = x - k in [-1/2, 1/2] (exact), 2^r by the degree-5 minimax
// polynomial of relative error 7.5e-8 (Remez exchange, E. Remez 1934),
// coefficients rounded to float; <= 2.1e-7 relative overall; exact ldexp
// (k = -150 gives 0 or the least subnormal).
TGS_HD float det_exp2_core(float x) {
    const float k = __builtin_rintf(x);
    const float r = x - k;
    float p = 0x1.5c08e6p-10f;
    p = __builtin_fmaf(p, r, 0x1.3d0c52p-7f);
    p = __builtin_fmaf(p, r, 0x1.c6b6e4p-5f);
    p = __builtin_fmaf(p, r, 0x1.ebf918p-3f);
    p = __builtin_fmaf(p, r, 0x1.62e428p-1f);
    p = __builtin_fmaf(p, r, 0x1.000002p+0f);
    return __builtin_ldexpf(p, (int)k);
}

// e^x for x <= 0 (the blend's exp(-sigma)); same bits as det_expf there.
TGS_HD float det_expf_nonpos(float x) {
    x = x < -103.97208404541015625f ? -104.0f : x;  // -104 -> k=-150, ldexp gives 0
    return det_expf_core(x);
}

// natural log, x > 0; 0 -> -inf, negative / NaN -> NaN.
TGS_HD float det_logf(float x) {
    if (!(x > 0.0f)) return (x == 0.0f) ? -__builtin_inff() : __builtin_nanf("");
    if (x == __builtin_inff()) return x;
    uint32_t u = f2u(x);
    int e = 0;
    if (u < 0x00800000u) {
        x = x * 8388608.0f;
        u = f2u(x);
        e = -23;
    }
    e += (int)((u >> 23) & 0xffu) - 127;
    float m = u2f((u & 0x007fffffu) | 0x3f800000u);
    if (m > 1.41421353816986083984375f) {
        m = m * 0.5f;
        e += 1;
    }
    const float f = m - 1.0f;
    const float s = f / (m + 1.0f);
    const float s2 = s * s;
    float p = 1.11111111111111111111e-01f;
    p = __builtin_fmaf(p, s2, 1.42857142857142857143e-01f);
    p = __builtin_fmaf(p, s2, 2.00000000000000000000e-01f);
    p = __builtin_fmaf(p, s2, 3.33333333333333333333e-01f);
    const float t = s2 * p;
    const float logm = 2.0f * __builtin_fmaf(s, t, s);
    const float ef = (float)e;
    return __builtin_fmaf(ef, 0.693145751953125f,
                          __builtin_fmaf(ef, 1.428606765330187045037746429443359375e-06f, logm));
}

// __saturatef: clamp to [0,1], NaN -> 0.
TGS_HD float saturate(float x) { return x > 0.0f ? (x < 1.0f ? x : 1.0f) : 0.0f; }

// Saturating float -> int32 with floor / ceil; NaN -> 0.
TGS_HD int32_t sat_floor_i32(float v) {
    if (v != v) return 0;
    const float f = __builtin_floorf(v);
    if (f >= 2147483647.0f) return 2147483647;
    if (f <= -2147483648.0f) return (int32_t)(-2147483647 - 1);
    return (int32_t)f;
}
TGS_HD int32_t sat_ceil_i32(float v) {
    if (v != v) return 0;
    const float f = __builtin_ceilf(v);
    if (f >= 2147483647.0f) return 2147483647;
    if (f <= -2147483648.0f) return (int32_t)(-2147483647 - 1);
    return (int32_t)f;
}

}  // namespace tgs
