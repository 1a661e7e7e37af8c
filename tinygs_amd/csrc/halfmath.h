// Canonical half-precision (IEEE binary16) arithmetic of the fp16-image
// rasterizer (FGS16), shared operation for operation with the CPU oracle
// (oracle/halfmath.h) so that its tile tests, pixels and per-bucket gradient
// sums are bit-identical there.
//
// The reference's FGS16 kernels (tinygs/src/rasterizer/fastgs_ours_fp16/)
// mix correctly rounded half2 intrinsics with approximate ones
// (ex2.approx.f16x2, __h2div) and directed-rounding conversions. The build
// fixes one definition for each:
//   h_rn      float -> half, round to nearest even (v_cvt_f16_f32)
//   h_rd      float -> half, round toward -inf: RN, then one step down when
//             RN rounded up
//   + - *     correctly rounded (v_add/v_sub/v_mul_f16, packed or not)
//   h_fma     correctly rounded fused multiply-add (v_fma_f16, v_pk_fma_f16)
//   h_div     correctly rounded: IEEE float quotient of the two halves,
//             rounded to half (float's 24 bits >= 2 * 11 + 2, so the double
//             rounding is innocuous; S. A. Figueroa, "When is double rounding
//             innocuous?", SIGNUM 1995)
//   h_div_blend  correctly rounded for divisors in [0x1.4p-7, 1] (Markstein's
//             iteration on v_rcp_f16; checked over all dividends and those
//             divisors)
//   h_exp2    correctly rounded 2^x of a half x (v_exp_f16; checked over all
//             65,536 inputs against the oracle's)
//   h_min     IEEE minNum: a NaN operand yields the other (the blend never
//             compares two zeros)        h_relu  x > 0 ? x : +0 (NaN -> +0)
//   h_sat     clamp to [0, 1], NaN -> 0
//   half_of_fixed  the correctly rounded half of S * 2^-24 (an exact integer
//             sum of half values), by integer shifts as in the oracle;
//             half_of_double_sum the same for a double (through float
//             rounded toward odd)
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"

namespace tgs {

typedef _Float16 h16;
typedef _Float16 h16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint16_t hbits(h16 x) { return __builtin_bit_cast(uint16_t, x); }
__device__ __forceinline__ h16 hfrom(uint16_t b) { return __builtin_bit_cast(h16, b); }
__device__ __forceinline__ uint32_t h2bits(h16x2 x) { return __builtin_bit_cast(uint32_t, x); }
__device__ __forceinline__ h16x2 h2from(uint32_t b) { return __builtin_bit_cast(h16x2, b); }
__device__ __forceinline__ h16x2 h2(h16 a, h16 b) {
    h16x2 r;
    r.x = a;
    r.y = b;
    return r;
}
__device__ __forceinline__ h16x2 h2s(h16 a) { return h2(a, a); }

__device__ __forceinline__ h16 h_rn(float x) { return (h16)f32_opaque(x); }   // of x as computed (common.h)
__device__ __forceinline__ float h2f(h16 x) { return (float)x; }

// next half toward -inf of a finite or infinite non-NaN half
__device__ __forceinline__ uint16_t h_step_down(uint16_t b) {
    if (b & 0x8000u) return (uint16_t)(b + 1u);   // more negative
    return b == 0u ? (uint16_t)0x8001u : (uint16_t)(b - 1u);
}

__device__ __forceinline__ h16 h_rd(float x) {
    const h16 r = (h16)x;
    return (float)r > x ? hfrom(h_step_down(hbits(r))) : r;
}

__device__ __forceinline__ h16 h_fma(h16 a, h16 b, h16 c) { return __builtin_elementwise_fma(a, b, c); }
__device__ __forceinline__ h16x2 h2_fma(h16x2 a, h16x2 b, h16x2 c) { return __builtin_elementwise_fma(a, b, c); }

// v_exp_f16 (no packed form) on both halves of x, the high result written
// straight into the high half of the low result's register (SDWA
// dst_sel:WORD_1, dst_unused:UNUSED_PRESERVE) instead of a separate pack. The
// s_nop 0s are the wait states around a transcendental op's operand and
// result. (For the reciprocal the pack costs nothing: the division's
// finishing fmas write the two halves directly only when each reciprocal has
// its own register.)
__device__ __forceinline__ uint32_t h2_trans_exp(uint32_t x) {
    uint32_t r;
    asm(
        "s_nop 0\n\t"
        "v_exp_f16_e32 %0, %1\n\t"
        "s_nop 0\n\t"
        "v_exp_f16_sdwa %0, %1 dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:WORD_1\n\t"
        "s_nop 0"
        : "=&v"(r)
        : "v"(x));
    return r;
}

__device__ __forceinline__ h16 h_div(h16 a, h16 b) { return (h16)((float)a / (float)b); }
// a / b correctly rounded for a divisor b in [0x1.4p-7, 1] (bits 0x2100 ..
// 0x3c00: the blend backward's 1 - alpha, alpha in [0, RN(0.99)]), by
// Markstein's iteration: y = RN(1 / b) (v_rcp_f16, equal to the correctly
// rounded reciprocal of every positive finite half), q0 = RN(a y) clamped to
// the finite halves, the residual r = b q0 - a exactly in float (its sign
// keeps a zero quotient's sign), q = RN(q0 - r y) rounded once from the
// exact value: v_fma_mixlo_f16 / v_fma_mixhi_f16 round the fused result
// straight to half. Rounding it to float first is not innocuous here (r y
// carries more bits than a half operation): a = 0x828d, b = 0x2353 lands on
// a half midpoint in float and rounds to 0x9992 instead of 0x9993. So the
// last step is written as those two instructions, not left to instruction
// selection. Equal to h_div in both lanes for every half a and every b of
// that range (all 4.5e8 pairs per lane, tgs_selftest_half_div_blend); other
// divisors are not covered. P. Markstein, "Computation of elementary
// functions on the IBM RISC System/6000 processor", IBM J. Res. Dev. 34, 1990.
__device__ __forceinline__ h16x2 h2_div_blend(h16x2 a, h16x2 b) {
    const h16x2 y = h2(__builtin_amdgcn_rcph(b.x), __builtin_amdgcn_rcph(b.y));
    const h16x2 lim = h2((h16)65504.0f, (h16)65504.0f);
    const h16x2 q0 = __builtin_elementwise_max(__builtin_elementwise_min(a * y, lim), -lim);
    const float rx = __builtin_fmaf((float)b.x, (float)q0.x, -(float)a.x);
    const float ry = __builtin_fmaf((float)b.y, (float)q0.y, -(float)a.y);
    // q.x = RN16(-rx y.x + q0.x), q.y = RN16(-ry y.y + q0.y); op_sel picks the
    // high halves of y and q0 for the high lane (op_sel_hi: f16 sources)
    uint32_t q;
    asm("v_fma_mixlo_f16 %0, -%1, %3, %4 op_sel_hi:[0,1,1]\n\t"
        "v_fma_mixhi_f16 %0, -%2, %3, %4 op_sel:[0,1,1] op_sel_hi:[0,1,1]"
        : "=&v"(q)
        : "v"(rx), "v"(ry), "v"(h2bits(y)), "v"(h2bits(q0)));
    return h2from(q);
}
__device__ __forceinline__ h16 h_div_blend(h16 a, h16 b) { return h2_div_blend(h2s(a), h2s(b)).x; }
__device__ __forceinline__ h16x2 h2_div(h16x2 a, h16x2 b) { return h2(h_div(a.x, b.x), h_div(a.y, b.y)); }

// 2^x: v_exp_f16, which is correctly rounded for every half input (checked
// over all 65,536 inputs against the oracle's correctly rounded exp2)
__device__ __forceinline__ h16 h_exp2(h16 x) { return __builtin_elementwise_exp2(x); }
__device__ __forceinline__ h16x2 h2_exp2(h16x2 x) { return h2from(h2_trans_exp(h2bits(x))); }

// IEEE minNum (v_min_f16 / v_pk_min_f16): a NaN operand yields the other
__device__ __forceinline__ h16 h_min(h16 a, h16 b) { return __builtin_elementwise_min(a, b); }
__device__ __forceinline__ h16x2 h2_min(h16x2 a, h16x2 b) { return __builtin_elementwise_min(a, b); }
__device__ __forceinline__ h16 h_relu(h16 x) { return x > (h16)0 ? x : (h16)0; }
__device__ __forceinline__ h16x2 h2_relu(h16x2 x) { return h2(h_relu(x.x), h_relu(x.y)); }
__device__ __forceinline__ h16 h_sat(h16 x) { return x > (h16)0 ? (x < (h16)1 ? x : (h16)1) : (h16)0; }

// Correctly rounded (to nearest even) half of S * 2^-24, returned as float.
__device__ __forceinline__ float half_of_fixed(int64_t S) {
    if (S == 0) return 0.0f;
    const uint64_t a = S < 0 ? 0ull - (uint64_t)S : (uint64_t)S;
    if (a >= (65520ull << 24)) return S < 0 ? -__builtin_inff() : __builtin_inff();
    const int msb = 63 - __builtin_clzll(a);
    uint64_t q = a;
    int shift = 0;
    if (msb > 10) {
        shift = msb - 10;
        q = a >> shift;
        const uint64_t rem = a - (q << shift), half = 1ull << (shift - 1);
        if (rem > half || (rem == half && (q & 1ull))) ++q;
    }
    const float v = __builtin_ldexpf((float)q, shift - 24);   // exact: q < 2^12
    return S < 0 ? -v : v;
}

// The correctly rounded half of a double s (the exact double sums of half
// records), returned as float; infinities pass, NaN gives NaN. Rounding s to
// float and then to half would round twice: s = m + 2^-24 just above a half
// midpoint m in [1, 2) is a float midpoint, rounds to m in float and then to
// even in half. Rounding to float toward odd instead (truncate, then set the
// last bit when inexact) keeps a sticky bit, and float's 24 bits >= 11 + 2
// make the second rounding exact (S. Boldo, G. Melquiond, "When double
// rounding is odd", IMACS 2005).
__device__ __forceinline__ float half_of_double_sum(double s) {
    if (s != s) return __builtin_nanf("");
    float f = (float)s;
    if ((double)f != s) {
        uint32_t u = __builtin_bit_cast(uint32_t, f);
        if (__builtin_fabs((double)f) > __builtin_fabs(s)) u -= 1u;   // the neighbour toward zero
        f = __builtin_bit_cast(float, u | 1u);
    }
    return (float)(h16)f;
}

}  // namespace tgs
