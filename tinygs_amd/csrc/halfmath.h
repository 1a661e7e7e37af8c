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
//   h_exp2    correctly rounded 2^x of a half x (checked exhaustively over all
//             65,536 inputs against the oracle's, see tests)
//   h_min     b < a ? b : a           h_relu  x > 0 ? x : +0 (NaN -> +0)
//   h_sat     clamp to [0, 1], NaN -> 0
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

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

__device__ __forceinline__ h16 h_rn(float x) { return (h16)x; }
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

__device__ __forceinline__ h16 h_div(h16 a, h16 b) { return (h16)((float)a / (float)b); }
__device__ __forceinline__ h16x2 h2_div(h16x2 a, h16x2 b) { return h2(h_div(a.x, b.x), h_div(a.y, b.y)); }

// 2^x: v_exp_f32 of the exact f32 value of x (about 1 f32 ulp), rounded to
// half; when that value lies within 8 f32 ulps of a point halfway between two
// halves, the rounding is redone from a double-precision 2^x
__device__ __forceinline__ h16 h_exp2(h16 x) {
    const float r = __builtin_amdgcn_exp2f((float)x);
    const h16 h = (h16)r;
    const float fh = (float)h;
    // the halfway point on r's side of h, and r's distance to it
    const uint16_t b = hbits(h);
    const uint16_t bo = r >= fh ? (uint16_t)(b + 1u) : (uint16_t)(b - 1u);   // positive r: the neighbour toward r
    const float other = (float)hfrom(bo);
    const float mid = 0.5f * (fh + other);   // exact: halves have 11 bits
    const float d = __builtin_fabsf(r - mid);
    const float tol = 8.0f * __builtin_fabsf(r) * 5.9604644775390625e-08f;   // 8 ulp(r) as 2^-24 |r|
    if (d <= tol && (b & 0x7c00u) != 0x7c00u && r > 0.f) {
        const double e = __ocml_exp2_f64((double)(float)x);
        const uint16_t lo = b < bo ? b : bo, hi = b < bo ? bo : b;
        const double md = (double)mid;
        return hfrom(e > md ? hi : (e < md ? lo : ((lo & 1u) ? hi : lo)));
    }
    return h;
}
__device__ __forceinline__ h16x2 h2_exp2(h16x2 x) { return h2(h_exp2(x.x), h_exp2(x.y)); }

__device__ __forceinline__ h16 h_min(h16 a, h16 b) { return b < a ? b : a; }
__device__ __forceinline__ h16x2 h2_min(h16x2 a, h16x2 b) { return h2(h_min(a.x, b.x), h_min(a.y, b.y)); }
__device__ __forceinline__ h16 h_relu(h16 x) { return x > (h16)0 ? x : (h16)0; }
__device__ __forceinline__ h16x2 h2_relu(h16x2 x) { return h2(h_relu(x.x), h_relu(x.y)); }
__device__ __forceinline__ h16 h_sat(h16 x) { return x > (h16)0 ? (x < (h16)1 ? x : (h16)1) : (h16)0; }

}  // namespace tgs
