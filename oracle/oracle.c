/* TEST INFRASTRUCTURE — the CPU oracle for the FastGS training path.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load liboracle.so; the product never does.
 *
 * Instantiates oracle_impl.inc twice:
 *   orc_f_*  float, deterministic exp/log, explicit fmaf  (the oracle)
 *   orc_d_*  double, libm exp/log                          (FD checks only)
 *
 * Parity pins (see tests/test_oracle.py):
 *   orc_expf / orc_logf        vs libm double exp/log (ulp bound), special cases
 *   orc_float_to_half_bits     vs numpy float16 (RNE) over a sweep
 *   preprocess                 closed-form EWA in double (conic * cov2d = I),
 *                              rotation invariance, SH constants vs a double
 *                              brute-force real-SH evaluation
 *   tile culling               brute force over pixel centres (no dropped tile
 *                              holds a pixel with alpha >= 1/255)
 *   bin                        numpy stable sort of 64-bit (tile<<32|depth) keys
 *   blend_forward              independent per-pixel numpy loop
 *   blend/preprocess backward  double-precision central differences of the
 *                              orc_d_ forward (exact_grad mode), plus closed-form
 *                              checks of the reference-specific quirks
 *   l1 / ssim                  closed form, FD (double), brute-force convolution
 *   adam                       closed form (Kingma & Ba 2015)
 */
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "detmath.h"
#include "halfmath.h"

/* ---------------- float instance (the oracle) ---------------- */
#define REAL float
#define SFX(name) orc_f_##name
#define R_EXP(x) orc_expf(x)
#define R_LOG(x) orc_logf(x)
#define R_SQRT(x) sqrtf(x)
#define R_FMA(a, b, c) fmaf(a, b, c)
#define R_FLOOR(x) floorf(x)
#define R_CEIL(x) ceilf(x)
#define R_FMIN(a, b) fminf(a, b)
#define R_FMAX(a, b) fmaxf(a, b)
#define R_FABS(a) fabsf(a)
#define R_COPYSIGN(a, b) copysignf(a, b)
#define R_HALF_ROUND(x) orc_round_half(x)
/* the blend forward's sigma in log2 units (conic prescaled by log2 e) and
 * its 2^(-sigma'), clamped at 150 */
#define R_SIG_HALF 0x1.715476p-1f
#define R_SIG_ONE 0x1.715476p+0f
#define R_ALPHA_EXP(s) orc_exp2_core(-fminf((s), 150.0f))
/* the blend forward's accept test: 0 <= sigma' <= thr' with thr' = ln(255 o) L
 * (float product), as one unsigned comparison of the bit patterns (thr' >= 0,
 * and sigma' is never -0 there). alpha >= 1/255 up to rounding at the edge. */
#define R_BLEND_ACCEPT(sigma, alpha, thr) (orc_float_to_bits(sigma) <= orc_float_to_bits((thr) * R_SIG_ONE))
#include "oracle_impl.inc"
#undef REAL
#undef SFX
#undef R_EXP
#undef R_LOG
#undef R_SQRT
#undef R_FMA
#undef R_FLOOR
#undef R_CEIL
#undef R_FMIN
#undef R_FMAX
#undef R_FABS
#undef R_COPYSIGN
#undef R_HALF_ROUND
#undef R_SIG_HALF
#undef R_SIG_ONE
#undef R_ALPHA_EXP
#undef R_BLEND_ACCEPT

/* ---------------- double instance (finite-difference checker) ---------------- */
#define REAL double
#define SFX(name) orc_d_##name
#define R_EXP(x) exp(x)
#define R_LOG(x) log(x)
#define R_SQRT(x) sqrt(x)
#define R_FMA(a, b, c) ((a) * (b) + (c))
#define R_FLOOR(x) floor(x)
#define R_CEIL(x) ceil(x)
#define R_FMIN(a, b) fmin(a, b)
#define R_FMAX(a, b) fmax(a, b)
#define R_FABS(a) fabs(a)
#define R_COPYSIGN(a, b) copysign(a, b)
#define R_HALF_ROUND(x) (x)
#define R_SIG_HALF 0.5
#define R_SIG_ONE 1.0
#define R_ALPHA_EXP(s) exp(-(s))
/* the reference's tests, kernels_forward.cuh:660-665 */
#define R_BLEND_ACCEPT(sigma, alpha, thr) ((sigma) >= 0 && (alpha) >= (REAL)(1.0f / 255.0f))
#include "oracle_impl.inc"

/* ---------------- the fp16-image rasterizer (FGS16), half arithmetic ---------------- */
#include "fgs16_impl.inc"

/* ---------------- exported helpers ---------------- */
void orc_expf_array(int64_t n, const float* x, float* y) { for (int64_t i = 0; i < n; ++i) y[i] = orc_expf(x[i]); }
void orc_logf_array(int64_t n, const float* x, float* y) { for (int64_t i = 0; i < n; ++i) y[i] = orc_logf(x[i]); }
void orc_exp2_core_array(int64_t n, const float* x, float* y) { for (int64_t i = 0; i < n; ++i) y[i] = orc_exp2_core(x[i]); }
void orc_half_bits_array(int64_t n, const float* x, uint16_t* y) { for (int64_t i = 0; i < n; ++i) y[i] = orc_float_to_half_bits(x[i]); }
void orc_round_half_array(int64_t n, const float* x, float* y) { for (int64_t i = 0; i < n; ++i) y[i] = orc_round_half(x[i]); }
/* The canonical half operations of oracle/halfmath.h on arrays of half bit
 * patterns (ops 7, 8 read floats from a), numbered as tgs_selftest_half. */
void orc_half_op_array(int op, int64_t n, const void* a, const uint16_t* b, const uint16_t* c, uint16_t* out) {
    const uint16_t* ah = (const uint16_t*)a;
    const float* af = (const float*)a;
    for (int64_t i = 0; i < n; ++i) {
        uint16_t r = 0;
        switch (op) {
            case 0: r = oh_exp2(ah[i]); break;
            case 2: r = oh_fma(ah[i], b[i], c[i]); break;
            case 3: r = oh_mul(ah[i], b[i]); break;
            case 4: r = oh_add(ah[i], b[i]); break;
            case 5: r = oh_div(ah[i], b[i]); break;
            case 6: r = (i & 1) ? oh_fma(b[i], c[i], ah[i]) : oh_fma(ah[i], b[i], c[i]); break;
            case 7: r = oh_rn(af[i]); break;
            case 8: r = oh_rd(af[i]); break;
            case 9: r = oh_sub(ah[i], b[i]); break;
            case 10: r = oh_min(ah[i], b[i]); break;
            case 11: r = oh_from_fixed(((const int64_t*)a)[i]); break;
            case 12: r = (i & 63) ? ah[i - 1] : b[i]; break;   /* wave_shr:1 of 64-lane waves */
            default: break;
        }
        out[i] = r;
    }
}

int orc_version(void) { return 1; }
/* Threads of the parallel loops (the results do not depend on it). */
void orc_set_threads(int n) { omp_set_num_threads(n > 0 ? n : 1); }
int orc_max_threads(void) { return omp_get_max_threads(); }
