// Device self tests: the deterministic exp/log evaluated on the GPU (checked
// bit for bit against the CPU oracle's copy) and the wave64 DPP primitives
// (checked against plain host arithmetic).
#include "common.h"
#include "kernels.h"

namespace tgs {

__global__ void detmath_kernel(int op, const float* in, float* out, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float x = in[i];
    float y;
    switch (op) {
        case 0: y = det_expf(x); break;
        case 1: y = det_logf(x); break;
        case 2: y = det_expf_nonpos(x <= 0.f ? x : -x); break;
        case 3: y = x / (x * 0.7f + 1.3f); break;       // correctly rounded division
        case 4: y = __builtin_sqrtf(x); break;           // correctly rounded sqrt
        case 5: y = __half2float(__float2half_rn(x)); break;
        case 6: y = det_exp2_core(x); break;   // -150 <= x <= 0
        default: y = 0.f; break;
    }
    out[i] = y;
}

void launch_detmath(int op, const float* in, float* out, int64_t n, hipStream_t s) {
    if (n <= 0) return;
    detmath_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(op, in, out, n);
}

// One wave of 64 inputs -> out[0..63] inclusive scan, out[64] sum,
// out[65] max, out[66] float-sum of (float)in as bits, out[67] lane id check.
__global__ void wave_selftest_kernel(const uint32_t* in, uint32_t* out) {
    const uint32_t lane = lane_id();
    const uint32_t v = in[lane];
    const uint32_t scan = wave_inclusive_scan_u32(v);
    out[lane] = scan;
    const uint32_t sum = wave_sum_u32(v);
    const uint32_t mx = wave_max_u32(v);
    const float fs = wave_sum_row3((float)v);
    const float fs63 = readlane_f32(fs, 63);
    const uint64_t m = ballot((v & 1u) != 0u);
    const uint32_t rank = mask_rank(m);
    out[128 + lane] = rank;
    // transposed 12-value reduction: value q of lane L = in[(L + 5 q) & 63] + q
    float vv[12], t[3];
    for (int q = 0; q < 12; ++q) vv[q] = (float)(in[(lane + 5u * (uint32_t)q) & 63u] + (uint32_t)q);
    wave_reduce12(vv, t);
    if ((lane & 15u) == 0u) {
        const uint32_t row = lane >> 4;
        for (int m = 0; m < 3; ++m) out[192 + 4 * m + row_value((uint32_t)row)] = f2u(t[m]);
    }
    if (lane == 0) {
        out[64] = sum;
        out[65] = mx;
        out[66] = f2u(fs63);
        out[67] = (uint32_t)__builtin_popcountll(m);
    }
}

void launch_wave_selftest(const uint32_t* in, uint32_t* out, hipStream_t s) {
    wave_selftest_kernel<<<1, 64, 0, s>>>(in, out);
}

}  // namespace tgs

#include "halfmath.h"

namespace tgs {

// Canonical half operations on element i: a, b, c are half bit patterns
// (op 7, 8: a holds floats; op 11: a holds int64; op 14: doubles), out
// receives the result's bits. Op 12 checks the lane layout of DPP
// wave_shr:1 (whole waves: n a multiple of 64); op 13 is the packed exp2,
// one lane per element.
__global__ void halfmath_kernel(int op, const uint16_t* a, const uint16_t* b, const uint16_t* c, uint16_t* out,
                                int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const h16 x = hfrom(a[i]);
    h16 r = (h16)0;
    switch (op) {
        case 0: r = h_exp2(x); break;
        case 1: r = __builtin_elementwise_exp2(x); break;   // v_exp_f16 (measured, not canonical)
        case 2: r = h_fma(x, hfrom(b[i]), hfrom(c[i])); break;
        case 3: r = x * hfrom(b[i]); break;
        case 4: r = x + hfrom(b[i]); break;
        case 5: r = h_div(x, hfrom(b[i])); break;
        case 6: {   // packed: lanes (a, b) * (b, c) + (c, a)
            const h16x2 p = h2_fma(h2(x, hfrom(b[i])), h2(hfrom(b[i]), hfrom(c[i])), h2(hfrom(c[i]), x));
            r = (i & 1) ? p.y : p.x;
            break;
        }
        case 7: r = h_rn(((const float*)a)[i]); break;
        case 8: r = h_rd(((const float*)a)[i]); break;
        case 9: r = x - hfrom(b[i]); break;
        case 10: r = h_min(x, hfrom(b[i])); break;
        case 11: r = h_rn(half_of_fixed(((const int64_t*)a)[i])); break;   // exact: the value is a half
        case 12: {   // DPP wave_shr:1 of a: lane l receives lane l - 1's value, lane 0 keeps b
            const uint32_t v = __builtin_amdgcn_update_dpp((uint32_t)b[i], (uint32_t)a[i], 0x138, 0xf, 0xf, false);
            r = hfrom((uint16_t)v);
            break;
        }
        case 14: r = h_rn(half_of_double_sum(((const double*)a)[i])); break;   // exact: the value is a half
        case 13: {   // packed exp2 of lanes (a, b): element i takes lane i & 1
            const h16x2 p = h2_exp2(h2(x, hfrom(b[i])));
            r = (i & 1) ? p.y : p.x;
            break;
        }
        default: break;
    }
    out[i] = hbits(r);
}

void launch_halfmath(int op, const uint16_t* a, const uint16_t* b, const uint16_t* c, uint16_t* out, int64_t n,
                     hipStream_t s) {
    if (n <= 0) return;
    halfmath_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(op, a, b, c, out, n);
}

// Exhaustive check of h_div: every pair (a, b) of half bit patterns with a
// finite, b finite and nonzero. q = h_div(a, b) is correctly rounded iff no
// half lies nearer to a / b (ties: q even), i.e. |a - q b| <= |a - q' b| for
// both neighbours q' of q (exact double residuals: fma of halves), with the
// overflow (|a / b| >= 65520 -> inf) and underflow (|a / b| <= 2^-25 -> 0)
// ends checked directly. out[0] mismatches, out[1] pairs checked, out[2..4]
// a, b, q of one mismatch.
__device__ __forceinline__ double hd(uint16_t h) { return (double)(float)hfrom(h); }

__global__ void __launch_bounds__(256) half_div_check_kernel(unsigned long long* out) {
    const uint32_t t = blockIdx.x * 256u + threadIdx.x;   // 2^24 threads
    const uint16_t a = (uint16_t)(t >> 8);
    unsigned long long checked = 0, bad = 0;
    if ((a & 0x7c00u) != 0x7c00u) {
        const double da = hd(a);
        for (uint32_t k = 0; k < 256; ++k) {
            const uint16_t b = (uint16_t)(((t & 255u) << 8) | k);
            if ((b & 0x7c00u) == 0x7c00u || (b & 0x7fffu) == 0u) continue;
            const double db = hd(b);
            const uint16_t q = hbits(h_div(hfrom(a), hfrom(b)));
            ++checked;
            const uint16_t mag = (uint16_t)(q & 0x7fffu);
            const bool neg = ((a ^ b) & 0x8000u) != 0u;
            bool ok;
            const double ax = __builtin_fabs(da), bx = __builtin_fabs(db);
            if (da == 0.0) {
                ok = mag == 0u && (((q & 0x8000u) != 0u) == neg);
            } else if (mag == 0x7c00u) {   // infinity
                ok = ax >= 65520.0 * bx && (((q & 0x8000u) != 0u) == neg);
            } else if (mag > 0x7c00u) {    // NaN
                ok = false;
            } else if (mag == 0u) {
                ok = ax <= 0x1p-25 * bx && (((q & 0x8000u) != 0u) == neg);
            } else {
                ok = (((q & 0x8000u) != 0u) == neg);
                const double dq = (double)(float)hfrom(mag);
                const double r0 = __builtin_fabs(__builtin_fma(-dq, bx, ax));
                const double dlo = (double)(float)hfrom((uint16_t)(mag - 1u));
                const double rlo = __builtin_fabs(__builtin_fma(-dlo, bx, ax));
                // above the largest finite half the next value is 65536 (rounds to infinity)
                const double dhi = mag == 0x7bffu ? 65536.0 : (double)(float)hfrom((uint16_t)(mag + 1u));
                const double rhi = __builtin_fabs(__builtin_fma(-dhi, bx, ax));
                const bool even = (mag & 1u) == 0u;
                if (r0 > rlo || r0 > rhi) ok = false;
                if ((r0 == rlo || r0 == rhi) && !even) ok = false;
            }
            if (!ok) {
                if (bad == 0 && atomicAdd(&out[5], 1ull) == 0ull) {
                    out[2] = a;
                    out[3] = b;
                    out[4] = q;
                }
                ++bad;
            }
        }
    }
    if (bad) atomicAdd(&out[0], bad);
    atomicAdd(&out[1], checked);
}

void launch_half_div_check(unsigned long long* out, hipStream_t s) {
    half_div_check_kernel<<<65536u, 256, 0, s>>>(out);
}

// h2_div_blend against h_div (itself checked over all pairs above) for every
// half a and every positive b with bits in [blo, bhi], in both lanes (the low
// lane divides a, the high lane a ^ 1, so each lane sees every dividend), and
// v_rcp_f16 against h_div(1, b) for those b. out: [0] quotient mismatches,
// [1] reciprocal mismatches, [2..4] a, b, quotient of one mismatch, [5] claim
// flag.
__global__ void __launch_bounds__(256) half_div_blend_check_kernel(unsigned long long* out, uint32_t blo,
                                                                   uint32_t bhi) {
    const uint64_t t = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    const bool on = t < 65536ull * (bhi - blo + 1u);
    const uint16_t a = (uint16_t)(t & 0xffffu);
    const uint16_t b = (uint16_t)(blo + (uint32_t)(t >> 16));
    bool rbad = false, bad = false;
    if (on) {
        if (a == 0u) rbad = hbits(__builtin_amdgcn_rcph(hfrom(b))) != hbits(h_div((h16)1.0f, hfrom(b)));
        const uint16_t a1 = (uint16_t)(a ^ 1u);
        const h16x2 q2 = h2_div_blend(h2(hfrom(a), hfrom(a1)), h2s(hfrom(b)));
        const bool bad0 = hbits(q2.x) != hbits(h_div(hfrom(a), hfrom(b)));
        const bool bad1 = hbits(q2.y) != hbits(h_div(hfrom(a1), hfrom(b)));
        bad = bad0 || bad1;
        if (bad && atomicAdd(&out[5], 1ull) == 0ull) {
            out[2] = bad0 ? a : a1;
            out[3] = b;
            out[4] = bad0 ? hbits(q2.x) : hbits(q2.y);
        }
    }
    const unsigned long long nbad = __popcll(__ballot(bad)), nr = __popcll(__ballot(rbad));
    if ((threadIdx.x & 63u) == 0u) {
        if (nbad) atomicAdd(&out[0], nbad);
        if (nr) atomicAdd(&out[1], nr);
    }
}

void launch_half_div_blend_check(unsigned long long* out, uint32_t blo, uint32_t bhi, hipStream_t s) {
    const uint64_t n = 65536ull * (bhi - blo + 1u);
    half_div_blend_check_kernel<<<(unsigned)((n + 255u) / 256u), 256, 0, s>>>(out, blo, bhi);
}

// The shader clock under a VALU load: each lane runs eight independent
// chains of packed-half fmas, and wave 0 of each workgroup reads the shader
// clock counter (s_memtime) and the constant-rate counter (s_memrealtime)
// before and after; out[2 b] and out[2 b + 1] are workgroup b's differences.
__global__ void __launch_bounds__(256) clock_probe_kernel(unsigned long long* out, uint32_t iters, float seed) {
    h16x2 a[8];
#pragma unroll
    for (int c = 0; c < 8; ++c)
        a[c] = h2((h16)(seed * (float)(threadIdx.x + c) * 1e-4f), (h16)(-seed * (float)c * 1e-3f));
    const h16x2 q = h2s((h16)0.25f);
    __syncthreads();
    const unsigned long long t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
    for (uint32_t i = 0; i < iters; ++i) {
#pragma unroll
        for (int c = 0; c < 8; ++c) a[c] = h2_fma(a[c], a[c], q);
    }
    float sum = 0.f;
#pragma unroll
    for (int c = 0; c < 8; ++c) sum += (float)a[c].x + (float)a[c].y;
    const unsigned long long t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
    if (threadIdx.x == 0u) {
        out[2u * blockIdx.x] = t1 - t0;
        out[2u * blockIdx.x + 1u] = r1 - r0;
    }
    if (sum == 12345.0f) out[0] = 0ull;   // keeps the chains
}

void launch_clock_probe(unsigned long long* out, uint32_t blocks, uint32_t iters, hipStream_t s) {
    clock_probe_kernel<<<blocks, 256, 0, s>>>(out, iters, 1.0f);
}

}  // namespace tgs
