// Shared device helpers for the gfx950 (CDNA4, wave64) kernels.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "detmath.h"

namespace tgs {

constexpr int kWave = 64;
constexpr int kTile = 16;               // screen tile edge (rasterization_config.h:31-35)
constexpr int kTilePixels = 256;
constexpr int kBucket = 32;            // Gaussians per backward checkpoint bucket (kernels_forward.cuh:644-653)
constexpr float kMinAlpha = 1.0f / 255.0f;
constexpr float kMaxAlpha = 0.999f;
constexpr float kTransmittanceMin = 1e-4f;
constexpr float kDilation = 0.3f;
constexpr float kLog2eF = 0x1.715476p+0f;      // log2(e) as float
constexpr float kHalfLog2e = 0x1.715476p-1f;   // log2(e) / 2 (exact)
constexpr int kGradStride = 12;         // floats of per-primitive 2D gradient record

// v as computed, hidden from instruction selection. A float fma or multiply
// followed by a conversion to half is otherwise fused into v_fma_mixlo_f16 /
// v_fma_mixhi_f16, which round the exact value to half once; the source (and
// the reference, whose float fmaf result is then converted) rounds to float
// first, and the two differ where the float result lands on a half midpoint
// (1 + 2^-11 + 2^-34 gives 1 through float, 1 + 2^-10 directly).
__device__ __forceinline__ float f32_opaque(float v) {
    asm("" : "+v"(v));
    return v;
}
// float -> __half to nearest even of the float value as computed
__device__ __forceinline__ __half f2h_rn(float v) { return __float2half_rn(f32_opaque(v)); }

// Camera and image parameters, passed to kernels by value (no pose-block copy).
struct CamParams {
    float fx, fy, cx, cy, near_, far_;
    float r1[4], r2[4], r3[4];   // rows 0..2 of the row-major world-to-camera matrix
    float cam_pos[3];
    float w, h;                  // image size as float (frustum clamp)
    // frustum clamp of the projected mean (kernels_forward.cuh:231-236), in
    // float on the host: (-0.15 w - cx) / fx, (1.15 w - cx) / fx,
    // (-0.15 h - cy) / fy, (1.15 h - cy) / fy
    float clip_left, clip_right, clip_top, clip_bottom;
    uint32_t width, height;
    uint32_t grid_w, grid_h;     // 16x16 tiles
    uint32_t tiled_w, tiled_h;   // 8x8 image blocks
};

// Physical index of pixel (row, col) in one plane of the 8x8-tiled layout
// (tinygs/include/tinygs/common.hpp:404-408).
TGS_HD uint32_t tiled_index(uint32_t row, uint32_t col, uint32_t tiled_width) {
    return ((((row >> 3) * tiled_width) + (col >> 3)) << 6) + ((row & 7u) << 3) + (col & 7u);
}

__device__ __forceinline__ uint32_t lane_id() { return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)); }

// Orders this wave's LDS accesses before and after the call (a wave's own
// LDS operations need no workgroup barrier).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// number of set bits of a 64-bit lane mask strictly below this lane
__device__ __forceinline__ uint32_t mask_rank(uint64_t m) {
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

__device__ __forceinline__ uint64_t ballot(bool p) { return __ballot(p); }

__device__ __forceinline__ uint32_t readlane_u32(uint32_t v, uint32_t lane) {
    return (uint32_t)__builtin_amdgcn_readlane((int)v, (int)lane);
}
__device__ __forceinline__ float readlane_f32(float v, uint32_t lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), (int)lane));
}

// DPP move: lanes whose source is disabled (row_mask / bank_mask) read 0.
template <int CTRL, int ROW_MASK = 0xF, int BANK_MASK = 0xF>
__device__ __forceinline__ float dpp_f32(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK,
                                                                 BANK_MASK, false));
}
// DPP row rotation (row_ror:n, CTRL 0x121..0x12F): every source lane is
// valid, so bound_ctrl changes nothing and spares the zero "old" operand.
template <int CTRL>
__device__ __forceinline__ float dpp_ror_f32(float v) {
    static_assert(CTRL >= 0x121 && CTRL <= 0x12F, "row_ror only");
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
template <int CTRL, int ROW_MASK = 0xF, int BANK_MASK = 0xF>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROW_MASK, BANK_MASK, false);
}

// Wave-wide sum; the total is valid in lanes 48..63 (row 3), read lane 63.
// Row butterfly with row_ror 8/4/2/1, then row_bcast15 / row_bcast31 across
// the four 16-lane rows. Fixed order: deterministic for a given input.
__device__ __forceinline__ float wave_sum_row3(float v) {
    v += dpp_f32<0x128>(v);        // row_ror:8
    v += dpp_f32<0x124>(v);        // row_ror:4
    v += dpp_f32<0x122>(v);        // row_ror:2
    v += dpp_f32<0x121>(v);        // row_ror:1
    v += dpp_f32<0x142, 0xA>(v);   // row_bcast:15 -> rows 1, 3
    v += dpp_f32<0x143, 0xC>(v);   // row_bcast:31 -> rows 2, 3
    return v;
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, dpp_u32<0x128>(v));
    v = max(v, dpp_u32<0x124>(v));
    v = max(v, dpp_u32<0x122>(v));
    v = max(v, dpp_u32<0x121>(v));
    v = max(v, dpp_u32<0x142, 0xA>(v));
    v = max(v, dpp_u32<0x143, 0xC>(v));
    return readlane_u32(v, 63);
}

// Workgroups are dispatched in linear-id order, round-robin over the 8
// XCDs (each with its own L2). This maps the dispatch index to a work index
// so that XCD x receives one contiguous run of work indices: neighbouring
// tiles then share an L2 and their halos are re-read from it, not from HBM.
// A bijection on [0, n).
__device__ __forceinline__ uint32_t xcd_contiguous_index(uint32_t linear, uint32_t n) {
    constexpr uint32_t kXcds = 8;
    const uint32_t per = n / kXcds, rem = n % kXcds;
    const uint32_t x = linear % kXcds, j = linear / kXcds;
    return x * per + min(x, rem) + j;
}

__device__ __forceinline__ uint32_t wave_or_u32(uint32_t v) {
    v |= dpp_u32<0x128>(v);
    v |= dpp_u32<0x124>(v);
    v |= dpp_u32<0x122>(v);
    v |= dpp_u32<0x121>(v);
    v |= dpp_u32<0x142, 0xA>(v);
    v |= dpp_u32<0x143, 0xC>(v);
    return readlane_u32(v, 63);
}

__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
    v += dpp_u32<0x128>(v);
    v += dpp_u32<0x124>(v);
    v += dpp_u32<0x122>(v);
    v += dpp_u32<0x121>(v);
    v += dpp_u32<0x142, 0xA>(v);
    v += dpp_u32<0x143, 0xC>(v);
    return readlane_u32(v, 63);
}

// Inclusive prefix sum across the wave (Hillis-Steele with ds_bpermute-free
// DPP row shifts plus row broadcasts).
__device__ __forceinline__ uint32_t wave_inclusive_scan_u32(uint32_t v) {
    v += dpp_u32<0x111>(v);          // row_shr:1
    v += dpp_u32<0x112>(v);          // row_shr:2
    v += dpp_u32<0x114>(v);          // row_shr:4
    v += dpp_u32<0x118>(v);          // row_shr:8
    v += dpp_u32<0x142, 0xA>(v);     // row_bcast:15
    v += dpp_u32<0x143, 0xC>(v);     // row_bcast:31
    return v;
}

// gfx950 cross-half swaps (v_permlane32_swap / v_permlane16_swap):
//   swap32(a, b) -> (x, y) with x = [a.lanes 0-31, b.lanes 0-31],
//                            y = [a.lanes 32-63, b.lanes 32-63];
//   swap16(a, b) -> (x, y) with x = rows (a0, b0, a2, b2), y = (a1, b1, a3, b3)
// (rows = 16-lane groups).
__device__ __forceinline__ void swap32(float& a, float& b) {
    auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b), false,
                                              false);
    a = __builtin_bit_cast(float, (uint32_t)r[0]);
    b = __builtin_bit_cast(float, (uint32_t)r[1]);
}
__device__ __forceinline__ void swap16(float& a, float& b) {
    auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b), false,
                                              false);
    a = __builtin_bit_cast(float, (uint32_t)r[0]);
    b = __builtin_bit_cast(float, (uint32_t)r[1]);
}

// Transposed wave reduction of 12 per-lane values v[0..11] into 12 wave sums.
// After the call, lane L of t[m] holds the sum of value 4m + row_value(L >> 4)
// (every lane of a 16-lane row holds the same total).
//   step 1: swap32 + add folds value pairs across the two 32-lane halves,
//   step 2: swap16 + add folds the results across rows 0/1 and 2/3,
//   step 3: row butterfly (row_ror 8, 4, 2, 1) on the three survivors.
// 6 + 3 swaps, 9 adds and 12 DPP adds instead of 12 x 6 dependent DPP adds.
// Value offset held by 16-lane row r after the swaps: rows 0..3 -> 0, 2, 1, 3.
// Arithmetic on purpose: a lane-indexed constant table becomes a global
// memory load inside the caller's loop.
__device__ __forceinline__ int row_value(uint32_t row) { return (int)(((row & 1u) << 1) | (row >> 1)); }
__device__ __forceinline__ void wave_reduce12(float v[12], float t[3]) {
#pragma unroll
    for (int k = 0; k < 6; ++k) {
        float a = v[2 * k], b = v[2 * k + 1];
        swap32(a, b);
        v[k] = a + b;   // lanes 0-31: value 2k, lanes 32-63: value 2k+1 (half sums)
    }
#pragma unroll
    for (int m = 0; m < 3; ++m) {
        float a = v[2 * m], b = v[2 * m + 1];
        swap16(a, b);
        t[m] = a + b;   // rows: values 4m, 4m+2, 4m+1, 4m+3 (quarter sums)
    }
#pragma unroll
    for (int m = 0; m < 3; ++m) t[m] += dpp_ror_f32<0x128>(t[m]);
#pragma unroll
    for (int m = 0; m < 3; ++m) t[m] += dpp_ror_f32<0x124>(t[m]);
#pragma unroll
    for (int m = 0; m < 3; ++m) t[m] += dpp_ror_f32<0x122>(t[m]);
#pragma unroll
    for (int m = 0; m < 3; ++m) t[m] += dpp_ror_f32<0x121>(t[m]);
}

// Two Gaussians' 9 values at once (v[0..8] and v[9..17]): lane L of t[m]
// (m < 5) holds the sum of value 4m + row_value(L >> 4) (values 18 and 19
// are zero). 9 + 5 swaps, 14 adds and 20 DPP adds: 48 against 2 x 28.
__device__ __forceinline__ void wave_reduce18(float v[18], float t[5]) {
#pragma unroll
    for (int k = 0; k < 9; ++k) {
        float a = v[2 * k], b = v[2 * k + 1];
        swap32(a, b);
        v[k] = a + b;   // lanes 0-31: value 2k, lanes 32-63: value 2k+1 (half sums)
    }
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        float a = v[2 * m], b = v[2 * m + 1];
        swap16(a, b);
        t[m] = a + b;   // rows: values 4m, 4m+2, 4m+1, 4m+3 (quarter sums)
    }
    {
        float a = v[8], b = 0.f;
        swap16(a, b);
        t[4] = a + b;   // rows: values 16, 18 (zero), 17, 19 (zero)
    }
#pragma unroll
    for (int m = 0; m < 5; ++m) t[m] += dpp_ror_f32<0x128>(t[m]);
#pragma unroll
    for (int m = 0; m < 5; ++m) t[m] += dpp_ror_f32<0x124>(t[m]);
#pragma unroll
    for (int m = 0; m < 5; ++m) t[m] += dpp_ror_f32<0x122>(t[m]);
#pragma unroll
    for (int m = 0; m < 5; ++m) t[m] += dpp_ror_f32<0x121>(t[m]);
}

// wave_reduce12 for v[9..11] == 0 on every lane: the same layout of t, with
// the swaps and adds that would only move zeros left out.
__device__ __forceinline__ void wave_reduce9(float v[12], float t[3]) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        float a = v[2 * k], b = v[2 * k + 1];
        swap32(a, b);
        v[k] = a + b;
    }
    {
        float a = v[8], b = 0.f;
        swap32(a, b);
        v[4] = a + b;   // lanes 0-31: value 8, lanes 32-63: zero (value 9)
    }
#pragma unroll
    for (int m = 0; m < 2; ++m) {
        float a = v[2 * m], b = v[2 * m + 1];
        swap16(a, b);
        t[m] = a + b;
    }
    {
        float a = v[4], b = 0.f;
        swap16(a, b);
        t[2] = a + b;   // row values 8, 10, 9, 11: only value 8 is nonzero
    }
#pragma unroll
    for (int m = 0; m < 3; ++m) t[m] += dpp_ror_f32<0x128>(t[m]);
#pragma unroll
    for (int m = 0; m < 3; ++m) t[m] += dpp_ror_f32<0x124>(t[m]);
#pragma unroll
    for (int m = 0; m < 3; ++m) t[m] += dpp_ror_f32<0x122>(t[m]);
#pragma unroll
    for (int m = 0; m < 3; ++m) t[m] += dpp_ror_f32<0x121>(t[m]);
}

// Exclusive scan of R striped values per thread over a workgroup of NW
// waves (R NW <= 64): value r of thread t is element r * 64 NW + t of the
// workgroup's chunk, so consecutive lanes hold consecutive elements in every
// round. s_rw: R NW words of LDS.
template <int R, int NW = 4>
__device__ __forceinline__ void striped_scan_u32(const uint32_t v[R], uint32_t ex[R], uint32_t* total,
                                                 uint32_t* s_rw) {
    static_assert(R >= 1 && R * NW <= 64, "at most 64 (round, wave) partial sums");
    const uint32_t lane = threadIdx.x & 63u, w = threadIdx.x >> 6;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t incl = wave_inclusive_scan_u32(v[r]);
        ex[r] = incl - v[r];
        if (lane == 63u) s_rw[r * NW + w] = incl;
    }
    __syncthreads();
    // (round, wave) partial sums in element order; every wave scans them itself
    const uint32_t x = lane < (uint32_t)(NW * R) ? s_rw[lane] : 0u;
    const uint32_t xi = wave_inclusive_scan_u32(x);
    *total = readlane_u32(xi, 63);
    const uint32_t xe = xi - x;
#pragma unroll
    for (int r = 0; r < R; ++r) ex[r] += readlane_u32(xe, (uint32_t)(r * NW) + w);
    __syncthreads();   // s_rw may be reused after this
}
__device__ __forceinline__ void striped_scan16_u32(const uint32_t v[16], uint32_t ex[16], uint32_t* total,
                                                   uint32_t* s_rw) {
    striped_scan_u32<16>(v, ex, total, s_rw);
}

template <typename T>
__device__ __forceinline__ float load_as_float(const T* p, int64_t i);
template <>
__device__ __forceinline__ float load_as_float<float>(const float* p, int64_t i) { return p[i]; }
template <>
__device__ __forceinline__ float load_as_float<__half>(const __half* p, int64_t i) { return __half2float(p[i]); }

}  // namespace tgs
