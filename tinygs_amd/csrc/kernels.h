// Host-side launchers of the HIP kernels (internal C++ interface of the library).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"

namespace tgs {

enum ShDtype : int { kShF32 = 0, kShF16 = 1 };

struct GaussianView {
    const float* means;
    const float* scales;
    const float* rotations;
    const float* opacities;
    const void* sh0;
    const void* sh_rest;
    int64_t n;
    int sh_degree;
    int sh_dtype;
};

struct GradView {
    float* means;
    float* scales;
    float* rotations;
    float* opacities;
    float* sh0;
    float* sh_rest;
};

// ---- preprocess (kernels_forward.cuh:157-412)
void launch_preprocess(const GaussianView& g, const CamParams& cam, uint32_t* n_touched, uint2* bounds,
                       float2* mean2d, float4* conic_opacity, float4* color_pt, uint32_t* depth_key,
                       float* densif, hipStream_t s);

// ---- scans / compaction / sort / binning
size_t scan_temp_bytes(int64_t n);
// exclusive scan of (n_touched[i] > 0) over [0, n); writes depth keys and
// indices of visible primitives in index order; *d_count = V.
void launch_compact_visible(const uint32_t* n_touched, const uint32_t* depth_key, int64_t n, uint32_t* keys_out,
                            uint32_t* vals_out, uint32_t* d_count, uint32_t* temp, hipStream_t s);
// offsets[k] = exclusive scan of n_touched[prims[k]] over k < *d_count; *d_total = I.
void launch_instance_offsets(const uint32_t* n_touched, const uint32_t* prims, const uint32_t* d_count,
                             int64_t max_count, uint32_t* offsets, uint32_t* d_total, uint32_t* temp, hipStream_t s);
// Stable LSD radix sort of (key, value) u32 pairs on bits [0, end_bit).
// Ping-pongs between buffers; returns the index (0/1) holding the result.
size_t radix_temp_bytes(int64_t max_n);
int radix_sort_pairs(uint32_t* keys[2], uint32_t* vals[2], const uint32_t* d_n, int64_t max_n, int end_bit,
                     uint32_t* temp, hipStream_t s);
void launch_emit_instances(const uint32_t* n_touched, const uint32_t* prims, const uint32_t* offsets, const uint32_t* d_count, int64_t max_count,
                           const uint2* bounds, const float2* mean2d, const float4* conic_opacity,
                           const float4* color_pt, uint32_t grid_w, uint32_t* inst_keys, uint32_t* inst_vals,
                           hipStream_t s);
void launch_tile_ranges(const uint32_t* inst_keys, int64_t n_inst, uint2* ranges, uint32_t n_tiles, hipStream_t s);

// ---- blend (kernels_forward.cuh:569-715, kernels_backward.cuh:675-927)
void launch_blend_forward(const CamParams& cam, const uint2* ranges, const uint32_t* inst_vals, const float2* mean2d,
                          const float4* conic_opacity, const float4* color_pt, float* image, uint32_t* n_contrib,
                          uint32_t* tile_max, unsigned long long* stats, hipStream_t s);
void launch_blend_backward(const CamParams& cam, const uint2* ranges, const uint32_t* inst_vals,
                           const float2* mean2d, const float4* conic_opacity, const float4* color_pt,
                           const float* image, const float* grad_image, const uint32_t* n_contrib,
                           const uint32_t* tile_max, float* grad2d, unsigned long long* stats, hipStream_t s);

// ---- preprocess backward (kernels_backward.cuh:88-352)
void launch_preprocess_backward(const GaussianView& g, const CamParams& cam, const uint32_t* n_touched,
                                const float4* conic_opacity, const float* grad2d, const GradView& out,
                                float* densif, bool assign, hipStream_t s);

// ---- utilities
void launch_fill_u32(uint32_t* p, uint32_t value, int64_t n, hipStream_t s);

// ---- losses (l1.cu:19-42, fused_ssim.cu:55-442)
void launch_l1(const float* pred, const float* target, float* loss, float* grad, int64_t n_padded, float s,
               hipStream_t st);
void launch_ssim_forward(uint32_t width, uint32_t height, float c1, float c2, float s, const float* pred,
                         const float* target, float* loss, float* dm_mu, float* dm_s1, float* dm_s12, hipStream_t st);
void launch_ssim_backward(uint32_t width, uint32_t height, float s, const float* pred, const float* target,
                          float* grad, const float* dm_mu, const float* dm_s1, const float* dm_s12, hipStream_t st);

// ---- SimpleAdam (simple_adam.cu:104-213, :457-580)
struct AdamGroup {
    void* theta;          // float or half
    const float* grad;
    float* m1;
    float* m2;
    int64_t count;
    float lr;
    int theta_half;       // 1: theta stored as fp16
    int lerp_form;        // 0: fma(t, g - m, m); 1: fma(t, g, fma(-t, m, m))
    int decay_kind;       // 0 none, 1 opacity logistic', 2 scale exp
    float decay_coef;
};
struct AdamArgs {
    AdamGroup groups[6];
    int n_groups;
    float beta1, beta2, eps, grad_scale, bc1, bc2_sqrt, max_grad;
};
void launch_adam(const AdamArgs& a, hipStream_t s);

// ---- self tests of wave primitives and deterministic math (debug entry points)
void launch_detmath(int op, const float* in, float* out, int64_t n, hipStream_t s);
void launch_wave_selftest(const uint32_t* in, uint32_t* out, hipStream_t s);

}  // namespace tgs
