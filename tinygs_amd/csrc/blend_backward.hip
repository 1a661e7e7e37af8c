// Backward of the blend, one 16x16 tile per workgroup, pixel-parallel.
//
// Reference: blend_backward_cu2 (tinygs/src/rasterizer/fastgs_ours/
// kernels_backward.cuh:675-927) assigns one warp per 32-Gaussian bucket,
// restarts each bucket from a (colour, transmittance) checkpoint written by
// the forward, and pipelines the 256 pixels through the lanes.
//
// MI355X design: a wave64 owns an 8x8 image block (one contiguous 256-byte
// run per plane), every lane one pixel. The workgroup walks the tile's
// Gaussians front to back; each pixel
//   * re-runs the forward recurrence (alpha >= 1/255 test, sigma < 0 skip) to
//     obtain the checkpoint state at every 32-Gaussian boundary, so the
//     forward stores no checkpoints (saves 2 x 128 B of HBM per instance);
//   * runs the reference backward recurrence inside each bucket (sigma
//     clamped at 0, no 1/255 test, state restarted at the bucket boundary),
//     which keeps the reference's bucket semantics exactly.
// Per-Gaussian gradient sums (11 values) are reduced across the wave with a
// transposed reduction (gfx950 v_permlane32_swap / v_permlane16_swap, then a
// DPP row butterfly; fixed order), the four waves' partials combined in LDS,
// and one float atomic per value and tile is issued to the per-primitive
// record.
//
// grad2d record (12 floats per primitive): [0,1] dL/dmean2d, [2,3] |.| sums
// (absgrad), [4..6] dL/dconic (a, b, c), [7..9] dL/dcolour (masked by
// colour >= 0), [10] sum of alpha * dL/dalpha (times (1 - opacity) later).
#include "common.h"
#include "kernels.h"

namespace tgs {

constexpr int kBwdBatch = 64;
constexpr int kBwdVals = 11;

__global__ void __launch_bounds__(256) blend_backward_kernel(
    CamParams cam, const uint2* __restrict__ ranges, const uint32_t* __restrict__ inst_vals,
    const float2* __restrict__ mean2d, const float4* __restrict__ conic_opacity, const float4* __restrict__ color_pt,
    const float* __restrict__ image, const float* __restrict__ grad_image, const uint32_t* __restrict__ n_contrib,
    const uint32_t* __restrict__ tile_max, float* __restrict__ grad2d, unsigned long long* __restrict__ stats) {
    __shared__ float4 s_a[kBwdBatch];   // mx, my, a/2, b
    __shared__ float4 s_b[kBwdBatch];   // c/2, opacity, a, c
    __shared__ float4 s_c[kBwdBatch];   // clamped colour, colour >= 0 mask bits
    __shared__ uint32_t s_p[kBwdBatch];
    __shared__ float s_part[4][kBwdVals][kBwdBatch];
    __shared__ uint32_t s_wmax[4];

    const uint32_t tile = blockIdx.x;
    const uint2 range = ranges[tile];
    const int32_t len = (int32_t)(range.y - range.x);
    const int32_t nproc = min(len, (int32_t)tile_max[tile]);
    if (nproc <= 0) return;
    if (stats && threadIdx.x == 0) atomicAdd(stats, (unsigned long long)nproc);

    const uint32_t gx = tile % cam.grid_w, gy = tile / cam.grid_w;
    const uint32_t tid = threadIdx.x, w = tid >> 6, lane = tid & 63u;
    const uint32_t px = gx * 16u + (w & 1u) * 8u + (lane & 7u);
    const uint32_t py = gy * 16u + (w >> 1) * 8u + (lane >> 3);
    const bool inside = px < cam.width && py < cam.height;
    const float pcx = (float)px + 0.5f, pcy = (float)py + 0.5f;

    float I0 = 0.f, I1 = 0.f, I2 = 0.f, g0 = 0.f, g1 = 0.f, g2 = 0.f;
    uint32_t last = 0;
    if (inside) {
        const uint32_t cs = cam.tiled_w * cam.tiled_h * 64u;
        const uint32_t pi = tiled_index(py, px, cam.tiled_w);
        I0 = image[pi]; I1 = image[pi + cs]; I2 = image[pi + 2 * cs];
        g0 = grad_image[pi]; g1 = grad_image[pi + cs]; g2 = grad_image[pi + 2 * cs];
        last = n_contrib[pi];
    }
    const uint32_t wmax = wave_max_u32(last);
    if (lane == 0) s_wmax[w] = wmax;

    // forward state (checkpoint source) and bucket-local backward state
    float Tf = 1.f, F0 = 0.f, F1 = 0.f, F2 = 0.f;
    float Tb = 1.f, A0 = 0.f, A1 = 0.f, A2 = 0.f;

    for (int32_t base = 0; base < nproc; base += kBwdBatch) {
        const int32_t nb = min(kBwdBatch, nproc - base);
        if ((int32_t)tid < nb) {
            const uint32_t p = inst_vals[range.x + (uint32_t)(base + (int32_t)tid)];
            const float2 m = mean2d[p];
            const float4 co = conic_opacity[p];
            const float4 c = color_pt[p];
            s_p[tid] = p;
            s_a[tid] = make_float4(m.x, m.y, 0.5f * co.x, co.y);
            s_b[tid] = make_float4(0.5f * co.z, co.w, co.x, co.z);
            const uint32_t mask = (c.x >= 0.f ? 1u : 0u) | (c.y >= 0.f ? 2u : 0u) | (c.z >= 0.f ? 4u : 0u);
            s_c[tid] = make_float4(__builtin_fmaxf(c.x, 0.f), __builtin_fmaxf(c.y, 0.f), __builtin_fmaxf(c.z, 0.f),
                                   u2f(mask));
        }
        __syncthreads();
        const int32_t wend = min(nb, max(0, (int32_t)wmax - base));
        for (int32_t k = 0; k < wend; ++k) {
            const int32_t j = base + k;
            if ((j & 31) == 0) {
                Tb = Tf;
                A0 = I0 - F0; A1 = I1 - F1; A2 = I2 - F2;
            }
            const bool act = (uint32_t)j < last;
            const float4 a = s_a[k];
            const float4 b = s_b[k];
            const float4 c = s_c[k];
            const float dx = a.x - pcx, dy = a.y - pcy;
            const float sigma = __builtin_fmaf(dx, __builtin_fmaf(a.z, dx, a.w * dy), (b.x * dy) * dy);
            const float G = det_expf_nonpos(-__builtin_fmaxf(sigma, 0.f));
            const float araw = b.y * G;
            // forward recurrence (bit-identical to blend_forward for j < last)
            if (act && sigma >= 0.f) {
                const float af = __builtin_fminf(araw, kMaxAlpha);
                if (af >= kMinAlpha) {
                    const float nT = Tf * (1.0f - af);
                    const float wf = Tf * af;
                    F0 = __builtin_fmaf(wf, c.x, F0);
                    F1 = __builtin_fmaf(wf, c.y, F1);
                    F2 = __builtin_fmaf(wf, c.z, F2);
                    Tf = nT;
                }
            }
            // reference backward step (kernels_backward.cuh:839-902)
            const float ab = act ? __builtin_fminf(araw, kMaxAlpha) : 0.f;
            const float wgt = Tb * ab;
            float v[12];
            v[0] = wgt * g0;
            v[1] = wgt * g1;
            v[2] = wgt * g2;
            A0 -= wgt * c.x;
            A1 -= wgt * c.y;
            A2 -= wgt * c.z;
            const float cg = c.x * g0 + c.y * g1 + c.z * g2;
            const float ag = A0 * g0 + A1 * g1 + A2 * g2;
            const float oma = 1.0f - ab;
            const float dalpha = Tb * cg - ag * __builtin_amdgcn_rcpf(oma);
            const float pp = ab * dalpha;
            const float hp = -0.5f * pp;
            v[3] = pp;
            v[4] = hp * (dx * dx);
            v[5] = hp * (dx * dy);
            v[6] = hp * (dy * dy);
            const float gmx = pp * (b.z * dx + a.w * dy);
            const float gmy = pp * (a.w * dx + b.w * dy);
            v[7] = -gmx;
            v[8] = -gmy;
            v[9] = __builtin_fabsf(gmx);
            v[10] = __builtin_fabsf(gmy);
            v[11] = 0.f;
            Tb *= oma;
            float t[3];
            wave_reduce12(v, t);
            if ((lane & 15u) == 0u) {
                const int row = (int)(lane >> 4);
                const int q0 = kRowValue[row];
                s_part[w][q0][k] = t[0];
                s_part[w][4 + q0][k] = t[1];
                if (8 + q0 < kBwdVals) s_part[w][8 + q0][k] = t[2];
            }
        }
        __syncthreads();
        if ((int32_t)tid < nb) {
            const int32_t k = (int32_t)tid;
            float acc[kBwdVals];
#pragma unroll
            for (int q = 0; q < kBwdVals; ++q) acc[q] = 0.f;
            for (int ww = 0; ww < 4; ++ww) {
                const int32_t we = min(nb, max(0, (int32_t)s_wmax[ww] - base));
                if (k < we) {
#pragma unroll
                    for (int q = 0; q < kBwdVals; ++q) acc[q] += s_part[ww][q][k];
                }
            }
            const uint32_t mask = f2u(s_c[k].w);
            if (!(mask & 1u)) acc[0] = 0.f;
            if (!(mask & 2u)) acc[1] = 0.f;
            if (!(mask & 4u)) acc[2] = 0.f;
            float* dst = grad2d + (size_t)s_p[k] * kGradStride;
            // record order: mean2d(2), abs(2), conic(3), colour(3), alpha partial
            const float outv[11] = {acc[7], acc[8], acc[9], acc[10], acc[4], acc[5], acc[6],
                                    acc[0], acc[1], acc[2], acc[3]};
#pragma unroll
            for (int q = 0; q < 11; ++q)
                if (outv[q] != 0.f) unsafeAtomicAdd(dst + q, outv[q]);
        }
        __syncthreads();
    }
}

void launch_blend_backward(const CamParams& cam, const uint2* ranges, const uint32_t* inst_vals, const float2* mean2d,
                           const float4* conic_opacity, const float4* color_pt, const float* image,
                           const float* grad_image, const uint32_t* n_contrib, const uint32_t* tile_max, float* grad2d,
                           unsigned long long* stats, hipStream_t s) {
    const uint32_t n_tiles = cam.grid_w * cam.grid_h;
    if (n_tiles == 0) return;
    blend_backward_kernel<<<n_tiles, 256, 0, s>>>(cam, ranges, inst_vals, mean2d, conic_opacity, color_pt, image,
                                                  grad_image, n_contrib, tile_max, grad2d, stats);
}

}  // namespace tgs
