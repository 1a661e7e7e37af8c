// Front-to-back alpha blending, one 16x16 screen tile per workgroup.
// Follows tinygs/src/rasterizer/fastgs_ours/kernels_forward.cuh:569-715.
//
// MI355X mapping: 256 threads = four wave64; wave w owns the 8x8 image block
// (w & 1, w >> 1) of the tile, which is exactly one 64-float run of the 8x8
// tiled image layout, so every image / n_contrib store of a wave is one
// contiguous 256-byte transaction per plane. Gaussians are staged through LDS
// in batches of 256 (one record per thread); a wave stops evaluating as soon
// as all of its 64 pixels have terminated and the workgroup stops fetching
// once all four waves have.
//
// Checkpoints: before Gaussian j of the tile's list with j % 32 == 0, j > 0,
// every still-active wave stores its pixels' (C, T) (kernels_forward.cuh:
// 644-653), one contiguous 1 KiB run per wave. At the end the tile appends one
// backward work item per 32-Gaussian bucket below its last contributor
// (tmax <= len, so every bucket of an item is inside the list).
//
// Numerics mirror the CPU oracle: sigma = fma(dx, fma(a/2, dx, b*dy),
// (c/2)*dy*dy), the deterministic exp, fminf alpha clamp, the 1/255 cut and
// the 1e-4 transmittance stop with the terminating Gaussian not composited.
#include "common.h"
#include "kernels.h"

namespace tgs {

__global__ void __launch_bounds__(256) blend_forward_kernel(CamParams cam, const uint2* __restrict__ ranges,
                                                            const uint32_t* __restrict__ inst_vals,
                                                            const float2* __restrict__ mean2d,
                                                            const float4* __restrict__ conic_opacity,
                                                            const float4* __restrict__ color_pt,
                                                            float* __restrict__ image,
                                                            uint32_t* __restrict__ n_contrib,
                                                            uint32_t* __restrict__ tile_max,
                                                            uint32_t* __restrict__ tile_loaded,
                                                            float4* __restrict__ ckpt,
                                                            uint4* __restrict__ items,
                                                            BinCtl* __restrict__ ctl) {
    __shared__ float4 s_a[256];   // mx, my, a/2, b
    __shared__ float2 s_b[256];   // c/2, opacity
    __shared__ float4 s_c[256];   // r, g, b (clamped), skip bound
    __shared__ uint32_t s_max[4];

    const uint32_t tile = blockIdx.x;
    const uint32_t gx = tile % cam.grid_w, gy = tile / cam.grid_w;
    const uint32_t tid = threadIdx.x, w = tid >> 6, lane = tid & 63u;
    const uint32_t px = gx * 16u + (w & 1u) * 8u + (lane & 7u);
    const uint32_t py = gy * 16u + (w >> 1) * 8u + (lane >> 3);
    const bool inside = px < cam.width && py < cam.height;
    const float pcx = (float)px + 0.5f, pcy = (float)py + 0.5f;

    const uint2 range = ranges[tile];
    const int32_t len = (int32_t)(range.y - range.x);
    const uint32_t slot0 = range.x / (uint32_t)kBucket + tile;   // first checkpoint slot of this tile

    float C0 = 0.f, C1 = 0.f, C2 = 0.f, T = 1.f;
    uint32_t ncontrib = 0;
    uint32_t loaded = 0;
    bool done = !inside;

    for (int32_t base = 0; base < len; base += 256) {
        if (__syncthreads_and(done)) break;
        const int32_t j = base + (int32_t)tid;
        if (j < len) {
            const uint32_t p = inst_vals[range.x + (uint32_t)j];
            const float2 m = mean2d[p];
            const float4 co = conic_opacity[p];
            const float4 c = color_pt[p];
            s_a[tid] = make_float4(m.x, m.y, 0.5f * co.x, co.y);
            s_b[tid] = make_float2(0.5f * co.z, co.w);
            // w: ln(255 * opacity) + 1e-3, the wave-skip bound (see below)
            s_c[tid] = make_float4(__builtin_fmaxf(c.x, 0.f), __builtin_fmaxf(c.y, 0.f), __builtin_fmaxf(c.z, 0.f),
                                   c.w + 1e-3f);
        }
        __syncthreads();
        const int32_t nb = min(256, len - base);
        loaded += (uint32_t)nb;
        for (int32_t k = 0; k < nb; ++k) {
            if (!__any(!done)) break;   // whole wave finished
            const int32_t j = base + k;
            if ((j & (kBucket - 1)) == 0 && j > 0)
                ckpt[(size_t)(slot0 + (uint32_t)(j / kBucket) - 1u) * kTilePixels + tid] = make_float4(C0, C1, C2, T);
            const float4 a = s_a[k];
            const float2 bb = s_b[k];
            const float dx = a.x - pcx, dy = a.y - pcy;
            const float sigma = __builtin_fmaf(dx, __builtin_fmaf(a.z, dx, a.w * dy), (bb.x * dy) * dy);
            // Exact wave-level skip: sigma > ln(255 o) + 1e-3 implies
            // o * exp(-sigma) < exp(-1e-3) / 255, below the 1/255 cut by far
            // more than the error of the deterministic exp / log (< 1e-6
            // relative), so such pixels would all take the alpha < 1/255 path.
            if (!__any(!done && sigma <= s_c[k].w)) continue;
            if (done) continue;
            if (sigma < 0.f) continue;
            const float alpha = __builtin_fminf(bb.y * det_expf_nonpos(-sigma), kMaxAlpha);
            if (alpha < kMinAlpha) continue;
            const float nT = T * (1.0f - alpha);
            if (nT < kTransmittanceMin) {
                done = true;
                continue;
            }
            const float wgt = T * alpha;
            const float4 c = s_c[k];
            C0 = __builtin_fmaf(wgt, c.x, C0);
            C1 = __builtin_fmaf(wgt, c.y, C1);
            C2 = __builtin_fmaf(wgt, c.z, C2);
            T = nT;
            ncontrib = (uint32_t)(base + k + 1);
        }
        __syncthreads();
    }

    const uint32_t pw = cam.tiled_w * 8u, ph = cam.tiled_h * 8u;
    if (px < pw && py < ph) {
        const uint32_t cs = cam.tiled_w * cam.tiled_h * 64u;
        const uint32_t pi = tiled_index(py, px, cam.tiled_w);
        image[pi] = inside ? C0 : 0.f;
        image[pi + cs] = inside ? C1 : 0.f;
        image[pi + 2 * cs] = inside ? C2 : 0.f;
        n_contrib[pi] = inside ? ncontrib : 0u;
    }
    const uint32_t wmax = wave_max_u32(ncontrib);
    if (lane == 0) s_max[w] = wmax;
    __syncthreads();
    if (w == 0) {
        const uint32_t tmax = max(max(s_max[0], s_max[1]), max(s_max[2], s_max[3]));
        const uint32_t nbk = (tmax + (uint32_t)kBucket - 1u) / (uint32_t)kBucket;
        uint32_t off = 0;
        if (lane == 0) {
            tile_max[tile] = tmax;
            tile_loaded[tile] = loaded;
            if (nbk) off = atomicAdd(&ctl->n_items, nbk);
        }
        off = (uint32_t)__builtin_amdgcn_readfirstlane((int)off);
        for (uint32_t b = lane; b < nbk; b += 64u)
            items[off + b] = make_uint4(tile, b, range.x + b * (uint32_t)kBucket,
                                        min((uint32_t)kBucket, tmax - b * (uint32_t)kBucket));
    }
}

size_t blend_ckpt_slots(int64_t n_instances, uint32_t n_tiles) {
    return (size_t)(n_instances > 0 ? n_instances : 0) / kBucket + n_tiles + 1;
}

void launch_blend_forward(const CamParams& cam, const uint2* ranges, const uint32_t* inst_vals, const float2* mean2d,
                          const float4* conic_opacity, const float4* color_pt, float* image, uint32_t* n_contrib,
                          uint32_t* tile_max, uint32_t* tile_loaded, float4* ckpt, uint4* items, BinCtl* ctl,
                          hipStream_t s) {
    const uint32_t n_tiles = cam.grid_w * cam.grid_h;
    if (n_tiles == 0) return;
    blend_forward_kernel<<<n_tiles, 256, 0, s>>>(cam, ranges, inst_vals, mean2d, conic_opacity, color_pt, image,
                                                 n_contrib, tile_max, tile_loaded, ckpt, items, ctl);
}

}  // namespace tgs
