// Front-to-back alpha blending, one 16x16 screen tile per workgroup.
// Follows tinygs/src/rasterizer/fastgs_ours/kernels_forward.cuh:569-715.
//
// MI355X mapping: 256 threads = four wave64; wave w owns the 8x8 image block
// (w & 1, w >> 1) of the tile, which is exactly one 64-float run of the 8x8
// tiled image layout, so every image / n_contrib store of a wave is one
// contiguous 256-byte transaction per plane. Gaussians are staged through LDS
// in batches of 256 (one record per thread).
//
// Per-block culling at staging: the staging thread bounds sigma from below
// over each 8x8 block's pixel-centre rectangle (minimum of the conic's
// quadratic form over the rectangle, minus a rounding allowance) and marks
// the blocks where alpha >= 1/255 is possible. Each wave then walks a
// compacted LDS list of only its marked Gaussians with a branch-free body, so
// Gaussians that miss a block cost that wave nothing. The cut is
// conservative: a skipped Gaussian would have taken the alpha < 1/255 path in
// every pixel of the block, so results are unchanged.
//
// Checkpoints: before Gaussian j of the tile's list with j % 32 == 0, j > 0,
// every still-active wave stores its pixels' (C, T) (kernels_forward.cuh:
// 644-653), one contiguous 1 KiB run per wave. At the end the tile appends one
// backward work item per 32-Gaussian bucket below its last contributor
// (tmax <= len, so every bucket of an item is inside the list).
//
// Numerics mirror the CPU oracle: alpha = min(o 2^-sigma', 0.999) with
// sigma' = fma(dx, fma(a L/2, dx, (b L) dy), ((c L/2) dy) dy) from the conic
// prescaled by L = log2(e) at staging and the deterministic exp2
// (det_exp2_core); the reference's sigma >= 0 and alpha >= 1/255 tests as
// 0 <= sigma' <= ln(255 o) L (the preprocess's power threshold times L, equal
// up to rounding at the edge), and the 1e-4 transmittance stop with the
// terminating Gaussian not composited. A pixel that stopped (or lies outside
// the image) carries T = 0: every later Gaussian then fails the transmittance
// test and changes nothing, so no separate flag is kept.
#include "common.h"
#include "kernels.h"

namespace tgs {

// Lower bound of sigma(dx, dy) = a/2 dx^2 + b dx dy + c/2 dy^2 over the box
// [dx0, dx1] x [dy0, dy1] (dx = mean - pixel centre), valid for the float
// evaluation the blend uses at any pixel centre in the box. Convex case
// (a > 0, c > 0, ac > b^2): 0 if the box holds the origin, else the least of
// the four edge minima (clamped 1-D minimisers); then minus 2^-16 of the
// largest term magnitude, far above the few-ulp rounding of either
// evaluation. Returns -inf (never cull) for a non-convex conic.
__device__ __forceinline__ float sigma_box_lower_bound(float a, float b, float c, float dx0, float dx1, float dy0,
                                                       float dy1) {
    if (!(a > 0.f) || !(c > 0.f) || !(a * c > b * b)) return -__builtin_inff();
    const float mx = __builtin_fmaxf(__builtin_fabsf(dx0), __builtin_fabsf(dx1));
    const float my = __builtin_fmaxf(__builtin_fabsf(dy0), __builtin_fabsf(dy1));
    const float slack = 1.52587890625e-05f * (0.5f * a * mx * mx + __builtin_fabsf(b) * mx * my + 0.5f * c * my * my);
    if (dx0 <= 0.f && dx1 >= 0.f && dy0 <= 0.f && dy1 >= 0.f) return -slack;
    auto q = [&](float x, float y) { return 0.5f * a * x * x + b * x * y + 0.5f * c * y * y; };
    const float ia = 1.0f / a, ic = 1.0f / c;
    float m = __builtin_inff();
    // edges x = dx0, dx1: minimiser y = -b x / c
    m = __builtin_fminf(m, q(dx0, __builtin_fminf(__builtin_fmaxf(-b * dx0 * ic, dy0), dy1)));
    m = __builtin_fminf(m, q(dx1, __builtin_fminf(__builtin_fmaxf(-b * dx1 * ic, dy0), dy1)));
    // edges y = dy0, dy1: minimiser x = -b y / a
    m = __builtin_fminf(m, q(__builtin_fminf(__builtin_fmaxf(-b * dy0 * ia, dx0), dx1), dy0));
    m = __builtin_fminf(m, q(__builtin_fminf(__builtin_fmaxf(-b * dy1 * ia, dx0), dx1), dy1));
    return m - slack;
}

// Tiles in roughly decreasing order of the bit length of their instance
// counts, for the forward to start with the heavy tiles: its length is set by
// the waves that start last. Workgroup c of kOrderChunks sorts the tiles
// t = c (mod kOrderChunks) by that bit length and writes its k-th tile to
// position k kOrderChunks + c, so the positions are a permutation of the
// tiles and each run of kOrderChunks positions holds one tile of every chunk
// in the same rank. (Order within a bin: whatever the LDS atomics give; it
// only affects scheduling.)
constexpr uint32_t kOrderChunks = 16;

__global__ void __launch_bounds__(512) tile_order_kernel(const uint2* __restrict__ ranges, uint32_t n_tiles,
                                                         uint32_t* __restrict__ order,
                                                         const BinCtl* __restrict__ ctl) {
    __shared__ uint32_t s_off[33];
    const uint32_t t = threadIdx.x, lane = t & 63u, c = blockIdx.x;
    if (t < 33u) s_off[t] = 0u;
    __syncthreads();
    const bool failed = (ctl->err & (kErrLookBack | kErrOffsets)) != 0u;
    const uint32_t n_c = n_tiles > c ? (n_tiles - c + kOrderChunks - 1u) / kOrderChunks : 0u;   // this chunk's tiles
    // bin: 32 - the bit length of the tile's instance count (0 for the longest)
    auto bin_at = [&](uint32_t k) {
        const uint2 r = ranges[c + k * kOrderChunks];
        const uint32_t len = failed || r.y <= r.x ? 0u : r.y - r.x;   // empty: (UINT32_MAX, 0)
        return len ? (uint32_t)__builtin_clz(len) : 32u;
    };
    // the lanes of the wave with the same bin (6 ballots), so that one lane
    // per bin and wave touches the LDS counters
    auto peers_of = [&](uint32_t bin, bool valid) {
        uint64_t m = __ballot(valid);
#pragma unroll
        for (int q = 0; q < 6; ++q) {
            const uint64_t bq = __ballot(((bin >> q) & 1u) != 0u);
            m &= ((bin >> q) & 1u) ? bq : ~bq;
        }
        return m;
    };
    // pass 1: counts per bin (the first 512 bins stay in registers for pass 2)
    uint32_t bin0 = 0u;
    for (uint32_t q = 0; q < n_c; q += 512u) {
        const uint32_t k = q + t;
        const bool valid = k < n_c;
        const uint32_t bin = valid ? bin_at(k) : 0u;
        if (q == 0u) bin0 = bin;
        const uint64_t peers = peers_of(bin, valid);
        if (valid && (peers & ((1ull << lane) - 1ull)) == 0ull) atomicAdd(&s_off[bin], (uint32_t)__popcll(peers));
    }
    __syncthreads();
    if (t < 64u) {   // exclusive scan of the 33 bin counts (one wave)
        const uint32_t v = t < 33u ? s_off[t] : 0u;
        const uint32_t incl = wave_inclusive_scan_u32(v);
        if (t < 33u) s_off[t] = incl - v;
    }
    __syncthreads();
    // pass 2: positions
    for (uint32_t q = 0; q < n_c; q += 512u) {
        const uint32_t k = q + t;
        const bool valid = k < n_c;
        const uint32_t bin = !valid ? 0u : q == 0u ? bin0 : bin_at(k);
        const uint64_t peers = peers_of(bin, valid);
        const uint64_t below = peers & ((1ull << lane) - 1ull);
        const uint32_t leader = valid ? (uint32_t)__builtin_ctzll(peers) : 0u;
        uint32_t base = 0;
        if (valid && below == 0ull) base = atomicAdd(&s_off[bin], (uint32_t)__popcll(peers));
        base = (uint32_t)__shfl((int)base, (int)leader);
        if (valid) order[(base + (uint32_t)__popcll(below)) * kOrderChunks + c] = c + k * kOrderChunks;
    }
}

bool launch_tile_order(const uint2* ranges, uint32_t n_tiles, uint32_t* order, const BinCtl* ctl, hipStream_t s) {
    if (!order || n_tiles == 0u || n_tiles > kOrderMaxTiles) return false;
    tile_order_kernel<<<kOrderChunks, 512, 0, s>>>(ranges, n_tiles, order, ctl);
    return true;
}

__global__ void __launch_bounds__(256) blend_forward_kernel(CamParams cam, uint2* __restrict__ ranges,
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
                                                            BinCtl* __restrict__ ctl,
                                                            const uint32_t* __restrict__ order) {
    // s_a, s_b and s_c are read at one LDS address per Gaussian (offsets 0, 4 and 8 KiB)
    __shared__ float4 s_a[256];       // mx, my, a L/2, b L
    __shared__ float4 s_b[256];       // c L/2, opacity, r, g (clamped colour)
    __shared__ float4 s_c[256];       // b (clamped colour), accept threshold ln(255 o) L, -, -
    __shared__ uint32_t s_mask[256];  // bit q: may reach alpha >= 1/255 in 8x8 block q
    __shared__ uint16_t s_list[4][256];
    __shared__ uint32_t s_max[4];

    const uint32_t tile = order ? order[blockIdx.x] : blockIdx.x;   // long tiles first
    const uint32_t gx = tile % cam.grid_w, gy = tile / cam.grid_w;
    const uint32_t tid = threadIdx.x, w = tid >> 6, lane = tid & 63u;
    const uint32_t px = gx * 16u + (w & 1u) * 8u + (lane & 7u);
    const uint32_t py = gy * 16u + (w >> 1) * 8u + (lane >> 3);
    const bool inside = px < cam.width && py < cam.height;
    const float pcx = (float)px + 0.5f, pcy = (float)py + 0.5f;

    uint2 range = ranges[tile];
    // a failed binning scan (reported by the host) leaves partial instance
    // lists: every tile renders as empty instead of reading them
    if (ctl->err & (kErrLookBack | kErrOffsets)) range = make_uint2(0u, 0u);
    if (range.y == 0u) {   // an empty tile, left as (UINT32_MAX, 0) by the tile sort: stored as (0, 0)
        range.x = 0u;
        if (tid == 0u) ranges[tile] = range;
    }
    const int32_t len = (int32_t)(range.y - range.x);
    const uint32_t slot0 = range.x / (uint32_t)kBucket + tile;   // first checkpoint slot of this tile

    float C0 = 0.f, C1 = 0.f, C2 = 0.f, T = inside ? 1.f : 0.f;
    uint32_t ncontrib = 0;
    uint32_t loaded = 0;
    int32_t next_ck = kBucket;   // next bucket boundary whose checkpoint this wave still owes

    for (int32_t base = 0; base < len; base += 256) {
        if (__syncthreads_and(T == 0.f)) break;
        const int32_t nb = min(256, len - base);
        {
            const int32_t j = base + (int32_t)tid;
            uint32_t mask = 0;
            if (j < len) {
                const uint32_t p = inst_vals[range.x + (uint32_t)j];
                const float2 m = mean2d[p];
                const float4 co = conic_opacity[p];
                const float4 c = color_pt[p];
                s_a[tid] = make_float4(m.x, m.y, co.x * kHalfLog2e, co.y * kLog2eF);
                s_b[tid] = make_float4(co.z * kHalfLog2e, co.w, __builtin_fmaxf(c.x, 0.f), __builtin_fmaxf(c.y, 0.f));
                s_c[tid] = make_float4(__builtin_fmaxf(c.z, 0.f), c.w * kLog2eF, 0.f, 0.f);
                // sigma > ln(255 o) + 1e-3 implies o 2^-sigma' < exp(-1e-3) / 255 (sigma' = sigma L to a few
                // ulps), below the 1/255 cut by far more than the error of the deterministic exp2 / log
                // (< 1e-6 relative)
                const float bound = c.w + 1e-3f;
#pragma unroll
                for (uint32_t q = 0; q < 4; ++q) {
                    const float x0 = (float)(gx * 16u + (q & 1u) * 8u) + 0.5f;
                    const float y0 = (float)(gy * 16u + (q >> 1) * 8u) + 0.5f;
                    const float lb = sigma_box_lower_bound(co.x, co.y, co.z, m.x - (x0 + 7.f), m.x - x0,
                                                           m.y - (y0 + 7.f), m.y - y0);
                    if (lb <= bound) mask |= 1u << q;
                }
            }
            s_mask[tid] = mask;
        }
        __syncthreads();
        loaded += (uint32_t)nb;
        // this wave's compacted list of Gaussians (batch positions) that may touch its block
        int32_t cnt = 0;
        for (int32_t c0 = 0; c0 < nb; c0 += 64) {
            const int32_t e = c0 + (int32_t)lane;
            const bool hit = e < nb && ((s_mask[e] >> w) & 1u);
            const uint64_t bal = ballot(hit);
            if (hit) s_list[w][cnt + (int32_t)mask_rank(bal)] = (uint16_t)e;
            cnt += (int32_t)__builtin_popcountll(bal);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

        // two marked Gaussians per step: both records are read before either is blended
        auto blend = [&](int32_t e, const float4& a, const float4& bb, const float4& cc) {
            const int32_t j = base + e;
            while (next_ck <= j) {   // bucket boundaries passed since the last marked Gaussian
                ckpt[(size_t)(slot0 + (uint32_t)(next_ck / kBucket) - 1u) * kTilePixels + tid] =
                    make_float4(C0, C1, C2, T);
                next_ck += kBucket;
            }
            const float dx = a.x - pcx, dy = a.y - pcy;
            const float sigma = __builtin_fmaf(dx, __builtin_fmaf(a.z, dx, a.w * dy), (bb.x * dy) * dy);
            // alpha only matters where ok holds (0 <= sigma' <= ln 255 L), so exp2 needs no clamp
            const float alpha = __builtin_fminf(bb.y * det_exp2_core(-sigma), kMaxAlpha);
            const float nT = T * (1.0f - alpha);
            // sigma >= 0 and alpha >= 1/255 as 0 <= sigma' <= thr': one unsigned compare of the
            // bit patterns (thr' >= 0; sigma' is never -0: its last term (c L/2 dy) dy is >= +0)
            const bool ok = f2u(sigma) <= f2u(cc.y);
            // a stopped pixel has T = 0, so nT = 0 fails the test
            const bool keep = nT >= kTransmittanceMin;
            const bool acc = ok && keep;
            // one select of the weight instead of three of the sums: fma(+0, c, C)
            // is C itself for the finite colours
            const float wgt = acc ? T * alpha : 0.f;
            C0 = __builtin_fmaf(wgt, bb.z, C0);
            C1 = __builtin_fmaf(wgt, bb.w, C1);
            C2 = __builtin_fmaf(wgt, cc.x, C2);
            T = ok ? (keep ? nT : 0.f) : T;
            ncontrib = acc ? (uint32_t)(j + 1) : ncontrib;
        };
        for (int32_t i = 0; i < cnt; i += 2) {
            if (!__any(T != 0.f)) break;   // whole wave finished
            const uint32_t pair = *(const uint32_t*)&s_list[w][i];   // i is even: 4-byte aligned
            const int32_t e0 = __builtin_amdgcn_readfirstlane((int)(pair & 0xffffu));
            const bool two = i + 1 < cnt;
            const int32_t e1 = two ? __builtin_amdgcn_readfirstlane((int)(pair >> 16)) : e0;
            const float4 a0 = s_a[e0], b0 = s_b[e0], c0 = s_c[e0];
            const float4 a1 = s_a[e1], b1 = s_b[e1], c1 = s_c[e1];
            blend(e0, a0, b0, c0);
            if (two) blend(e1, a1, b1, c1);
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

void launch_blend_forward(const CamParams& cam, uint2* ranges, const uint32_t* inst_vals, const float2* mean2d,
                          const float4* conic_opacity, const float4* color_pt, float* image, uint32_t* n_contrib,
                          uint32_t* tile_max, uint32_t* tile_loaded, float4* ckpt, uint4* items, BinCtl* ctl,
                          uint32_t* order, hipStream_t s) {
    const uint32_t n_tiles = cam.grid_w * cam.grid_h;
    if (n_tiles == 0) return;
    if (!launch_tile_order(ranges, n_tiles, order, ctl, s)) order = nullptr;
    blend_forward_kernel<<<n_tiles, 256, 0, s>>>(cam, ranges, inst_vals, mean2d, conic_opacity, color_pt, image,
                                                 n_contrib, tile_max, tile_loaded, ckpt, items, ctl, order);
}

}  // namespace tgs
