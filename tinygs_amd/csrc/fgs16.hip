// Blend forward and backward of the fp16-image rasterizer (FGS16).
//
// Reference: blend_cu2 (tinygs/src/rasterizer/fastgs_ours_fp16/
// kernels_forward.cuh:917-1171) and blend_backward_cu2 (kernels_backward.cuh:
// 861-1389). Their numerics are kept: half mean / conic in 16-pixel tile
// units with the conic scaled by 16, an 8-bit colour, 255-scaled colour and
// transmittance, alpha = min(o * 2^(-sigma log2 e), 0.99) with no 1/255 cut,
// the transmittance stop nT < RD(255e-4) with the stopping Gaussian not
// composited, a 16-bit saturating count of processed Gaussians per pixel,
// checkpoints every 32 Gaussians, and a backward that weighs every Gaussian of
// a bucket at every pixel of the tile (as compiled: TINYGS_SAFE_MATH is never
// defined). Every half operation is the canonical one of halfmath.h, in the
// operation order of the CPU oracle (oracle/fgs16_impl.inc), so pixels,
// counts, checkpoints and the per-(primitive, bucket) gradient records are
// bit-identical to it.
//
// MI355X mapping:
//   * forward: two wave64s per tile. Wave k owns blocks 2k and 2k + 1 of
//     the tile, lane L pixel L of each (in-tile pixels 64 q + L), held as
//     one half2; every image / count / checkpoint access of a block is one
//     contiguous run. Each wave stages the tile's Gaussians 64 at a time,
//     one per lane, in LDS; each Gaussian's words then reach every lane as
//     a broadcast read (no VALU). Tiles are taken roughly long ones first
//     (tile_order_kernel): the kernel's length was set by long tiles whose
//     waves started late.
//   * backward: one (tile, 32-Gaussian bucket) work item per half wave, two
//     per wave. As in the reference, lane l of the half owns Gaussian l of the
//     bucket and the tile's 128 pixel pairs stream through the lanes: at step
//     s lane l processes pair s - l with the state Gaussians 0..l-1 left, then
//     hands the state to lane l + 1 with one DPP wave_shr:1 per register
//     (lanes 0 and 32 load the next pair from LDS instead). Each Gaussian so
//     accumulates its sums over the pairs in the reference's order.
//   * the per-(primitive, bucket) results are 12-float records in the slots
//     binning reserved (as the fp32 path); the preprocess backward sums them
//     exactly (halfmath.h half_of_fixed) instead of the reference's half2
//     atomics, whose rounding depends on the order buckets finish in.
#include <type_traits>

#include "common.h"
#include "fgs16.h"
#include "kernels.h"

namespace tgs {

namespace {

constexpr uint16_t kH255 = 0x5bf8;   // 255
constexpr uint16_t kHUnscale = 0x1c04;   // RN(1/255)
// 16 RN(-log2 e) = -23.078125, exact. The reference scales the power by 16,
// then by RN(-log2 e): (x * 16) * k and x * (16 k) are the same half for
// every half x (16 x is exact, and where it overflows so does x * 16 k).
constexpr uint16_t kHNeg16Log2e = 0xcdc5;


// The half pixel-centre offsets of blend_cu2 (kernels_forward.cuh:960-967) in
// tile units: x of an even in-tile column lx = fma(1/16, lx, 1/32), of an odd
// one 1/16 + that of lx - 1; y = fma(1/16, ly, 1/32).
__device__ __forceinline__ h16 offset_x(uint32_t lx) {
    const h16 base = h_fma((h16)0.0625f, (h16)(float)(lx & ~1u), (h16)(1.0f / 32.0f));
    return (lx & 1u) ? (h16)0.0625f + base : base;
}
__device__ __forceinline__ h16 offset_y(uint32_t ly) {
    return h_fma((h16)0.0625f, (h16)(float)ly, (h16)(1.0f / 32.0f));
}

// ge / select on half2 lanes
__device__ __forceinline__ h16x2 sel2(bool cx, bool cy, h16x2 a, h16x2 b) {
    return h2(cx ? a.x : b.x, cy ? a.y : b.y);
}

}  // namespace

// ---------------------------------------------------------------- forward

namespace {
typedef int16_t i16x2 __attribute__((ext_vector_type(2)));
// 0xffff in each 16-bit half whose half value is negative (sign bit set)
__device__ __forceinline__ uint32_t neg_mask16(h16x2 d) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(i16x2, d) >> (i16x2){15, 15});
}
// m ? a : b, bit by bit
__device__ __forceinline__ uint32_t bsel(uint32_t m, uint32_t a, uint32_t b) { return (a & m) | (b & ~m); }
}  // namespace

// info[p] = (conic a | b << 16, c | opacity << 16, r | g << 8 | b << 16, 0)
// ckpt16: per slot 256 pixels of (C.r | C.g << 16, C.b | T << 16) halves, in-tile index 64 q + L.
//
// Two waves per tile (two tiles per 256-thread workgroup): wave k of a tile
// owns blocks 2k and 2k + 1, lane L their pixel L as the two halves of a
// half2, so a tile's pixels are split over two waves (the heaviest tiles set
// the kernel's length). A pixel's state is (C, T) plus a 16-bit mask, all
// ones while the pixel is unfinished: the accept test nT >= thr is the sign
// of nT - thr (exact: a half difference is zero only for equal operands),
// and the masks select T, the composited weight and the count with bit
// operations. An unfinished pixel has processed every Gaussian so far, so
// its count after Gaussian j is min(j + 1, 65535): one select per Gaussian,
// and the saturation stop (:1115) is the same for every unfinished pixel.
__global__ void __launch_bounds__(256) blend16_forward_kernel(
    CamParams cam, uint2* __restrict__ ranges, const uint32_t* __restrict__ inst_vals,
    const float2* __restrict__ mean2d, const uint4* __restrict__ info, uint16_t* __restrict__ image,
    uint16_t* __restrict__ n_contrib, uint32_t* __restrict__ tile_max, uint32_t* __restrict__ tile_loaded,
    uint2* __restrict__ ckpt, uint4* __restrict__ items, BinCtl* __restrict__ ctl,
    const uint32_t* __restrict__ order) {
    __shared__ uint32_t s_tmax[4], s_loaded[4];
    __shared__ uint4 s_gw[4][64][2];   // per wave, the staged batch: five words per Gaussian
    const uint32_t n_tiles = cam.grid_w * cam.grid_h;
    const uint32_t w = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t opos = blockIdx.x * 2u + (w >> 1), k = w & 1u;
    const bool tile_ok = opos < n_tiles;   // (no early return: the workgroup meets at a barrier)
    const uint32_t tile = tile_ok && order ? order[opos] : opos;
    const uint32_t gx = tile_ok ? tile % cam.grid_w : 0u, gy = tile_ok ? tile / cam.grid_w : 0u;
    const uint32_t lx = lane & 7u, ly = lane >> 3;

    const h16 thr = h_rd(1e-4f * 255.0f);
    const h16x2 maxa = h2s((h16)0.99f), unscale = h2s(hfrom(kHUnscale)), h05 = h2s((h16)0.5f),
                nthr = h2s(-thr);
    // .x: block 2k (in-tile column lx), .y: block 2k + 1 (column lx + 8); row 8k + ly
    const h16x2 offx = h2(offset_x(lx), offset_x(lx + 8u));
    const h16x2 offy = h2s(offset_y(ly + 8u * k));
    const uint32_t px0 = gx * 16u + lx, py = gy * 16u + 8u * k + ly;
    const bool in0 = tile_ok && px0 < cam.width && py < cam.height;
    const bool in1 = tile_ok && px0 + 8u < cam.width && py < cam.height;

    uint2 range = tile_ok ? ranges[tile] : make_uint2(0u, 0u);
    // a failed binning scan (reported by the host) leaves partial instance
    // lists: every tile renders as empty instead of reading them
    if (ctl->err & (kErrLookBack | kErrOffsets)) range = make_uint2(0u, 0u);
    if (range.y == 0u) {   // an empty tile, left as (UINT32_MAX, 0) by the tile sort: stored as (0, 0)
        range.x = 0u;
        if (tile_ok && k == 0u && lane == 0u) ranges[tile] = range;
    }
    const int32_t len = (int32_t)(range.y - range.x);
    const uint32_t slot0 = range.x / (uint32_t)kBucket + tile;

    h16x2 C0 = h2s((h16)0.0f), C1 = C0, C2 = C0, T = h2s(hfrom(kH255));
    uint32_t live = (in0 ? 0x0000ffffu : 0u) | (in1 ? 0xffff0000u : 0u);
    uint32_t nc = 0;   // the two pixels' counts, u16 each
    uint32_t loaded = 0;
    uint32_t jn = 0;   // Gaussians processed

    // staging (kernels_forward.cuh:1044-1056), 64 Gaussians at a time, one
    // per lane: the next batch's indices are loaded when a batch starts and
    // their rows after its first group of 8, so the loads overlap the blend
    uint32_t pn = (int32_t)lane < len ? inst_vals[range.x + lane] : 0u;
    float2 mn = (int32_t)lane < len ? mean2d[pn] : make_float2(0.f, 0.f);
    uint4 inn = (int32_t)lane < len ? info[pn] : make_uint4(0u, 0u, 0u, 0u);
    for (int32_t base = 0; base < len; base += 64) {
        if (!__any(live != 0u)) break;
        const int32_t nb = min(64, len - base);
        uint32_t w0 = 0, w1 = 0, w2 = 0, w3 = 0, w4 = 0;
        if ((int32_t)lane < nb) {
            const h16 mx = h_rn(mn.x / 16.0f - (float)gx), my = h_rn(mn.y / 16.0f - (float)gy);
            const h16 cxh = hfrom((uint16_t)(inn.x & 0xffffu)) * (h16)16.0f;
            const h16 cyh = hfrom((uint16_t)(inn.x >> 16)) * (h16)16.0f;
            const h16 czh = hfrom((uint16_t)(inn.y & 0xffffu)) * (h16)16.0f;
            const h16 o = hfrom((uint16_t)(inn.y >> 16)) * (h16)1.0f;
            w0 = (uint32_t)hbits(mx) | ((uint32_t)hbits(my) << 16);
            w1 = (uint32_t)hbits(cxh) | ((uint32_t)hbits(cyh) << 16);
            w2 = (uint32_t)hbits(czh) | ((uint32_t)hbits(o) << 16);
            w3 = (uint32_t)hbits((h16)(float)(inn.z & 0xffu)) |
                 ((uint32_t)hbits((h16)(float)((inn.z >> 8) & 0xffu)) << 16);
            w4 = (uint32_t)hbits((h16)(float)((inn.z >> 16) & 0xffu));
        }
        // the batch to LDS: each Gaussian's words reach every lane as a
        // broadcast read (no VALU), and the previous batch's reads are done
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        s_gw[w][lane][0] = make_uint4(w0, w1, w2, w3);
        s_gw[w][lane][1].x = w4;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const int32_t nxt = len - base - 64;   // Gaussians after this batch
        pn = (int32_t)lane < nxt ? inst_vals[range.x + (uint32_t)(base + 64) + lane] : 0u;
        loaded += (uint32_t)nb;
        for (int32_t e0 = 0; e0 < nb; e0 += 8) {
            if (e0 == 8 && nxt > 0) {
                mn = (int32_t)lane < nxt ? mean2d[pn] : make_float2(0.f, 0.f);
                inn = (int32_t)lane < nxt ? info[pn] : make_uint4(0u, 0u, 0u, 0u);
            }
            const int32_t j0 = base + e0;
            if ((j0 & (kBucket - 1)) == 0 && j0 > 0) {   // checkpoint before Gaussian j0 (:1000-1012)
                uint2* ck = ckpt + (size_t)(slot0 + (uint32_t)(j0 / kBucket) - 1u) * kTilePixels + lane;
                ck[(2u * k) * 64u] = make_uint2((uint32_t)hbits(C0.x) | ((uint32_t)hbits(C1.x) << 16),
                                                (uint32_t)hbits(C2.x) | ((uint32_t)hbits(T.x) << 16));
                ck[(2u * k + 1u) * 64u] = make_uint2((uint32_t)hbits(C0.y) | ((uint32_t)hbits(C1.y) << 16),
                                                     (uint32_t)hbits(C2.y) | ((uint32_t)hbits(T.y) << 16));
            }
            const int32_t ng = min(8, nb - e0);
            // one Gaussian: its power, exp2 and alpha do not depend on the
            // pixel state, so a full group's eight interleave freely
            auto blend_one = [&](int32_t e, int32_t j) {
                const uint4 q = s_gw[w][e][0];
                const h16x2 g0 = h2from(q.x), g1 = h2from(q.y), g2 = h2from(q.z);
                const h16x2 g3 = h2from(q.w), g4 = h2from(s_gw[w][e][1].x);
                const h16x2 mx2 = h2s(g0.x), my2 = h2s(g0.y), cx2 = h2s(g1.x), cy2 = h2s(g1.y);
                const h16x2 cz2 = h2s(g2.x), o2 = h2s(g2.y), r2 = h2s(g3.x), gg2 = h2s(g3.y), b2 = h2s(g4.x);
                // :1069-1105
                const h16x2 dx = mx2 - offx, dy = my2 - offy;
                const h16x2 qxx = dx * (cx2 * dx);
                const h16x2 qzz = dy * (cz2 * dy);
                const h16x2 qxy = dx * (cy2 * dy);
                const h16x2 quad = qxx + qzz;
                const h16x2 gss = h2_exp2(h2_fma(h05, quad, qxy) * h2s(hfrom(kHNeg16Log2e)));
                const h16x2 alpha = h2_min(o2 * gss, maxa);
                const h16x2 nT = h2_fma(-alpha, T, T);
                // enabled: unfinished and nT >= thr
                const uint32_t en = live & ~neg_mask16(nT + nthr);
                const h16x2 tah = h2from(h2bits((T * alpha) * unscale) & en);
                C0 = h2_fma(r2, tah, C0);
                C1 = h2_fma(gg2, tah, C1);
                C2 = h2_fma(b2, tah, C2);
                T = h2from(bsel(en, h2bits(nT), h2bits(T)));
                nc = bsel(live, min((uint32_t)j + 1u, 0xffffu) * 0x10001u, nc);
                live = en;
            };
            if (ng == 8) {
#pragma unroll
                for (int32_t u = 0; u < 8; ++u) blend_one(e0 + u, j0 + u);
            } else {
                for (int32_t u = 0; u < ng; ++u) blend_one(e0 + u, j0 + u);
            }
            const int32_t jl = j0 + ng - 1;   // the group's last Gaussian
            jn = (uint32_t)jl + 1u;
            // :1115: after each 32 Gaussians, a saturated count stops the pixel
            // (bucket ends and the last Gaussian close a group)
            if (((jl & (kBucket - 1)) == kBucket - 1 || jl + 1 == len) && (uint32_t)jl + 1u >= 0xffffu) live = 0u;
            if (!__any(live != 0u)) break;
        }
    }

    const uint32_t pw = cam.tiled_w * 8u, ph = cam.tiled_h * 8u;
    const uint32_t cs = cam.tiled_w * cam.tiled_h * 64u;
    const h16 us = hfrom(kHUnscale);
#pragma unroll
    for (uint32_t hi = 0; hi < 2u; ++hi) {
        const uint32_t px = px0 + 8u * hi;
        if (tile_ok && px < pw && py < ph) {
            const uint32_t pi = tiled_index(py, px, cam.tiled_w);
            const bool in = hi ? in1 : in0;
            const h16 c0 = hi ? C0.y : C0.x, c1 = hi ? C1.y : C1.x, c2 = hi ? C2.y : C2.x;
            image[pi] = in ? hbits(c0 * us) : (uint16_t)0u;
            image[pi + cs] = in ? hbits(c1 * us) : (uint16_t)0u;
            image[pi + 2 * cs] = in ? hbits(c2 * us) : (uint16_t)0u;
            n_contrib[pi] = in ? (uint16_t)(hi ? nc >> 16 : nc & 0xffffu) : (uint16_t)0u;
        }
    }
    const uint32_t wmax = wave_max_u32(max(nc & 0xffffu, nc >> 16));
    if (lane == 0u) {
        s_tmax[w] = wmax;
        s_loaded[w] = loaded;
    }
    __syncthreads();
    if (!tile_ok) return;
    const uint32_t w0 = w & ~1u;
    const uint32_t tmax = max(s_tmax[w0], s_tmax[w0 + 1u]);
    // backward work items: every bucket below the tile's largest count, each
    // with all its Gaussians (the backward does not stop at a pixel's count)
    const uint32_t nbk = (tmax + (uint32_t)kBucket - 1u) / (uint32_t)kBucket;
    // the checkpoints of buckets below that count which this wave stopped
    // short of (the other wave of the tile ran on): its pixels were all
    // finished, so their state there is the final one
    for (uint32_t m = jn ? (jn - 1u) / (uint32_t)kBucket + 1u : 1u; m < nbk; ++m) {
        uint2* ck = ckpt + (size_t)(slot0 + m - 1u) * kTilePixels + lane;
        ck[(2u * k) * 64u] = make_uint2((uint32_t)hbits(C0.x) | ((uint32_t)hbits(C1.x) << 16),
                                        (uint32_t)hbits(C2.x) | ((uint32_t)hbits(T.x) << 16));
        ck[(2u * k + 1u) * 64u] = make_uint2((uint32_t)hbits(C0.y) | ((uint32_t)hbits(C1.y) << 16),
                                             (uint32_t)hbits(C2.y) | ((uint32_t)hbits(T.y) << 16));
    }
    if (k != 0u) return;
    uint32_t off = 0;
    if (lane == 0) {
        tile_max[tile] = tmax;
        tile_loaded[tile] = max(s_loaded[w], s_loaded[w + 1u]);
        if (nbk) off = atomicAdd(&ctl->n_items, nbk);
    }
    off = (uint32_t)__builtin_amdgcn_readfirstlane((int)off);
    for (uint32_t b = lane; b < nbk; b += 64u)
        items[off + b] = make_uint4(tile, b, range.x + b * (uint32_t)kBucket,
                                    min((uint32_t)kBucket, (uint32_t)len - b * (uint32_t)kBucket));
}

void launch_blend16_forward(const CamParams& cam, uint2* ranges, const uint32_t* inst_vals,
                            const float2* mean2d, const uint4* info, uint16_t* image, uint16_t* n_contrib,
                            uint32_t* tile_max, uint32_t* tile_loaded, uint2* ckpt, uint4* items, BinCtl* ctl,
                            uint32_t* order, hipStream_t s) {
    const uint32_t n_tiles = cam.grid_w * cam.grid_h;
    if (n_tiles == 0) return;
    if (!launch_tile_order(ranges, n_tiles, order, ctl, s)) order = nullptr;   // tiles in index order
    blend16_forward_kernel<<<(n_tiles + 1u) / 2u, 256, 0, s>>>(cam, ranges, inst_vals, mean2d, info, image,
                                                                n_contrib, tile_max, tile_loaded, ckpt, items, ctl,
                                                                order);
}

// ---------------------------------------------------------------- backward

namespace {

// LDS byte address of a __shared__ object, and the 16 bytes at one
typedef uint32_t v4u32 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) const v4u32 lds_v4;
__device__ __forceinline__ uint32_t lds_addr(const uint4* p) { return (uint32_t)(uintptr_t)(lds_v4*)p; }
__device__ __forceinline__ uint4 lds_u4_at(uint32_t a) {
    const v4u32 v = *(lds_v4*)(uintptr_t)a;
    return make_uint4(v.x, v.y, v.z, v.w);
}

// s_pair[0]: per wave, half wave and pixel pair the static words (grad r, g,
// b, (offx, offy)); s_pair[1] the state at the bucket start (colour after r,
// g, b, T), kPairInitOfs bytes after the pair's static words
constexpr uint32_t kPairInitOfs = 4u * 2u * 128u * 16u;

__device__ __forceinline__ uint32_t shr1(uint32_t x) {
    // DPP wave_shr:1: lane l receives lane l - 1 (lane 0: 0, bound_ctrl)
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x138, 0xf, 0xf, true);
}

}  // namespace

__global__ void __launch_bounds__(256) blend16_backward_kernel(
    CamParams cam, const uint32_t* __restrict__ inst_vals, const float2* __restrict__ mean2d,
    const uint4* __restrict__ info, const uint16_t* __restrict__ image, const uint16_t* __restrict__ grad_image,
    const uint2* __restrict__ ckpt, const uint4* __restrict__ items, BinCtl* __restrict__ ctl,
    uint32_t* __restrict__ rec_count, const uint32_t* __restrict__ first_slot, float4* __restrict__ records) {
    __shared__ uint4 s_pair[2][4][2][128];   // static words, then the bucket-start state

    const uint32_t w = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t half = lane >> 5, l = lane & 31u;
    const uint32_t n_items = ctl->n_items;
    const uint32_t cs = cam.tiled_w * cam.tiled_h * 64u;
    const uint32_t queue = (blockIdx.x * 4u + w) % (uint32_t)kBwdQueues;
    uint32_t* qctr = &ctl->bwd_queue[queue * 32u];
    uint32_t next = 0;
    if (lane == 0) next = atomicAdd(qctr, 1u);
    next = (uint32_t)__builtin_amdgcn_readfirstlane((int)next);

    const h16x2 h05 = h2s((h16)0.5f), one = h2s((h16)1.0f), maxa = h2s((h16)0.99f),
                nk = h2s(hfrom(kHNeg16Log2e)), inv16 = h2s((h16)0.0625f);

    while (true) {
        const uint32_t pr = bwd_queue_item(queue, next);   // item pair, increasing in next
        if (2u * pr >= n_items) break;
        uint32_t after = 0;
        if (lane == 0) after = atomicAdd(qctr, 1u);
        const uint32_t it = 2u * pr + half;
        const bool have = it < n_items;
        const uint4 item = have ? items[it] : make_uint4(0u, 0u, 0u, 0u);
        const uint32_t tile = item.x, b = item.y, first = item.z;
        const uint32_t cnt = item.w;   // 0 for a missing second item
        const uint32_t gx = tile % cam.grid_w, gy = tile / cam.grid_w;

        // ---- this lane's Gaussian (kernels_backward.cuh:1019-1037); its record slot
        h16x2 mxp = h2s((h16)0.f), my2 = mxp, cx2 = mxp, cy2 = mxp, cz2 = mxp, o2 = mxp;
        h16x2 cr2 = mxp, cg2 = mxp, cb2 = mxp;
        uint32_t p = 0, slot = 0;
        if (l < cnt) {
            p = inst_vals[first + l];
            slot = first_slot[p] + atomicAdd(rec_count + p, 1u);
            const float2 m = mean2d[p];
            const uint4 in = info[p];
            const float mfx = m.x / 16.0f - (float)gx, mfy = m.y / 16.0f - (float)gy;
            const h16 mx0 = h_rn(mfx - 1.0f / 32.0f), my = h_rn(mfy - 1.0f / 32.0f);
            const h16 mx1 = mx0 - (h16)(1.0f / 16.0f);
            mxp = h2(mx0, mx1);
            my2 = h2s(my);
            cx2 = h2s(hfrom((uint16_t)(in.x & 0xffffu)) * (h16)16.0f);
            cy2 = h2s(hfrom((uint16_t)(in.x >> 16)) * (h16)16.0f);
            cz2 = h2s(hfrom((uint16_t)(in.y & 0xffffu)) * (h16)16.0f);
            o2 = h2s(hfrom((uint16_t)(in.y >> 16)));
            cr2 = h2s((h16)(float)(in.z & 0xffu));
            cg2 = h2s((h16)(float)((in.z >> 8) & 0xffu));
            cb2 = h2s((h16)(float)((in.z >> 16) & 0xffu));
        }

        // ---- pixel-pair state at the bucket start (:1095-1136), four pairs per lane
        if (cnt) {
            const uint32_t slot0 = (first - b * (uint32_t)kBucket) / (uint32_t)kBucket + tile;
            const uint2* ck = ckpt + (size_t)(b > 0 ? slot0 + b - 1u : 0u) * kTilePixels;
#pragma unroll
            for (uint32_t r = 0; r < 4; ++r) {
                const uint32_t i = l + 32u * r;   // pair index 0..127
                const uint32_t e = 2u * i, local_tile = e >> 6, intile = e & 63u;
                const uint32_t dx_ = (intile & 7u) + (local_tile & 1u) * 8u, dy_ = (intile >> 3) + (local_tile >> 1) * 8u;
                const uint32_t px = gx * 16u + dx_, py = gy * 16u + dy_;
                const bool start_valid = (gx * 16u + (local_tile & 1u) * 8u < cam.width) &&
                                         (gy * 16u + (local_tile >> 1) * 8u < cam.height);
                const bool ok = start_valid && px < cam.width && py < cam.height;
                uint4 a = make_uint4(0u, 0u, 0u, 0u), c = make_uint4(0u, 0u, 0u, 0u);
                if (ok) {
                    const uint32_t pi = tiled_index(py, px, cam.tiled_w);   // even: the pair is one aligned word
                    const uint32_t* gi = (const uint32_t*)(grad_image + pi);
                    const uint32_t* im = (const uint32_t*)(image + pi);
                    const h16x2 G0 = h2from(gi[0]), G1 = h2from(gi[cs / 2u]), G2 = h2from(gi[cs]);
                    const h16x2 I0 = h2from(im[0]), I1 = h2from(im[cs / 2u]), I2 = h2from(im[cs]);
                    uint4 k4 = make_uint4(0u, (uint32_t)kH255 << 16, 0u, (uint32_t)kH255 << 16);
                    if (b > 0) k4 = *(const uint4*)(ck + e);
                    // (C.r | C.g, C.b | T) of the even pixel in k4.x, k4.y, of the odd one in k4.z, k4.w
                    const h16x2 K0 = h2(hfrom((uint16_t)(k4.x & 0xffffu)), hfrom((uint16_t)(k4.z & 0xffffu)));
                    const h16x2 K1 = h2(hfrom((uint16_t)(k4.x >> 16)), hfrom((uint16_t)(k4.z >> 16)));
                    const h16x2 K2 = h2(hfrom((uint16_t)(k4.y & 0xffffu)), hfrom((uint16_t)(k4.w & 0xffffu)));
                    const h16x2 KT = h2(hfrom((uint16_t)(k4.y >> 16)), hfrom((uint16_t)(k4.w >> 16)));
                    const h16x2 sc = h2s(hfrom(kH255));
                    a = make_uint4(h2bits(G0), h2bits(G1), h2bits(G2), h2bits(h2_fma(I0, sc, -K0)));
                    c = make_uint4(h2bits(h2_fma(I1, sc, -K1)), h2bits(h2_fma(I2, sc, -K2)),
                                   h2bits(KT * h2s(hfrom(kHUnscale))), 0u);
                }
                c.w = (uint32_t)hbits((h16)(float)dx_) | ((uint32_t)hbits((h16)(float)dy_) << 16);
                s_pair[0][w][half][i] = make_uint4(a.x, a.y, a.z, c.w);
                s_pair[1][w][half][i] = make_uint4(a.w, c.x, c.y, c.z);
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

        // ---- the pipeline (:1194-1355)
        h16x2 a_mx = h2s((h16)0.f), a_my = a_mx, a_ax = a_mx, a_ay = a_mx, a_cx = a_mx, a_cy = a_mx, a_cz = a_mx;
        h16x2 a_op = a_mx, a_r = a_mx, a_g = a_mx, a_b = a_mx;
        // lane l at step s works on pair s - l: its static words from LDS
        // (loaded a step ahead), its state (colour after, T) from lane l - 1
        // (lanes 0 and 32: the pair's state at the bucket start, from LDS).
        // Steps 31..127 have every lane on a pair (no per-lane test) and steps
        // below 128 start a pair at lanes 0 and 32; the loops run two steps
        // per iteration, so the staged words need no register copy.
        uint32_t st[4] = {0u, 0u, 0u, 0u};
        const uint32_t a_lo = lds_addr(&s_pair[0][w][half][0]), a_hi = a_lo + 127u * 16u;
        uint32_t a = a_lo + 16u * (1u - l);   // entry s - l + 1 at step s (unclamped)
        const uint32_t cmax = max(readlane_u32(cnt, 0), readlane_u32(cnt, 32));
        const uint32_t steps = cmax ? 128u + cmax - 1u : 0u;
        uint4 cur = lds_u4_at(min(max(a - 16u, a_lo), a_hi));
        auto step = [&](uint32_t s, const uint4& words, auto start, auto check) {
            if constexpr (decltype(start)::value)
                if (l == 0u) {   // pair s's state at the bucket start: entry s of the init words
                    const uint4 c = lds_u4_at(a - 16u + kPairInitOfs);
                    st[0] = c.x; st[1] = c.y; st[2] = c.z; st[3] = c.w;
                }
            bool act = l < cnt;
            if constexpr (decltype(check)::value) act = act && s - l < 128u;
            if (act) {
                const h16x2 G0 = h2from(words.x), G1 = h2from(words.y), G2 = h2from(words.z);
                h16x2 Ca0 = h2from(st[0]), Ca1 = h2from(st[1]), Ca2 = h2from(st[2]);
                const h16x2 T = h2from(st[3]);
                const h16x2 off = h2from(words.w);
                const h16x2 offx = h2s(off.x), offy = h2s(off.y);
                const h16x2 dlx = h2_fma(inv16, -offx, mxp);
                const h16x2 dly = h2_fma(inv16, -offy, my2);
                const h16x2 cx_dx = cx2 * dlx, cy_dx = cy2 * dlx, cz_dy = cz2 * dly, cy_dy = cy2 * dly;
                const h16x2 cz_dyy = dly * cz_dy, cy_dxy = dlx * cy_dy;
                const h16x2 quad = h2_fma(dlx, cx_dx, cz_dyy);
                const h16x2 prep_x = cx_dx + cy_dy;
                const h16x2 gss = h2_exp2(h2_relu(h2_fma(h05, quad, cy_dxy)) * nk);
                const h16x2 prep_y = cy_dx + cz_dy;
                const h16x2 alpha_p = o2 * gss;
                const h16x2 cdg = h2_fma(cr2, G0, h2_fma(cg2, G1, cb2 * G2));
                const h16x2 alpha = h2_min(alpha_p, maxa);
                const h16x2 bw = T * alpha;
                const h16x2 oma = one - alpha;
                a_r = h2_fma(bw, G0, a_r);
                a_g = h2_fma(bw, G1, a_g);
                a_b = h2_fma(bw, G2, a_b);
                Ca0 = h2_fma(-bw, cr2, Ca0);
                Ca1 = h2_fma(-bw, cg2, Ca1);
                Ca2 = h2_fma(-bw, cb2, Ca2);
                const h16x2 cadg = h2_fma(Ca0, G0, h2_fma(Ca1, G1, Ca2 * G2));
                const h16x2 dal = h2_fma(T, cdg, -h2_div_blend(cadg, oma));   // oma in [0x1.4p-7, 1]
                const h16x2 part = alpha * dal;
                a_op = part + a_op;
                const h16x2 dxdx = dlx * dlx, dxdy = dlx * dly, dydy = dly * dly;
                a_cx = part * dxdx + a_cx;
                a_cy = part * dxdy + a_cy;
                a_cz = part * dydy + a_cz;
                const h16x2 nT = T * oma;
                const h16x2 dmx = part * prep_x, dmy = part * prep_y;
                a_mx = dmx + a_mx;
                a_my = dmy + a_my;
                a_ax = h2from(h2bits(dmx) & 0x7fff7fffu) + a_ax;
                a_ay = h2from(h2bits(dmy) & 0x7fff7fffu) + a_ay;
                st[0] = h2bits(Ca0);
                st[1] = h2bits(Ca1);
                st[2] = h2bits(Ca2);
                st[3] = h2bits(nT);
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) st[q] = shr1(st[q]);
            a += 16u;
        };
        // the next step's static words; clamped to the half's entries where
        // some lane is off its pair (steps 31..127 read entries 1..128: entry
        // 128, the word after the half's last, lies inside s_pair and is read
        // only by lane 0 for step 128, where it is off its pair)
        auto next_words = [&](auto check) {
            if constexpr (decltype(check)::value)
                return lds_u4_at(min(max(a, a_lo), a_hi));
            else
                return lds_u4_at(a);
        };
        auto run = [&](uint32_t s, uint32_t end, auto start, auto check) {
            for (; s + 1u < end; s += 2u) {
                const uint4 n = next_words(check);
                step(s, cur, start, check);
                cur = next_words(check);
                step(s + 1u, n, start, check);
            }
            if (s < end) {
                const uint4 n = next_words(check);
                step(s, cur, start, check);
                cur = n;
            }
        };
        using yes = std::true_type;
        using no = std::false_type;
        if (steps) {
            run(0u, 31u, yes{}, yes{});        // lanes l <= s on a pair
            run(31u, 128u, yes{}, no{});       // every lane on a pair
            run(128u, steps, no{}, yes{});     // lanes l > s - 128 on a pair
        }

        // ---- the bucket's record (:1357-1387), rounded as the reference's atomics receive it
        if (l < cnt) {
            auto sum = [](h16x2 v) { return (float)v.x + (float)v.y; };
            float4* dst = records + 3 * (size_t)slot;
            const float o = (float)o2.x;
            dst[0] = make_float4((float)h_rn(-sum(a_mx) / 255.0f), (float)h_rn(-sum(a_my) / 255.0f),
                                 (float)h_rn(sum(a_ax) / 255.0f), (float)h_rn(sum(a_ay) / 255.0f));
            dst[1] = make_float4((float)h_rn(-128.0f * sum(a_cx) / 255.0f), (float)h_rn(-128.0f * sum(a_cy) / 255.0f),
                                 (float)h_rn(-128.0f * sum(a_cz) / 255.0f), (float)h_rn(sum(a_r)));
            // [11]: the instance index (bits), for tests; the sums do not read it
            dst[2] = make_float4((float)h_rn(sum(a_g)), (float)h_rn(sum(a_b)), (sum(a_op) / 255.0f) * (1.0f - o),
                                 u2f(first + l));
        }
        next = (uint32_t)__builtin_amdgcn_readfirstlane((int)after);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
}

static int g_blocks16 = 0;

void launch_blend16_backward(const CamParams& cam, const uint32_t* inst_vals, const float2* mean2d,
                             const uint4* info, const uint16_t* image, const uint16_t* grad_image, const uint2* ckpt,
                             const uint4* items, BinCtl* ctl, uint32_t* rec_count, const uint32_t* first_slot,
                             float4* records, hipStream_t s) {
    const uint32_t n_tiles = cam.grid_w * cam.grid_h;
    if (n_tiles == 0) return;
    if (g_blocks16 <= 0) {
        int dev = 0, cus = 0, per_cu = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, blend16_backward_kernel, 256, 0) != hipSuccess ||
            per_cu <= 0)
            per_cu = 4;
        g_blocks16 = cus * per_cu;
    }
    blend16_backward_kernel<<<(uint32_t)g_blocks16, 256, 0, s>>>(cam, inst_vals, mean2d, info, image, grad_image,
                                                                  ckpt, items, ctl, rec_count, first_slot, records);
}

}  // namespace tgs
