// Backward of the blend: one (tile, 32-Gaussian bucket) work item per wave64,
// four pixels per lane.
//
// Reference: blend_backward_cu2 (tinygs/src/rasterizer/fastgs_ours/
// kernels_backward.cuh:675-927) assigns one warp per 32-Gaussian bucket and
// restarts each bucket from the (colour, transmittance) checkpoint written by
// the forward (kernels_forward.cuh:644-653); inside a bucket it runs the
// backward recurrence with sigma clamped at 0 and no 1/255 test.
//
// MI355X design:
//   * the work item is the same bucket, but the wave is pixel-parallel: lane
//     l owns pixels l, 64 + l, 128 + l, 192 + l of the tile, i.e. one lane of
//     each 8x8 block, so every image / gradient / checkpoint access of a
//     block is one contiguous 256-byte (1 KiB for checkpoints) run;
//   * the 32 records of the bucket are staged in a wave-private LDS slice and
//     read back as three broadcast float4 per Gaussian;
//   * per Gaussian, each lane first sums its four pixels in registers, then
//     the 11 sums are reduced across the wave once (gfx950
//     v_permlane32_swap / v_permlane16_swap + DPP row butterfly), so the
//     cross-lane work is shared by 256 pixels;
//   * waves take items from a device-side list (built by the forward, one
//     entry per bucket below the tile's last contributor, carrying its first
//     instance and count) through 64 queue counters on separate cache lines,
//     so long and short tiles balance across the CUs without every wave
//     contending for one address; the next index is fetched while the
//     current item runs;
//   * no deterministic exp is needed here (the backward makes no threshold
//     decision): exp(-sigma) is v_exp_f32 of sigma * log2(e), with log2(e)
//     folded into the staged conic.
//
// Output: one 12-float record per (primitive, bucket) instead of float
// atomics (device-scope atomics on MI355X are performed at the memory side,
// one DRAM read-modify-write each): [0,1] dL/dmean2d, [2,3] |.| sums
// (absgrad), [4..6] dL/dconic (a, b, c), [7..9] dL/dcolour (masked by
// colour >= 0), [10] sum of alpha * dL/dalpha (times (1 - opacity) later).
// The record of the instance with rank k among its primitive's instances
// (carried through the tile sort) goes to slot first_slot[p] + k of the
// instance slots binning reserved for the primitive; a bit (a non-returning
// atomic OR: for ranks below 32 in the primitive's own mask word, for the
// others in a per-slot bit array) marks it written and a per-primitive
// counter (a non-returning atomic add) counts it: where a record lands does not
// depend on the order in which the buckets finish, so the preprocess
// backward's per-primitive sums run in a fixed order (rank order, the order
// of the primitive's tiles) and a step's gradients repeat bit for bit.
#include "common.h"
#include "kernels.h"

namespace tgs {

constexpr int kBwdVals = 11;
constexpr float kLog2e = 1.4426950408889634f;

// ABS: also sum |dL/dmean2d| per pixel (the densification statistic); the
// sums are only read when densification info is requested.
template <bool ABS>
__global__ void __launch_bounds__(256) blend_backward_kernel(
    CamParams cam, const uint32_t* __restrict__ inst_vals, const uint16_t* __restrict__ inst_ranks,
    const float2* __restrict__ mean2d, const float4* __restrict__ conic_opacity, const float4* __restrict__ color_pt,
    const float* __restrict__ image, const float* __restrict__ grad_image, const uint32_t* __restrict__ n_contrib,
    const float4* __restrict__ ckpt, const uint4* __restrict__ items, BinCtl* __restrict__ ctl,
    uint32_t* __restrict__ rec_bits, uint32_t* __restrict__ rec_mask, uint32_t* __restrict__ rec_count,
    const uint32_t* __restrict__ first_slot, float4* __restrict__ records) {
    __shared__ float4 s_rec[4][3][kBucket];
    __shared__ float s_part[4][kBwdVals + 1][kBucket + 1];   // +1: the four row writers hit four banks

    const uint32_t w = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const int q0 = row_value(lane >> 4);   // first value index this lane's row holds after wave_reduce12
    const uint32_t n_items = ctl->n_items;
    const uint32_t cs = cam.tiled_w * cam.tiled_h * 64u;
    // this wave's queue (its items: bwd_queue_item); its counter has a cache line to itself
    const uint32_t queue = (blockIdx.x * 4u + w) % (uint32_t)kBwdQueues;
    uint32_t* qctr = &ctl->bwd_queue[queue * 32u];
    uint32_t next = 0;
    if (lane == 0) next = atomicAdd(qctr, 1u);
    next = (uint32_t)__builtin_amdgcn_readfirstlane((int)next);

    while (true) {
        const uint32_t it = bwd_queue_item(queue, next);   // increasing in next
        if (it >= n_items) break;
        // fetch the following index now; its latency hides behind this item
        uint32_t after = 0;
        if (lane == 0) after = atomicAdd(qctr, 1u);
        const uint4 item = items[it];
        const uint32_t tile = item.x, b = item.y, first = item.z;
        const int32_t j0 = (int32_t)(b * kBucket);
        const int32_t cnt = (int32_t)item.w;

        // ---- stage the bucket's records (wave-private LDS slice); each of
        // its primitives fills its 2D-gradient record slot at the end of the item
        uint32_t p = 0, slot = 0, rank = 0;
        if ((int32_t)lane < cnt) {
            p = inst_vals[first + lane];
            rank = inst_ranks[first + lane];
            slot = first_slot[p] + rank;
            const float2 m = mean2d[p];
            const float4 co = conic_opacity[p];
            const float4 c = color_pt[p];
            const float hl = 0.5f * kLog2e;
            s_rec[w][0][lane] = make_float4(m.x, m.y, hl * co.x, kLog2e * co.y);
            s_rec[w][1][lane] = make_float4(hl * co.z, co.w, co.x, co.z);
            const uint32_t mask = (c.x >= 0.f ? 1u : 0u) | (c.y >= 0.f ? 2u : 0u) | (c.z >= 0.f ? 4u : 0u);
            s_rec[w][2][lane] = make_float4(__builtin_fmaxf(c.x, 0.f), __builtin_fmaxf(c.y, 0.f),
                                            __builtin_fmaxf(c.z, 0.f), co.y);
            s_part[w][kBwdVals][lane] = u2f(mask);
        }

        // ---- per-pixel state at the bucket start. Pixel s of this lane sits
        // at column x[s & 1], row y[s >> 1] (two columns and two rows 8 apart)
        const uint32_t gx = tile % cam.grid_w, gy = tile / cam.grid_w;
        const uint32_t slot0 = (first - (uint32_t)j0) / (uint32_t)kBucket + tile;   // tile's first checkpoint slot
        const float pcx0 = (float)(gx * 16u + (lane & 7u)) + 0.5f, pcx1 = pcx0 + 8.0f;
        const float pcy0 = (float)(gy * 16u + (lane >> 3)) + 0.5f, pcy1 = pcy0 + 8.0f;
        float g0[4], g1[4], g2[4], Tb[4], AG[4];
        int32_t lk[4];
        uint32_t pix[4];
        bool in[4];
        // two dependent rounds of loads for all four pixels: contributor
        // counts, then colour / gradient / checkpoint (a checkpoint slot of
        // an existing bucket is always allocated, whatever the pixel)
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const uint32_t px = gx * 16u + (uint32_t)(s & 1) * 8u + (lane & 7u);
            const uint32_t py = gy * 16u + (uint32_t)(s >> 1) * 8u + (lane >> 3);
            in[s] = px < cam.width && py < cam.height;
            // outside pixels read element 0 (always allocated) and are masked below
            pix[s] = in[s] ? tiled_index(py, px, cam.tiled_w) : 0u;
            lk[s] = (int32_t)n_contrib[pix[s]] - j0;
        }
        const size_t ck_base = (size_t)(b > 0 ? slot0 + b - 1u : 0u) * kTilePixels + lane;
        int32_t kmax = 0;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const uint32_t pi = pix[s];
            const float i0 = image[pi], i1 = image[pi + cs], i2 = image[pi + 2 * cs];
            const float q0v = grad_image[pi], q1v = grad_image[pi + cs], q2v = grad_image[pi + 2 * cs];
            float4 ck = ckpt[ck_base + (uint32_t)s * 64u];
            if (b == 0) ck = make_float4(0.f, 0.f, 0.f, 1.f);
            const bool act = in[s] && lk[s] > 0;
            lk[s] = act ? lk[s] : 0;
            kmax = max(kmax, lk[s]);
            g0[s] = act ? q0v : 0.f; g1[s] = act ? q1v : 0.f; g2[s] = act ? q2v : 0.f;
            Tb[s] = act ? ck.w : 0.f;
            // (colour still to come behind this Gaussian) . dL/dpixel, carried as
            // one scalar: it drops by wgt * (colour . dL/dpixel) per Gaussian
            AG[s] = act ? __builtin_fmaf(i2 - ck.z, q2v, __builtin_fmaf(i1 - ck.y, q1v, (i0 - ck.x) * q0v)) : 0.f;
        }
        kmax = min((int32_t)wave_max_u32((uint32_t)kmax), cnt);
        // bit k: some pixel's last contributor in this bucket is k - 1; from
        // Gaussian k on its transmittance and remaining colour are zero, which
        // makes every later term of that pixel exactly zero
        uint32_t stops = 0;
#pragma unroll
        for (int s = 0; s < 4; ++s)
            stops |= (lk[s] > 0 && lk[s] < kmax) ? 1u << lk[s] : 0u;
        stops = wave_or_u32(stops);
        wave_lds_sync();

        // Gaussian k of the bucket: updates the pixels' state and leaves the
        // wave's per-lane sums in acc[0..8] (and the |dL/dmean2d| sums in 9, 10)
        auto gaussian = [&](int32_t k, float* acc) {
            const float4 r0 = s_rec[w][0][k];   // mx, my, a/2 L, b L
            const float4 r1 = s_rec[w][1][k];   // c/2 L, opacity, a, c
            const float4 r2 = s_rec[w][2][k];   // clamped colour, b
            if ((stops >> k) & 1u) {
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    Tb[s] = lk[s] == k ? 0.f : Tb[s];
                    AG[s] = lk[s] == k ? 0.f : AG[s];
                }
            }
            // offsets of the two columns and rows; sigma' = X (A X + B Y) + C Y^2
            // with its X and Y^2 parts formed once per column / row
            const float X[2] = {r0.x - pcx0, r0.x - pcx1}, Y[2] = {r0.y - pcy0, r0.y - pcy1};
            const float AX[2] = {r0.z * X[0], r0.z * X[1]};
            const float CYY[2] = {(r1.x * Y[0]) * Y[0], (r1.x * Y[1]) * Y[1]};
            acc[11] = 0.f;
            if constexpr (!ABS) acc[9] = acc[10] = 0.f;
            float pp[4];
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const int xi = s & 1, yi = s >> 1;
                const float sg = __builtin_fmaf(X[xi], __builtin_fmaf(r0.w, Y[yi], AX[xi]), CYY[yi]);
                const float G = __builtin_amdgcn_exp2f(-__builtin_fmaxf(sg, 0.f));
                const float ab = __builtin_fminf(r1.y * G, kMaxAlpha);
                const float wgt = Tb[s] * ab;
                const float cg = __builtin_fmaf(r2.z, g2[s], __builtin_fmaf(r2.y, g1[s], r2.x * g0[s]));
                AG[s] = __builtin_fmaf(-wgt, cg, AG[s]);
                const float oma = 1.0f - ab;
                const float dalpha = __builtin_fmaf(Tb[s], cg, -(AG[s] * __builtin_amdgcn_rcpf(oma)));
                pp[s] = ab * dalpha;
                // colour sums; pixel 0 starts each (no add of a zero)
                acc[0] = s == 0 ? wgt * g0[s] : __builtin_fmaf(wgt, g0[s], acc[0]);
                acc[1] = s == 0 ? wgt * g1[s] : __builtin_fmaf(wgt, g1[s], acc[1]);
                acc[2] = s == 0 ? wgt * g2[s] : __builtin_fmaf(wgt, g2[s], acc[2]);
                if constexpr (ABS) {   // |dL/dmean2d| needs each pixel's own value
                    const float hp = pp[s] * X[xi], hq = pp[s] * Y[yi];
                    const float gmx = __builtin_fmaf(hp, r1.z, hq * r2.w);
                    const float gmy = __builtin_fmaf(hp, r2.w, hq * r1.w);
                    acc[9] = s == 0 ? __builtin_fabsf(gmx) : acc[9] + __builtin_fabsf(gmx);
                    acc[10] = s == 0 ? __builtin_fabsf(gmy) : acc[10] + __builtin_fabsf(gmy);
                }
                Tb[s] *= oma;
            }
            // sums of pp, pp X^2, pp X Y, pp Y^2, pp X, pp Y over the four pixels
            // from the column sums (pixels 0 + 2, 1 + 3) and row sums (0 + 1, 2 + 3)
            {
                const float R0 = pp[0] + pp[1], R1 = pp[2] + pp[3];
                const float C0 = pp[0] + pp[2], C1 = pp[1] + pp[3];
                acc[3] = R0 + R1;
                acc[4] = __builtin_fmaf(X[0] * X[0], C0, (X[1] * X[1]) * C1);
                acc[5] = __builtin_fmaf(Y[0], __builtin_fmaf(X[0], pp[0], X[1] * pp[1]),
                                        Y[1] * __builtin_fmaf(X[0], pp[2], X[1] * pp[3]));
                acc[6] = __builtin_fmaf(Y[0] * Y[0], R0, (Y[1] * Y[1]) * R1);
                acc[7] = __builtin_fmaf(X[0], C0, X[1] * C1);
                acc[8] = __builtin_fmaf(Y[0], R0, Y[1] * R1);
            }
        };
        auto store = [&](int32_t k, const float* t, int nt) {
            if ((lane & 15u) == 0u)
                for (int m = 0; m < nt; ++m)
                    if (4 * m + q0 < kBwdVals) s_part[w][4 * m + q0][k] = t[m];
        };
        int32_t k = 0;
        if constexpr (!ABS) {
            // two Gaussians per reduction (values 9 and 10 stay the zeros written below)
            for (; k + 1 < kmax; k += 2) {
                float acc2[18], acc1[12];
                gaussian(k, acc1);
#pragma unroll
                for (int q = 0; q < 9; ++q) acc2[q] = acc1[q];
                gaussian(k + 1, acc1);
#pragma unroll
                for (int q = 0; q < 9; ++q) acc2[9 + q] = acc1[q];
                float t[5];
                wave_reduce18(acc2, t);
                if ((lane & 15u) == 0u) {
#pragma unroll
                    for (int m = 0; m < 5; ++m) {
                        const int i = 4 * m + q0;   // value i % 9 of Gaussian k + i / 9
                        if (i < 18) s_part[w][i % 9][k + i / 9] = t[m];
                    }
                    if (q0 == 0) {
                        s_part[w][9][k] = s_part[w][10][k] = 0.f;
                        s_part[w][9][k + 1] = s_part[w][10][k + 1] = 0.f;
                    }
                }
            }
        }
        for (; k < kmax; ++k) {
            float acc[12];
            gaussian(k, acc);
            float t[3];
            if constexpr (ABS)
                wave_reduce12(acc, t);
            else
                wave_reduce9(acc, t);   // values 9-11 are zero: their swaps are skipped
            store(k, t, 3);
        }
        wave_lds_sync();

        if ((int32_t)lane < cnt) {
            const uint32_t k = lane;
            const bool ev = (int32_t)lane < kmax;   // evaluated (always true: kmax == cnt by construction)
            const uint32_t mask = f2u(s_part[w][kBwdVals][k]);
            auto val = [&](int q) { return ev ? s_part[w][q][k] : 0.f; };
            // record order: mean2d(2), abs(2), conic(3), colour(3), alpha partial, 0
            float4* dst = records + 3 * (size_t)slot;
            // dL/dmean2d = conic . (sum pp X, sum pp Y), applied once per Gaussian
            const float a = s_rec[w][1][k].z, c = s_rec[w][1][k].w, bq = s_rec[w][2][k].w;
            const float gmx = __builtin_fmaf(a, val(7), bq * val(8));
            const float gmy = __builtin_fmaf(bq, val(7), c * val(8));
            dst[0] = make_float4(-gmx, -gmy, val(9), val(10));
            dst[1] = make_float4(-0.5f * val(4), -0.5f * val(5), -0.5f * val(6), (mask & 1u) ? val(0) : 0.f);
            dst[2] = make_float4((mask & 2u) ? val(1) : 0.f, (mask & 4u) ? val(2) : 0.f, val(3), 0.f);
            // the mark: ranks below 32 in the primitive's own mask word, the rest by slot
            if (rank < 32u)
                __hip_atomic_fetch_or(rec_mask + p, 1u << rank, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            else
                __hip_atomic_fetch_or(rec_bits + (slot >> 5), 1u << (slot & 31u), __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_fetch_add(rec_count + p, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        next = (uint32_t)__builtin_amdgcn_readfirstlane((int)after);
        wave_lds_sync();
    }
}

// Rows the blend backward will write (each primitive of an item's bucket
// range takes one record, whatever its pixels), marked from the forward's
// items: two items per wave, lane & 31 = the bucket's Gaussian. rows is
// zeroed by the caller.
__global__ void __launch_bounds__(256) backward_rows_kernel(const uint4* __restrict__ items,
                                                            const uint32_t* __restrict__ inst_vals,
                                                            const BinCtl* __restrict__ ctl,
                                                            uint8_t* __restrict__ rows) {
    const uint32_t n_items = ctl->n_items;
    const uint32_t l = threadIdx.x & 31u;
    for (uint32_t it = blockIdx.x * 8u + (threadIdx.x >> 5); it < n_items; it += gridDim.x * 8u) {
        const uint4 item = items[it];
        if (l < item.w) rows[inst_vals[item.z + l]] = 1u;
    }
}

void launch_backward_rows(const uint4* items, const uint32_t* inst_vals, const BinCtl* ctl, uint8_t* rows,
                          hipStream_t s) {
    backward_rows_kernel<<<1024, 256, 0, s>>>(items, inst_vals, ctl, rows);
}

static int g_blocks = 0;

void launch_blend_backward(const CamParams& cam, const uint32_t* inst_vals, const uint16_t* inst_ranks,
                           const float2* mean2d, const float4* conic_opacity, const float4* color_pt,
                           const float* image, const float* grad_image, const uint32_t* n_contrib, const float4* ckpt,
                           const uint4* items, BinCtl* ctl, uint32_t* rec_bits, uint32_t* rec_mask,
                           uint32_t* rec_count, const uint32_t* first_slot, float4* records, bool with_abs,
                           hipStream_t s) {
    const uint32_t n_tiles = cam.grid_w * cam.grid_h;
    if (n_tiles == 0) return;
    if (g_blocks <= 0) {
        // persistent workgroups: exactly as many as can be resident at once
        int dev = 0, cus = 0, per_cu = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, blend_backward_kernel<true>, 256, 0) !=
                hipSuccess ||
            per_cu <= 0)
            per_cu = 4;
        g_blocks = cus * per_cu;
    }
    if (with_abs)
        blend_backward_kernel<true><<<(uint32_t)g_blocks, 256, 0, s>>>(
            cam, inst_vals, inst_ranks, mean2d, conic_opacity, color_pt, image, grad_image, n_contrib, ckpt, items,
            ctl, rec_bits, rec_mask, rec_count, first_slot, records);
    else
        blend_backward_kernel<false><<<(uint32_t)g_blocks, 256, 0, s>>>(
            cam, inst_vals, inst_ranks, mean2d, conic_opacity, color_pt, image, grad_image, n_contrib, ckpt, items,
            ctl, rec_bits, rec_mask, rec_count, first_slot, records);
}

}  // namespace tgs
