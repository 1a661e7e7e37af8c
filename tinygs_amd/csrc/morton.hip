// Morton (Z-order) ordering of the Gaussians by their means, for the
// storage reorder of Orchestrator::reorder_gaussians
// (tinygs/src/orchestrator.cu:26-90, 1038-1061).
//
// The reference: bounding box of the means (thrust reductions with fminf /
// fmaxf), per-axis inverse extents 1 / max(max - min, 1e-8) in float on the
// host, each coordinate normalised to [0, 1] and clamped, scaled by 1023 and
// truncated to 10 bits, the three 10-bit values interleaved into a 30-bit
// code (x in bits 3k, y in 3k + 1, z in 3k + 2), then a stable radix sort of
// (code, index) over those 30 bits; the sorted indices are the new order
// (row i takes old row indices[i]).
//
// Here: one grid-strided pass of per-workgroup minima / maxima, one
// workgroup that folds them and forms the inverse extents with the same
// float division, one pass that writes the codes, and the binning's stable
// LSD radix sort (its depth-sort configuration: 4096 keys per workgroup,
// digits up to 9 bits) in four passes of 8, 8, 7 and 7 bits. min / max are
// exact, so the result does not depend on the reduction order.
#include "common.h"
#include "kernels.h"

namespace tgs {

constexpr int kMortonThreads = 256;
constexpr int kMortonBlocks = 1024;   // partial min / max workgroups at most

__global__ void __launch_bounds__(kMortonThreads) morton_bounds_partial_kernel(const float* __restrict__ means,
                                                                               int64_t n,
                                                                               float* __restrict__ partial) {
    __shared__ float s_v[6][kMortonThreads / 64];
    float lo[3] = {3.402823466e+38f, 3.402823466e+38f, 3.402823466e+38f};
    float hi[3] = {-3.402823466e+38f, -3.402823466e+38f, -3.402823466e+38f};
    for (int64_t i = (int64_t)blockIdx.x * kMortonThreads + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * kMortonThreads) {
#pragma unroll
        for (int a = 0; a < 3; ++a) {
            const float v = means[3 * i + a];
            lo[a] = fminf(lo[a], v);
            hi[a] = fmaxf(hi[a], v);
        }
    }
#pragma unroll
    for (int a = 0; a < 3; ++a)
        for (int off = 32; off > 0; off >>= 1) {
            lo[a] = fminf(lo[a], __shfl_down(lo[a], off, 64));
            hi[a] = fmaxf(hi[a], __shfl_down(hi[a], off, 64));
        }
    const uint32_t lane = threadIdx.x & 63u, w = threadIdx.x >> 6;
    if (lane == 0u)
        for (int a = 0; a < 3; ++a) {
            s_v[a][w] = lo[a];
            s_v[3 + a][w] = hi[a];
        }
    __syncthreads();
    if (threadIdx.x < 6u) {
        const int k = (int)threadIdx.x;
        float v = s_v[k][0];
        for (int q = 1; q < kMortonThreads / 64; ++q) v = k < 3 ? fminf(v, s_v[k][q]) : fmaxf(v, s_v[k][q]);
        partial[6 * blockIdx.x + k] = v;
    }
}

// box[0..2] = min, box[3..5] = 1 / max(max - min, 1e-8) (orchestrator.cu:49-51)
__global__ void __launch_bounds__(64) morton_bounds_final_kernel(const float* __restrict__ partial, int n_partial,
                                                                 float* __restrict__ box) {
    if (threadIdx.x >= 3u) return;
    const int a = (int)threadIdx.x;
    float lo = 3.402823466e+38f, hi = -3.402823466e+38f;
    for (int b = 0; b < n_partial; ++b) {
        lo = fminf(lo, partial[6 * b + a]);
        hi = fmaxf(hi, partial[6 * b + 3 + a]);
    }
    const float ext = hi - lo;
    box[a] = lo;
    box[3 + a] = 1.0f / (ext < 1e-8f ? 1e-8f : ext);   // std::max(ext, 1e-8f)
}

// The 10 low bits of v spread to bits 0, 3, 6, ..., 27 (shift-and-mask
// spreading: each step moves the upper half of every group apart).
__device__ __forceinline__ uint32_t spread3(uint32_t v) {
    v &= 0x3ffu;
    v = (v | (v << 16)) & 0x030000ffu;
    v = (v | (v << 8)) & 0x0300f00fu;
    v = (v | (v << 4)) & 0x030c30c3u;
    v = (v | (v << 2)) & 0x09249249u;
    return v;
}

__global__ void __launch_bounds__(kMortonThreads) morton_codes_kernel(const float* __restrict__ means, int64_t n,
                                                                      const float* __restrict__ box,
                                                                      uint32_t* __restrict__ codes,
                                                                      uint32_t* __restrict__ index) {
    const int64_t i = (int64_t)blockIdx.x * kMortonThreads + threadIdx.x;
    if (i >= n) return;
    uint32_t q[3];
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        // orchestrator.cu:61-68: normalise, clamp to [0, 1], scale by 1023, truncate
        const float t = fminf(fmaxf((means[3 * i + a] - box[a]) * box[3 + a], 0.0f), 1.0f);
        q[a] = (uint32_t)(t * 1023.0f);
    }
    codes[i] = spread3(q[0]) | (spread3(q[1]) << 1) | (spread3(q[2]) << 2);
    index[i] = (uint32_t)i;
}

int64_t morton_scratch_words(int64_t n) {
    const int64_t nn = n > 0 ? n : 1;
    // codes and indices, double-buffered; radix count matrix; partials + box
    return 4 * nn + radix_count_entries(nn, true) + 6 * kMortonBlocks + 8;
}

int morton_order(const float* means, int64_t n, uint32_t* indices, uint32_t* scratch, uint64_t* status,
                 BinCtl* ctl, hipStream_t s) {
    if (n <= 0) return 0;
    const int64_t nn = n;
    uint32_t* codes0 = scratch;
    uint32_t* codes1 = codes0 + nn;
    uint32_t* idx0 = codes1 + nn;
    uint32_t* idx1 = idx0 + nn;
    uint32_t* counts = idx1 + nn;
    float* partial = (float*)(counts + radix_count_entries(nn, true));
    float* box = partial + 6 * kMortonBlocks;
    const int blocks = (int)std::min<int64_t>(kMortonBlocks, (n + kMortonThreads - 1) / kMortonThreads);
    morton_bounds_partial_kernel<<<blocks, kMortonThreads, 0, s>>>(means, n, partial);
    morton_bounds_final_kernel<<<1, 64, 0, s>>>(partial, blocks, box);
    morton_codes_kernel<<<(unsigned)((n + kMortonThreads - 1) / kMortonThreads), kMortonThreads, 0, s>>>(
        means, n, box, codes0, idx0);
    uint32_t* keys[2] = {codes0, codes1};
    uint32_t* vals[2] = {idx0, idx1};
    const int shifts[4] = {0, 8, 16, 23}, bits[4] = {8, 8, 7, 7};
    uint32_t epoch = 0;
    const int sel = radix_sort(keys, vals, nullptr, nullptr, n, true, 4, shifts, bits, counts,
                               ctl->tickets + kTicketDepth, status, &ctl->epoch_base, epoch, &ctl->err, nullptr,
                               nullptr, nullptr, nullptr, 0u, nullptr, nullptr, nullptr, s);
    if (sel < 0) return -1;
    // (a failed copy surfaces at the caller's error check after the wait)
    (void)hipMemcpyAsync(indices, vals[sel], sizeof(uint32_t) * (size_t)n, hipMemcpyDeviceToDevice, s);
    return 0;
}

// orchestrator.cu:1023-1032 (densification_update): out[i] = info[indices[i]], 16-byte rows
__global__ void __launch_bounds__(256) rows16_gather_kernel(const uint4* __restrict__ src, uint4* __restrict__ dst,
                                                            const uint32_t* __restrict__ indices, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) dst[i] = src[indices[i]];
}

void launch_rows16_gather(const void* src, void* dst, const uint32_t* indices, int64_t n, hipStream_t s) {
    if (n <= 0) return;
    rows16_gather_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>((const uint4*)src, (uint4*)dst, indices, n);
}

}  // namespace tgs
