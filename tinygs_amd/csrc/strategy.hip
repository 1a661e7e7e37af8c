// Densification of the Gaussian set: the kernels behind DefaultStrategy
// (tinygs/src/strategy/default.cu:26-341), GPUGaussian3d::remove / append
// (tinygs/src/core/gpu_gaussian.cu:117-170), SimpleAdam::remove / duplicate /
// reset_opacity (tinygs/src/optim/simple_adam.cu:841-985) and the random
// numbers of the split (tinygs/include/tinygs/random/device.cuh:38-79,
// pcg32.hpp).
//
// MI355X layout: one thread per Gaussian (or per grown Gaussian), 256-thread
// workgroups. Index lists (grown sources, kept rows) are built in index order
// by chunk-local compaction: a counting pass writes one count per chunk of
// 2048 flags, the host scans the counts (it needs the totals anyway to size
// the new arrays) and a second pass writes each chunk's run. No device-wide
// counter (returning atomics on one address serialise on MI355X).
//
// Transcendentals are the deterministic det_expf / det_logf with IEEE
// division and square root, so every result is reproducible by the CPU
// restatement bit for bit (the reference compiles with fast math, whose
// results are not reproducible).
#include "common.h"
#include "kernels.h"
#include "pcg32.h"

namespace tgs {

// logit of common.hpp:362-364: -log(1 / clamp(x, 1e-9, 1 - 1e-9) - 1)
TGS_HD float det_logit(float x) {
    const float c = fminf(fmaxf(x, 1e-9f), 1.0f - 1e-9f);
    return -det_logf(1.0f / c - 1.0f);
}
// logistic of common.hpp:358-360
TGS_HD float det_logistic(float x) { return 1.0f / (1.0f + det_expf(-x)); }

// Thread i of ceil(n / 4) takes stream positions 4 i .. 4 i + 3 for the
// elements i, i + T, i + 2 T, i + 3 T (T = thread count), as the reference's
// generate_random_kernel does; the caller then advances the stream by n.
__global__ void random_logistic_kernel(int64_t n, int64_t n_threads, uint64_t state, uint64_t inc, float mean,
                                       float stddev, float* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_threads) return;
    uint64_t s = pcg_advance(state, inc, (uint64_t)(4 * i));
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t idx = i + n_threads * j;
        if (idx >= n) return;
        const float u = pcg_float(s, inc);
        out[idx] = det_logit(u) * stddev * 0.551328895f + mean;
    }
}

void launch_random_logistic(uint64_t state, uint64_t inc, int64_t n, float mean, float stddev, float* out,
                            hipStream_t s) {
    if (n <= 0) return;
    const int64_t threads = (n + 3) / 4;
    random_logistic_kernel<<<(unsigned)((threads + 255) / 256), 256, 0, s>>>(n, threads, state, inc, mean, stddev,
                                                                            out);
}

// ------------------------------------------------------------------ flags -> index lists

constexpr int kListRounds = 8;
constexpr int kListChunk = 256 * kListRounds;
static_assert(kListChunk == kListChunkElems, "chunk size shared with the host");

int64_t list_chunks(int64_t n) { return n > 0 ? (n + kListChunk - 1) / kListChunk : 0; }

// counts[c] = (flags != 0, flags == 1) over chunk c
__global__ void __launch_bounds__(256) flag_count_kernel(const uint8_t* __restrict__ flags, int64_t n,
                                                         uint2* __restrict__ counts) {
    __shared__ uint32_t s_a[4], s_b[4];
    const uint32_t t = threadIdx.x, lane = t & 63u, w = t >> 6;
    const int64_t base = (int64_t)blockIdx.x * kListChunk + t;
    uint32_t a = 0, b = 0;
#pragma unroll
    for (int r = 0; r < kListRounds; ++r) {
        const int64_t i = base + (int64_t)r * 256;
        const uint8_t f = i < n ? flags[i] : (uint8_t)0;
        a += f != 0 ? 1u : 0u;
        b += f == 1 ? 1u : 0u;
    }
    a = wave_sum_u32(a);
    b = wave_sum_u32(b);
    if (lane == 0) {
        s_a[w] = a;
        s_b[w] = b;
    }
    __syncthreads();
    if (t == 0) counts[blockIdx.x] = make_uint2(s_a[0] + s_a[1] + s_a[2] + s_a[3], s_b[0] + s_b[1] + s_b[2] + s_b[3]);
}

// out[offsets[c] + rank] = i for every i of chunk c with flags[i] != 0, in index order
__global__ void __launch_bounds__(256) flag_compact_kernel(const uint8_t* __restrict__ flags, int64_t n,
                                                           const uint32_t* __restrict__ offsets,
                                                           int32_t* __restrict__ out) {
    __shared__ uint32_t s_rw[4 * kListRounds];
    const uint32_t t = threadIdx.x;
    const int64_t base = (int64_t)blockIdx.x * kListChunk + t;
    uint32_t v[kListRounds], ex[kListRounds];
#pragma unroll
    for (int r = 0; r < kListRounds; ++r) {
        const int64_t i = base + (int64_t)r * 256;
        v[r] = (i < n && flags[i] != 0) ? 1u : 0u;
    }
    uint32_t total;
    striped_scan_u32<kListRounds>(v, ex, &total, s_rw);
    const uint32_t o = offsets[blockIdx.x];
#pragma unroll
    for (int r = 0; r < kListRounds; ++r)
        if (v[r]) out[o + ex[r]] = (int32_t)(base + (int64_t)r * 256);
}

// offsets[c] = exclusive prefix of counts[c].x over the chunks (c < chunks);
// totals[0] = sum of .x, totals[1] = sum of .y. One 1024-thread workgroup:
// thread t owns a run of consecutive chunks, a workgroup scan of the run
// sums places it.
__global__ void __launch_bounds__(1024) chunk_offsets_kernel(const uint2* __restrict__ counts, int64_t chunks,
                                                             uint32_t* __restrict__ offsets,
                                                             uint32_t* __restrict__ totals) {
    __shared__ uint32_t s_a[16], s_b[16];
    const uint32_t t = threadIdx.x, lane = t & 63u, w = t >> 6;
    const int64_t per = (chunks + 1023) / 1024;
    const int64_t c0 = (int64_t)t * per, c1 = min(c0 + per, chunks);
    uint32_t a = 0, b = 0;
    for (int64_t c = c0; c < c1; ++c) {
        const uint2 v = counts[c];
        a += v.x;
        b += v.y;
    }
    const uint32_t incl = wave_inclusive_scan_u32(a);
    const uint32_t wb = wave_sum_u32(b);
    if (lane == 63u) s_a[w] = incl;
    if (lane == 0u) s_b[w] = wb;
    __syncthreads();
    uint32_t off = 0, ta = 0, tb = 0;
    for (uint32_t k = 0; k < 16u; ++k) {
        off += k < w ? s_a[k] : 0u;
        ta += s_a[k];
        tb += s_b[k];
    }
    uint32_t e = off + incl - a;
    for (int64_t c = c0; c < c1; ++c) {
        offsets[c] = e;
        e += counts[c].x;
    }
    if (t == 0) {
        totals[0] = ta;
        totals[1] = tb;
    }
}

void launch_chunk_offsets(const uint2* counts, int64_t chunks, uint32_t* offsets, uint32_t* totals, hipStream_t s) {
    chunk_offsets_kernel<<<1, 1024, 0, s>>>(counts, chunks, offsets, totals);
}

void launch_flag_count(const uint8_t* flags, int64_t n, uint2* counts, hipStream_t s) {
    if (n <= 0) return;
    flag_count_kernel<<<(unsigned)list_chunks(n), 256, 0, s>>>(flags, n, counts);
}
void launch_flag_compact(const uint8_t* flags, int64_t n, const uint32_t* offsets, int32_t* out, hipStream_t s) {
    if (n <= 0) return;
    flag_compact_kernel<<<(unsigned)list_chunks(n), 256, 0, s>>>(flags, n, offsets, out);
}

// ------------------------------------------------------------------ selection

// default.cu:151-171: grow where the mean 2D gradient (|.| sums with absgrad)
// exceeds grow_grad; split when the largest activated scale exceeds
// grow_scale, else duplicate (1 duplicate, 2 split).
__global__ void densify_select_kernel(int64_t n, const float4* __restrict__ info, const float* __restrict__ scales,
                                      float grow_grad, float grow_scale, int absgrad,
                                      uint8_t* __restrict__ flags) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float4 d = info[i];
    const float accum = absgrad ? d.z : d.y;
    const float grad = accum / fmaxf(d.x, 1.0f);
    uint8_t f = 0;
    if (grad > grow_grad && d.x > 0.0f) {
        const float s = fmaxf(fmaxf(det_expf(scales[3 * i]), det_expf(scales[3 * i + 1])), det_expf(scales[3 * i + 2]));
        f = s > grow_scale ? 2 : 1;
    }
    flags[i] = f;
}

void launch_densify_select(int64_t n, const float4* info, const float* scales, float grow_grad, float grow_scale,
                           int absgrad, uint8_t* flags, hipStream_t s) {
    if (n <= 0) return;
    densify_select_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(n, info, scales, grow_grad, grow_scale, absgrad,
                                                                     flags);
}

// default.cu:306-330: alive when opaque enough, not degenerate, and (unless
// large ones are kept) small in world space and on screen; rows at or past
// n_info (grown in this step) have no screen radius yet.
__global__ void prune_select_kernel(int64_t n, const float* __restrict__ opac, const float* __restrict__ scales,
                                    const float* __restrict__ rots, const float4* __restrict__ info, int64_t n_info,
                                    float scale_limit, float radius_limit, float min_opacity, int prune_large,
                                    uint8_t* __restrict__ alive) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float s = fmaxf(fmaxf(det_expf(scales[3 * i]), det_expf(scales[3 * i + 1])), det_expf(scales[3 * i + 2]));
    const bool not_large_ws = s < scale_limit;
    const bool not_large_ss = i >= n_info || info[i].w < radius_limit;
    const bool not_transparent = det_logistic(opac[i]) > min_opacity;
    const float qs = ((fabsf(rots[4 * i]) + fabsf(rots[4 * i + 1])) + fabsf(rots[4 * i + 2])) + fabsf(rots[4 * i + 3]);
    const bool not_degenerate = qs > 1.1920928955078125e-07f;   // FLT_EPSILON
    alive[i] = (not_transparent && ((not_large_ws && not_large_ss) || !prune_large) && not_degenerate) ? 1 : 0;
}

void launch_prune_select(int64_t n, const float* opac, const float* scales, const float* rots, const float4* info,
                         int64_t n_info, float scale_limit, float radius_limit, float min_opacity, int prune_large,
                         uint8_t* alive, hipStream_t s) {
    if (n <= 0) return;
    prune_select_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(n, opac, scales, rots, info, n_info, scale_limit,
                                                                   radius_limit, min_opacity, prune_large, alive);
}

// ------------------------------------------------------------------ duplicate / split

// default.cu:235-297 for grown Gaussian i (source src[i], target n_old + i):
// rotation and SH are copied; a duplicate copies mean, scale and opacity; a
// split moves source and target by M (r_k * (exp(scale) + 1e-5)) with the
// six logistic numbers r of row i, divides the activated scale by 1.6 and
// sets the opacity to 1 - sqrt(1 - o). M is the glm matrix the reference
// builds from the raw quaternion (its columns are the rows of the usual
// rotation matrix R), so the offset is R^T applied to the scaled numbers.
template <typename ShT>
__global__ void densify_apply_kernel(int64_t n_grow, int64_t n_old, const int32_t* __restrict__ src,
                                     const uint8_t* __restrict__ flags, const float* __restrict__ rnd,
                                     float* __restrict__ means, float* __restrict__ scales,
                                     float* __restrict__ rots, float* __restrict__ opac, ShT* __restrict__ sh0,
                                     ShT* __restrict__ shr) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_grow) return;
    const int64_t s = src[i], t = n_old + i;
    const uint8_t f = flags[s];
    if (f == 0) return;
    const float r = rots[4 * s], x = rots[4 * s + 1], y = rots[4 * s + 2], z = rots[4 * s + 3];
    for (int c = 0; c < 4; ++c) rots[4 * t + c] = rots[4 * s + c];
    for (int c = 0; c < 3; ++c) sh0[3 * t + c] = sh0[3 * s + c];
    for (int c = 0; c < 45; ++c) shr[45 * t + c] = shr[45 * s + c];
    if (f == 1) {
        for (int c = 0; c < 3; ++c) {
            means[3 * t + c] = means[3 * s + c];
            scales[3 * t + c] = scales[3 * s + c];
        }
        opac[t] = opac[s];
        return;
    }
    // columns of M (glm::mat3 takes its nine arguments column by column)
    const float m00 = 1.f - 2.f * (y * y + z * z), m01 = 2.f * (x * y - r * z), m02 = 2.f * (x * z + r * y);
    const float m10 = 2.f * (x * y + r * z), m11 = 1.f - 2.f * (x * x + z * z), m12 = 2.f * (y * z - r * x);
    const float m20 = 2.f * (x * z - r * y), m21 = 2.f * (y * z + r * x), m22 = 1.f - 2.f * (x * x + y * y);
    float act[3];
    for (int c = 0; c < 3; ++c) act[c] = det_expf(scales[3 * s + c]);
    const float new_o = 1.0f - __builtin_sqrtf(1.0f - det_logistic(opac[s]));
    const float o_logit = det_logit(new_o);
    const float* r1 = rnd + 6 * i;
    const float* r2 = r1 + 3;
    float v1[3], v2[3];
    for (int c = 0; c < 3; ++c) {
        v1[c] = r1[c] * (act[c] + 1e-5f);
        v2[c] = r2[c] * (act[c] + 1e-5f);
    }
    // (M v)_k = M[0][k] v0 + M[1][k] v1 + M[2][k] v2, summed left to right
    const float o1[3] = {m00 * v1[0] + m10 * v1[1] + m20 * v1[2], m01 * v1[0] + m11 * v1[1] + m21 * v1[2],
                         m02 * v1[0] + m12 * v1[1] + m22 * v1[2]};
    const float o2[3] = {m00 * v2[0] + m10 * v2[1] + m20 * v2[2], m01 * v2[0] + m11 * v2[1] + m21 * v2[2],
                         m02 * v2[0] + m12 * v2[1] + m22 * v2[2]};
    for (int c = 0; c < 3; ++c) {
        const float m = means[3 * s + c];
        const float ls = det_logf(act[c] / 1.6f);
        means[3 * t + c] = m + o1[c];
        scales[3 * t + c] = ls;
        means[3 * s + c] = m + o2[c];
        scales[3 * s + c] = ls;
    }
    opac[t] = o_logit;
    opac[s] = o_logit;
}

void launch_densify_apply(int64_t n_grow, int64_t n_old, const int32_t* src, const uint8_t* flags, const float* rnd,
                          float* means, float* scales, float* rots, float* opac, void* sh0, void* shr, int sh_dtype,
                          hipStream_t s) {
    if (n_grow <= 0) return;
    const unsigned grid = (unsigned)((n_grow + 255) / 256);
    if (sh_dtype == kShF16)
        densify_apply_kernel<__half><<<grid, 256, 0, s>>>(n_grow, n_old, src, flags, rnd, means, scales, rots, opac,
                                                          (__half*)sh0, (__half*)shr);
    else
        densify_apply_kernel<float><<<grid, 256, 0, s>>>(n_grow, n_old, src, flags, rnd, means, scales, rots, opac,
                                                         (float*)sh0, (float*)shr);
}

// ------------------------------------------------------------------ row gather / opacity reset

// dst row k = src row rows[k] (k < n_dst) of an array of `width` elements of
// `esize` bytes per row: one thread per 4-byte word of the destination.
__global__ void gather_rows_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                   const int32_t* __restrict__ rows, int64_t n_dst, int row_bytes) {
    const int64_t words = (int64_t)row_bytes / 4;
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= n_dst * words) return;
    const int64_t k = e / words, w = e - k * words;
    const int64_t r = rows[k];
    ((uint32_t*)dst)[k * words + w] = ((const uint32_t*)src)[r * words + w];
}

// row_bytes a multiple of 4 (the fp32 arrays); fp16 rows go through gather_rows16
void launch_gather_rows(const void* src, void* dst, const int32_t* rows, int64_t n_dst, int row_bytes,
                        hipStream_t s) {
    if (n_dst <= 0) return;
    const int64_t total = n_dst * (row_bytes / 4);
    gather_rows_kernel<<<(unsigned)((total + 255) / 256), 256, 0, s>>>((const uint8_t*)src, (uint8_t*)dst, rows,
                                                                      n_dst, row_bytes);
}

// 2-byte elements: dst row k = src row rows[k], one thread per element
__global__ void gather_rows16_kernel(const uint16_t* __restrict__ src, uint16_t* __restrict__ dst,
                                     const int32_t* __restrict__ rows, int64_t n_dst, int width) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= n_dst * width) return;
    const int64_t k = e / width, c = e - k * width;
    dst[k * width + c] = src[(int64_t)rows[k] * width + c];
}

void launch_gather_rows16(const void* src, void* dst, const int32_t* rows, int64_t n_dst, int width, hipStream_t s) {
    if (n_dst <= 0) return;
    const int64_t total = n_dst * width;
    gather_rows16_kernel<<<(unsigned)((total + 255) / 256), 256, 0, s>>>((const uint16_t*)src, (uint16_t*)dst, rows,
                                                                        n_dst, width);
}

// dst row rows[k] = 0 (k < n_rows) of an array of `words` 4-byte words per
// row (simple_adam.cu:944-979): one thread per word; repeated rows are fine.
__global__ void zero_rows_kernel(uint32_t* __restrict__ dst, const int32_t* __restrict__ rows, int64_t n_rows,
                                 int words) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= n_rows * words) return;
    const int64_t k = e / words, w = e - k * words;
    dst[(int64_t)rows[k] * words + w] = 0u;
}

void launch_zero_rows(void* dst, const int32_t* rows, int64_t n_rows, int words, hipStream_t s) {
    if (n_rows <= 0) return;
    const int64_t total = n_rows * words;
    zero_rows_kernel<<<(unsigned)((total + 255) / 256), 256, 0, s>>>((uint32_t*)dst, rows, n_rows, words);
}

// bad[0] |= 1 when some index is negative or >= bound
__global__ void check_indices_kernel(const int32_t* __restrict__ idx, int64_t n, int64_t bound,
                                     uint32_t* __restrict__ bad) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    bool b = i < n && (idx[i] < 0 || (int64_t)idx[i] >= bound);
    if (__any(b) && lane_id() == 0) atomicOr(bad, 1u);
}

void launch_check_indices(const int32_t* idx, int64_t n, int64_t bound, uint32_t* bad, hipStream_t s) {
    if (n <= 0) return;
    check_indices_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(idx, n, bound, bad);
}

// default.cu:26-37: opacity = logit(min(logistic(opacity), max_opacity))
__global__ void reset_opacity_kernel(float* __restrict__ opac, int64_t n, float max_opacity) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    opac[i] = det_logit(fminf(det_logistic(opac[i]), max_opacity));
}

void launch_reset_opacity(float* opac, int64_t n, float max_opacity, hipStream_t s) {
    if (n <= 0) return;
    reset_opacity_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(opac, n, max_opacity);
}

}  // namespace tgs
