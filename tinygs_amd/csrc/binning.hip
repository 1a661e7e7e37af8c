// Binning: deterministic visible-primitive compaction, stable LSD radix sort
// (LDS ranking, wave64 ballot match), per-primitive instance offsets,
// instance emission and per-tile ranges.
//
// Reference stages (tinygs/src/rasterizer/fastgs_ours/forward.cu:146-229):
// depth SortPairs, apply_depth_ordering + ExclusiveSum, create_instances
// (kernels_forward.cuh:427-530), tile SortPairs, extract_instance_ranges
// (:532-551). The reference compacts visible primitives with atomicAdd, so
// its order on equal depths is arbitrary; here compaction is a prefix scan in
// index order and every sort is stable, which yields the canonical per-tile
// order (tile, depth bits, primitive index) -- the order of a stable sort of
// 64-bit keys (tile << 32 | depth bits). The low 32 key bits are sorted once
// per primitive (V elements) before duplication; duplication preserves that
// order, so the remaining passes only sort the ceil(log2 T) tile bits over
// the I instances.
#include "common.h"
#include "kernels.h"

namespace tgs {

constexpr int kScanThreads = 256;
constexpr int kScanItems = 16;
constexpr int kScanChunk = kScanThreads * kScanItems;  // 4096 elements per workgroup

// ---------------------------------------------------------------- workgroup scan

// Exclusive scan of one value per thread across a 256-thread workgroup.
// Returns the exclusive prefix; *total receives the workgroup sum.
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, uint32_t* s_wave, uint32_t* total) {
    const uint32_t lane = threadIdx.x & 63u, w = threadIdx.x >> 6;
    const uint32_t incl = wave_inclusive_scan_u32(v);
    if (lane == 63u) s_wave[w] = incl;
    __syncthreads();
    uint32_t wave_off = 0, sum = 0;
    for (uint32_t k = 0; k < 4; ++k) {
        const uint32_t c = s_wave[k];
        wave_off += (k < w) ? c : 0u;
        sum += c;
    }
    __syncthreads();
    *total = sum;
    return wave_off + incl - v;
}

// ---------------------------------------------------------------- generic 3-phase scan

struct LoadPlain {
    const uint32_t* p;
    __device__ uint32_t operator()(int64_t i) const { return p[i]; }
};
struct LoadVisible {
    const uint32_t* n_touched;
    __device__ uint32_t operator()(int64_t i) const { return n_touched[i] > 0u ? 1u : 0u; }
};
struct LoadTouchedByPrim {
    const uint32_t* n_touched;
    const uint32_t* prims;
    __device__ uint32_t operator()(int64_t i) const { return n_touched[prims[i]]; }
};

__device__ __forceinline__ int64_t resolve_n(const uint32_t* d_n, int64_t max_n) {
    return d_n ? (int64_t)min((int64_t)*d_n, max_n) : max_n;
}

// phase 1: per-chunk sums
template <class Load>
__global__ void __launch_bounds__(kScanThreads) scan_reduce_kernel(Load load, const uint32_t* d_n, int64_t max_n,
                                                                   uint32_t* block_sums) {
    __shared__ uint32_t s_wave[4];
    const int64_t n = resolve_n(d_n, max_n);
    const int64_t base = (int64_t)blockIdx.x * kScanChunk;
    uint32_t acc = 0;
    for (int k = 0; k < kScanItems; ++k) {
        const int64_t i = base + (int64_t)k * kScanThreads + threadIdx.x;
        if (i < n) acc += load(i);
    }
    uint32_t total;
    block_exclusive_scan(acc, s_wave, &total);
    if (threadIdx.x == 0) block_sums[blockIdx.x] = total;
}

// phase 2: exclusive scan of the block sums in place (one workgroup), total
__global__ void __launch_bounds__(kScanThreads) scan_partials_kernel(uint32_t* block_sums, uint32_t nblocks,
                                                                     uint32_t* d_total) {
    __shared__ uint32_t s_wave[4];
    uint32_t carry = 0;
    for (uint32_t base = 0; base < nblocks; base += kScanThreads) {
        const uint32_t i = base + threadIdx.x;
        const uint32_t v = i < nblocks ? block_sums[i] : 0u;
        uint32_t total;
        const uint32_t ex = block_exclusive_scan(v, s_wave, &total);
        if (i < nblocks) block_sums[i] = carry + ex;
        carry += total;
    }
    if (threadIdx.x == 0 && d_total) *d_total = carry;
}

// phase 3: blocked per-thread scan of 16 consecutive items + workgroup scan
template <class Load, class Store>
__global__ void __launch_bounds__(kScanThreads) scan_apply_kernel(Load load, Store store, const uint32_t* d_n,
                                                                  int64_t max_n, const uint32_t* block_offsets) {
    __shared__ uint32_t s_wave[4];
    const int64_t n = resolve_n(d_n, max_n);
    const int64_t base = (int64_t)blockIdx.x * kScanChunk + (int64_t)threadIdx.x * kScanItems;
    uint32_t vals[kScanItems];
    uint32_t acc = 0;
#pragma unroll
    for (int k = 0; k < kScanItems; ++k) {
        const int64_t i = base + k;
        vals[k] = i < n ? load(i) : 0u;
        acc += vals[k];
    }
    uint32_t total;
    uint32_t run = block_exclusive_scan(acc, s_wave, &total) + block_offsets[blockIdx.x];
#pragma unroll
    for (int k = 0; k < kScanItems; ++k) {
        const int64_t i = base + k;
        if (i < n) store(i, run, vals[k]);
        run += vals[k];
    }
}

struct StoreCompact {
    const uint32_t* depth_key;
    uint32_t* keys_out;
    uint32_t* vals_out;
    __device__ void operator()(int64_t i, uint32_t pos, uint32_t flag) const {
        if (flag) {
            keys_out[pos] = depth_key[i];
            vals_out[pos] = (uint32_t)i;
        }
    }
};
struct StorePlain {
    uint32_t* out;
    __device__ void operator()(int64_t i, uint32_t pos, uint32_t) const { out[i] = pos; }
};

static inline uint32_t n_chunks(int64_t n) { return (uint32_t)((n + kScanChunk - 1) / kScanChunk); }

size_t scan_temp_bytes(int64_t n) { return sizeof(uint32_t) * ((size_t)n_chunks(n) + 64); }

template <class Load, class Store>
static void scan3(Load load, Store store, const uint32_t* d_n, int64_t max_n, uint32_t* d_total, uint32_t* temp,
                  hipStream_t s) {
    const uint32_t nb = n_chunks(max_n);
    if (nb == 0) {
        if (d_total) launch_fill_u32(d_total, 0u, 1, s);
        return;
    }
    scan_reduce_kernel<<<nb, kScanThreads, 0, s>>>(load, d_n, max_n, temp);
    scan_partials_kernel<<<1, kScanThreads, 0, s>>>(temp, nb, d_total);
    scan_apply_kernel<<<nb, kScanThreads, 0, s>>>(load, store, d_n, max_n, temp);
}

void launch_compact_visible(const uint32_t* n_touched, const uint32_t* depth_key, int64_t n, uint32_t* keys_out,
                            uint32_t* vals_out, uint32_t* d_count, uint32_t* temp, hipStream_t s) {
    scan3(LoadVisible{n_touched}, StoreCompact{depth_key, keys_out, vals_out}, nullptr, n, d_count, temp, s);
}

void launch_instance_offsets(const uint32_t* n_touched, const uint32_t* prims, const uint32_t* d_count,
                             int64_t max_count, uint32_t* offsets, uint32_t* d_total, uint32_t* temp, hipStream_t s) {
    scan3(LoadTouchedByPrim{n_touched, prims}, StorePlain{offsets}, d_count, max_count, d_total, temp, s);
}

// ---------------------------------------------------------------- radix sort

constexpr int kRadixBits = 8;
constexpr int kRadixBins = 256;
constexpr int kRadixRounds = 16;
constexpr int kRadixChunk = 256 * kRadixRounds;  // 4096 keys per workgroup

__global__ void __launch_bounds__(256) radix_hist_kernel(const uint32_t* __restrict__ keys, const uint32_t* d_n,
                                                         int64_t max_n, int shift, uint32_t* __restrict__ hist,
                                                         uint32_t nblocks) {
    __shared__ uint32_t s_hist[4][kRadixBins];
    const uint32_t w = threadIdx.x >> 6;
    for (int k = threadIdx.x; k < 4 * kRadixBins; k += 256) (&s_hist[0][0])[k] = 0;
    __syncthreads();
    const int64_t n = resolve_n(d_n, max_n);
    const int64_t base = (int64_t)blockIdx.x * kRadixChunk;
    for (int r = 0; r < kRadixRounds; ++r) {
        const int64_t i = base + (int64_t)r * 256 + threadIdx.x;
        if (i < n) atomicAdd(&s_hist[w][(keys[i] >> shift) & 0xffu], 1u);
    }
    __syncthreads();
    const uint32_t d = threadIdx.x;
    hist[(size_t)d * nblocks + blockIdx.x] = s_hist[0][d] + s_hist[1][d] + s_hist[2][d] + s_hist[3][d];
}

// Stable scatter of one 8-bit digit. Wave w of the workgroup owns keys
// [w * 1024, (w + 1) * 1024) of the workgroup's 4096-key chunk and ranks them
// in 16 rounds of 64 with ballot matching against a wave-private LDS
// histogram (a wave's LDS operations complete in issue order, so no barrier
// is needed between rounds). One barrier then turns the four private
// histograms into per-wave bases, and every key is written to
// global offset(digit, workgroup) + wave base + rank within the wave.
__global__ void __launch_bounds__(256) radix_scatter_kernel(const uint32_t* __restrict__ keys_in,
                                                            const uint32_t* __restrict__ vals_in,
                                                            uint32_t* __restrict__ keys_out,
                                                            uint32_t* __restrict__ vals_out, const uint32_t* d_n,
                                                            int64_t max_n, int shift,
                                                            const uint32_t* __restrict__ offsets, uint32_t nblocks) {
    __shared__ uint32_t s_cnt[4][kRadixBins];
    const uint32_t lane = threadIdx.x & 63u, w = threadIdx.x >> 6, t = threadIdx.x;
    const int64_t n = resolve_n(d_n, max_n);
    const int64_t blk = (int64_t)blockIdx.x * kRadixChunk;
    if (blk >= n) return;
    for (int k = t; k < 4 * kRadixBins; k += 256) (&s_cnt[0][0])[k] = 0;
    const uint32_t gofs = offsets[(size_t)t * nblocks + blockIdx.x];
    __syncthreads();
    const int64_t base = blk + (int64_t)w * (kRadixChunk / 4);
    uint32_t key[kRadixRounds], val[kRadixRounds], pos[kRadixRounds];
#pragma unroll
    for (int r = 0; r < kRadixRounds; ++r) {
        const int64_t i = base + (int64_t)r * 64 + lane;
        const bool valid = i < n;
        key[r] = valid ? keys_in[i] : 0u;
        val[r] = valid ? vals_in[i] : 0u;
    }
#pragma unroll
    for (int r = 0; r < kRadixRounds; ++r) {
        const int64_t i = base + (int64_t)r * 64 + lane;
        const bool valid = i < n;
        const uint32_t d = (key[r] >> shift) & 0xffu;
        uint64_t peers = ballot(valid);
#pragma unroll
        for (int b = 0; b < kRadixBits; ++b) {
            const bool bit = (d >> b) & 1u;
            const uint64_t m = ballot(bit);
            peers &= bit ? m : ~m;
        }
        const uint32_t rank = mask_rank(peers);
        const uint32_t running = s_cnt[w][d];
        pos[r] = running + rank;
        if (valid && rank == 0u) s_cnt[w][d] = running + (uint32_t)__builtin_popcountll(peers);
    }
    __syncthreads();
    {
        const uint32_t c0 = s_cnt[0][t], c1 = s_cnt[1][t], c2 = s_cnt[2][t];
        s_cnt[0][t] = gofs;
        s_cnt[1][t] = gofs + c0;
        s_cnt[2][t] = gofs + c0 + c1;
        s_cnt[3][t] = gofs + c0 + c1 + c2;
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < kRadixRounds; ++r) {
        const int64_t i = base + (int64_t)r * 64 + lane;
        if (i < n) {
            const uint32_t d = (key[r] >> shift) & 0xffu;
            const uint32_t o = s_cnt[w][d] + pos[r];
            keys_out[o] = key[r];
            vals_out[o] = val[r];
        }
    }
}

size_t radix_temp_bytes(int64_t max_n) {
    const size_t nb = (size_t)((max_n + kRadixChunk - 1) / kRadixChunk);
    const size_t hist = nb * kRadixBins;
    return sizeof(uint32_t) * (hist + (hist + kScanChunk - 1) / kScanChunk + 64);
}

int radix_sort_pairs(uint32_t* keys[2], uint32_t* vals[2], const uint32_t* d_n, int64_t max_n, int end_bit,
                     uint32_t* temp, hipStream_t s) {
    const uint32_t nb = (uint32_t)((max_n + kRadixChunk - 1) / kRadixChunk);
    if (nb == 0) return 0;
    const int64_t hist_n = (int64_t)nb * kRadixBins;
    uint32_t* hist = temp;
    uint32_t* scan_tmp = temp + hist_n;
    int cur = 0;
    for (int shift = 0; shift < end_bit; shift += kRadixBits) {
        radix_hist_kernel<<<nb, 256, 0, s>>>(keys[cur], d_n, max_n, shift, hist, nb);
        scan3(LoadPlain{hist}, StorePlain{hist}, nullptr, hist_n, nullptr, scan_tmp, s);
        radix_scatter_kernel<<<nb, 256, 0, s>>>(keys[cur], vals[cur], keys[cur ^ 1], vals[cur ^ 1], d_n, max_n,
                                                shift, hist, nb);
        cur ^= 1;
    }
    return cur;
}

// ---------------------------------------------------------------- instance emission

// kernels_forward.cuh:49-84 (same expression as in preprocess.hip)
__device__ __forceinline__ bool will_contribute_e(float mx, float my, float ca, float cb, float cc, uint32_t tile_x,
                                                  uint32_t tile_y, float power_threshold) {
    const float rminx = (float)(tile_x * 16u), rminy = (float)(tile_y * 16u);
    const float rmaxx = (float)((tile_x + 1u) * 16u - 1u), rmaxy = (float)((tile_y + 1u) * 16u - 1u);
    const float x_min_diff = rminx - mx;
    const float x_left = x_min_diff > 0.0f ? 1.0f : 0.0f;
    const float not_in_x = x_left + (mx > rmaxx ? 1.0f : 0.0f);
    const float y_min_diff = rminy - my;
    const float y_above = y_min_diff > 0.0f ? 1.0f : 0.0f;
    const float not_in_y = y_above + (my > rmaxy ? 1.0f : 0.0f);
    if (not_in_y + not_in_x == 0.0f) return true;
    const float ccx = rmaxx + x_left * (rminx - rmaxx);
    const float ccy = rmaxy + y_above * (rminy - rmaxy);
    const float diffx = mx - ccx, diffy = my - ccy;
    const float dx = __builtin_copysignf(15.0f, x_min_diff);
    const float dy = __builtin_copysignf(15.0f, y_min_diff);
    const float tx = not_in_y * saturate((dx * ca * diffx + dx * cb * diffy) / (dx * ca * dx));
    const float ty = not_in_x * saturate((dy * cb * diffx + dy * cc * diffy) / (dy * cc * dy));
    const float px = ccx + tx * dx, py = ccy + ty * dy;
    const float ddx = mx - px, ddy = my - py;
    const float max_power = 0.5f * (ca * ddx * ddx + cc * ddy * ddy) + cb * ddx * ddy;
    return max_power <= power_threshold;
}

__global__ void __launch_bounds__(256) emit_kernel(const uint32_t* __restrict__ n_touched,
                                                   const uint32_t* __restrict__ prims,
                                                   const uint32_t* __restrict__ offsets, const uint32_t* d_count,
                                                   int64_t max_count, const uint2* __restrict__ bounds,
                                                   const float2* __restrict__ mean2d,
                                                   const float4* __restrict__ conic_opacity,
                                                   const float4* __restrict__ color_pt, uint32_t grid_w,
                                                   uint32_t* __restrict__ inst_keys,
                                                   uint32_t* __restrict__ inst_vals) {
    const int64_t count = resolve_n(d_count, max_count);
    const int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if ((int64_t)blockIdx.x * blockDim.x >= count) return;  // whole workgroup idle
    const bool active = k < count;
    const uint32_t lane = lane_id();
    uint32_t p = 0, off = 0, cap = 0, x0 = 0, x1 = 0, y0 = 0, y1 = 0;
    float smx = 0.f, smy = 0.f, ca = 0.f, cb = 0.f, cc = 0.f, pt = 0.f;
    if (active) {
        p = prims[k];
        off = offsets[k];
        cap = n_touched[p];   // slots reserved for this primitive
        const uint2 b = bounds[p];
        x0 = b.x & 0xffffu; x1 = b.x >> 16; y0 = b.y & 0xffffu; y1 = b.y >> 16;
        const float2 m = mean2d[p];
        smx = m.x - 0.5f;
        smy = m.y - 0.5f;
        const float4 co = conic_opacity[p];
        ca = co.x; cb = co.y; cc = co.z;
        pt = color_pt[p].w;
    }
    const uint32_t bw = x1 - x0;
    const uint32_t nrect = bw * (y1 - y0);
    uint32_t written = 0;
    if (active) {
        const uint32_t first = nrect < 8u ? nrect : 8u;
        for (uint32_t q = 0; q < first; ++q) {
            const uint32_t tx = x0 + q % bw, ty = y0 + q / bw;
            if (will_contribute_e(smx, smy, ca, cb, cc, tx, ty, pt) && written < cap) {
                inst_keys[off + written] = ty * grid_w + tx;
                inst_vals[off + written] = p;
                ++written;
            }
        }
    }
    uint64_t coop = ballot(active && nrect > 8u);
    while (coop) {
        const uint32_t src = (uint32_t)__builtin_ctzll(coop);
        coop &= coop - 1;
        const float s_mx = readlane_f32(smx, src), s_my = readlane_f32(smy, src);
        const float s_a = readlane_f32(ca, src), s_b = readlane_f32(cb, src), s_c = readlane_f32(cc, src);
        const float s_t = readlane_f32(pt, src);
        const uint32_t s_x0 = readlane_u32(x0, src), s_y0 = readlane_u32(y0, src);
        const uint32_t s_bw = readlane_u32(bw, src), s_n = readlane_u32(nrect, src);
        const uint32_t s_p = readlane_u32(p, src);
        const uint32_t s_end = readlane_u32(off, src) + readlane_u32(cap, src);
        uint32_t s_off = readlane_u32(off, src) + readlane_u32(written, src);
        for (uint32_t base = 8u; base < s_n; base += kWave) {
            const uint32_t q = base + lane;
            bool hit = false;
            uint32_t tx = 0, ty = 0;
            if (q < s_n) {
                tx = s_x0 + q % s_bw;
                ty = s_y0 + q / s_bw;
                hit = will_contribute_e(s_mx, s_my, s_a, s_b, s_c, tx, ty, s_t);
            }
            const uint64_t m = ballot(hit);
            const uint32_t pos = s_off + mask_rank(m);
            if (hit && pos < s_end) {
                inst_keys[pos] = ty * grid_w + tx;
                inst_vals[pos] = s_p;
            }
            s_off += (uint32_t)__builtin_popcountll(m);
        }
    }
}

void launch_emit_instances(const uint32_t* n_touched, const uint32_t* prims, const uint32_t* offsets, const uint32_t* d_count, int64_t max_count,
                           const uint2* bounds, const float2* mean2d, const float4* conic_opacity,
                           const float4* color_pt, uint32_t grid_w, uint32_t* inst_keys, uint32_t* inst_vals,
                           hipStream_t s) {
    if (max_count <= 0) return;
    emit_kernel<<<(unsigned)((max_count + 255) / 256), 256, 0, s>>>(n_touched, prims, offsets, d_count, max_count, bounds, mean2d,
                                                                   conic_opacity, color_pt, grid_w, inst_keys,
                                                                   inst_vals);
}

// ---------------------------------------------------------------- ranges

__global__ void fill_u32_kernel(uint32_t* p, uint32_t v, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

void launch_fill_u32(uint32_t* p, uint32_t value, int64_t n, hipStream_t s) {
    if (n <= 0) return;
    fill_u32_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(p, value, n);
}

// kernels_forward.cuh:532-551
__global__ void tile_ranges_kernel(const uint32_t* __restrict__ keys, int64_t n, uint2* __restrict__ ranges) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint32_t t = keys[i];
    if (i == 0) {
        ranges[t].x = 0;
    } else {
        const uint32_t prev = keys[i - 1];
        if (t != prev) {
            ranges[prev].y = (uint32_t)i;
            ranges[t].x = (uint32_t)i;
        }
    }
    if (i == n - 1) ranges[t].y = (uint32_t)n;
}

void launch_tile_ranges(const uint32_t* inst_keys, int64_t n_inst, uint2* ranges, uint32_t n_tiles, hipStream_t s) {
    launch_fill_u32((uint32_t*)ranges, 0u, 2 * (int64_t)n_tiles, s);
    if (n_inst <= 0) return;
    tile_ranges_kernel<<<(unsigned)((n_inst + 255) / 256), 256, 0, s>>>(inst_keys, n_inst, ranges);
}

}  // namespace tgs
