// L1 and fused-SSIM loss / gradient on the 8x8-tiled channel-planar image.
// L1 follows tinygs/src/loss/l1.cu:19-42 (+ host scaling :109-151);
// SSIM follows tinygs/src/loss/fused_ssim.cu:55-267 (forward),
// :275-442 (backward), :797-916 (host): per channel, inputs rounded to fp16
// for the statistics, zero padding outside the image, separable 11-tap
// Gaussian (sigma 1.5), and the three partial-derivative maps convolved back
// in fp32 with the fp32 prediction and target.
//
// MI355X design: one workgroup per 32x32 output tile (42x42 with the 5-pixel
// halo, filled through whole 8x8 blocks: coalesced 256-byte runs) and
// channel. The horizontal pass gives each thread
// four adjacent output columns of one row (14 inputs feed 4 x 11 taps), the
// vertical pass four adjacent rows of one column (14 rows of horizontal sums
// feed 4 x 11 taps), so every LDS value read is used several times. The SSIM
// forward also evaluates L1 on the same pixels when asked (one launch for
// 0.8 L1 + 0.2 (1 - SSIM) and its gradient's L1 part), and in assign mode
// writes loss / gradient instead of accumulating, which spares the caller
// zeroing them.
//
// Results accumulate unless assign: loss[i] += ..., grad[i] += ...; the L1
// term is added before the SSIM term, as two separate reference launches
// would. SSIM sums differ from the reference's summation order by rounding
// only (the oracle comparison is normwise 1e-5).
//
// fp16 images (l1.cu:43-107, fused_ssim.cu:445-693): the same float
// arithmetic on the half inputs; each stored loss / gradient value is the
// float result (including the accumulated half value) rounded to nearest
// half, once per reference launch (the L1 term's sum is rounded before the
// SSIM term is added). The three derivative maps stay float.
#include <algorithm>

#include "common.h"
#include "kernels.h"

namespace tgs {

// element access of fp32 / fp16 images
__device__ __forceinline__ float ld(const float* p, size_t i) { return p[i]; }
__device__ __forceinline__ float ld(const __half* p, size_t i) { return __half2float(p[i]); }
__device__ __forceinline__ void st(float* p, size_t i, float v) { p[i] = v; }
__device__ __forceinline__ void st(__half* p, size_t i, float v) { p[i] = f2h_rn(v); }
// a value as the image type holds it
__device__ __forceinline__ float held(const float*, float v) { return v; }
__device__ __forceinline__ float held(const __half*, float v) { return __half2float(f2h_rn(v)); }

__constant__ float kGauss[11] = {0.001028380123898387f,  0.0075987582094967365f, 0.036000773310661316f,
                                 0.10936068743467331f,   0.21300552785396576f,   0.26601171493530273f,
                                 0.21300552785396576f,   0.10936068743467331f,   0.036000773310661316f,
                                 0.0075987582094967365f, 0.001028380123898387f};

// Vectorised over 16-byte groups (the padded image is a multiple of 64
// floats per channel); kernels_forward of the same numerics: p = sat(pred),
// loss += |p - t| s, grad += sign(p - t) s with sign(+0) = +1 (l1.cu:28-41).
__global__ void l1_kernel(const float4* __restrict__ pred, const float4* __restrict__ target,
                          float4* __restrict__ loss, float4* __restrict__ grad, int64_t n4, float s) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n4) return;
    const float4 p4 = pred[i], t4 = target[i];
    const float pv[4] = {p4.x, p4.y, p4.z, p4.w}, tv[4] = {t4.x, t4.y, t4.z, t4.w};
    float l[4], g[4];
    float4 lo = loss ? loss[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    float4 go = grad ? grad[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    const float lv[4] = {lo.x, lo.y, lo.z, lo.w}, gv[4] = {go.x, go.y, go.z, go.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const float d = saturate(pv[q]) - tv[q];
        l[q] = __builtin_fmaf(__builtin_fabsf(d), s, lv[q]);
        g[q] = __builtin_fmaf(__builtin_copysignf(1.0f, d), s, gv[q]);
    }
    if (loss) loss[i] = make_float4(l[0], l[1], l[2], l[3]);
    if (grad) grad[i] = make_float4(g[0], g[1], g[2], g[3]);
}

// fp16 (l1_kernel_f16_h2, l1.cu:67-107): eight halves per thread
__global__ void l1_f16_kernel(const uint4* __restrict__ pred, const uint4* __restrict__ target,
                              uint4* __restrict__ loss, uint4* __restrict__ grad, int64_t n8, float s) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n8) return;
    const uint4 p4 = pred[i], t4 = target[i];
    const uint4 l4 = loss ? loss[i] : make_uint4(0u, 0u, 0u, 0u);
    const uint4 g4 = grad ? grad[i] : make_uint4(0u, 0u, 0u, 0u);
    const __half* ph = (const __half*)&p4;
    const __half* th = (const __half*)&t4;
    const __half* lh = (const __half*)&l4;
    const __half* gh = (const __half*)&g4;
    uint4 lo, go;
    __half* lr = (__half*)&lo;
    __half* gr = (__half*)&go;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        const float d = saturate(__half2float(ph[q])) - __half2float(th[q]);
        lr[q] = f2h_rn(__builtin_fmaf(__builtin_fabsf(d), s, __half2float(lh[q])));
        gr[q] = f2h_rn(__builtin_fmaf(__builtin_copysignf(1.0f, d), s, __half2float(gh[q])));
    }
    if (loss) loss[i] = lo;
    if (grad) grad[i] = go;
}

void launch_l1(const float* pred, const float* target, float* loss, float* grad, int64_t n_padded, float s,
               hipStream_t st) {
    if (n_padded <= 0) return;
    const int64_t n4 = n_padded / 4;   // padded planes hold whole 8x8 blocks
    l1_kernel<<<(unsigned)((n4 + 255) / 256), 256, 0, st>>>((const float4*)pred, (const float4*)target,
                                                            (float4*)loss, (float4*)grad, n4, s);
}

void launch_l1_f16(const void* pred, const void* target, void* loss, void* grad, int64_t n_padded, float s,
                   hipStream_t st) {
    if (n_padded <= 0) return;
    const int64_t n8 = n_padded / 8;   // whole 8x8 blocks: a multiple of 64 halves per plane
    l1_f16_kernel<<<(unsigned)((n8 + 255) / 256), 256, 0, st>>>((const uint4*)pred, (const uint4*)target,
                                                                (uint4*)loss, (uint4*)grad, n8, s);
}

constexpr int kOT = 32;           // output tile edge
constexpr int kIT = kOT + 10;     // input tile edge (5-pixel halo)

// Halo fill through whole 8x8 blocks of the tiled layout: the 42x42 region
// at (bx - 5, by - 5) lies inside the 6x6 blocks starting at block
// (bx / 8 - 1, by / 8 - 1) (bx, by multiples of 32), at offset 3 in both
// directions. Wave w loads blocks w, w + 4, ... (one contiguous 256-byte run
// per plane each), lane = pixel of the block. The block of a round is
// wave-uniform, so its base address and bounds are scalar and a lane only
// compares its own (x, y) inside the block against them; pixels outside
// W x H read as 0 (the reference's zero padding).
constexpr int kHaloBlocks = 36;
constexpr int kHaloRounds = kHaloBlocks / 4;   // 9 blocks per wave
constexpr int kHT = 48;                        // 6 blocks of 8

struct HaloRound {
    size_t base;   // element offset of the block in a plane (0 when the block lies outside the planes)
    int cx, cy;    // block position among the 6 x 6
    bool in;       // this lane's pixel lies inside W x H
};

__device__ __forceinline__ HaloRound halo_round(int r, int bx, int by, uint32_t W, uint32_t H, uint32_t tw,
                                                uint32_t th) {
    const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lane = (int)(threadIdx.x & 63u);
    const int b = w + 4 * r;
    HaloRound h;
    h.cx = b % 6;
    h.cy = b / 6;
    const int bcx = bx / 8 - 1 + h.cx, bcy = by / 8 - 1 + h.cy;
    const bool blk = bcx >= 0 && bcy >= 0 && bcx < (int)tw && bcy < (int)th;
    h.base = blk ? ((size_t)bcy * tw + (size_t)bcx) * 64u : 0u;
    h.in = blk && (lane & 7) < (int)W - bcx * 8 && (lane >> 3) < (int)H - bcy * 8;
    return h;
}

// (tile x, tile y, channel) of this workgroup: the grid is (tiles x, tiles
// y, 3) and tiles are taken in row-major order per channel, each XCD a
// contiguous run of them.
__device__ __forceinline__ void ssim_tile_of(uint32_t& tx, uint32_t& ty, uint32_t& ch) {
    const uint32_t gx = gridDim.x, gy = gridDim.y;
    const uint32_t linear = blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z);
    const uint32_t k = xcd_contiguous_index(linear, gx * gy * gridDim.z);
    tx = k % gx;
    ty = (k / gx) % gy;
    ch = k / (gx * gy);
}

// Fused L1 + SSIM forward. The SSIM value and all three derivative maps
// depend on the variances only through sigma1^2 + sigma2^2, so the two second
// moments are filtered as one, E[x^2 + y^2] (the filter is linear): four
// filtered moments instead of the reference's five (fused_ssim.cu:232-240
// uses sigma1^2 and sigma2^2 only in B), which changes the sums by rounding
// only. s_l1 == 0 disables L1; assign writes loss / grad
// instead of accumulating (grad then holds the L1 part, or 0). dm_* may be
// NULL (loss only). SSIM terms only inside W x H; L1 over the whole padded
// image, like the reference's L1 over all padded elements. One workgroup per
// (32x32 tile, channel): no state is carried across channels, which keeps
// the register footprint small enough for four workgroups per CU.
template <typename T, bool ASSIGN>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(6))) l1_ssim_forward_kernel(uint32_t W, uint32_t H, float C1, float C2,
                                                              float s_ssim, float s_l1,
                                                              const T* __restrict__ pred,
                                                              const T* __restrict__ target,
                                                              T* __restrict__ loss, T* __restrict__ grad,
                                                              float* __restrict__ dm_mu, float* __restrict__ dm_s1,
                                                              float* __restrict__ dm_s12) {
    // s_in: the fp16-rounded (pred, target) halo, exactly the values the sums
    // use; s_h: the horizontal sums x, x^2 + y^2, y, xy, overlaying s_in once
    // every thread holds its sums in registers (22 KB of LDS instead of 31 KB)
    __shared__ float s_buf[4 * kIT * (kOT + 1)];
    // s_in rows of 49 words: the horizontal pass's lanes (8 rows x 8 groups of
    // 4 columns) then meet 2-way bank conflicts instead of 4-way
    constexpr int kInStride = kHT + 1;
    static_assert(kHT * kInStride <= 4 * kIT * (kOT + 1), "s_in fits inside s_h");
    auto s_in = reinterpret_cast<__half2 (*)[kInStride]>(s_buf);
    auto s_h = reinterpret_cast<float (*)[kIT][kOT + 1]>(s_buf);
    const int t = (int)threadIdx.x;
    uint32_t tx, ty, ch;
    ssim_tile_of(tx, ty, ch);
    const int bx = (int)tx * kOT, by = (int)ty * kOT;
    const uint32_t tw = (W + 7u) >> 3, th = (H + 7u) >> 3;
    const uint32_t cs = tw * th * 64u;
    const int pw = (int)tw * 8, ph = (int)th * 8;
    const size_t co = (size_t)ch * cs;
    pred += co;
    target += co;
    {
        const int lane = t & 63;
        float pv[kHaloRounds], tv[kHaloRounds];
#pragma unroll
        for (int r = 0; r < kHaloRounds; ++r) {
            const HaloRound h = halo_round(r, bx, by, W, H, tw, th);
            const T* __restrict__ pp = pred + h.base;   // wave-uniform block base
            const T* __restrict__ tp = target + h.base;
            const float x = ld(pp, lane), y = ld(tp, lane);
            pv[r] = h.in ? x : 0.f;
            tv[r] = h.in ? y : 0.f;
        }
#pragma unroll
        for (int r = 0; r < kHaloRounds; ++r) {
            const HaloRound h = halo_round(r, bx, by, W, H, tw, th);
            s_in[h.cy * 8 + (lane >> 3)][h.cx * 8 + (lane & 7)] = __floats2half2_rn(pv[r], tv[r]);
        }
    }
    __syncthreads();
    // horizontal: row r, output columns 4 g .. 4 g + 3; items t and t + 256
    static_assert(kIT * 8 <= 2 * 256, "two horizontal items per thread");
    float hs[2][4][4];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int wi = t + 256 * k;
        if (wi >= kIT * 8) break;
        const int r = wi >> 3, g = wi & 7;
        float x[14], y[14], q[14], xy[14];
#pragma unroll
        for (int d = 0; d < 14; ++d) {
            const float2 v = __half22float2(s_in[r + 3][4 * g + d + 3]);
            x[d] = v.x;
            y[d] = v.y;
            q[d] = __builtin_fmaf(v.x, v.x, v.y * v.y);
            xy[d] = v.x * v.y;
        }
#pragma unroll
        for (int o = 0; o < 4; ++o) {
            float sx = 0.f, sq = 0.f, sy = 0.f, sxy = 0.f;
#pragma unroll
            for (int d = 0; d < 11; ++d) {
                const float wv = kGauss[d];
                sx = __builtin_fmaf(x[o + d], wv, sx);
                sq = __builtin_fmaf(q[o + d], wv, sq);
                sy = __builtin_fmaf(y[o + d], wv, sy);
                sxy = __builtin_fmaf(xy[o + d], wv, sxy);
            }
            hs[k][0][o] = sx;
            hs[k][1][o] = sq;
            hs[k][2][o] = sy;
            hs[k][3][o] = sxy;
        }
    }
    __syncthreads();   // every s_in read done before s_h overwrites it
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int wi = t + 256 * k;
        if (wi >= kIT * 8) break;
        const int r = wi >> 3, g = wi & 7;
#pragma unroll
        for (int v = 0; v < 4; ++v)
#pragma unroll
            for (int o = 0; o < 4; ++o) s_h[v][r][4 * g + o] = hs[k][v][o];
    }
    __syncthreads();
    // vertical: column vc, output rows 4 vr .. 4 vr + 3
    const int vc = t & 31, vr = t >> 5;
    if (loss) loss += co;
    if (grad) grad += co;
    // epilogue in 8x8-block order: wave w takes blocks w, w + 4, w + 8, w + 12
    // of the tile (4 x 4 blocks), lane = pixel of the block, so each of its
    // loads and stores is one 256-byte run. Its own pixels (L1 terms,
    // accumulated values) are loaded before the vertical pass, so their
    // latency hides behind it.
    const int lane = t & 63, wv = t >> 6;
    const bool acc_l = !ASSIGN && loss, acc_g = !ASSIGN && grad, l1 = s_l1 != 0.f;
    float pp[4], pt[4], pl[4], pg[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int b = wv + 4 * q;
        const int px = bx + 8 * (b & 3) + (lane & 7), py = by + 8 * (b >> 2) + (lane >> 3);
        const bool in = px < pw && py < ph;
        const uint32_t idx = in ? tiled_index((uint32_t)py, (uint32_t)px, tw) : 0u;
        pp[q] = in && l1 ? ld(pred, idx) : 0.f;
        pt[q] = in && l1 ? ld(target, idx) : 0.f;
        pl[q] = in && acc_l ? ld(loss, idx) : 0.f;
        pg[q] = in && acc_g ? ld(grad, idx) : 0.f;
    }
    float o[4][4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        float col[14];
#pragma unroll
        for (int d = 0; d < 14; ++d) col[d] = s_h[v][4 * vr + d][vc];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            float acc = 0.f;
#pragma unroll
            for (int d = 0; d < 11; ++d) acc = __builtin_fmaf(col[q + d], kGauss[d], acc);
            o[v][q] = acc;
        }
    }
    // the four filtered moments change hands through LDS (over s_h, once every
    // thread has read its columns); rows of 40 words: conflict-free for the
    // column-order writes and the block-order reads on 64 banks
    constexpr int kOStride = kOT + 8;
    auto s_o = reinterpret_cast<float (*)[kOT][kOStride]>(s_buf);
    static_assert(4 * kOT * kOStride <= 4 * kIT * (kOT + 1), "moments fit in s_buf");
    __syncthreads();
#pragma unroll
    for (int v = 0; v < 4; ++v)
#pragma unroll
        for (int q = 0; q < 4; ++q) s_o[v][4 * vr + q][vc] = o[v][q];
    __syncthreads();
    if (dm_mu) {
        dm_mu += co;
        dm_s1 += co;
        dm_s12 += co;
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int b = wv + 4 * q;
        const int lx = 8 * (b & 3) + (lane & 7), ly = 8 * (b >> 2) + (lane >> 3);
        const int px = bx + lx, py = by + ly;
        if (px >= pw || py >= ph) continue;
        const uint32_t idx = tiled_index((uint32_t)py, (uint32_t)px, tw);
        float lv = pl[q];
        float gv = pg[q];
        if (l1) {
            const float d = saturate(pp[q]) - pt[q];
            lv = held(pred, __builtin_fmaf(__builtin_fabsf(d), s_l1, lv));
            gv = __builtin_fmaf(__builtin_copysignf(1.0f, d), s_l1, gv);
        }
        if (px < (int)W && py < (int)H) {
            const float mu1 = s_o[0][ly][lx], mu2 = s_o[2][ly][lx];
            const float mu1_sq = mu1 * mu1, mu2_sq = mu2 * mu2;
            const float s12 = s_o[3][ly][lx] - mu1 * mu2;
            const float A = mu1_sq + mu2_sq + C1;
            const float B = ((s_o[1][ly][lx] - mu1_sq) - mu2_sq) + C2;   // sigma1^2 + sigma2^2 + C2
            const float Cc = 2.0f * mu1 * mu2 + C1;
            const float D = 2.0f * s12 + C2;
            // one reciprocal each of A and B replaces the reference's seven divisions
            const float iA = __builtin_amdgcn_rcpf(A), iB = __builtin_amdgcn_rcpf(B);
            const float inv = iA * iB;
            const float val = (Cc * D) * inv;
            lv = __builtin_fmaf(1.0f - val, s_ssim, lv);
            if (dm_mu) {
                dm_mu[idx] = 2.0f * inv * (mu2 * (D - Cc) + mu1 * (Cc * D) * (iB - iA));
                dm_s1[idx] = -(Cc * D) * inv * iB;
                dm_s12[idx] = 2.0f * Cc * inv;
            }
        }
        if (loss) st(loss, idx, lv);
        if (grad && (ASSIGN || s_l1 != 0.f)) st(grad, idx, gv);
    }
}

// SSIM backward: grad += -s (dm_mu * w + 2 p (dm_s1 * w) + t (dm_s12 * w))
// with * the 11x11 separable convolution (fused_ssim.cu:366-438). One
// workgroup per (32x32 tile, channel).
template <typename T>
__global__ void __launch_bounds__(256) ssim_backward_kernel(uint32_t W, uint32_t H, float s,
                                                            const T* __restrict__ pred,
                                                            const T* __restrict__ target,
                                                            T* __restrict__ grad, const float* __restrict__ dm_mu,
                                                            const float* __restrict__ dm_s1,
                                                            const float* __restrict__ dm_s12) {
    // s_d: the three maps with halo; s_h: their horizontal sums, overlaying
    // s_d once every thread has read its inputs (21.2 KB of LDS instead of
    // 37.8 KB)
    __shared__ float s_buf[3 * kIT * kIT];
    auto s_d = reinterpret_cast<float (*)[kIT][kIT]>(s_buf);
    auto s_h = reinterpret_cast<float (*)[kIT][kOT + 1]>(s_buf);
    static_assert(kOT + 1 <= kIT, "s_h fits inside s_d");
    static_assert(kIT * 8 <= 2 * 256, "two horizontal items per thread");
    const int t = (int)threadIdx.x;
    uint32_t tx, ty, ch;
    ssim_tile_of(tx, ty, ch);
    const int bx = (int)tx * kOT, by = (int)ty * kOT;
    const uint32_t tw = (W + 7u) >> 3, th = (H + 7u) >> 3;
    const uint32_t cs = tw * th * 64u;
    const size_t co = (size_t)ch * cs;
    {
        const int lane = t & 63;
        const float* __restrict__ m0 = dm_mu + co;
        const float* __restrict__ m1 = dm_s1 + co;
        const float* __restrict__ m2 = dm_s12 + co;
        float av[kHaloRounds], bv[kHaloRounds], dv[kHaloRounds];
#pragma unroll
        for (int r = 0; r < kHaloRounds; ++r) {
            const HaloRound h = halo_round(r, bx, by, W, H, tw, th);
            const float* __restrict__ p0 = m0 + h.base;   // wave-uniform block base
            const float* __restrict__ p1 = m1 + h.base;
            const float* __restrict__ p2 = m2 + h.base;
            const float x = p0[lane], y = p1[lane], z = p2[lane];
            av[r] = h.in ? x : 0.f;
            bv[r] = h.in ? y : 0.f;
            dv[r] = h.in ? z : 0.f;
        }
#pragma unroll
        for (int r = 0; r < kHaloRounds; ++r) {
            const HaloRound h = halo_round(r, bx, by, W, H, tw, th);
            // the 42x42 region starts 3 pixels into the 6x6 blocks
            const int lx = h.cx * 8 + (lane & 7) - 3, ly = h.cy * 8 + (lane >> 3) - 3;
            if ((unsigned)lx < (unsigned)kIT && (unsigned)ly < (unsigned)kIT) {
                s_d[0][ly][lx] = av[r];
                s_d[1][ly][lx] = bv[r];
                s_d[2][ly][lx] = dv[r];
            }
        }
    }
    __syncthreads();
    float hs[2][3][4];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int wi = t + 256 * k;
        if (wi >= kIT * 8) break;
        const int r = wi >> 3, g = wi & 7;
#pragma unroll
        for (int v = 0; v < 3; ++v) {
            float x[14];
#pragma unroll
            for (int d = 0; d < 14; ++d) x[d] = s_d[v][r][4 * g + d];
#pragma unroll
            for (int o = 0; o < 4; ++o) {
                float acc = 0.f;
#pragma unroll
                for (int d = 0; d < 11; ++d) acc = __builtin_fmaf(x[o + d], kGauss[d], acc);
                hs[k][v][o] = acc;
            }
        }
    }
    __syncthreads();   // every s_d read done before s_h overwrites it
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int wi = t + 256 * k;
        if (wi >= kIT * 8) break;
        const int r = wi >> 3, g = wi & 7;
#pragma unroll
        for (int v = 0; v < 3; ++v)
#pragma unroll
            for (int o = 0; o < 4; ++o) s_h[v][r][4 * g + o] = hs[k][v][o];
    }
    __syncthreads();
    const int vc = t & 31, vr = t >> 5;
    pred += co;
    target += co;
    grad += co;
    // the epilogue's pixels, loaded before the vertical pass so that their
    // latency hides behind it
    uint32_t pidx[4];
    float pp[4], pt[4], pg[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int px = bx + vc, py = by + 4 * vr + q;
        const bool in = px < (int)W && py < (int)H;
        pidx[q] = in ? tiled_index((uint32_t)py, (uint32_t)px, tw) : 0u;
        pp[q] = in ? ld(pred, pidx[q]) : 0.f;
        pt[q] = in ? ld(target, pidx[q]) : 0.f;
        pg[q] = in ? ld(grad, pidx[q]) : 0.f;
    }
    float o[3][4];
#pragma unroll
    for (int v = 0; v < 3; ++v) {
        float col[14];
#pragma unroll
        for (int d = 0; d < 14; ++d) col[d] = s_h[v][4 * vr + d][vc];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            float acc = 0.f;
#pragma unroll
            for (int d = 0; d < 11; ++d) acc = __builtin_fmaf(col[q + d], kGauss[d], acc);
            o[v][q] = acc;
        }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int px = bx + vc, py = by + 4 * vr + q;
        if (px >= (int)W || py >= (int)H) continue;
        const float dl = __builtin_fmaf(pt[q], o[2][q], __builtin_fmaf(2.0f * pp[q], o[1][q], o[0][q]));
        st(grad, pidx[q], __builtin_fmaf(-s, dl, pg[q]));
    }
}

void launch_l1_ssim_forward(uint32_t width, uint32_t height, float c1, float c2, float s_ssim, float s_l1,
                            bool assign, const float* pred, const float* target, float* loss, float* grad,
                            float* dm_mu, float* dm_s1, float* dm_s12, hipStream_t st) {
    if (width == 0 || height == 0) return;
    dim3 grid((width + kOT - 1) / kOT, (height + kOT - 1) / kOT, 3);
    if (assign)
        l1_ssim_forward_kernel<float, true><<<grid, 256, 0, st>>>(width, height, c1, c2, s_ssim, s_l1, pred, target,
                                                                  loss, grad, dm_mu, dm_s1, dm_s12);
    else
        l1_ssim_forward_kernel<float, false><<<grid, 256, 0, st>>>(width, height, c1, c2, s_ssim, s_l1, pred, target,
                                                                   loss, grad, dm_mu, dm_s1, dm_s12);
}

void launch_l1_ssim_forward_f16(uint32_t width, uint32_t height, float c1, float c2, float s_ssim, float s_l1,
                                bool assign, const void* pred, const void* target, void* loss, void* grad,
                                float* dm_mu, float* dm_s1, float* dm_s12, hipStream_t st) {
    if (width == 0 || height == 0) return;
    dim3 grid((width + kOT - 1) / kOT, (height + kOT - 1) / kOT, 3);
    if (assign)
        l1_ssim_forward_kernel<__half, true><<<grid, 256, 0, st>>>(width, height, c1, c2, s_ssim, s_l1,
                                                                   (const __half*)pred, (const __half*)target,
                                                                   (__half*)loss, (__half*)grad, dm_mu, dm_s1, dm_s12);
    else
        l1_ssim_forward_kernel<__half, false><<<grid, 256, 0, st>>>(width, height, c1, c2, s_ssim, s_l1,
                                                                    (const __half*)pred, (const __half*)target,
                                                                    (__half*)loss, (__half*)grad, dm_mu, dm_s1, dm_s12);
}

void launch_ssim_backward(uint32_t width, uint32_t height, float s, const float* pred, const float* target,
                          float* grad, const float* dm_mu, const float* dm_s1, const float* dm_s12, hipStream_t st) {
    if (width == 0 || height == 0) return;
    dim3 grid((width + kOT - 1) / kOT, (height + kOT - 1) / kOT, 3);
    ssim_backward_kernel<float><<<grid, 256, 0, st>>>(width, height, s, pred, target, grad, dm_mu, dm_s1, dm_s12);
}

void launch_ssim_backward_f16(uint32_t width, uint32_t height, float s, const void* pred, const void* target,
                              void* grad, const float* dm_mu, const float* dm_s1, const float* dm_s12,
                              hipStream_t st) {
    if (width == 0 || height == 0) return;
    dim3 grid((width + kOT - 1) / kOT, (height + kOT - 1) / kOT, 3);
    ssim_backward_kernel<__half><<<grid, 256, 0, st>>>(width, height, s, (const __half*)pred, (const __half*)target,
                                                       (__half*)grad, dm_mu, dm_s1, dm_s12);
}

// ------------------------------------------------------------------ PSNR

// psnr.cu:24-36 and :72-128: sum over the padded elements of
// (saturate(pred) - target)^2. One double partial per workgroup (grid-strided
// float4 reads, wave then workgroup reduction), then one workgroup adds the
// partials in index order: the same sum on every run.
__global__ void __launch_bounds__(256) sq_diff_partial_kernel(const float4* __restrict__ pred,
                                                               const float4* __restrict__ target, int64_t n4,
                                                               double* __restrict__ partial) {
    __shared__ double s_w[4];
    double acc = 0.0;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (int64_t)gridDim.x * 256) {
        const float4 p = pred[i], t = target[i];
        const float d0 = saturate(p.x) - t.x, d1 = saturate(p.y) - t.y;
        const float d2 = saturate(p.z) - t.z, d3 = saturate(p.w) - t.w;
        acc += (double)(d0 * d0) + (double)(d1 * d1) + (double)(d2 * d2) + (double)(d3 * d3);
    }
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_down(acc, off, 64);
    if ((threadIdx.x & 63u) == 0u) s_w[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) partial[blockIdx.x] = (s_w[0] + s_w[1]) + (s_w[2] + s_w[3]);
}

// The same over half images (psnr.cu:38-70): each half widened to float
// before saturate; 16-byte loads of 8 halves.
__global__ void __launch_bounds__(256) sq_diff_partial_f16_kernel(const uint4* __restrict__ pred,
                                                                   const uint4* __restrict__ target, int64_t n8,
                                                                   double* __restrict__ partial) {
    __shared__ double s_w[4];
    double acc = 0.0;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n8; i += (int64_t)gridDim.x * 256) {
        const uint4 p = pred[i], t = target[i];
        const uint32_t pw[4] = {p.x, p.y, p.z, p.w}, tw[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const __half* ph = (const __half*)&pw[k];
            const __half* th = (const __half*)&tw[k];
            const float d0 = saturate(__half2float(ph[0])) - __half2float(th[0]);
            const float d1 = saturate(__half2float(ph[1])) - __half2float(th[1]);
            acc += (double)(d0 * d0) + (double)(d1 * d1);
        }
    }
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_down(acc, off, 64);
    if ((threadIdx.x & 63u) == 0u) s_w[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) partial[blockIdx.x] = (s_w[0] + s_w[1]) + (s_w[2] + s_w[3]);
}

__global__ void __launch_bounds__(64) sum_partials_kernel(const double* __restrict__ partial, int n,
                                                          double* __restrict__ out) {
    double acc = 0.0;
    for (int i = (int)threadIdx.x; i < n; i += 64) acc += partial[i];
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_down(acc, off, 64);
    if (threadIdx.x == 0) *out = acc;
}

constexpr int kPsnrBlocks = 1024;
int psnr_scratch_doubles() { return kPsnrBlocks + 1; }

void launch_sq_diff_sum(const float* pred, const float* target, int64_t n_padded, double* scratch, hipStream_t s) {
    const int64_t n4 = n_padded / 4;   // padded planes hold whole 8x8 blocks
    const int blocks = (int)std::min<int64_t>(kPsnrBlocks, std::max<int64_t>(1, (n4 + 255) / 256));
    sq_diff_partial_kernel<<<blocks, 256, 0, s>>>((const float4*)pred, (const float4*)target, n4, scratch);
    sum_partials_kernel<<<1, 64, 0, s>>>(scratch, blocks, scratch + kPsnrBlocks);
}

void launch_sq_diff_sum_f16(const void* pred, const void* target, int64_t n_padded, double* scratch, hipStream_t s) {
    const int64_t n8 = n_padded / 8;   // padded planes hold whole 8x8 blocks
    const int blocks = (int)std::min<int64_t>(kPsnrBlocks, std::max<int64_t>(1, (n8 + 255) / 256));
    sq_diff_partial_f16_kernel<<<blocks, 256, 0, s>>>((const uint4*)pred, (const uint4*)target, n8, scratch);
    sum_partials_kernel<<<1, 64, 0, s>>>(scratch, blocks, scratch + kPsnrBlocks);
}

}  // namespace tgs
