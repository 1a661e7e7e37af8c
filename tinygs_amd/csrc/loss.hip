// L1 and fused-SSIM loss / gradient on the 8x8-tiled channel-planar image.
// L1 follows tinygs/src/loss/l1.cu:19-42 (+ host scaling :109-151);
// SSIM follows tinygs/src/loss/fused_ssim.cu:55-267 (forward),
// :275-442 (backward), :797-916 (host): per channel, 16x16 output tiles with a
// 5-pixel halo in LDS, inputs rounded to fp16 for the statistics, zero
// padding outside the image, separable 11-tap Gaussian (sigma 1.5), and the
// three partial-derivative maps convolved back in fp32.
// Both accumulate into loss / grad (loss[i] += ..., grad[i] += ...).
// Sums use explicit fma in the order of the reference loops so the results
// match the CPU oracle's evaluation.
#include "common.h"
#include "kernels.h"

namespace tgs {

__constant__ float kGauss[11] = {0.001028380123898387f,  0.0075987582094967365f, 0.036000773310661316f,
                                 0.10936068743467331f,   0.21300552785396576f,   0.26601171493530273f,
                                 0.21300552785396576f,   0.10936068743467331f,   0.036000773310661316f,
                                 0.0075987582094967365f, 0.001028380123898387f};

__global__ void l1_kernel(const float* __restrict__ pred, const float* __restrict__ target, float* __restrict__ loss,
                          float* __restrict__ grad, int64_t n, float s) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float p = saturate(pred[i]);
    const float d = p - target[i];
    if (loss) loss[i] = __builtin_fmaf(__builtin_fabsf(d), s, loss[i]);
    if (grad) grad[i] = __builtin_fmaf(__builtin_copysignf(1.0f, d), s, grad[i]);
}

void launch_l1(const float* pred, const float* target, float* loss, float* grad, int64_t n_padded, float s,
               hipStream_t st) {
    if (n_padded <= 0) return;
    l1_kernel<<<(unsigned)((n_padded + 255) / 256), 256, 0, st>>>(pred, target, loss, grad, n_padded, s);
}

constexpr int kSX = 26;  // 16 + 2 * 5

__device__ __forceinline__ float round_half(float x) { return __half2float(__float2half_rn(x)); }

__global__ void __launch_bounds__(256) ssim_forward_kernel(uint32_t W, uint32_t H, float C1, float C2, float s,
                                                           const float* __restrict__ pred,
                                                           const float* __restrict__ target,
                                                           float* __restrict__ loss, float* __restrict__ dm_mu,
                                                           float* __restrict__ dm_s1, float* __restrict__ dm_s12) {
    __shared__ float2 sT[kSX][kSX];
    __shared__ float xc[kSX][16][5];
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    const int bx = blockIdx.x * 16, by = blockIdx.y * 16;
    const uint32_t tw = (W + 7u) >> 3, th = (H + 7u) >> 3;
    const uint32_t cs = tw * th * 64u;
    const int pxx = bx + tx, pyy = by + ty;
    const bool inside = pxx < (int)W && pyy < (int)H;
    const uint32_t pi = inside ? tiled_index((uint32_t)pyy, (uint32_t)pxx, tw) : 0u;
    for (int c = 0; c < 3; ++c) {
        for (int k = threadIdx.x; k < kSX * kSX; k += 256) {
            const int ly = k / kSX, lx = k % kSX;
            const int gx = bx + lx - 5, gy = by + ly - 5;
            float2 v = make_float2(0.f, 0.f);
            if (gx >= 0 && gy >= 0 && gx < (int)W && gy < (int)H) {
                const uint32_t q = tiled_index((uint32_t)gy, (uint32_t)gx, tw) + (uint32_t)c * cs;
                v = make_float2(round_half(pred[q]), round_half(target[q]));
            }
            sT[ly][lx] = v;
        }
        __syncthreads();
        for (int ly = ty; ly < kSX; ly += 16) {
            float sx = 0.f, sx2 = 0.f, sy = 0.f, sy2 = 0.f, sxy = 0.f;
#pragma unroll
            for (int d = 0; d < 11; ++d) {
                const float wv = kGauss[d];
                const float2 v = sT[ly][tx + d];
                sx = __builtin_fmaf(v.x, wv, sx);
                sx2 = __builtin_fmaf(v.x * v.x, wv, sx2);
                sy = __builtin_fmaf(v.y, wv, sy);
                sy2 = __builtin_fmaf(v.y * v.y, wv, sy2);
                sxy = __builtin_fmaf(v.x * v.y, wv, sxy);
            }
            xc[ly][tx][0] = sx; xc[ly][tx][1] = sx2; xc[ly][tx][2] = sy; xc[ly][tx][3] = sy2; xc[ly][tx][4] = sxy;
        }
        __syncthreads();
        if (inside) {
            float o0 = 0.f, o1 = 0.f, o2 = 0.f, o3 = 0.f, o4 = 0.f;
#pragma unroll
            for (int d = 0; d < 11; ++d) {
                const float wv = kGauss[d];
                const float* cur = xc[ty + d][tx];
                o0 = __builtin_fmaf(cur[0], wv, o0);
                o1 = __builtin_fmaf(cur[1], wv, o1);
                o2 = __builtin_fmaf(cur[2], wv, o2);
                o3 = __builtin_fmaf(cur[3], wv, o3);
                o4 = __builtin_fmaf(cur[4], wv, o4);
            }
            const float mu1 = o0, mu2 = o2;
            const float mu1_sq = mu1 * mu1, mu2_sq = mu2 * mu2;
            const float s1 = o1 - mu1_sq, s2 = o3 - mu2_sq, s12 = o4 - mu1 * mu2;
            const float A = mu1_sq + mu2_sq + C1;
            const float B = s1 + s2 + C2;
            const float Cc = 2.0f * mu1 * mu2 + C1;
            const float D = 2.0f * s12 + C2;
            const float val = (Cc * D) / (A * B);
            const uint32_t q = pi + (uint32_t)c * cs;
            if (loss) loss[q] = __builtin_fmaf(1.0f - val, s, loss[q]);
            if (dm_mu) {
                dm_mu[q] = (mu2 * 2.0f * D) / (A * B) - (mu2 * 2.0f * Cc) / (A * B) -
                           (mu1 * 2.0f * Cc * D) / (A * A * B) + (mu1 * 2.0f * Cc * D) / (A * B * B);
                dm_s1[q] = (-Cc * D) / (A * B * B);
                dm_s12[q] = (2.0f * Cc) / (A * B);
            }
        }
        __syncthreads();
    }
}

__global__ void __launch_bounds__(256) ssim_backward_kernel(uint32_t W, uint32_t H, float s,
                                                            const float* __restrict__ pred,
                                                            const float* __restrict__ target,
                                                            float* __restrict__ grad, const float* __restrict__ dm_mu,
                                                            const float* __restrict__ dm_s1,
                                                            const float* __restrict__ dm_s12) {
    __shared__ float sD[3][kSX][kSX];
    __shared__ float sS[kSX][16][3];
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    const int bx = blockIdx.x * 16, by = blockIdx.y * 16;
    const uint32_t tw = (W + 7u) >> 3, th = (H + 7u) >> 3;
    const uint32_t cs = tw * th * 64u;
    const int pxx = bx + tx, pyy = by + ty;
    const bool inside = pxx < (int)W && pyy < (int)H;
    const uint32_t pi = inside ? tiled_index((uint32_t)pyy, (uint32_t)pxx, tw) : 0u;
    for (int c = 0; c < 3; ++c) {
        for (int k = threadIdx.x; k < kSX * kSX; k += 256) {
            const int ly = k / kSX, lx = k % kSX;
            const int gx = bx + lx - 5, gy = by + ly - 5;
            float a = 0.f, b = 0.f, d = 0.f;
            if (gx >= 0 && gy >= 0 && gx < (int)W && gy < (int)H) {
                const uint32_t q = tiled_index((uint32_t)gy, (uint32_t)gx, tw) + (uint32_t)c * cs;
                a = dm_mu[q]; b = dm_s1[q]; d = dm_s12[q];
            }
            sD[0][ly][lx] = a; sD[1][ly][lx] = b; sD[2][ly][lx] = d;
        }
        __syncthreads();
        for (int yy = ty; yy < kSX; yy += 16) {
            const int lx = tx + 5;
            float a0 = 0.f, a1 = 0.f, a2 = 0.f;
#pragma unroll
            for (int d = 1; d <= 5; ++d) {
                const float wv = kGauss[5 - d];
                a0 = __builtin_fmaf(sD[0][yy][lx - d] + sD[0][yy][lx + d], wv, a0);
                a1 = __builtin_fmaf(sD[1][yy][lx - d] + sD[1][yy][lx + d], wv, a1);
                a2 = __builtin_fmaf(sD[2][yy][lx - d] + sD[2][yy][lx + d], wv, a2);
            }
            const float wc = kGauss[5];
            a0 = __builtin_fmaf(sD[0][yy][lx], wc, a0);
            a1 = __builtin_fmaf(sD[1][yy][lx], wc, a1);
            a2 = __builtin_fmaf(sD[2][yy][lx], wc, a2);
            sS[yy][tx][0] = a0; sS[yy][tx][1] = a1; sS[yy][tx][2] = a2;
        }
        __syncthreads();
        if (inside) {
            const int ly = ty + 5;
            float a0 = 0.f, a1 = 0.f, a2 = 0.f;
#pragma unroll
            for (int d = 1; d <= 5; ++d) {
                const float wv = kGauss[5 - d];
                a0 = __builtin_fmaf(sS[ly - d][tx][0] + sS[ly + d][tx][0], wv, a0);
                a1 = __builtin_fmaf(sS[ly - d][tx][1] + sS[ly + d][tx][1], wv, a1);
                a2 = __builtin_fmaf(sS[ly - d][tx][2] + sS[ly + d][tx][2], wv, a2);
            }
            const float wc = kGauss[5];
            a0 = __builtin_fmaf(sS[ly][tx][0], wc, a0);
            a1 = __builtin_fmaf(sS[ly][tx][1], wc, a1);
            a2 = __builtin_fmaf(sS[ly][tx][2], wc, a2);
            const uint32_t q = pi + (uint32_t)c * cs;
            const float p1 = pred[q], p2 = target[q];
            const float dl = __builtin_fmaf(p2, a2, __builtin_fmaf(2.0f * p1, a1, a0));
            grad[q] = __builtin_fmaf(-s, dl, grad[q]);
        }
        __syncthreads();
    }
}

void launch_ssim_forward(uint32_t width, uint32_t height, float c1, float c2, float s, const float* pred,
                         const float* target, float* loss, float* dm_mu, float* dm_s1, float* dm_s12, hipStream_t st) {
    if (width == 0 || height == 0) return;
    dim3 grid((width + 15) / 16, (height + 15) / 16);
    ssim_forward_kernel<<<grid, 256, 0, st>>>(width, height, c1, c2, s, pred, target, loss, dm_mu, dm_s1, dm_s12);
}

void launch_ssim_backward(uint32_t width, uint32_t height, float s, const float* pred, const float* target,
                          float* grad, const float* dm_mu, const float* dm_s1, const float* dm_s12, hipStream_t st) {
    if (width == 0 || height == 0) return;
    dim3 grid((width + 15) / 16, (height + 15) / 16);
    ssim_backward_kernel<<<grid, 256, 0, st>>>(width, height, s, pred, target, grad, dm_mu, dm_s1, dm_s12);
}

}  // namespace tgs
