// Per-Gaussian preprocess: projection, EWA covariance, conic, tile bounds,
// exact tile count and SH -> RGB.
// Follows tinygs/src/rasterizer/fastgs_ours/kernels_forward.cuh:157-412
// (with will_primitive_contribute :49-84, compute_exact_n_touched_tiles
// :87-153, convert_sh_to_color :22-46).
//
// MI355X layout: one thread per Gaussian, 256-thread workgroups (4 wave64).
// Per-primitive outputs are SoA with 8/16-byte records so the blend's LDS
// staging loads are single dwordx2/x4 transactions. The exact tile count
// spreads the rect tiles of a wave's 64 primitives over its lanes, 64 tile
// tests per iteration, so neither outliers nor uneven small rects leave lanes
// idle.
//
// Every floating-point expression here mirrors the CPU oracle operation for
// operation (this file is compiled with -ffp-contract=off), so visibility,
// bounds and tile counts are bit-identical to it.
#include "common.h"
#include "kernels.h"
#include "fgs16.h"
#include "rect_tasks.h"

namespace tgs {

// kernels_forward.cuh:49-84, on the mean shifted by -0.5 (:94).
__device__ __forceinline__ bool will_contribute(float mx, float my, float ca, float cb, float cc, uint32_t tile_x,
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

// Exact tile counts of the wave's 64 primitives, their rect tiles spread over
// the wave's lanes (rect_tasks.h). Hits are counted, and the outcomes of rect
// tiles 0..31 kept as a bit mask, with LDS atomics: the results do not depend
// on the order of the tests. test(par, tile_x, tile_y) sees the owner's NP
// parameter words. s: this wave's kRectSlice words. Called by the whole wave.
constexpr int kRectSlice = 3 * 64;

template <int NP, class Test>
__device__ __forceinline__ void wave_rect_tests(uint32_t nrect, uint32_t xmin, uint32_t ymin, uint32_t bw,
                                                const uint32_t (&par)[NP], uint32_t* s, uint32_t& cnt,
                                                uint32_t& bits, Test test) {
    const uint32_t lane = lane_id();
    uint32_t* s_mark = s;
    uint32_t* s_cnt = s + 64;
    uint32_t* s_bits = s + 128;
    const uint32_t incl = wave_inclusive_scan_u32(nrect);
    const uint32_t total = readlane_u32(incl, 63);
    const uint32_t ex = incl - nrect, org = xmin | (ymin << 16);
    s_cnt[lane] = 0u;
    s_bits[lane] = 0u;
    uint32_t carry = 0;
    for (uint32_t base = 0; base < total; base += kWave) {
        const uint32_t j = wave_task_owner(s_mark, nrect, ex, base, carry);
        const uint32_t exj = lane_gather(j, ex), orgj = lane_gather(j, org), w = lane_gather(j, bw);
        uint32_t pj[NP];
#pragma unroll
        for (int q = 0; q < NP; ++q) pj[q] = lane_gather(j, par[q]);
        const uint32_t t = base + lane;
        if (t < total) {
            const uint32_t k = t - exj;
            uint32_t col, row;
            rect_tile_of(k, w, col, row);
            if (test(pj, (orgj & 0xffffu) + col, (orgj >> 16) + row)) {
                atomicAdd(&s_cnt[j], 1u);
                if (k < 32u) atomicOr(&s_bits[j], 1u << k);
            }
        }
    }
    wave_lds_sync();
    cnt = s_cnt[lane];
    bits = s_bits[lane];
}

template <typename ShT>
__device__ __forceinline__ void sh_to_color(const ShT* __restrict__ sh0, const ShT* r, int64_t i, float px, float py,
                                            float pz, const CamParams& cam, int bases, float* out) {
    for (int c = 0; c < 3; ++c) out[c] = 0.5f + 0.28209479177387814f * load_as_float(sh0, 3 * i + c);
    if (bases <= 1) return;
    const float vx = px - cam.cam_pos[0], vy = py - cam.cam_pos[1], vz = pz - cam.cam_pos[2];
    const float inv = 1.0f / __builtin_sqrtf(vx * vx + vy * vy + vz * vz);
    const float x = vx * inv, y = vy * inv, z = vz * inv;
    float k[15];
    k[0] = -0.48860251190291987f * y;
    k[1] = 0.48860251190291987f * z;
    k[2] = -0.48860251190291987f * x;
    int nb = 3;
    if (bases > 4) {
        const float xx = x * x, yy = y * y, zz = z * z;
        const float xy = x * y, xz = x * z, yz = y * z;
        k[3] = 1.0925484305920792f * xy;
        k[4] = -1.0925484305920792f * yz;
        k[5] = 0.94617469575755997f * zz - 0.31539156525251999f;
        k[6] = -1.0925484305920792f * xz;
        k[7] = 0.54627421529603959f * xx - 0.54627421529603959f * yy;
        nb = 8;
        if (bases > 9) {
            k[8] = 0.59004358992664352f * y * (-3.0f * xx + yy);
            k[9] = 2.8906114426405538f * xy * z;
            k[10] = 0.45704579946446572f * y * (1.0f - 5.0f * zz);
            k[11] = 0.3731763325901154f * z * (5.0f * zz - 3.0f);
            k[12] = 0.45704579946446572f * x * (1.0f - 5.0f * zz);
            k[13] = 1.4453057213202769f * z * (xx - yy);
            k[14] = 0.59004358992664352f * x * (-xx + 3.0f * yy);
            nb = 15;
        }
    }
    for (int b = 0; b < nb; ++b)
        for (int c = 0; c < 3; ++c) out[c] = out[c] + k[b] * load_as_float(r, 3 * b + c);
}

// SH-rest coefficients of a workgroup's 256 primitives are one contiguous
// run, staged in LDS with 16-byte lane-contiguous loads. sh_stage_load issues
// the loads first and holds them in registers through the projection and the
// tile tests; sh_stage_store writes them to LDS and synchronises the
// workgroup just before the colour (every thread must reach it).
template <typename ShT>
struct ShStage {
    static constexpr int kVec = (256 * 45 * (int)sizeof(ShT) + 16 * 256 - 1) / (16 * 256);   // uint4 per thread
    uint4 v[kVec];
    int64_t blk0;
    int count, nvec;
};

template <typename ShT>
__device__ __forceinline__ void sh_stage_load(ShStage<ShT>& st, const ShT* __restrict__ shr, int64_t n, int bases) {
    st.blk0 = (int64_t)blockIdx.x * 256;
    st.count = bases > 1 ? (int)min((int64_t)256, n - st.blk0) * 45 : 0;
    st.nvec = (st.count * (int)sizeof(ShT)) >> 4;
    const uint4* s4 = (const uint4*)(shr + st.blk0 * 45);
#pragma unroll
    for (int q = 0; q < ShStage<ShT>::kVec; ++q) {
        const int v = (int)threadIdx.x + 256 * q;
        st.v[q] = v < st.nvec ? s4[v] : make_uint4(0u, 0u, 0u, 0u);
    }
}

template <typename ShT>
__device__ __forceinline__ void sh_stage_store(const ShStage<ShT>& st, ShT* s_sh, const ShT* __restrict__ shr) {
    uint4* d4 = (uint4*)s_sh;
#pragma unroll
    for (int q = 0; q < ShStage<ShT>::kVec; ++q) {
        const int v = (int)threadIdx.x + 256 * q;
        if (v < st.nvec) d4[v] = st.v[q];
    }
    // the elements after the last whole 16 bytes
    for (int e = (st.nvec << 4) / (int)sizeof(ShT) + (int)threadIdx.x; e < st.count; e += 256)
        s_sh[e] = shr[st.blk0 * 45 + e];
    __syncthreads();
}

template <typename ShT>
__global__ void __launch_bounds__(256) preprocess_kernel(
    const float* __restrict__ means, const float* __restrict__ scales, const float* __restrict__ rots,
    const float* __restrict__ opac, const ShT* __restrict__ sh0, const ShT* __restrict__ shr, int64_t n, int bases,
    CamParams cam, uint32_t* __restrict__ n_touched, uint4* __restrict__ erec,
    float2* __restrict__ mean2d, float4* __restrict__ conic_opacity, float4* __restrict__ color_pt, uint32_t* __restrict__ depth_key,
    float4* __restrict__ densif, BinCtl* __restrict__ ctl) {
    __shared__ __align__(16) ShT s_sh[256 * 45];
    __shared__ uint32_t s_rect[4][kRectSlice];
    if (ctl != nullptr && blockIdx.x == 0) bin_ctl_reset_block(ctl);   // (read first by the compaction)
    ShStage<ShT> shs;
    sh_stage_load(shs, shr, n, bases);
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    bool active = i < n;
    const int64_t ii = active ? i : n - 1;
    const uint32_t lane = lane_id();

    const float mx = means[3 * ii], my = means[3 * ii + 1], mz = means[3 * ii + 2];
    const float depth = cam.r3[0] * mx + cam.r3[1] * my + cam.r3[2] * mz + cam.r3[3];
    if (depth < cam.near_ || depth > cam.far_) active = false;
    const float opacity = 1.0f / (1.0f + det_expf(-opac[ii]));
    if (opacity < kMinAlpha) active = false;
    const float e0 = det_expf(scales[3 * ii]), e1 = det_expf(scales[3 * ii + 1]), e2 = det_expf(scales[3 * ii + 2]);
    const float vx = e0 * e0, vy = e1 * e1, vz = e2 * e2;
    const float qr = rots[4 * ii], qx = rots[4 * ii + 1], qy = rots[4 * ii + 2], qz = rots[4 * ii + 3];
    const float qrr = qr * qr, qxx_r = qx * qx, qyy_r = qy * qy, qzz_r = qz * qz;
    const float qn = qrr + qxx_r + qyy_r + qzz_r;
    if (qn < 1e-8f) active = false;
    // The reference's 32-lane warps leave together only when none of their
    // threads is still active (kernels_forward.cuh:261-263); every thread of
    // a warp that stays, culled or not, folds its own screen radius into the
    // densification info (:342-348). Here a wave64 holds two such groups.
    const uint64_t live = ballot(active);
    const bool radius = densif != nullptr && i < n && (lane < 32u ? (uint32_t)live : (uint32_t)(live >> 32)) != 0u;

    uint32_t xmin = 0, xmax = 0, ymin = 0, ymax = 0, nmax = 0;
    float ca = 0.f, cb = 0.f, cc = 0.f, m2x = 0.f, m2y = 0.f, pthr = 0.f;
    if (active || radius) {
        const float qxx = 2.0f * qxx_r / qn, qyy = 2.0f * qyy_r / qn, qzz = 2.0f * qzz_r / qn;
        const float qxy = 2.0f * qx * qy / qn, qxz = 2.0f * qx * qz / qn, qyz = 2.0f * qy * qz / qn;
        const float qrx = 2.0f * qr * qx / qn, qry = 2.0f * qr * qy / qn, qrz = 2.0f * qr * qz / qn;
        const float R11 = 1.0f - (qyy + qzz), R12 = qxy - qrz, R13 = qry + qxz;
        const float R21 = qrz + qxy, R22 = 1.0f - (qxx + qzz), R23 = qyz - qrx;
        const float R31 = qxz - qry, R32 = qrx + qyz, R33 = 1.0f - (qxx + qyy);
        const float S11 = R11 * vx, S12 = R12 * vy, S13 = R13 * vz;
        const float S21 = R21 * vx, S22 = R22 * vy, S23 = R23 * vz;
        const float S31 = R31 * vx, S32 = R32 * vy, S33 = R33 * vz;
        const float c11 = S11 * R11 + S12 * R12 + S13 * R13;
        const float c12 = S11 * R21 + S12 * R22 + S13 * R23;
        const float c13 = S11 * R31 + S12 * R32 + S13 * R33;
        const float c22 = S21 * R21 + S22 * R22 + S23 * R23;
        const float c23 = S21 * R31 + S22 * R32 + S23 * R33;
        const float c33 = S31 * R31 + S32 * R32 + S33 * R33;
        const float x = (cam.r1[0] * mx + cam.r1[1] * my + cam.r1[2] * mz + cam.r1[3]) / depth;
        const float y = (cam.r2[0] * mx + cam.r2[1] * my + cam.r2[2] * mz + cam.r2[3]) / depth;
        const float clip_left = cam.clip_left, clip_right = cam.clip_right;
        const float clip_top = cam.clip_top, clip_bottom = cam.clip_bottom;
        const float tx = __builtin_fmaxf(clip_left, __builtin_fminf(x, clip_right));
        const float ty = __builtin_fmaxf(clip_top, __builtin_fminf(y, clip_bottom));
        const float j11 = cam.fx / depth, j13 = -j11 * tx, j22 = cam.fy / depth, j23 = -j22 * ty;
        const float jw1x = j11 * cam.r1[0] + j13 * cam.r3[0], jw1y = j11 * cam.r1[1] + j13 * cam.r3[1],
                    jw1z = j11 * cam.r1[2] + j13 * cam.r3[2];
        const float jw2x = j22 * cam.r2[0] + j23 * cam.r3[0], jw2y = j22 * cam.r2[1] + j23 * cam.r3[1],
                    jw2z = j22 * cam.r2[2] + j23 * cam.r3[2];
        const float a1x = jw1x * c11 + jw1y * c12 + jw1z * c13;
        const float a1y = jw1x * c12 + jw1y * c22 + jw1z * c23;
        const float a1z = jw1x * c13 + jw1y * c23 + jw1z * c33;
        const float a2x = jw2x * c11 + jw2y * c12 + jw2z * c13;
        const float a2y = jw2x * c12 + jw2y * c22 + jw2z * c23;
        const float a2z = jw2x * c13 + jw2y * c23 + jw2z * c33;
        float cv_a = a1x * jw1x + a1y * jw1y + a1z * jw1z;
        const float cv_b = a1x * jw2x + a1y * jw2y + a1z * jw2z;
        float cv_c = a2x * jw2x + a2y * jw2y + a2z * jw2z;
        cv_a += kDilation;
        cv_c += kDilation;
        const float det = cv_a * cv_c - cv_b * cv_b;
        if (det < 1e-8f) active = false;
        if (radius) {
            // kernels_forward.cuh:342-348: fmaxf(old, r); a NaN radius keeps the old value
            const float mid = 0.5f * (cv_a + cv_c);
            const float l1 = mid + __builtin_sqrtf(__builtin_fmaxf(0.1f, mid * mid - det));
            const float l2 = mid - __builtin_sqrtf(__builtin_fmaxf(0.1f, mid * mid - det));
            const float rad = __builtin_ceilf(3.0f * __builtin_sqrtf(__builtin_fmaxf(l1, l2)));
            const float old = densif[ii].w;
            const float nv = __builtin_fmaxf(old, rad);
            if (f2u(nv) != f2u(old)) densif[ii].w = nv;
        }
        if (active) {
            ca = cv_c / det;
            cb = -cv_b / det;
            cc = cv_a / det;
            m2x = x * cam.fx + cam.cx;
            m2y = y * cam.fy + cam.cy;
            pthr = det_logf(opacity * 255.0f);
            const float pfac = __builtin_sqrtf(2.0f * pthr);
            const float ext_x = __builtin_fmaxf(pfac * __builtin_sqrtf(cv_a) - 0.5f, 0.0f);
            const float ext_y = __builtin_fmaxf(pfac * __builtin_sqrtf(cv_c) - 0.5f, 0.0f);
            const int32_t bx0 = sat_floor_i32((m2x - ext_x) / 16.0f);
            const int32_t bx1 = sat_ceil_i32((m2x + ext_x) / 16.0f);
            const int32_t by0 = sat_floor_i32((m2y - ext_y) / 16.0f);
            const int32_t by1 = sat_ceil_i32((m2y + ext_y) / 16.0f);
            xmin = min((uint32_t)max(bx0, 0), cam.grid_w);
            xmax = min((uint32_t)max(bx1, 0), cam.grid_w);
            ymin = min((uint32_t)max(by0, 0), cam.grid_h);
            ymax = min((uint32_t)max(by1, 0), cam.grid_h);
            nmax = (xmax - xmin) * (ymax - ymin);
            if (nmax == 0) active = false;
        }
    }

    // exact tile count over the rect (kernels_forward.cuh:87-153); the
    // outcomes for rect tiles 0..31 (row-major in the rect) are kept as a bit
    // mask, so the instance emission need not repeat the test there
    const float smx = m2x - 0.5f, smy = m2y - 0.5f;
    uint32_t cnt = 0, bits = 0;
    {
        const uint32_t par[6] = {f2u(smx), f2u(smy), f2u(ca), f2u(cb), f2u(cc), f2u(pthr)};
        wave_rect_tests(active ? nmax : 0u, xmin, ymin, xmax - xmin, par, s_rect[threadIdx.x >> 6], cnt, bits,
                        [&](const uint32_t(&pj)[6], uint32_t tx_, uint32_t ty_) {
                            return will_contribute(u2f(pj[0]), u2f(pj[1]), u2f(pj[2]), u2f(pj[3]), u2f(pj[4]), tx_,
                                                   ty_, u2f(pj[5]));
                        });
    }

    sh_stage_store(shs, s_sh, shr);
    if (i >= n) return;
    if (!active || cnt == 0) {
        n_touched[i] = 0;
        return;
    }
    n_touched[i] = cnt;
    erec[i] = make_uint4(xmin | (xmax << 16), ymin | (ymax << 16), bits, 0u);
    mean2d[i] = make_float2(m2x, m2y);
    conic_opacity[i] = make_float4(ca, cb, cc, opacity);
    float col[3];
    sh_to_color(sh0, s_sh + 45 * threadIdx.x, i, mx, my, mz, cam, bases, col);
    color_pt[i] = make_float4(col[0], col[1], col[2], pthr);
    depth_key[i] = f2u(depth);
}

// preprocess_cu of the fp16-image rasterizer (FGS16), tinygs/src/rasterizer/
// fastgs_ours_fp16/kernels_forward.cuh:249-500: the fp32 projection with the
// logit rounded to half before the sigmoid (and read only for primitives
// still in [near, far]), the quaternion read only for active primitives, a
// half conic and opacity, the power threshold from the half opacity, the
// half tile test (fgs16.h) and an 8-bit colour, saturate(c) * 255 truncated
// (rasterization_config.h:104-108). Outputs: n_touched, the emission record
// as the fp32 preprocess, mean2d, conic_opacity (the halves as floats) and
// info[i] = (a | b << 16, c | opacity << 16, r | g << 8 | b << 16, power
// threshold bits), which the instance emission's exact test also reads.
template <typename ShT>
__global__ void __launch_bounds__(256) preprocess16_kernel(
    const float* __restrict__ means, const float* __restrict__ scales, const float* __restrict__ rots,
    const float* __restrict__ opac, const ShT* __restrict__ sh0, const ShT* __restrict__ shr, int64_t n, int bases,
    CamParams cam, uint32_t* __restrict__ n_touched, uint4* __restrict__ erec,
    float2* __restrict__ mean2d, float4* __restrict__ conic_opacity, uint4* __restrict__ info,
    uint32_t* __restrict__ depth_key, float4* __restrict__ densif, BinCtl* __restrict__ ctl) {
    __shared__ __align__(16) ShT s_sh[256 * 45];
    __shared__ uint32_t s_rect[4][kRectSlice];
    if (ctl != nullptr && blockIdx.x == 0) bin_ctl_reset_block(ctl);   // (read first by the compaction)
    ShStage<ShT> shs;
    sh_stage_load(shs, shr, n, bases);
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    bool active = i < n;
    const int64_t ii = active ? i : n - 1;
    const uint32_t lane = lane_id();

    const float mx = means[3 * ii], my = means[3 * ii + 1], mz = means[3 * ii + 2];
    const float depth = cam.r3[0] * mx + cam.r3[1] * my + cam.r3[2] * mz + cam.r3[3];
    if (depth < cam.near_ || depth > cam.far_) active = false;
    const h16 raw_o = active ? h_rn(opac[ii]) : (h16)0.0f;
    const float f_opacity = 1.0f / (1.0f + det_expf(-(float)raw_o));
    if (f_opacity < kMinAlpha) active = false;
    const h16 opacity = h_rn(f_opacity);
    const float e0 = det_expf(scales[3 * ii]), e1 = det_expf(scales[3 * ii + 1]), e2 = det_expf(scales[3 * ii + 2]);
    const float vx = e0 * e0, vy = e1 * e1, vz = e2 * e2;
    float qr = 0.f, qx = 0.f, qy = 0.f, qz = 0.f;
    if (active) {
        qr = rots[4 * ii];
        qx = rots[4 * ii + 1];
        qy = rots[4 * ii + 2];
        qz = rots[4 * ii + 3];
    }
    const float qrr = qr * qr, qxx_r = qx * qx, qyy_r = qy * qy, qzz_r = qz * qz;
    const float qn = qrr + qxx_r + qyy_r + qzz_r;
    if (qn < 1e-8f) active = false;
    // the reference's 32-lane warps: radius folding per 32-primitive group (kernels_forward.cuh:326-329,405-411)
    const uint64_t live = ballot(active);
    const bool radius = densif != nullptr && i < n && (lane < 32u ? (uint32_t)live : (uint32_t)(live >> 32)) != 0u;

    uint32_t xmin = 0, xmax = 0, ymin = 0, ymax = 0, nmax = 0;
    float m2x = 0.f, m2y = 0.f, pthr = 0.f;
    h16 hca = (h16)0.f, hcb = (h16)0.f, hcc = (h16)0.f;
    if (active || radius) {
        const float qxx = 2.0f * qxx_r / qn, qyy = 2.0f * qyy_r / qn, qzz = 2.0f * qzz_r / qn;
        const float qxy = 2.0f * qx * qy / qn, qxz = 2.0f * qx * qz / qn, qyz = 2.0f * qy * qz / qn;
        const float qrx = 2.0f * qr * qx / qn, qry = 2.0f * qr * qy / qn, qrz = 2.0f * qr * qz / qn;
        const float R11 = 1.0f - (qyy + qzz), R12 = qxy - qrz, R13 = qry + qxz;
        const float R21 = qrz + qxy, R22 = 1.0f - (qxx + qzz), R23 = qyz - qrx;
        const float R31 = qxz - qry, R32 = qrx + qyz, R33 = 1.0f - (qxx + qyy);
        const float S11 = R11 * vx, S12 = R12 * vy, S13 = R13 * vz;
        const float S21 = R21 * vx, S22 = R22 * vy, S23 = R23 * vz;
        const float S31 = R31 * vx, S32 = R32 * vy, S33 = R33 * vz;
        const float c11 = S11 * R11 + S12 * R12 + S13 * R13;
        const float c12 = S11 * R21 + S12 * R22 + S13 * R23;
        const float c13 = S11 * R31 + S12 * R32 + S13 * R33;
        const float c22 = S21 * R21 + S22 * R22 + S23 * R23;
        const float c23 = S21 * R31 + S22 * R32 + S23 * R33;
        const float c33 = S31 * R31 + S32 * R32 + S33 * R33;
        const float x = (cam.r1[0] * mx + cam.r1[1] * my + cam.r1[2] * mz + cam.r1[3]) / depth;
        const float y = (cam.r2[0] * mx + cam.r2[1] * my + cam.r2[2] * mz + cam.r2[3]) / depth;
        const float clip_left = cam.clip_left, clip_right = cam.clip_right;
        const float clip_top = cam.clip_top, clip_bottom = cam.clip_bottom;
        const float tx = __builtin_fmaxf(clip_left, __builtin_fminf(x, clip_right));
        const float ty = __builtin_fmaxf(clip_top, __builtin_fminf(y, clip_bottom));
        const float j11 = cam.fx / depth, j13 = -j11 * tx, j22 = cam.fy / depth, j23 = -j22 * ty;
        const float jw1x = j11 * cam.r1[0] + j13 * cam.r3[0], jw1y = j11 * cam.r1[1] + j13 * cam.r3[1],
                    jw1z = j11 * cam.r1[2] + j13 * cam.r3[2];
        const float jw2x = j22 * cam.r2[0] + j23 * cam.r3[0], jw2y = j22 * cam.r2[1] + j23 * cam.r3[1],
                    jw2z = j22 * cam.r2[2] + j23 * cam.r3[2];
        const float a1x = jw1x * c11 + jw1y * c12 + jw1z * c13;
        const float a1y = jw1x * c12 + jw1y * c22 + jw1z * c23;
        const float a1z = jw1x * c13 + jw1y * c23 + jw1z * c33;
        const float a2x = jw2x * c11 + jw2y * c12 + jw2z * c13;
        const float a2y = jw2x * c12 + jw2y * c22 + jw2z * c23;
        const float a2z = jw2x * c13 + jw2y * c23 + jw2z * c33;
        float cv_a = a1x * jw1x + a1y * jw1y + a1z * jw1z;
        const float cv_b = a1x * jw2x + a1y * jw2y + a1z * jw2z;
        float cv_c = a2x * jw2x + a2y * jw2y + a2z * jw2z;
        cv_a += kDilation;
        cv_c += kDilation;
        const float det = cv_a * cv_c - cv_b * cv_b;
        if (det < 1e-8f) active = false;
        if (radius) {
            const float mid = 0.5f * (cv_a + cv_c);
            const float l1 = mid + __builtin_sqrtf(__builtin_fmaxf(0.1f, mid * mid - det));
            const float l2 = mid - __builtin_sqrtf(__builtin_fmaxf(0.1f, mid * mid - det));
            const float rad = __builtin_ceilf(3.0f * __builtin_sqrtf(__builtin_fmaxf(l1, l2)));
            const float old = densif[ii].w;
            const float nv = __builtin_fmaxf(old, rad);
            if (f2u(nv) != f2u(old)) densif[ii].w = nv;
        }
        if (active) {
            const float ca = cv_c / det, cb = -cv_b / det, cc = cv_a / det;
            m2x = x * cam.fx + cam.cx;
            m2y = y * cam.fy + cam.cy;
            hca = h_rn(ca);
            hcb = h_rn(cb);
            hcc = h_rn(cc);
            pthr = det_logf((float)opacity * 255.0f);
            const float pfac = __builtin_sqrtf(2.0f * pthr);
            const float ext_x = __builtin_fmaxf(pfac * __builtin_sqrtf(cv_a) - 0.5f, 0.0f);
            const float ext_y = __builtin_fmaxf(pfac * __builtin_sqrtf(cv_c) - 0.5f, 0.0f);
            const int32_t bx0 = sat_floor_i32((m2x - ext_x) / 16.0f);
            const int32_t bx1 = sat_ceil_i32((m2x + ext_x) / 16.0f);
            const int32_t by0 = sat_floor_i32((m2y - ext_y) / 16.0f);
            const int32_t by1 = sat_ceil_i32((m2y + ext_y) / 16.0f);
            xmin = min((uint32_t)max(bx0, 0), cam.grid_w);
            xmax = min((uint32_t)max(bx1, 0), cam.grid_w);
            ymin = min((uint32_t)max(by0, 0), cam.grid_h);
            ymax = min((uint32_t)max(by1, 0), cam.grid_h);
            nmax = (xmax - xmin) * (ymax - ymin);
            if (nmax == 0) active = false;
        }
    }

    const float smx = m2x - 0.5f, smy = m2y - 0.5f;
    uint32_t cnt = 0, bits = 0;
    {
        const uint32_t par[5] = {f2u(smx), f2u(smy), (uint32_t)hbits(hca) | ((uint32_t)hbits(hcb) << 16),
                                 (uint32_t)hbits(hcc), f2u(pthr)};
        wave_rect_tests(active ? nmax : 0u, xmin, ymin, xmax - xmin, par, s_rect[threadIdx.x >> 6], cnt, bits,
                        [&](const uint32_t(&pj)[5], uint32_t tx_, uint32_t ty_) {
                            return will_contribute_half(u2f(pj[0]), u2f(pj[1]), hfrom((uint16_t)(pj[2] & 0xffffu)),
                                                        hfrom((uint16_t)(pj[2] >> 16)), hfrom((uint16_t)pj[3]), tx_,
                                                        ty_, u2f(pj[4]));
                        });
    }

    sh_stage_store(shs, s_sh, shr);
    if (i >= n) return;
    if (!active || cnt == 0) {
        n_touched[i] = 0;
        return;
    }
    n_touched[i] = cnt;
    erec[i] = make_uint4(xmin | (xmax << 16), ymin | (ymax << 16), bits, 0u);
    const uint32_t c01 = (uint32_t)hbits(hca) | ((uint32_t)hbits(hcb) << 16);
    const uint32_t c2o = (uint32_t)hbits(hcc) | ((uint32_t)hbits(opacity) << 16);
    mean2d[i] = make_float2(m2x, m2y);
    conic_opacity[i] = make_float4((float)hca, (float)hcb, (float)hcc, (float)opacity);
    float col[3];
    sh_to_color(sh0, s_sh + 45 * threadIdx.x, i, mx, my, mz, cam, bases, col);
    uint32_t rgb = 0;
    for (int c = 0; c < 3; ++c) rgb |= (uint32_t)(uint8_t)(saturate(col[c]) * 255.0f) << (8 * c);
    info[i] = make_uint4(c01, c2o, rgb, f2u(pthr));
    depth_key[i] = f2u(depth);
}

void launch_preprocess16(const GaussianView& g, const CamParams& cam, uint32_t* n_touched, uint4* erec,
                         float2* mean2d, float4* conic_opacity, uint4* info, uint32_t* depth_key,
                         float* densif, BinCtl* ctl, hipStream_t s) {
    if (g.n <= 0) {
        if (ctl) launch_bin_ctl_reset(ctl, s);
        return;
    }
    const int bases = (g.sh_degree + 1) * (g.sh_degree + 1);
    const unsigned grid = (unsigned)((g.n + 255) / 256);
    if (g.sh_dtype == kShF16)
        preprocess16_kernel<__half><<<grid, 256, 0, s>>>(g.means, g.scales, g.rotations, g.opacities,
                                                         (const __half*)g.sh0, (const __half*)g.sh_rest, g.n, bases,
                                                         cam, n_touched, erec, mean2d, conic_opacity, info,
                                                         depth_key, (float4*)densif, ctl);
    else
        preprocess16_kernel<float><<<grid, 256, 0, s>>>(g.means, g.scales, g.rotations, g.opacities,
                                                        (const float*)g.sh0, (const float*)g.sh_rest, g.n, bases, cam,
                                                        n_touched, erec, mean2d, conic_opacity, info,
                                                        depth_key, (float4*)densif, ctl);
}

void launch_preprocess(const GaussianView& g, const CamParams& cam, uint32_t* n_touched, uint4* erec,
                       float2* mean2d, float4* conic_opacity, float4* color_pt, uint32_t* depth_key, float* densif,
                       BinCtl* ctl, hipStream_t s) {
    if (g.n <= 0) {
        if (ctl) launch_bin_ctl_reset(ctl, s);
        return;
    }
    const int bases = (g.sh_degree + 1) * (g.sh_degree + 1);
    const unsigned grid = (unsigned)((g.n + 255) / 256);
    if (g.sh_dtype == kShF16) {
        preprocess_kernel<__half><<<grid, 256, 0, s>>>(g.means, g.scales, g.rotations, g.opacities,
                                                       (const __half*)g.sh0, (const __half*)g.sh_rest, g.n, bases,
                                                       cam, n_touched, erec, mean2d, conic_opacity,
                                                       color_pt, depth_key, (float4*)densif, ctl);
    } else {
        preprocess_kernel<float><<<grid, 256, 0, s>>>(g.means, g.scales, g.rotations, g.opacities,
                                                      (const float*)g.sh0, (const float*)g.sh_rest, g.n, bases, cam,
                                                      n_touched, erec, mean2d, conic_opacity, color_pt,
                                                      depth_key, (float4*)densif, ctl);
    }
}

}  // namespace tgs
