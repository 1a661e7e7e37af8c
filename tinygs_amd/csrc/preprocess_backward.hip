// Per-Gaussian backward: 2D gradients -> 3D mean, log-scale, quaternion,
// SH coefficients (and the opacity logit).
// Follows tinygs/src/rasterizer/fastgs_ours/kernels_backward.cuh:88-352 with
// convert_sh_to_color_backward :22-86. Runs only for primitives with
// n_touched > 0 (:117). Parameter gradients are accumulated (+=) as in the
// reference; the caller zeroes them.
//
// Reference semantics kept: dSigma2 with (det + 1e-8)^-2 and the symmetric-
// matrix off-diagonal convention (:204-214); tx/ty clamp mask (:244-247);
// quaternion gradient divided by |q|^3 (:332); the three double-precision
// literals of the SH direction gradient (:55-57). The opacity gradient is
// (sum of alpha * dL/dalpha) * (1 - opacity) (:921-922); the blend backward
// leaves the sum in its 2D-gradient records and it is applied here.
//
// The fp16-image rasterizer (FGS16, fastgs_ours_fp16/kernels_backward.cuh:
// 93-405) runs the same chain on half 2D gradients: its records hold half
// values (as floats) and the opacity-logit gradient with (1 - opacity)
// already applied per bucket (:1380). Half mode (kHalf) sums the half fields
// exactly, as integers in units of 2^-24 (every finite half is a multiple),
// and rounds each sum to half once (half_of_fixed); infinities and NaNs are
// tracked apart. The reference adds them with half2 atomics, whose rounding
// depends on the order the buckets finish in; the exact sum is the same for
// every order. The opacity gradient is summed in double and rounded to float.
//
// Only primitives that some tile's blend backward reached (a nonzero record
// count) run the chain; for the other visible ones every gradient is exactly
// zero, so their parameters are never read (at 1M Gaussians most visible
// primitives sit behind others and fall in this class). SH-rest parameter
// rows are read per thread, and only for primitives with gradients.
#include "common.h"
#include "halfmath.h"
#include "kernels.h"

namespace tgs {

// Gradients of one primitive's parameters (all but SH-rest).
struct PrimGrad {
    float m[3], s[3], sh0[3], r[4], o;
    float dc[3];   // dL/dmean in camera space (the pose gradient's factor)
};

// Per-primitive part: everything except the SH-rest gradient write, which the
// block performs cooperatively from k[] (basis values) and gc[] (dL/dcolour).
// The primitive's parameters come in registers: mean pm, log-scale ps,
// quaternion pq, SH-rest coefficients shr (45, used up to the active
// bases) and opacity.
__device__ __forceinline__ void preprocess_backward_one(
    int64_t i, const float pm[3], const float ps[3], const float pq[4], const float shr[45], float opacity,
    int bases, const CamParams& cam, const float4 gA, const float4 gB, const float4 gC,
    float4* __restrict__ densif, PrimGrad& out, float gc_out[3], float k[15], int& nb_out) {
    // gA: dmx, dmy, absx, absy; gB: dca, dcb, dcc, dr; gC: dg, db, alpha partial, -
    const float mx = pm[0], my = pm[1], mz = pm[2];

    // ---- SH backward (kernels_backward.cuh:22-86)
    const float gc[3] = {gB.w, gC.x, gC.y};
    for (int c = 0; c < 3; ++c) gc_out[c] = gc[c];
    for (int c = 0; c < 3; ++c) out.sh0[c] = 0.28209479177387814f * gc[c];
    float dmc0 = 0.f, dmc1 = 0.f, dmc2 = 0.f;
    nb_out = 0;
    if (bases > 1) {
        const float xr = mx - cam.cam_pos[0], yr = my - cam.cam_pos[1], zr = mz - cam.cam_pos[2];
        const float inv = 1.0f / __builtin_sqrtf(xr * xr + yr * yr + zr * zr);
        const float x = xr * inv, y = yr * inv, z = zr * inv;
        float gdx[3], gdy[3], gdz[3];
        k[0] = -0.48860251190291987f * y;
        k[1] = 0.48860251190291987f * z;
        k[2] = -0.48860251190291987f * x;
        int nb = 3;
        for (int c = 0; c < 3; ++c) {
            gdx[c] = -0.48860251190291987f * shr[3 * 2 + c];
            gdy[c] = -0.48860251190291987f * shr[3 * 0 + c];
            gdz[c] = 0.48860251190291987f * shr[3 * 1 + c];
        }
        if (bases > 4) {
            const float xx = x * x, yy = y * y, zz = z * z;
            const float xy = x * y, xz = x * z, yz = y * z;
            k[3] = 1.0925484305920792f * xy;
            k[4] = -1.0925484305920792f * yz;
            k[5] = 0.94617469575755997f * zz - 0.31539156525251999f;
            k[6] = -1.0925484305920792f * xz;
            k[7] = 0.54627421529603959f * xx - 0.54627421529603959f * yy;
            nb = 8;
            const float f7x = (float)(1.0925484305920792 * (double)x);
            const float f7y = (float)(-1.0925484305920792 * (double)y);
            const float f5z = (float)(1.8923493915151202 * (double)z);
            for (int c = 0; c < 3; ++c) {
                const float s3 = shr[9 + c], s4 = shr[12 + c];
                const float s5 = shr[15 + c], s6 = shr[18 + c];
                const float s7 = shr[21 + c];
                gdx[c] = gdx[c] + (1.0925484305920792f * y) * s3 + (-1.0925484305920792f * z) * s6 + f7x * s7;
                gdy[c] = gdy[c] + (1.0925484305920792f * x) * s3 + (-1.0925484305920792f * z) * s4 + f7y * s7;
                gdz[c] = gdz[c] + (-1.0925484305920792f * y) * s4 + f5z * s5 + (-1.0925484305920792f * x) * s6;
            }
            if (bases > 9) {
                k[8] = 0.59004358992664352f * y * (-3.0f * xx + yy);
                k[9] = 2.8906114426405538f * xy * z;
                k[10] = 0.45704579946446572f * y * (1.0f - 5.0f * zz);
                k[11] = 0.3731763325901154f * z * (5.0f * zz - 3.0f);
                k[12] = 0.45704579946446572f * x * (1.0f - 5.0f * zz);
                k[13] = 1.4453057213202769f * z * (xx - yy);
                k[14] = 0.59004358992664352f * x * (-xx + 3.0f * yy);
                nb = 15;
                for (int c = 0; c < 3; ++c) {
                    const float s8 = shr[24 + c], s9 = shr[27 + c];
                    const float s10 = shr[30 + c], s11 = shr[33 + c];
                    const float s12 = shr[36 + c], s13 = shr[39 + c];
                    const float s14 = shr[42 + c];
                    gdx[c] = gdx[c] + (-3.5402615395598609f * xy) * s8 + (2.8906114426405538f * yz) * s9 +
                             (0.45704579946446572f - 2.2852289973223288f * zz) * s12 +
                             (2.8906114426405538f * xz) * s13 +
                             (-1.7701307697799304f * xx + 1.7701307697799304f * yy) * s14;
                    gdy[c] = gdy[c] + (-1.7701307697799304f * xx + 1.7701307697799304f * yy) * s8 +
                             (2.8906114426405538f * xz) * s9 +
                             (0.45704579946446572f - 2.2852289973223288f * zz) * s10 +
                             (-2.8906114426405538f * yz) * s13 + (3.5402615395598609f * xy) * s14;
                    gdz[c] = gdz[c] + (2.8906114426405538f * xy) * s9 + (-4.5704579946446566f * yz) * s10 +
                             (5.597644988851731f * zz - 1.1195289977703462f) * s11 +
                             (-4.5704579946446566f * xz) * s12 +
                             (1.4453057213202769f * xx - 1.4453057213202769f * yy) * s13;
                }
            }
        }
        nb_out = nb;
        const float gx = gdx[0] * gc[0] + gdx[1] * gc[1] + gdx[2] * gc[2];
        const float gy = gdy[0] * gc[0] + gdy[1] * gc[1] + gdy[2] * gc[2];
        const float gz = gdz[0] * gc[0] + gdz[1] * gc[1] + gdz[2] * gc[2];
        const float xx_ = xr * xr, yy_ = yr * yr, zz_ = zr * zr;
        const float xy_ = xr * yr, xz_ = xr * zr, yz_ = yr * zr;
        const float nsq = xx_ + yy_ + zz_;
        const float sc = 1.0f / __builtin_sqrtf(nsq * nsq * nsq);
        dmc0 = ((yy_ + zz_) * gx - xy_ * gy - xz_ * gz) * sc;
        dmc1 = (-xy_ * gx + (xx_ + zz_) * gy - yz_ * gz) * sc;
        dmc2 = (-xz_ * gx - yz_ * gy + (xx_ + yy_) * gz) * sc;
    }

    // ---- projection / covariance backward (kernels_backward.cuh:132-336)
    const float* r1 = cam.r1;
    const float* r2 = cam.r2;
    const float* r3 = cam.r3;
    const float depth = r3[0] * mx + r3[1] * my + r3[2] * mz + r3[3];
    const float x = (r1[0] * mx + r1[1] * my + r1[2] * mz + r1[3]) / depth;
    const float y = (r2[0] * mx + r2[1] * my + r2[2] * mz + r2[3]) / depth;
    const float e0 = det_expf(ps[0]), e1 = det_expf(ps[1]), e2 = det_expf(ps[2]);
    const float vx = e0 * e0, vy = e1 * e1, vz = e2 * e2;
    const float qr = pq[0], qx = pq[1], qy = pq[2], qz = pq[3];
    const float qrr = qr * qr, qxx_r = qx * qx, qyy_r = qy * qy, qzz_r = qz * qz;
    const float qn = qrr + qxx_r + qyy_r + qzz_r;
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
    const float clip_left = cam.clip_left, clip_right = cam.clip_right;
    const float clip_top = cam.clip_top, clip_bottom = cam.clip_bottom;
    const float tx = __builtin_fmaxf(clip_left, __builtin_fminf(x, clip_right));
    const float ty = __builtin_fmaxf(clip_top, __builtin_fminf(y, clip_bottom));
    const float j11 = cam.fx / depth, j13 = -j11 * tx, j22 = cam.fy / depth, j23 = -j22 * ty;
    const float jw1x = j11 * r1[0] + j13 * r3[0], jw1y = j11 * r1[1] + j13 * r3[1], jw1z = j11 * r1[2] + j13 * r3[2];
    const float jw2x = j22 * r2[0] + j23 * r3[0], jw2y = j22 * r2[1] + j23 * r3[1], jw2z = j22 * r2[2] + j23 * r3[2];
    const float a1x = jw1x * c11 + jw1y * c12 + jw1z * c13;
    const float a1y = jw1x * c12 + jw1y * c22 + jw1z * c23;
    const float a1z = jw1x * c13 + jw1y * c23 + jw1z * c33;
    const float a2x = jw2x * c11 + jw2y * c12 + jw2z * c13;
    const float a2y = jw2x * c12 + jw2y * c22 + jw2z * c23;
    const float a2z = jw2x * c13 + jw2y * c23 + jw2z * c33;
    const float a = (a1x * jw1x + a1y * jw1y + a1z * jw1z) + kDilation;
    const float b = a1x * jw2x + a1y * jw2y + a1z * jw2z;
    const float c = (a2x * jw2x + a2y * jw2y + a2z * jw2z) + kDilation;
    const float aa = a * a, bb = b * b, cc_ = c * c;
    const float ac = a * c, ab = a * b, bc = b * c;
    const float det = ac - bb;
    const float drcp = 1.0f / (det + 1e-8f);
    const float drcp2 = drcp * drcp;
    const float gca = gB.x, gcb = gB.y, gcc = gB.z;
    const float dca = drcp2 * (2.0f * bc * gcb - cc_ * gca - bb * gcc);
    const float dcb = drcp2 * (bc * gca - (ac + bb) * gcb + ab * gcc);
    const float dcc = drcp2 * (2.0f * ab * gcb - bb * gca - aa * gcc);
    const float d11 = (jw1x * jw1x) * dca + 2.0f * (jw1x * jw2x) * dcb + (jw2x * jw2x) * dcc;
    const float d12 = (jw1x * jw1y) * dca + (jw1x * jw2y + jw1y * jw2x) * dcb + (jw2x * jw2y) * dcc;
    const float d13 = (jw1x * jw1z) * dca + (jw1x * jw2z + jw1z * jw2x) * dcb + (jw2x * jw2z) * dcc;
    const float d22 = (jw1y * jw1y) * dca + 2.0f * (jw1y * jw2y) * dcb + (jw2y * jw2y) * dcc;
    const float d23 = (jw1y * jw1z) * dca + (jw1y * jw2z + jw1z * jw2y) * dcb + (jw2y * jw2z) * dcc;
    const float d33 = (jw1z * jw1z) * dca + 2.0f * (jw1z * jw2z) * dcb + (jw2z * jw2z) * dcc;
    const float dj1x = 2.0f * (a1x * dca + a2x * dcb), dj1y = 2.0f * (a1y * dca + a2y * dcb),
                dj1z = 2.0f * (a1z * dca + a2z * dcb);
    const float dj2x = 2.0f * (a1x * dcb + a2x * dcc), dj2y = 2.0f * (a1y * dcb + a2y * dcc),
                dj2z = 2.0f * (a1z * dcb + a2z * dcc);
    const float dL_dj11 = r1[0] * dj1x + r1[1] * dj1y + r1[2] * dj1z;
    const float dL_dj22 = r2[0] * dj2x + r2[1] * dj2y + r2[2] * dj2z;
    const float dL_dj13 = r3[0] * dj1x + r3[1] * dj1y + r3[2] * dj1z;
    const float dL_dj23 = r3[0] * dj2x + r3[1] * dj2y + r3[2] * dj2z;
    const float mask_x = (x > clip_left && x < clip_right) ? 1.0f : 0.0f;
    const float mask_y = (y > clip_top && y < clip_bottom) ? 1.0f : 0.0f;
    const float dj13c = dL_dj13 * mask_x, dj23c = dL_dj23 * mask_y;
    const float h1 = dL_dj11 - 2.0f * tx * dj13c;
    const float h2 = dL_dj22 - 2.0f * ty * dj23c;
    const float gm2x = gA.x, gm2y = gA.y;
    const float dcx = j11 * (gm2x - dj13c / depth);
    const float dcy = j22 * (gm2y - dj23c / depth);
    const float dcz = -j11 * (x * gm2x + h1 / depth) - j22 * (y * gm2y + h2 / depth);
    out.dc[0] = dcx;
    out.dc[1] = dcy;
    out.dc[2] = dcz;
    const float gmx = r1[0] * dcx + r2[0] * dcy + r3[0] * dcz;
    const float gmy = r1[1] * dcx + r2[1] * dcy + r3[1] * dcz;
    const float gmz = r1[2] * dcx + r2[2] * dcy + r3[2] * dcz;
    out.m[0] = (gmx + dmc0);
    out.m[1] = (gmy + dmc1);
    out.m[2] = (gmz + dmc2);
    const float dvx = R11 * R11 * d11 + R21 * R21 * d22 + R31 * R31 * d33 +
                      2.0f * (R11 * R21 * d12 + R11 * R31 * d13 + R21 * R31 * d23);
    const float dvy = R12 * R12 * d11 + R22 * R22 * d22 + R32 * R32 * d33 +
                      2.0f * (R12 * R22 * d12 + R12 * R32 * d13 + R22 * R32 * d23);
    const float dvz = R13 * R13 * d11 + R23 * R23 * d22 + R33 * R33 * d33 +
                      2.0f * (R13 * R23 * d12 + R13 * R33 * d13 + R23 * R33 * d23);
    out.s[0] = (2.0f * e0 * e0 * dvx);
    out.s[1] = (2.0f * e1 * e1 * dvy);
    out.s[2] = (2.0f * e2 * e2 * dvz);
    const float D11 = 2.0f * (S11 * d11 + S21 * d12 + S31 * d13);
    const float D12 = 2.0f * (S12 * d11 + S22 * d12 + S32 * d13);
    const float D13 = 2.0f * (S13 * d11 + S23 * d12 + S33 * d13);
    const float D21 = 2.0f * (S11 * d12 + S21 * d22 + S31 * d23);
    const float D22 = 2.0f * (S12 * d12 + S22 * d22 + S32 * d23);
    const float D23 = 2.0f * (S13 * d12 + S23 * d22 + S33 * d23);
    const float D31 = 2.0f * (S11 * d13 + S21 * d23 + S31 * d33);
    const float D32 = 2.0f * (S12 * d13 + S22 * d23 + S32 * d33);
    const float D33 = 2.0f * (S13 * d13 + S23 * d23 + S33 * d33);
    const float gqxx = -D22 - D33, gqyy = -D11 - D33, gqzz = -D11 - D22;
    const float gqxy = D12 + D21, gqxz = D13 + D31, gqyz = D23 + D32;
    const float gqrx = D32 - D23, gqry = D13 - D31, gqrz = D21 - D12;
    const float hlp = qxx * gqxx + qyy * gqyy + qzz * gqzz + qxy * gqxy + qxz * gqxz + qyz * gqyz + qrx * gqrx +
                      qry * gqry + qrz * gqrz;
    const float den = qn * __builtin_sqrtf(qn);
    out.r[0] = (2.0f * (qx * gqrx + qy * gqry + qz * gqrz - qr * hlp) / den);
    out.r[1] = (2.0f * (2.0f * qx * gqxx + qy * gqxy + qz * gqxz + qr * gqrx - qx * hlp) / den);
    out.r[2] = (2.0f * (2.0f * qy * gqyy + qx * gqxy + qz * gqyz + qr * gqry - qy * hlp) / den);
    out.r[3] = (2.0f * (2.0f * qz * gqzz + qx * gqxz + qy * gqyz + qr * gqrz - qz * hlp) / den);
    out.o = (gC.z * (1.0f - opacity));
    if (densif) {
        float4 d = densif[i];
        d.x += 1.0f;
        const float ux = gm2x * (0.5f * cam.w), uy = gm2y * (0.5f * cam.h);
        d.y += __builtin_sqrtf(ux * ux + uy * uy);
        const float wx = gA.z * (0.5f * cam.w), wy = gA.w * (0.5f * cam.h);
        d.z += __builtin_sqrtf(wx * wx + wy * wy);
        densif[i] = d;
    }
}

// ---- exact sums of half records (half mode)
//
// Every record field is a half: a multiple of 2^-24 below 2^16 in magnitude.
// A double sum of up to 8192 of them is therefore exact (its magnitude stays
// below 2^29), and infinities and NaNs propagate as IEEE sums do (+inf and
// -inf give NaN). The exact sum is rounded to half once (half_of_double_sum:
// through float rounded toward odd; rounding to nearest float first would
// round twice). Heavy primitives with more records (only grids of more than
// 8192 tiles) take the integer sums below.
struct HalfSumsD {
    double s[10];
    double op;
};

__device__ __forceinline__ void hsd_zero(HalfSumsD& h) {
#pragma unroll
    for (int q = 0; q < 10; ++q) h.s[q] = 0.0;
    h.op = 0.0;
}

__device__ __forceinline__ void hsd_add(HalfSumsD& h, const float4& a, const float4& b, const float4& c) {
    const float v[10] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w, c.x, c.y};
#pragma unroll
    for (int q = 0; q < 10; ++q) h.s[q] += (double)v[q];
    h.op += (double)c.z;
}

__device__ __forceinline__ float hsd_value(double s) { return half_of_double_sum(s); }

__device__ __forceinline__ void hsd_result(const HalfSumsD& h, float4& gA, float4& gB, float4& gC) {
    gA = make_float4(hsd_value(h.s[0]), hsd_value(h.s[1]), hsd_value(h.s[2]), hsd_value(h.s[3]));
    gB = make_float4(hsd_value(h.s[4]), hsd_value(h.s[5]), hsd_value(h.s[6]), hsd_value(h.s[7]));
    gC = make_float4(hsd_value(h.s[8]), hsd_value(h.s[9]), (float)h.op, 0.f);
}

constexpr uint32_t kHalfDoubleRecords = 8192;   // exact double sums up to this many records

struct HalfSums {
    int64_t s[10];
    uint32_t fl;   // per field q, bits 3q..3q+2: +inf, -inf, NaN seen
    double op;
};

__device__ __forceinline__ void hs_zero(HalfSums& h) {
#pragma unroll
    for (int q = 0; q < 10; ++q) h.s[q] = 0;
    h.fl = 0u;
    h.op = 0.0;
}

__device__ __forceinline__ void hs_add(HalfSums& h, const float4& a, const float4& b, const float4& c) {
    const float v[10] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w, c.x, c.y};
#pragma unroll
    for (int q = 0; q < 10; ++q) {
        const float x = v[q];
        if (x != x)
            h.fl |= 4u << (3 * q);
        else if (__builtin_isinf(x))
            h.fl |= (x > 0.f ? 1u : 2u) << (3 * q);
        else
            h.s[q] += (int64_t)(x * 16777216.0f);   // exact: a half times 2^24 is an integer below 2^40
    }
    h.op += (double)c.z;
}

__device__ __forceinline__ float hs_value(const HalfSums& h, int q) {
    const uint32_t f = (h.fl >> (3 * q)) & 7u;
    if ((f & 4u) || f == 3u) return __builtin_nanf("");
    if (f & 1u) return __builtin_inff();
    if (f & 2u) return -__builtin_inff();
    return half_of_fixed(h.s[q]);
}

__device__ __forceinline__ void hs_result(const HalfSums& h, float4& gA, float4& gB, float4& gC) {
    gA = make_float4(hs_value(h, 0), hs_value(h, 1), hs_value(h, 2), hs_value(h, 3));
    gB = make_float4(hs_value(h, 4), hs_value(h, 5), hs_value(h, 6), hs_value(h, 7));
    gC = make_float4(hs_value(h, 8), hs_value(h, 9), (float)h.op, 0.f);
}

// One workgroup per chunk of 2048 primitives runs three phases (one launch;
// the chunk's lists and heavy sums never leave the workgroup's own slices, so
// the phases only need workgroup barriers). Chunk c holds the 64-primitive
// units c, c + C, ..., c + 15 C (C chunks), one wave per unit and round:
// spread over the whole index range, so every chunk gets a similar share of
// the primitives that received a gradient even when the index order is
// spatial (after Morton reordering the visible primitives are a few
// contiguous index runs: contiguous chunks of 2048 took 0.05 -> 0.51 ms).
//
// ---- phase 1: classify every primitive, list the live ones
//
// kClassRounds rounds, one 64-primitive unit per wave and round. A
// primitive is live when some bucket of the blend
// backward left a record for it (the counters of all others are zero). Dead
// visible primitives only count for densification (kernels_backward.cuh:345
// adds zero sums); sparse mode records the row mask; assign mode zeroes
// every gradient row of the chunk (the live rows are overwritten by phase
// 3). The chunk's live primitives and its heavy ones (more than
// kLightRecords records) are listed in the chunk's own slice of the two
// lists: no device-wide counter (returning atomics on one address
// serialise, about 10 ns each on MI355X). Entries: fp32 images, live
// (index, min(count, kLightRecords + 1) | span << 5, first slot, mask word of
// ranks 0..31) and heavy (index, first slot + span, first slot, mask word);
// fp16 images (index, count, first slot, 0) in both lists.
constexpr int kClassRounds = 4;
constexpr int kClassChunk = 256 * kClassRounds;

int64_t pb_chunks(int64_t n) { return n > 0 ? (n + kClassChunk - 1) / kClassChunk : 0; }

// Zeroes dst[0, n) with the lanes of one wave.
__device__ __forceinline__ void zero_run(float* __restrict__ dst, int64_t n) {
    // the arrays are 16-byte aligned and a run starts at a multiple of 64
    // rows, so the run is too
    const int64_t nv = n >> 2, lane = threadIdx.x & 63u;
    for (int64_t v = lane; v < nv; v += 64) ((float4*)dst)[v] = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int64_t e = (nv << 2) + lane; e < n; e += 64) dst[e] = 0.f;
}

template <bool kHalf>
__device__ __forceinline__ void classify_chunk(int64_t n, const uint32_t* __restrict__ rec_count,
                                               const uint32_t* __restrict__ rec_mask,
                                               const uint32_t* __restrict__ first_slot, const uint32_t* n_touched,
                                               float4* __restrict__ densif, int mode, uint8_t* __restrict__ row_mask,
                                               const GradView& out, uint4* __restrict__ live,
                                               uint4* __restrict__ heavy, uint32_t slot_limit, uint32_t* s_rw,
                                               uint32_t& n_live,
                                               uint32_t& n_heavy) {
    const uint32_t t = threadIdx.x;
    const int64_t c0 = (int64_t)blockIdx.x * kClassChunk;   // the chunk's slice of the lists
    // round r, wave v: unit blockIdx.x + (4 r + v) gridDim.x of 64 primitives
    auto unit = [&](int r) { return (int64_t)blockIdx.x + (int64_t)(4 * r + (int)(t >> 6)) * gridDim.x; };
    auto prim = [&](int r) { return unit(r) * 64 + (t & 63u); };
    uint32_t nrec[kClassRounds], msk[kClassRounds], lv[kClassRounds], hv[kClassRounds], ex[kClassRounds],
        exh[kClassRounds];
#pragma unroll
    for (int r = 0; r < kClassRounds; ++r) {
        const int64_t i = prim(r);
        nrec[r] = i < n ? rec_count[i] : 0u;
        msk[r] = !kHalf && i < n ? rec_mask[i] : 0u;
        lv[r] = nrec[r] ? 1u : 0u;
        hv[r] = nrec[r] > kLightRecords ? 1u : 0u;
    }
    // first slots of the live primitives, tile counts of the fp32 live ones
    // (their entries carry the span of their slots) and, for densification,
    // of the dead ones: all loads issued together
    uint32_t fsr[kClassRounds], ntr[kClassRounds];
#pragma unroll
    for (int r = 0; r < kClassRounds; ++r) {
        const int64_t i = prim(r);
        fsr[r] = lv[r] ? first_slot[i] : 0u;
        ntr[r] = i < n && ((!kHalf && lv[r]) || (densif && !nrec[r])) ? n_touched[i] : 0u;
    }
    if (densif) {
#pragma unroll
        for (int r = 0; r < kClassRounds; ++r) {
            const int64_t i = prim(r);
            if (i < n && !nrec[r] && ntr[r] != 0u) densif[i].x += 1.0f;
        }
    }
    if (mode == kGradSparse) {
#pragma unroll
        for (int r = 0; r < kClassRounds; ++r) {
            const int64_t i = prim(r);
            if (i < n) row_mask[i] = (uint8_t)lv[r];
        }
    }
    if (mode == kGradAssign) {   // each wave zeroes the rows of its units
        for (int r = 0; r < kClassRounds; ++r) {
            const int64_t r0 = unit(r) * 64;
            if (r0 >= n) break;
            const int64_t rows = min((int64_t)64, n - r0);
            zero_run(out.means + 3 * r0, 3 * rows);
            zero_run(out.scales + 3 * r0, 3 * rows);
            zero_run(out.rotations + 4 * r0, 4 * rows);
            zero_run(out.opacities + r0, rows);
            zero_run(out.sh0 + 3 * r0, 3 * rows);
            zero_run(out.sh_rest + 45 * r0, 45 * rows);
        }
    }
    striped_scan_u32<kClassRounds>(lv, ex, &n_live, s_rw);
    striped_scan_u32<kClassRounds>(hv, exh, &n_heavy, s_rw);
#pragma unroll
    for (int r = 0; r < kClassRounds; ++r) {
        const uint32_t i = (uint32_t)prim(r);
        if (lv[r]) {
            const uint32_t fs = fsr[r];
            if constexpr (kHalf) {
                const uint4 entry = make_uint4(i, nrec[r], fs, 0u);
                live[c0 + ex[r]] = entry;
                if (hv[r]) heavy[c0 + exh[r]] = entry;
            } else {
                // the slots that can hold its records: [fs, fs + n_touched),
                // cut at the instance capacity (a no-sync forward that outgrew
                // it emitted no slot past it); spans are at most 65,536
                const uint32_t span = fs < slot_limit ? min(ntr[r], slot_limit - fs) : 0u;
                live[c0 + ex[r]] = make_uint4(i, min(nrec[r], kLightRecords + 1u) | (span << 5), fs, msk[r]);
                if (hv[r]) heavy[c0 + exh[r]] = make_uint4(i, fs + span, fs, msk[r]);
            }
        }
    }
}

// Adds the records at the slots of the (up to) four lowest set bits of m
// (bit i: slot base + off(i); off increasing) into v, in bit order, and
// clears those bits; m must not be zero. The four loads are issued
// unconditionally (a missing record re-reads the first one) so that they are
// all in flight together; a record's adds are skipped when it is missing
// (adding zero would turn a -0 sum into +0).
template <typename Off>
__device__ __forceinline__ void add_records4(const float4* __restrict__ records, uint32_t base, uint32_t& m,
                                             float v[12], Off off) {
    uint32_t sl[4];
    bool on[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        on[u] = m != 0u;
        sl[u] = on[u] ? base + off((uint32_t)__builtin_ctz(m)) : sl[0];
        m &= m - 1u;   // (0 stays 0)
    }
    float4 a[4], b[4], d[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const float4* src = records + 3 * (size_t)sl[u];
        a[u] = src[0];
        b[u] = src[1];
        d[u] = src[2];
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
        if (on[u]) {
            v[0] += a[u].x; v[1] += a[u].y; v[2] += a[u].z; v[3] += a[u].w;
            v[4] += b[u].x; v[5] += b[u].y; v[6] += b[u].z; v[7] += b[u].w;
            v[8] += d[u].x; v[9] += d[u].y; v[10] += d[u].z; v[11] += d[u].w;
        }
}
struct SlotBit {   // bit i of a mask over consecutive slots
    __device__ uint32_t operator()(uint32_t i) const { return i; }
};
struct SlotByteStride {   // bit 8 q + i of four slot bytes 16 apart: slot 128 q + i
    __device__ uint32_t operator()(uint32_t i) const { return ((i >> 3) << 7) + (i & 7u); }
};

// Sums, in rank order, the records of the nr (at most 16) marked slots of a
// primitive with marked-slot span [fs, fs + span) into v: ranks below 32
// from its mask word m (slot fs + rank), the others (primitives over more
// than 32 tiles only) from rec_bits over [fs + 32, fs + span).
__device__ __forceinline__ void add_marked_light(const uint32_t* __restrict__ rec_bits,
                                                 const float4* __restrict__ records, uint32_t fs, uint32_t m,
                                                 uint32_t nr, uint32_t span, float v[12]) {
    uint32_t taken = (uint32_t)__builtin_popcount(m);
    const uint32_t a = fs + 32u, e = fs + span;
    const bool more = taken < nr && a < e;
    // slot words over [a, e), four loaded at a time (the first four before
    // the mask ranks' records), until all nr are found
    const uint32_t first = a >> 5, last = more ? (e - 1u) >> 5 : 0u;
    const uint32_t head = ~0u << (a & 31u), tail = (e & 31u) ? (1u << (e & 31u)) - 1u : ~0u;
    uint32_t mw[4];
    auto load4 = [&](uint32_t w0) {
#pragma unroll
        for (uint32_t q = 0; q < 4u; ++q) mw[q] = more && w0 + q <= last ? rec_bits[w0 + q] : 0u;
    };
    load4(first);
    while (m) add_records4(records, fs, m, v, SlotBit{});
    for (uint32_t w0 = first; more && w0 <= last && taken < nr;) {
#pragma unroll
        for (uint32_t q = 0; q < 4u; ++q) {
            const uint32_t w = w0 + q;
            if (w == first) mw[q] &= head;
            if (w == last) mw[q] &= tail;
            taken += (uint32_t)__builtin_popcount(mw[q]);
            while (mw[q]) add_records4(records, w << 5, mw[q], v, SlotBit{});
        }
        w0 += 4u;
        if (w0 <= last && taken < nr) load4(w0);
    }
}

// ---- phase 2: 2D-gradient sums of the heavy primitives
//
// Sixteen lanes (one DPP row) per heavy primitive of the chunk, four per
// wave. fp32 images: the record of rank k (slot fs + k) goes to lane k mod 16
// for k < 32, and otherwise to lane (b - b_first) mod 16, where b = (fs + k)
// / 8 is its 8-slot byte of the slot bits and b_first = (fs + 32) / 8; each
// lane adds its records in rank order, and an xor butterfly (partners 8, 4,
// 2, 1) then leaves the same 12 sums in every lane: a fixed order, whatever
// order the buckets finished in. Lane l reads mask bits l and l + 16 and
// slot bytes b_first + l + 16 q, four bytes and four records at a time.
// fp16 images: the lanes stride over the packed records with exact sums.
// Lanes 0-2 of the row store the sums to grad2d[12 p] in record layout.
template <bool kHalf>
__device__ __forceinline__ void gather_heavy_chunk(const uint4* __restrict__ list, uint32_t nh,
                                                   const float4* __restrict__ records,
                                                   const uint32_t* __restrict__ rec_bits,
                                                   float* __restrict__ grad2d) {
    const uint32_t row = threadIdx.x >> 4, sub = threadIdx.x & 15u;
    for (uint32_t h0 = 0; h0 < nh; h0 += 16u) {
        const uint32_t h = h0 + row;
        const bool on = h < nh;
        const uint4 e = on ? list[h] : make_uint4(0u, 0u, 0u, 0u);
        if constexpr (kHalf) {
            if (e.y <= kHalfDoubleRecords) {   // (row-uniform)
                HalfSumsD hs;
                hsd_zero(hs);
                uint32_t r = sub;
                for (; r + 48u < e.y; r += 64u) {   // four strides' loads issued together (exact sums: any order)
                    float4 a[4], b[4], d[4];
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const float4* src = records + 3 * (size_t)(e.z + r + 16u * (uint32_t)u);
                        a[u] = src[0];
                        b[u] = src[1];
                        d[u] = src[2];
                    }
#pragma unroll
                    for (int u = 0; u < 4; ++u) hsd_add(hs, a[u], b[u], d[u]);
                }
                for (; r < e.y; r += 16u) {
                    const float4* src = records + 3 * (size_t)(e.z + r);
                    hsd_add(hs, src[0], src[1], src[2]);
                }
                for (int m = 8; m >= 1; m >>= 1) {
#pragma unroll
                    for (int q = 0; q < 10; ++q) hs.s[q] += __shfl_xor(hs.s[q], m, 16);
                    hs.op += __shfl_xor(hs.op, m, 16);
                }
                if (on && sub == 0u) {
                    float4 gA, gB, gC;
                    hsd_result(hs, gA, gB, gC);
                    float4* g = (float4*)(grad2d + (size_t)e.x * kGradStride);
                    g[0] = gA;
                    g[1] = gB;
                    g[2] = gC;
                }
                continue;
            }
            HalfSums hs;
            hs_zero(hs);
            uint32_t r = sub;
            for (; r + 48u < e.y; r += 64u) {   // four strides' loads issued together (exact sums: any order)
                float4 a[4], b[4], d[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const float4* src = records + 3 * (size_t)(e.z + r + 16u * (uint32_t)u);
                    a[u] = src[0];
                    b[u] = src[1];
                    d[u] = src[2];
                }
#pragma unroll
                for (int u = 0; u < 4; ++u) hs_add(hs, a[u], b[u], d[u]);
            }
            for (; r < e.y; r += 16u) {
                const float4* src = records + 3 * (size_t)(e.z + r);
                hs_add(hs, src[0], src[1], src[2]);
            }
            // exact integer sums and flag unions over the 16 lanes of the row
            for (int m = 8; m >= 1; m >>= 1) {
#pragma unroll
                for (int q = 0; q < 10; ++q) hs.s[q] += __shfl_xor(hs.s[q], m, 16);
                hs.fl |= (uint32_t)__shfl_xor((int)hs.fl, m, 16);
                hs.op += __shfl_xor(hs.op, m, 16);
            }
            if (on && sub == 0u) {
                float4 gA, gB, gC;
                hs_result(hs, gA, gB, gC);
                float4* g = (float4*)(grad2d + (size_t)e.x * kGradStride);
                g[0] = gA;
                g[1] = gB;
                g[2] = gC;
            }
            continue;
        }
        float v[12];
#pragma unroll
        for (int q = 0; q < 12; ++q) v[q] = 0.f;
        if (on) {
            // e.y: the end of the primitive's marked slots, e.z its first slot
            const uint32_t a0 = e.z + 32u;
            const bool wide = e.y > a0;
            const uint32_t bfirst = a0 >> 3, blast = wide ? (e.y - 1u) >> 3 : 0u;
            const uint32_t head = (0xffu << (a0 & 7u)) & 0xffu, tail = (e.y & 7u) ? (1u << (e.y & 7u)) - 1u : 0xffu;
            // bytes b0 + 16 q (q < 4) as one mask: bit 8 q + i is slot 8 (b0 + 16 q) + i
            // (the first four loaded before the mask ranks' records)
            uint32_t wd[4];
            auto load4 = [&](uint32_t b0) {
#pragma unroll
                for (uint32_t q = 0; q < 4u; ++q) {
                    const uint32_t bb = b0 + 16u * q;
                    wd[q] = wide && bb <= blast ? rec_bits[bb >> 2] : 0u;
                }
            };
            load4(bfirst + sub);
            uint32_t mm = ((e.w >> sub) & 1u) | (((e.w >> (sub + 16u)) & 1u) << 16);
            if (mm) add_records4(records, e.z + sub, mm, v, SlotBit{});   // ranks sub, sub + 16
            for (uint32_t b0 = bfirst + sub; wide && b0 <= blast;) {
                uint32_t m4 = 0;
#pragma unroll
                for (uint32_t q = 0; q < 4u; ++q) {
                    const uint32_t bb = b0 + 16u * q;
                    uint32_t byte = (wd[q] >> (8u * (bb & 3u))) & 0xffu;
                    if (bb == bfirst) byte &= head;
                    if (bb == blast) byte &= tail;
                    m4 |= byte << (8u * q);
                }
                const uint32_t base = b0 << 3;
                b0 += 64u;
                if (b0 <= blast) load4(b0);
                while (m4) add_records4(records, base, m4, v, SlotByteStride{});
            }
        }
        // a + b == b + a: both partners of each step hold the same sum after it
        for (int m = 8; m >= 1; m >>= 1)
#pragma unroll
            for (int q = 0; q < 12; ++q) v[q] += __shfl_xor(v[q], m, 16);
        if (on && sub < 3u) {
            float4* g = (float4*)(grad2d + (size_t)e.x * kGradStride);
            const float4 f = sub == 0u ? make_float4(v[0], v[1], v[2], v[3])
                             : sub == 1u ? make_float4(v[4], v[5], v[6], v[7])
                                         : make_float4(v[8], v[9], v[10], v[11]);
            g[sub] = f;
        }
    }
}

// ---- phase 3: the gradient chain, one thread per live primitive of the chunk
//
// Light primitives sum their (at most kLightRecords) records here, heavy ones
// read grad2d. The record counter is cleared for the next backward. Rows are
// scattered (live primitives are sparse), so every row access is one request
// per lane: the 90-byte fp16 SH-rest row is read as 8-byte pieces of its
// 8-byte-aligned window, realigned through the thread's LDS slot, and the
// 180-byte SH-rest gradient row is written as 8-byte pairs (which pairs
// depends on the row's 8-byte phase). Assign / sparse store the rows,
// accumulate adds to them; the SH-rest gradient row gets k_b * dL/dcolour_c
// for the active bases b (kernels_backward.cuh:41-65) and, when stored,
// zero for the others.
constexpr int kShWin = 13;   // 8-byte words per LDS slot (an odd word stride)

template <typename ShT>
__device__ __forceinline__ void load_sh_row(const ShT* __restrict__ shr_all, int64_t ip, int nsh, uint2* slot,
                                            float shv[45]) {
    const ShT* sr = shr_all + 45 * ip;
#pragma unroll
    for (int b = 0; b < 45; ++b) shv[b] = b < nsh ? load_as_float(sr, b) : 0.f;
}
template <>
__device__ __forceinline__ void load_sh_row<__half>(const __half* __restrict__ shr_all, int64_t ip, int nsh,
                                                    uint2* slot, float shv[45]) {
    // row bytes [B, B + 90), window [a, a + 96) with a = B & ~7, o = B - a in {0, 2, 4, 6}:
    // 11 whole 8-byte words lie inside the row; of the 12th, only its first o + 2 bytes do
    const uint64_t B = 90u * (uint64_t)ip, a = B & ~7ull;
    const uint32_t o = (uint32_t)(B - a);
    const uint2* win = (const uint2*)((const char*)shr_all + a);
#pragma unroll
    for (int q = 0; q < 11; ++q) slot[q] = win[q];
    const uint16_t* tail = (const uint16_t*)(win + 11);
    uint16_t* stail = (uint16_t*)(slot + 11);
#pragma unroll
    for (uint32_t q = 0; q < 4; ++q)
        if (2u * q <= o) stail[q] = tail[q];
    const __half* h = (const __half*)((const char*)slot + o);
#pragma unroll
    for (int b = 0; b < 45; ++b) shv[b] = b < nsh ? __half2float(h[b]) : 0.f;
}

// Pose gradient (kernels_backward.cuh:256-269): with kPose, each thread also
// sums dL/dmean_cam[k] * (mean, 1) over its primitives, and the workgroup's
// sum of those 12 numbers goes to pose_partial[12 * chunk] (every workgroup
// writes its slot, zero when it has no live primitive), in a fixed order.
template <typename ShT, bool kPose, bool kHalf>
__global__ void __launch_bounds__(256) preprocess_backward_chunk_kernel(
    int64_t n, const uint32_t* __restrict__ n_touched, const uint32_t* __restrict__ first_slot,
    uint8_t* __restrict__ row_mask, uint4* __restrict__ live, uint4* __restrict__ heavy,
    const float* __restrict__ means, const float* __restrict__ scales, const float* __restrict__ rots,
    const ShT* __restrict__ shr_all, int bases, CamParams cam, const float4* __restrict__ conic_opacity,
    uint32_t* __restrict__ rec_count, uint32_t* __restrict__ rec_mask, const uint32_t* __restrict__ rec_bits,
    uint32_t slot_limit, const float4* __restrict__ records, float* grad2d, GradView out,
    float4* __restrict__ densif, int mode, float* __restrict__ pose_partial, float* keep2d) {
    __shared__ uint32_t s_rw[4 * kClassRounds];
    __shared__ uint2 s_win[256 * kShWin];
    const uint32_t t = threadIdx.x;
    // phase 1: the chunk's lists; phase 2: its heavy primitives' sums into grad2d
    uint32_t nl, nh;
    classify_chunk<kHalf>(n, rec_count, rec_mask, first_slot, n_touched, densif, mode, row_mask, out, live, heavy,
                          slot_limit, s_rw, nl, nh);
    __syncthreads();   // the lists (global, this chunk's slices) seen by the whole workgroup
    if (nh) {
        gather_heavy_chunk<kHalf>(heavy + (size_t)blockIdx.x * kClassChunk, nh, records, rec_bits, grad2d);
        __syncthreads();   // grad2d rows of the heavy primitives
    }
    // phase 3
    float pacc[12];
#pragma unroll
    for (int q = 0; q < 12; ++q) pacc[q] = 0.f;
    const uint4* list = live + (size_t)blockIdx.x * kClassChunk;
    const bool store = mode != kGradAccumulate;
    const int nsh = 3 * (bases - 1);   // SH-rest coefficients of the active bases
    for (uint32_t g = t; g < nl; g += 256u) {
        const uint4 e = list[g];
        const int64_t ip = e.x;
        const uint32_t nr = kHalf ? e.y : e.y & 31u;   // (fp32: the count, capped at kLightRecords + 1)
        float4 gA = make_float4(0.f, 0.f, 0.f, 0.f), gB = gA, gC = gA;
        if (nr > kLightRecords) {
            const float* gr = grad2d + (size_t)ip * kGradStride;
            gA = *(const float4*)(gr);
            gB = *(const float4*)(gr + 4);
            gC = *(const float4*)(gr + 8);
        } else if constexpr (kHalf) {
            const float4* rec = records + 3 * (size_t)e.z;
            HalfSumsD hs;
            hsd_zero(hs);
            for (uint32_t r = 0; r < nr; ++r) hsd_add(hs, rec[3 * r], rec[3 * r + 1], rec[3 * r + 2]);
            hsd_result(hs, gA, gB, gC);
        } else {
            // the marked slots in slot (rank) order
            float v[12];
#pragma unroll
            for (int q = 0; q < 12; ++q) v[q] = 0.f;
            // (the thread's SH staging slot holds its slot list until the SH row is read)
            add_marked_light(rec_bits, records, e.z, e.w, nr, e.y >> 5, v);
            gA = make_float4(v[0], v[1], v[2], v[3]);
            gB = make_float4(v[4], v[5], v[6], v[7]);
            gC = make_float4(v[8], v[9], v[10], 0.f);
        }
        rec_count[ip] = 0u;
        if constexpr (!kHalf) rec_mask[ip] = 0u;
        if (keep2d) {   // the summed 2D gradients, for parity tests (heavy: already there)
            float4* k2 = (float4*)(keep2d + (size_t)ip * kGradStride);
            if (nr <= kLightRecords) {
                k2[0] = gA;
                k2[1] = gB;
            }
            // fp32: the 12th float carries the mask word of record ranks 0..31
            k2[2] = make_float4(gC.x, gC.y, gC.z, kHalf ? gC.w : u2f(e.w));
        }
        float pm[3], ps[3], pq[4], shv[45];
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            pm[c] = means[3 * ip + c];
            ps[c] = scales[3 * ip + c];
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) pq[c] = rots[4 * ip + c];
        // half mode: the records carry (1 - opacity) already
        const float opacity = kHalf ? 0.0f : conic_opacity[ip].w;
        load_sh_row<ShT>(shr_all, ip, nsh, s_win + kShWin * t, shv);
        PrimGrad pg;
        float gc[3], k[15];
        for (int b = 0; b < 15; ++b) k[b] = 0.f;
        int nb = 0;
        preprocess_backward_one(ip, pm, ps, pq, shv, opacity, bases, cam, gA, gB, gC, densif, pg, gc, k, nb);
        if constexpr (kPose) {
#pragma unroll
            for (int r = 0; r < 3; ++r) {
                pacc[4 * r] += pg.dc[r] * pm[0];
                pacc[4 * r + 1] += pg.dc[r] * pm[1];
                pacc[4 * r + 2] += pg.dc[r] * pm[2];
                pacc[4 * r + 3] += pg.dc[r];
            }
        }
        float* gm = out.means + 3 * ip;
        float* gs = out.scales + 3 * ip;
        float* gh = out.sh0 + 3 * ip;
        float* gq = out.rotations + 4 * ip;
        if (store) {
            for (int c = 0; c < 3; ++c) {
                gm[c] = pg.m[c];
                gs[c] = pg.s[c];
                gh[c] = pg.sh0[c];
            }
            for (int c = 0; c < 4; ++c) gq[c] = pg.r[c];
            out.opacities[ip] = pg.o;
        } else {
            for (int c = 0; c < 3; ++c) {
                gm[c] += pg.m[c];
                gs[c] += pg.s[c];
                gh[c] += pg.sh0[c];
            }
            for (int c = 0; c < 4; ++c) gq[c] += pg.r[c];
            out.opacities[ip] += pg.o;
        }
        float v[45];
#pragma unroll
        for (int b = 0; b < 15; ++b)
#pragma unroll
            for (int c = 0; c < 3; ++c) v[3 * b + c] = b < nb ? k[b] * gc[c] : 0.f;
        float* gr = out.sh_rest + 45 * ip;
        if (store) {
            // row bytes [R, R + 180): s = 1 when R is 4 mod 8; 8-byte pairs at R + 4 s + 8 j
            // hold elements (s + 2 j, s + 2 j + 1); the one element left over is 0 or 44
            const uint32_t s1 = (uint32_t)(ip & 1);   // 180 ip = 4 ip (mod 8)
            float2* pairs = (float2*)(gr + s1);
#pragma unroll
            for (int j = 0; j < 22; ++j)
                pairs[j] = s1 ? make_float2(v[2 * j + 1], v[2 * j + 2]) : make_float2(v[2 * j], v[2 * j + 1]);
            if (s1)
                gr[0] = v[0];
            else
                gr[44] = v[44];
        } else {
#pragma unroll
            for (int j = 0; j < 45; ++j)   // constant indices keep v in registers
                if (j < 3 * nb) gr[j] += v[j];
        }
    }
    if constexpr (kPose) {
        __shared__ float s_pose[4][12];
#pragma unroll
        for (int q = 0; q < 12; ++q) {
            float v = pacc[q];
            for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
            pacc[q] = v;
        }
        if ((t & 63u) == 0u)
            for (int q = 0; q < 12; ++q) s_pose[t >> 6][q] = pacc[q];
        __syncthreads();
        if (t < 12u)
            pose_partial[12 * (size_t)blockIdx.x + t] = ((s_pose[0][t] + s_pose[1][t]) + s_pose[2][t]) + s_pose[3][t];
    }
}

// Sum of the per-workgroup pose partials in a fixed order (thread j takes
// chunks j, j + 256, ...; then a fixed tree), written as the 4 x 4 dL/dw2c in
// column-major order ([4 c + r] = row r, column c) with row 3 zero, as the
// reference hands it to the caller (fastgs.cu:373-383: the device's row-major
// block transposed into glm).
__global__ void __launch_bounds__(256) pose_reduce_kernel(const float* __restrict__ partial, int64_t chunks,
                                                          float* __restrict__ out) {
    __shared__ float s_sum[4][12];
    const uint32_t t = threadIdx.x;
    float acc[12];
#pragma unroll
    for (int q = 0; q < 12; ++q) acc[q] = 0.f;
    for (int64_t c = t; c < chunks; c += 256)
#pragma unroll
        for (int q = 0; q < 12; ++q) acc[q] += partial[12 * c + q];
#pragma unroll
    for (int q = 0; q < 12; ++q) {
        float v = acc[q];
        for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
        acc[q] = v;
    }
    if ((t & 63u) == 0u)
        for (int q = 0; q < 12; ++q) s_sum[t >> 6][q] = acc[q];
    __syncthreads();
    if (t < 16u) {
        const uint32_t r = t & 3u, c = t >> 2;   // out[4 c + r]
        out[t] = r < 3u ? ((s_sum[0][4 * r + c] + s_sum[1][4 * r + c]) + s_sum[2][4 * r + c]) + s_sum[3][4 * r + c]
                        : 0.f;
    }
}

template <typename ShT, bool kPose>
static void launch_chunks(const GaussianView& g, int bases, const CamParams& cam, const uint32_t* n_touched,
                          const uint32_t* first_slot, uint8_t* row_mask, uint4* live, uint4* heavy,
                          const float4* conic_opacity, uint32_t* rec_count, uint32_t* rec_mask,
                          const uint32_t* rec_bits, uint32_t slot_limit, const float4* records, float* grad2d,
                          const GradView& out,
                          float* densif, int mode, float* pose_partial, bool keep2d, bool half_sums, unsigned chunks,
                          hipStream_t s) {
    if (half_sums)
        preprocess_backward_chunk_kernel<ShT, kPose, true><<<chunks, 256, 0, s>>>(
            g.n, n_touched, first_slot, row_mask, live, heavy, g.means, g.scales, g.rotations,
            (const ShT*)g.sh_rest, bases, cam, conic_opacity, rec_count, rec_mask, rec_bits, slot_limit, records, grad2d,
            out,
            (float4*)densif, mode, pose_partial, keep2d ? grad2d : nullptr);
    else
        preprocess_backward_chunk_kernel<ShT, kPose, false><<<chunks, 256, 0, s>>>(
            g.n, n_touched, first_slot, row_mask, live, heavy, g.means, g.scales, g.rotations,
            (const ShT*)g.sh_rest, bases, cam, conic_opacity, rec_count, rec_mask, rec_bits, slot_limit, records, grad2d,
            out,
            (float4*)densif, mode, pose_partial, keep2d ? grad2d : nullptr);
}

void launch_preprocess_backward(const GaussianView& g, const CamParams& cam, const uint32_t* n_touched,
                                const float4* conic_opacity, uint32_t* rec_count, uint32_t* rec_mask,
                                const uint32_t* rec_bits, int64_t slot_limit, const uint32_t* first_slot,
                                const float4* records, float* grad2d,
                                const GradView& out, float* densif, int mode, uint8_t* row_mask, uint4* live,
                                uint4* heavy, float* pose_partial, float* pose_out, bool keep2d, bool half_sums,
                                hipStream_t s) {
    if (g.n <= 0) {
        if (pose_out) launch_fill_u32((uint32_t*)pose_out, 0u, 16, s);
        return;
    }
    if (keep2d) launch_fill_u32((uint32_t*)grad2d, 0u, (int64_t)kGradStride * g.n, s);
    const int bases = (g.sh_degree + 1) * (g.sh_degree + 1);
    const unsigned chunks = (unsigned)pb_chunks(g.n);
    const bool f16 = g.sh_dtype == kShF16;
    const uint32_t lim = (uint32_t)std::min<int64_t>(std::max<int64_t>(slot_limit, 0), 0xffffffffll);
    if (pose_out) {
        if (f16)
            launch_chunks<__half, true>(g, bases, cam, n_touched, first_slot, row_mask, live, heavy, conic_opacity,
                                        rec_count, rec_mask, rec_bits, lim, records, grad2d, out, densif, mode, pose_partial, keep2d,
                                        half_sums, chunks, s);
        else
            launch_chunks<float, true>(g, bases, cam, n_touched, first_slot, row_mask, live, heavy, conic_opacity,
                                       rec_count, rec_mask, rec_bits, lim, records, grad2d, out, densif, mode, pose_partial, keep2d,
                                       half_sums, chunks, s);
        pose_reduce_kernel<<<1, 256, 0, s>>>(pose_partial, (int64_t)chunks, pose_out);
    } else if (f16) {
        launch_chunks<__half, false>(g, bases, cam, n_touched, first_slot, row_mask, live, heavy, conic_opacity,
                                     rec_count, rec_mask, rec_bits, lim, records, grad2d, out, densif, mode, nullptr, keep2d,
                                     half_sums, chunks, s);
    } else {
        launch_chunks<float, false>(g, bases, cam, n_touched, first_slot, row_mask, live, heavy, conic_opacity,
                                    rec_count, rec_mask, rec_bits, lim, records, grad2d, out, densif, mode, nullptr, keep2d,
                                    half_sums, chunks, s);
    }
}

}  // namespace tgs
