// Device pieces of the fp16-image rasterizer (FGS16) shared by its
// preprocess and the instance emission: the half tile test and the record
// packing. Arithmetic is the canonical half arithmetic of halfmath.h, in the
// operation order of the oracle's orc_h_will_contribute.
#pragma once

#include "common.h"
#include "halfmath.h"

namespace tgs {

// will_primitive_contribute_half, tinygs/src/rasterizer/fastgs_ours_fp16/
// kernels_forward.cuh:125-170, on the mean shifted by -0.5.
__device__ __forceinline__ bool will_contribute_half(float mx, float my, h16 cx, h16 cy, h16 cz, uint32_t tile_x,
                                                     uint32_t tile_y, float power_threshold) {
    const h16 one = (h16)1.0f, zero = (h16)0.0f;
    const h16 tile_size = h_rd(15.0f / 16.0f);
    const h16 mdx = h_rd((float)tile_x - mx * (1.0f / 16.0f));
    const h16 mdy = h_rd((float)tile_y - my * (1.0f / 16.0f));
    const h16 Mdx = mdx + tile_size, Mdy = mdy + tile_size;
    // unordered comparisons (__hgtu2, __hltu2): 1 or 0
    const h16 xl = !(mdx <= zero) ? one : zero, ya = !(mdy <= zero) ? one : zero;
    const h16 xr = !(Mdx >= zero) ? one : zero, yb = !(Mdy >= zero) ? one : zero;
    const h16 nx = xl + xr, ny = ya + yb;
    if (nx == zero && ny == zero) return true;
    const h16 dx = hfrom((uint16_t)((hbits(tile_size) & 0x7fffu) | (hbits(mdx) & 0x8000u)));
    const h16 dy = hfrom((uint16_t)((hbits(tile_size) & 0x7fffu) | (hbits(mdy) & 0x8000u)));
    // diff = -lerp(max, min, t) = -fma(t, min, fma(-t, max, max))
    const h16 ex = -h_fma(xl, mdx, h_fma(-xl, Mdx, Mdx));
    const h16 ey = -h_fma(ya, mdy, h_fma(-ya, Mdy, Mdy));
    const h16 numx = ((dx * cx) * ex) + ((dx * cy) * ey);
    const h16 numy = ((dy * cy) * ex) + ((dy * cz) * ey);
    const h16 denx = (dx * dx) * cx, deny = (dy * dy) * cz;
    const h16 trx = h_div(numx, denx), trY = h_div(numy, deny);
    const h16 tx = h_sat(trx * ny), ty = h_sat(trY * nx);   // __hmul2_sat with the lanes swapped
    const float ddx = (float)(ex - tx * dx) * 16.0f;
    const float ddy = (float)(ey - ty * dy) * 16.0f;
    const float fx = (float)cx, fy = (float)cy, fz = (float)cz;
    const float max_power = 0.5f * (fx * ddx * ddx + fz * ddy * ddy) + fy * ddx * ddy;
    return max_power <= power_threshold;
}

}  // namespace tgs
