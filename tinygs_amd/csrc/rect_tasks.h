// Rect tiles of a wave's 64 primitives as one task list spread over the
// wave's lanes (the preprocess's exact tile count and the instance emission).
//
// Task t < sum of the rect sizes is rect tile t - ex[j] (row major in the
// rect) of lane j's primitive, ex the exclusive prefix of the rect sizes.
// Each window of 64 consecutive tasks runs one per lane, whatever the sizes,
// so neither large nor uneven small rects leave lanes idle. The owner j of a
// task is the last lane whose rect starts at or before it: every rect that
// starts inside the window marks its start position in LDS, and a prefix
// maximum over the window, carrying the previous window's last owner, spreads
// the marks. The owner's values then come over ds_bpermute.
#pragma once
#include "common.h"

namespace tgs {

__device__ __forceinline__ uint32_t wave_inclusive_max_u32(uint32_t v) {
    v = max(v, dpp_u32<0x111>(v));          // row_shr:1
    v = max(v, dpp_u32<0x112>(v));          // row_shr:2
    v = max(v, dpp_u32<0x114>(v));          // row_shr:4
    v = max(v, dpp_u32<0x118>(v));          // row_shr:8
    v = max(v, dpp_u32<0x142, 0xA>(v));     // row_bcast:15
    v = max(v, dpp_u32<0x143, 0xC>(v));     // row_bcast:31
    return v;
}

// lane j's value of v (every lane of the wave must execute the call)
__device__ __forceinline__ uint32_t lane_gather(uint32_t j, uint32_t v) {
    return (uint32_t)__builtin_amdgcn_ds_bpermute((int)(j << 2), (int)v);
}

// Owner lane of task base + lane. nrect, ex: this lane's rect size and
// exclusive prefix; s_mark: 64 words of this wave's LDS; carry: 1 + the
// owner of the previous window's last task (0 before the first window),
// updated for the next window. Called by the whole wave.
__device__ __forceinline__ uint32_t wave_task_owner(uint32_t* s_mark, uint32_t nrect, uint32_t ex, uint32_t base,
                                                    uint32_t& carry) {
    const uint32_t lane = lane_id();
    s_mark[lane] = 0u;
    wave_lds_sync();
    if (nrect > 0u && ex >= base && ex - base < (uint32_t)kWave) s_mark[ex - base] = lane + 1u;
    wave_lds_sync();
    const uint32_t j = max(wave_inclusive_max_u32(s_mark[lane]), carry) - 1u;
    carry = readlane_u32(j, 63) + 1u;
    return j;
}

// (column, row) of rect tile k in a rect of width w: k / w through a float
// reciprocal. k < 2^16 and w <= 2^16 (grids are at most 2^16 tiles) are exact
// floats, and the estimate is off by at most one, corrected once.
__device__ __forceinline__ void rect_tile_of(uint32_t k, uint32_t w, uint32_t& col, uint32_t& row) {
    uint32_t q = (uint32_t)((float)k * __builtin_amdgcn_rcpf((float)w));
    int32_t r = (int32_t)k - (int32_t)(q * w);
    if (r < 0) {
        --q;
        r += (int32_t)w;
    } else if (r >= (int32_t)w) {
        ++q;
        r -= (int32_t)w;
    }
    col = (uint32_t)r;
    row = q;
}

}  // namespace tgs
