// SimpleAdam: one fused launch over all six parameter groups.
// Follows tinygs/src/optim/simple_adam.cu:104-213 (per-scalar update) and
// :457-580 (six launches, per-group learning rates). The reference runs six
// kernels, four of them through a float4 view that can read and write up to
// three floats past the end of a vec3 array (:176,487); here a single launch
// walks the groups with exact bounds, every access coalesced (lane-strided
// vectors), 28 bytes of HBM traffic per fp32 scalar.
//
// Per-group specifics kept: the lerp form (fma(t, g - m, m) for the groups the
// reference runs through helper_math's float4 lerp, fma(t, g, fma(-t, m, m))
// for the scalar opacity kernel, simple_adam.cu:24-26), the optional L1 decay
// terms, and |g| clipping at max_grad_1. Groups may store theta as fp16 (SH
// storage mode); moments and gradients stay fp32.
#include "common.h"
#include "kernels.h"

namespace tgs {

// Non-temporal 16-byte access for the streams nothing reads again soon
// (gradients, moments): measured 0.245 -> 0.19 ms at 1M Gaussians. theta
// keeps ordinary accesses (the next forward reads it; non-temporal theta
// measured slower).
typedef float v4f __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 ntld(const float* p) {
    const v4f v = __builtin_nontemporal_load((const v4f*)p);
    return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void ntst(float* p, float4 a) {
    v4f v = {a.x, a.y, a.z, a.w};
    __builtin_nontemporal_store(v, (v4f*)p);
}

struct AdamLaunch {
    AdamArgs a;
    int64_t block_start[7];
};

constexpr int kAdamThreads = 256;
constexpr int kAdamVecPerThread = 2;                       // 4-element vectors per thread (2 beat 1, 4, 8)
constexpr int kAdamChunk = kAdamThreads * kAdamVecPerThread * 4;

__device__ __forceinline__ float adam_one(float th, float gr_raw, float& m, float& v, const AdamGroup& g,
                                          const AdamArgs& a, float t1, float t2, float bc1, float bc2_sqrt) {
    float gr = a.grad_scale * gr_raw;
    if (g.decay_coef != 0.0f) {
        if (g.decay_kind == 1) {
            const float o = 1.0f / (1.0f + det_expf(-th));
            gr = __builtin_fmaf(g.decay_coef, o * (1.0f - o), gr);
        } else if (g.decay_kind == 2) {
            gr = __builtin_fmaf(g.decay_coef, det_expf(th), gr);
        }
    }
    if (a.max_grad != 0.0f) gr = __builtin_copysignf(__builtin_fminf(__builtin_fabsf(gr), a.max_grad), gr);
    const float gg = gr * gr;
    if (g.lerp_form == 0) {
        m = __builtin_fmaf(t1, gr - m, m);
        v = __builtin_fmaf(t2, gg - v, v);
    } else {
        m = __builtin_fmaf(t1, gr, __builtin_fmaf(-t1, m, m));
        v = __builtin_fmaf(t2, gg, __builtin_fmaf(-t2, v, v));
    }
    const float mh = m / bc1;
    const float den = __builtin_sqrtf(v) / bc2_sqrt + a.eps;
    return th - (mh * g.lr) / den;
}

// Primitive (row) of element e of a group whose rows hold w elements.
__device__ __forceinline__ uint32_t row_of(uint32_t e, int w) {
    switch (w) {
        case 1: return e;
        case 3: return e / 3u;
        case 4: return e >> 2;
        default: return e / 45u;
    }
}

// simple_adam.cu:475-480: the bias corrections of step t, in double, rounded
// to float (1 - beta1^t and sqrt(1 - beta2^t)), as float bits at out[0], out[1]
__device__ __forceinline__ void adam_state_corrections(uint32_t* out, uint32_t t, float beta1, float beta2) {
    const double st = (double)t;
    out[0] = f2u((float)(1.0 - pow((double)beta1, st)));
    out[1] = f2u((float)sqrt(1.0 - pow((double)beta2, st)));
}

// Device step state [0] count t, [1..2] the corrections of t, [3..4] those of
// t + 1: one step on (an advancing launch used [3..4]); the next step's
// corrections are computed here, once per launch, so a launch's workgroups
// only read them.
__device__ __forceinline__ void adam_state_advance(uint32_t* state, float beta1, float beta2) {
    const uint32_t t = state[0] + 1u;
    state[0] = t;
    state[1] = state[3];
    state[2] = state[4];
    adam_state_corrections(state + 3, t + 1u, beta1, beta2);
}

// Each thread updates kAdamVecPerThread 4-element vectors with 16-byte loads
// and stores (8-byte for fp16 theta); lanes of a wave cover consecutive
// vectors. All loads of a thread are issued before any arithmetic.
// SEL: 0 every row, kAdamRowsUnmarked / kAdamRowsMarked one part of the rows
// (a compile-time choice: the selection costs VALU the full step does not need)
template <int SEL>
__global__ void __launch_bounds__(kAdamThreads) adam_kernel(AdamLaunch L) {
    const int64_t b = blockIdx.x;
    int gi = 0;
#pragma unroll
    for (int k = 1; k < 6; ++k)
        if (k < L.a.n_groups && b >= L.block_start[k]) gi = k;
    const AdamGroup& g = L.a.groups[gi];
    const float t1 = 1.0f - L.a.beta1, t2 = 1.0f - L.a.beta2;
    float bc1 = L.a.bc1, bc2s = L.a.bc2_sqrt;
    if (L.a.dev_bc) {   // this count's corrections ([1], [2]) or the next one's ([3], [4])
        bc1 = u2f(L.a.dev_bc[L.a.dev_advance ? 3 : 1]);
        bc2s = u2f(L.a.dev_bc[L.a.dev_advance ? 4 : 2]);
    }
    const int64_t vbase = (b - L.block_start[gi]) * (kAdamChunk / 4) + threadIdx.x;
    constexpr int sel = SEL;
    float th[kAdamVecPerThread][4];
    float4 gv[kAdamVecPerThread], mv[kAdamVecPerThread], vv[kAdamVecPerThread];
    bool full[kAdamVecPerThread];
    uint32_t upd[kAdamVecPerThread];   // bit q: element q of the vector is updated
#pragma unroll
    for (int k = 0; k < kAdamVecPerThread; ++k) {
        const int64_t e0 = 4 * (vbase + (int64_t)k * kAdamThreads);
        full[k] = e0 + 3 < g.count;
        upd[k] = 0xfu;
        if (full[k]) {
            bool lv[4] = {true, true, true, true};
            if (L.a.row_mask) {
#pragma unroll
                for (int q = 0; q < 4; ++q) lv[q] = L.a.row_mask[row_of((uint32_t)(e0 + q), g.row_width)] != 0;
                if constexpr (sel != 0) {
                    upd[k] = 0u;
#pragma unroll
                    for (int q = 0; q < 4; ++q) upd[k] |= (lv[q] == (sel == kAdamRowsMarked)) ? 1u << q : 0u;
                }
            }
            if (sel != 0 && upd[k] == 0u) continue;   // rows of the other part: untouched
            if (g.theta_half) {
                const uint2 hv = *(const uint2*)((const __half*)g.theta + e0);
                const __half* h = (const __half*)&hv;
                for (int q = 0; q < 4; ++q) th[k][q] = __half2float(h[q]);
            } else {
                const float4 tv = *(const float4*)((const float*)g.theta + e0);
                th[k][0] = tv.x; th[k][1] = tv.y; th[k][2] = tv.z; th[k][3] = tv.w;
            }
            if (L.a.row_mask) {
                // rows without gradient are zero and not read
                float4 gg = make_float4(0.f, 0.f, 0.f, 0.f);
                if (lv[0] || lv[1] || lv[2] || lv[3]) gg = ntld(g.grad + e0);
                gv[k] = make_float4(lv[0] ? gg.x : 0.f, lv[1] ? gg.y : 0.f, lv[2] ? gg.z : 0.f, lv[3] ? gg.w : 0.f);
            } else {
                gv[k] = ntld(g.grad + e0);
            }
            mv[k] = ntld(g.m1 + e0);
            vv[k] = ntld(g.m2 + e0);
        }
    }
#pragma unroll
    for (int k = 0; k < kAdamVecPerThread; ++k) {
        const int64_t e0 = 4 * (vbase + (int64_t)k * kAdamThreads);
        if (full[k]) {
            if (sel != 0 && upd[k] == 0u) continue;
            th[k][0] = adam_one(th[k][0], gv[k].x, mv[k].x, vv[k].x, g, L.a, t1, t2, bc1, bc2s);
            th[k][1] = adam_one(th[k][1], gv[k].y, mv[k].y, vv[k].y, g, L.a, t1, t2, bc1, bc2s);
            th[k][2] = adam_one(th[k][2], gv[k].z, mv[k].z, vv[k].z, g, L.a, t1, t2, bc1, bc2s);
            th[k][3] = adam_one(th[k][3], gv[k].w, mv[k].w, vv[k].w, g, L.a, t1, t2, bc1, bc2s);
            if (sel == 0 || upd[k] == 0xfu) {
                if (g.theta_half) {
                    uint2 hv;
                    __half* h = (__half*)&hv;
                    for (int q = 0; q < 4; ++q) h[q] = f2h_rn(th[k][q]);
                    *(uint2*)((__half*)g.theta + e0) = hv;
                } else {
                    *(float4*)((float*)g.theta + e0) = make_float4(th[k][0], th[k][1], th[k][2], th[k][3]);
                }
                ntst(g.m1 + e0, mv[k]);
                ntst(g.m2 + e0, vv[k]);
            } else {   // a vector across the two parts: element stores of this part's rows
                const float mq[4] = {mv[k].x, mv[k].y, mv[k].z, mv[k].w};
                const float vq[4] = {vv[k].x, vv[k].y, vv[k].z, vv[k].w};
                for (int q = 0; q < 4; ++q) {
                    if (!((upd[k] >> q) & 1u)) continue;
                    if (g.theta_half)
                        ((__half*)g.theta)[e0 + q] = f2h_rn(th[k][q]);
                    else
                        ((float*)g.theta)[e0 + q] = th[k][q];
                    g.m1[e0 + q] = mq[q];
                    g.m2[e0 + q] = vq[q];
                }
            }
        } else if (e0 < g.count) {
            for (int64_t i = e0; i < g.count; ++i) {
                const bool live = !L.a.row_mask || L.a.row_mask[row_of((uint32_t)i, g.row_width)] != 0;
                if (sel != 0 && live != (sel == kAdamRowsMarked)) continue;
                float t = g.theta_half ? __half2float(((const __half*)g.theta)[i]) : ((const float*)g.theta)[i];
                float m = g.m1[i], v = g.m2[i];
                t = adam_one(t, live ? g.grad[i] : 0.f, m, v, g, L.a, t1, t2, bc1, bc2s);
                if (g.theta_half)
                    ((__half*)g.theta)[i] = f2h_rn(t);
                else
                    ((float*)g.theta)[i] = t;
                g.m1[i] = m;
                g.m2[i] = v;
            }
        }
    }
    // An advancing launch: the last workgroup to finish stores the advanced
    // count and the next corrections (every workgroup read them before
    // counting itself done). Workgroups count themselves done in
    // kAdamDoneGroups counters on their own cache lines (workgroup b in
    // b mod kAdamDoneGroups), so no address takes more than a group's share
    // of the atomics; the last of a group counts the group in one more
    // counter. (Relaxed atomics: the counters' resets and the new state are
    // read only by later launches.)
    if (L.a.dev_bc && L.a.dev_advance) __syncthreads();   // every wave of the workgroup has read them
    if (L.a.dev_bc && L.a.dev_advance && threadIdx.x == 0) {
        const uint32_t g = blockIdx.x % kAdamDoneGroups;
        const uint32_t quota = (gridDim.x - g + kAdamDoneGroups - 1u) / kAdamDoneGroups;
        uint32_t* grp = L.a.dev_bc + kAdamDoneStride * (1u + g);
        if (atomicAdd(grp, 1u) == quota - 1u) {
            *grp = 0u;
            uint32_t* all = L.a.dev_bc + kAdamDoneStride * (1u + kAdamDoneGroups);
            if (atomicAdd(all, 1u) == min(gridDim.x, kAdamDoneGroups) - 1u) {
                *all = 0u;
                adam_state_advance(L.a.dev_bc, L.a.beta1, L.a.beta2);
            }
        }
    }
}

// The device-side step count of a captured (or replayed) step.
__global__ void adam_seed_steps_kernel(uint32_t* state, uint32_t steps, float beta1, float beta2) {
    if (threadIdx.x == 0) {
        state[0] = steps;
        adam_state_corrections(state + 1, steps, beta1, beta2);
        adam_state_corrections(state + 3, steps + 1u, beta1, beta2);
    }
    // the done counters of an advancing Adam launch
    for (uint32_t g = threadIdx.x; g <= kAdamDoneGroups; g += blockDim.x) state[kAdamDoneStride * (1u + g)] = 0u;
}

// The stored corrections of the device count t and of t + 1 under new betas.
__global__ void adam_rebeta_kernel(uint32_t* state, float beta1, float beta2) {
    if (threadIdx.x == 0) {
        adam_state_corrections(state + 1, state[0], beta1, beta2);
        adam_state_corrections(state + 3, state[0] + 1u, beta1, beta2);
    }
}

// An advancing step without an Adam launch (no rows).
__global__ void adam_bias_kernel(uint32_t* state, float beta1, float beta2) {
    if (threadIdx.x == 0) adam_state_advance(state, beta1, beta2);
}

void launch_adam_seed_steps(uint32_t* state, uint32_t steps, float beta1, float beta2, hipStream_t s) {
    adam_seed_steps_kernel<<<1, 64, 0, s>>>(state, steps, beta1, beta2);
}

void launch_adam_rebeta(uint32_t* state, float beta1, float beta2, hipStream_t s) {
    adam_rebeta_kernel<<<1, 64, 0, s>>>(state, beta1, beta2);
}

void launch_adam_bias(uint32_t* state, float beta1, float beta2, hipStream_t s) {
    adam_bias_kernel<<<1, 64, 0, s>>>(state, beta1, beta2);
}

void launch_adam(const AdamArgs& a, hipStream_t s) {
    AdamLaunch L;
    L.a = a;
    int64_t acc = 0;
    for (int k = 0; k < 7; ++k) L.block_start[k] = 0;
    for (int k = 0; k < a.n_groups; ++k) {
        L.block_start[k] = acc;
        acc += (a.groups[k].count + kAdamChunk - 1) / kAdamChunk;
    }
    for (int k = a.n_groups; k < 7; ++k) L.block_start[k] = acc;
    if (acc == 0) {   // no rows: the count still advances
        if (a.dev_bc && a.dev_advance) launch_adam_bias(a.dev_bc, a.beta1, a.beta2, s);
        return;
    }
    const int sel = a.row_mask ? a.row_select : 0;
    if (sel == kAdamRowsUnmarked)
        adam_kernel<kAdamRowsUnmarked><<<(unsigned)acc, kAdamThreads, 0, s>>>(L);
    else if (sel == kAdamRowsMarked)
        adam_kernel<kAdamRowsMarked><<<(unsigned)acc, kAdamThreads, 0, s>>>(L);
    else
        adam_kernel<0><<<(unsigned)acc, kAdamThreads, 0, s>>>(L);
}

}  // namespace tgs
