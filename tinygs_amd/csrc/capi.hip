// C ABI (include/tinygs_amd.h): handles, grow-only device scratch, the
// forward / backward stage order of FastGSRasterizer and the loss and
// optimizer plugins.
//
// Stage order follows tinygs/src/rasterizer/fastgs_ours/forward.cu:20-292 and
// backward.cu:211-349. Differences, each deliberate:
//   * one host synchronisation per forward (to size the instance buffers)
//     instead of three; no helper stream or events;
//   * the pose block is not copied to the device: w2c rows and the camera
//     centre travel as kernel arguments;
//   * visible primitives are compacted by prefix scan (deterministic order);
//   * no per-bucket checkpoints (the backward recomputes them).
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/tinygs_amd.h"
#include "common.h"
#include "kernels.h"
#include "pcg32.h"
#include "status.h"

using namespace tgs;

namespace tgs {

thread_local std::string g_error;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_error = buf;
    return code;
}

}  // namespace tgs

namespace {

struct DevBuf {
    void* p = nullptr;
    size_t bytes = 0;
    template <typename T>
    T* as() const { return (T*)p; }
};

// Grow-only device allocation. A grown buffer is released only after the
// stream has drained, so kernels of earlier calls never see freed memory.
int ensure(DevBuf& b, size_t bytes, hipStream_t s) {
    if (bytes <= b.bytes && b.p) return TGS_OK;
    if (b.p) {
        TGS_HIP(hipStreamSynchronize(s));
        TGS_HIP(hipFree(b.p));
        b.p = nullptr;
        b.bytes = 0;
    }
    size_t nb = bytes + bytes / 4 + 256;
    TGS_HIP(hipMalloc(&b.p, nb));
    b.bytes = nb;
    return TGS_OK;
}

void release(DevBuf& b) {
    if (b.p) (void)hipFree(b.p);
    b.p = nullptr;
    b.bytes = 0;
}

// ---- stage timing: HIP events recorded on the launch stream around the
// stages selected by tgs_profiling_set (process-wide, single host thread).
constexpr int kStageCount = 10;
// Largest tile grid of fp16 images (27-bit tile keys: four sort passes of at
// most 8 bits; ranges and tile maxima alone take 12 B per tile)
constexpr uint32_t kMaxTiles16 = 1u << 27;
const char* const kStageNames[kStageCount] = {
    "preprocess", "depth_sort", "emit_instances", "tile_sort", "blend_forward",
    "l1", "fused_ssim", "blend_backward", "preprocess_backward", "adam"};
enum { ST_PRE = 0, ST_DEPTH, ST_EMIT, ST_TILES, ST_BLENDF, ST_L1, ST_SSIM, ST_BLENDB, ST_PREB, ST_ADAM };

struct EventPair {
    hipEvent_t a, b;
};
struct Profiler {
    uint32_t mask = 0;
    std::vector<EventPair> pending[kStageCount];
    std::vector<EventPair> pool;
    double total_ms[kStageCount] = {};
    int64_t count[kStageCount] = {};
};
Profiler g_prof;

struct StageScope {
    int st;
    hipStream_t s;
    bool on = false;
    EventPair p{};
    StageScope(int stage, hipStream_t stream) : st(stage), s(stream) {
        if (!(g_prof.mask & (1u << stage))) return;
        if (!g_prof.pool.empty()) {
            p = g_prof.pool.back();
            g_prof.pool.pop_back();
        } else if (hipEventCreate(&p.a) != hipSuccess || hipEventCreate(&p.b) != hipSuccess) {
            return;
        }
        on = hipEventRecord(p.a, s) == hipSuccess;
    }
    ~StageScope() {
        if (!on) return;
        if (hipEventRecord(p.b, s) == hipSuccess) g_prof.pending[st].push_back(p);
    }
};

int build_camera(const tgs_camera* c, CamParams& cp) {
    if (!c) return fail(TGS_ERR_INVALID, "camera is NULL");
    if (c->width == 0 || c->height == 0) return fail(TGS_ERR_INVALID, "image size %ux%u", c->width, c->height);
    if (c->width > 65535u * 16u || c->height > 65535u * 16u)
        return fail(TGS_ERR_INVALID, "image too large for 16-bit tile bounds");
    memset(&cp, 0, sizeof(cp));
    cp.fx = c->K[0];
    cp.fy = c->K[4];
    cp.cx = c->K[6];
    cp.cy = c->K[7];
    cp.near_ = c->near_plane;
    cp.far_ = c->far_plane;
    // glm column-major: element (row r, col k) at w2c[k * 4 + r]; rows are
    // glm::transpose(w2c) as uploaded by fastgs.cu:99.
    for (int k = 0; k < 4; ++k) {
        cp.r1[k] = c->w2c[k * 4 + 0];
        cp.r2[k] = c->w2c[k * 4 + 1];
        cp.r3[k] = c->w2c[k * 4 + 2];
    }
    // camera centre = column 3 of inverse(w2c) (fastgs.cu:96,100), in double
    double m[16], inv[16];
    for (int r = 0; r < 4; ++r)
        for (int k = 0; k < 4; ++k) m[r * 4 + k] = c->w2c[k * 4 + r];
    // Gauss-Jordan with partial pivoting on the row-major copy
    double a[4][8];
    for (int r = 0; r < 4; ++r) {
        for (int k = 0; k < 4; ++k) a[r][k] = m[r * 4 + k];
        for (int k = 0; k < 4; ++k) a[r][4 + k] = (r == k) ? 1.0 : 0.0;
    }
    for (int col = 0; col < 4; ++col) {
        int piv = col;
        for (int r = col + 1; r < 4; ++r)
            if (fabs(a[r][col]) > fabs(a[piv][col])) piv = r;
        if (fabs(a[piv][col]) < 1e-30) return fail(TGS_ERR_INVALID, "w2c is singular");
        if (piv != col)
            for (int k = 0; k < 8; ++k) {
                double t = a[col][k];
                a[col][k] = a[piv][k];
                a[piv][k] = t;
            }
        const double d = a[col][col];
        for (int k = 0; k < 8; ++k) a[col][k] /= d;
        for (int r = 0; r < 4; ++r) {
            if (r == col) continue;
            const double f = a[r][col];
            for (int k = 0; k < 8; ++k) a[r][k] -= f * a[col][k];
        }
    }
    for (int r = 0; r < 4; ++r)
        for (int k = 0; k < 4; ++k) inv[r * 4 + k] = a[r][4 + k];
    cp.cam_pos[0] = (float)inv[0 * 4 + 3];
    cp.cam_pos[1] = (float)inv[1 * 4 + 3];
    cp.cam_pos[2] = (float)inv[2 * 4 + 3];
    cp.w = (float)c->width;
    cp.h = (float)c->height;
    // float arithmetic (this file is built without contraction), the same
    // operations the device would do
    cp.clip_left = (-0.15f * cp.w - cp.cx) / cp.fx;
    cp.clip_right = (1.15f * cp.w - cp.cx) / cp.fx;
    cp.clip_top = (-0.15f * cp.h - cp.cy) / cp.fy;
    cp.clip_bottom = (1.15f * cp.h - cp.cy) / cp.fy;
    cp.width = c->width;
    cp.height = c->height;
    cp.grid_w = (c->width + 15u) / 16u;
    cp.grid_h = (c->height + 15u) / 16u;
    cp.tiled_w = (c->width + 7u) >> 3;
    cp.tiled_h = (c->height + 7u) >> 3;
    return TGS_OK;
}

int check_gaussians(const tgs_gaussians* g, bool is_grad) {
    if (!g) return fail(TGS_ERR_INVALID, "gaussians is NULL");
    if (g->n < 0 || g->n > (int64_t)0xffffffffll) return fail(TGS_ERR_INVALID, "invalid gaussian count %lld", (long long)g->n);
    if (g->n > 0 && (!g->means || !g->scales || !g->rotations || !g->opacities || !g->sh0 || !g->sh_rest))
        return fail(TGS_ERR_INVALID, "a gaussian SoA pointer is NULL");
    // kernels move whole blocks of these arrays with 16-byte vector accesses
    const uintptr_t al = (uintptr_t)g->means | (uintptr_t)g->scales | (uintptr_t)g->rotations |
                         (uintptr_t)g->opacities | (uintptr_t)g->sh0 | (uintptr_t)g->sh_rest;
    if (al & 15u) return fail(TGS_ERR_INVALID, "gaussian SoA arrays must be 16-byte aligned");
    if (!is_grad && (g->sh_degree < 0 || g->sh_degree > 3)) return fail(TGS_ERR_INVALID, "sh_degree %d", g->sh_degree);
    if (!is_grad && g->sh_dtype != TGS_DTYPE_FLOAT32 && g->sh_dtype != TGS_DTYPE_FLOAT16)
        return fail(TGS_ERR_INVALID, "sh_dtype %d", g->sh_dtype);
    return TGS_OK;
}

}  // namespace

struct tgs_rasterizer {
    tgs_gaussians g{};
    bool has_g = false;
    // per primitive
    DevBuf n_touched, erec, mean2d, conic_opacity, color, depth_key, offs;
    DevBuf pkeys[2], pvals[2], pnt[2];   // depth sort: key, primitive, n_touched
    // per instance
    DevBuf ikeys[2], ivals[2];
    // per tile / pixel
    DevBuf ranges, tile_max, n_contrib;
    DevBuf ckpt, items;   // blend checkpoints (float4 x 256 per slot), backward work items (uint4)
    DevBuf tile_loaded;   // Gaussians staged per tile by the last forward (work statistic)
    DevBuf tile_order;    // tiles, long ones first, for the fp16-image blend forward
    // backward 2D-gradient records: per primitive first instance slot, record
    // count (kept zero between backwards), records (3 float4 per instance
    // slot), heavy-gather list
    DevBuf first_slot, rec_count, records;
    // fp32 images: each instance's rank among its primitive's instances
    // (u16, sorted with the tile keys) and one bit per instance slot marking
    // the records the last backward wrote (record of instance rank k of p at
    // slot first_slot[p] + k, so the per-primitive sums run in a fixed order)
    DevBuf iranks, rec_bits;
    DevBuf rec_mask;   // fp32 images: per primitive, the record marks of ranks 0..31 (zero between backwards)
    DevBuf live, heavy;   // preprocess backward: per-chunk lists of primitives with records
    DevBuf row_mask;     // per-primitive byte mask of the last sparse backward
    bool row_mask_valid = false;
    DevBuf bwd_rows;     // rows the backward of the last forward writes (tgs_rasterizer_backward_rows)
    bool bwd_rows_valid = false;
    DevBuf pose_partial, pose_grad;   // pose gradient: per-chunk partial sums, the 4 x 4 result
    bool pose_valid = false;
    bool grad2d_valid = false;   // grad2d holds every primitive's 2D sums (TGS_BACKWARD_KEEP_2D)
    uint32_t depth_key_base = 0;   // the sorted depth keys are key - depth_key_base
    // temp
    DevBuf grad2d;
    DevBuf radix_counts;   // per-workgroup digit counts of the radix passes
    DevBuf block_n;        // visible primitives per compaction block (the depth sort's first-pass blocks)
    DevBuf bin_ctl;     // BinCtl (zeroed at creation; all but err cleared every forward)
    hipEvent_t ev_counts = nullptr;   // recorded after the counts copy of a forward
    hipEvent_t ev_err = nullptr;      // recorded after the error-word copy that follows the tile sort
    DevBuf lb_status;   // look-back status words (u64), epoch-tagged
    // look-back launches of the current forward so far: its k-th launch uses
    // epoch BinCtl::epoch_base + k (the base advances on the device per forward)
    uint32_t epoch = 0;
    uint64_t forwards = 0;   // forwards queued by this host (eager; graph replays not counted)
    uint32_t* h_counters = nullptr;   // pinned copy of BinCtl {V, I, err}; [4]: err after the tile sort
    // state of the last forward
    bool fwd_done = false;
    bool ikeys_from_ranges = false;   // the sorted tile keys exist only as the tile ranges
    int64_t tile_sort_cap = 0;        // the tile sort's key capacity (instances past it are dropped)
    bool bwd_queues_clear = false;   // backward queue counters still zero since the last forward
    CamParams cam{};
    int64_t n = 0, V = 0, I = 0;
    int64_t inst_cap = 0;            // reserved instance capacity (tgs_rasterizer_reserve)
    bool counts_on_device = false;   // the last forward did not wait for V, I
    int psel = 0, isel = 0;
    bool fgs16 = false;              // the last forward rendered an fp16 image (FGS16)
};

// Look-back status words for `entries` slots. A (re)allocated array is
// cleared (all words "not ready"), and so is the array once every 2^22
// forwards, long before the 30-bit epochs (2^24 forwards apart) could alias.
static int ensure_status(tgs_rasterizer* r, int64_t entries, hipStream_t s) {
    const void* before = r->lb_status.p;
    TGS_TRY(ensure(r->lb_status, sizeof(uint64_t) * (size_t)(entries > 0 ? entries : 1), s));
    if (r->lb_status.p != before || (r->forwards & ((1ull << 22) - 1ull)) == 0)
        launch_fill_u32(r->lb_status.as<uint32_t>(), 0u, (int64_t)(r->lb_status.bytes / 4), s);
    return TGS_OK;
}

// Instance-sized buffers for up to `inst` instances over T tiles: sort
// pairs, blend checkpoints and backward work items, 2D-gradient records.
static int ensure_instances(tgs_rasterizer* r, int64_t inst, uint32_t T, hipStream_t s) {
    const int64_t ii = inst > 0 ? inst : 1;
    for (int k = 0; k < 2; ++k) {
        TGS_TRY(ensure(r->ikeys[k], 4 * ii, s));
        TGS_TRY(ensure(r->ivals[k], 4 * ii, s));
    }
    const size_t slots = blend_ckpt_slots(inst > 0 ? inst : 0, T);
    TGS_TRY(ensure(r->ckpt, sizeof(float4) * kTilePixels * slots, s));
    TGS_TRY(ensure(r->items, sizeof(uint4) * slots, s));
    TGS_TRY(ensure(r->records, 3 * sizeof(float4) * (size_t)ii, s));
    TGS_TRY(ensure(r->iranks, sizeof(uint16_t) * (size_t)ii, s));
    TGS_TRY(ensure(r->rec_bits, sizeof(uint32_t) * (size_t)record_bit_words(ii), s));
    return TGS_OK;
}

struct tgs_loss {
    int type = 0;  // 0 l1, 1 fused_ssim
    DevBuf dm[3];
};

struct tgs_adam {
    tgs_gaussians params{};
    tgs_gaussians grads{};
    DevBuf m1[6], m2[6];
    int64_t rows = 0;   // Gaussians the moments are sized for
    tgs_adam_params p{};
    float global_lr = 1.0f;
    int64_t steps = 0;
    DevBuf dev_state;           // TGS_ADAM_DEVICE_STEP: step count and bias corrections on the device
    bool dev_seeded = false;    // dev_state's count equals `steps` (set by the first device step)
    float dev_beta1 = 0.f, dev_beta2 = 0.f;   // the betas dev_state's corrections were computed with
    bool last_dev = false;      // the last step's mode (TGS_ADAM_SAME_STEP repeats it)
};

extern "C" {

const char* tgs_last_error(void) { return g_error.c_str(); }
int tgs_version(void) { return 1; }

// ------------------------------------------------------------------ rasterizer

int tgs_rasterizer_create(const char* type, tgs_rasterizer** out) {
    if (!out) return fail(TGS_ERR_INVALID, "out is NULL");
    *out = nullptr;
    std::string t = type ? type : "";
    for (auto& ch : t) ch = (char)tolower(ch);
    if (t != "fastgs") return fail(TGS_ERR_UNSUPPORTED, "Unknown rasterizer type: %s", type ? type : "(null)");
    tgs_rasterizer* r = new tgs_rasterizer();
    hipError_t e = hipHostMalloc((void**)&r->h_counters, 64, hipHostMallocDefault);
    if (e == hipSuccess) e = hipMalloc(&r->bin_ctl.p, sizeof(BinCtl));
    if (e == hipSuccess) {
        r->bin_ctl.bytes = sizeof(BinCtl);
        e = hipMemset(r->bin_ctl.p, 0, sizeof(BinCtl));
    }
    if (e == hipSuccess) e = hipEventCreateWithFlags(&r->ev_counts, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&r->ev_err, hipEventDisableTiming);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        if (r->h_counters) (void)hipHostFree(r->h_counters);
        if (r->ev_counts) (void)hipEventDestroy(r->ev_counts);
        if (r->ev_err) (void)hipEventDestroy(r->ev_err);
        release(r->bin_ctl);
        delete r;
        return fail(TGS_ERR_HIP, "rasterizer allocation: %s", hipGetErrorString(e));
    }
    *out = r;
    return TGS_OK;
}

int tgs_rasterizer_destroy(tgs_rasterizer* r) {
    if (!r) return TGS_OK;
    (void)hipDeviceSynchronize();
    DevBuf* all[] = {&r->n_touched, &r->erec, &r->mean2d, &r->conic_opacity, &r->color, &r->depth_key,
                     &r->offs, &r->pkeys[0], &r->pkeys[1], &r->pvals[0], &r->pvals[1], &r->pnt[0], &r->pnt[1],
                     &r->radix_counts, &r->block_n, &r->ikeys[0],
                     &r->ikeys[1], &r->ivals[0], &r->ivals[1], &r->ranges, &r->tile_max, &r->n_contrib,
                     &r->ckpt, &r->items, &r->tile_loaded, &r->tile_order, &r->first_slot,
                     &r->rec_count, &r->records, &r->iranks, &r->rec_bits, &r->rec_mask, &r->heavy, &r->live,
                     &r->row_mask,
                     &r->grad2d,
                     &r->bwd_rows, &r->pose_partial, &r->pose_grad, &r->bin_ctl, &r->lb_status};
    for (DevBuf* b : all) release(*b);
    if (r->h_counters) (void)hipHostFree(r->h_counters);
    if (r->ev_counts) (void)hipEventDestroy(r->ev_counts);
    if (r->ev_err) (void)hipEventDestroy(r->ev_err);
    delete r;
    return TGS_OK;
}

int tgs_rasterizer_set_gaussians(tgs_rasterizer* r, const tgs_gaussians* g) {
    if (!r) return fail(TGS_ERR_INVALID, "rasterizer is NULL");
    TGS_TRY(check_gaussians(g, false));
    r->g = *g;
    r->has_g = true;
    r->fwd_done = false;
    return TGS_OK;
}

static GaussianView view_of(const tgs_gaussians& g) {
    GaussianView v;
    v.means = (const float*)g.means;
    v.scales = (const float*)g.scales;
    v.rotations = (const float*)g.rotations;
    v.opacities = (const float*)g.opacities;
    v.sh0 = g.sh0;
    v.sh_rest = g.sh_rest;
    v.n = g.n;
    v.sh_degree = g.sh_degree;
    v.sh_dtype = g.sh_dtype;
    return v;
}

// Depth-sort digit plan: visible depths lie in [near, far] (preprocess culls
// the rest), so with near > 0 the keys (float bits) minus bits(near) span
// only the bits of bits(far) - bits(near): 27 for near 0.01, far 100, i.e.
// three passes of 9-bit digits instead of four of 8.
struct SortPlan {
    uint32_t key_base = 0;
    int n_dp = 4, dshift[4] = {0, 0, 0, 0}, dbits[4] = {0, 0, 0, 0};
    int n_tp = 1, tshift[4] = {0, 0, 0, 0}, tbits[4] = {0, 0, 0, 0};
};

static int plan_sorts(const CamParams& cam, SortPlan& sp) {
    int key_bits = 32;
    if (cam.near_ > 0.f && cam.far_ >= cam.near_ && cam.far_ <= 3.0e38f) {
        sp.key_base = f2u(cam.near_);
        const uint32_t range = f2u(cam.far_) - sp.key_base;
        key_bits = range ? 32 - __builtin_clz(range) : 1;
    }
    sp.n_dp = key_bits <= 9 ? 1 : key_bits <= 18 ? 2 : key_bits <= 27 ? 3 : 4;
    for (int p = 0; p < sp.n_dp; ++p) {
        sp.dbits[p] = (key_bits + sp.n_dp - 1) / sp.n_dp;
        sp.dshift[p] = p * sp.dbits[p];
    }
    // tile key bits: passes of at most 8 bits, as even as possible, the later
    // passes taking the odd bits: 16 bits (65,536 tiles, the fp32 limit) in
    // two passes, up to 24 in three, up to 27 (fp16 images) in four. The
    // first pass reads the instances in emission order, where one
    // primitive's keys run over consecutive tiles, and scatters into fewer
    // buckets that way: at 545M instances over 15 tile bits its downsweep
    // took 3.9-4.0 ms with 128 buckets, against 3.6 or 5.4 ms (varying from
    // run to run) with 256
    const uint32_t T = cam.grid_w * cam.grid_h;
    int bits = 1;
    while (bits < 32 && (1u << bits) < T) ++bits;
    sp.n_tp = (bits + 7) / 8;
    for (int p = 0, sh = 0; p < sp.n_tp; ++p) {
        sp.tbits[p] = bits / sp.n_tp + (p >= sp.n_tp - bits % sp.n_tp ? 1 : 0);
        sp.tshift[p] = sh;
        sh += sp.tbits[p];
    }
    if (!radix_digits_fit(true, sp.n_dp, sp.dbits) || !radix_digits_fit(false, sp.n_tp, sp.tbits))
        return fail(TGS_ERR_UNSUPPORTED, "no radix digit plan for %d depth-key bits / %u tiles", key_bits, T);
    return TGS_OK;
}

static int rasterizer_forward(tgs_rasterizer* r, const tgs_camera* camera, void* image, int32_t image_dtype,
                              void* densification_info, int32_t flags, void* stream) {
    if (!r) return fail(TGS_ERR_INVALID, "rasterizer is NULL");
    if (!r->has_g) return fail(TGS_ERR_STATE, "Gaussians not set");
    if (!image) return fail(TGS_ERR_INVALID, "image is NULL");
    // fastgs.cu:143-188: the image dtype selects the rasterizer (fp16: FGS16)
    if (image_dtype != TGS_DTYPE_FLOAT32 && image_dtype != TGS_DTYPE_FLOAT16)
        return fail(TGS_ERR_UNSUPPORTED, "image dtype %d: float32 or float16 images only", image_dtype);
    const bool f16 = image_dtype == TGS_DTYPE_FLOAT16;
    if (flags & ~TGS_FORWARD_NO_SYNC) return fail(TGS_ERR_INVALID, "unknown forward flags 0x%x", flags);
    const bool nosync = (flags & TGS_FORWARD_NO_SYNC) != 0;
    hipStream_t s = (hipStream_t)stream;
    CamParams cam;
    TGS_TRY(build_camera(camera, cam));
    const uint64_t T64 = (uint64_t)cam.grid_w * cam.grid_h;
    // fp32 images: instance tile keys are 16-bit in the reference
    // (kernels_forward.cuh:477,521; forward.cu:214 sorts 16 bits), which caps
    // the grid at 65,536 tiles. fp16 images: 32-bit tile keys
    // (fastgs_ours_fp16/kernels_forward.cuh:622-623, forward.cu:205-211);
    // here up to kMaxTiles16 (2^27) tiles, four sort passes
    if (!f16 && T64 > 65536u)
        return fail(TGS_ERR_UNSUPPORTED, "%ux%u tiles exceed the 65,536 tiles of 16-bit tile keys", cam.grid_w,
                    cam.grid_h);
    if (f16 && T64 > kMaxTiles16)
        return fail(TGS_ERR_UNSUPPORTED, "%ux%u tiles exceed the %u tiles of fp16-image tile keys", cam.grid_w,
                    cam.grid_h, kMaxTiles16);
    const uint32_t T = (uint32_t)T64;
    if (nosync && r->inst_cap <= 0)
        return fail(TGS_ERR_STATE, "TGS_FORWARD_NO_SYNC needs an instance capacity (tgs_rasterizer_reserve)");
    SortPlan sp;
    TGS_TRY(plan_sorts(cam, sp));
    r->fwd_done = false;
    r->row_mask_valid = false;
    r->bwd_rows_valid = false;
    r->pose_valid = false;
    r->grad2d_valid = false;
    const int64_t n = r->g.n;
    const size_t cs = (size_t)cam.tiled_w * cam.tiled_h * 64u;
    const int64_t nn = n > 0 ? n : 1;
    TGS_TRY(ensure(r->n_touched, 4 * nn, s));
    TGS_TRY(ensure(r->erec, 16 * nn, s));
    TGS_TRY(ensure(r->mean2d, 8 * nn, s));
    TGS_TRY(ensure(r->conic_opacity, 16 * nn, s));
    TGS_TRY(ensure(r->color, 16 * nn, s));
    TGS_TRY(ensure(r->depth_key, 4 * nn, s));
    TGS_TRY(ensure(r->offs, 4 * (nn + 1), s));
    TGS_TRY(ensure(r->first_slot, 4 * nn, s));
    {
        const void* before = r->rec_count.p;
        TGS_TRY(ensure(r->rec_count, 4 * nn, s));
        if (r->rec_count.p != before)   // counters are zero between backwards; a new buffer starts so
            launch_fill_u32(r->rec_count.as<uint32_t>(), 0u, (int64_t)(r->rec_count.bytes / 4), s);
        const void* mbefore = r->rec_mask.p;
        TGS_TRY(ensure(r->rec_mask, 4 * nn, s));
        if (r->rec_mask.p != mbefore)   // (the same for the mask words)
            launch_fill_u32(r->rec_mask.as<uint32_t>(), 0u, (int64_t)(r->rec_mask.bytes / 4), s);
    }
    for (int k = 0; k < 2; ++k) {
        TGS_TRY(ensure(r->pkeys[k], 4 * nn, s));
        TGS_TRY(ensure(r->pvals[k], 4 * nn, s));
        TGS_TRY(ensure(r->pnt[k], 4 * nn, s));
    }
    TGS_TRY(ensure(r->ranges, 8 * (size_t)T, s));
    TGS_TRY(ensure(r->block_n, 4 * (size_t)std::max<int64_t>(scan_status_entries(nn), 1), s));
    TGS_TRY(ensure(r->tile_max, 4 * (size_t)T, s));
    TGS_TRY(ensure(r->tile_loaded, 4 * (size_t)T, s));
    TGS_TRY(ensure(r->tile_order, 4 * (size_t)T, s));
    TGS_TRY(ensure(r->n_contrib, 4 * cs, s));
    // without a host wait the instance buffers are sized by the reserved capacity up front
    const int64_t cap0 = nosync ? r->inst_cap : 0;
    TGS_TRY(ensure(r->radix_counts, 4 * (size_t)std::max(radix_count_entries(nn, true),
                                                          radix_count_entries(cap0 > 0 ? cap0 : 1, false)), s));
    TGS_TRY(ensure_status(r, std::max({scan_status_entries(nn), scan_status_entries(radix_count_entries(nn, true)),
                                       scan_status_entries(radix_count_entries(cap0 > 0 ? cap0 : 1, false))}), s));
    if (nosync) TGS_TRY(ensure_instances(r, cap0, T, s));

    GaussianView gv = view_of(r->g);
    BinCtl* ctl = r->bin_ctl.as<BinCtl>();
    uint64_t* status = r->lb_status.as<uint64_t>();
    // the same launch sequence, epochs included, every forward: what a graph replays
    r->epoch = 0;
    {
        // (the preprocess's first workgroup resets ctl, advancing the look-back epoch base)
        StageScope sc(ST_PRE, s);
        if (f16)
            launch_preprocess16(gv, cam, r->n_touched.as<uint32_t>(), r->erec.as<uint4>(),
                                r->mean2d.as<float2>(), r->conic_opacity.as<float4>(),
                                r->color.as<uint4>(), r->depth_key.as<uint32_t>(), (float*)densification_info, ctl,
                                s);
        else
            launch_preprocess(gv, cam, r->n_touched.as<uint32_t>(), r->erec.as<uint4>(), r->mean2d.as<float2>(),
                              r->conic_opacity.as<float4>(), r->color.as<float4>(), r->depth_key.as<uint32_t>(),
                              (float*)densification_info, ctl, s);
    }
    TGS_CHECK_LAUNCH();
    uint32_t* pk[2] = {r->pkeys[0].as<uint32_t>(), r->pkeys[1].as<uint32_t>()};
    uint32_t* pv[2] = {r->pvals[0].as<uint32_t>(), r->pvals[1].as<uint32_t>()};
    uint32_t* pn[2] = {r->pnt[0].as<uint32_t>(), r->pnt[1].as<uint32_t>()};
    int psel;
    {
        StageScope sc(ST_DEPTH, s);
        launch_compact_visible(r->n_touched.as<uint32_t>(), r->depth_key.as<uint32_t>(), n, sp.key_base,
                               sp.dshift[0], sp.dbits[0], pk[0], pv[0], pn[0], r->radix_counts.as<uint32_t>(),
                               r->block_n.as<uint32_t>(), ctl, s);
        if (!nosync) {
            // V, I and the sticky error flag go to the host while the depth sort runs
            TGS_HIP(hipMemcpyAsync(r->h_counters, ctl, 3 * sizeof(uint32_t), hipMemcpyDeviceToHost, s));
            TGS_HIP(hipEventRecord(r->ev_counts, s));
        }
        bool offs_done = false;
        psel = radix_sort(pk, pv, pn, &ctl->V, n, true, sp.n_dp, sp.dshift, sp.dbits, r->radix_counts.as<uint32_t>(),
                          ctl->tickets + kTicketDepth, status, &ctl->epoch_base, r->epoch, &ctl->err,
                          r->block_n.as<uint32_t>(), r->offs.as<uint32_t>(), &offs_done, nullptr, 0u, nullptr,
                          nullptr, nullptr, s);
        if (psel < 0) return fail(TGS_ERR_STATE, "depth sort digit width");
        r->depth_key_base = sp.key_base;
        if (!offs_done) launch_instance_offsets(pn[psel], n, r->offs.as<uint32_t>(), ctl, status, r->epoch, s);
    }
    TGS_CHECK_LAUNCH();
    int64_t V = -1, I = -1, cap = cap0;
    if (!nosync) {
        TGS_HIP(hipEventSynchronize(r->ev_counts));
        // (a capacity flag left by an earlier no-sync forward does not concern this one)
        if (const uint32_t bad = r->h_counters[2] & ~kErrCapacity) {
            launch_clear_err_bits(ctl, bad, s);   // reported once
            return fail(TGS_ERR_STATE, "binning failed on the device (error flags 0x%x)", bad);
        }
        V = r->h_counters[0];
        I = r->h_counters[1];
        cap = I;
        TGS_TRY(ensure(r->radix_counts,
                       4 * (size_t)std::max(radix_count_entries(I > 0 ? I : 1, false), radix_count_entries(nn, true)),
                       s));
        TGS_TRY(ensure_status(r, scan_status_entries(radix_count_entries(I > 0 ? I : 1, false)), s));
        TGS_TRY(ensure_instances(r, I, T, s));
        status = r->lb_status.as<uint64_t>();
    }
    {
        StageScope sc(ST_EMIT, s);
        // the exact tile test's words: conic_opacity and color_pt (threshold in w), or FGS16's info
        const uint4* conic_words = f16 ? r->color.as<uint4>() : r->conic_opacity.as<uint4>();
        launch_emit_instances(pv[psel], r->offs.as<uint32_t>(), ctl, n, cap, r->mean2d.as<float2>(), conic_words,
                              r->color.as<uint4>(), r->erec.as<uint4>(), cam.grid_w, r->ikeys[0].as<uint32_t>(),
                              r->ivals[0].as<uint32_t>(), r->first_slot.as<uint32_t>(), f16, s);
    }
    uint32_t* ik[2] = {r->ikeys[0].as<uint32_t>(), r->ikeys[1].as<uint32_t>()};
    uint32_t* iv[2] = {r->ivals[0].as<uint32_t>(), r->ivals[1].as<uint32_t>()};
    // without a host wait the instance count is read on the device (min(I, capacity))
    const uint32_t* d_inst = nosync ? &ctl->I : nullptr;
    int isel;
    bool ranges_done = false;   // the tile sort's last pass reduced the tile ranges
    {
        StageScope sc(ST_TILES, s);
        // fp32: the instances' ranks out of the keys' high bits, record bits cleared
        isel = radix_sort(ik, iv, nullptr, d_inst, cap, false, sp.n_tp, sp.tshift, sp.tbits,
                          r->radix_counts.as<uint32_t>(), ctl->tickets + kTicketTile, status, &ctl->epoch_base,
                          r->epoch, &ctl->err, nullptr, nullptr, nullptr, r->ranges.as<uint2>(), (uint32_t)T,
                          &ranges_done, f16 ? nullptr : r->iranks.as<uint16_t>(),
                          f16 ? nullptr : r->rec_bits.as<uint32_t>(), s);
        if (isel < 0) return fail(TGS_ERR_STATE, "tile sort digit width");
        if (r->epoch >= kEpochStride) return fail(TGS_ERR_STATE, "look-back launches per forward exceed the epoch stride");
        if (!ranges_done) launch_tile_ranges(ik[isel], d_inst, cap, r->ranges.as<uint2>(), T, s);
        r->ikeys_from_ranges = ranges_done;
        r->tile_sort_cap = cap;
    }
    // (a no-sync forward's capacity check is in the emission)
    if (!nosync) {
        // the depth and tile sorts' look-back scans and the emission's offset
        // check ran after the counts copy: their error word, read once the
        // blend below is queued (the blend and the emission skip their work
        // when it is set, so a failed scan's partial output is never read)
        TGS_HIP(hipMemcpyAsync(r->h_counters + 4, &ctl->err, sizeof(uint32_t), hipMemcpyDeviceToHost, s));
        TGS_HIP(hipEventRecord(r->ev_err, s));
    }
    {
        StageScope sc(ST_BLENDF, s);
        if (f16)
            launch_blend16_forward(cam, r->ranges.as<uint2>(), iv[isel], r->mean2d.as<float2>(), r->color.as<uint4>(),
                                   (uint16_t*)image, r->n_contrib.as<uint16_t>(), r->tile_max.as<uint32_t>(),
                                   r->tile_loaded.as<uint32_t>(), r->ckpt.as<uint2>(), r->items.as<uint4>(), ctl,
                                   r->tile_order.as<uint32_t>(), s);
        else
            launch_blend_forward(cam, r->ranges.as<uint2>(), iv[isel], r->mean2d.as<float2>(),
                                 r->conic_opacity.as<float4>(), r->color.as<float4>(), (float*)image,
                                 r->n_contrib.as<uint32_t>(), r->tile_max.as<uint32_t>(),
                                 r->tile_loaded.as<uint32_t>(), r->ckpt.as<float4>(), r->items.as<uint4>(), ctl,
                                 cap >= (int64_t)T * kOrderHeavyTile ? r->tile_order.as<uint32_t>() : nullptr, s);
    }
    TGS_CHECK_LAUNCH();
    if (!nosync) {
        TGS_HIP(hipEventSynchronize(r->ev_err));
        if (const uint32_t bad = r->h_counters[4] & ~kErrCapacity) {
            launch_clear_err_bits(ctl, bad, s);   // reported once
            return fail(TGS_ERR_STATE, "binning failed on the device (error flags 0x%x)", bad);
        }
    }
    r->cam = cam;
    r->n = n;
    r->V = V;
    r->I = I;
    r->counts_on_device = nosync;
    r->psel = psel;
    r->isel = isel;
    r->fgs16 = f16;
    r->forwards += 1;
    r->fwd_done = true;
    r->bwd_queues_clear = true;
    return TGS_OK;
}

int tgs_rasterizer_forward(tgs_rasterizer* r, const tgs_camera* camera, void* image, int32_t image_dtype,
                           void* densification_info, void* stream) {
    return rasterizer_forward(r, camera, image, image_dtype, densification_info, 0, stream);
}

int tgs_rasterizer_forward_ex(tgs_rasterizer* r, const tgs_camera* camera, void* image, int32_t image_dtype,
                              void* densification_info, int32_t flags, void* stream) {
    return rasterizer_forward(r, camera, image, image_dtype, densification_info, flags, stream);
}

int tgs_rasterizer_reserve(tgs_rasterizer* r, int64_t max_instances, int32_t grid_tiles, void* stream) {
    if (!r) return fail(TGS_ERR_INVALID, "rasterizer is NULL");
    if (max_instances < 1 || max_instances > (int64_t)0xffffffffll || grid_tiles < 1 ||
        (uint32_t)grid_tiles > kMaxTiles16)
        return fail(TGS_ERR_INVALID, "reserve: %lld instances, %d tiles", (long long)max_instances, grid_tiles);
    hipStream_t s = (hipStream_t)stream;
    const void* before[5] = {r->ikeys[0].p, r->ivals[0].p, r->ckpt.p, r->items.p, r->records.p};
    TGS_TRY(ensure(r->radix_counts, 4 * (size_t)radix_count_entries(max_instances, false), s));
    TGS_TRY(ensure_status(r, scan_status_entries(radix_count_entries(max_instances, false)), s));
    TGS_TRY(ensure_instances(r, max_instances, (uint32_t)grid_tiles, s));
    const void* after[5] = {r->ikeys[0].p, r->ivals[0].p, r->ckpt.p, r->items.p, r->records.p};
    // grown buffers do not keep the last forward's instance lists and checkpoints
    if (memcmp(before, after, sizeof(before)) != 0) r->fwd_done = false;
    r->inst_cap = max_instances;
    return TGS_OK;
}

int tgs_rasterizer_status(tgs_rasterizer* r, int32_t clear_capacity_flag, void* stream) {
    if (!r) return fail(TGS_ERR_INVALID, "rasterizer is NULL");
    hipStream_t s = (hipStream_t)stream;
    uint32_t w[3] = {0, 0, 0};
    TGS_HIP(hipMemcpyAsync(w, r->bin_ctl.p, sizeof(w), hipMemcpyDeviceToHost, s));
    TGS_HIP(hipStreamSynchronize(s));
    if (r->fwd_done && r->counts_on_device) {
        r->V = w[0];
        r->I = w[1];
        r->counts_on_device = false;
    }
    if (w[2] & kErrCapacity) {
        if (clear_capacity_flag) launch_clear_err_bits(r->bin_ctl.as<BinCtl>(), kErrCapacity, s);
        TGS_CHECK_LAUNCH();
        return fail(TGS_ERR_CAPACITY, "forward needed %u instances, %lld reserved", w[1], (long long)r->inst_cap);
    }
    if (w[2]) {
        launch_clear_err_bits(r->bin_ctl.as<BinCtl>(), w[2], s);   // reported once
        TGS_CHECK_LAUNCH();
        return fail(TGS_ERR_STATE, "binning failed on the device (error flags 0x%x)", w[2]);
    }
    return TGS_OK;
}

int tgs_rasterizer_backward(tgs_rasterizer* r, const void* grad_image, const void* image, const tgs_gaussians* grads,
                            void* densification_info, void* stream) {
    return tgs_rasterizer_backward_ex(r, grad_image, image, grads, densification_info, 0, stream);
}

int tgs_rasterizer_backward_ex(tgs_rasterizer* r, const void* grad_image, const void* image,
                               const tgs_gaussians* grads, void* densification_info, int32_t flags, void* stream) {
    if (!r) return fail(TGS_ERR_INVALID, "rasterizer is NULL");
    if (!r->has_g || !grads) return fail(TGS_ERR_STATE, "Gaussians or gradient gaussians not set");
    if (!r->fwd_done) return fail(TGS_ERR_STATE, "backward called without a preceding forward");
    TGS_TRY(check_gaussians(grads, true));
    if (grads->n != r->g.n) return fail(TGS_ERR_INVALID, "gradient count %lld != %lld", (long long)grads->n,
                                        (long long)r->g.n);
    if (!grad_image || !image) return fail(TGS_ERR_INVALID, "grad_image / image is NULL");
    hipStream_t s = (hipStream_t)stream;
    const int64_t n = r->n;
    TGS_TRY(ensure(r->grad2d, sizeof(float) * kGradStride * (size_t)(n > 0 ? n : 1), s));
    TGS_TRY(ensure(r->heavy, sizeof(uint4) * (size_t)(n > 0 ? n : 1), s));
    TGS_TRY(ensure(r->live, sizeof(uint4) * (size_t)(n > 0 ? n : 1), s));
    if (flags & ~(TGS_BACKWARD_ASSIGN | TGS_BACKWARD_SPARSE | TGS_BACKWARD_POSE | TGS_BACKWARD_KEEP_2D))
        return fail(TGS_ERR_INVALID, "unknown backward flags 0x%x", flags);
    if ((flags & TGS_BACKWARD_ASSIGN) && (flags & TGS_BACKWARD_SPARSE))
        return fail(TGS_ERR_INVALID, "TGS_BACKWARD_ASSIGN and TGS_BACKWARD_SPARSE are exclusive");
    const int mode = (flags & TGS_BACKWARD_SPARSE) ? kGradSparse : ((flags & TGS_BACKWARD_ASSIGN) ? kGradAssign : kGradAccumulate);
    if (mode == kGradSparse) TGS_TRY(ensure(r->row_mask, (size_t)(n > 0 ? n : 1), s));
    r->row_mask_valid = false;
    r->pose_valid = false;
    const bool pose = (flags & TGS_BACKWARD_POSE) != 0;
    const bool keep2d = (flags & TGS_BACKWARD_KEEP_2D) != 0;
    r->grad2d_valid = false;
    if (pose) {
        TGS_TRY(ensure(r->pose_partial, sizeof(float) * 12 * (size_t)std::max<int64_t>(pb_chunks(n), 1), s));
        TGS_TRY(ensure(r->pose_grad, sizeof(float) * 16, s));
    }
    const CamParams& cam = r->cam;
    BinCtl* ctl = r->bin_ctl.as<BinCtl>();
    if (!r->bwd_queues_clear)   // a second backward after one forward: clear the queue counters again
        launch_fill_u32(ctl->bwd_queue, 0u, kBwdCtlWords, s);
    {
        StageScope sc(ST_BLENDB, s);
        if (r->fgs16)   // fastgs.cu:273-274: half image and gradient image
            launch_blend16_backward(cam, r->ivals[r->isel].as<uint32_t>(), r->mean2d.as<float2>(),
                                    r->color.as<uint4>(), (const uint16_t*)image, (const uint16_t*)grad_image,
                                    r->ckpt.as<uint2>(), r->items.as<uint4>(), ctl, r->rec_count.as<uint32_t>(),
                                    r->first_slot.as<uint32_t>(), r->records.as<float4>(), s);
        else
            launch_blend_backward(cam, r->ivals[r->isel].as<uint32_t>(), r->iranks.as<uint16_t>(),
                                  r->mean2d.as<float2>(), r->conic_opacity.as<float4>(), r->color.as<float4>(),
                                  (const float*)image, (const float*)grad_image, r->n_contrib.as<uint32_t>(),
                                  r->ckpt.as<float4>(), r->items.as<uint4>(), ctl, r->rec_bits.as<uint32_t>(),
                                  r->rec_mask.as<uint32_t>(), r->rec_count.as<uint32_t>(),
                                  r->first_slot.as<uint32_t>(), r->records.as<float4>(),
                                  densification_info != nullptr, s);
    }
    r->bwd_queues_clear = false;
    TGS_CHECK_LAUNCH();
    GradView gv{(float*)grads->means, (float*)grads->scales, (float*)grads->rotations, (float*)grads->opacities,
                (float*)grads->sh0, (float*)grads->sh_rest};
    {
        StageScope sc(ST_PREB, s);
        launch_preprocess_backward(view_of(r->g), cam, r->n_touched.as<uint32_t>(), r->conic_opacity.as<float4>(),
                                   r->rec_count.as<uint32_t>(), r->rec_mask.as<uint32_t>(),
                                   r->rec_bits.as<uint32_t>(), r->tile_sort_cap,
                                   r->first_slot.as<uint32_t>(), r->records.as<float4>(),
                                   r->grad2d.as<float>(), gv, (float*)densification_info, mode,
                                   r->row_mask.as<uint8_t>(), r->live.as<uint4>(), r->heavy.as<uint4>(),
                                   pose ? r->pose_partial.as<float>() : nullptr,
                                   pose ? r->pose_grad.as<float>() : nullptr, keep2d, r->fgs16, s);
    }
    TGS_CHECK_LAUNCH();
    r->row_mask_valid = mode == kGradSparse;
    r->pose_valid = pose;
    r->grad2d_valid = keep2d;
    return TGS_OK;
}

int tgs_rasterizer_grad_w2c(tgs_rasterizer* r, float* w2c_grad, void* stream) {
    if (!r || !w2c_grad) return fail(TGS_ERR_INVALID, "NULL argument");
    if (!r->pose_valid) return fail(TGS_ERR_STATE, "no TGS_BACKWARD_POSE backward since the last forward");
    hipStream_t s = (hipStream_t)stream;
    TGS_HIP(hipMemcpyAsync(w2c_grad, r->pose_grad.p, sizeof(float) * 16, hipMemcpyDeviceToHost, s));
    TGS_HIP(hipStreamSynchronize(s));
    return TGS_OK;
}

int tgs_rasterizer_backward_rows(tgs_rasterizer* r, const uint8_t** rows, void* stream) {
    if (!r || !rows) return fail(TGS_ERR_INVALID, "NULL argument");
    if (!r->fwd_done) return fail(TGS_ERR_STATE, "backward rows asked for without a preceding forward");
    hipStream_t s = (hipStream_t)stream;
    const int64_t n = r->n;
    const int64_t words = (n + 3) / 4;
    TGS_TRY(ensure(r->bwd_rows, (size_t)std::max<int64_t>(words, 1) * 4, s));
    if (!r->bwd_rows_valid) {
        launch_fill_u32(r->bwd_rows.as<uint32_t>(), 0u, std::max<int64_t>(words, 1), s);
        launch_backward_rows(r->items.as<uint4>(), r->ivals[r->isel].as<uint32_t>(), r->bin_ctl.as<BinCtl>(),
                             r->bwd_rows.as<uint8_t>(), s);
        TGS_CHECK_LAUNCH();
        r->bwd_rows_valid = true;
    }
    *rows = r->bwd_rows.as<uint8_t>();
    return TGS_OK;
}

int tgs_rasterizer_grad_row_mask(tgs_rasterizer* r, const uint8_t** mask) {
    if (!r || !mask) return fail(TGS_ERR_INVALID, "NULL argument");
    if (!r->row_mask_valid) return fail(TGS_ERR_STATE, "no TGS_BACKWARD_SPARSE backward since the last forward");
    *mask = r->row_mask.as<uint8_t>();
    return TGS_OK;
}

// V and I of a forward that did not wait for them: read from the device
// once the work queued so far has finished.
static int sync_counts(tgs_rasterizer* r) {
    if (!r->counts_on_device) return TGS_OK;
    uint32_t w[2] = {0, 0};
    TGS_HIP(hipDeviceSynchronize());
    TGS_HIP(hipMemcpy(w, r->bin_ctl.p, sizeof(w), hipMemcpyDeviceToHost));
    r->V = w[0];
    r->I = w[1];
    r->counts_on_device = false;
    return TGS_OK;
}

int tgs_rasterizer_counts(tgs_rasterizer* r, int64_t* n_visible, int64_t* n_instances, int64_t* n_tiles) {
    if (!r) return fail(TGS_ERR_INVALID, "rasterizer is NULL");
    if (!r->fwd_done) return fail(TGS_ERR_STATE, "no forward yet");
    TGS_TRY(sync_counts(r));
    if (n_visible) *n_visible = r->V;
    if (n_instances) *n_instances = r->I;
    if (n_tiles) *n_tiles = (int64_t)r->cam.grid_w * r->cam.grid_h;
    return TGS_OK;
}

int tgs_rasterizer_debug_view(tgs_rasterizer* r, tgs_debug_view* out) {
    if (!r || !out) return fail(TGS_ERR_INVALID, "NULL argument");
    if (!r->fwd_done) return fail(TGS_ERR_STATE, "no forward yet");
    TGS_TRY(sync_counts(r));
    out->n_touched = r->n_touched.as<uint32_t>();
    out->bounds = r->erec.as<uint32_t>();
    out->mean2d = r->mean2d.as<float>();
    out->conic_opacity = r->conic_opacity.as<float>();
    out->color = r->color.as<float>();
    out->depth_sorted_keys = r->pkeys[r->psel].as<uint32_t>();
    out->depth_key_base = r->depth_key_base;
    out->depth_sorted_prims = r->pvals[r->psel].as<uint32_t>();
    if (r->ikeys_from_ranges) {   // the tile sort kept its keys only as ranges: written out here
        const uint32_t T = r->cam.grid_w * r->cam.grid_h;
        TGS_HIP(hipDeviceSynchronize());
        launch_keys_from_ranges(r->ranges.as<uint2>(), T, r->tile_sort_cap, r->ikeys[r->isel].as<uint32_t>(), nullptr);
        TGS_HIP(hipGetLastError());
        TGS_HIP(hipDeviceSynchronize());
        r->ikeys_from_ranges = false;
    }
    out->instance_tiles = r->ikeys[r->isel].as<uint32_t>();
    out->instance_prims = r->ivals[r->isel].as<uint32_t>();
    out->tile_ranges = r->ranges.as<uint32_t>();
    out->n_contrib = r->n_contrib.as<uint32_t>();
    out->tile_max = r->tile_max.as<uint32_t>();
    // the summed 2D gradients exist only after a TGS_BACKWARD_KEEP_2D backward
    out->grad2d = r->grad2d_valid ? r->grad2d.as<float>() : nullptr;
    out->n_visible = r->V;
    // a no-sync forward past its capacity counted more instances than its
    // buffers hold; the view covers the ones the tile sort kept (the true
    // count stays with tgs_rasterizer_counts)
    out->n_instances = std::min<int64_t>(r->I, r->tile_sort_cap);
    out->n_tiles = (int64_t)r->cam.grid_w * r->cam.grid_h;
    out->image_dtype = r->fgs16 ? TGS_DTYPE_FLOAT16 : TGS_DTYPE_FLOAT32;
    out->first_slot = r->first_slot.as<uint32_t>();
    out->records = r->records.as<float>();
    out->instance_ranks = r->fgs16 ? nullptr : r->iranks.as<uint16_t>();
    out->record_bits = r->fgs16 ? nullptr : r->rec_bits.as<uint32_t>();
    return TGS_OK;
}

// ------------------------------------------------------------------ losses

int tgs_loss_create(const char* type, tgs_loss** out) {
    if (!out) return fail(TGS_ERR_INVALID, "out is NULL");
    *out = nullptr;
    std::string t = type ? type : "";
    for (auto& ch : t) ch = (char)tolower(ch);
    int kind;
    if (t == "l1")
        kind = 0;
    else if (t == "fused_ssim")
        kind = 1;
    else
        return fail(TGS_ERR_UNSUPPORTED, "Unknown loss type: %s", type ? type : "(null)");
    tgs_loss* l = new tgs_loss();
    l->type = kind;
    *out = l;
    return TGS_OK;
}

int tgs_loss_destroy(tgs_loss* l) {
    if (!l) return TGS_OK;
    (void)hipDeviceSynchronize();
    for (auto& b : l->dm) release(b);
    delete l;
    return TGS_OK;
}

// One fused forward / SSIM backward pair for either image type.
static void loss_forward(bool f16, const tgs_loss_context* c, float c1, float c2, float s_ssim, float s_l1,
                         bool assign, void* loss, void* grad, float* d0, float* d1, float* d2, hipStream_t s) {
    if (f16)
        launch_l1_ssim_forward_f16(c->width, c->height, c1, c2, s_ssim, s_l1, assign, c->pred, c->target, loss, grad,
                                   d0, d1, d2, s);
    else
        launch_l1_ssim_forward(c->width, c->height, c1, c2, s_ssim, s_l1, assign, (const float*)c->pred,
                               (const float*)c->target, (float*)loss, (float*)grad, d0, d1, d2, s);
}
static void loss_ssim_backward(bool f16, const tgs_loss_context* c, float s_ssim, const float* d0, const float* d1,
                               const float* d2, hipStream_t s) {
    if (f16)
        launch_ssim_backward_f16(c->width, c->height, s_ssim, c->pred, c->target, c->grad, d0, d1, d2, s);
    else
        launch_ssim_backward(c->width, c->height, s_ssim, (const float*)c->pred, (const float*)c->target,
                             (float*)c->grad, d0, d1, d2, s);
}

int tgs_loss_evaluate(tgs_loss* l, const tgs_loss_context* c, float scale, void* stream) {
    if (!l || !c) return fail(TGS_ERR_INVALID, "NULL argument");
    // l1.cu:109-151, fused_ssim.cu:797-916: float32 and float16 images
    if (c->dtype != TGS_DTYPE_FLOAT32 && c->dtype != TGS_DTYPE_FLOAT16)
        return fail(TGS_ERR_UNSUPPORTED, "loss dtype %d: float32 or float16 images only", c->dtype);
    const bool f16 = c->dtype == TGS_DTYPE_FLOAT16;
    if (!c->pred || !c->target) return fail(TGS_ERR_INVALID, "pred / target is NULL");
    if (c->width == 0 || c->height == 0 || c->channel == 0) return fail(TGS_ERR_INVALID, "empty image");
    hipStream_t s = (hipStream_t)stream;
    const uint32_t tw = (c->width + 7u) >> 3, th = (c->height + 7u) >> 3;
    const int64_t padded = (int64_t)tw * th * 64 * c->channel;
    if (l->type == 0) {
        // l1.cu:117-121: scale / (W * H * C)
        const int npix = (int)(c->width * c->height * c->channel);
        StageScope sc(ST_L1, s);
        if (f16)
            launch_l1_f16(c->pred, c->target, c->loss, c->grad, padded, scale / (float)npix, s);
        else
            launch_l1((const float*)c->pred, (const float*)c->target, (float*)c->loss, (float*)c->grad, padded,
                      scale / (float)npix, s);
        TGS_CHECK_LAUNCH();
        return TGS_OK;
    }
    if (c->channel != 3) return fail(TGS_ERR_UNSUPPORTED, "fused_ssim needs 3 channels");
    // fused_ssim.cu:811: scale / (H * W)
    const float actual = scale / (float)(int)(c->height * c->width);
    const float C1 = 0.01f * 0.01f, C2 = 0.03f * 0.03f;
    StageScope sc(ST_SSIM, s);
    if (c->grad) {
        for (auto& b : l->dm) TGS_TRY(ensure(b, sizeof(float) * (size_t)padded, s));
        loss_forward(f16, c, C1, C2, actual, 0.0f, false, c->loss, nullptr, l->dm[0].as<float>(),
                     l->dm[1].as<float>(), l->dm[2].as<float>(), s);
        loss_ssim_backward(f16, c, actual, l->dm[0].as<float>(), l->dm[1].as<float>(), l->dm[2].as<float>(), s);
    } else {
        loss_forward(f16, c, C1, C2, actual, 0.0f, false, c->loss, nullptr, nullptr, nullptr, nullptr, s);
    }
    TGS_CHECK_LAUNCH();
    return TGS_OK;
}

int tgs_loss_l1_ssim(tgs_loss* l, const tgs_loss_context* c, float l1_scale, float ssim_scale, int32_t flags,
                     void* stream) {
    if (!l || !c) return fail(TGS_ERR_INVALID, "NULL argument");
    if (c->dtype != TGS_DTYPE_FLOAT32 && c->dtype != TGS_DTYPE_FLOAT16)
        return fail(TGS_ERR_UNSUPPORTED, "loss dtype %d: float32 or float16 images only", c->dtype);
    const bool f16 = c->dtype == TGS_DTYPE_FLOAT16;
    if (!c->pred || !c->target) return fail(TGS_ERR_INVALID, "pred / target is NULL");
    if (c->width == 0 || c->height == 0) return fail(TGS_ERR_INVALID, "empty image");
    if (c->channel != 3) return fail(TGS_ERR_UNSUPPORTED, "fused L1 + SSIM needs 3 channels");
    if (flags & ~TGS_LOSS_ASSIGN) return fail(TGS_ERR_INVALID, "unknown loss flags 0x%x", flags);
    hipStream_t s = (hipStream_t)stream;
    const bool assign = (flags & TGS_LOSS_ASSIGN) != 0;
    const uint32_t tw = (c->width + 7u) >> 3, th = (c->height + 7u) >> 3;
    const int64_t padded = (int64_t)tw * th * 64 * 3;
    // the two reference normalisations: l1.cu:117-121 (W H C), fused_ssim.cu:811 (H W)
    const float s_l1 = l1_scale / (float)(int)(c->width * c->height * 3u);
    const float s_ssim = ssim_scale / (float)(int)(c->height * c->width);
    const float C1 = 0.01f * 0.01f, C2 = 0.03f * 0.03f;
    StageScope sc(ST_SSIM, s);
    if (c->grad) {
        for (auto& b : l->dm) TGS_TRY(ensure(b, sizeof(float) * (size_t)padded, s));
        loss_forward(f16, c, C1, C2, s_ssim, s_l1, assign, c->loss, c->grad, l->dm[0].as<float>(),
                     l->dm[1].as<float>(), l->dm[2].as<float>(), s);
        loss_ssim_backward(f16, c, s_ssim, l->dm[0].as<float>(), l->dm[1].as<float>(), l->dm[2].as<float>(), s);
    } else {
        loss_forward(f16, c, C1, C2, s_ssim, s_l1, assign, c->loss, nullptr, nullptr, nullptr, nullptr, s);
    }
    TGS_CHECK_LAUNCH();
    return TGS_OK;
}

int tgs_psnr(const tgs_loss_context* c, float* psnr, void* stream) {
    if (!c || !psnr || !c->pred || !c->target) return fail(TGS_ERR_INVALID, "NULL argument");
    // psnr.cu:72-128: float32 and float16 images
    if (c->dtype != TGS_DTYPE_FLOAT32 && c->dtype != TGS_DTYPE_FLOAT16)
        return fail(TGS_ERR_UNSUPPORTED, "PSNR: float32 or float16 images only");
    if (c->width == 0 || c->height == 0 || c->channel == 0) return fail(TGS_ERR_INVALID, "empty image");
    hipStream_t s = (hipStream_t)stream;
    static thread_local DevBuf scratch;
    TGS_TRY(ensure(scratch, sizeof(double) * (size_t)psnr_scratch_doubles(), s));
    const int64_t npad = (int64_t)((c->width + 7u) / 8u) * ((c->height + 7u) / 8u) * 64 * c->channel;
    if (c->dtype == TGS_DTYPE_FLOAT16)
        launch_sq_diff_sum_f16(c->pred, c->target, npad, scratch.as<double>(), s);
    else
        launch_sq_diff_sum((const float*)c->pred, (const float*)c->target, npad, scratch.as<double>(), s);
    TGS_CHECK_LAUNCH();
    double sum = 0.0;
    TGS_HIP(hipMemcpyAsync(&sum, scratch.as<double>() + psnr_scratch_doubles() - 1, sizeof(double),
                           hipMemcpyDeviceToHost, s));
    TGS_HIP(hipStreamSynchronize(s));
    const float mse = (float)sum / (float)((uint64_t)c->width * c->height * c->channel);
    *psnr = mse == 0.0f ? 100.0f : -10.0f * log10f(mse);
    return TGS_OK;
}

// ------------------------------------------------------------------ SimpleAdam

static void default_adam_params(tgs_adam_params& p) {
    // SimpleAdamParameters (simple_adam.hpp:8-27) and GaussianOptimizationParams (optim.hpp:12-24)
    p.beta1 = 0.9f;
    p.beta2 = 0.999f;
    p.epsilon = 1e-8f;
    p.means_lr = 1.6e-4f;
    p.shs_lr = 2.5e-3f;
    p.opacities_lr = 5.0e-2f;
    p.scales_lr = 5.0e-3f;
    p.rotations_lr = 1.0e-3f;
    p.max_grad_1 = 1.0f;
    p.opacities_l1 = 0.0f;
    p.scales_l1 = 0.0f;
    p.decay_mean = 1;
}

static const int kGroupMult[6] = {3, 1, 4, 3, 3, 45};

int tgs_adam_create(const tgs_gaussians* params, const tgs_gaussians* grads, tgs_adam** out) {
    if (!out) return fail(TGS_ERR_INVALID, "out is NULL");
    *out = nullptr;
    TGS_TRY(check_gaussians(params, false));
    TGS_TRY(check_gaussians(grads, true));
    if (params->n != grads->n)
        return fail(TGS_ERR_INVALID, "SimpleAdam::step: gaussians and gaussians_grad must have same size");
    tgs_adam* a = new tgs_adam();
    a->params = *params;
    a->grads = *grads;
    a->rows = params->n;
    default_adam_params(a->p);
    for (int k = 0; k < 6; ++k) {
        const size_t bytes = sizeof(float) * (size_t)kGroupMult[k] * (size_t)(params->n > 0 ? params->n : 1);
        if (ensure(a->m1[k], bytes, nullptr) != TGS_OK || ensure(a->m2[k], bytes, nullptr) != TGS_OK ||
            hipMemset(a->m1[k].p, 0, a->m1[k].bytes) != hipSuccess ||
            hipMemset(a->m2[k].p, 0, a->m2[k].bytes) != hipSuccess) {
            for (int q = 0; q < 6; ++q) {
                release(a->m1[q]);
                release(a->m2[q]);
            }
            delete a;
            return fail(TGS_ERR_HIP, "moment allocation failed");
        }
    }
    *out = a;
    return TGS_OK;
}

int tgs_adam_destroy(tgs_adam* a) {
    if (!a) return TGS_OK;
    (void)hipDeviceSynchronize();
    for (int k = 0; k < 6; ++k) {
        release(a->m1[k]);
        release(a->m2[k]);
    }
    release(a->dev_state);
    delete a;
    return TGS_OK;
}

int tgs_adam_set_params(tgs_adam* a, const tgs_adam_params* p) {
    if (!a || !p) return fail(TGS_ERR_INVALID, "NULL argument");
    a->p = *p;
    return TGS_OK;
}

int tgs_adam_get_params(tgs_adam* a, tgs_adam_params* p) {
    if (!a || !p) return fail(TGS_ERR_INVALID, "NULL argument");
    *p = a->p;
    return TGS_OK;
}

int tgs_adam_set_lr(tgs_adam* a, float lr) {
    if (!a) return fail(TGS_ERR_INVALID, "NULL argument");
    a->global_lr = lr;
    return TGS_OK;
}

float tgs_adam_get_lr(tgs_adam* a) { return a ? a->global_lr : 0.0f; }

int tgs_adam_set_gaussians(tgs_adam* a, const tgs_gaussians* params, const tgs_gaussians* grads) {
    if (!a) return fail(TGS_ERR_INVALID, "NULL argument");
    TGS_TRY(check_gaussians(params, false));
    TGS_TRY(check_gaussians(grads, true));
    if (params->n != a->rows || grads->n != a->rows)
        return fail(TGS_ERR_INVALID, "moments are sized for %lld Gaussians, got %lld / %lld (resize them with "
                    "tgs_adam_gather / tgs_adam_append)", (long long)a->rows, (long long)params->n,
                    (long long)grads->n);
    a->params = *params;
    a->grads = *grads;
    return TGS_OK;
}

int tgs_adam_step(tgs_adam* a, float scale, void* stream) { return tgs_adam_step_ex(a, scale, nullptr, 0, stream); }

int tgs_adam_step_masked(tgs_adam* a, float scale, const uint8_t* row_mask, void* stream) {
    return tgs_adam_step_ex(a, scale, row_mask, 0, stream);
}

// The device-step count (TGS_ADAM_DEVICE_STEP) becomes the host's: graph
// replays advance only the device count. Waits for the stream.
static int adam_sync_steps(tgs_adam* a, hipStream_t s) {
    uint32_t w = 0;
    TGS_HIP(hipMemcpyAsync(&w, a->dev_state.p, sizeof(w), hipMemcpyDeviceToHost, s));
    TGS_HIP(hipStreamSynchronize(s));
    a->steps = w;
    return TGS_OK;
}

int tgs_adam_step_ex(tgs_adam* a, float scale, const uint8_t* row_mask, int32_t flags, void* stream) {
    if (!a) return fail(TGS_ERR_INVALID, "NULL argument");
    if (flags & ~(TGS_ADAM_DEVICE_STEP | TGS_ADAM_ROWS_UNMARKED | TGS_ADAM_ROWS_MARKED | TGS_ADAM_SAME_STEP))
        return fail(TGS_ERR_INVALID, "unknown Adam step flags 0x%x", flags);
    const int rows_sel = (flags & TGS_ADAM_ROWS_UNMARKED) ? kAdamRowsUnmarked
                                                          : ((flags & TGS_ADAM_ROWS_MARKED) ? kAdamRowsMarked : 0);
    if ((flags & TGS_ADAM_ROWS_UNMARKED) && (flags & TGS_ADAM_ROWS_MARKED))
        return fail(TGS_ERR_INVALID, "TGS_ADAM_ROWS_UNMARKED and TGS_ADAM_ROWS_MARKED are exclusive");
    if (rows_sel && !row_mask) return fail(TGS_ERR_INVALID, "a row selection needs the row mask");
    const bool dev = (flags & TGS_ADAM_DEVICE_STEP) != 0;
    const bool same = (flags & TGS_ADAM_SAME_STEP) != 0;
    if (same && (a->steps == 0 || dev != a->last_dev || (dev && !a->dev_seeded)))
        return fail(TGS_ERR_STATE, "TGS_ADAM_SAME_STEP needs a step of the same mode before it");
    hipStream_t hs = (hipStream_t)stream;
    // graph replays advance only the device count: a host-counted step after
    // device steps continues from it (one wait on the stream)
    if (!dev && a->dev_seeded) TGS_TRY(adam_sync_steps(a, hs));
    if (dev && !same) {
        TGS_TRY(ensure(a->dev_state, 4 * (size_t)kAdamStateWords, hs));
        if (!a->dev_seeded) {   // the device count starts from the host's
            if (a->steps > 0xfffffffell) return fail(TGS_ERR_INVALID, "step count beyond 32 bits");
            launch_adam_seed_steps(a->dev_state.as<uint32_t>(), (uint32_t)a->steps, a->p.beta1, a->p.beta2, hs);
            a->dev_seeded = true;
        } else if (a->p.beta1 != a->dev_beta1 || a->p.beta2 != a->dev_beta2) {
            // betas changed since: the stored corrections again, at the device count
            launch_adam_rebeta(a->dev_state.as<uint32_t>(), a->p.beta1, a->p.beta2, hs);
        }
        a->dev_beta1 = a->p.beta1;
        a->dev_beta2 = a->p.beta2;
    } else if (!dev) {
        a->dev_seeded = false;   // a later device step restarts from the host count
    }
    a->last_dev = dev;
    const int64_t n = a->params.n;
    if (!same) a->steps += 1;
    // simple_adam.cu:475-480: bias corrections in double, rounded to float
    const double st = (double)a->steps;
    const float bc1 = (float)(1.0 - pow((double)a->p.beta1, st));
    const float bc2 = (float)sqrt(1.0 - pow((double)a->p.beta2, st));
    const float g_scale = a->p.decay_mean ? 1.0f / (float)(n > 0 ? n : 1) : 1.0f;
    const float glr = a->global_lr;
    AdamArgs args;
    memset(&args, 0, sizeof(args));
    args.n_groups = 6;
    args.beta1 = a->p.beta1;
    args.beta2 = a->p.beta2;
    args.eps = a->p.epsilon;
    args.grad_scale = scale;
    args.bc1 = bc1;
    args.bc2_sqrt = bc2;
    args.max_grad = a->p.max_grad_1;
    args.row_mask = row_mask;
    args.row_select = rows_sel;
    args.dev_bc = dev ? a->dev_state.as<uint32_t>() : nullptr;
    args.dev_advance = dev && !same;   // the Adam launch advances the device count itself
    void* th[6] = {a->params.means, a->params.opacities, a->params.rotations, a->params.scales, a->params.sh0,
                   a->params.sh_rest};
    const float* gr[6] = {(const float*)a->grads.means, (const float*)a->grads.opacities,
                          (const float*)a->grads.rotations, (const float*)a->grads.scales,
                          (const float*)a->grads.sh0, (const float*)a->grads.sh_rest};
    // learning rates as formed in simple_adam.cu:493,508,524,540,556,571
    const float lrs[6] = {a->p.means_lr * a->params.scene_scale * glr, a->p.opacities_lr * glr,
                          a->p.rotations_lr * glr, a->p.scales_lr * glr, a->p.shs_lr * glr,
                          a->p.shs_lr * 0.05f * glr};
    for (int k = 0; k < 6; ++k) {
        AdamGroup& g = args.groups[k];
        g.theta = th[k];
        g.grad = gr[k];
        g.m1 = a->m1[k].as<float>();
        g.m2 = a->m2[k].as<float>();
        g.count = (int64_t)kGroupMult[k] * n;
        g.lr = lrs[k];
        g.theta_half = (k >= 4 && a->params.sh_dtype == TGS_DTYPE_FLOAT16) ? 1 : 0;
        g.lerp_form = (k == 1) ? 1 : 0;
        g.decay_kind = (k == 1) ? 1 : (k == 3 ? 2 : 0);
        g.decay_coef = (k == 1) ? a->p.opacities_l1 * g_scale : (k == 3 ? a->p.scales_l1 * g_scale : 0.0f);
        g.row_width = kGroupMult[k];
    }
    {
        StageScope sc(ST_ADAM, (hipStream_t)stream);
        launch_adam(args, (hipStream_t)stream);
    }
    TGS_CHECK_LAUNCH();
    return TGS_OK;
}

int tgs_adam_reset(tgs_adam* a, void* stream) {
    if (!a) return fail(TGS_ERR_INVALID, "NULL argument");
    for (int k = 0; k < 6; ++k) {
        launch_fill_u32(a->m1[k].as<uint32_t>(), 0u, (int64_t)(a->m1[k].bytes / 4), (hipStream_t)stream);
        launch_fill_u32(a->m2[k].as<uint32_t>(), 0u, (int64_t)(a->m2[k].bytes / 4), (hipStream_t)stream);
    }
    TGS_CHECK_LAUNCH();
    a->steps = 0;
    a->dev_seeded = false;
    return TGS_OK;
}

int64_t tgs_adam_global_steps(tgs_adam* a) {
    if (!a) return -1;
    // device steps may have run (graph replays) that the host did not count
    if (a->dev_seeded && (hipDeviceSynchronize() != hipSuccess || adam_sync_steps(a, nullptr) != TGS_OK)) return -1;
    return a->steps;
}

int tgs_adam_device_steps(tgs_adam* a, int64_t* steps, void* stream) {
    if (!a || !steps) return fail(TGS_ERR_INVALID, "NULL argument");
    if (a->dev_seeded) TGS_TRY(adam_sync_steps(a, (hipStream_t)stream));
    *steps = a->steps;
    return TGS_OK;
}

int tgs_adam_moments(tgs_adam* a, int32_t group, float** first, float** second) {
    if (!a || group < 0 || group >= 6) return fail(TGS_ERR_INVALID, "bad group");
    if (first) *first = a->m1[group].as<float>();
    if (second) *second = a->m2[group].as<float>();
    return TGS_OK;
}

}  // extern "C"

// Replaces every moment buffer by one of `rows` rows built by `fill(k, dst)`
// (k: group); the old buffers are released once the stream has finished.
template <typename F>
static int adam_rebuild(tgs_adam* a, int64_t rows, hipStream_t s, F fill) {
    DevBuf n1[6], n2[6];
    for (int k = 0; k < 6; ++k) {
        const size_t bytes = sizeof(float) * (size_t)kGroupMult[k] * (size_t)(rows > 0 ? rows : 1);
        if (ensure(n1[k], bytes, s) != TGS_OK || ensure(n2[k], bytes, s) != TGS_OK) {
            for (int q = 0; q < 6; ++q) {
                release(n1[q]);
                release(n2[q]);
            }
            return fail(TGS_ERR_HIP, "moment allocation failed");
        }
        fill(k, a->m1[k], n1[k]);
        fill(k, a->m2[k], n2[k]);
    }
    TGS_CHECK_LAUNCH();
    TGS_HIP(hipStreamSynchronize(s));
    for (int k = 0; k < 6; ++k) {
        release(a->m1[k]);
        release(a->m2[k]);
        a->m1[k] = n1[k];
        a->m2[k] = n2[k];
        n1[k] = DevBuf{};
        n2[k] = DevBuf{};
    }
    a->rows = rows;
    return TGS_OK;
}

// Indices of the nonzero flags in index order into `out`; totals of nonzero
// flags and of flags equal to 1. Synchronises the stream.
static int compact_flags(const uint8_t* flags, int64_t n, int32_t* out, int64_t* n_nonzero, int64_t* n_ones,
                         hipStream_t s) {
    *n_nonzero = 0;
    if (n_ones) *n_ones = 0;
    if (n <= 0) return TGS_OK;
    const int64_t chunks = list_chunks(n);
    DevBuf counts, offsets;
    int rc = ensure(counts, sizeof(uint2) * (size_t)chunks, s);
    if (rc == TGS_OK) rc = ensure(offsets, sizeof(uint32_t) * (size_t)chunks, s);
    if (rc != TGS_OK) {
        release(counts);
        release(offsets);
        return rc;
    }
    std::vector<uint2> h(chunks);
    std::vector<uint32_t> off(chunks);
    launch_flag_count(flags, n, counts.as<uint2>(), s);
    hipError_t e = hipMemcpyAsync(h.data(), counts.p, sizeof(uint2) * (size_t)chunks, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e == hipSuccess) {
        uint64_t acc = 0, ones = 0;
        for (int64_t c = 0; c < chunks; ++c) {
            off[c] = (uint32_t)acc;
            acc += h[c].x;
            ones += h[c].y;
        }
        *n_nonzero = (int64_t)acc;
        if (n_ones) *n_ones = (int64_t)ones;
        e = hipMemcpyAsync(offsets.p, off.data(), sizeof(uint32_t) * (size_t)chunks, hipMemcpyHostToDevice, s);
    }
    if (e == hipSuccess) launch_flag_compact(flags, n, offsets.as<uint32_t>(), out, s);
    if (e == hipSuccess) e = hipGetLastError();
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    release(counts);
    release(offsets);
    if (e != hipSuccess) return fail(TGS_ERR_HIP, "flag compaction: %s", hipGetErrorString(e));
    return TGS_OK;
}

extern "C" {

int tgs_adam_gather(tgs_adam* a, const int32_t* rows, int64_t n_rows, void* stream) {
    if (!a || n_rows < 0 || (n_rows > 0 && !rows)) return fail(TGS_ERR_INVALID, "bad argument");
    hipStream_t s = (hipStream_t)stream;
    return adam_rebuild(a, n_rows, s, [&](int k, DevBuf& src, DevBuf& dst) {
        launch_gather_rows(src.p, dst.p, rows, n_rows, 4 * kGroupMult[k], s);
    });
}

int tgs_adam_append(tgs_adam* a, int64_t n_new, void* stream) {
    if (!a || n_new < 0) return fail(TGS_ERR_INVALID, "bad argument");
    hipStream_t s = (hipStream_t)stream;
    const int64_t old = a->rows;
    return adam_rebuild(a, old + n_new, s, [&](int k, DevBuf& src, DevBuf& dst) {
        const int64_t m = kGroupMult[k];
        if (old > 0) (void)hipMemcpyAsync(dst.p, src.p, sizeof(float) * (size_t)(m * old), hipMemcpyDeviceToDevice, s);
        launch_fill_u32(dst.as<uint32_t>() + m * old, 0u, m * n_new, s);
    });
}

// Whether every idx[k], k < n, lies in [0, bound). Synchronises the stream.
static int indices_in_range(const int32_t* idx, int64_t n, int64_t bound, hipStream_t s, bool* ok) {
    *ok = true;
    if (n <= 0) return TGS_OK;
    DevBuf bad;
    TGS_TRY(ensure(bad, sizeof(uint32_t), s));
    uint32_t h = 0;
    launch_fill_u32(bad.as<uint32_t>(), 0u, 1, s);
    launch_check_indices(idx, n, bound, bad.as<uint32_t>(), s);
    hipError_t e = hipGetLastError();
    if (e == hipSuccess) e = hipMemcpyAsync(&h, bad.p, sizeof(h), hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    release(bad);
    if (e != hipSuccess) return fail(TGS_ERR_HIP, "index check: %s", hipGetErrorString(e));
    *ok = h == 0;
    return TGS_OK;
}

int tgs_adam_reset_rows(tgs_adam* a, const int32_t* rows, int64_t n_rows, void* stream) {
    if (!a || n_rows < 0 || (n_rows > 0 && !rows)) return fail(TGS_ERR_INVALID, "bad argument");
    hipStream_t s = (hipStream_t)stream;
    bool ok = true;
    TGS_TRY(indices_in_range(rows, n_rows, a->rows, s, &ok));
    if (!ok) return fail(TGS_ERR_INVALID, "SimpleAdam::reset: an index is outside [0, %lld)", (long long)a->rows);
    for (int k = 0; k < 6; ++k) {
        launch_zero_rows(a->m1[k].p, rows, n_rows, kGroupMult[k], s);
        launch_zero_rows(a->m2[k].p, rows, n_rows, kGroupMult[k], s);
    }
    TGS_CHECK_LAUNCH();
    return TGS_OK;
}

int tgs_adam_reorder(tgs_adam* a, const uint32_t* indices, void* stream) {
    if (!a || (a->rows > 0 && !indices)) return fail(TGS_ERR_INVALID, "bad argument");
    if (a->rows > (int64_t)0x7fffffff) return fail(TGS_ERR_UNSUPPORTED, "reorder of more than 2^31 - 1 rows");
    hipStream_t s = (hipStream_t)stream;
    const int32_t* rows = (const int32_t*)indices;
    bool ok = true;
    TGS_TRY(indices_in_range(rows, a->rows, a->rows, s, &ok));
    if (!ok) return fail(TGS_ERR_INVALID, "SimpleAdam::reorder: an index is outside [0, %lld)", (long long)a->rows);
    return adam_rebuild(a, a->rows, s, [&](int k, DevBuf& src, DevBuf& dst) {
        launch_gather_rows(src.p, dst.p, rows, a->rows, 4 * kGroupMult[k], s);
    });
}

int tgs_adam_reset_opacity(tgs_adam* a, void* stream) {
    if (!a) return fail(TGS_ERR_INVALID, "NULL argument");
    const int64_t words = a->rows > 0 ? a->rows : 0;
    launch_fill_u32(a->m1[1].as<uint32_t>(), 0u, words, (hipStream_t)stream);
    launch_fill_u32(a->m2[1].as<uint32_t>(), 0u, words, (hipStream_t)stream);
    TGS_CHECK_LAUNCH();
    return TGS_OK;
}

// ------------------------------------------------------------------ densification

void tgs_pcg32_seed(tgs_pcg32* rng, uint64_t initstate, uint64_t initseq) {
    if (rng) pcg_seed(rng->state, rng->inc, initstate, initseq);
}

uint32_t tgs_pcg32_next_uint(tgs_pcg32* rng, uint32_t bound) {
    if (!rng) return 0u;
    return bound ? pcg_next_bounded(rng->state, rng->inc, bound) : pcg_next(rng->state, rng->inc);
}

int tgs_random_logistic(tgs_pcg32* rng, int64_t n, float* out, float mean, float stddev, void* stream) {
    if (!rng || n < 0 || (n > 0 && !out)) return fail(TGS_ERR_INVALID, "bad argument");
    launch_random_logistic(rng->state, rng->inc, n, mean, stddev, out, (hipStream_t)stream);
    TGS_CHECK_LAUNCH();
    rng->state = pcg_advance(rng->state, rng->inc, (uint64_t)n);
    return TGS_OK;
}

int tgs_densify_select(const tgs_gaussians* g, const float* densif, float grad_threshold, float scale_threshold,
                       int32_t absgrad, uint8_t* flags, int32_t* src_indices, int64_t* n_duplicate,
                       int64_t* n_split, void* stream) {
    TGS_TRY(check_gaussians(g, false));
    if (!n_duplicate || !n_split || (g->n > 0 && (!densif || !flags || !src_indices)))
        return fail(TGS_ERR_INVALID, "NULL argument");
    hipStream_t s = (hipStream_t)stream;
    launch_densify_select(g->n, (const float4*)densif, (const float*)g->scales, grad_threshold, scale_threshold,
                          absgrad, flags, s);
    TGS_CHECK_LAUNCH();
    int64_t grow = 0, dup = 0;
    TGS_TRY(compact_flags(flags, g->n, src_indices, &grow, &dup, s));
    *n_duplicate = dup;
    *n_split = grow - dup;
    return TGS_OK;
}

int tgs_densify_apply(const tgs_gaussians* g, int64_t n_old, const int32_t* src_indices, int64_t n_grow,
                      const uint8_t* flags, const float* rand6, void* stream) {
    TGS_TRY(check_gaussians(g, false));
    if (n_old < 0 || n_grow < 0 || n_old + n_grow != g->n)
        return fail(TGS_ERR_INVALID, "gaussians hold %lld rows, expected %lld + %lld", (long long)g->n,
                    (long long)n_old, (long long)n_grow);
    if (n_grow > 0 && (!src_indices || !flags || !rand6)) return fail(TGS_ERR_INVALID, "NULL argument");
    launch_densify_apply(n_grow, n_old, src_indices, flags, rand6, (float*)g->means, (float*)g->scales,
                         (float*)g->rotations, (float*)g->opacities, (void*)g->sh0, (void*)g->sh_rest,
                         g->sh_dtype == TGS_DTYPE_FLOAT16 ? kShF16 : kShF32, (hipStream_t)stream);
    TGS_CHECK_LAUNCH();
    return TGS_OK;
}

int tgs_prune_select(const tgs_gaussians* g, const float* densif, int64_t n_info, float opacity_threshold,
                     float scale_limit, float radius_limit, int32_t prune_large, uint8_t* alive,
                     int32_t* kept_indices, int64_t* n_kept, void* stream) {
    TGS_TRY(check_gaussians(g, false));
    if (!n_kept || (g->n > 0 && (!alive || !kept_indices)) || n_info < 0 || (n_info > 0 && !densif))
        return fail(TGS_ERR_INVALID, "NULL argument");
    hipStream_t s = (hipStream_t)stream;
    launch_prune_select(g->n, (const float*)g->opacities, (const float*)g->scales, (const float*)g->rotations,
                        (const float4*)densif, n_info, scale_limit, radius_limit, opacity_threshold, prune_large,
                        alive, s);
    TGS_CHECK_LAUNCH();
    return compact_flags(alive, g->n, kept_indices, n_kept, nullptr, s);
}

int tgs_gaussians_gather(const tgs_gaussians* src, const tgs_gaussians* dst, const int32_t* rows, void* stream) {
    TGS_TRY(check_gaussians(src, false));
    TGS_TRY(check_gaussians(dst, false));
    if (src->sh_dtype != dst->sh_dtype) return fail(TGS_ERR_INVALID, "SH dtypes differ");
    if (dst->n > 0 && !rows) return fail(TGS_ERR_INVALID, "rows is NULL");
    hipStream_t s = (hipStream_t)stream;
    const int64_t n = dst->n;
    launch_gather_rows(src->means, dst->means, rows, n, 12, s);
    launch_gather_rows(src->scales, dst->scales, rows, n, 12, s);
    launch_gather_rows(src->rotations, dst->rotations, rows, n, 16, s);
    launch_gather_rows(src->opacities, dst->opacities, rows, n, 4, s);
    if (src->sh_dtype == TGS_DTYPE_FLOAT16) {
        launch_gather_rows16(src->sh0, dst->sh0, rows, n, 3, s);
        launch_gather_rows16(src->sh_rest, dst->sh_rest, rows, n, 45, s);
    } else {
        launch_gather_rows(src->sh0, dst->sh0, rows, n, 12, s);
        launch_gather_rows(src->sh_rest, dst->sh_rest, rows, n, 180, s);
    }
    TGS_CHECK_LAUNCH();
    return TGS_OK;
}

int tgs_gaussians_reorder(const tgs_gaussians* g, const uint32_t* indices, void* stream) {
    TGS_TRY(check_gaussians(g, false));
    const int64_t n = g->n;
    if (n > 0 && !indices) return fail(TGS_ERR_INVALID, "indices is NULL");
    if (n > (int64_t)0x7fffffff) return fail(TGS_ERR_UNSUPPORTED, "reorder of more than 2^31 - 1 rows");
    if (n == 0) return TGS_OK;
    hipStream_t s = (hipStream_t)stream;
    const int32_t* rows = (const int32_t*)indices;
    bool ok = true;
    TGS_TRY(indices_in_range(rows, n, n, s, &ok));
    if (!ok) return fail(TGS_ERR_INVALID, "GPUGaussian3d::reorder: an index is outside [0, %lld)", (long long)n);
    const bool half = g->sh_dtype == TGS_DTYPE_FLOAT16;
    const size_t shb = half ? 2 : 4;
    void* arr[6] = {g->means, g->scales, g->rotations, g->opacities, g->sh0, g->sh_rest};
    const size_t row_bytes[6] = {12, 12, 16, 4, 3 * shb, 45 * shb};
    DevBuf tmp;
    TGS_TRY(ensure(tmp, row_bytes[5] * (size_t)n, s));
    hipError_t e = hipSuccess;
    for (int k = 0; k < 6 && e == hipSuccess; ++k) {
        if (k >= 4 && half)
            launch_gather_rows16(arr[k], tmp.p, rows, n, (int)(row_bytes[k] / 2), s);
        else
            launch_gather_rows(arr[k], tmp.p, rows, n, (int)row_bytes[k], s);
        e = hipGetLastError();
        if (e == hipSuccess) e = hipMemcpyAsync(arr[k], tmp.p, row_bytes[k] * (size_t)n, hipMemcpyDeviceToDevice, s);
    }
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    release(tmp);
    if (e != hipSuccess) return fail(TGS_ERR_HIP, "GPUGaussian3d::reorder: %s", hipGetErrorString(e));
    return TGS_OK;
}

int tgs_morton_order(const float* means, int64_t n, uint32_t* indices, void* stream) {
    if (n < 0 || (n > 0 && (!means || !indices))) return fail(TGS_ERR_INVALID, "bad argument");
    if (n > (int64_t)0x7fffffff) return fail(TGS_ERR_UNSUPPORTED, "Morton order of more than 2^31 - 1 means");
    if (n == 0) return TGS_OK;
    hipStream_t s = (hipStream_t)stream;
    DevBuf scratch, status, ctl;
    int rc = TGS_OK;
    const int64_t st_entries = scan_status_entries(radix_count_entries(n, true));
    if ((rc = ensure(scratch, sizeof(uint32_t) * (size_t)morton_scratch_words(n), s)) == TGS_OK &&
        (rc = ensure(status, sizeof(uint64_t) * (size_t)std::max<int64_t>(st_entries, 1), s)) == TGS_OK &&
        (rc = ensure(ctl, sizeof(BinCtl), s)) == TGS_OK) {
        // zero status words (not published) and a zero control block (tickets, epoch base, error)
        launch_fill_u32(status.as<uint32_t>(), 0u, (int64_t)(status.bytes / 4), s);
        launch_fill_u32(ctl.as<uint32_t>(), 0u, (int64_t)(sizeof(BinCtl) / 4), s);
        if (morton_order(means, n, indices, scratch.as<uint32_t>(), status.as<uint64_t>(), ctl.as<BinCtl>(), s) != 0)
            rc = fail(TGS_ERR_STATE, "Morton order: radix digit plan");
        uint32_t err = 0;
        hipError_t e = hipGetLastError();
        if (e == hipSuccess) e = hipMemcpyAsync(&err, (const char*)ctl.p + offsetof(BinCtl, err), sizeof(err),
                                                hipMemcpyDeviceToHost, s);
        if (e == hipSuccess) e = hipStreamSynchronize(s);
        if (e != hipSuccess)
            rc = fail(TGS_ERR_HIP, "Morton order: %s", hipGetErrorString(e));
        else if (rc == TGS_OK && err)
            rc = fail(TGS_ERR_STATE, "Morton order: the sort failed on the device (error flags 0x%x)", err);
    }
    release(scratch);
    release(status);
    release(ctl);
    return rc;
}

int tgs_densification_reorder(const void* info, void* out, const uint32_t* indices, int64_t n, void* stream) {
    if (n < 0 || (n > 0 && (!info || !out || !indices))) return fail(TGS_ERR_INVALID, "bad argument");
    if (n > (int64_t)0x7fffffff) return fail(TGS_ERR_UNSUPPORTED, "reorder of more than 2^31 - 1 rows");
    if (info == out) return fail(TGS_ERR_INVALID, "densification reorder: out must not alias info");
    if (n == 0) return TGS_OK;
    hipStream_t s = (hipStream_t)stream;
    bool ok = true;
    TGS_TRY(indices_in_range((const int32_t*)indices, n, n, s, &ok));
    if (!ok) return fail(TGS_ERR_INVALID, "densification reorder: an index is outside [0, %lld)", (long long)n);
    launch_rows16_gather(info, out, indices, n, s);
    TGS_CHECK_LAUNCH();
    return TGS_OK;
}

int tgs_flags_compact(const uint8_t* flags, int64_t n, int32_t* out, int64_t* count, void* stream) {
    if (!count || n < 0 || (n > 0 && (!flags || !out))) return fail(TGS_ERR_INVALID, "bad argument");
    return compact_flags(flags, n, out, count, nullptr, (hipStream_t)stream);
}

int tgs_reset_opacity(const tgs_gaussians* g, float max_opacity, void* stream) {
    TGS_TRY(check_gaussians(g, false));
    launch_reset_opacity((float*)g->opacities, g->n, max_opacity, (hipStream_t)stream);
    TGS_CHECK_LAUNCH();
    return TGS_OK;
}

}  // extern "C"

// ------------------------------------------------------------------ index lists without allocation
//
// tgs_flags_compact_noalloc keeps its per-chunk counts, offsets and totals in
// this file-scope array instead of hipMalloc'd buffers. Every GPU the library
// runs on holds one copy (384 KiB) until the process ends. Its address on a
// device comes from hipGetSymbolAddress, taken once per device on the first
// call there; the array's name itself is only a host-side stand-in. Calls on
// one GPU share the array (each fully writes what it reads before reading
// it), so calls that overlap on one GPU race.
constexpr int64_t kNoAllocMaxFlags = 1ll << 26;
constexpr int64_t kNoAllocChunks = kNoAllocMaxFlags / kListChunkElems;
constexpr int kNoAllocWords = (int)(3 * kNoAllocChunks + 64);   // counts (uint2), offsets, totals
static __device__ __align__(256) uint32_t scratch[kNoAllocWords];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static uint32_t* g_scratch_ptr[kMaxDevices];

// The current device's copy of `scratch`, looked up on the first call there.
static int scratch_on_current_device(uint32_t** out) {
    int dev = -1;
    TGS_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) return fail(TGS_ERR_UNSUPPORTED, "device %d beyond %d devices", dev, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return fail(TGS_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
        g_scratch_ptr[dev] = (uint32_t*)p;
    }
    *out = g_scratch_ptr[dev];
    return TGS_OK;
}

extern "C" {

int tgs_flags_compact_noalloc(const uint8_t* flags, int64_t n, int32_t* out, int64_t* count, void* stream) {
    if (!count || n < 0 || (n > 0 && (!flags || !out))) return fail(TGS_ERR_INVALID, "bad argument");
    if (n > kNoAllocMaxFlags)
        return fail(TGS_ERR_INVALID, "tgs_flags_compact_noalloc: %lld flags, at most %lld", (long long)n,
                    (long long)kNoAllocMaxFlags);
    *count = 0;
    if (n == 0) return TGS_OK;
    hipStream_t s = (hipStream_t)stream;
    uint32_t* base = nullptr;
    TGS_TRY(scratch_on_current_device(&base));
    const int64_t chunks = list_chunks(n);
    uint2* counts = (uint2*)base;
    uint32_t* offsets = base + 2 * kNoAllocChunks;
    uint32_t* totals = offsets + kNoAllocChunks;
    launch_flag_count(flags, n, counts, s);
    launch_chunk_offsets(counts, chunks, offsets, totals, s);
    launch_flag_compact(flags, n, offsets, out, s);
    TGS_CHECK_LAUNCH();
    uint32_t h[2] = {0, 0};
    TGS_HIP(hipMemcpyAsync(h, totals, sizeof(h), hipMemcpyDeviceToHost, s));
    TGS_HIP(hipStreamSynchronize(s));
    *count = h[0];
    return TGS_OK;
}

// ------------------------------------------------------------------ measurement

int tgs_profiling_set(uint32_t stage_mask) {
    g_prof.mask = stage_mask;
    return TGS_OK;
}

int tgs_profiling_read(int32_t stage, double* total_ms, int64_t* count, int32_t reset) {
    if (stage < 0 || stage >= kStageCount) return fail(TGS_ERR_INVALID, "bad stage %d", stage);
    for (EventPair& p : g_prof.pending[stage]) {
        float ms = 0.f;
        TGS_HIP(hipEventSynchronize(p.b));
        TGS_HIP(hipEventElapsedTime(&ms, p.a, p.b));
        g_prof.total_ms[stage] += ms;
        g_prof.count[stage] += 1;
        g_prof.pool.push_back(p);
    }
    g_prof.pending[stage].clear();
    if (total_ms) *total_ms = g_prof.total_ms[stage];
    if (count) *count = g_prof.count[stage];
    if (reset) {
        g_prof.total_ms[stage] = 0.0;
        g_prof.count[stage] = 0;
    }
    return TGS_OK;
}

const char* tgs_stage_name(int32_t stage) {
    return (stage >= 0 && stage < kStageCount) ? kStageNames[stage] : "";
}

int tgs_rasterizer_work_stats(tgs_rasterizer* r, int64_t* fwd_loaded, int64_t* bwd_processed, int32_t reset) {
    (void)reset;
    if (!r) return fail(TGS_ERR_INVALID, "rasterizer is NULL");
    if (!r->fwd_done) return fail(TGS_ERR_STATE, "no forward yet");
    const size_t T = (size_t)r->cam.grid_w * r->cam.grid_h;
    std::vector<uint32_t> loaded(T), tmax(T), ranges(2 * T);
    TGS_HIP(hipDeviceSynchronize());
    if (T) {
        TGS_HIP(hipMemcpy(loaded.data(), r->tile_loaded.p, 4 * T, hipMemcpyDeviceToHost));
        TGS_HIP(hipMemcpy(tmax.data(), r->tile_max.p, 4 * T, hipMemcpyDeviceToHost));
        TGS_HIP(hipMemcpy(ranges.data(), r->ranges.p, 8 * T, hipMemcpyDeviceToHost));
    }
    int64_t fl = 0, bp = 0;
    for (size_t t = 0; t < T; ++t) {
        fl += loaded[t];
        bp += std::min<int64_t>((int64_t)ranges[2 * t + 1] - (int64_t)ranges[2 * t], tmax[t]);
    }
    if (fwd_loaded) *fwd_loaded = fl;
    if (bwd_processed) *bwd_processed = bp;
    return TGS_OK;
}

// ------------------------------------------------------------------ self tests

int tgs_selftest_detmath(int32_t op, const float* in, float* out, int64_t n, void* stream) {
    launch_detmath(op, in, out, n, (hipStream_t)stream);
    TGS_CHECK_LAUNCH();
    return TGS_OK;
}

int tgs_selftest_half(int32_t op, const void* a, const void* b, const void* c, void* out, int64_t n, void* stream) {
    if (n < 0 || (n > 0 && (!a || !out))) return fail(TGS_ERR_INVALID, "bad argument");
    if ((op == 2 || op == 6) && n > 0 && (!b || !c)) return fail(TGS_ERR_INVALID, "bad argument");
    if ((op == 3 || op == 4 || op == 5 || op == 9 || op == 10 || op == 12 || op == 13) && n > 0 && !b)
        return fail(TGS_ERR_INVALID, "bad argument");
    if (op < 0 || op > 14 || (op == 12 && n % 64 != 0)) return fail(TGS_ERR_INVALID, "op %d, n %lld", op, (long long)n);
    launch_halfmath(op, (const uint16_t*)a, (const uint16_t*)b, (const uint16_t*)c, (uint16_t*)out, n,
                    (hipStream_t)stream);
    TGS_CHECK_LAUNCH();
    return TGS_OK;
}

int tgs_selftest_half_div_exhaustive(int64_t* out, void* stream) {
    if (!out) return fail(TGS_ERR_INVALID, "bad argument");
    hipStream_t s = (hipStream_t)stream;
    launch_fill_u32((uint32_t*)out, 0u, 16, s);
    launch_half_div_check((unsigned long long*)out, s);
    TGS_CHECK_LAUNCH();
    return TGS_OK;
}

int tgs_selftest_half_div_blend(int64_t* out, uint32_t b_lo, uint32_t b_hi, void* stream) {
    if (!out || b_lo == 0u || b_lo > b_hi || b_hi >= 0x7c00u) return fail(TGS_ERR_INVALID, "bad argument");
    hipStream_t s = (hipStream_t)stream;
    launch_fill_u32((uint32_t*)out, 0u, 16, s);
    launch_half_div_blend_check((unsigned long long*)out, b_lo, b_hi, s);
    TGS_CHECK_LAUNCH();
    return TGS_OK;
}

int tgs_selftest_clock(double* core_mhz, void* stream) {
    if (!core_mhz) return fail(TGS_ERR_INVALID, "bad argument");
    hipStream_t s = (hipStream_t)stream;
    int dev = 0, cus = 0, wall_khz = 0;
    TGS_HIP(hipGetDevice(&dev));
    TGS_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    TGS_HIP(hipDeviceGetAttribute(&wall_khz, hipDeviceAttributeWallClockRate, dev));
    if (cus <= 0 || wall_khz <= 0) return fail(TGS_ERR_HIP, "no compute units or wall clock rate reported");
    const uint32_t blocks = (uint32_t)cus * 8u;   // eight waves per SIMD
    std::vector<unsigned long long> h(2u * blocks);
    unsigned long long* d = nullptr;
    TGS_HIP(hipMalloc(&d, h.size() * sizeof(unsigned long long)));
    launch_clock_probe(d, blocks, 8192u, s);
    hipError_t e = hipGetLastError();
    if (e == hipSuccess) e = hipMemcpyAsync(h.data(), d, h.size() * sizeof(unsigned long long), hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    (void)hipFree(d);
    if (e != hipSuccess) return fail(TGS_ERR_HIP, "clock probe: %s", hipGetErrorString(e));
    double cycles = 0.0, ticks = 0.0;
    for (uint32_t b = 0; b < blocks; ++b) {
        cycles += (double)h[2u * b];
        ticks += (double)h[2u * b + 1u];
    }
    if (ticks <= 0.0) return fail(TGS_ERR_HIP, "clock probe: no constant-rate ticks");
    *core_mhz = cycles / ticks * (double)wall_khz / 1000.0;
    return TGS_OK;
}

int tgs_selftest_lookback_spins(uint32_t spins) {
    if (set_lookback_spin_limit(spins == 0xffffffffu ? (1u << 22) : spins) != 0)
        return fail(TGS_ERR_HIP, "look-back spin bound: %s", hipGetErrorString(hipGetLastError()));
    return TGS_OK;
}

int tgs_selftest_wave(const uint32_t* in, uint32_t* out, void* stream) {
    launch_wave_selftest(in, out, (hipStream_t)stream);
    TGS_CHECK_LAUNCH();
    return TGS_OK;
}

}  // extern "C"
