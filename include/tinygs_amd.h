/* tinygs_amd — C ABI of the MI355X (gfx950) FastGS training path.
 *
 * This is the drop-in boundary for tinygs's rasterizer / loss / optimizer
 * plugin interfaces. Every entry point takes plain device pointers, sizes and
 * a hipStream_t (passed as void*), returns a status code (0 = success) and
 * leaves a message for tgs_last_error() on failure. The C++ classes in
 * include/tinygs_amd/tinygs.hpp wrap these calls with the reference's class
 * names and signatures and rethrow failures as std::runtime_error, as the
 * reference does (CUDA_CHECK_THROW, tinygs/include/tinygs/cuda/common_host.hpp:104).
 *
 * Threading: a handle is not re-entrant (as FastGSRasterizer::Impl). Calls on
 * different handles may run concurrently on different streams.
 * Memory: parameters, gradients, images and loss buffers are owned by the
 * caller; every handle owns its grow-only device scratch.
 * Images are fp32 (or fp16 for the fp16-image rasterizer and losses),
 * channel-planar, padded to multiples of 8 and 8x8-tiled
 * (tinygs/include/tinygs/common.hpp:366-414).
 */
#ifndef TINYGS_AMD_H
#define TINYGS_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TGS_OK 0
#define TGS_ERR_INVALID 1
#define TGS_ERR_HIP 2
#define TGS_ERR_STATE 3
#define TGS_ERR_UNSUPPORTED 4
#define TGS_ERR_CAPACITY 5   /* a no-sync forward needed more instances than reserved */

#define TGS_DTYPE_FLOAT32 0
#define TGS_DTYPE_FLOAT16 1
#define TGS_DTYPE_UINT8 2   /* images only: tgs_image_* and tgs_convert */

/* SoA Gaussian parameters (or their gradients), as GPUGaussian3d
 * (tinygs/include/tinygs/core/gpu_gaussian.hpp:9-73): means[3n], scales[3n]
 * (log), rotations[4n] (r,x,y,z), opacities[n] (logit), sh0[3n],
 * sh_rest[45n] (15 bases per Gaussian whatever the degree). sh_dtype applies
 * to sh0 and sh_rest of parameters; gradients are always float32. Every array
 * must be 16-byte aligned (hipMalloc and torch allocations are). */
typedef struct tgs_gaussians {
    void* means;
    void* scales;
    void* rotations;
    void* opacities;
    void* sh0;
    void* sh_rest;
    int64_t n;
    int32_t sh_degree;
    int32_t sh_dtype;
    float scene_scale;
} tgs_gaussians;

/* Camera as GPUBatchInput (tinygs/include/tinygs/dataloader/dataloader.hpp:8-14):
 * K and w2c in glm column-major memory order (fx = K[0], fy = K[4],
 * cx = K[6], cy = K[7]; translation in w2c[12..14]). */
typedef struct tgs_camera {
    uint32_t width;
    uint32_t height;
    float near_plane;
    float far_plane;
    float K[9];
    float w2c[16];
} tgs_camera;

/* DensificationInfo per Gaussian (tinygs/include/tinygs/core/gaussian.hpp:18-23):
 * {accum_counter, accum_grad_mean2d, accum_absgrad_mean2d, max_radii_screen}. */

typedef struct tgs_rasterizer tgs_rasterizer;
typedef struct tgs_loss tgs_loss;
typedef struct tgs_adam tgs_adam;

/* Thread-local message of the last failing call on this thread. */
const char* tgs_last_error(void);
/* Library version (monotonic integer). */
int tgs_version(void);

/* ---- rasterizer: replaces create_rasterizer("fastgs") / FastGSRasterizer
 * (tinygs/src/rasterizer/rasterizer.cpp:44-53, tinygs/src/rasterizer/fastgs.cu:85-398). */
int tgs_rasterizer_create(const char* type, tgs_rasterizer** out);
int tgs_rasterizer_destroy(tgs_rasterizer* r);
/* FastGSRasterizer::set_gaussians (fastgs.cu:388-392). Pointers are kept, not copied. */
int tgs_rasterizer_set_gaussians(tgs_rasterizer* r, const tgs_gaussians* g);
/* FastGSRasterizer::forward (fastgs.cu:89-236). image: [3 * channel_stride]
 * of image_dtype: TGS_DTYPE_FLOAT32, or TGS_DTYPE_FLOAT16 for the fp16-image
 * rasterizer (fastgs.cu:143-188, fastgs_ours_fp16/: half conic and opacity,
 * 8-bit colour, 255-scaled blending; the backward then takes a half gradient
 * image and half image). densification_info: optional device float4[n]
 * (max_radii_screen updated). */
int tgs_rasterizer_forward(tgs_rasterizer* r, const tgs_camera* cam, void* image, int32_t image_dtype,
                           void* densification_info, void* stream);
/* FastGSRasterizer::forward with flags. TGS_FORWARD_NO_SYNC: the forward
 * does not wait for the visible / instance counts (the reference waits three
 * times, forward.cu:133-148,185-187) and sizes the instance buffers by the
 * capacity of tgs_rasterizer_reserve instead, so a whole iteration can be
 * queued ahead or captured into a HIP graph. A forward that needs more
 * instances than reserved renders only the first ones and sets a sticky flag
 * that tgs_rasterizer_status reports as TGS_ERR_CAPACITY. A captured forward
 * must not grow a buffer: run one with the same sizes before capturing.
 * No counterpart in the reference. */
#define TGS_FORWARD_NO_SYNC 1
int tgs_rasterizer_forward_ex(tgs_rasterizer* r, const tgs_camera* cam, void* image, int32_t image_dtype,
                              void* densification_info, int32_t flags, void* stream);
/* Allocates the instance-sized buffers for up to max_instances instances over
 * up to grid_tiles tiles (16 x 16 pixels each) and makes that the capacity of
 * TGS_FORWARD_NO_SYNC forwards. May synchronise the stream. When a buffer has
 * to grow, the last forward's state is dropped (a backward then needs a new
 * forward), so reserve before a forward, not between it and its backward.
 * No counterpart in the reference (its scratch grows inside forward,
 * fastgs.cu:75-82). */
int tgs_rasterizer_reserve(tgs_rasterizer* r, int64_t max_instances, int32_t grid_tiles, void* stream);
/* Synchronises the stream and reports the device-side state of the forwards
 * queued so far: TGS_ERR_CAPACITY when a no-sync forward overflowed its
 * capacity (the flag is cleared when clear_capacity_flag is nonzero),
 * TGS_ERR_STATE when a binning scan failed (those flags are cleared once
 * reported; the forwards that saw them rendered nothing). Also makes the
 * counts of a no-sync forward available to tgs_rasterizer_counts without a
 * further wait. A forward that waits (no TGS_FORWARD_NO_SYNC) reports a
 * failed binning scan itself: it fails with TGS_ERR_STATE, and a backward
 * after it is refused. */
int tgs_rasterizer_status(tgs_rasterizer* r, int32_t clear_capacity_flag, void* stream);
/* FastGSRasterizer::backward (fastgs.cu:238-384). Accumulates (+=) into grads.
 * Must follow a forward on the same Gaussians and camera. */
int tgs_rasterizer_backward(tgs_rasterizer* r, const void* grad_image, const void* image,
                            const tgs_gaussians* grads, void* densification_info, void* stream);
/* Same as tgs_rasterizer_backward with flags. TGS_BACKWARD_ASSIGN: gradients
 * are assigned (zero for culled primitives) instead of accumulated, i.e. the
 * caller's zeroing (tinygs/src/orchestrator.cu:351-353) fused into the write.
 * No counterpart in the reference; for callers that zero before every backward. */
#define TGS_BACKWARD_ASSIGN 1
/* TGS_BACKWARD_SPARSE: rows (per primitive, every gradient array) that
 * received a nonzero 2D gradient are assigned; all other rows are left as they
 * were (their true gradient is exactly zero) and the per-primitive byte mask
 * returned by tgs_rasterizer_grad_row_mask marks the assigned rows (1) and
 * the skipped ones (0). Pair it with tgs_adam_step_masked, which then reads
 * only the marked rows. No counterpart in the reference: it spares writing
 * and re-reading the zero rows (most rows at 1M Gaussians). */
#define TGS_BACKWARD_SPARSE 2
/* TGS_BACKWARD_POSE: also compute the pose-optimisation gradient dL/dw2c of
 * FastGSRasterizer::backward with enable_pose_opt (fastgs.cu:264-271,373-383;
 * kernels_backward.cuh:256-269; backward.cu:332-348): the sum over the
 * primitives with a gradient of dL/dmean_cam[k] * (mean, 1) in row k < 3,
 * row 3 zero; the mean's path only, as in the reference. Read it with
 * tgs_rasterizer_grad_w2c. Combines with the other flags. */
#define TGS_BACKWARD_POSE 4
/* TGS_BACKWARD_KEEP_2D: also leave every primitive's summed 2D gradients in
 * the debug view's grad2d (12 floats per primitive: dL/dmean2d x, y; the
 * |dL/dmean2d| sums x, y (with densification info); dL/dconic a, b, c;
 * dL/dcolour r, g, b; the sum of alpha * dL/dalpha; 0), zero for primitives
 * without a gradient. For parity tests of the blend backward on its own; no
 * counterpart in the reference. */
#define TGS_BACKWARD_KEEP_2D 8
/* (fp32 images: the 12th float of each grad2d row then carries, as bits, the
 * primitive's mask word of written records of ranks 0..31; see
 * tgs_debug_view.record_bits) */
int tgs_rasterizer_backward_ex(tgs_rasterizer* r, const void* grad_image, const void* image,
                               const tgs_gaussians* grads, void* densification_info, int32_t flags, void* stream);
/* Device byte mask [n] of the last TGS_BACKWARD_SPARSE backward (1: row
 * assigned, 0: row skipped, its gradient is zero). Valid until the next
 * backward or the next forward that grows the Gaussian count. */
int tgs_rasterizer_grad_row_mask(tgs_rasterizer* r, const uint8_t** mask);
/* Device byte mask [n] of the rows a TGS_BACKWARD_SPARSE backward after the
 * last forward will assign, known before that backward runs (queued on the
 * stream: two small kernels over the forward's work items). It equals the
 * mask tgs_rasterizer_grad_row_mask returns after that backward. Valid until
 * the next forward. It lets the optimiser update the rows without gradient
 * (TGS_ADAM_ROWS_UNMARKED) on another stream while the backward runs, then
 * the others (TGS_ADAM_ROWS_MARKED | TGS_ADAM_SAME_STEP). No counterpart in
 * the reference. */
int tgs_rasterizer_backward_rows(tgs_rasterizer* r, const uint8_t** rows, void* stream);
/* ctx.grad_input.w2c of the last TGS_BACKWARD_POSE backward (fastgs.cu:373-383):
 * 16 floats into host memory, glm column-major like tgs_camera.w2c
 * (w2c_grad[4 c + r] = dL/dw2c(r, c)). Synchronises the stream. */
int tgs_rasterizer_grad_w2c(tgs_rasterizer* r, float* w2c_grad, void* stream);
/* Counts of the last forward: visible primitives, instances, tiles. After a
 * TGS_FORWARD_NO_SYNC forward this waits for the device. */
int tgs_rasterizer_counts(tgs_rasterizer* r, int64_t* n_visible, int64_t* n_instances, int64_t* n_tiles);

/* Internal buffers of the last forward, for parity tests (device pointers). */
typedef struct tgs_debug_view {
    const uint32_t* n_touched;     /* [n] */
    const uint32_t* bounds;        /* [4n] records: x_min | x_max << 16, y_min | y_max << 16, the exact
                                      test's outcome for rect tiles 0..31 (bit k: row-major tile k), 0 */
    const float* mean2d;           /* [2n] */
    const float* conic_opacity;    /* [4n] */
    const float* color;            /* [4n]: r, g, b (unclamped), ln(255 * opacity) */
    const uint32_t* depth_sorted_keys;  /* [n_visible] depth bits - depth_key_base, ascending */
    const uint32_t* depth_sorted_prims; /* [n_visible] */
    const uint32_t* instance_tiles;     /* [n_instances] sorted (written from tile_ranges by this call:
                                           the tile sort keeps them only as ranges) */
    const uint32_t* instance_prims;     /* [n_instances] */
    const uint32_t* tile_ranges;        /* [2 * n_tiles]: [start, end) per tile, (0, 0) when empty */
    const uint32_t* n_contrib;          /* [channel_stride] (fp16 images: uint16_t) */
    const uint32_t* tile_max;           /* [n_tiles] */
    const float* grad2d;                /* [12n] after a TGS_BACKWARD_KEEP_2D backward, else NULL */
    int64_t n_visible;
    int64_t n_instances;
    int64_t n_tiles;
    uint32_t depth_key_base;            /* bits of the near plane (0 when near <= 0) */
    uint32_t image_dtype;               /* of the last forward. TGS_DTYPE_FLOAT16 (FGS16): the
                                           records' second half is conic a | b << 16, c | opacity
                                           << 16 (halves), 0, ln(255 opacity); conic_opacity the
                                           halves as floats; color the words a | b << 16,
                                           c | opacity << 16, r | g << 8 | b << 16 (bytes), 0 */
    const uint32_t* first_slot;         /* [n] first 2D-gradient record slot of each visible primitive */
    const float* records;               /* [12 * n_instances] 2D-gradient records of the last backward.
                                           fp32 images: the record of the instance of rank k among
                                           primitive p's instances (instance_ranks) sits at slot
                                           first_slot[p] + k; for k < 32 its mark is bit k of p's mask
                                           word (grad2d[12 p + 11] after a TGS_BACKWARD_KEEP_2D
                                           backward), for k >= 32 bit first_slot[p] + k of record_bits.
                                           FGS16: the buckets that reached p fill
                                           first_slot[p], first_slot[p] + 1, ... in completion order
                                           ([11] holds the instance index's bits) */
    const uint16_t* instance_ranks;     /* [n_instances] fp32 images: each sorted instance's rank
                                           among its primitive's instances (in tile order); else NULL */
    const uint32_t* record_bits;        /* [ceil(n_instances / 32)] fp32 images: one bit per record
                                           slot, set for the records of rank >= 32 the last backward
                                           wrote; else NULL */
} tgs_debug_view;
int tgs_rasterizer_debug_view(tgs_rasterizer* r, tgs_debug_view* out);

/* ---- losses: replace create_loss("l1" | "fused_ssim") and LossBase::evaluate
 * (tinygs/src/loss/loss.cu:13-27, tinygs/include/tinygs/loss/loss.hpp:6-28).
 * Accumulate: loss[i] += ..., grad[i] += ... (loss and grad may be NULL for l1,
 * grad may be NULL for fused_ssim). dtype TGS_DTYPE_FLOAT32 or
 * TGS_DTYPE_FLOAT16 (pred, target, loss and grad all of it; l1.cu:130-146,
 * fused_ssim.cu:863-906): fp16 computes in float and rounds each stored value
 * to nearest half. */
typedef struct tgs_loss_context {
    const void* pred;
    const void* target;
    void* loss;
    void* grad;
    uint32_t width;
    uint32_t height;
    uint32_t channel;
    int32_t dtype;
} tgs_loss_context;
int tgs_loss_create(const char* type, tgs_loss** out);
int tgs_loss_destroy(tgs_loss* l);
int tgs_loss_evaluate(tgs_loss* l, const tgs_loss_context* ctx, float scale, void* stream);

/* Fused 0.8-L1 + 0.2-SSIM style evaluation: the L1 term (scale l1_scale,
 * normalised by W*H*3 as l1.cu:117-121) and the SSIM term (scale ssim_scale,
 * normalised by H*W as fused_ssim.cu:811) of one prediction in two launches,
 * equal to tgs_loss_evaluate of an "l1" and then a "fused_ssim" loss (the
 * L1 term is added first). No counterpart method in the reference: it is the
 * loss_l1_ssim entry of the boundary, for callers that evaluate both losses
 * of Orchestrator::evaluate_losses (tinygs/src/orchestrator.cu:763-807)
 * together. Any loss handle works (it supplies the SSIM scratch maps).
 * flags: TGS_LOSS_ASSIGN writes loss / grad instead of accumulating, the same
 * as zeroing them first (orchestrator.cu:354-355). */
#define TGS_LOSS_ASSIGN 1
int tgs_loss_l1_ssim(tgs_loss* l, const tgs_loss_context* ctx, float l1_scale, float ssim_scale, int32_t flags,
                     void* stream);

/* PsnrMetric::evaluate (tinygs/src/loss/psnr.cu:72-128): -10 log10(MSE),
 * MSE = sum over the padded elements of (saturate(pred) - target)^2 / (W H C),
 * 100 for a zero MSE. Float32 tiled images of ctx (loss / grad unused).
 * Synchronises the stream. */
int tgs_psnr(const tgs_loss_context* ctx, float* psnr, void* stream);

/* ---- SimpleAdam: replaces create_optimizer("simple_adam") / SimpleAdam
 * (tinygs/src/optim/optim.cu:86-105, tinygs/src/optim/simple_adam.cu:406-580). */
typedef struct tgs_adam_params {
    float beta1, beta2, epsilon;
    float means_lr, shs_lr, opacities_lr, scales_lr, rotations_lr;
    float max_grad_1;
    float opacities_l1, scales_l1;
    int32_t decay_mean;  /* decay_reduction == "mean": L1 decay scaled by 1/n */
} tgs_adam_params;
int tgs_adam_create(const tgs_gaussians* params, const tgs_gaussians* grads, tgs_adam** out);
int tgs_adam_destroy(tgs_adam* a);
int tgs_adam_set_params(tgs_adam* a, const tgs_adam_params* p);
int tgs_adam_get_params(tgs_adam* a, tgs_adam_params* p);
int tgs_adam_set_lr(tgs_adam* a, float global_lr);
float tgs_adam_get_lr(tgs_adam* a);
/* Rebind parameter / gradient pointers (sizes must match the moments). */
int tgs_adam_set_gaussians(tgs_adam* a, const tgs_gaussians* params, const tgs_gaussians* grads);
/* OptimizerBase::step(scale, stream): gradients multiplied by scale. */
int tgs_adam_step(tgs_adam* a, float scale, void* stream);
/* tgs_adam_step where row i of every gradient array is read only if
 * row_mask[i] != 0 and is taken as zero otherwise (the mask of a
 * TGS_BACKWARD_SPARSE backward). Same results as tgs_adam_step on gradients
 * whose unmarked rows are zero. No counterpart in the reference. */
int tgs_adam_step_masked(tgs_adam* a, float scale, const uint8_t* row_mask, void* stream);
/* tgs_adam_step_masked with flags (row_mask may be NULL). TGS_ADAM_DEVICE_STEP:
 * the step count and the bias corrections (simple_adam.cu:475-480, in double
 * rounded to float, the same values as the host computes) live on the device
 * and are advanced by a kernel of the step, so the launch sequence is the
 * same every step and a captured step replays with the right count. The
 * first device step after creation, a host-counted step or a reset seeds the
 * device count from the host's (capture only after one device step); graph
 * replays advance only the device count (tgs_adam_device_steps reads it).
 * No counterpart in the reference (its bias corrections are host
 * arithmetic per step). */
#define TGS_ADAM_DEVICE_STEP 1
/* Row selection (needs row_mask; the two are exclusive): TGS_ADAM_ROWS_UNMARKED
 * updates only the rows whose mask byte is 0 (as zero-gradient rows, no
 * gradient read), TGS_ADAM_ROWS_MARKED only the others; nothing of the rows
 * left out is read or written, so the two parts may be updated at different
 * times. TGS_ADAM_SAME_STEP: the step count and bias corrections of the
 * previous call (which must be of the same TGS_ADAM_DEVICE_STEP mode) instead
 * of a new step; in device-step mode the call must be ordered after that
 * call's launch. Together: one step in two parts, bit-identical to a single
 * masked step. No counterpart in the reference. */
#define TGS_ADAM_ROWS_UNMARKED 2
#define TGS_ADAM_ROWS_MARKED 4
#define TGS_ADAM_SAME_STEP 8
int tgs_adam_step_ex(tgs_adam* a, float scale, const uint8_t* row_mask, int32_t flags, void* stream);
/* The step count of the device-step mode (synchronises the stream; the host
 * count when no device step was taken since the last host-counted one). */
int tgs_adam_device_steps(tgs_adam* a, int64_t* steps, void* stream);
/* OptimizerBase::reset(): zero moments and the step counter. */
int tgs_adam_reset(tgs_adam* a, void* stream);
int64_t tgs_adam_global_steps(tgs_adam* a);
/* Device pointers of a group's moments; group in 0..5 =
 * means, opacities, rotations, scales, sh0, sh_rest. */
int tgs_adam_moments(tgs_adam* a, int32_t group, float** first, float** second);
/* SimpleAdam::remove (simple_adam.cu:841-906): moment row k becomes old row
 * rows[k] for k < n_rows (device int32 array); the moments then hold n_rows
 * rows and tgs_adam_set_gaussians takes arrays of that size. */
int tgs_adam_gather(tgs_adam* a, const int32_t* rows, int64_t n_rows, void* stream);
/* SimpleAdam::duplicate (simple_adam.cu:908-924): n_new zero moment rows
 * appended. */
int tgs_adam_append(tgs_adam* a, int64_t n_new, void* stream);
/* SimpleAdam::reset_opacity (simple_adam.cu:981-985): opacity moments zeroed. */
int tgs_adam_reset_opacity(tgs_adam* a, void* stream);
/* SimpleAdam::reset(int* indices, int num_reset) (simple_adam.cu:944-979):
 * both moments of rows rows[0 .. n_rows) (device int32) zeroed in every group.
 * Indices outside the moments' rows are refused before anything is written
 * (the reference does not check). Synchronises the stream. */
int tgs_adam_reset_rows(tgs_adam* a, const int32_t* rows, int64_t n_rows, void* stream);
/* SimpleAdam::reorder(uint* indices) (simple_adam.cu:1037-1097; pure virtual
 * at optim.hpp:70-73): a gather over all rows, new[i] = old[indices[i]]
 * (device array of the moments' row count). Refuses out-of-range indices.
 * Synchronises the stream. */
int tgs_adam_reorder(tgs_adam* a, const uint32_t* indices, void* stream);

/* ---- densification: the device work of DefaultStrategy
 * (tinygs/src/strategy/default.cu:26-341) and GPUGaussian3d::remove
 * (tinygs/src/core/gpu_gaussian.cu:117-160). Array sizing (append / remove of
 * rows) belongs to the caller, as the arrays are the caller's. densif is the
 * (n, 4) float DensificationInfo array (counter, grad sum, |grad| sum, max
 * screen radius) a forward / backward with densification info fills. */
/* pcg32 state (tinygs/include/tinygs/random/pcg32.hpp:35-53). */
typedef struct tgs_pcg32 {
    uint64_t state, inc;
} tgs_pcg32;
/* pcg32::seed(initstate, initseq) (host only). */
void tgs_pcg32_seed(tgs_pcg32* rng, uint64_t initstate, uint64_t initseq);
/* pcg32::next_uint(bound) (pcg32.hpp:68-94, host only): uniform in [0, bound)
 * by rejection; bound 0 returns next_uint(). */
uint32_t tgs_pcg32_next_uint(tgs_pcg32* rng, uint32_t bound);
/* generate_random_logistic(rng, n, out, mean, stddev) (random/device.cuh:38-84):
 * out[i] = logit(u) * stddev * 0.551328895 + mean with the reference's
 * assignment of stream positions to elements; rng advanced by n. */
int tgs_random_logistic(tgs_pcg32* rng, int64_t n, float* out, float mean, float stddev, void* stream);
/* default.cu:151-214: flags[i] = 0 / 1 (duplicate) / 2 (split) for the n
 * Gaussians of g; src_indices (device, capacity n) receives the flagged
 * indices in order; counts on the host. grad_threshold includes the grad
 * scaler, scale_threshold the scene scale. Synchronises the stream. */
int tgs_densify_select(const tgs_gaussians* g, const float* densif, float grad_threshold, float scale_threshold,
                       int32_t absgrad, uint8_t* flags, int32_t* src_indices, int64_t* n_duplicate,
                       int64_t* n_split, void* stream);
/* default.cu:235-297: g already holds n_old + n_grow rows; grown row i
 * (target n_old + i) is made from source src_indices[i] per flags, with the
 * six logistic numbers rand6[6 i .. 6 i + 5] of a split. */
int tgs_densify_apply(const tgs_gaussians* g, int64_t n_old, const int32_t* src_indices, int64_t n_grow,
                      const uint8_t* flags, const float* rand6, void* stream);
/* default.cu:300-341: alive[i] for the n Gaussians of g (densif rows at or
 * past n_info count as small on screen); kept_indices (device, capacity n)
 * receives the alive indices in order, *n_kept their count. Synchronises. */
int tgs_prune_select(const tgs_gaussians* g, const float* densif, int64_t n_info, float opacity_threshold,
                     float scale_limit, float radius_limit, int32_t prune_large, uint8_t* alive,
                     int32_t* kept_indices, int64_t* n_kept, void* stream);
/* Row k of every array of dst (k < dst->n) = row rows[k] of src (same SH
 * dtype): the copy of GPUGaussian3d::remove with its mapping. */
int tgs_gaussians_gather(const tgs_gaussians* src, const tgs_gaussians* dst, const int32_t* rows, void* stream);
/* GPUGaussian3d::reorder(uint* indices, stream) (gpu_gaussian.cu:273-310): in
 * place, row i of every array becomes old row indices[i] (device array of
 * g->n indices, each in [0, n); out-of-range indices are refused before
 * anything is written). Uses one temporary array; synchronises the stream. */
int tgs_gaussians_reorder(const tgs_gaussians* g, const uint32_t* indices, void* stream);
/* The reorder() of Orchestrator::reorder_gaussians (orchestrator.cu:26-90):
 * indices (device, n) receives the Gaussians' order by the 30-bit Morton
 * code of their means (means: device float[3n]) in the means' bounding box
 * (per axis (v - min) / max(max - min, 1e-8), clamped to [0, 1], times 1023,
 * truncated), stable for equal codes, as CUB's radix sort over bits 0..29.
 * Feed it to tgs_gaussians_reorder / tgs_adam_reorder. Allocates its scratch
 * and synchronises the stream. */
int tgs_morton_order(const float* means, int64_t n, uint32_t* indices, void* stream);
/* densification_update of Orchestrator::reorder_gaussians
 * (orchestrator.cu:1023-1032, 1052-1059): out[i] = info[indices[i]] for the
 * n DensificationInfo rows (device float4[n] each; out must not alias info).
 * Out-of-range indices are refused before anything is written
 * (synchronises the stream for that check). */
int tgs_densification_reorder(const void* info, void* out, const uint32_t* indices, int64_t n, void* stream);
/* thrust::copy_if of the flag indices (default.cu:198-203, gpu_gaussian.cu:120-124): out
 * (device, capacity n) receives the i < n with flags[i] != 0 in order, *count their number.
 * Synchronises. */
int tgs_flags_compact(const uint8_t* flags, int64_t n, int32_t* out, int64_t* count, void* stream);
/* tgs_flags_compact without any allocation. No counterpart in the reference:
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). Same
 * arguments and results as tgs_flags_compact; n at most 2^26 (larger n is
 * refused with TGS_ERR_INVALID before anything runs). Its counts live in a
 * 384 KiB static device array that each GPU holds until the process ends and
 * that every call on that GPU shares: calls that overlap on one GPU race.
 * Synchronises the stream. */
int tgs_flags_compact_noalloc(const uint8_t* flags, int64_t n, int32_t* out, int64_t* count, void* stream);
/* reset_opacity (default.cu:26-37): opacity = logit(min(sigmoid(opacity), max_opacity)). */
int tgs_reset_opacity(const tgs_gaussians* g, float max_opacity, void* stream);

/* ---- on-disk formats: PLY (tinygs/src/core/pointcloud.cpp:19-240, written
 * through hapPLY, tinygs/src/core/happly.h). */
/* save_ply(filename, gaussians, full_features) (pointcloud.cpp:111-240), as
 * the orchestrator's export calls it (tinygs/src/orchestrator.cu:581-583) but
 * from the device arrays of g: a binary little-endian PLY with hapPLY's header
 * and one "vertex" element of g->n rows: x y z, red green blue (uchar), and
 * with full_features f_dc_r/g/b, f_rest_{r,g,b}_k (k = 0..14), opacity,
 * scale_0..2, rot_w rot_x rot_y rot_z. fp16 SH are written as float. The rows
 * are packed on the device; synchronises the stream. */
int tgs_ply_save(const char* filename, const tgs_gaussians* g, int32_t full_features, void* stream);
/* Vertex count and contents of a PLY file (ascii or binary). format: 0 ascii,
 * 1 binary little endian, 2 binary big endian. has_gaussians: every property
 * tgs_ply_load_gaussians needs is present. No counterpart in the reference
 * (its hapPLY reader parses the header in load_ply, pointcloud.cpp:75-92). */
typedef struct tgs_ply_info {
    int64_t n_vertices;
    int32_t format;
    int32_t has_gaussians;
    int32_t has_colors;
} tgs_ply_info;
int tgs_ply_read_info(const char* filename, tgs_ply_info* info);
/* The inverse of save_ply with full features, to restart from an exported
 * file (the reference has no Gaussian reader; it exports PLY at evaluation
 * and keeps no other checkpoint). g (device arrays, g->n == the file's vertex
 * count) receives every parameter; properties are found by name in any order
 * and type, under the reference's names or the common 3DGS ones (f_dc_0..2,
 * f_rest_i with i = channel * 15 + k, rot_0..3). fp16 SH are rounded to
 * nearest even. Synchronises the stream. */
int tgs_ply_load_gaussians(const char* filename, const tgs_gaussians* g, void* stream);
/* load_point_cloud (pointcloud.cpp:94-109): ".ply" -> load_ply (:75-92,
 * positions and uchar colours / 255); ".txt" -> load_from_colmap (:19-73,
 * COLMAP points3D.txt). Host arrays points[3 n], colors[3 n]. With points ==
 * NULL only *n is set (the count); otherwise *n is the capacity on entry and
 * the count on return. */
int tgs_point_cloud_load(const char* filename, int64_t* n, float* points, float* colors);

/* ---- image layout converters (tinygs/src/utils/image_format.cu:68-139;
 * tinygs/src/dataloader/dataloader.cu:18-95). Tiled images are channel-planar,
 * 8x8-tiled and padded to multiples of 8, of type TGS_DTYPE_FLOAT32 / FLOAT16
 * / UINT8; float <- u8 is (1 / 255) * v, u8 <- float is the truncation of
 * clamp(255 v, 0, 255) (orchestrator.cu:896-937). All device pointers. */
/* from_cv2 (image_format.cu:68-90) with bgr = 1 (channels must be 3), an RGB /
 * any-channel interleaved image with bgr = 0; dst_dtype FLOAT32 / FLOAT16 folds
 * the loader's widening in. The padding is written as zero (the reference
 * leaves it unwritten). */
int tgs_image_from_hwc_u8(const uint8_t* src, uint32_t width, uint32_t height, uint32_t channels, int32_t bgr,
                          void* dst, int32_t dst_dtype, void* stream);
/* to_cv2 (image_format.cu:93-114) for a UINT8 source, Orchestrator::to_opencv
 * (orchestrator.cu:896-937) for a FLOAT32 / FLOAT16 one (bgr = 1). */
int tgs_image_to_hwc_u8(const void* src, int32_t src_dtype, uint32_t width, uint32_t height, uint32_t channels,
                        int32_t bgr, uint8_t* dst, void* stream);
/* Elementwise: half_to_float_gpu / float_to_half_gpu (image_format.cu:117-139),
 * convert_u8_float / convert_u8_half (dataloader.cu:26-95), and u8 <- float. */
int tgs_convert(const void* src, int32_t src_dtype, void* dst, int32_t dst_dtype, int64_t n, void* stream);

/* ---- measurement (no counterpart in the reference, which uses NVTX ranges,
 * tinygs/src/rasterizer/fastgs_ours/nvtx_gs.h): HIP events recorded on the
 * launch stream around the selected stages; stage ids 0..9 = preprocess,
 * depth_sort, emit_instances, tile_sort, blend_forward, l1, fused_ssim,
 * blend_backward, preprocess_backward, adam. Process-wide, one host thread. */
int tgs_profiling_set(uint32_t stage_mask);
int tgs_profiling_read(int32_t stage, double* total_ms, int64_t* count, int32_t reset);
const char* tgs_stage_name(int32_t stage);
/* Work counters of the last forward: Gaussians staged by the blend forward
 * (summed over tiles) and Gaussians the blend backward processes (sum over
 * tiles of min(list length, tile max contributor)). Synchronises the device.
 * `reset` is ignored (kept for ABI compatibility). */
int tgs_rasterizer_work_stats(tgs_rasterizer* r, int64_t* fwd_loaded, int64_t* bwd_processed, int32_t reset);

/* ---- self tests (device): deterministic exp/log over arrays, wave primitives. */
int tgs_selftest_detmath(int32_t op, const float* in, float* out, int64_t n, void* stream);
int tgs_selftest_wave(const uint32_t* in, uint32_t* out, void* stream);
/* The fp16 rasterizer's canonical half operations on arrays of half bit
 * patterns (ops 7, 8 take floats in a, op 11 int64, op 14 doubles): 0 exp2,
 * 1 the hardware v_exp_f16 (measurement only), 2 fma(a, b, c), 3 a * b,
 * 4 a + b, 5 a / b, 6 packed fma, 7 float -> half nearest, 8 float -> half
 * toward -inf, 9 a - b, 10 minNum(a, b), 11 the nearest half of a * 2^-24,
 * 12 the lane shift the fp16 blend backward uses (out[i] = a[i - 1] within
 * each 64-lane wave, b[i] at lane 0; n a multiple of 64), 13 the packed exp2
 * of the pair (a[i], b[i]), out[i] its lane i & 1, 14 the nearest half of an
 * exact double sum of halves. Tests only. */
int tgs_selftest_half(int32_t op, const void* a, const void* b, const void* c, void* out, int64_t n, void* stream);
/* The half division of the fp16 rasterizer over every finite operand pair
 * with a nonzero divisor, checked on the device against the correctly
 * rounded quotient. out: device int64[8]: [0] mismatches, [1] pairs checked,
 * [2..4] a, b, quotient bits of one mismatch. Tests only. */
int tgs_selftest_half_div_exhaustive(int64_t* out, void* stream);
/* The FGS16 backward's division (fastgs_ours_fp16/kernels_backward.cuh
 * __h2div(cadg, 1 - alpha)) is Markstein's iteration on the half reciprocal,
 * correctly rounded for divisors in [0x1.4p-7, 1]. Checks it against the
 * correctly rounded division for every half dividend and every positive
 * divisor with bits in [b_lo, b_hi], and the half reciprocal against the
 * correctly rounded one for those divisors. out (device int64[16]): [0]
 * quotient mismatches, [1] reciprocal mismatches, [2..4] a, b, quotient of one
 * mismatch. No counterpart in the reference. */
int tgs_selftest_half_div_blend(int64_t* out, uint32_t b_lo, uint32_t b_hi, void* stream);
/* The shader (core) clock of the current device under a VALU load, in MHz:
 * a probe kernel at eight waves per SIMD runs packed-half fma chains for
 * about a millisecond and reads the shader clock counter and the
 * constant-rate counter around them (their ratio times the wall clock rate).
 * Synchronises the stream. For the VALU issue peak a measurement quotes (one
 * wave64 VALU instruction per CU per clock). No counterpart in the
 * reference. */
int tgs_selftest_clock(double* core_mhz, void* stream);
/* Spin bound of the binning's look-back waits on the current device, for
 * tests of the error path: 0 makes every look-back that has a predecessor
 * give up at once (as a wait that ran out would), setting the look-back error
 * flag; every kernel still runs to its end, and the emission and the blend
 * skip their work when the flag is set. spins = 0xffffffff restores the
 * default bound. Process-wide; not for use while forwards are queued. No
 * counterpart in the reference. */
int tgs_selftest_lookback_spins(uint32_t spins);

#ifdef __cplusplus
}
#endif

#endif
