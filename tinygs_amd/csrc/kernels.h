// Host-side launchers of the HIP kernels (internal C++ interface of the library).
#pragma once

#include <cstddef>

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"

namespace tgs {

enum ShDtype : int { kShF32 = 0, kShF16 = 1 };

struct GaussianView {
    const float* means;
    const float* scales;
    const float* rotations;
    const float* opacities;
    const void* sh0;
    const void* sh_rest;
    int64_t n;
    int sh_degree;
    int sh_dtype;
};

struct GradView {
    float* means;
    float* scales;
    float* rotations;
    float* opacities;
    float* sh0;
    float* sh_rest;
};

// ---- preprocess (kernels_forward.cuh:157-412)
// erec[i] (emission record, 16 B, the part the instance emission always reads):
// {x_min | x_max << 16, y_min | y_max << 16, exact-test outcome of the rect
// tiles 0..31 (bit k: row-major rect tile k), 0}. ctl (may be null): the
// binning control block, reset by the first workgroup (bin_ctl_reset_block).
struct BinCtl;
void launch_preprocess(const GaussianView& g, const CamParams& cam, uint32_t* n_touched, uint4* erec,
                       float2* mean2d, float4* conic_opacity, float4* color_pt, uint32_t* depth_key,
                       float* densif, BinCtl* ctl, hipStream_t s);

// ---- scans / compaction / sort / binning
// Device control block of the binning launches. Everything but `err` is
// cleared at the start of every forward; err (look-back error flag) is
// sticky so that a failure is reported by the next host check.
enum { kTicketCompact = 0, kTicketOffsets = 1, kTicketDepth = 2, kTicketTile = 6, kTicketCount = 10 };
// Backward work queues. Queue q hands out its items in runs of kBwdRun
// consecutive ones: item R (q + Q (n / R)) + n % R is its n-th (R = kBwdRun,
// Q = kBwdQueues), so a tile's buckets (consecutive items) mostly go to one
// queue. The backward kernels serve queue q from workgroups b with 4 b + w =
// q (mod Q), which all sit on the XCD b mod 8 (workgroups go to the 8 XCDs
// in turn), so that XCD's L2 holds the tile's image, gradient and checkpoint
// lines for the tile's later buckets.
constexpr int kBwdQueues = 64;
constexpr int kBwdRun = 4;
__device__ __forceinline__ uint32_t bwd_queue_item(uint32_t q, uint32_t n) {
    return (uint32_t)kBwdRun * (q + (n / (uint32_t)kBwdRun) * (uint32_t)kBwdQueues) + n % (uint32_t)kBwdRun;
}
struct BinCtl {
    // epoch_base: look-back epochs of the current forward are epoch_base + k
    // for the forward's k-th look-back launch (k < kEpochStride); advanced by
    // kEpochStride on the device at the start of every forward, so a
    // replayed (graph-captured) forward never mistakes the previous replay's
    // status words for its own
    uint32_t V, I, err, epoch_base;
    uint32_t tickets[kTicketCount];
    uint32_t n_items;                     // backward work items listed by the blend forward
    uint32_t pad2[17];
    uint32_t bwd_queue[kBwdQueues * 32];  // next local index of queue q at [32 q] (one line each, from byte 128)
};
static_assert(offsetof(BinCtl, bwd_queue) == 128, "backward queue counters start on their own cache line");
// Bits of BinCtl::err (sticky across forwards until cleared):
constexpr uint32_t kErrLookBack = 1u;   // a look-back scan gave up waiting (spin bound)
constexpr uint32_t kErrOffsets = 2u;    // instance offsets beyond the instance buffers
constexpr uint32_t kErrCapacity = 4u;   // more instances than the reserved capacity (no-sync forward)
// Clears the given err bits.
void launch_clear_err_bits(BinCtl* ctl, uint32_t bits, hipStream_t s);
// Words of bwd_queue: what a backward needs cleared.
constexpr int kBwdCtlWords = kBwdQueues * 32;
// Clears every BinCtl word except err and advances epoch_base (the
// forward's reset; the preprocess does it in its first workgroup, this
// launch only when there is no primitive to preprocess).
void launch_bin_ctl_reset(BinCtl* ctl, hipStream_t s);
constexpr uint32_t kEpochMask = 0x3fffffffu;   // 30-bit launch epoch of look-back status words
constexpr uint32_t kEpochStride = 64u;          // look-back launches per forward, at most
// The reset by the threads of one workgroup.
__device__ __forceinline__ void bin_ctl_reset_block(BinCtl* ctl) {
    uint32_t* p = (uint32_t*)ctl;
    constexpr uint32_t words = sizeof(BinCtl) / 4;
    constexpr uint32_t keep = offsetof(BinCtl, err) / 4, ep = offsetof(BinCtl, epoch_base) / 4;
    for (uint32_t i = threadIdx.x; i < words; i += blockDim.x) {
        if (i == ep)
            p[i] = (p[i] + kEpochStride) & kEpochMask;
        else if (i != keep)
            p[i] = 0u;
    }
}

// Status-word entries (u64) needed by a look-back scan over max_n elements.
int64_t scan_status_entries(int64_t max_n);
// Visible primitives (n_touched > 0) in index order -> (depth key, index,
// n_touched) triples; ctl->V, ctl->I; depth-key digit histograms.
// keys_out receives depth_key - key_base (key_base <= every visible key, so
// the order is that of the keys).
// Compacted inside each depth-sort block: block b's visible primitives at
// [4096 b, 4096 b + block_n[b]) in index order; counts[d * nb + b] the
// block's counts of the first depth pass's digit ((key >> shift) & (2^bits -
// 1)), nb = ceil(n / 4096); V and I added into ctl (zero before).
void launch_compact_visible(const uint32_t* n_touched, const uint32_t* depth_key, int64_t n, uint32_t key_base,
                            int shift, int bits, uint32_t* keys_out, uint32_t* vals_out, uint32_t* nt_out,
                            uint32_t* counts, uint32_t* block_n, BinCtl* ctl, hipStream_t s);
// offs[k] = exclusive scan of nt_sorted[k] over k < ctl->V; offs[V] = total.
void launch_instance_offsets(const uint32_t* nt_sorted, int64_t max_count, uint32_t* offs, BinCtl* ctl,
                             uint64_t* status, uint32_t& epoch, hipStream_t s);
// Entries of the per-workgroup digit-count matrix of radix_sort.
int64_t radix_count_entries(int64_t max_n, bool depth);
// Stable LSD radix sort of (key, value[, value2]) u32 triples; pass p sorts
// bits[p] bits at shifts[p]. v2 may be NULL. depth selects the workgroup
// size class. Each pass uses one ticket (tickets[p]) and one epoch for the
// scan of its count matrix. Ping-pongs between the buffers; returns the
// index (0/1) of the result. first_block_n (depth sort): the first pass's
// input blocks hold first_block_n[b] keys each (launch_compact_visible's
// blocks) and its digit counts are already in counts. offs (depth sort, v2 =
// n_touched): with two passes or more the last pass writes the instance
// offsets (offs[k] = sum of v2 over sorted positions < k, offs[n] = the
// total) instead of the sorted v2, and sets *offs_done; otherwise the
// caller runs launch_instance_offsets on the sorted v2. ranges (tile sort,
// n_tiles tiles): the last pass also reduces each tile's instance range
// [x, y) into ranges and sets *ranges_done; empty tiles are left as
// (UINT32_MAX, 0), which the forward blend rewrites as (0, 0); that pass
// writes no sorted keys (launch_keys_from_ranges restores them from the
// ranges). Without *ranges_done the caller runs launch_tile_ranges on the
// sorted keys.
// ranks (tile sort, with ranges): the last pass also writes ranks[o] = the
// key's bits 16..31 of sorted position o (the emission's per-primitive
// instance rank on fp32 images; the tile is then the key's sorted bits).
// clear_bits (tile sort): the first pass's upsweep zeroes
// record_bit_words(max_n) words there (one bit per instance position).
int radix_sort(uint32_t* keys[2], uint32_t* vals[2], uint32_t* v2[2], const uint32_t* d_n, int64_t max_n, bool depth,
               int n_passes, const int* shifts, const int* bits, uint32_t* counts, uint32_t* tickets,
               uint64_t* status, const uint32_t* epoch_base, uint32_t& epoch, uint32_t* err,
               const uint32_t* first_block_n, uint32_t* offs, bool* offs_done, uint2* ranges, uint32_t n_tiles,
               bool* ranges_done, uint16_t* ranks, uint32_t* clear_bits, hipStream_t s);
// Words of the record-bit array for up to max_inst instances (whole
// workgroups of the tile sort's first upsweep).
int64_t record_bit_words(int64_t max_inst);
// Instances in depth order: thread per depth-sorted primitive k < ctl->V,
// slots [offs[k], offs[k + 1]).
// Rect tiles past the first 32 take the exact tile test with mean2d[p], the
// conic words x, y, z of conic_words[p] and the power threshold in the w of
// thr_words[p] (conic_opacity and color_pt for fp32 images, info for both
// with FGS16).
// Also writes first_slot[p] = offs[k] for every visible primitive p = prims[k]:
// the first of the n_touched[p] instance slots reserved for p. Slots at or
// beyond max_inst (the instance buffers' size) are never written; offsets
// that would need them set bit 1 of ctl->err.
void launch_emit_instances(const uint32_t* prims, const uint32_t* offs, BinCtl* ctl, int64_t max_count,
                           int64_t max_inst, const float2* mean2d, const uint4* conic_words,
                           const uint4* thr_words, const uint4* erec, uint32_t grid_w,
                           uint32_t* inst_keys, uint32_t* inst_vals, uint32_t* first_slot, bool half_test,
                           hipStream_t s);
// [start, end) per tile, (0, 0) for empty tiles; every entry written. The
// instance count is min(*d_n, max_inst) (max_inst when d_n is null).
// inst_keys[i] = t for every i in the range [x, min(y, max_inst)) of tile t
// (ranges as the forward blend leaves them)
void launch_keys_from_ranges(const uint2* ranges, uint32_t n_tiles, int64_t max_inst, uint32_t* inst_keys,
                             hipStream_t s);
void launch_tile_ranges(const uint32_t* inst_keys, const uint32_t* d_n, int64_t max_inst, uint2* ranges,
                        uint32_t n_tiles, hipStream_t s);
// Sets the spin bound of every look-back wait on the current device (default
// 2^22 polls; 0: give up at once). Returns 0, or -1 on a HIP error.
int set_lookback_spin_limit(uint32_t spins);
// Whether radix_sort accepts these digit widths (host check, before any launch).
bool radix_digits_fit(bool depth, int n_passes, const int* bits);

// ---- Morton order (orchestrator.cu:26-90)
// u32 words of scratch morton_order needs for n means.
int64_t morton_scratch_words(int64_t n);
// indices[i] = the i-th mean in stable order of its 30-bit Morton code in the
// means' bounding box. status: zeroed look-back words for a depth-class sort
// of n keys; ctl: a zeroed control block (tickets, epoch base, error flag).
// Returns -1 when the sort's digit plan is refused (nothing launched after).
int morton_order(const float* means, int64_t n, uint32_t* indices, uint32_t* scratch, uint64_t* status,
                 BinCtl* ctl, hipStream_t s);
// dst[i] = src[indices[i]] for 16-byte rows (densification info).
void launch_rows16_gather(const void* src, void* dst, const uint32_t* indices, int64_t n, hipStream_t s);

// ---- fp16-image rasterizer (FGS16, tinygs/src/rasterizer/fastgs_ours_fp16/)
// Preprocess: as launch_preprocess with the FGS16 rules; info[i] = (conic a | b
// << 16, c | opacity << 16 (halves), r | g << 8 | b << 16, power threshold
// (float bits)).
void launch_preprocess16(const GaussianView& g, const CamParams& cam, uint32_t* n_touched, uint4* erec,
                         float2* mean2d, float4* conic_opacity, uint4* info, uint32_t* depth_key,
                         float* densif, BinCtl* ctl, hipStream_t s);

// Fills order (u32[n_tiles]) with the tiles in decreasing order of the bit
// length of their instance counts (from the ranges; all tiles count as empty
// after a failed binning scan), for a blend forward to take long tiles first
// (order null: index order). One workgroup: returns false, and launches
// nothing, beyond kOrderMaxTiles tiles or without an order buffer. The fp16
// forward uses it (one wave pair per tile: long tiles that start late set its
// length); the fp32 forward measured slower with it (index order keeps
// neighbouring tiles, which share Gaussians, together in the caches).
constexpr uint32_t kOrderMaxTiles = 1u << 20;
// The fp32 blend forward takes tiles long ones first only from this many
// instances per tile on average (heavy scenes): measured 12% slower at 632
// per tile (the order costs locality between neighbouring tiles), even at
// 8.4k; at 16.8k (3M Gaussians at 3840x2160) fwd + bwd took 16.1-17.7 ms
// ordered against 16.1-18.2 ms in index order over three runs each (the
// runs there split into a fast and a slow mode either way).
constexpr int64_t kOrderHeavyTile = 8192;
bool launch_tile_order(const uint2* ranges, uint32_t n_tiles, uint32_t* order, const BinCtl* ctl, hipStream_t s);

// Blend of FGS16 (fgs16.hip): image / grad image are 3 half planes of the
// padded 8x8-tiled layout, n_contrib u16 per pixel, ckpt 256 uint2 per slot
// (the fp32 path's slots), items as the fp32 path's but with every Gaussian of
// the bucket; records as the fp32 path's, half mode.
void launch_blend16_forward(const CamParams& cam, uint2* ranges, const uint32_t* inst_vals,
                            const float2* mean2d, const uint4* info, uint16_t* image, uint16_t* n_contrib,
                            uint32_t* tile_max, uint32_t* tile_loaded, uint2* ckpt, uint4* items, BinCtl* ctl,
                            uint32_t* order, hipStream_t s);
void launch_blend16_backward(const CamParams& cam, const uint32_t* inst_vals, const float2* mean2d,
                             const uint4* info, const uint16_t* image, const uint16_t* grad_image, const uint2* ckpt,
                             const uint4* items, BinCtl* ctl, uint32_t* rec_count, const uint32_t* first_slot,
                             float4* records, hipStream_t s);

// ---- blend (kernels_forward.cuh:569-715, kernels_backward.cuh:675-927)
// Checkpoints: the state (C, T) of every pixel before Gaussian 32 b of its
// tile's list, b >= 1, at slot (range.x / 32 + tile + b - 1), 256 float4 per
// slot in tile pixel order; slots of different tiles never overlap and stay
// below I / 32 + T. Work items: one uint4 {tile, b, first instance, count}
// per 32-Gaussian bucket below the tile's last contributor, appended through
// ctl->n_items (at most I / 32 + T entries). tile_loaded[t]: Gaussians the
// tile staged before it finished (a work statistic).
size_t blend_ckpt_slots(int64_t n_instances, uint32_t n_tiles);
void launch_blend_forward(const CamParams& cam, uint2* ranges, const uint32_t* inst_vals, const float2* mean2d,
                          const float4* conic_opacity, const float4* color_pt, float* image, uint32_t* n_contrib,
                          uint32_t* tile_max, uint32_t* tile_loaded, float4* ckpt, uint4* items, BinCtl* ctl,
                          uint32_t* order, hipStream_t s);
// 2D gradient records: each (primitive p, bucket) the backward processes
// writes 12 floats at record index first_slot[p] + k, k the instance's rank
// among p's instances (inst_ranks, from the tile sort; below n_touched[p]: a
// primitive is in a tile's list once), marks it (bit k of rec_mask[p] for
// k < 32, zero between backwards; bit first_slot[p] + k of rec_bits, cleared
// by the forward's tile sort, otherwise) and counts it in rec_count[p] (zero
// between backwards): dL/dmean2d (2), |.| sums
// (2; 0 unless with_abs: only densification reads them), dL/dconic (3),
// dL/dcolour (3), sum of alpha dL/dalpha, 0. The preprocess backward sums
// each primitive's marked records in a fixed order: in rank order in the
// primitive's own thread up to kLightRecords of them, otherwise 16 lanes,
// lane l summing (in rank order) the primitive's records l, l + 16, ...,
// then an xor butterfly over the 16 lane sums (into grad2d[12 p]). 16 measured
// faster than 4, 8 and 32 at config 3. (The fp16-image backward packs its
// records at first_slot[p] + a counter: its sums are exact, in any order.)
constexpr uint32_t kLightRecords = 16;
// ctl->bwd_queue must be zero on entry (the forward's control reset clears it).
void launch_blend_backward(const CamParams& cam, const uint32_t* inst_vals, const uint16_t* inst_ranks,
                           const float2* mean2d, const float4* conic_opacity, const float4* color_pt,
                           const float* image, const float* grad_image, const uint32_t* n_contrib, const float4* ckpt,
                           const uint4* items, BinCtl* ctl, uint32_t* rec_bits, uint32_t* rec_mask,
                           uint32_t* rec_count, const uint32_t* first_slot, float4* records, bool with_abs,
                           hipStream_t s);

// ---- preprocess backward (kernels_backward.cuh:88-352)
// mode: 0 accumulate, 1 assign, 2 sparse (assign rows with gradient, write
// row_mask[i] = 1 for them and 0 for the others, leave the others untouched).
enum { kGradAccumulate = 0, kGradAssign = 1, kGradSparse = 2 };
// Scratch: live and heavy (n uint4 each) lists of the primitives with
// records, grad2d (12 n floats).
int64_t pb_chunks(int64_t n);
// Records are counted by rec_count (cleared here for the next backward) and
// on fp32 images marked by rec_mask (cleared here) and rec_bits.
// slot_limit: the instance capacity of the forward (records lie below it).
void launch_preprocess_backward(const GaussianView& g, const CamParams& cam, const uint32_t* n_touched,
                                const float4* conic_opacity, uint32_t* rec_count, uint32_t* rec_mask,
                                const uint32_t* rec_bits,
                                int64_t slot_limit, const uint32_t* first_slot, const float4* records, float* grad2d,
                                const GradView& out, float* densif, int mode, uint8_t* row_mask, uint4* live,
                                uint4* heavy, float* pose_partial, float* pose_out, bool keep2d, bool half_sums,
                                hipStream_t s);

// ---- PSNR (psnr.cu:72-128): scratch[psnr_scratch_doubles() - 1] receives the
// sum of (saturate(pred) - target)^2 over the n_padded elements
int psnr_scratch_doubles();
void launch_sq_diff_sum(const float* pred, const float* target, int64_t n_padded, double* scratch, hipStream_t s);
void launch_sq_diff_sum_f16(const void* pred, const void* target, int64_t n_padded, double* scratch, hipStream_t s);

// ---- densification (tinygs/src/strategy/default.cu, gpu_gaussian.cu:117-170,
// simple_adam.cu:841-985)
void launch_random_logistic(uint64_t state, uint64_t inc, int64_t n, float mean, float stddev, float* out,
                            hipStream_t s);
int64_t list_chunks(int64_t n);
constexpr int64_t kListChunkElems = 2048;   // flags per chunk of the index-list kernels
// offsets[c] = exclusive prefix over chunks of counts[c].x; totals[0] = sum
// of .x, totals[1] = sum of .y (one workgroup; chunks of any count)
void launch_chunk_offsets(const uint2* counts, int64_t chunks, uint32_t* offsets, uint32_t* totals, hipStream_t s);
// counts[c] = (nonzero flags, flags == 1) of chunk c (list_chunks(n) chunks)
void launch_flag_count(const uint8_t* flags, int64_t n, uint2* counts, hipStream_t s);
// indices of the nonzero flags in index order, chunk c's run at offsets[c]
void launch_flag_compact(const uint8_t* flags, int64_t n, const uint32_t* offsets, int32_t* out, hipStream_t s);
void launch_densify_select(int64_t n, const float4* info, const float* scales, float grow_grad, float grow_scale,
                           int absgrad, uint8_t* flags, hipStream_t s);
void launch_prune_select(int64_t n, const float* opac, const float* scales, const float* rots, const float4* info,
                         int64_t n_info, float scale_limit, float radius_limit, float min_opacity, int prune_large,
                         uint8_t* alive, hipStream_t s);
void launch_densify_apply(int64_t n_grow, int64_t n_old, const int32_t* src, const uint8_t* flags, const float* rnd,
                          float* means, float* scales, float* rots, float* opac, void* sh0, void* shr, int sh_dtype,
                          hipStream_t s);
void launch_gather_rows(const void* src, void* dst, const int32_t* rows, int64_t n_dst, int row_bytes,
                        hipStream_t s);
void launch_gather_rows16(const void* src, void* dst, const int32_t* rows, int64_t n_dst, int width, hipStream_t s);
void launch_reset_opacity(float* opac, int64_t n, float max_opacity, hipStream_t s);
// Zeroes rows rows[0 .. n_rows) of an array of `words` 4-byte words per row.
void launch_zero_rows(void* dst, const int32_t* rows, int64_t n_rows, int words, hipStream_t s);
// bad[0] |= 1 when some idx[k] (k < n) lies outside [0, bound).
void launch_check_indices(const int32_t* idx, int64_t n, int64_t bound, uint32_t* bad, hipStream_t s);

// ---- utilities
void launch_fill_u32(uint32_t* p, uint32_t value, int64_t n, hipStream_t s);

// ---- losses (l1.cu:19-42, fused_ssim.cu:55-442)
void launch_l1(const float* pred, const float* target, float* loss, float* grad, int64_t n_padded, float s,
               hipStream_t st);
// Fused L1 + SSIM forward: s_l1 == 0 disables L1; assign writes loss / grad
// instead of accumulating (grad gets the L1 part, or 0); dm_* may be NULL
// (loss only). The SSIM backward then adds its part to grad.
void launch_l1_ssim_forward(uint32_t width, uint32_t height, float c1, float c2, float s_ssim, float s_l1,
                            bool assign, const float* pred, const float* target, float* loss, float* grad,
                            float* dm_mu, float* dm_s1, float* dm_s12, hipStream_t st);
void launch_ssim_backward(uint32_t width, uint32_t height, float s, const float* pred, const float* target,
                          float* grad, const float* dm_mu, const float* dm_s1, const float* dm_s12, hipStream_t st);
// fp16 images (l1.cu:43-107, fused_ssim.cu:445-693): half pred / target /
// loss / grad, float arithmetic, each stored value rounded to nearest half
void launch_l1_f16(const void* pred, const void* target, void* loss, void* grad, int64_t n_padded, float s,
                   hipStream_t st);
void launch_l1_ssim_forward_f16(uint32_t width, uint32_t height, float c1, float c2, float s_ssim, float s_l1,
                                bool assign, const void* pred, const void* target, void* loss, void* grad,
                                float* dm_mu, float* dm_s1, float* dm_s12, hipStream_t st);
void launch_ssim_backward_f16(uint32_t width, uint32_t height, float s, const void* pred, const void* target,
                              void* grad, const float* dm_mu, const float* dm_s1, const float* dm_s12,
                              hipStream_t st);

// ---- SimpleAdam (simple_adam.cu:104-213, :457-580)
struct AdamGroup {
    void* theta;          // float or half
    const float* grad;
    float* m1;
    float* m2;
    int64_t count;
    float lr;
    int theta_half;       // 1: theta stored as fp16
    int lerp_form;        // 0: fma(t, g - m, m); 1: fma(t, g, fma(-t, m, m))
    int decay_kind;       // 0 none, 1 opacity logistic', 2 scale exp
    float decay_coef;
    int row_width;        // elements per primitive: 3, 1, 4, 3, 3 or 45
};
struct AdamArgs {
    AdamGroup groups[6];
    const uint8_t* row_mask;   // optional: row i's gradient read only if row_mask[i] != 0, else zero
    // with row_mask: 0 updates every row; kAdamRowsUnmarked only the rows with
    // row_mask[i] == 0 (zero gradient, none read), kAdamRowsMarked only the
    // others; the elements of the rows left out are neither read nor written
    int row_select;
    // optional: the bias corrections come from this device state
    // (kAdamStateWords words: [0] step count t, [1] bc1 and [2] bc2_sqrt of t,
    // [3] and [4] those of t + 1, as float bits; done counters from word
    // kAdamDoneStride on) instead of bc1 / bc2_sqrt. dev_advance: this launch
    // is step t + 1 (reads [3], [4]; its last workgroup to finish advances the
    // state, no separate launch_adam_bias); otherwise it repeats step t
    // (reads [1], [2])
    uint32_t* dev_bc;
    int dev_advance;
    int n_groups;
    float beta1, beta2, eps, grad_scale, bc1, bc2_sqrt, max_grad;
};
// Byte mask of the rows (primitives) the blend backward of the last forward
// writes: one per primitive of every work item's bucket range. rows must be
// zeroed before.
void launch_backward_rows(const uint4* items, const uint32_t* inst_vals, const BinCtl* ctl, uint8_t* rows,
                          hipStream_t s);
constexpr uint32_t kAdamDoneGroups = 64;   // done counters of an advancing Adam launch
constexpr uint32_t kAdamDoneStride = 32;   // words between them (one 128-byte line each)
constexpr uint32_t kAdamStateWords = kAdamDoneStride * (kAdamDoneGroups + 2u);
constexpr int kAdamRowsUnmarked = 1;
constexpr int kAdamRowsMarked = 2;
void launch_adam(const AdamArgs& a, hipStream_t s);
// Device-side step count for SimpleAdam (the state of AdamArgs::dev_bc):
// seeds it at `steps` (with the corrections of steps and steps + 1, and the
// done counters cleared), or advances it by one step without an Adam launch
// (simple_adam.cu:475-480: corrections in double, rounded to float), so a
// captured step replays with the right count.
void launch_adam_seed_steps(uint32_t* state, uint32_t steps, float beta1, float beta2, hipStream_t s);
void launch_adam_bias(uint32_t* state, float beta1, float beta2, hipStream_t s);
// Recomputes the stored corrections for new betas, keeping the count.
void launch_adam_rebeta(uint32_t* state, float beta1, float beta2, hipStream_t s);

// ---- self tests of wave primitives and deterministic math (debug entry points)
void launch_detmath(int op, const float* in, float* out, int64_t n, hipStream_t s);
void launch_wave_selftest(const uint32_t* in, uint32_t* out, hipStream_t s);
// canonical half operation `op` (tests): out[i] = op(a[i], b[i], c[i]) as bits
// out[8] (zeroed by the caller): mismatches, pairs checked, a / b / q of one mismatch
void launch_half_div_check(unsigned long long* out, hipStream_t s);
void launch_half_div_blend_check(unsigned long long* out, uint32_t blo, uint32_t bhi, hipStream_t s);
// clock_probe_kernel over `blocks` workgroups of 256 threads: out[2 b] the
// shader clock cycles, out[2 b + 1] the constant-rate counter ticks of
// workgroup b's timed loop
void launch_clock_probe(unsigned long long* out, uint32_t blocks, uint32_t iters, hipStream_t s);
void launch_halfmath(int op, const uint16_t* a, const uint16_t* b, const uint16_t* c, uint16_t* out, int64_t n,
                     hipStream_t s);

}  // namespace tgs
