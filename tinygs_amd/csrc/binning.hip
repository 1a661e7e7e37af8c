// Binning: deterministic visible-primitive compaction, stable LSD radix sort
// (LDS ranking, wave64 ballot match), per-primitive instance offsets,
// instance emission and per-tile ranges.
//
// Reference stages (tinygs/src/rasterizer/fastgs_ours/forward.cu:146-229):
// depth SortPairs, apply_depth_ordering + ExclusiveSum, create_instances
// (kernels_forward.cuh:427-530), tile SortPairs, extract_instance_ranges
// (:532-551). The reference compacts visible primitives with atomicAdd, so
// its order on equal depths is arbitrary; here compaction is a prefix scan in
// index order and every sort is stable, which yields the canonical per-tile
// order (tile, depth bits, primitive index) -- the order of a stable sort of
// 64-bit keys (tile << 32 | depth bits). The low 32 key bits are sorted once
// per primitive (V elements) before duplication; duplication preserves that
// order, so the remaining passes only sort the ceil(log2 T) tile bits over
// the I instances.
//
// MI355X notes that shaped this file (measured): a store or load instruction
// whose 64 lanes touch 64 different cache lines runs at a small fraction of
// HBM bandwidth, so every kernel here reads and writes lane-contiguous runs
// (striped element assignment, LDS staging before the radix scatter); and a
// decoupled look-back whose predecessors all start at once is a serial chain
// of cross-XCD loads, so the radix passes use reduce-then-scan (per-workgroup
// digit counts, one row-scan launch, then the ranked scatter) and only the
// two single-value scans use look-back, with a 64-wide window read by a whole
// wave.
#include "common.h"
#include "kernels.h"
#include "fgs16.h"
#include "rect_tasks.h"

namespace tgs {

constexpr int kThreads = 256;
constexpr int kScanChunk = 4096;                        // elements per scan / compaction workgroup
constexpr int kScanWaves = 16;                          // scan / compaction workgroups: 1024 threads x 4 elements
constexpr int kScanThreads = 64 * kScanWaves;
constexpr int kScanRounds = kScanChunk / kScanThreads;
constexpr int kDepthKeysPerThread = 16;                 // depth passes: 4096 keys per workgroup
constexpr int kTileKeysPerThread = 16;                  // tile passes: 4096 keys per workgroup (2048: 3 us slower, 8192: 17 us)
// LDS histograms per digit count (lane & (kHistCopies - 1) picks one): keys
// that arrive clustered do not serialise their atomic adds on one address.
// The copies are kHistPad words longer than the digit count, so the copies
// of one digit fall into different LDS banks.
constexpr int kHistCopies = 8;
constexpr int kHistPad = 1;
constexpr int kDepthMaxDigits = 512;                    // depth passes: digits of up to 9 bits
constexpr int kTileMaxDigits = 256;                     // tile passes: digits of up to 8 bits
constexpr int kDepthSortWaves = 16;                     // depth up / downsweeps: 1024 threads x 4 keys
constexpr int kTileSortWaves = 8;                       // tile up / downsweeps: 512 threads x 8 keys (1024 x 4: 1 us slower)

// ---------------------------------------------------------------- workgroup scans

// Exclusive scan of one value per thread across a workgroup of NW waves.
// Returns the exclusive prefix; *total receives the workgroup sum.
template <int NW = 4>
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, uint32_t* s_wave, uint32_t* total) {
    const uint32_t lane = threadIdx.x & 63u, w = threadIdx.x >> 6;
    const uint32_t incl = wave_inclusive_scan_u32(v);
    if (lane == 63u) s_wave[w] = incl;
    __syncthreads();
    uint32_t wave_off = 0, sum = 0;
    for (uint32_t k = 0; k < (uint32_t)NW; ++k) {
        const uint32_t c = s_wave[k];
        wave_off += (k < w) ? c : 0u;
        sum += c;
    }
    __syncthreads();
    *total = sum;
    return wave_off + incl - v;
}

// ---------------------------------------------------------------- decoupled look-back (single value)

// status word: [63:62] flag (0 not ready, 1 aggregate, 2 inclusive prefix),
// [61:32] epoch of the launch that wrote it, [31:0] value.
constexpr uint64_t kFlagMask = 3ull << 62;
constexpr uint64_t kFlagAggregate = 1ull << 62;
constexpr uint64_t kFlagPrefix = 2ull << 62;
constexpr uint32_t kSpinLimit = 1u << 22;
// The bound in force (tgs_selftest_lookback_spins changes it for tests of
// the error path; 0 gives up at once wherever a predecessor must be read).
__device__ uint32_t g_lookback_spins = kSpinLimit;

__device__ __forceinline__ uint64_t status_word(uint64_t flag, uint32_t epoch, uint32_t value) {
    return flag | ((uint64_t)(epoch & kEpochMask) << 32) | (uint64_t)value;
}
__device__ __forceinline__ uint64_t load_status(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_status(uint64_t* p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Ticket in launch order, broadcast to the workgroup (contains a barrier).
__device__ __forceinline__ uint32_t take_ticket(uint32_t* ticket, uint32_t* s_bid) {
    if (threadIdx.x == 0) *s_bid = atomicAdd(ticket, 1u);
    __syncthreads();
    return *s_bid;
}

// Called by one whole wave: publishes the workgroup total for ticket `bid`
// and returns (in every lane) the exclusive prefix over smaller tickets.
// Lane q reads the status of ticket bid - 1 - q - 64 m in window m; the
// window is consumed up to its nearest inclusive prefix once every word up
// to that one is ready. Every predecessor is already running and publishes
// its aggregate before it waits on anything, so each wait ends; the spin
// bound only turns a broken invariant into an error flag (checked by the
// host) instead of a hang.
__device__ uint32_t wave_look_back(uint64_t* status, uint32_t bid, uint32_t total, uint32_t epoch, uint32_t* err) {
    const uint32_t lane = lane_id();
    if (lane == 0) store_status(status + bid, status_word(bid == 0 ? kFlagPrefix : kFlagAggregate, epoch, total));
    if (bid == 0) return 0;
    const uint32_t ep = epoch & kEpochMask;
    const uint32_t spin_limit = g_lookback_spins;
    uint32_t excl = 0, spins = 0;
    int64_t j = (int64_t)bid - 1;
    while (true) {
        if (spin_limit == 0u) {   // (tests: the bounded wait gives up at once)
            if (lane == 0) atomicOr(err, kErrLookBack);
            break;
        }
        const int64_t src = j - (int64_t)lane;
        const uint64_t v = src >= 0 ? load_status(status + src) : kFlagPrefix;   // before ticket 0: prefix 0
        const uint64_t fl = v & kFlagMask;
        const bool ready = fl != 0 && (src < 0 || ((uint32_t)(v >> 32) & kEpochMask) == ep);
        const uint64_t pm = ballot(ready && fl == kFlagPrefix);
        const uint64_t rm = ballot(ready);
        const uint32_t first = pm ? (uint32_t)__builtin_ctzll(pm) : 64u;
        const uint64_t need = first >= 63u ? ~0ull : ((2ull << first) - 1ull);
        if ((rm & need) == need) {
            excl += wave_sum_u32(lane <= first ? (uint32_t)v : 0u);
            if (first < 64u) break;
            j -= 64;
            continue;
        }
        if (++spins > spin_limit) {
            if (lane == 0) atomicOr(err, kErrLookBack);
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    if (lane == 0) store_status(status + bid, status_word(kFlagPrefix, epoch, excl + total));
    return excl;
}

__device__ __forceinline__ int64_t resolve_n(const uint32_t* d_n, int64_t max_n) {
    return d_n ? (int64_t)min((int64_t)*d_n, max_n) : max_n;
}

// Ballot match of an n-bit digit: lanes of the wave with the same digit
// (among `valid` lanes).
__device__ __forceinline__ uint64_t match_digit(uint32_t d, int bits, bool valid) {
    uint64_t peers = ballot(valid);
    for (int b = 0; b < bits; ++b) {
        const bool bit = (d >> b) & 1u;
        const uint64_t m = ballot(bit);
        peers &= bit ? m : ~m;
    }
    return peers;
}

// ---------------------------------------------------------------- compaction

// Visible primitives (n_touched > 0) in index order -> (depth key, index,
// n_touched) triples, compacted inside each 4096-primitive block (block b's
// visible ones at [4096 b, 4096 b + block_n[b]), in index order): the depth
// sort's first pass takes these blocks as its input blocks, so the same kernel
// counts their first-pass digits (counts[d * nb + b], the pass's upsweep) and
// no device-wide scan is needed. V and I = sum of n_touched by one atomic add
// per block each (integer sums: the same totals in any order).
static_assert(kScanChunk == kThreads * kDepthKeysPerThread, "compaction blocks are the depth sort's blocks");
__global__ void __launch_bounds__(kScanThreads) compact_count_kernel(const uint32_t* __restrict__ n_touched,
                                                                 const uint32_t* __restrict__ depth_key, int64_t n,
                                                                 uint32_t key_base, int shift, int bits,
                                                                 uint32_t* __restrict__ keys_out,
                                                                 uint32_t* __restrict__ vals_out,
                                                                 uint32_t* __restrict__ nt_out,
                                                                 uint32_t* __restrict__ counts,
                                                                 uint32_t* __restrict__ block_n, BinCtl* ctl) {
    __shared__ uint32_t s_rw[64];
    __shared__ uint32_t s_nt[kScanWaves];
    __shared__ uint32_t s_hist[kHistCopies][kDepthMaxDigits + kHistPad];
    const uint32_t t = threadIdx.x, lane = t & 63u, w = t >> 6;
    const uint32_t b = blockIdx.x, nb = gridDim.x;
    const uint32_t bins = 1u << bits, dmask = bins - 1u;
    for (uint32_t e = t; e < (uint32_t)(kHistCopies * (kDepthMaxDigits + kHistPad)); e += kScanThreads)
        (&s_hist[0][0])[e] = 0u;
    const int64_t blk = (int64_t)b * kScanChunk;
    const int64_t base = blk + t;
    uint32_t key[kScanRounds], nt[kScanRounds], vis[kScanRounds], ex[kScanRounds];
    uint32_t ntsum = 0;
#pragma unroll
    for (int r = 0; r < kScanRounds; ++r) {
        const int64_t i = base + (int64_t)r * kScanThreads;
        nt[r] = i < n ? n_touched[i] : 0u;
        key[r] = i < n ? depth_key[i] - key_base : 0u;
    }
#pragma unroll
    for (int r = 0; r < kScanRounds; ++r) {
        vis[r] = nt[r] > 0u ? 1u : 0u;
        ntsum += nt[r];
    }
    const uint32_t wnt = wave_sum_u32(ntsum);
    if (lane == 0) s_nt[w] = wnt;
    uint32_t total;
    striped_scan_u32<kScanRounds, kScanWaves>(vis, ex, &total, s_rw);   // barriers inside: s_nt and the zeroed histograms visible after it
#pragma unroll
    for (int r = 0; r < kScanRounds; ++r) {
        if (vis[r]) {
            const int64_t pos = blk + ex[r];
            keys_out[pos] = key[r];
            vals_out[pos] = (uint32_t)(base + (int64_t)r * kScanThreads);
            nt_out[pos] = nt[r];
            atomicAdd(&s_hist[lane & (kHistCopies - 1)][(key[r] >> shift) & dmask], 1u);
        }
    }
    if (t == 0) {
        block_n[b] = total;
        if (total) atomicAdd(&ctl->V, total);
        uint32_t bsum = 0;
        for (int k = 0; k < kScanWaves; ++k) bsum += s_nt[k];
        if (bsum) atomicAdd(&ctl->I, bsum);
    }
    __syncthreads();
    for (uint32_t d = t; d < bins; d += kScanThreads) {
        uint32_t c = 0;
#pragma unroll
        for (int k = 0; k < kHistCopies; ++k) c += s_hist[k][d];
        counts[(size_t)d * nb + b] = c;
    }
}

void launch_compact_visible(const uint32_t* n_touched, const uint32_t* depth_key, int64_t n, uint32_t key_base,
                            int shift, int bits, uint32_t* keys_out, uint32_t* vals_out, uint32_t* nt_out,
                            uint32_t* counts, uint32_t* block_n, BinCtl* ctl, hipStream_t s) {
    if (n <= 0) return;
    const uint32_t nb = (uint32_t)((n + kScanChunk - 1) / kScanChunk);
    compact_count_kernel<<<nb, kScanThreads, 0, s>>>(n_touched, depth_key, n, key_base, shift, bits, keys_out, vals_out,
                                                 nt_out, counts, block_n, ctl);
}

// ---------------------------------------------------------------- instance offsets

// offs[k] = exclusive scan of nt[k] (n_touched in depth order) over k < V;
// offs[V] = the total.
__global__ void __launch_bounds__(kScanThreads) offsets_kernel(const uint32_t* __restrict__ nt, int64_t max_count,
                                                           uint32_t* __restrict__ offs, BinCtl* ctl,
                                                           uint64_t* status, uint32_t epoch) {
    __shared__ uint32_t s_rw[64];
    __shared__ uint32_t s_bid, s_base;
    const uint32_t t = threadIdx.x, lane = t & 63u, w = t >> 6;
    const uint32_t bid = take_ticket(&ctl->tickets[kTicketOffsets], &s_bid);
    const int64_t n = resolve_n(&ctl->V, max_count);
    if ((int64_t)bid * kScanChunk >= n) return;
    const int64_t base = (int64_t)bid * kScanChunk + t;
    uint32_t c[kScanRounds], ex[kScanRounds];
#pragma unroll
    for (int r = 0; r < kScanRounds; ++r) {
        const int64_t i = base + (int64_t)r * kScanThreads;
        c[r] = i < n ? nt[i] : 0u;
    }
    uint32_t total;
    striped_scan_u32<kScanRounds, kScanWaves>(c, ex, &total, s_rw);
    if (w == 0) {
        const uint32_t excl = wave_look_back(status, bid, total, ctl->epoch_base + epoch, &ctl->err);
        if (lane == 0) {
            s_base = excl;
            if ((int64_t)(bid + 1) * kScanChunk >= n) offs[n] = excl + total;
        }
    }
    __syncthreads();
    const uint32_t b0 = s_base;
#pragma unroll
    for (int r = 0; r < kScanRounds; ++r) {
        const int64_t i = base + (int64_t)r * kScanThreads;
        if (i < n) offs[i] = b0 + ex[r];
    }
}

void launch_instance_offsets(const uint32_t* nt_sorted, int64_t max_count, uint32_t* offs, BinCtl* ctl,
                             uint64_t* status, uint32_t& epoch, hipStream_t s) {
    if (max_count <= 0) return;
    const uint32_t nb = (uint32_t)((max_count + kScanChunk - 1) / kScanChunk);
    offsets_kernel<<<nb, kScanThreads, 0, s>>>(nt_sorted, max_count, offs, ctl, status, ++epoch);
}

int64_t scan_status_entries(int64_t max_n) { return (max_n + kScanChunk - 1) / kScanChunk; }

// ---------------------------------------------------------------- radix sort (reduce-then-scan)

// Wave w of a workgroup owns 64 * KPT consecutive keys: round r, lane l is
// key blk + w * 64 * KPT + r * 64 + l. Digit ranks come from ballot matching
// against a wave-private LDS histogram (a wave's LDS operations complete in
// issue order, so rounds need no barrier).
template <int KPT, int MAXB>
__device__ __forceinline__ void rank_keys(const uint32_t key[KPT], int64_t base, int64_t n, int shift, int bits,
                                          uint32_t (*s_cnt)[MAXB], uint32_t pos[KPT]) {
    const uint32_t lane = threadIdx.x & 63u, w = threadIdx.x >> 6;
    const uint32_t dmask = (1u << bits) - 1u;
#pragma unroll
    for (int r = 0; r < KPT; ++r) {
        const bool valid = base + (int64_t)r * 64 + lane < n;
        const uint32_t d = (key[r] >> shift) & dmask;
        const uint64_t peers = match_digit(d, bits, valid);
        const uint32_t rank = mask_rank(peers);
        const uint32_t running = s_cnt[w][d];
        pos[r] = running + rank;
        if (valid && rank == 0u) s_cnt[w][d] = running + (uint32_t)__builtin_popcountll(peers);
    }
}

// Per-workgroup digit counts: counts[d * nb + b] (digit-major). Workgroups
// past the end write zeros. Counting needs no ranks: one LDS atomic add per
// key into one of kHistCopies histograms (by lane), summed at the end: keys
// that arrive clustered (the instances of one primitive share their tile
// digits) would otherwise serialise on one address.
// NTSUM (the depth sort's last pass): the same matrix of the payload's sums
// (n_touched) per (digit, workgroup) goes to ntsums, from which the last
// downsweep writes the instance offsets.
template <int KPT, int MAXB, int NW, bool NTSUM = false>
__global__ void __launch_bounds__(64 * NW) radix_upsweep_kernel(const uint32_t* __restrict__ keys,
                                                                const uint32_t* __restrict__ v2,
                                                                const uint32_t* d_n, int64_t max_n, int shift,
                                                                int bits, uint32_t* __restrict__ counts,
                                                                uint32_t* __restrict__ ntsums, uint32_t nb,
                                                                uint2* __restrict__ rinit, uint32_t n_tiles,
                                                                uint32_t* __restrict__ clear_bits) {
    constexpr int kNT = 64 * NW;
    // rinit: the tile ranges the next downsweep reduces into, set to (UINT32_MAX, 0)
    if (rinit)
        for (uint32_t j = blockIdx.x * kNT + threadIdx.x; j < n_tiles; j += gridDim.x * kNT)
            rinit[j] = make_uint2(0xffffffffu, 0u);
    // clear_bits: one bit per key position (the 2D-gradient record marks of
    // the next backward); this workgroup's 64 KPT NW positions are whole words
    if (clear_bits)
        for (uint32_t j = threadIdx.x; j < (uint32_t)(KPT * NW * 2); j += kNT)
            clear_bits[(size_t)blockIdx.x * (KPT * NW * 2) + j] = 0u;
    __shared__ uint32_t s_hist[kHistCopies][MAXB + kHistPad];
    __shared__ uint32_t s_hsum[NTSUM ? kHistCopies : 1][NTSUM ? MAXB + kHistPad : 1];
    const uint32_t t = threadIdx.x, lane = t & 63u, w = t >> 6;
    const uint32_t bins = 1u << bits, dmask = bins - 1u;
    for (uint32_t b = t; b < (uint32_t)(kHistCopies * (MAXB + kHistPad)); b += kNT) {
        (&s_hist[0][0])[b] = 0u;
        if constexpr (NTSUM) (&s_hsum[0][0])[b] = 0u;
    }
    __syncthreads();
    const int64_t n = resolve_n(d_n, max_n);
    const int64_t base = (int64_t)blockIdx.x * (kNT * KPT) + (int64_t)w * (64 * KPT);
    uint32_t key[KPT], nt[NTSUM ? KPT : 1];
#pragma unroll
    for (int r = 0; r < KPT; ++r) {
        const int64_t i = base + (int64_t)r * 64 + lane;
        key[r] = i < n ? keys[i] : 0u;
        if constexpr (NTSUM) nt[r] = i < n ? v2[i] : 0u;
    }
#pragma unroll
    for (int r = 0; r < KPT; ++r)
        if (base + (int64_t)r * 64 + lane < n) {
            const uint32_t d = (key[r] >> shift) & dmask, c = lane & (kHistCopies - 1);
            atomicAdd(&s_hist[c][d], 1u);
            if constexpr (NTSUM) atomicAdd(&s_hsum[c][d], nt[r]);
        }
    __syncthreads();
    for (uint32_t b = t; b < bins; b += kNT) {
        uint32_t c = 0, sum = 0;
#pragma unroll
        for (int k = 0; k < kHistCopies; ++k) {
            c += s_hist[k][b];
            if constexpr (NTSUM) sum += s_hsum[k][b];
        }
        counts[(size_t)b * nb + blockIdx.x] = c;
        if constexpr (NTSUM) ntsums[(size_t)b * nb + blockIdx.x] = sum;
    }
}

// In-place exclusive scan of a u32 array of n elements (single pass,
// decoupled look-back). Applied to the digit-major count matrix it yields
// every (digit, workgroup) output offset: digit start + counts of earlier
// workgroups for that digit.
__global__ void __launch_bounds__(kScanThreads) exclusive_scan_kernel(uint32_t* __restrict__ data, int64_t n,
                                                                  uint32_t* ticket, uint64_t* status,
                                                                  const uint32_t* epoch_base, uint32_t epoch,
                                                                  uint32_t* err) {
    __shared__ uint32_t s_rw[64];
    __shared__ uint32_t s_bid, s_base;
    const uint32_t t = threadIdx.x, lane = t & 63u, w = t >> 6;
    const uint32_t bid = take_ticket(ticket, &s_bid);
    const int64_t base = (int64_t)bid * kScanChunk + t;
    uint32_t c[kScanRounds], ex[kScanRounds];
#pragma unroll
    for (int r = 0; r < kScanRounds; ++r) {
        const int64_t i = base + (int64_t)r * kScanThreads;
        c[r] = i < n ? data[i] : 0u;
    }
    uint32_t total;
    striped_scan_u32<kScanRounds, kScanWaves>(c, ex, &total, s_rw);
    if (w == 0) {
        const uint32_t excl = wave_look_back(status, bid, total, *epoch_base + epoch, err);
        if (lane == 0) s_base = excl;
    }
    __syncthreads();
    const uint32_t b0 = s_base;
#pragma unroll
    for (int r = 0; r < kScanRounds; ++r) {
        const int64_t i = base + (int64_t)r * kScanThreads;
        if (i < n) data[i] = b0 + ex[r];
    }
}

// Ranked scatter of one pass: keys (and one or two u32 payloads) go to
// offset(digit, workgroup) + rank within the workgroup's run of that digit.
// The workgroup's keys are first placed in LDS in digit order and written
// out by consecutive threads, so each store instruction covers contiguous
// runs.
//
// OFFS (the depth sort's last pass, payload 2 = n_touched): instead of the
// sorted n_touched, writes offs[o] = the sum of n_touched over the sorted
// positions before o (the instance offsets) and offs[n] = the total. ntscan
// is the exclusive scan of [counts, ntsums] (one look-back scan of both
// matrices): ntscan[j] - ntscan[0] is the n_touched sum of the keys of
// digit < d plus those of digit d in earlier workgroups, for j = d nb + b;
// the workgroup adds its own sum before the key, from one scan of its keys in
// LDS (digit) order less that scan at the start of the key's digit run.
//
// RANGES (the tile sort's last pass, all key bits sorted): also reduces the
// per-tile instance ranges. The output is then sorted by the whole key, and a
// workgroup's keys in LDS order are its runs of equal keys; the first key of
// each run takes atomicMin into ranges[key].x and the last atomicMax of its
// position + 1 into ranges[key].y (set to (UINT32_MAX, 0) by the upsweep), so
// a tile's range ends as the first and past-the-last position of its key:
// the global first key of a tile is always the first of a workgroup run.
// Empty tiles keep (UINT32_MAX, 0) (the forward blend writes (0, 0) there).
// The sorted keys are not written: the ranges hold them
// (launch_keys_from_ranges restores them).
template <int KPT, bool PAYLOAD2, int MAXB, int NW, bool OFFS = false, bool RANGES = false>
__global__ void __launch_bounds__(64 * NW) radix_downsweep_kernel(
    const uint32_t* __restrict__ keys_in, const uint32_t* __restrict__ vals_in, const uint32_t* __restrict__ v2_in,
    uint32_t* __restrict__ keys_out, uint32_t* __restrict__ vals_out, uint32_t* __restrict__ v2_out,
    const uint32_t* d_n, int64_t max_n, int shift, int bits, const uint32_t* __restrict__ offsets, uint32_t nb,
    const uint32_t* __restrict__ block_n, const uint32_t* __restrict__ ntscan, uint32_t* __restrict__ offs,
    uint2* __restrict__ ranges, uint32_t n_tiles, uint16_t* __restrict__ ranks) {
    constexpr int kNT = 64 * NW;             // threads
    constexpr int kChunk = kNT * KPT;
    constexpr int kBpt = MAXB > kNT ? MAXB / kNT : 1;   // digits per thread in the workgroup scan
    static_assert(MAXB % kNT == 0 || kNT % MAXB == 0, "digits split evenly over the threads");
    static_assert(!OFFS || (PAYLOAD2 && KPT * NW <= 64), "offsets from the n_touched payload, one striped scan");
    __shared__ uint32_t s_cnt[NW][MAXB];
    __shared__ uint32_t s_gofs[MAXB];
    __shared__ uint32_t s_key[kChunk], s_val[kChunk], s_v2[PAYLOAD2 ? kChunk : 1];
    __shared__ uint32_t s_wave[NW];
    __shared__ uint32_t s_ntg[OFFS ? MAXB : 1], s_est[OFFS ? MAXB : 1], s_rw[OFFS ? 64 : 1];
    const uint32_t t = threadIdx.x, lane = t & 63u, w = t >> 6;
    const uint32_t bins = 1u << bits, dmask = bins - 1u;
    const int64_t blk = (int64_t)blockIdx.x * kChunk;
    // block_n: this block holds block_n[b] keys from its start (a compacted
    // block of the first depth pass); otherwise the first n keys are dense
    const int64_t n = block_n ? blk + (int64_t)block_n[blockIdx.x] : resolve_n(d_n, max_n);
    if (blk >= n) return;
    for (int k = t; k < NW * MAXB; k += kNT) (&s_cnt[0][0])[k] = 0;
    uint32_t gofs[kBpt];   // thread t owns digits kBpt t .. kBpt t + kBpt - 1
#pragma unroll
    for (int q = 0; q < kBpt; ++q) {
        const uint32_t d = kBpt * t + (uint32_t)q;
        gofs[q] = d < bins ? offsets[(size_t)d * nb + blockIdx.x] : 0u;
        if constexpr (OFFS)
            if (d < bins) s_ntg[d] = ntscan[(size_t)d * nb + blockIdx.x] - ntscan[0];
    }
    __syncthreads();
    const int64_t base = blk + (int64_t)w * (64 * KPT);
    uint32_t key[KPT], val[KPT], v2[PAYLOAD2 ? KPT : 1], pos[KPT];
#pragma unroll
    for (int r = 0; r < KPT; ++r) {
        const int64_t i = base + (int64_t)r * 64 + lane;
        const bool valid = i < n;
        key[r] = valid ? keys_in[i] : 0u;
        val[r] = valid ? vals_in[i] : 0u;
        if constexpr (PAYLOAD2) v2[r] = valid ? v2_in[i] : 0u;
    }
    rank_keys<KPT, MAXB>(key, base, n, shift, bits, s_cnt, pos);
    __syncthreads();
    uint32_t c[kBpt][NW], tot[kBpt], total = 0;
#pragma unroll
    for (int q = 0; q < kBpt; ++q) {
        const uint32_t d = kBpt * t + (uint32_t)q;
        tot[q] = 0;
#pragma unroll
        for (int k = 0; k < NW; ++k) {
            c[q][k] = d < bins ? s_cnt[k][d] : 0u;
            tot[q] += c[q][k];
        }
        total += tot[q];
    }
    uint32_t unused;
    uint32_t lstart = block_exclusive_scan<NW>(total, s_wave, &unused);   // digit start inside the workgroup
#pragma unroll
    for (int q = 0; q < kBpt; ++q) {
        const uint32_t d = kBpt * t + (uint32_t)q;
        if (d < bins) {
            s_gofs[d] = gofs[q] - lstart;
            uint32_t run = lstart;
#pragma unroll
            for (int k = 0; k < NW; ++k) {
                s_cnt[k][d] = run;
                run += c[q][k];
            }
        }
        lstart += tot[q];
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < KPT; ++r) {
        if (base + (int64_t)r * 64 + lane < n) {
            const uint32_t l = s_cnt[w][(key[r] >> shift) & dmask] + pos[r];
            s_key[l] = key[r];
            s_val[l] = val[r];
            if constexpr (PAYLOAD2) s_v2[l] = v2[r];
        }
    }
    __syncthreads();
    const uint32_t cnt = (uint32_t)min((int64_t)kChunk, n - blk);
    if constexpr (OFFS) {
        // n_touched prefix over the LDS (digit) order; the prefix at each digit run's start
        uint32_t nt[KPT], ex[KPT], sum;
#pragma unroll
        for (int r = 0; r < KPT; ++r) {
            const uint32_t i = t + (uint32_t)r * kNT;
            nt[r] = i < cnt ? s_v2[i] : 0u;
        }
        striped_scan_u32<KPT, NW>(nt, ex, &sum, s_rw);
#pragma unroll
        for (int r = 0; r < KPT; ++r) {
            const uint32_t i = t + (uint32_t)r * kNT;
            if (i < cnt) {
                const uint32_t d = (s_key[i] >> shift) & dmask;
                if (i == 0u || ((s_key[i - 1] >> shift) & dmask) != d) s_est[d] = ex[r];
            }
        }
        __syncthreads();
#pragma unroll
        for (int r = 0; r < KPT; ++r) {
            const uint32_t i = t + (uint32_t)r * kNT;
            if (i < cnt) {
                const uint32_t k = s_key[i], d = (k >> shift) & dmask;
                const uint32_t o = s_gofs[d] + i;
                if (o < (uint64_t)max_n) {   // always true when the counts match the keys
                    const uint32_t off = s_ntg[d] + (ex[r] - s_est[d]);
                    keys_out[o] = k;
                    vals_out[o] = s_val[i];
                    offs[o] = off;
                    if ((int64_t)o + 1 == n) offs[n] = off + nt[r];   // the total after the last key
                }
            }
        }
        return;
    }
    // RANGES: the key's sorted bits (all bits below shift + bits) are the
    // tile; bits above them carry the instance's rank among its primitive's
    // instances (fp32 images), written to ranks
    const uint32_t tmask = shift + bits >= 32 ? 0xffffffffu : (1u << (shift + bits)) - 1u;
    for (uint32_t i = t; i < cnt; i += kNT) {
        const uint32_t k = s_key[i];
        const uint32_t o = s_gofs[(k >> shift) & dmask] + i;
        if (o < (uint64_t)max_n) {   // always true when the counts match the keys
            if constexpr (!RANGES) keys_out[o] = k;
            vals_out[o] = s_val[i];
            if constexpr (PAYLOAD2) v2_out[o] = s_v2[i];
            if constexpr (RANGES) {
                const uint32_t tk = k & tmask;
                if (ranks) ranks[o] = (uint16_t)(k >> 16);
                if (tk < n_tiles) {
                    if (i == 0u || (s_key[i - 1u] & tmask) != tk) atomicMin(&ranges[tk].x, o);
                    if (i + 1u == cnt || (s_key[i + 1u] & tmask) != tk) atomicMax(&ranges[tk].y, o + 1u);
                }
            }
        }
    }
}

int64_t radix_count_entries(int64_t max_n, bool depth) {
    const int64_t chunk = kThreads * (depth ? kDepthKeysPerThread : kTileKeysPerThread);
    // the depth sort's last pass also holds the n_touched sums
    return ((max_n + chunk - 1) / chunk) * (depth ? 2 * kDepthMaxDigits : kTileMaxDigits);
}

// DW: waves per upsweep / downsweep workgroup; the keys per thread shrink so
// that a workgroup still covers 256 KPT keys.
// offs (depth sort, n_touched in v2): the last pass writes the instance
// offsets (offs_done = true) when it has its own upsweep (two passes or
// more); otherwise the caller scans them (launch_instance_offsets).
// ranges (tile sort): the last pass reduces the tile ranges (ranges_done =
// true) whenever it runs; otherwise the caller derives them
// (launch_tile_ranges).
template <int KPT, int MAXB, int DW>
static int radix_passes(uint32_t* keys[2], uint32_t* vals[2], uint32_t* v2[2], const uint32_t* d_n, int64_t max_n,
                        int n_passes, const int* shifts, const int* bits, uint32_t* counts, uint32_t* tickets,
                        uint64_t* status, const uint32_t* epoch_base, uint32_t& epoch, uint32_t* err,
                        const uint32_t* first_block_n, uint32_t* offs, bool* offs_done, uint2* ranges,
                        uint32_t n_tiles, bool* ranges_done, uint16_t* ranks, uint32_t* clear_bits, hipStream_t s) {
    int cur = 0;
    if (offs_done) *offs_done = false;
    if (ranges_done) *ranges_done = false;
    if (max_n <= 0) return cur;
    const uint32_t nb = (uint32_t)((max_n + kThreads * KPT - 1) / (kThreads * KPT));
    constexpr int kDownKpt = KPT * (kThreads / 64) / DW;
    static_assert(kDownKpt * 64 * DW == KPT * kThreads, "blocks of 256 KPT keys");
    for (int p = 0; p < n_passes; ++p) {
        if ((1 << bits[p]) > MAXB) return -1;
        const int64_t cn = (int64_t)nb << bits[p];
        // first_block_n: the first pass's blocks and digit counts come from the compaction
        const uint32_t* block_n = p == 0 ? first_block_n : nullptr;
        const bool with_offs = offs && offs_done && v2 && p == n_passes - 1 && p > 0;
        if constexpr (MAXB == kDepthMaxDigits) {
            if (with_offs) {
                radix_upsweep_kernel<kDownKpt, MAXB, DW, true><<<nb, 64 * DW, 0, s>>>(
                    keys[cur], v2[cur], d_n, max_n, shifts[p], bits[p], counts, counts + cn, nb, nullptr, 0u,
                    nullptr);
                exclusive_scan_kernel<<<(unsigned)((2 * cn + kScanChunk - 1) / kScanChunk), kScanThreads, 0, s>>>(
                    counts, 2 * cn, tickets + p, status, epoch_base, ++epoch, err);
                radix_downsweep_kernel<kDownKpt, true, MAXB, DW, true><<<nb, 64 * DW, 0, s>>>(
                    keys[cur], vals[cur], v2[cur], keys[cur ^ 1], vals[cur ^ 1], nullptr, d_n, max_n, shifts[p],
                    bits[p], counts, nb, nullptr, counts + cn, offs, nullptr, 0u, nullptr);
                *offs_done = true;
                cur ^= 1;
                continue;
            }
        }
        const bool with_ranges = ranges && ranges_done && !v2 && !block_n && p == n_passes - 1;
        if (!block_n)
            radix_upsweep_kernel<kDownKpt, MAXB, DW><<<nb, 64 * DW, 0, s>>>(
                keys[cur], nullptr, d_n, max_n, shifts[p], bits[p], counts, nullptr, nb,
                with_ranges ? ranges : nullptr, n_tiles, p == 0 ? clear_bits : nullptr);
        exclusive_scan_kernel<<<(unsigned)((cn + kScanChunk - 1) / kScanChunk), kScanThreads, 0, s>>>(
            counts, cn, tickets + p, status, epoch_base, ++epoch, err);
        if (v2)
            radix_downsweep_kernel<kDownKpt, true, MAXB, DW><<<nb, 64 * DW, 0, s>>>(
                keys[cur], vals[cur], v2[cur], keys[cur ^ 1], vals[cur ^ 1], v2[cur ^ 1], d_n, max_n, shifts[p],
                bits[p], counts, nb, block_n, nullptr, nullptr, nullptr, 0u, nullptr);
        else if (with_ranges) {
            radix_downsweep_kernel<kDownKpt, false, MAXB, DW, false, true><<<nb, 64 * DW, 0, s>>>(
                keys[cur], vals[cur], nullptr, keys[cur ^ 1], vals[cur ^ 1], nullptr, d_n, max_n, shifts[p], bits[p],
                counts, nb, nullptr, nullptr, nullptr, ranges, n_tiles, ranks);
            *ranges_done = true;
        } else
            radix_downsweep_kernel<kDownKpt, false, MAXB, DW><<<nb, 64 * DW, 0, s>>>(
                keys[cur], vals[cur], nullptr, keys[cur ^ 1], vals[cur ^ 1], nullptr, d_n, max_n, shifts[p], bits[p],
                counts, nb, block_n, nullptr, nullptr, nullptr, 0u, nullptr);
        cur ^= 1;
    }
    return cur;
}

int radix_sort(uint32_t* keys[2], uint32_t* vals[2], uint32_t* v2[2], const uint32_t* d_n, int64_t max_n, bool depth,
               int n_passes, const int* shifts, const int* bits, uint32_t* counts, uint32_t* tickets,
               uint64_t* status, const uint32_t* epoch_base, uint32_t& epoch, uint32_t* err,
               const uint32_t* first_block_n, uint32_t* offs, bool* offs_done, uint2* ranges, uint32_t n_tiles,
               bool* ranges_done, uint16_t* ranks, uint32_t* clear_bits, hipStream_t s) {
    if (depth)
        return radix_passes<kDepthKeysPerThread, kDepthMaxDigits, kDepthSortWaves>(
            keys, vals, v2, d_n, max_n, n_passes, shifts, bits, counts, tickets, status, epoch_base, epoch, err,
            first_block_n, offs, offs_done, nullptr, 0u, ranges_done, nullptr, nullptr, s);
    return radix_passes<kTileKeysPerThread, kTileMaxDigits, kTileSortWaves>(
        keys, vals, v2, d_n, max_n, n_passes, shifts, bits, counts, tickets, status, epoch_base, epoch, err,
        first_block_n, nullptr, offs_done, ranges, n_tiles, ranges_done, ranks, clear_bits, s);
}

int64_t record_bit_words(int64_t max_inst) {
    const int64_t chunk = kThreads * kTileKeysPerThread;   // the tile passes' workgroup positions
    return ((max_inst > 0 ? max_inst : 1) + chunk - 1) / chunk * (chunk / 32);
}

// ---------------------------------------------------------------- instance emission

// kernels_forward.cuh:49-84 (same expression as in preprocess.hip)
__device__ __forceinline__ bool will_contribute_e(float mx, float my, float ca, float cb, float cc, uint32_t tile_x,
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

// Thread per depth-sorted primitive: its 16-byte emission record (bounds and
// the preprocess's outcomes for rect tiles 0..31) is gathered once, its mean,
// conic and threshold only for primitives with more than 32 rect tiles (from
// the blend's own per-primitive arrays); its instances fill the slots [offs[k], offs[k + 1]),
// so the instance array comes out in depth order. (The gathers are random:
// depth order is not index order, and each costs a whole memory line.) The
// rect tiles of a wave's 64 primitives are walked as one task list, 64 per
// step, whatever the rect sizes.
// The workgroup's 256 primitives own one contiguous slot range; when it fits
// in LDS the instances are staged there and written out by consecutive
// threads (contiguous stores), otherwise written directly. 2048 slots (256
// primitives average about 1300 instances at config 3) keep the LDS at
// 17 KB, so eight workgroups fit a CU; 4096 slots halved that (7 us slower).
constexpr uint32_t kEmitStage = 2048;

// The tile test of the record's rasterizer: fp32 (conic floats in w0..w2) or
// FGS16 (half conic a | b << 16 in w0, c | opacity << 16 in w1).
template <bool kHalf>
__device__ __forceinline__ bool emit_test(float mx, float my, uint32_t w0, uint32_t w1, uint32_t w2, uint32_t tx,
                                          uint32_t ty, float pt) {
    if constexpr (kHalf)
        return will_contribute_half(mx, my, hfrom((uint16_t)(w0 & 0xffffu)), hfrom((uint16_t)(w0 >> 16)),
                                    hfrom((uint16_t)(w1 & 0xffffu)), tx, ty, pt);
    else
        return will_contribute_e(mx, my, u2f(w0), u2f(w1), u2f(w2), tx, ty, pt);
}

template <bool kHalf>
__global__ void __launch_bounds__(256) emit_kernel(const uint32_t* __restrict__ prims,
                                                   const uint32_t* __restrict__ offs, BinCtl* ctl,
                                                   int64_t max_count, int64_t max_inst,
                                                   const float2* __restrict__ mean2d,
                                                   const uint4* __restrict__ conic_words,
                                                   const uint4* __restrict__ thr_words,
                                                   const uint4* __restrict__ erec, uint32_t grid_w,
                                                   uint32_t* __restrict__ inst_keys,
                                                   uint32_t* __restrict__ inst_vals,
                                                   uint32_t* __restrict__ first_slot) {
    __shared__ uint32_t s_key[kEmitStage], s_val[kEmitStage];
    __shared__ uint32_t s_marks[4][kWave];
    const uint32_t t = threadIdx.x;
    // more instances than the buffers hold (a no-sync forward's reserved
    // capacity; a waiting forward sizes them to the count): flagged for
    // tgs_rasterizer_status, the slots beyond it are not written
    if (blockIdx.x == 0 && t == 0 && (int64_t)ctl->I > max_inst) atomicOr(&ctl->err, kErrCapacity);
    const int64_t n = min((int64_t)ctl->V, max_count);
    const int64_t k0 = (int64_t)blockIdx.x * blockDim.x;
    if (k0 >= n) return;
    // a failed look-back scan of the depth sort (set before this launch, so
    // the same for every thread) leaves a partial order: nothing is emitted
    if (ctl->err & kErrLookBack) return;
    const uint32_t range_a = offs[k0], range_b = offs[min(k0 + (int64_t)blockDim.x, n)];
    // Slots come from the offsets scan and stay below the instance count the
    // buffers were sized for; a slot beyond it (offsets broken by a failed
    // scan) is dropped and flagged instead of written.
    const bool in_range = range_a <= range_b && (int64_t)range_b <= max_inst;
    const bool staged = in_range && range_b - range_a <= kEmitStage;
    // (past a reserved capacity that the instances exceed is kErrCapacity's case)
    if (t == 0 && !in_range && (int64_t)ctl->I <= max_inst) atomicOr(&ctl->err, kErrOffsets);
    auto put = [&](uint32_t pos, uint32_t tile, uint32_t prim) {
        if (staged) {
            const uint32_t l = pos - range_a;   // < kEmitStage whenever the offsets are monotone
            if (l < kEmitStage) {
                s_key[l] = tile;
                s_val[l] = prim;
            }
        } else if ((int64_t)pos < max_inst) {
            inst_keys[pos] = tile;
            inst_vals[pos] = prim;
        }
    };
    const int64_t k = k0 + t;
    const bool active = k < n;
    const uint32_t lane = lane_id();
    uint32_t p = 0, off = 0, cap = 0, x0 = 0, x1 = 0, y0 = 0, y1 = 0, bits = 0;
    float smx = 0.f, smy = 0.f, pt = 0.f;
    uint32_t cw0 = 0, cw1 = 0, cw2 = 0;
    if (active) {
        p = prims[k];
        off = offs[k];
        cap = offs[k + 1] - off;   // slots reserved for this primitive (= its n_touched)
        // a capacity the instances outgrow (no-sync forward): the slots below
        // it are still all written, so the sorted prefix holds valid pairs only
        if ((int64_t)off + cap > max_inst) cap = (int64_t)off < max_inst ? (uint32_t)(max_inst - off) : 0u;
        first_slot[p] = off;
        const uint4 e = erec[p];
        x0 = e.x & 0xffffu; x1 = e.x >> 16; y0 = e.y & 0xffffu; y1 = e.y >> 16;
        bits = e.z;
        if ((x1 - x0) * (y1 - y0) > 32u) {   // tiles past the first 32 need the exact test
            const float2 m = mean2d[p];
            const uint4 cw = conic_words[p];
            smx = m.x - 0.5f;
            smy = m.y - 0.5f;
            cw0 = cw.x; cw1 = cw.y; cw2 = cw.z;
            pt = u2f(kHalf ? cw.w : thr_words[p].w);
        }
    }
    // The wave's rect tiles as one task list (rect_tasks.h); rect tiles
    // 0..31 were tested by the preprocess (emission record). A hit's slot is
    // its primitive's first slot plus the number of its hits before it: the
    // hits in earlier windows (only the primitive carried into the window has
    // any) and those of this window on lower lanes of its segment.
    const uint32_t bw = x1 - x0;
    const uint32_t nr = active ? bw * (y1 - y0) : 0u;
    const uint32_t incl = wave_inclusive_scan_u32(nr);
    const uint32_t total = readlane_u32(incl, 63);
    const uint32_t ex = incl - nr, org = x0 | (y0 << 16), end = off + cap;
    uint32_t* s_mark = s_marks[t >> 6];
    uint32_t carry = 0, carry_hits = 0;
    for (uint32_t base = 0; base < total; base += kWave) {
        const uint32_t prev = carry;
        const uint32_t j = wave_task_owner(s_mark, nr, ex, base, carry);
        const uint32_t exj = lane_gather(j, ex), orgj = lane_gather(j, org), wj = lane_gather(j, bw);
        const uint32_t bitsj = lane_gather(j, bits), offj = lane_gather(j, off), endj = lane_gather(j, end);
        const uint32_t pj = lane_gather(j, p);
        const uint32_t tt = base + lane;
        const uint32_t q = tt - exj;
        uint32_t tx = 0, ty = 0;
        bool hit = false;
        if (tt < total) {
            uint32_t col, row;
            rect_tile_of(q, wj, col, row);
            tx = (orgj & 0xffffu) + col;
            ty = (orgj >> 16) + row;
            hit = q < 32u && ((bitsj >> q) & 1u) != 0u;
        }
        if (ballot(tt < total && q >= 32u)) {   // the exact test, with the owner's record
            const float s_mx = u2f(lane_gather(j, f2u(smx))), s_my = u2f(lane_gather(j, f2u(smy)));
            const uint32_t s_a = lane_gather(j, cw0), s_b = lane_gather(j, cw1), s_c = lane_gather(j, cw2);
            const float s_t = u2f(lane_gather(j, f2u(pt)));
            if (tt < total && q >= 32u) hit = emit_test<kHalf>(s_mx, s_my, s_a, s_b, s_c, tx, ty, s_t);
        }
        const uint64_t hm = ballot(hit);
        const uint32_t seg = exj > base ? exj - base : 0u;   // the owner's first lane in this window
        const uint64_t below = hm & ((1ull << lane) - 1ull) & ~((1ull << seg) - 1ull);
        const uint32_t pos = offj + (j + 1u == prev ? carry_hits : 0u) + (uint32_t)__builtin_popcountll(below);
        // fp32 images: the key's bits from 16 up carry the instance's rank
        // among its primitive's instances (tile keys there are below 2^16)
        if (hit && pos < endj) put(pos, (ty * grid_w + tx) | (kHalf ? 0u : (pos - offj) << 16), pj);
        // hits so far of the primitive carried into the next window (lane 63's owner)
        const uint32_t seg63 = readlane_u32(seg, 63);
        const uint32_t h63 = (uint32_t)__builtin_popcountll(hm & ~((1ull << seg63) - 1ull));
        carry_hits = (carry == prev ? carry_hits : 0u) + h63;
    }
    if (staged) {
        __syncthreads();
        for (uint32_t i = t; i < range_b - range_a; i += blockDim.x) {
            inst_keys[range_a + i] = s_key[i];
            inst_vals[range_a + i] = s_val[i];
        }
    }
}

void launch_emit_instances(const uint32_t* prims, const uint32_t* offs, BinCtl* ctl, int64_t max_count,
                           int64_t max_inst, const float2* mean2d, const uint4* conic_words,
                           const uint4* thr_words, const uint4* erec, uint32_t grid_w, uint32_t* inst_keys,
                           uint32_t* inst_vals, uint32_t* first_slot, bool half_test, hipStream_t s) {
    if (max_count <= 0) return;
    const unsigned grid = (unsigned)((max_count + 255) / 256);
    if (half_test)
        emit_kernel<true><<<grid, 256, 0, s>>>(prims, offs, ctl, max_count, max_inst, mean2d, conic_words,
                                               thr_words, erec, grid_w, inst_keys, inst_vals, first_slot);
    else
        emit_kernel<false><<<grid, 256, 0, s>>>(prims, offs, ctl, max_count, max_inst, mean2d, conic_words,
                                                thr_words, erec, grid_w, inst_keys, inst_vals, first_slot);
}

// ---------------------------------------------------------------- ranges

__global__ void fill_u32_kernel(uint32_t* p, uint32_t v, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

__global__ void __launch_bounds__(256) bin_ctl_reset_kernel(BinCtl* ctl) { bin_ctl_reset_block(ctl); }

void launch_bin_ctl_reset(BinCtl* ctl, hipStream_t s) { bin_ctl_reset_kernel<<<1, 256, 0, s>>>(ctl); }

void launch_fill_u32(uint32_t* p, uint32_t value, int64_t n, hipStream_t s) {
    if (n <= 0) return;
    fill_u32_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(p, value, n);
}

// kernels_forward.cuh:532-551, plus (0, 0) for the empty tiles: boundary i
// (0 <= i <= n) sits between keys[i - 1] and keys[i] (sentinels -1 and
// n_tiles), closes the previous tile's range, opens the next one and clears
// the tiles strictly between them. Each thread takes 8 consecutive
// boundaries, their keys read as two 16-byte vectors.
constexpr int kRangeSpan = 8;

__device__ __forceinline__ void tile_boundary(int64_t i, int64_t n, int64_t prev, int64_t cur, uint2* ranges,
                                              uint32_t n_tiles) {
    if (prev == (int64_t)n_tiles || cur == prev) return;
    if (i > 0) ranges[prev].y = (uint32_t)i;
    if (i < n && cur < (int64_t)n_tiles) ranges[cur].x = (uint32_t)i;
    for (int64_t tt = prev + 1; tt < cur; ++tt) ranges[tt] = make_uint2(0u, 0u);
}

__global__ void tile_ranges_kernel(const uint32_t* __restrict__ keys, const uint32_t* d_n, int64_t max_n,
                                   uint2* __restrict__ ranges, uint32_t n_tiles) {
    const int64_t n = resolve_n(d_n, max_n);
    const int64_t i0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * kRangeSpan;
    if (i0 > n) return;
    // keys are tile ids < n_tiles; min() keeps a corrupt key from writing out of range
    uint32_t k[kRangeSpan];
    if (i0 + kRangeSpan <= n) {   // the buffer is 16-byte aligned and i0 a multiple of 8
        const uint4 a = *(const uint4*)(keys + i0), b = *(const uint4*)(keys + i0 + 4);
        k[0] = a.x; k[1] = a.y; k[2] = a.z; k[3] = a.w; k[4] = b.x; k[5] = b.y; k[6] = b.z; k[7] = b.w;
    } else {
#pragma unroll
        for (int q = 0; q < kRangeSpan; ++q) k[q] = i0 + q < n ? keys[i0 + q] : n_tiles;
    }
    int64_t prev = i0 > 0 ? (int64_t)min(keys[i0 - 1], n_tiles) : -1;
#pragma unroll
    for (int q = 0; q < kRangeSpan; ++q) {
        const int64_t i = i0 + q;
        if (i > n) break;
        const int64_t cur = i < n ? (int64_t)min(k[q], n_tiles) : (int64_t)n_tiles;
        tile_boundary(i, n, prev, cur, ranges, n_tiles);
        prev = cur;
    }
}

// keys[i] = t for i in ranges[t] (workgroup per tile): the sorted tile keys
// of a tile sort whose last pass wrote only the ranges
__global__ void keys_from_ranges_kernel(const uint2* __restrict__ ranges, uint32_t n_tiles, int64_t max_n,
                                        uint32_t* __restrict__ keys) {
    const uint32_t t = blockIdx.x;
    if (t >= n_tiles) return;
    const uint2 r = ranges[t];
    const uint32_t end = (uint32_t)min((int64_t)r.y, max_n);
    for (uint32_t i = r.x + threadIdx.x; i < end; i += blockDim.x) keys[i] = t;
}

void launch_keys_from_ranges(const uint2* ranges, uint32_t n_tiles, int64_t max_inst, uint32_t* inst_keys,
                             hipStream_t s) {
    if (n_tiles) keys_from_ranges_kernel<<<n_tiles, 256, 0, s>>>(ranges, n_tiles, max_inst, inst_keys);
}

void launch_tile_ranges(const uint32_t* inst_keys, const uint32_t* d_n, int64_t max_inst, uint2* ranges,
                        uint32_t n_tiles, hipStream_t s) {
    const int64_t threads = (max_inst + 1 + kRangeSpan - 1) / kRangeSpan;
    tile_ranges_kernel<<<(unsigned)((threads + 255) / 256), 256, 0, s>>>(inst_keys, d_n, max_inst, ranges,
                                                                        n_tiles);
}

__global__ void clear_err_bits_kernel(BinCtl* ctl, uint32_t bits) {
    if (threadIdx.x == 0) atomicAnd(&ctl->err, ~bits);
}

void launch_clear_err_bits(BinCtl* ctl, uint32_t bits, hipStream_t s) {
    clear_err_bits_kernel<<<1, 64, 0, s>>>(ctl, bits);
}

int set_lookback_spin_limit(uint32_t spins) {
    return hipMemcpyToSymbol(HIP_SYMBOL(g_lookback_spins), &spins, sizeof(spins)) == hipSuccess ? 0 : -1;
}

bool radix_digits_fit(bool depth, int n_passes, const int* bits) {
    const int maxb = depth ? kDepthMaxDigits : kTileMaxDigits;
    if (n_passes < 1 || n_passes > 4) return false;
    for (int p = 0; p < n_passes; ++p)
        if (bits[p] < 1 || (1 << bits[p]) > maxb) return false;
    return true;
}

}  // namespace tgs
