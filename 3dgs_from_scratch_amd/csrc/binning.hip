// Binning: per-Gaussian tile counts, a depth sort, and the per-tile lists.
//
// The reference (src/cuda/rasterizer.cpp:292-359, src/cuda/kernel.cu:784-914,
// 1341-1388) emits one 64-bit key (tile_id << 32 | depth_bits) per touched tile
// in Gaussian order and stably sorts all 64 bits.  The same order -- (tile,
// depth bits, Gaussian index) -- is produced here without ever storing or
// sorting the K (tile, Gaussian) keys:
//   1. gs_bin_count: a packed tile rectangle and a depth key per Gaussian and
//      the totals K and M; a stable LSD sort of the depth keys of the Gaussians
//      with tiles (32 bits); then, with at most 256 supertiles (8 x 8 tiles),
//      the per-block supertile counts of level 1 and their positions, else a
//      scan of the supertile counts in depth order.
//   2. gs_bin_sort level 1: one (supertile, Gaussian) entry per touched
//      supertile, in depth order, stably sorted by supertile id -> for every
//      supertile, the Gaussians meeting it in depth order (M << K entries):
//      written straight to their places from those positions, or emitted and
//      radix-sorted by supertile id on larger grids.
//   3. gs_bin_sort level 2: each supertile list is cut into 512-entry blocks;
//      per wave, 8 row and 8 column ballots give every local tile's count,
//      one workgroup per supertile scans the counts over its blocks (and the
//      tile offsets over the grid), and each block then writes its Gaussians
//      covering each tile straight to their final positions.
// Every stage is stable, so each tile's run is in depth order with ties in
// Gaussian index order.
//
// Radix sort: LSD passes of <= 8 bits, each
//   upsweep    per-block digit histogram (wave64 ballot matching, one LDS atomic
//              per distinct digit per wave), digit-major table,
//   digit scan one block per digit scans its column and writes the digit total,
//   downsweep  stable local ranks from the same ballot matching, digit offsets
//              from the totals, a scatter into LDS in digit order, and
//              contiguous runs written to HBM.
// No kernel waits on another workgroup, so no launch can deadlock.

#include "wave_ops.h"
#include "preprocess_math.h"

namespace gs {

constexpr int kSortThreads = 256;
constexpr int kSortWaves = kSortThreads / kWave;
constexpr int kRadixMaxBits = 8;
constexpr int kRadixMax = 1 << kRadixMaxBits;
// Keys per thread in a radix pass: few, so that the N- and M-sized sorts launch
// enough waves to hide memory latency (these passes are latency-bound).
constexpr int kDepthItems = 4;  // the depth sort (N keys)
constexpr int kTileItems = 4;   // the supertile sort (M keys)

constexpr int kSuper = 8;                       // supertile edge, in tiles
constexpr int kSuperLocal = kSuper * kSuper;    // tiles per supertile (one mask bit each)
constexpr int kL2Threads = 512;                 // supertile-list positions per level-2 block
constexpr int kL2Waves = kL2Threads / kWave;

constexpr int kScanThreads = 256;
constexpr int kScanItems = 16;
constexpr int kScanTile = kScanThreads * kScanItems;

inline size_t align256(size_t x) { return (x + 255) / 256 * 256; }

// Workgroups are dealt to the kBinXcds XCDs round robin (workgroup w runs on
// XCD w % kBinXcds).  xcd_block maps w to a logical block so that each XCD
// runs a contiguous range of logical blocks, base + (x < rem) of them from
// x * base + min(x, rem): kernels whose neighbouring blocks write neighbouring
// positions of the same lists then fill those cache lines within one L2.  A
// bijection of [0, nblocks).
constexpr int kBinXcds = 8;

__device__ __forceinline__ int64_t xcd_block(int64_t w, int64_t nblocks) {
    const int64_t base = nblocks / kBinXcds, rem = nblocks % kBinXcds;
    const int64_t x = w % kBinXcds, i = w / kBinXcds;
    return x * base + (x < rem ? x : rem) + i;
}

// The inverse of xcd_block: the workgroup index that xcd_block maps to logical
// block b.
__device__ __forceinline__ int64_t xcd_block_inverse(int64_t b, int64_t nblocks) {
    const int64_t base = nblocks / kBinXcds, rem = nblocks % kBinXcds;
    const int64_t big = rem * (base + 1);  // the first rem ranges hold base + 1 blocks
    const int64_t x = b < big ? b / (base + 1) : rem + (b - big) / base;
    const int64_t i = b - (x * base + (x < rem ? x : rem));
    return i * kBinXcds + x;
}

// The same over the first `live` workgroups only (the ones with work: a grid
// sized by an upper bound leaves the rest idle, and spreading those evenly
// keeps every XCD's share of the work equal); the others map to themselves.
__device__ __forceinline__ int64_t xcd_block_live(int64_t w, int64_t live) {
    return w < live ? xcd_block(w, live) : w;
}

// ------------------------------------------------------------------ scan

// Per-workgroup sums of kScanTile consecutive elements.
template <typename T>
__global__ __launch_bounds__(kScanThreads) void scan_reduce_kernel(const T *__restrict__ in,
                                                                   int64_t n,
                                                                   T *__restrict__ sums) {
    __shared__ T tmp[kScanThreads / kWave + 1];
    const int64_t base = (int64_t)blockIdx.x * kScanTile;
    T acc = 0;
#pragma unroll
    for (int it = 0; it < kScanItems; ++it) {
        const int64_t i = base + (int64_t)it * kScanThreads + threadIdx.x;
        if (i < n) acc += in[i];
    }
    T total;
    block_exclusive_scan<T, kScanThreads>(acc, tmp, total);
    if (threadIdx.x == 0) sums[blockIdx.x] = total;
}

// Exclusive scan of NT*ITEMS consecutive elements per workgroup, offset by
// `offsets[blockIdx.x]` (or 0 when offsets is null).  In-place safe.  The last
// workgroup writes the grand total to *total when total is not null.
template <typename T, int NT, int ITEMS>
__global__ __launch_bounds__(NT) void scan_apply_kernel(const T *in, T *out, int64_t n,
                                                        const T *__restrict__ offsets,
                                                        T *__restrict__ total) {
    __shared__ T tmp[NT / kWave + 1];
    const int64_t base = (int64_t)blockIdx.x * (NT * ITEMS) + (int64_t)threadIdx.x * ITEMS;
    T v[ITEMS];
    T acc = 0;
#pragma unroll
    for (int it = 0; it < ITEMS; ++it) {
        const int64_t i = base + it;
        v[it] = i < n ? in[i] : (T)0;
        acc += v[it];
    }
    T block_total;
    T run = block_exclusive_scan<T, NT>(acc, tmp, block_total);
    const T off = offsets ? offsets[blockIdx.x] : (T)0;
    run += off;
#pragma unroll
    for (int it = 0; it < ITEMS; ++it) {
        const int64_t i = base + it;
        if (i < n) out[i] = run;
        run += v[it];
    }
    if (total && blockIdx.x == gridDim.x - 1 && threadIdx.x == 0) *total = off + block_total;
}

// Bytes of scratch needed by scan_exclusive for n elements.
template <typename T>
size_t scan_workspace_bytes(int64_t n) {
    size_t bytes = 0;
    while (n > kScanTile) {
        const int64_t nb = (n + kScanTile - 1) / kScanTile;
        bytes += align256(nb * sizeof(T));
        n = nb;
    }
    return bytes;
}

// Exclusive scan of n elements (out may alias in).  Writes the total to
// *total (device pointer) when not null.  One launch up to kScanTile elements,
// reduce / scan-of-sums / apply above.
template <typename T>
int scan_exclusive(const T *in, T *out, int64_t n, T *total, void *ws, hipStream_t stream) {
    if (n <= 0) return total ? zero_bytes(total, sizeof(T), stream) : GS_OK;
    if (n > kScanTile && n <= 1024 * kScanItems) {  // one 1024-thread workgroup
        hipLaunchKernelGGL((scan_apply_kernel<T, 1024, kScanItems>), dim3(1), dim3(1024), 0,
                           stream, in, out, n, (const T *)nullptr, total);
        return launch_status();
    }
    const int64_t nb = (n + kScanTile - 1) / kScanTile;
    if (nb == 1) {
        hipLaunchKernelGGL((scan_apply_kernel<T, kScanThreads, kScanItems>), dim3(1),
                           dim3(kScanThreads), 0, stream, in, out, n, (const T *)nullptr, total);
        return launch_status();
    }
    T *sums = reinterpret_cast<T *>(ws);
    void *ws_next = reinterpret_cast<char *>(ws) + align256(nb * sizeof(T));
    hipLaunchKernelGGL(scan_reduce_kernel<T>, dim3(nb), dim3(kScanThreads), 0, stream, in, n,
                       sums);
    int st = launch_status();
    if (st) return st;
    st = scan_exclusive<T>(sums, sums, nb, (T *)nullptr, ws_next, stream);
    if (st) return st;
    hipLaunchKernelGGL((scan_apply_kernel<T, kScanThreads, kScanItems>), dim3(nb),
                       dim3(kScanThreads), 0, stream, in, out, n, (const T *)sums, total);
    return launch_status();
}

// ------------------------------------------------------------ radix sort

__device__ __forceinline__ uint32_t digit_of(uint32_t key, int shift, uint32_t dmask) {
    return (key >> shift) & dmask;
}

// Depth bucket of a key (the depth sort's DepthXform {kmin, shift}): bits
// shift .. shift + 15 of key - kmin, clamped to [0, 0xFFFF] -- keys at or below
// kmin in bucket 0, keys past the 16 bits in bucket 0xFFFF.  Non-decreasing in
// the key, so ordering by bucket and then by the full key is ordering by key,
// whatever the transform; with the least and greatest key of the sort it never
// clamps.  `on` false: the identity (the passes that are not depth passes).
struct BucketFn {
    uint32_t kmin = 0;
    int shift = 0;
    bool on = false;
    __device__ __forceinline__ uint32_t operator()(uint32_t key) const {
        if (!on) return key;
        if (key <= kmin) return 0u;
        const uint32_t b = (key - kmin) >> shift;
        return b < 0xFFFFu ? b : 0xFFFFu;
    }
};

__device__ __forceinline__ BucketFn bucket_fn(const uint32_t *xform) {
    BucketFn f;
    if (xform) {
        f.kmin = xform[0];
        f.shift = (int)xform[1];
        f.on = true;
    }
    return f;
}

// Tile rectangle packed as (tx0 | tx1 << 16, ty0 | ty1 << 16); tile coordinates
// fit 16 bits (gs_bin_sort rejects larger grids).
__device__ __forceinline__ uint2 pack_rect(const TileRect &r) {
    return make_uint2((uint32_t)r.tx0 | ((uint32_t)r.tx1 << 16),
                      (uint32_t)r.ty0 | ((uint32_t)r.ty1 << 16));
}

__device__ __forceinline__ TileRect unpack_rect(uint2 p) {
    TileRect r;
    r.tx0 = (int)(p.x & 0xffffu);
    r.tx1 = (int)(p.x >> 16);
    r.ty0 = (int)(p.y & 0xffffu);
    r.ty1 = (int)(p.y >> 16);
    return r;
}

// Packed tile rectangle of a Gaussian without tiles: tx0 > tx1.
constexpr uint2 kEmptyRect = {0xffffu, 0xffffu};

// rects[val] for a Gaussian index val < n, else kEmptyRect.  The load is from a
// clamped index (a global load of the rectangle array in every case, then a
// select): a choice between two addresses, one of them the constant, compiles
// to a flat load, which makes every later store wait for it and all before it.
__device__ __forceinline__ uint2 rect_or_empty(const uint2 *__restrict__ rects, uint32_t val,
                                               int64_t n) {
    const bool in = val < (uint64_t)n;
    const uint2 r = rects[in ? val : 0u];
    return in ? r : kEmptyRect;
}

// Tiles of a packed rectangle (0 for kEmptyRect).
__device__ __forceinline__ uint32_t rect_tiles(uint2 packed) {
    const TileRect t = unpack_rect(packed);
    if (t.tx0 > t.tx1) return 0u;
    return (uint32_t)((t.tx1 - t.tx0 + 1) * (t.ty1 - t.ty0 + 1));
}

// Supertiles (kSuper x kSuper tiles) a packed rectangle meets (0 for kEmptyRect).
__device__ __forceinline__ uint32_t rect_supertiles(uint2 packed) {
    const TileRect t = unpack_rect(packed);
    if (t.tx0 > t.tx1) return 0u;
    return (uint32_t)((t.tx1 / kSuper - t.tx0 / kSuper + 1) *
                      (t.ty1 / kSuper - t.ty0 / kSuper + 1));
}

// Depth key of a Gaussian without tiles: the first depth pass drops these keys.
constexpr uint32_t kNoTilesKey = 0xFFFFFFFFu;

// kPayload: each value carries an 8-byte payload (a packed tile rectangle).
template <int ITEMS, bool kPayload = false>
struct SortLds {
    uint32_t wave_count[kSortWaves][kRadixMax];
    uint32_t global_start[kRadixMax];
    uint32_t local_start[kRadixMax];
    uint32_t skeys[kSortThreads * ITEMS];
    uint32_t svals[kSortThreads * ITEMS];
    uint2 spay[kPayload ? kSortThreads * ITEMS : 1];
    uint32_t scan_tmp[kSortThreads / kWave + 1];
};

// Key slot `it` of this thread: index within the block = wave*(64*ITEMS) + it*64 + lane,
// so one load instruction covers 64 consecutive keys and keys stay in index order
// (slot-major inside a wave, wave-major across the block).
template <int ITEMS>
__device__ __forceinline__ int slot_index(int it) {
    return (threadIdx.x / kWave) * (kWave * ITEMS) + it * kWave + (threadIdx.x % kWave);
}

// Adds the block's digit counts (keys in registers) to `counts` (LDS, zeroed).
template <int ITEMS>
__device__ __forceinline__ void block_count_digits(const uint32_t (&k)[ITEMS],
                                                   const bool (&valid)[ITEMS], int shift,
                                                   int nbits, uint32_t *counts,
                                                   BucketFn bf = BucketFn()) {
    const uint32_t dmask = (1u << nbits) - 1u;
#pragma unroll
    for (int it = 0; it < ITEMS; ++it) {
        const uint32_t d = digit_of(bf(k[it]), shift, dmask);
        const uint64_t active = __ballot(valid[it]);
        const uint64_t peers = match_digit(d, nbits, active);
        if (valid[it] && (peers & lanemask_lt()) == 0)
            atomicAdd(&counts[d], (uint32_t)__popcll(peers));
    }
}

// Per-pass histogram table, digit-major: entry d * nblocks + b counts the keys
// of block b with digit d; digit_scan_kernel turns it in place into the first
// output position of (digit, block).
__device__ __forceinline__ int64_t hist_index(int d, int b, int nblocks) {
    return (int64_t)d * nblocks + b;
}

// Per-block sums of count_tiles (tiles, supertile entries, Gaussians with
// tiles; three per block) reduced by one workgroup of kScanThreads to
// sums_out[0] = K, sums_out[1] = M and *live_out (K and M also to sums_dev, a
// device copy, when set); with minmax (count_tiles' per-block least and
// greatest key with tiles) also sums_out[2] and sums_out[3] = the least and
// greatest key with tiles over all blocks (0xFFFFFFFF and 0 when there is none).
__device__ __forceinline__ void reduce_block_sums(const unsigned long long *__restrict__ sums,
                                                  const uint32_t *__restrict__ minmax,
                                                  int nblocks, int64_t *__restrict__ sums_out,
                                                  int64_t *__restrict__ live_out,
                                                  int64_t *__restrict__ sums_dev) {
    __shared__ unsigned long long tmp[kScanThreads / kWave + 1];
    __shared__ uint32_t mm[2][kScanThreads / kWave];
    unsigned long long acc[3] = {0ull, 0ull, 0ull};
    uint32_t lo = 0xFFFFFFFFu, hi = 0u;
    for (int b = threadIdx.x; b < nblocks; b += kScanThreads) {
#pragma unroll
        for (int f = 0; f < 3; ++f) acc[f] += sums[(int64_t)b * 3 + f];
        if (minmax) {
            lo = min(lo, minmax[2 * (int64_t)b]);
            hi = max(hi, minmax[2 * (int64_t)b + 1]);
        }
    }
    unsigned long long total[3];
#pragma unroll
    for (int f = 0; f < 3; ++f)
        block_exclusive_scan<unsigned long long, kScanThreads>(acc[f], tmp, total[f]);
    if (minmax) {
        for (int o = kWave / 2; o > 0; o >>= 1) {
            lo = min(lo, (uint32_t)__shfl_xor((int)lo, o, kWave));
            hi = max(hi, (uint32_t)__shfl_xor((int)hi, o, kWave));
        }
        if (threadIdx.x % kWave == 0) {
            mm[0][threadIdx.x / kWave] = lo;
            mm[1][threadIdx.x / kWave] = hi;
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        sums_out[0] = (int64_t)total[0];
        sums_out[1] = (int64_t)total[1];
        *live_out = (int64_t)total[2];
        if (sums_dev) {
            sums_dev[0] = (int64_t)total[0];
            sums_dev[1] = (int64_t)total[1];
        }
        if (minmax) {
            lo = 0xFFFFFFFFu;
            hi = 0u;
#pragma unroll
            for (int w = 0; w < kScanThreads / kWave; ++w) {
                lo = min(lo, mm[0][w]);
                hi = max(hi, mm[1][w]);
            }
            sums_out[2] = (int64_t)lo;
            sums_out[3] = (int64_t)hi;
        }
    }
}

// Block d scans column d of the histogram table over the nblocks blocks in
// place (first position of (d, block) among the keys with digit d) and writes
// the column total to totals[d].  The downsweep adds the keys of smaller digits.
// With block_sums, one more block (the last) runs reduce_block_sums (with
// block_minmax when it is set).
constexpr int kDigitScanItems = 8;  // column entries per thread held in registers

__global__ __launch_bounds__(kScanThreads) void digit_scan_kernel(
    uint32_t *__restrict__ table, int nblocks, uint32_t *__restrict__ totals,
    const unsigned long long *__restrict__ block_sums, const uint32_t *__restrict__ block_minmax,
    int nsum_blocks, int64_t *__restrict__ sums_out, int64_t *__restrict__ live_out,
    int64_t *__restrict__ sums_dev) {
    __shared__ uint32_t tmp[kScanThreads / kWave + 1];
    const int d = blockIdx.x;
    if (block_sums && d == (int)gridDim.x - 1) {
        reduce_block_sums(block_sums, block_minmax, nsum_blocks, sums_out, live_out, sums_dev);
        return;
    }
    uint32_t run = 0;
    uint32_t *col = table + (int64_t)d * nblocks;
    // chunks of kScanThreads * kDigitScanItems entries: thread t holds the
    // consecutive entries [t * items, (t + 1) * items) of the chunk, so that all
    // of a chunk's loads are issued before its one block scan
    for (int b0 = 0; b0 < nblocks; b0 += kScanThreads * kDigitScanItems) {
        const int first = b0 + threadIdx.x * kDigitScanItems;
        uint32_t c[kDigitScanItems];
        uint32_t mine = 0;
#pragma unroll
        for (int it = 0; it < kDigitScanItems; ++it) {
            c[it] = first + it < nblocks ? col[first + it] : 0u;
            mine += c[it];
        }
        uint32_t chunk;
        uint32_t pos = run + block_exclusive_scan<uint32_t, kScanThreads>(mine, tmp, chunk);
#pragma unroll
        for (int it = 0; it < kDigitScanItems; ++it) {
            if (first + it < nblocks) col[first + it] = pos;
            pos += c[it];
        }
        run += chunk;
    }
    if (threadIdx.x == 0) totals[d] = run;
}

// Stable rank of the block's keys (registers) by digit, staged through LDS in
// digit order and written to keys_out/vals_out (and, with kPayload, the
// payloads to pay_out).  `table` holds the position of each (digit, block)
// among the keys of its digit, `totals` the keys per digit.  When counts_out
// is set, counts_out[dst] = rect_supertiles(rects[value]) is written as well,
// and when rects_out is set, rects_out[dst] = rects[value].
template <typename KeyT, int ITEMS, bool kPayload>
__device__ __forceinline__ void block_scatter(const uint32_t (&k)[ITEMS],
                                              const uint32_t (&v)[ITEMS],
                                              const uint2 (&pay)[ITEMS],
                                              const bool (&valid)[ITEMS], int shift, int nbits,
                                              int nblocks, const uint32_t *__restrict__ table,
                                              KeyT *__restrict__ keys_out,
                                              uint32_t *__restrict__ vals_out,
                                              uint2 *__restrict__ pay_out, int64_t n,
                                              bool write_keys, SortLds<ITEMS, kPayload> &s,
                                              const uint32_t *__restrict__ totals,
                                              uint64_t *__restrict__ counts_out,
                                              const uint2 *__restrict__ rects,
                                              uint2 *__restrict__ rects_out, int blk,
                                              BucketFn bf) {
    const int radix = 1 << nbits;
    const uint32_t dmask = (uint32_t)radix - 1u;
    const int wave = threadIdx.x / kWave;
    static_assert(kRadixMax <= kSortThreads, "one digit per thread");
    const int dt = threadIdx.x;
    const uint32_t tot = dt < radix ? totals[dt] : 0u;
    const uint32_t first = dt < radix ? table[hist_index(dt, blk, nblocks)] : 0u;
    uint32_t all_keys;
    const uint32_t smaller = block_exclusive_scan<uint32_t, kSortThreads>(tot, s.scan_tmp, all_keys);
    if (dt < radix) {
#pragma unroll
        for (int w = 0; w < kSortWaves; ++w) s.wave_count[w][dt] = 0;
        s.global_start[dt] = smaller + first;
    }
    __syncthreads();
    uint32_t rank[ITEMS];
#pragma unroll
    for (int it = 0; it < ITEMS; ++it) {
        const uint32_t d = digit_of(bf(k[it]), shift, dmask);
        const uint64_t active = __ballot(valid[it]);
        const uint64_t peers = match_digit(d, nbits, active);
        const uint32_t before = valid[it] ? s.wave_count[wave][d] : 0u;
        const uint32_t r = (uint32_t)__popcll(peers & lanemask_lt());
        if (valid[it] && r == 0) s.wave_count[wave][d] = before + (uint32_t)__popcll(peers);
        rank[it] = before + r;
    }
    __syncthreads();
    uint32_t digit_total = 0;
    if (threadIdx.x < radix) {
#pragma unroll
        for (int w = 0; w < kSortWaves; ++w) {
            const uint32_t c = s.wave_count[w][threadIdx.x];
            s.wave_count[w][threadIdx.x] = digit_total;
            digit_total += c;
        }
    }
    uint32_t block_count;
    const uint32_t ls =
        block_exclusive_scan<uint32_t, kSortThreads>(digit_total, s.scan_tmp, block_count);
    if (threadIdx.x < radix) s.local_start[threadIdx.x] = ls;
    __syncthreads();
#pragma unroll
    for (int it = 0; it < ITEMS; ++it) {
        if (valid[it]) {
            const uint32_t d = digit_of(bf(k[it]), shift, dmask);
            const uint32_t p = s.local_start[d] + s.wave_count[wave][d] + rank[it];
            s.skeys[p] = k[it];
            s.svals[p] = v[it];
            if (kPayload) s.spay[p] = pay[it];
        }
    }
    __syncthreads();
    for (uint32_t p = threadIdx.x; p < block_count; p += kSortThreads) {
        const uint32_t key = s.skeys[p];
        const uint32_t d = digit_of(bf(key), shift, dmask);
        const uint32_t dst = s.global_start[d] + (p - s.local_start[d]);
        if (dst < (uint64_t)n) {  // always true for a consistent histogram; guards the store
            const uint32_t val = s.svals[p];
            if (write_keys) keys_out[dst] = (KeyT)key;
            vals_out[dst] = val;
            if (kPayload) pay_out[dst] = s.spay[p];
            if (counts_out || rects_out) {
                const uint2 r = rect_or_empty(rects, val, n);
                if (counts_out) counts_out[dst] = rect_supertiles(r);
                if (rects_out) rects_out[dst] = r;
            }
        }
    }
}

// hist[d * nblocks + block] = number of keys of this block with digit d.  The
// keys are the first *n_live (when given, else n) of the array.
template <typename KeyT, int ITEMS>
__global__ __launch_bounds__(kSortThreads) void radix_upsweep_kernel(
    const KeyT *__restrict__ keys, int64_t n, const int64_t *__restrict__ n_live, int shift,
    int nbits, int nblocks, uint32_t *__restrict__ hist, const uint32_t *__restrict__ xform) {
    __shared__ uint32_t counts[kRadixMax];
    const int radix = 1 << nbits;
    for (int d = threadIdx.x; d < radix; d += kSortThreads) counts[d] = 0;
    if (n_live) n = *n_live;
    const BucketFn bf = bucket_fn(xform);  // digits of the depth buckets (see BucketFn)
    const int64_t base = (int64_t)blockIdx.x * (kSortThreads * ITEMS);
    uint32_t k[ITEMS];
    bool valid[ITEMS];
#pragma unroll
    for (int it = 0; it < ITEMS; ++it) {
        const int64_t i = base + slot_index<ITEMS>(it);
        valid[it] = i < n;
        k[it] = valid[it] ? (uint32_t)keys[i] : 0u;
    }
    __syncthreads();
    block_count_digits<ITEMS>(k, valid, shift, nbits, counts, bf);
    __syncthreads();
    for (int d = threadIdx.x; d < radix; d += kSortThreads)
        hist[hist_index(d, blockIdx.x, nblocks)] = counts[d];
}

// Optional inputs and outputs of a radix pass besides its keys and values.
struct PassExtras {
    bool hist_ready = false;            // the caller wrote this pass's histogram table
    bool drop_no_tiles = false;         // keys equal to kNoTilesKey are not sorted
    const int64_t *n_live = nullptr;    // device: sort only the first *n_live keys
    const uint2 *pin = nullptr;         // kPayload: 8-byte payload per key
    uint2 *pout = nullptr;
    const uint2 *rects = nullptr;       // gathered by value (last pass):
    uint64_t *counts_out = nullptr;     //   rect_supertiles(rects[value])
    uint2 *rects_out = nullptr;         //   rects[value]
    const unsigned long long *block_sums = nullptr;  // count_tiles' per-block sums,
    int64_t *sums_out = nullptr;        //   reduced to sums_out[0..1] (K, M)
    int64_t *live_out = nullptr;        //   and *live_out (keys with tiles);
    const uint32_t *block_minmax = nullptr;  // with it, sums_out[2..3] = least and
                                             //   greatest key with tiles
    int64_t *sums_dev = nullptr;        // device copy of K and M
    const uint32_t *xform = nullptr;    // device DepthXform: digits of the keys' depth buckets
};

template <typename KeyT>
struct DownArgs {
    const KeyT *keys_in;
    const uint32_t *vals_in;  // null: the value of key i is i
    const uint2 *pay_in;
    KeyT *keys_out;
    uint32_t *vals_out;
    uint2 *pay_out;
    int64_t n;
    const int64_t *n_live;
    int shift, nbits, nblocks, write_keys, drop_no_tiles;
    const uint32_t *table, *totals;
    uint64_t *counts_out;
    const uint2 *rects;
    uint2 *rects_out;
    const uint32_t *xform;
};

// With n_live, only the first *n_live keys are sorted, and a pass that writes
// no keys (the last) fills output positions *n_live .. n - 1 of its block's
// range with a value of 0xFFFFFFFF, a count of 0 and kEmptyRect.
template <typename KeyT, int ITEMS, bool kPayload>
__global__ __launch_bounds__(kSortThreads) void radix_downsweep_kernel(DownArgs<KeyT> a) {
    __shared__ SortLds<ITEMS, kPayload> s;
    const int64_t live = a.n_live ? *a.n_live : a.n;
    // neighbouring ranges on one XCD (over the workgroups with keys)
    const int blk = (int)xcd_block_live(blockIdx.x, (live + kSortThreads * ITEMS - 1) /
                                                        (kSortThreads * ITEMS));
    const int64_t base = (int64_t)blk * (kSortThreads * ITEMS);
    const int shift = a.shift;
    const BucketFn bf = bucket_fn(a.xform);
    uint32_t k[ITEMS], v[ITEMS];
    uint2 pay[ITEMS];
    bool valid[ITEMS];
#pragma unroll
    for (int it = 0; it < ITEMS; ++it) {
        const int64_t i = base + slot_index<ITEMS>(it);
        const bool in = i < live;
        k[it] = in ? (uint32_t)a.keys_in[i] : 0u;
        v[it] = in ? (a.vals_in ? a.vals_in[i] : (uint32_t)i) : 0u;
        pay[it] = (kPayload && in) ? a.pay_in[i] : make_uint2(0u, 0u);
        valid[it] = in && !(a.drop_no_tiles && k[it] == kNoTilesKey);
        k[it] = valid[it] ? k[it] : 0u;
    }
    block_scatter<KeyT, ITEMS, kPayload>(k, v, pay, valid, shift, a.nbits, a.nblocks, a.table,
                                         a.keys_out, a.vals_out, a.pay_out, a.n,
                                         a.write_keys != 0, s, a.totals, a.counts_out, a.rects,
                                         a.rects_out, blk, bf);
    if (a.n_live && !a.write_keys) {
        for (int t = threadIdx.x; t < kSortThreads * ITEMS; t += kSortThreads) {
            const int64_t j = base + t;
            if (j < live || j >= a.n) continue;
            a.vals_out[j] = 0xFFFFFFFFu;
            if (a.counts_out) a.counts_out[j] = 0u;
            if (a.rects_out) a.rects_out[j] = kEmptyRect;
        }
    }
}

struct SortPlan {
    int passes;
    int bits_per_pass;
};

// At least one pass (a 0-bit pass is a stable copy).
inline SortPlan plan_sort(int total_bits) {
    SortPlan p;
    p.passes = total_bits <= 0 ? 1 : (total_bits + kRadixMaxBits - 1) / kRadixMaxBits;
    p.bits_per_pass = total_bits <= 0 ? 0 : (total_bits + p.passes - 1) / p.passes;
    return p;
}

inline int pass_bits(const SortPlan &plan, int total_bits, int p) {
    const int rest = total_bits - p * plan.bits_per_pass;
    return rest < plan.bits_per_pass ? (rest > 0 ? rest : 0) : plan.bits_per_pass;
}

template <int ITEMS>
inline int64_t sort_blocks(int64_t n) {
    return (n + kSortThreads * ITEMS - 1) / (kSortThreads * ITEMS);
}

// Histogram table of one pass, then the kRadixMax digit totals.

template <int ITEMS>
size_t radix_table_bytes(int64_t n) {
    return align256((size_t)sort_blocks<ITEMS>(n) * kRadixMax * sizeof(uint32_t));
}

template <int ITEMS>
size_t radix_workspace_bytes(int64_t n) {
    return radix_table_bytes<ITEMS>(n) + align256(kRadixMax * sizeof(uint32_t));
}

template <int ITEMS>
uint32_t *radix_totals(void *ws, int64_t n) {
    return reinterpret_cast<uint32_t *>(reinterpret_cast<char *>(ws) +
                                        radix_table_bytes<ITEMS>(n));
}

// One LSD pass from arrays: histogram (unless the caller already wrote this
// pass's table), digit scan, scatter; `x` adds the optional inputs and outputs.
template <typename KeyT, int ITEMS, bool kPayload = false>
int radix_pass(const KeyT *kin, const uint32_t *vin, KeyT *kout, uint32_t *vout, int64_t n,
               int shift, int nbits, bool write_keys, void *ws, hipStream_t stream,
               const PassExtras &x = PassExtras()) {
    const int nblocks = (int)sort_blocks<ITEMS>(n);
    uint32_t *hist = reinterpret_cast<uint32_t *>(ws);
    uint32_t *totals = radix_totals<ITEMS>(ws, n);
    int st;
    if (!x.hist_ready) {
        hipLaunchKernelGGL((radix_upsweep_kernel<KeyT, ITEMS>), dim3(nblocks), dim3(kSortThreads),
                           0, stream, kin, n, x.n_live, shift, nbits, nblocks, hist, x.xform);
        st = launch_status();
        if (st) return st;
    }
    const int sums_block = x.block_sums ? 1 : 0;
    hipLaunchKernelGGL(digit_scan_kernel, dim3((1 << nbits) + sums_block), dim3(kScanThreads), 0,
                       stream, hist, nblocks, totals, x.block_sums, x.block_minmax, nblocks,
                       x.sums_out, x.live_out, x.sums_dev);
    st = launch_status();
    if (st) return st;
    DownArgs<KeyT> a;
    a.keys_in = kin;
    a.vals_in = vin;
    a.pay_in = x.pin;
    a.keys_out = kout;
    a.vals_out = vout;
    a.pay_out = x.pout;
    a.n = n;
    a.n_live = x.n_live;
    a.shift = shift;
    a.nbits = nbits;
    a.nblocks = nblocks;
    a.write_keys = write_keys ? 1 : 0;
    a.drop_no_tiles = x.drop_no_tiles ? 1 : 0;
    a.table = hist;
    a.totals = totals;
    a.counts_out = x.counts_out;
    a.rects = x.rects;
    a.rects_out = x.rects_out;
    a.xform = x.xform;
    hipLaunchKernelGGL((radix_downsweep_kernel<KeyT, ITEMS, kPayload>), dim3(nblocks),
                       dim3(kSortThreads), 0, stream, a);
    return launch_status();
}

// ------------------------------------------------------- depth segment sort
// The depth sort runs on key' = key - kmin (kmin the least key with tiles:
// the same order and the same ties) and is two stable 8-bit passes over the 16
// bucket bits of key' (bits shift .. shift + 15, every higher bit being 0: see
// DepthXform), which leave the keys ordered by (bucket, Gaussian index),
// followed by segment_sort_kernel: each workgroup takes the buckets that begin
// in its nominal range of kSegChunk positions and sorts them by the full key,
// stably, so that the result is ordered by (key, index) as a full 32-bit
// stable sort is.  A chunk of at most kSegMax keys is sorted in LDS (LSD
// passes of at most 8 bits over the bits below its highest differing bit); a
// larger one (a bucket of more than about kSegMax - kSegChunk keys: exact ties,
// or depths packed far more densely than elsewhere) is sorted by the same
// workgroup through global memory.
constexpr int kSegThreads = 256;
constexpr int kSegWaves = kSegThreads / kWave;
constexpr int kSegItems = 4;
constexpr int kSegMax = kSegThreads * kSegItems;  // keys of a chunk sorted in LDS
constexpr int kSegChunk = 512;                    // nominal positions per workgroup
static_assert(kSegMax < 65536, "window counts are packed in 16 bits");

struct SegLds {
    uint32_t keys[2][kSegMax];
    uint32_t vals[2][kSegMax];
    uint32_t wave_count[kSegWaves][kRadixMax];
    uint32_t digit_start[kRadixMax];
    uint32_t running[kRadixMax];
    uint32_t scan_tmp[kSegThreads / kWave + 1];
    uint32_t red[kSegWaves];
};

// Sum (add) or bitwise OR (!add) of `x` over the workgroup (contains barriers).
template <bool kAdd>
__device__ __forceinline__ uint32_t seg_reduce(uint32_t x, SegLds &s) {
    for (int o = kWave / 2; o > 0; o >>= 1) {
        const uint32_t y = (uint32_t)__shfl_xor((int)x, o, kWave);
        x = kAdd ? x + y : x | y;
    }
    __syncthreads();
    if (threadIdx.x % kWave == 0) s.red[threadIdx.x / kWave] = x;
    __syncthreads();
    uint32_t r = 0;
#pragma unroll
    for (int w = 0; w < kSegWaves; ++w) r = kAdd ? r + s.red[w] : r | s.red[w];
    return r;
}

// First position q in [lo, live) whose bucket bf(key) exceeds b, given
// that every position in [p0, lo) has a bucket <= b (keys[0 .. live) are
// ordered by bucket); live when there is none.  Rounds of kSegThreads strided
// probes, each narrowing the interval by kSegThreads.
__device__ uint32_t bucket_end_search(const uint32_t *__restrict__ keys, uint32_t lo,
                                      uint32_t live, BucketFn bf, uint32_t b, SegLds &s) {
    uint32_t hi = live;  // the answer lies in [lo, hi]
    while (lo < hi) {
        const uint32_t len = hi - lo;
        const uint32_t stride = (len + kSegThreads - 1) / kSegThreads;
        const uint32_t q = lo + threadIdx.x * stride;
        const uint32_t c = seg_reduce<true>((q < hi && bf(keys[q]) <= b) ? 1u : 0u, s);
        if (c == 0) return lo;
        if (stride == 1) return lo + c;
        const uint32_t last_le = lo + (c - 1) * stride;  // a probe <= b
        const uint32_t first_gt = lo + c * stride;       // a probe > b, or past hi
        lo = last_le + 1;
        hi = min(hi, first_gt);
    }
    return lo;
}

// Position of item `it` of this thread in a tile of up to kSegMax keys cut
// into ipw items per lane: wave-major, then item, then lane, so that one load
// instruction covers 64 consecutive positions and the order of (wave, item,
// lane) is the position order.  A tile of `size` keys uses
// ipw = seg_items(size), spreading it evenly over the waves.
__device__ __forceinline__ int seg_slot(int it, int ipw) {
    return (threadIdx.x / kWave) * (kWave * ipw) + it * kWave + (threadIdx.x % kWave);
}

__device__ __forceinline__ int seg_items(uint32_t size) {
    return (int)((size + kSegThreads - 1) / kSegThreads);
}

// Stable LDS rank of a tile of keys -- item it of this thread at position
// seg_slot(it, ipw), items it < ipw -- by the nbits-bit digit at `shift`
// (nbits <= kSegDigitBits): pos[it] = the item's rank in digit order;
// s.digit_start[d] = the first rank of digit d and digit_total (thread d) = the
// keys of digit d.  Invalid items are ignored.  Contains barriers.
constexpr int kSegDigitBits = kRadixMaxBits;

__device__ __forceinline__ void seg_rank(const uint32_t (&k)[kSegItems],
                                         const bool (&valid)[kSegItems], int ipw, int shift,
                                         int nbits, uint32_t (&pos)[kSegItems], SegLds &s,
                                         uint32_t &digit_total) {
    const int wave = threadIdx.x / kWave;
    const uint32_t dmask = (1u << nbits) - 1u;
    for (int i = threadIdx.x; i < kSegWaves * kRadixMax; i += kSegThreads)
        (&s.wave_count[0][0])[i] = 0u;
    __syncthreads();
    uint32_t rank[kSegItems];
#pragma unroll
    for (int it = 0; it < kSegItems; ++it) {
        rank[it] = 0u;
        if (it >= ipw) continue;  // uniform
        const uint32_t d = digit_of(k[it], shift, dmask);
        const uint64_t active = __ballot(valid[it]);
        const uint64_t peers = match_digit(d, nbits, active);
        const uint32_t before = valid[it] ? s.wave_count[wave][d] : 0u;
        const uint32_t r = (uint32_t)__popcll(peers & lanemask_lt());
        if (valid[it] && r == 0) s.wave_count[wave][d] = before + (uint32_t)__popcll(peers);
        rank[it] = before + r;
    }
    __syncthreads();
    // per digit (thread t = digit): prefix over the waves, then over the digits
    uint32_t tot = 0;
    {
        const int t = threadIdx.x;
#pragma unroll
        for (int w = 0; w < kSegWaves; ++w) {
            const uint32_t c = s.wave_count[w][t];
            s.wave_count[w][t] = tot;
            tot += c;
        }
    }
    uint32_t all;
    const uint32_t start = block_exclusive_scan<uint32_t, kSegThreads>(tot, s.scan_tmp, all);
    s.digit_start[threadIdx.x] = start;
    digit_total = tot;
    __syncthreads();
#pragma unroll
    for (int it = 0; it < kSegItems; ++it) {
        const uint32_t d = digit_of(k[it], shift, dmask);
        pos[it] = s.digit_start[d] + s.wave_count[wave][d] + rank[it];
    }
    __syncthreads();
}

static_assert(kRadixMax == kSegThreads, "one digit per thread in seg_rank");
static_assert(kRadixMax == kSegThreads, "one digit per thread in seg_rank");

// LSD plan over the bits below the highest set bit of `diff` (the OR of every
// key XOR the first): passes of at most kSegDigitBits bits, as few as
// possible, of equal width.
struct SegPlan {
    int passes, width, bits;
};

__device__ __forceinline__ SegPlan seg_plan(uint32_t diff) {
    SegPlan p;
    p.bits = diff == 0 ? 0 : 32 - __clz(diff);
    p.passes = (p.bits + kSegDigitBits - 1) / kSegDigitBits;
    p.width = p.passes ? (p.bits + p.passes - 1) / p.passes : 0;
    return p;
}

struct SegArgs {
    // (a): ordered by bucket; the values end in full depth order.  The keys of
    // (a) are never written: other workgroups search bucket boundaries in them.
    const uint32_t *keys;
    uint32_t *vals;
    uint32_t *keys_b, *vals_b, *keys_c;  // scratch of the global-memory path
    const int64_t *n_live;          // device: live keys
    const uint32_t *xform;          // device DepthXform (the bucket shift)
    int64_t n;                      // positions (Gaussians)
    const uint2 *rects;             // packed tile rectangle per Gaussian
    uint64_t *counts_out;           // general level 1: supertile count per depth position
    uint2 *rects_out;               // one-pass level 1: rectangle per depth position
    // one-pass level 1: its (supertile, block) entry counts, added here per emitted
    // position (hist_index(s, p / kL1Threads, l1_nblocks), zeroed by count_tiles_kernel)
    uint32_t *l1_hist;
    int super_x, l1_nblocks;
};

// Per-position outputs of the sorted order: the rectangle or the supertile
// count of the Gaussian at depth position p (sentinels past the live keys).
__device__ __forceinline__ void seg_store(const SegArgs &a, int64_t p, uint2 r) {
    if (a.counts_out) a.counts_out[p] = rect_supertiles(r);
    if (a.rects_out) a.rects_out[p] = r;
}

__device__ __forceinline__ void seg_emit(const SegArgs &a, int64_t p, uint32_t val) {
    seg_store(a, p, rect_or_empty(a.rects, val, a.n));
}

// Level-1 positions per workgroup (the blocks of the one-pass level 1's counts).
constexpr int kL1Threads = 512;

// Calls f(s) for every supertile the packed tile rectangle r meets (none when empty).
template <typename F>
__device__ __forceinline__ void for_each_supertile(uint2 r, int super_x, F f) {
    const TileRect t = unpack_rect(r);
    if (t.tx0 > t.tx1) return;
    for (int y = t.ty0 / kSuper; y <= t.ty1 / kSuper; ++y)
        for (int x = t.tx0 / kSuper; x <= t.tx1 / kSuper; ++x) f(y * super_x + x);
}

// The LDS path's level-1 counts: the chunk [start, start + size) meets at most
// three kL1Threads-position blocks (size <= kSegMax); each is counted per
// supertile in the now free key buffer and its non-zero counts added to the
// table.  Every thread of the workgroup calls it (it contains barriers).
__device__ void seg_l1_counts(const SegArgs &a, uint32_t start, uint32_t size,
                              const uint2 (&r)[kSegItems], const bool (&valid)[kSegItems],
                              int ipw, SegLds &s) {
    uint32_t *cnt = s.keys[0];  // 3 x kRadixMax counters
    const uint32_t b0 = start / kL1Threads;
    const uint32_t nb = (start + size - 1) / kL1Threads - b0 + 1;  // 1..3
    __syncthreads();  // every thread has read its sorted keys out of the buffers
    for (int i = threadIdx.x; i < 3 * kRadixMax; i += kSegThreads) cnt[i] = 0u;
    __syncthreads();
#pragma unroll
    for (int it = 0; it < kSegItems; ++it) {
        if (!valid[it]) continue;
        const uint32_t row = (start + (uint32_t)seg_slot(it, ipw)) / kL1Threads - b0;
        for_each_supertile(r[it], a.super_x,
                           [&](int st) { atomicAdd(&cnt[row * kRadixMax + st], 1u); });
    }
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < nb * kRadixMax; i += kSegThreads) {
        const uint32_t c = cnt[i];
        if (c)
            atomicAdd(&a.l1_hist[hist_index((int)(i % kRadixMax), (int)(b0 + i / kRadixMax),
                                            a.l1_nblocks)],
                      c);
    }
}


// The chunk [start, end) (more than kSegMax keys) sorted by this workgroup
// through global memory: LSD passes over the varying digits at the chunk's
// positions, the keys from (a) into (b) and then between (b) and (c), the
// values between (a) and (b); the values end in (a).
__device__ void seg_sort_global(const SegArgs &a, uint32_t start, uint32_t end, SegLds &s) {
    const uint32_t size = end - start;
    const uint32_t k0 = a.keys[start];
    uint32_t diff = 0;
    for (uint32_t t = threadIdx.x; t < size; t += kSegThreads) diff |= a.keys[start + t] ^ k0;
    const SegPlan plan = seg_plan(seg_reduce<false>(diff, s));
    const uint32_t *src_k = a.keys;
    uint32_t *src_v = a.vals, *dst_k = a.keys_b, *dst_v = a.vals_b;
    for (int p = 0; p < plan.passes; ++p) {
        const int shift = p * plan.width;
        const int nbits = min(plan.width, plan.bits - shift);
        const uint32_t dmask = (1u << nbits) - 1u;
        s.running[threadIdx.x] = 0u;
        __syncthreads();
        // digit histogram of the chunk
        for (uint32_t t0 = 0; t0 < size; t0 += kSegMax) {
            const uint32_t tsize = min((uint32_t)kSegMax, size - t0);
            const int ipw = seg_items(tsize);
#pragma unroll
            for (int it = 0; it < kSegItems; ++it) {
                if (it >= ipw) continue;  // uniform
                const uint32_t q = (uint32_t)seg_slot(it, ipw);
                const bool valid = q < tsize;
                const uint32_t d = digit_of(valid ? src_k[start + t0 + q] : 0u, shift, dmask);
                const uint64_t peers = match_digit(d, nbits, __ballot(valid));
                if (valid && (peers & lanemask_lt()) == 0)
                    atomicAdd(&s.running[d], (uint32_t)__popcll(peers));
            }
        }
        __syncthreads();
        uint32_t all;
        const uint32_t first =
            block_exclusive_scan<uint32_t, kSegThreads>(s.running[threadIdx.x], s.scan_tmp, all);
        s.running[threadIdx.x] = first;  // next free offset of each digit
        __syncthreads();
        // stable scatter, tile by tile in order
        for (uint32_t t0 = 0; t0 < size; t0 += kSegMax) {
            const uint32_t tsize = min((uint32_t)kSegMax, size - t0);
            const int ipw = seg_items(tsize);
            uint32_t k[kSegItems], v[kSegItems], pos[kSegItems];
            bool valid[kSegItems];
#pragma unroll
            for (int it = 0; it < kSegItems; ++it) {
                const uint32_t q = (uint32_t)seg_slot(it, ipw);
                valid[it] = it < ipw && q < tsize;
                k[it] = valid[it] ? src_k[start + t0 + q] : 0u;
                v[it] = valid[it] ? src_v[start + t0 + q] : 0u;
            }
            uint32_t tile_total;
            seg_rank(k, valid, ipw, shift, nbits, pos, s, tile_total);
            const uint32_t base_d = s.running[threadIdx.x];
#pragma unroll
            for (int it = 0; it < kSegItems; ++it) {
                if (!valid[it]) continue;
                const uint32_t d = digit_of(k[it], shift, dmask);
                // rank within the tile's keys of digit d, after the digit's keys
                // of the earlier tiles
                const uint32_t dst = s.running[d] + (pos[it] - s.digit_start[d]);
                if (dst < size) {  // always true for consistent counts; guards the store
                    dst_k[start + dst] = k[it];
                    dst_v[start + dst] = v[it];
                }
            }
            __syncthreads();
            s.running[threadIdx.x] = base_d + tile_total;
            __syncthreads();
        }
        uint32_t *written_k = dst_k, *tv = src_v;
        dst_k = written_k == a.keys_b ? a.keys_c : a.keys_b;
        src_k = written_k;
        src_v = dst_v;
        dst_v = tv;
        __syncthreads();
    }
    // the values end in (a)
    if (src_v != a.vals)
        for (uint32_t t = threadIdx.x; t < size; t += kSegThreads) a.vals[start + t] = src_v[start + t];
    __syncthreads();
    for (uint32_t t = threadIdx.x; t < size; t += kSegThreads) {
        const uint32_t p = start + t;
        const uint2 r = rect_or_empty(a.rects, a.vals[p], a.n);
        seg_store(a, p, r);
        if (a.l1_hist)  // a rare path: one table atomic per (position, supertile)
            for_each_supertile(r, a.super_x, [&](int st) {
                atomicAdd(&a.l1_hist[hist_index(st, (int)(p / kL1Threads), a.l1_nblocks)], 1u);
            });
    }
}

__global__ __launch_bounds__(kSegThreads) void segment_sort_kernel(SegArgs a) {
    __shared__ SegLds s;
    const int64_t live64 = *a.n_live;
    const uint32_t live = (uint32_t)(live64 < a.n ? live64 : a.n);
    const uint32_t lo = (uint32_t)blockIdx.x * kSegChunk;
    const uint32_t hi = (uint32_t)min((int64_t)lo + kSegChunk, a.n);
    // positions past the live keys: sentinels
    for (uint32_t p = max(lo, live) + threadIdx.x; p < hi; p += kSegThreads) {
        a.vals[p] = 0xFFFFFFFFu;
        seg_emit(a, p, 0xFFFFFFFFu);
    }
    if (lo >= live) return;  // uniform across the workgroup
    const BucketFn bf = bucket_fn(a.xform);
    // The chunk [start, end): start = the first bucket beginning at or after lo
    // (0 for lo = 0), end = the first bucket beginning at or after hi (live
    // past the live keys).  Both come from the window [lo, lo + wlen) loaded
    // here, which also holds the chunk's keys unless its last bucket runs past
    // the window; the buckets <= that of position lo - 1 (resp. hi - 1) form a
    // prefix of the window.
    const uint32_t wlen = min((uint32_t)kSegMax, live - lo);
    const int wipw = seg_items(wlen);
    const uint32_t b_lo = lo > 0 ? bf(a.keys[lo - 1]) : 0u;
    const bool end_in = hi < live;  // else end = live
    const uint32_t b_hi = end_in ? bf(a.keys[hi - 1]) : 0u;
    uint32_t wk[kSegItems], wv[kSegItems];
    uint32_t c_lo = 0, c_hi = 0;
#pragma unroll
    for (int it = 0; it < kSegItems; ++it) {
        const uint32_t j = (uint32_t)seg_slot(it, wipw);
        const bool in = it < wipw && j < wlen;
        wk[it] = in ? a.keys[lo + j] : 0u;
        wv[it] = in ? a.vals[lo + j] : 0u;
        c_lo += (in && lo > 0 && bf(wk[it]) <= b_lo) ? 1u : 0u;
        c_hi += (in && end_in && bf(wk[it]) <= b_hi) ? 1u : 0u;
    }
    const uint32_t packed = seg_reduce<true>(c_lo | (c_hi << 16), s);
    c_lo = packed & 0xFFFFu;
    c_hi = packed >> 16;
    uint32_t start = lo + c_lo;
    if (c_lo == wlen && lo + wlen < live)  // the bucket of lo - 1 runs past the window
        start = bucket_end_search(a.keys, lo + wlen, live, bf, b_lo, s);
    uint32_t end = live;
    if (end_in) {
        end = lo + c_hi;
        if (c_hi == wlen && lo + wlen < live)
            end = bucket_end_search(a.keys, lo + wlen, live, bf, b_hi, s);
    }
    if (start >= end) return;  // uniform: no bucket begins in this range
    const uint32_t size = end - start;
    if (size > (uint32_t)kSegMax) {
        seg_sort_global(a, start, end, s);
        return;
    }
    // LDS path: the chunk in buffer 0 (from the window, or loaded again when its
    // last bucket runs past the window), then LSD passes between the buffers
    if (end <= lo + wlen) {
        const uint32_t off = start - lo;
#pragma unroll
        for (int it = 0; it < kSegItems; ++it) {
            const uint32_t j = (uint32_t)seg_slot(it, wipw);
            if (it < wipw && j >= off && j < off + size) {
                s.keys[0][j - off] = wk[it];
                s.vals[0][j - off] = wv[it];
            }
        }
    } else {
        for (uint32_t q = threadIdx.x; q < size; q += kSegThreads) {
            s.keys[0][q] = a.keys[start + q];
            s.vals[0][q] = a.vals[start + q];
        }
    }
    __syncthreads();
    const int ipw = seg_items(size);
    uint32_t k[kSegItems], v[kSegItems];
    bool valid[kSegItems];
    uint32_t diff = 0;
    const uint32_t k0 = s.keys[0][0];
#pragma unroll
    for (int it = 0; it < kSegItems; ++it) {
        const uint32_t q = (uint32_t)seg_slot(it, ipw);
        valid[it] = it < ipw && q < size;
        k[it] = valid[it] ? s.keys[0][q] : 0u;
        v[it] = valid[it] ? s.vals[0][q] : 0u;
        diff |= valid[it] ? (k[it] ^ k0) : 0u;
    }
    const SegPlan plan = seg_plan(seg_reduce<false>(diff, s));
    for (int p = 0; p < plan.passes; ++p) {
        const int sh = p * plan.width;
        uint32_t pos[kSegItems], total;
        seg_rank(k, valid, ipw, sh, min(plan.width, plan.bits - sh), pos, s, total);
        uint32_t *dk = s.keys[(p + 1) & 1], *dv = s.vals[(p + 1) & 1];
#pragma unroll
        for (int it = 0; it < kSegItems; ++it) {
            if (valid[it] && pos[it] < (uint32_t)kSegMax) {
                dk[pos[it]] = k[it];
                dv[pos[it]] = v[it];
            }
        }
        __syncthreads();
#pragma unroll
        for (int it = 0; it < kSegItems; ++it) {
            const int q = seg_slot(it, ipw);
            if (valid[it]) {
                k[it] = dk[q];
                v[it] = dv[q];
            }
        }
    }
    // sorted: item it of this thread is position seg_slot(it, ipw) of the chunk;
    // every rectangle is loaded before the first store, so the loads overlap
    uint2 r[kSegItems];
#pragma unroll
    for (int it = 0; it < kSegItems; ++it)
        r[it] = rect_or_empty(a.rects, valid[it] ? v[it] : 0xFFFFFFFFu, a.n);
#pragma unroll
    for (int it = 0; it < kSegItems; ++it) {
        if (!valid[it]) continue;
        const uint32_t p = start + (uint32_t)seg_slot(it, ipw);
        a.vals[p] = v[it];
        seg_store(a, p, r[it]);
    }
    if (a.l1_hist) seg_l1_counts(a, start, size, r, valid, ipw, s);  // uniform
}

// ------------------------------------------------------------- binning

// Tile rectangle and depth sort key per Gaussian (tiles_touched and the keys'
// depth bits: src/cuda/kernel.cu:784-818).  Gaussians without tiles get the
// key kNoTilesKey and kEmptyRect (the first depth pass drops them); so does a
// Gaussian whose depth bits equal kNoTilesKey (a NaN), which therefore gets no
// tiles.  block_sums[3 b + f] = the block's tiles (f = 0), supertile entries
// (f = 1) and Gaussians with tiles (f = 2); block_minmax[2 b] and [2 b + 1] =
// the least and greatest key of the block's Gaussians with tiles (0xFFFFFFFF
// and 0 when it has none).
template <int ITEMS>
__global__ __launch_bounds__(kSortThreads) void count_tiles_kernel(
    int64_t n, const float *__restrict__ points_image, const float *__restrict__ radii,
    const float *__restrict__ depths, const uint8_t *__restrict__ mask, int width, int height,
    int tile_size, uint2 *__restrict__ rects, uint32_t *__restrict__ depth_keys,
    unsigned long long *__restrict__ block_sums, uint32_t *__restrict__ block_minmax,
    uint32_t hint_kmin, int hint_shift, uint32_t *__restrict__ hist,
    uint32_t *__restrict__ xform, uint32_t *__restrict__ zero_words, int64_t zero_count) {
    // the one-pass level 1's count table, which the segment sort adds into
    for (int64_t i = (int64_t)blockIdx.x * kSortThreads + threadIdx.x; i < zero_count;
         i += (int64_t)gridDim.x * kSortThreads)
        zero_words[i] = 0u;
    // per-wave tiles and supertile entries; Gaussians with tiles, least and
    // greatest key
    __shared__ unsigned long long wave_sum[2][kSortThreads / kWave];
    __shared__ uint32_t wave_red[3][kSortThreads / kWave];
    __shared__ uint32_t counts[kRadixMax];
    if (hist) {  // with a depth hint: the first depth pass's histogram, zeroed here
        for (int d = threadIdx.x; d < kRadixMax; d += kSortThreads) counts[d] = 0;
        if (blockIdx.x == 0 && threadIdx.x == 0) {
            xform[0] = hint_kmin;
            xform[1] = (uint32_t)hint_shift;
        }
    }
    const int64_t base = (int64_t)blockIdx.x * (kSortThreads * ITEMS);
    unsigned long long my_tiles = 0, my_entries = 0;
    uint32_t my_live = 0;
    uint32_t kmin = 0xFFFFFFFFu, kmax = 0u;
    uint32_t keys[ITEMS];
    bool live[ITEMS];
    // all loads first (clamped index, no control dependence) so they overlap
    float2 pt[ITEMS], rd[ITEMS];
    float dp[ITEMS];
    uint8_t mk[ITEMS];
#pragma unroll
    for (int it = 0; it < ITEMS; ++it) {
        const int64_t i0 = base + slot_index<ITEMS>(it);
        const int64_t i = i0 < n ? i0 : n - 1;
        pt[it] = reinterpret_cast<const float2 *>(points_image)[i];
        rd[it] = reinterpret_cast<const float2 *>(radii)[i];
        dp[it] = depths[i];
        mk[it] = mask[i];
    }
#pragma unroll
    for (int it = 0; it < ITEMS; ++it) {
        const int64_t i = base + slot_index<ITEMS>(it);
        keys[it] = 0u;
        live[it] = false;
        if (i >= n) continue;
        TileRect r{0, 0, 0, 0};
        const uint32_t bits = __float_as_uint(dp[it]);
        const bool has = mk[it] && bits != kNoTilesKey &&
                         tile_rect(pt[it].x, pt[it].y, rd[it].x, rd[it].y, width, height,
                                   tile_size, r);
        const uint2 packed = has ? pack_rect(r) : kEmptyRect;
        rects[i] = packed;
        depth_keys[i] = has ? bits : kNoTilesKey;
        my_tiles += rect_tiles(packed);
        my_entries += rect_supertiles(packed);
        my_live += has ? 1u : 0u;
        kmin = has ? min(kmin, bits) : kmin;
        kmax = has ? max(kmax, bits) : kmax;
        keys[it] = bits;
        live[it] = has;
    }
    // the block's totals: wave reductions, then one barrier (which also orders
    // the zeroing of the histogram before its use)
    for (int o = kWave / 2; o > 0; o >>= 1) {
        my_tiles += (unsigned long long)__shfl_xor((long long)my_tiles, o, kWave);
        my_entries += (unsigned long long)__shfl_xor((long long)my_entries, o, kWave);
        my_live += (uint32_t)__shfl_xor((int)my_live, o, kWave);
        kmin = min(kmin, (uint32_t)__shfl_xor((int)kmin, o, kWave));
        kmax = max(kmax, (uint32_t)__shfl_xor((int)kmax, o, kWave));
    }
    const int wave = threadIdx.x / kWave;
    if (threadIdx.x % kWave == 0) {
        wave_sum[0][wave] = my_tiles;
        wave_sum[1][wave] = my_entries;
        wave_red[0][wave] = my_live;
        wave_red[1][wave] = kmin;
        wave_red[2][wave] = kmax;
    }
    __syncthreads();
    if (hist) {
        BucketFn bf;
        bf.kmin = hint_kmin;
        bf.shift = hint_shift;
        bf.on = true;
        // the first depth pass's digit: the bucket's low byte
        block_count_digits<ITEMS>(keys, live, 0, kRadixMaxBits, counts, bf);
    }
    if (threadIdx.x == 0) {
        unsigned long long t = 0, e = 0;
        uint32_t l = 0, lo = 0xFFFFFFFFu, hi = 0u;
#pragma unroll
        for (int w = 0; w < kSortThreads / kWave; ++w) {
            t += wave_sum[0][w];
            e += wave_sum[1][w];
            l += wave_red[0][w];
            lo = min(lo, wave_red[1][w]);
            hi = max(hi, wave_red[2][w]);
        }
        block_sums[(int64_t)blockIdx.x * 3 + 0] = t;
        block_sums[(int64_t)blockIdx.x * 3 + 1] = e;
        block_sums[(int64_t)blockIdx.x * 3 + 2] = l;
        block_minmax[2 * (int64_t)blockIdx.x] = lo;
        block_minmax[2 * (int64_t)blockIdx.x + 1] = hi;
    }
    if (hist) {
        __syncthreads();
        for (int d = threadIdx.x; d < kRadixMax; d += kSortThreads)
            hist[hist_index(d, blockIdx.x, gridDim.x)] = counts[d];
    }
}

// DepthXform {kmin, shift}: the least key with tiles, and the shift that leaves
// 16 bits of key - kmin (its bucket: bits shift .. shift + 15, with every
// higher bit 0).  The depth passes sort by the bucket (BucketFn); the segment
// sort by the whole key.  A caller's depth hint replaces it by a transform
// chosen before the keys are known (count_tiles_kernel writes it); BucketFn's
// clamp keeps the order correct for keys outside its range.
__device__ __forceinline__ uint2 depth_xform(uint32_t kmin, uint32_t kmax) {
    if (kmin > kmax) return make_uint2(0u, 0u);  // no Gaussian with tiles
    const uint32_t range = kmax - kmin;
    const int hb = range == 0 ? -1 : 31 - __clz(range);
    return make_uint2(kmin, (uint32_t)max(hb - 15, 0));
}

// Upsweep of the first depth pass: every workgroup reduces count_tiles' block
// minima and maxima to the DepthXform (workgroup 0 stores it), then counts the
// low byte of the depth bucket (BucketFn) of its keys with tiles.
template <int ITEMS>
__global__ __launch_bounds__(kSortThreads) void depth_upsweep0_kernel(
    const uint32_t *__restrict__ keys, int64_t n, const uint32_t *__restrict__ block_minmax,
    int n_count_blocks, int nblocks, uint32_t *__restrict__ hist,
    uint32_t *__restrict__ xform) {
    __shared__ uint32_t counts[kRadixMax];
    __shared__ uint32_t mm[2][kSortThreads / kWave];
    for (int d = threadIdx.x; d < kRadixMax; d += kSortThreads) counts[d] = 0;
    uint32_t lo = 0xFFFFFFFFu, hi = 0u;
    for (int b = threadIdx.x; b < n_count_blocks; b += kSortThreads) {
        lo = min(lo, block_minmax[2 * (int64_t)b]);
        hi = max(hi, block_minmax[2 * (int64_t)b + 1]);
    }
    for (int o = kWave / 2; o > 0; o >>= 1) {
        lo = min(lo, (uint32_t)__shfl_xor((int)lo, o, kWave));
        hi = max(hi, (uint32_t)__shfl_xor((int)hi, o, kWave));
    }
    if (threadIdx.x % kWave == 0) {
        mm[0][threadIdx.x / kWave] = lo;
        mm[1][threadIdx.x / kWave] = hi;
    }
    __syncthreads();
    lo = 0xFFFFFFFFu;
    hi = 0u;
#pragma unroll
    for (int w = 0; w < kSortThreads / kWave; ++w) {
        lo = min(lo, mm[0][w]);
        hi = max(hi, mm[1][w]);
    }
    const uint2 xf = depth_xform(lo, hi);
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        xform[0] = xf.x;
        xform[1] = xf.y;
    }
    const int64_t base = (int64_t)blockIdx.x * (kSortThreads * ITEMS);
    uint32_t k[ITEMS];
    bool valid[ITEMS];
#pragma unroll
    for (int it = 0; it < ITEMS; ++it) {
        const int64_t i = base + slot_index<ITEMS>(it);
        const uint32_t key = i < n ? keys[i] : kNoTilesKey;
        valid[it] = key != kNoTilesKey;
        k[it] = valid[it] ? key : 0u;
    }
    BucketFn bf;
    bf.kmin = xf.x;
    bf.shift = (int)xf.y;
    bf.on = true;
    block_count_digits<ITEMS>(k, valid, 0, kRadixMaxBits, counts, bf);
    __syncthreads();
    for (int d = threadIdx.x; d < kRadixMax; d += kSortThreads)
        hist[hist_index(d, blockIdx.x, nblocks)] = counts[d];
}

struct EmitArgs {
    const uint2 *rects;       // packed tile rectangle per Gaussian
    const uint32_t *order;    // Gaussians in depth order
    const uint64_t *offsets;  // first entry of each depth-ordered Gaussian
    int64_t n, k;
    int tiles_x;              // width of the grid the entries index
};

// indexing_offset[t] = first sorted position whose tile is >= t.
template <typename KeyT>
__global__ __launch_bounds__(256) void tile_ranges_kernel(int n_tiles,
                                                          const KeyT *__restrict__ tiles,
                                                          int64_t k,
                                                          int32_t *__restrict__ offsets) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n_tiles) return;
    int64_t lo = 0, hi = k;
    while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        if ((uint32_t)tiles[mid] < (uint32_t)t)
            lo = mid + 1;
        else
            hi = mid;
    }
    offsets[t] = (int32_t)lo;
}

// tiles_touched per Gaussian from its packed tile rectangle.
__global__ __launch_bounds__(256) void tiles_from_rects_kernel(int64_t n,
                                                               const uint2 *__restrict__ rects,
                                                               int32_t *__restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = (int32_t)rect_tiles(rects[i]);
}

// ----------------------------------------------------- level 2: tiles

// Level 1 leaves, for every supertile s, the ids of the Gaussians whose tile
// rectangle meets s, in depth order (list positions super_off[s] ..
// super_off[s + 1]).  Level 2 cuts each list into chunks of kL2Threads
// (512) positions (block b <-> supertile s, chunk b - chunk_start[s]); a lane holds
// one Gaussian and the 64-bit mask of the supertile's tiles its rectangle
// covers.  Per local tile j, one ballot gives the lanes (in list order) that
// write an entry: l2_count_kernel counts them per block and per tile,
// l2_scatter_kernel writes the ids to
//   indexing_offset[t] + (entries of t in earlier blocks of s) +
//   (entries of t in earlier waves of the block) + (rank in the ballot).
// Within a tile the entries therefore keep the depth order of the lists.
struct L2Args {
    const int32_t *super_off;     // n_super: first list position of each supertile
    const int32_t *super_ids;     // m: Gaussian ids per supertile, depth order
    const uint32_t *chunk_start;  // n_super + 1: first level-2 block of each supertile
    const uint4 *block_map;       // per level-2 workgroup w: (supertile, first and end list
                                  // position, logical block xcd_block(w, chunks)), laid out
                                  // so that each XCD takes a contiguous range of the
                                  // chunks; supertile kNoBlock past the last chunk
    const uint2 *super_rects;     // m: packed tile rectangle of each list entry
    int64_t n, m, k;
    int n_super, super_x, tiles_x, tiles_y, width, height, tile_size;
    int64_t nblocks;              // level-2 blocks the grid covers (a bound on the chunks)
    // capped sort (gs_bin_sort_capped): device K and M; k and m above are then the
    // capacities.  K > k or M > m: no output (every tile empty at offset k).
    // Otherwise the positions are shifted by k - K, so that the last tile's list
    // ends at k, the capacity (ids[0 .. k - K) are not part of any list).
    const int64_t *cap_totals;
};

__device__ __forceinline__ bool capped_overflow(const L2Args &a) {
    return a.cap_totals && (a.cap_totals[0] > a.k || a.cap_totals[1] > a.m);
}

// block_map entry of the blocks past the last chunk (the grid is sized by a bound).
constexpr uint32_t kNoBlock = 0xFFFFFFFFu;

// One workgroup: chunks of every supertile's list (kL2Threads entries each),
// their exclusive scan chunk_start (chunk_start[n_super] = all chunks), the
// block map (entry xcd_block_inverse(b, chunks) = (supertile, first and end
// list position, b) for every logical level-2 block b, kNoBlock past the last
// chunk) and zeroed per-tile entry counters.  Thread i handles a contiguous run
// of supertiles.
constexpr int kPlanThreads = 1024;

__global__ __launch_bounds__(kPlanThreads) void l2_plan_kernel(
    int n_super, int64_t m, const int32_t *__restrict__ super_off,
    uint32_t *__restrict__ chunk_start, uint4 *__restrict__ block_map, int64_t nblocks,
    int n_tiles, uint32_t *__restrict__ tile_counts) {
    __shared__ uint32_t tmp[kPlanThreads / kWave + 1];
    for (int t = threadIdx.x; t < n_tiles; t += kPlanThreads) tile_counts[t] = 0u;
    const int per = (n_super + kPlanThreads - 1) / kPlanThreads;
    const int s0 = min((int)threadIdx.x * per, n_super), s1 = min(s0 + per, n_super);
    auto chunks_of = [&](int s) {
        const int64_t end = s + 1 < n_super ? super_off[s + 1] : m;
        return (uint32_t)((end - super_off[s] + kL2Threads - 1) / kL2Threads);
    };
    uint32_t mine = 0;
    for (int s = s0; s < s1; ++s) mine += chunks_of(s);
    uint32_t total;
    uint32_t b = block_exclusive_scan<uint32_t, kPlanThreads>(mine, tmp, total);
    for (int s = s0; s < s1; ++s) {
        chunk_start[s] = b;
        const uint32_t first = (uint32_t)super_off[s], c = chunks_of(s);
        const uint32_t end = (uint32_t)(s + 1 < n_super ? super_off[s + 1] : m);
        for (uint32_t i = 0; i < c; ++i) {
            const uint32_t e0 = first + i * kL2Threads;
            block_map[xcd_block_inverse(b + i, total)] =
                make_uint4((uint32_t)s, e0, min(e0 + kL2Threads, end), b + i);
        }
        b += c;
    }
    if (threadIdx.x == 0) chunk_start[n_super] = total;
    for (int64_t q = (int64_t)total + threadIdx.x; q < nblocks; q += kPlanThreads)
        block_map[q] = make_uint4(kNoBlock, 0u, 0u, 0u);
}

// Tile id of local tile j of supertile s, or -1 outside the tile grid.
__device__ __forceinline__ int tile_of_local(const L2Args &a, int s, int j) {
    const int tx = (s % a.super_x) * kSuper + (j % kSuper);
    const int ty = (s / a.super_x) * kSuper + (j / kSuper);
    return (tx < a.tiles_x && ty < a.tiles_y) ? ty * a.tiles_x + tx : -1;
}

struct L2Block {
    int s;
    uint32_t b;
    uint32_t trow;  // table[b * kSuperLocal + thread] for the first kSuperLocal threads
    int32_t g;
    uint64_t mask;
    int lx0, lx1, ly0, ly1;  // the mask as a rectangle of local tiles (empty: lx0 > lx1)
};

// Bit j (= ly * kSuper + lx) set for every tile of supertile s that Gaussian
// g (list entry e, whose tile rectangle is super_rects[e]) covers; the covered
// local rectangle goes to x.
__device__ __forceinline__ uint64_t local_mask(const L2Args &a, int32_t g, uint2 packed, int s,
                                               L2Block &x) {
    x.lx0 = x.ly0 = 1;
    x.lx1 = x.ly1 = 0;
    if (g < 0 || (int64_t)g >= a.n) return 0;
    const TileRect r = unpack_rect(packed);  // Gaussians in the lists have tiles
    const int ox = (s % a.super_x) * kSuper, oy = (s / a.super_x) * kSuper;
    const int x0 = max(r.tx0 - ox, 0), x1 = min(r.tx1 - ox, kSuper - 1);
    const int y0 = max(r.ty0 - oy, 0), y1 = min(r.ty1 - oy, kSuper - 1);
    if (x0 > x1 || y0 > y1) return 0;
    x.lx0 = x0;
    x.lx1 = x1;
    x.ly0 = y0;
    x.ly1 = y1;
    const uint64_t row = ((1ull << (x1 - x0 + 1)) - 1ull) << x0;
    uint64_t m = 0;
    for (int y = y0; y <= y1; ++y) m |= row << (y * kSuper);
    return m;
}

// Block -> supertile, this lane's Gaussian and mask.  Returns false (uniformly)
// for the blocks past the last chunk (the grid is sized by an upper bound).
// Workgroup w handles block w - skip (the first `skip` workgroups, a multiple of
// kBinXcds, do other work).
__device__ __forceinline__ bool l2_block(const L2Args &a, L2Block &x, uint32_t skip = 0,
                                         const uint32_t *__restrict__ table = nullptr) {
    // workgroup -> logical block through the map (no dependent read of the chunk
    // count): the live chunks are spread over the XCDs whatever the grid's bound
    const uint4 map = a.block_map[blockIdx.x - skip];
    if (map.x == kNoBlock || capped_overflow(a)) return false;
    x.b = map.w;  // the logical block: its row of the table
    // this block's row of the table, loaded beside the list entries
    x.trow = table && threadIdx.x < kSuperLocal ? table[(int64_t)x.b * kSuperLocal + threadIdx.x]
                                                : 0u;
    x.s = (int)map.x;
    const int64_t end = (int64_t)map.z;
    const int64_t e = (int64_t)map.y + threadIdx.x;
    // every lane loads (a block holds at least one entry, so the clamped position
    // is in its list): no load on a conditional path, which would make the
    // compiler wait for all memory operations, stores included, before each of the
    // scatter's stores of x.g
    const int64_t ec = e < end ? e : end - 1;
    const int32_t g = a.super_ids[ec];
    const uint2 packed = a.super_rects[ec];
    x.g = e < end ? g : -1;
    x.mask = local_mask(a, x.g, packed, x.s, x);
    return true;
}

// The lanes of this wave covering local row q (rows[q]) and local column q
// (cols[q]) of the supertile, one ballot each (uniform masks); returns, in lane
// j = (ly, lx), the number of lanes covering local tile j: the lanes covering
// both its row and its column.
__device__ __forceinline__ uint32_t wave_masks(const L2Block &x, uint64_t (&rows)[kSuper],
                                               uint64_t (&cols)[kSuper]) {
    const int lane = threadIdx.x % kWave;
    uint64_t mine_row = 0, mine_col = 0;
#pragma unroll
    for (int q = 0; q < kSuper; ++q) {
        rows[q] = __ballot(x.ly0 <= q && q <= x.ly1);
        cols[q] = __ballot(x.lx0 <= q && q <= x.lx1);
        mine_row = lane / kSuper == q ? rows[q] : mine_row;
        mine_col = lane % kSuper == q ? cols[q] : mine_col;
    }
    return (uint32_t)__popcll(mine_row & mine_col);
}

// table[b * kSuperLocal + j] = entries of local tile j in level-2 block b;
// tile_counts[t] += the same count for tile t.
__global__ __launch_bounds__(kL2Threads) void l2_count_kernel(L2Args a,
                                                              uint32_t *__restrict__ table,
                                                              uint32_t *__restrict__ tile_counts) {
    __shared__ uint32_t wave_cnt[kL2Waves][kSuperLocal];
    L2Block x;
    if (!l2_block(a, x)) return;
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    uint64_t rows[kSuper], cols[kSuper];
    wave_cnt[wave][lane] = wave_masks(x, rows, cols);
    __syncthreads();
    if (threadIdx.x < kSuperLocal) {
        const int j = threadIdx.x;
        uint32_t c = 0;
#pragma unroll
        for (int w = 0; w < kL2Waves; ++w) c += wave_cnt[w][j];
        table[(int64_t)x.b * kSuperLocal + j] = c;
        const int t = tile_of_local(a, x.s, j);
        if (c && t >= 0) atomicAdd(&tile_counts[t], c);
    }
}

// Largest tile grid whose entry-count scan each l2_prefix_kernel workgroup
// computes itself (larger grids use a separate scan into indexing_offset).
constexpr int kFusedTileScanMax = 16384;
constexpr int kPrefixBatch = 16;  // chunk rows read per batch (independent loads)

// One workgroup per supertile s.  First the first output position of each of
// its tiles: the exclusive scan of tile_counts over the tile grid, computed
// here when the grid has at most kFusedTileScanMax tiles (and written to
// indexing_offset), else read from indexing_offset.  Then, per local tile j,
// the exclusive scan of table[b][j] over the supertile's level-2 blocks b,
// started at that position, in place: wave v scans a contiguous run of
// blocks, after the sums of the runs before it.
__global__ __launch_bounds__(kL2Threads) void l2_prefix_kernel(
    L2Args a, const uint32_t *__restrict__ tile_counts, int n_tiles, int fused_scan,
    int32_t *__restrict__ indexing_offset, uint32_t *__restrict__ table) {
    __shared__ uint32_t tmp[kL2Waves + 1];
    __shared__ uint32_t thread_base[kL2Threads];
    __shared__ uint32_t tile_pre[kFusedTileScanMax];  // prefix within the owning thread's run
    __shared__ uint32_t tile_off[kSuperLocal];
    __shared__ uint32_t run_sum[kL2Waves][kSuperLocal];
    const int s = blockIdx.x;
    const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
    if (capped_overflow(a)) {  // no lists: every tile empty at the capacity
        if (tid < kSuperLocal) {
            const int t = tile_of_local(a, s, tid);
            if (t >= 0) indexing_offset[t] = (int32_t)a.k;
        }
        return;
    }
    // capped sort: lists end at the capacity k (see L2Args)
    const uint32_t shift = a.cap_totals ? (uint32_t)(a.k - a.cap_totals[0]) : 0u;
    const int per = (n_tiles + kL2Threads - 1) / kL2Threads;
    if (fused_scan) {
        const int t0 = min(tid * per, n_tiles), t1 = min(t0 + per, n_tiles);
        uint32_t mine = 0;
#pragma unroll 8
        for (int t = t0; t < t1; ++t) {
            tile_pre[t] = mine;
            mine += tile_counts[t];
        }
        uint32_t total;
        thread_base[tid] = block_exclusive_scan<uint32_t, kL2Threads>(mine, tmp, total);
        __syncthreads();
    }
    if (tid < kSuperLocal) {
        const int t = tile_of_local(a, s, tid);
        uint32_t off = 0;
        if (t >= 0) {
            if (fused_scan) {
                off = thread_base[t / per] + tile_pre[t] + shift;
                indexing_offset[t] = (int32_t)off;
            } else {
                off = (uint32_t)indexing_offset[t];
            }
        }
        tile_off[tid] = off;
    }
    // the supertile's blocks [q0, q1); wave v takes [q0 + v * per_w, ...)
    const uint32_t q0 = a.chunk_start[s], q1 = a.chunk_start[s + 1];
    const uint32_t per_w = (q1 - q0 + kL2Waves - 1) / kL2Waves;
    const uint32_t r0 = min(q0 + wave * per_w, q1), r1 = min(r0 + per_w, q1);
    uint32_t sum = 0;
    for (uint32_t q = r0; q < r1; ++q) sum += table[(int64_t)q * kSuperLocal + lane];
    run_sum[wave][lane] = sum;
    __syncthreads();
    uint32_t pos = tile_off[lane];
    for (int w = 0; w < wave; ++w) pos += run_sum[w][lane];
    for (uint32_t q = r0; q < r1; q += kPrefixBatch) {
        uint32_t c[kPrefixBatch];
#pragma unroll
        for (int i = 0; i < kPrefixBatch; ++i)
            c[i] = q + i < r1 ? table[(int64_t)(q + i) * kSuperLocal + lane] : 0u;
#pragma unroll
        for (int i = 0; i < kPrefixBatch; ++i) {
            if (q + i < r1) table[(int64_t)(q + i) * kSuperLocal + lane] = pos;
            pos += c[i];
        }
    }
}

// Writes each entry's Gaussian id at its final position: lane j of every wave
// holds the first position of the wave's entries of local tile j, read back
// with readlane in the loop over tiles.  The lanes covering local tile
// (lx, ly) are those covering row ly and column lx (the rectangles' row and
// column ballots, uniform masks built once), so a tile's lane mask, its count
// and the bounds check of its run are scalar work; each covering lane stores at
// the run's start plus its rank in the mask.  k32: positions fit 32 bits
// (K < 2^30), so a store is a 32-bit offset from the uniform base.
// Blend launch order of XCD range x of the tile grid (the ranges the blend
// kernels give the XCDs: x * base + min(x, rem) onwards, base + (x < rem) tiles,
// base = n_tiles / kBinXcds): the range's tiles by ascending bit length of their
// list length (0, 1, 2-3, 4-7, ...), in tile order within a bucket.  A stable
// counting sort over 32 buckets by one workgroup of kL2Threads: a histogram,
// then the range in chunks of kL2Threads tiles, each tile placed at its
// bucket's running start plus its rank among the chunk's tiles of that bucket
// (ballot matching within a wave, per-wave counts across the waves).
__device__ void tile_launch_order(int x, int n_tiles, int64_t k, const int32_t *__restrict__ offsets,
                                  int32_t *__restrict__ order) {
    constexpr int kBuckets = 32;
    __shared__ uint32_t start_of[kBuckets];
    __shared__ uint32_t wave_cnt[kL2Waves][kBuckets];
    const int base = n_tiles / kBinXcds, rem = n_tiles % kBinXcds;
    const int first = x * base + min(x, rem), len = base + (x < rem ? 1 : 0);
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    auto bucket = [&](int t) -> uint32_t {
        const int64_t end = t + 1 < n_tiles ? (int64_t)offsets[t + 1] : k;
        const int64_t n_t = end - (int64_t)offsets[t];
        const uint32_t c = n_t > 0 ? (uint32_t)min(n_t, (int64_t)0x7fffffff) : 0u;
        return c == 0u ? 0u : 32u - (uint32_t)__clz(c);  // bit length: 0..31
    };
    if (threadIdx.x < kBuckets) start_of[threadIdx.x] = 0u;
    __syncthreads();
    for (int i = threadIdx.x; i < len; i += kL2Threads) atomicAdd(&start_of[bucket(first + i)], 1u);
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t run = 0;
        for (int d = 0; d < kBuckets; ++d) {
            const uint32_t c = start_of[d];
            start_of[d] = run;
            run += c;
        }
    }
    for (int c0 = 0; c0 < len; c0 += kL2Threads) {
        if (lane < kBuckets) wave_cnt[wave][lane] = 0u;
        __syncthreads();
        const int i = c0 + (int)threadIdx.x;
        const bool valid = i < len;
        const uint32_t d = valid ? bucket(first + i) : 0u;
        const uint64_t peers = match_digit(d, 5, __ballot(valid));
        if (valid && (peers & lanemask_lt()) == 0) wave_cnt[wave][d] = (uint32_t)__popcll(peers);
        __syncthreads();
        if (valid) {
            uint32_t pos = start_of[d] + (uint32_t)__popcll(peers & lanemask_lt());
            for (int w = 0; w < wave; ++w) pos += wave_cnt[w][d];
            order[first + (int)pos] = first + i;
        }
        __syncthreads();
        if (threadIdx.x < kBuckets) {
            uint32_t c = 0;
#pragma unroll
            for (int w = 0; w < kL2Waves; ++w) c += wave_cnt[w][threadIdx.x];
            start_of[threadIdx.x] += c;
        }
        __syncthreads();  // counts read before the next chunk clears them
    }
}

// The level-2 scatter's loop over the 64 local tiles: the lanes covering tile j
// (the AND of its row and column ballots) store their id at the tile's base for
// this wave plus their rank among those lanes.  kCheck: skip a tile whose run
// would end past ids_out.
template <bool k32, bool kCheck>
__device__ __forceinline__ void scatter_runs(const uint64_t (&rows)[kSuper],
                                             const uint64_t (&cols)[kSuper], uint32_t my_base,
                                             uint32_t k_lo, int64_t k, int32_t g,
                                             int32_t *__restrict__ ids_out) {
#pragma unroll
    for (int j = 0; j < kSuperLocal; ++j) {
        const uint64_t bal = rows[j / kSuper] & cols[j % kSuper];
        if (bal == 0) continue;  // uniform: no lane covers tile j
        const uint32_t b = __builtin_amdgcn_readlane(my_base, j);
        if (kCheck) {
            const uint32_t cnt = (uint32_t)__popcll(bal);
            if (k32 ? (b + cnt > k_lo) : ((int64_t)b + cnt > k)) continue;  // run inside ids_out
        }
        if (__builtin_amdgcn_inverse_ballot_w64(bal)) {
            // rank among the tile's lanes; the run's start joins as a scalar
            const uint32_t r = __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32),
                                                         __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
            if (k32)  // byte offset (b + r) * 4 < 2^32: a 32-bit offset from the uniform base
                *reinterpret_cast<int32_t *>(reinterpret_cast<char *>(ids_out) + ((r << 2) + (b << 2))) = g;
            else
                ids_out[(int64_t)b + r] = g;
        }
    }
}

// With launch_order, the grid has kBinXcds more workgroups than the scatter
// needs (the first ones, one per XCD): each writes the blend launch order of
// one XCD range while the scatter runs.
template <bool k32>
__global__ __launch_bounds__(kL2Threads) void l2_scatter_kernel(L2Args a,
                                                                const uint32_t *__restrict__ table,
                                                                int32_t *__restrict__ ids_out,
                                                                const int32_t *__restrict__ offsets,
                                                                int32_t *__restrict__ launch_order) {
    __shared__ uint32_t base[kL2Waves][kSuperLocal];
    if (launch_order && blockIdx.x < kBinXcds) {
        tile_launch_order((int)blockIdx.x, a.tiles_x * a.tiles_y, a.k, offsets, launch_order);
        return;
    }
    L2Block x;
    if (!l2_block(a, x, launch_order ? kBinXcds : 0, table)) return;
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    uint64_t rows[kSuper], cols[kSuper];
    const uint32_t my_cnt = wave_masks(x, rows, cols);  // lane j: this wave's entries of tile j
    base[wave][lane] = my_cnt;
    __syncthreads();
    if (threadIdx.x < kSuperLocal) {  // first position of each wave's entries of tile j
        uint32_t pos = x.trow;  // from l2_prefix_kernel
#pragma unroll
        for (int w = 0; w < kL2Waves; ++w) {
            const uint32_t c = base[w][threadIdx.x];
            base[w][threadIdx.x] = pos;
            pos += c;
        }
    }
    __syncthreads();
    const uint32_t my_base = base[wave][lane];  // lane j: tile j
    // k32: K < 2^30, so b + count cannot wrap in 32 bits (a scalar compare)
    const uint32_t k_lo = (uint32_t)(a.k < 0xffffffffLL ? a.k : 0xffffffffLL);
    // every run of the wave inside ids_out (always, for consistent counts): one
    // check for the wave instead of one per tile, which leaves the loop's scalar
    // work (the per-tile masks and the exec mask) at about two thirds
    const bool outside = my_cnt != 0u && (k32 ? my_base + my_cnt > k_lo
                                               : (int64_t)my_base + my_cnt > a.k);
    if (__ballot(outside) == 0)
        scatter_runs<k32, false>(rows, cols, my_base, k_lo, a.k, x.g, ids_out);
    else
        scatter_runs<k32, true>(rows, cols, my_base, k_lo, a.k, x.g, ids_out);
}

// Level-1 entries: for the Gaussian at depth-order position r, one entry per
// supertile of its rectangle (row-major), at offsets[r].. (thread per position).
template <typename KeyT>
__global__ __launch_bounds__(256) void emit_super_kernel(
    int64_t n, int64_t m, const uint32_t *__restrict__ order,
    const uint64_t *__restrict__ offsets, const uint2 *__restrict__ rects, int super_x,
    KeyT *__restrict__ keys_out, uint32_t *__restrict__ vals_out,
    uint2 *__restrict__ rects_out) {
    const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= n) return;
    const uint32_t g = order[r];
    if (g >= (uint64_t)n) return;  // past the Gaussians with tiles
    const uint2 packed = rects[g];
    const TileRect t = unpack_rect(packed);
    if (t.tx0 > t.tx1) return;
    int64_t o = (int64_t)offsets[r];
    for (int y = t.ty0 / kSuper; y <= t.ty1 / kSuper; ++y)
        for (int x = t.tx0 / kSuper; x <= t.tx1 / kSuper; ++x, ++o) {
            if (o >= m) return;
            keys_out[o] = (KeyT)(y * super_x + x);
            vals_out[o] = g;
            rects_out[o] = packed;
        }
}

// ---------------------------------------------- level 1 in one radix pass
// With at most kRadixMax supertiles the supertile id is a single radix digit:
// block b of kL1Threads handles the depth-ordered Gaussians [b * kL1Threads,
// ...) and enumerates their (supertile, Gaussian) entries on the fly, without
// storing them.  A Gaussian meets each supertile once, so in LDS
// lanes[w][s] has bit L set when lane L of wave w meets supertile s; the
// block's count of s is the sum of popcounts over its waves, and an entry's
// rank among the block's entries of s is the popcount of the lanes before it.
// The segment sort adds each block's counts to a digit-major table as it emits
// the depth order (seg_l1_counts), digit_scan_kernel turns them into positions,
// and l1_scatter_kernel writes every entry's id and packed tile rectangle at
// its position in the supertile-sorted list, which is stable: (supertile, depth
// order).

constexpr int kL1Waves = kL1Threads / kWave;

struct L1Args {
    const uint32_t *order;       // Gaussians in depth order
    const uint2 *rects_depth;    // their packed tile rectangles, in the same order
    const int64_t *n_live;       // device: the first *n_live positions hold Gaussians with tiles
    int64_t n, m;                // Gaussians, entries (capped sort: the entry capacity)
    int super_x, nblocks;
    const int64_t *cap_totals = nullptr;  // capped sort: device K and M (see L2Args)
};

// Whether this workgroup's positions start before *n_live (the later ones hold
// only the sentinels of Gaussians without tiles); uniform per workgroup.
__device__ __forceinline__ bool l1_live_block(const L1Args &a, int64_t blk) {
    return blk * kL1Threads < *a.n_live;
}

// Workgroups whose positions start before *n_live.
__device__ __forceinline__ int64_t l1_live_blocks(const L1Args &a) {
    return (*a.n_live + kL1Threads - 1) / kL1Threads;
}

// This thread's Gaussian and the supertile range its tile rectangle meets
// (false: none).
__device__ __forceinline__ bool l1_gaussian(const L1Args &a, int64_t blk, uint32_t &g,
                                            uint2 &packed, TileRect &sr) {
    const int64_t r = blk * kL1Threads + threadIdx.x;
    if (r >= a.n) return false;
    g = a.order[r];
    packed = a.rects_depth[r];
    const TileRect t = unpack_rect(packed);
    if (g >= (uint64_t)a.n || t.tx0 > t.tx1) return false;
    sr.tx0 = t.tx0 / kSuper;
    sr.tx1 = t.tx1 / kSuper;
    sr.ty0 = t.ty0 / kSuper;
    sr.ty1 = t.ty1 / kSuper;
    return true;
}

// lanes[w][s] for the block (zeroed here); returns whether this lane has entries.
__device__ __forceinline__ bool l1_lane_masks(const L1Args &a, int64_t blk,
                                              uint64_t (*lanes)[kRadixMax], uint32_t &g,
                                              uint2 &packed, TileRect &sr) {
    for (int i = threadIdx.x; i < kL1Waves * kRadixMax; i += kL1Threads) lanes[0][i] = 0ull;
    __syncthreads();
    const int wave = threadIdx.x / kWave;
    const uint64_t bit = 1ull << (threadIdx.x % kWave);
    const bool has = l1_gaussian(a, blk, g, packed, sr);
    if (has)
        for (int y = sr.ty0; y <= sr.ty1; ++y)
            for (int x = sr.tx0; x <= sr.tx1; ++x)
                atomicOr(reinterpret_cast<unsigned long long *>(&lanes[wave][y * a.super_x + x]),
                         (unsigned long long)bit);
    __syncthreads();
    return has;
}

// The level-2 block plan, from block 0 of l1_scatter_kernel (thread d holds
// supertile d's entry count `tot` and first list position `first`): chunks of
// kL2Threads list positions per supertile, their exclusive scan chunk_start
// (chunk_start[n_super] = all chunks) and the block map: entry w = (supertile,
// first and end list position, b) of logical block b = xcd_block(w, chunks), so
// that each XCD's workgroups take a contiguous range of chunks, and kNoBlock
// for the workgroups past the last chunk up to nblocks.  Contains
// __syncthreads().
__device__ __forceinline__ void l1_block_plan(int n_super, uint32_t tot, uint32_t first,
                                              uint32_t *scan_tmp, uint32_t *lds_start,
                                              uint32_t *lds_first, uint32_t *lds_end,
                                              uint32_t *__restrict__ chunk_start,
                                              uint4 *__restrict__ block_map, int64_t nblocks) {
    const int d = threadIdx.x;
    const uint32_t c = d < n_super ? (tot + kL2Threads - 1) / kL2Threads : 0u;
    uint32_t all;
    const uint32_t b0 = block_exclusive_scan<uint32_t, kL1Threads>(c, scan_tmp, all);
    if (d < n_super) {
        lds_start[d] = b0;
        lds_first[d] = first;
        lds_end[d] = first + tot;
        chunk_start[d] = b0;
    }
    if (d == 0) chunk_start[n_super] = all;
    __syncthreads();
    for (uint32_t w = d; w < all; w += kL1Threads) {
        const uint32_t b = (uint32_t)xcd_block(w, all);  // workgroup w's logical block
        // the last supertile whose first block is <= b (supertiles without
        // chunks share their first block with the next one)
        int lo = 0, hi = n_super - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (lds_start[mid] <= b)
                lo = mid;
            else
                hi = mid - 1;
        }
        const uint32_t e0 = lds_first[lo] + (b - lds_start[lo]) * kL2Threads;
        block_map[w] = make_uint4((uint32_t)lo, e0, min(e0 + kL2Threads, lds_end[lo]), b);
    }
    for (int64_t q = (int64_t)all + d; q < nblocks; q += kL1Threads)
        block_map[q] = make_uint4(kNoBlock, 0u, 0u, 0u);
}

// `hist` holds, after digit_scan_kernel, the first position of (s, block)
// among the entries of s and `totals` the entries of each s.  Writes
// super_ids / super_rects, zeroes the per-tile entry counters of level 2 and,
// from block 0, super_off[s] = entries with a smaller supertile and the
// level-2 block plan (l1_block_plan).
__global__ __launch_bounds__(kL1Threads) void l1_scatter_kernel(
    L1Args a, const uint32_t *__restrict__ hist, const uint32_t *__restrict__ totals,
    int n_super, int32_t *__restrict__ super_ids, uint2 *__restrict__ super_rects,
    int32_t *__restrict__ super_off, uint32_t *__restrict__ chunk_start,
    uint4 *__restrict__ block_map, int64_t l2_nblocks, int n_tiles,
    uint32_t *__restrict__ tile_counts) {
    __shared__ uint64_t lanes[kL1Waves][kRadixMax];
    __shared__ uint32_t wave_pos[kL1Waves][kRadixMax];
    __shared__ uint32_t scan_tmp[kL1Threads / kWave + 1];
    for (int64_t t = (int64_t)blockIdx.x * kL1Threads + threadIdx.x; t < n_tiles;
         t += (int64_t)gridDim.x * kL1Threads)
        tile_counts[t] = 0u;
    if (a.cap_totals && a.cap_totals[1] > a.m) return;  // past the entry capacity: no output
    const int64_t blk = blockIdx.x;  // (round robin over the XCDs measured faster here)
    if (blk != 0 && !l1_live_block(a, blk)) return;  // no entries (block 0 writes the plan)
    uint32_t g = 0;
    uint2 packed = make_uint2(0u, 0u);
    TileRect sr{0, -1, 0, -1};
    const bool has = l1_lane_masks(a, blk, lanes, g, packed, sr);
    const int d = threadIdx.x;
    const uint32_t tot = d < n_super ? totals[d] : 0u;
    uint32_t all;
    const uint32_t smaller = block_exclusive_scan<uint32_t, kL1Threads>(tot, scan_tmp, all);
    if (blk == 0) {  // uniform per workgroup; wave_pos serves as staging
        if (d < n_super) super_off[d] = (int32_t)smaller;
        l1_block_plan(n_super, tot, smaller, scan_tmp, wave_pos[0], wave_pos[1], wave_pos[2],
                      chunk_start, block_map, l2_nblocks);
        __syncthreads();
    }
    if (d < kRadixMax) {
        uint32_t pos = smaller + (d < n_super ? hist[hist_index(d, (int)blk, a.nblocks)] : 0u);
#pragma unroll
        for (int w = 0; w < kL1Waves; ++w) {
            wave_pos[w][d] = pos;
            pos += (uint32_t)__popcll(lanes[w][d]);
        }
    }
    __syncthreads();
    if (has) {
        const int wave = threadIdx.x / kWave;
        const uint64_t below = lanemask_lt();
        for (int y = sr.ty0; y <= sr.ty1; ++y)
            for (int x = sr.tx0; x <= sr.tx1; ++x) {
                const int s = y * a.super_x + x;
                const uint32_t p = wave_pos[wave][s] + (uint32_t)__popcll(lanes[wave][s] & below);
                if ((int64_t)p < a.m) {  // always true for consistent counts; guards the store
                    super_ids[p] = (int32_t)g;
                    super_rects[p] = packed;
                }
            }
    }
}

// keys[i] = tile << 32 | depth bits of ids[i], the tile being the last one
// whose offset is <= i (the reference's sorted 64-bit keys).
__global__ __launch_bounds__(256) void keys_from_offsets_kernel(
    int64_t k, int64_t n, int n_tiles, const int32_t *__restrict__ offsets,
    const int32_t *__restrict__ ids, const float *__restrict__ depths,
    uint64_t *__restrict__ keys) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= k) return;
    int lo = 0, hi = n_tiles - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if ((int64_t)offsets[mid] <= i)
            lo = mid;
        else
            hi = mid - 1;
    }
    const int32_t g = ids[i];
    const uint32_t bits = (g >= 0 && g < n) ? __float_as_uint(depths[g]) : 0u;
    keys[i] = ((uint64_t)(uint32_t)lo << 32) | (uint64_t)bits;
}

// ------------------------------------------------------ workspace layout

struct Carve {
    char *base;
    size_t off = 0;
    template <typename T>
    T *take(int64_t count) {
        off = align256(off);
        T *p = reinterpret_cast<T *>(base ? base + off : nullptr);
        off += (size_t)count * sizeof(T);
        return p;
    }
};

inline int64_t l1_blocks(int64_t n) { return (n + kL1Threads - 1) / kL1Threads; }

struct CountWs {
    uint32_t *dkeys_a, *dvals_a, *dkeys_b, *dvals_b, *dkeys_c;
    uint2 *rects;        // packed tile rectangle per Gaussian (kEmptyRect: no tiles)
    uint2 *rects_depth;  // the same in depth order (one-pass level 1)
    uint64_t *counts, *offsets;
    unsigned long long *block_sums;  // count_tiles: 3 sums per block
    uint32_t *block_minmax;          // count_tiles: least and greatest key per block
    uint32_t *xform;                 // DepthXform {kmin, shift}
    int64_t *n_live;                 // Gaussians with tiles (keys of depth passes 1..)
    int64_t *dev_totals;             // K and M in device memory (read by gs_bin_sort_capped)
    uint64_t *m_scan;                // the general level 1's entry total (equals M)
    uint32_t *l1_hist;               // one-pass level 1: kRadixMax x l1_blocks(n) table
    uint32_t *l1_totals;             // one-pass level 1: entries per supertile
    void *sort_ws, *scan_ws;
    size_t bytes;
};

inline CountWs carve_count(void *base, int64_t n) {
    Carve c{reinterpret_cast<char *>(base)};
    CountWs w;
    w.rects = c.take<uint2>(n);
    w.dkeys_a = c.take<uint32_t>(n);
    w.dvals_a = c.take<uint32_t>(n);
    w.dkeys_b = c.take<uint32_t>(n);
    w.dvals_b = c.take<uint32_t>(n);
    w.dkeys_c = c.take<uint32_t>(n);
    w.rects_depth = c.take<uint2>(n);
    w.counts = c.take<uint64_t>(n);
    w.offsets = c.take<uint64_t>(n + 1);
    w.block_sums = c.take<unsigned long long>(sort_blocks<kDepthItems>(n) * 3);
    w.block_minmax = c.take<uint32_t>(sort_blocks<kDepthItems>(n) * 2);
    w.xform = c.take<uint32_t>(2);
    w.dev_totals = c.take<int64_t>(2);
    w.n_live = c.take<int64_t>(1);
    w.m_scan = c.take<uint64_t>(1);
    w.l1_hist = c.take<uint32_t>(kRadixMax * l1_blocks(n));
    w.l1_totals = c.take<uint32_t>(kRadixMax);
    w.sort_ws = c.take<char>((int64_t)radix_workspace_bytes<kDepthItems>(n));
    w.scan_ws = c.take<char>((int64_t)scan_workspace_bytes<uint64_t>(n));
    w.bytes = align256(c.off);
    return w;
}

// One-pass level-1 arguments over the depth order the count workspace holds
// (the last depth pass writes into the (a) buffers); m bounds the scatter.
inline L1Args l1_args(const CountWs &cw, int64_t n, int64_t m, int super_x) {
    L1Args la;
    la.order = cw.dvals_a;
    la.rects_depth = cw.rects_depth;
    la.n_live = cw.n_live;
    la.n = n;
    la.m = m;
    la.super_x = super_x;
    la.nblocks = (int)l1_blocks(n);
    return la;
}

// The depth sort: two radix passes over the bucket bits of key - kmin (bits
// shift .. shift + 7, then shift + 8 .. shift + 15), (a) -> (b) -> (a), then
// segment_sort_kernel in place on (a).  The first pass drops the Gaussians
// without tiles and writes key - kmin; the segment sort fills the tail.
constexpr int kDepthPassShift[2] = {0, 8};  // digit p: bits 8p .. 8p + 7 of the depth bucket

inline bool use_u16_keys(int tile_bits) { return tile_bits <= 16; }

// Level 1: the (supertile, Gaussian) entries and their sort by supertile.
struct SortWs {
    void *keys_a, *keys_b;  // supertile keys (u16 or u32)
    uint32_t *vals_tmp;
    uint2 *rects_tmp;       // packed tile rectangle of each entry (payload of the sort)
    void *pass_ws;  // histogram table + digit totals of each pass
    size_t bytes;
};

inline SortWs carve_sort(Carve &c, int64_t m, int super_bits) {
    SortWs w;
    const int64_t kb = use_u16_keys(super_bits) ? 2 : 4;
    w.keys_a = c.take<char>(m * kb);
    w.keys_b = c.take<char>(m * kb);
    w.vals_tmp = c.take<uint32_t>(m);
    w.rects_tmp = c.take<uint2>(m);
    w.pass_ws = c.take<char>((int64_t)radix_workspace_bytes<kTileItems>(m));
    w.bytes = 0;
    return w;
}

// Geometry of the tile and supertile grids.
struct Grid {
    int tiles_x, tiles_y, n_tiles;
    int super_x, super_y, n_super, super_bits;
};

inline bool make_grid(int32_t width, int32_t height, int32_t tile_size, Grid &g) {
    const int64_t tx = (width + (int64_t)tile_size - 1) / tile_size;
    const int64_t ty = (height + (int64_t)tile_size - 1) / tile_size;
    if (tx * ty > 0x7fffffffLL) return false;
    g.tiles_x = (int)tx;
    g.tiles_y = (int)ty;
    g.n_tiles = (int)(tx * ty);
    g.super_x = (int)((tx + kSuper - 1) / kSuper);
    g.super_y = (int)((ty + kSuper - 1) / kSuper);
    g.n_super = g.super_x * g.super_y;
    int b = 0;
    while (b < 31 && ((int64_t)(g.n_super - 1) >> b) != 0) ++b;
    g.super_bits = b;
    return true;
}

inline int64_t l2_blocks_bound(int64_t m, int n_super) {
    return (m + kL2Threads - 1) / kL2Threads + n_super;
}


struct BinWs {
    SortWs lvl1;            // general level 1 (more than kRadixMax supertiles)
    int32_t *super_off;     // n_super (+1 spare)
    int32_t *super_ids;     // m
    uint2 *super_rects;     // m: packed tile rectangle of each super_ids entry
    uint32_t *chunk_start;  // n_super + 1: first level-2 block of each supertile
    uint4 *block_map;       // level-2 block -> (supertile, first and end list position, 0)
    uint32_t *table;        // level-2 blocks x 64 local tiles
    uint32_t *tile_counts;  // entries per tile
    void *scan_ws;          // tile-count scan of grids above kFusedTileScanMax tiles
    size_t bytes;
};

inline BinWs carve_bins(void *base, int64_t n, int64_t m, const Grid &g) {
    Carve c{reinterpret_cast<char *>(base)};
    BinWs w{};
    (void)n;
    if (g.n_super > kRadixMax) w.lvl1 = carve_sort(c, m, g.super_bits);
    w.super_off = c.take<int32_t>((int64_t)g.n_super + 1);
    w.super_ids = c.take<int32_t>(m);
    w.super_rects = c.take<uint2>(m);
    w.chunk_start = c.take<uint32_t>((int64_t)g.n_super + 1);
    w.block_map = c.take<uint4>(l2_blocks_bound(m, g.n_super));
    w.table = c.take<uint32_t>(l2_blocks_bound(m, g.n_super) * kSuperLocal);
    w.tile_counts = c.take<uint32_t>(g.n_tiles);
    w.scan_ws = c.take<char>((int64_t)scan_workspace_bytes<uint32_t>(g.n_tiles));
    w.bytes = align256(c.off);
    return w;
}

inline int bits_for(int64_t max_value) {
    int b = 0;
    while (b < 63 && (max_value >> b) != 0) ++b;
    return b;
}

// Level 1: the (supertile, Gaussian) entries in depth order, stably sorted by
// supertile id; writes the per-supertile list starts and the sorted ids.
template <typename KeyT>
int super_sort(const EmitArgs &a, const SortWs &w, int super_bits, int n_super,
               int32_t *super_off, int32_t *super_ids, uint2 *super_rects, hipStream_t stream) {
    const SortPlan plan = plan_sort(super_bits);
    const int P = plan.passes;
    KeyT *ka = reinterpret_cast<KeyT *>(w.keys_a), *kb = reinterpret_cast<KeyT *>(w.keys_b);
    uint32_t *out = reinterpret_cast<uint32_t *>(super_ids);
    // pass p writes (kb, out, super_rects) when P-1-p is even, (ka, vals_tmp,
    // rects_tmp) otherwise; the entries (pass -1) go to the other set than pass 0.
    // Each entry carries its Gaussian's packed tile rectangle, so that level 2
    // reads it in list order.
    auto keys_for = [&](int p) { return ((P - 1 - p) % 2 == 0) ? kb : ka; };
    auto vals_for = [&](int p) { return ((P - 1 - p) % 2 == 0) ? out : w.vals_tmp; };
    auto rects_for = [&](int p) { return ((P - 1 - p) % 2 == 0) ? super_rects : w.rects_tmp; };
    hipLaunchKernelGGL(emit_super_kernel<KeyT>, dim3(ceil_div(a.n, 256)), dim3(256), 0, stream,
                       a.n, a.k, a.order, a.offsets, a.rects, a.tiles_x, keys_for(-1),
                       vals_for(-1), rects_for(-1));
    int st = launch_status();
    if (st) return st;
    for (int p = 0; p < P; ++p) {
        PassExtras x;
        x.pin = rects_for(p - 1);
        x.pout = rects_for(p);
        st = radix_pass<KeyT, kTileItems, true>(keys_for(p - 1), vals_for(p - 1), keys_for(p),
                                                vals_for(p), a.k, p * plan.bits_per_pass,
                                                pass_bits(plan, super_bits, p), true, w.pass_ws,
                                                stream, x);
        if (st) return st;
    }
    hipLaunchKernelGGL(tile_ranges_kernel<KeyT>, dim3(ceil_div(n_super, 256)), dim3(256), 0,
                       stream, n_super, kb, a.k, super_off);
    return launch_status();
}

}  // namespace gs

using namespace gs;

extern "C" int gs_bin_count_workspace_size(int64_t n, size_t *bytes) {
    if (n < 0 || !bytes) return GS_ERR_INVALID_ARGUMENT;
    *bytes = carve_count(nullptr, n).bytes;
    return GS_OK;
}

namespace gs {

// Arguments shared by the two phases of gs_bin_count.
struct CountCall {
    const float *points_image, *radii, *depths;
    const uint8_t *mask;
    int64_t n;
    int32_t width, height, tile_size;
    void *workspace;
    size_t workspace_bytes;
    int64_t *totals;
    // depth hint {kmin, shift} for the bucket transform (hint_shift < 0: none,
    // the transform comes from the keys' least and greatest value); with
    // totals4, totals has 4 entries: K, M, least and greatest key with tiles
    uint32_t hint_kmin = 0;
    int hint_shift = -1;
    bool totals4 = false;
};

int check_count_call(const CountCall &c, CountWs &w) {
    if (c.n < 0 || c.width <= 0 || c.height <= 0 || c.tile_size <= 0 || !c.totals)
        return GS_ERR_INVALID_ARGUMENT;
    if (c.n > 0x7fffffffLL) return GS_ERR_INVALID_ARGUMENT;  // Gaussian ids are int32
    w = carve_count(c.workspace, c.n);
    if (c.n > 0 && (!c.workspace || c.workspace_bytes < w.bytes))
        return GS_ERR_WORKSPACE_TOO_SMALL;
    if (c.n > 0 && (!c.points_image || !c.radii || !c.depths || !c.mask))
        return GS_ERR_INVALID_ARGUMENT;
    if (c.hint_shift > 16) return GS_ERR_INVALID_ARGUMENT;  // 16 bucket bits of 32
    return GS_OK;
}

// Up to kRadixMax supertiles level 1 enumerates the entries from the depth
// order directly (counted as the segment sort emits it, scattered by
// l1_scatter_kernel), reading the tile rectangles written in depth order; otherwise it places them with the supertile
// counts' exclusive scan in depth order, also written by the last pass.
bool one_pass_level1(const CountCall &c, Grid &grid) {
    return make_grid(c.width, c.height, c.tile_size, grid) && grid.n_super <= kRadixMax;
}

// Depth pass p of 2 over the bucket bits: (a) -> (b) -> (a).  The first pass
// takes the histogram depth_upsweep0_kernel (or, with a depth hint,
// count_tiles_kernel) wrote, numbers the values itself, drops the Gaussians
// without tiles and reduces count_tiles' sums (K, M, the n_live Gaussians with
// tiles and, for a caller's four totals, the least and greatest key); the
// second sorts the n_live keys.
int depth_pass(const CountCall &c, const CountWs &w, int p, hipStream_t stream) {
    PassExtras x;
    x.xform = w.xform;
    if (p == 0) {
        x.hist_ready = true;
        x.drop_no_tiles = true;
        x.block_sums = w.block_sums;
        x.block_minmax = c.totals4 ? w.block_minmax : nullptr;
        x.sums_out = c.totals;
        x.sums_dev = w.dev_totals;
        x.live_out = w.n_live;
    } else {
        x.n_live = w.n_live;
    }
    const bool from_a = p == 0;
    return radix_pass<uint32_t, kDepthItems>(
        from_a ? w.dkeys_a : w.dkeys_b, p == 0 ? nullptr : w.dvals_b,
        from_a ? w.dkeys_b : w.dkeys_a, from_a ? w.dvals_b : w.dvals_a, c.n, kDepthPassShift[p],
        kRadixMaxBits, true, w.sort_ws, stream, x);
}

// The four totals of no Gaussians: no keys, no entries, no least or greatest key.
__global__ __launch_bounds__(kWave) void empty_totals_kernel(int64_t *__restrict__ totals) {
    if (threadIdx.x < 4) totals[threadIdx.x] = threadIdx.x == 2 ? 0xFFFFFFFFLL : 0;
}

// Phase 1: tile rectangles, depth keys, the first depth pass; totals are final.
int bin_count_begin(const CountCall &c, hipStream_t stream) {
    CountWs w;
    int st = check_count_call(c, w);
    if (st) return st;
    if (c.n == 0) {
        if (!c.totals4) return zero_bytes(c.totals, 2 * sizeof(int64_t), stream);
        hipLaunchKernelGGL(empty_totals_kernel, dim3(1), dim3(kWave), 0, stream, c.totals);
        return launch_status();
    }
    const int nblocks = (int)sort_blocks<kDepthItems>(c.n);
    uint32_t *hist = reinterpret_cast<uint32_t *>(w.sort_ws);
    const bool hinted = c.hint_shift >= 0;
    // with a depth hint the count kernel writes the transform and the first
    // pass's histogram itself; otherwise the upsweep derives the transform from
    // the keys' least and greatest value
    // the one-pass level 1 adds its counts into a table the count kernel zeroes
    // (its rows of the grid's supertiles: the level-1 scan reads no others)
    Grid grid;
    const bool one_pass_l1 = one_pass_level1(c, grid);
    hipLaunchKernelGGL((count_tiles_kernel<kDepthItems>), dim3(nblocks), dim3(kSortThreads), 0,
                       stream, c.n, c.points_image, c.radii, c.depths, c.mask, c.width, c.height,
                       c.tile_size, w.rects, w.dkeys_a, w.block_sums, w.block_minmax,
                       c.hint_kmin, hinted ? c.hint_shift : 0, hinted ? hist : nullptr, w.xform,
                       one_pass_l1 ? w.l1_hist : nullptr,
                       one_pass_l1 ? (int64_t)grid.n_super * l1_blocks(c.n) : (int64_t)0);
    st = launch_status();
    if (st) return st;
    if (!hinted) {
        hipLaunchKernelGGL((depth_upsweep0_kernel<kDepthItems>), dim3(nblocks),
                           dim3(kSortThreads), 0, stream, (const uint32_t *)w.dkeys_a, c.n,
                           (const uint32_t *)w.block_minmax, nblocks, nblocks, hist, w.xform);
        st = launch_status();
        if (st) return st;
    }
    return depth_pass(c, w, 0, stream);
}

// Phase 2: the second depth pass and the segment sort, then the one-pass level
// 1's counts and positions (they need neither K nor M) or the general level 1's
// entry offsets.
int bin_count_finish(const CountCall &c, hipStream_t stream) {
    CountWs w;
    int st = check_count_call(c, w);
    if (st || c.n == 0) return st;
    Grid grid;
    const bool one_pass_l1 = one_pass_level1(c, grid);
    st = depth_pass(c, w, 1, stream);
    if (st) return st;
    SegArgs sa;
    sa.keys = w.dkeys_a;
    sa.vals = w.dvals_a;
    sa.keys_b = w.dkeys_b;
    sa.vals_b = w.dvals_b;
    sa.keys_c = w.dkeys_c;
    sa.n_live = w.n_live;
    sa.xform = w.xform;
    sa.n = c.n;
    sa.rects = w.rects;
    sa.counts_out = one_pass_l1 ? nullptr : w.counts;
    sa.rects_out = one_pass_l1 ? w.rects_depth : nullptr;
    // the one-pass level 1's (supertile, block) counts, added as the positions are
    // emitted into the table count_tiles_kernel zeroed
    sa.l1_hist = one_pass_l1 ? w.l1_hist : nullptr;
    sa.super_x = grid.super_x;
    sa.l1_nblocks = (int)l1_blocks(c.n);
    hipLaunchKernelGGL(segment_sort_kernel, dim3(ceil_div(c.n, kSegChunk)), dim3(kSegThreads), 0,
                       stream, sa);
    st = launch_status();
    if (st) return st;
    if (one_pass_l1) {
        const L1Args la = l1_args(w, c.n, 0, grid.super_x);
        hipLaunchKernelGGL(digit_scan_kernel, dim3(grid.n_super), dim3(kScanThreads), 0, stream,
                           w.l1_hist, la.nblocks, w.l1_totals, nullptr, nullptr, 0, nullptr,
                           nullptr, nullptr);
        return launch_status();
    }
    // supertile entry offsets in depth order (the total equals count_tiles' M; it
    // goes to the workspace: totals is not written after the first phase, so a
    // caller may keep it in host memory and read it once that phase has run)
    return scan_exclusive<uint64_t>(w.counts, w.offsets, c.n, w.m_scan, w.scan_ws, stream);
}

}  // namespace gs


extern "C" int gs_bin_count(const float *points_image, const float *radii, const float *depths,
                            const uint8_t *mask, int64_t n, int32_t width, int32_t height,
                            int32_t tile_size, void *workspace, size_t workspace_bytes,
                            int64_t *totals, hipStream_t stream) {
    const CountCall c{points_image, radii, depths, mask, n, width, height, tile_size, workspace,
                      workspace_bytes, totals};
    const int st = bin_count_begin(c, stream);
    return st ? st : bin_count_finish(c, stream);
}

extern "C" int gs_bin_count_begin(const float *points_image, const float *radii,
                                  const float *depths, const uint8_t *mask, int64_t n,
                                  int32_t width, int32_t height, int32_t tile_size,
                                  void *workspace, size_t workspace_bytes, int64_t *totals,
                                  hipStream_t stream) {
    const CountCall c{points_image, radii, depths, mask, n, width, height, tile_size, workspace,
                      workspace_bytes, totals};
    return bin_count_begin(c, stream);
}

extern "C" int gs_bin_count_begin_hinted(const float *points_image, const float *radii,
                                         const float *depths, const uint8_t *mask, int64_t n,
                                         int32_t width, int32_t height, int32_t tile_size,
                                         void *workspace, size_t workspace_bytes,
                                         uint32_t hint_kmin, int32_t hint_shift,
                                         int64_t *totals, hipStream_t stream) {
    CountCall c{points_image, radii, depths, mask, n, width, height, tile_size, workspace,
                workspace_bytes, totals};
    c.hint_kmin = hint_kmin;
    c.hint_shift = hint_shift < 0 ? -1 : hint_shift;
    c.totals4 = true;
    return bin_count_begin(c, stream);
}

extern "C" int gs_bin_count_finish(const float *points_image, const float *radii,
                                   const float *depths, const uint8_t *mask, int64_t n,
                                   int32_t width, int32_t height, int32_t tile_size,
                                   void *workspace, size_t workspace_bytes, int64_t *totals,
                                   hipStream_t stream) {
    const CountCall c{points_image, radii, depths, mask, n, width, height, tile_size, workspace,
                      workspace_bytes, totals};
    return bin_count_finish(c, stream);
}

extern "C" int gs_bin_sort_workspace_size(int64_t n, int64_t k, int64_t m, int32_t width,
                                          int32_t height, int32_t tile_size, size_t *bytes) {
    (void)k;
    Grid g;
    if (n < 0 || m < 0 || width <= 0 || height <= 0 || tile_size <= 0 || !bytes ||
        !make_grid(width, height, tile_size, g))
        return GS_ERR_INVALID_ARGUMENT;
    *bytes = carve_bins(nullptr, n, m, g).bytes;
    return GS_OK;
}

namespace gs {

// Identity order of each range (band order): the launch order when K = 0.
__global__ __launch_bounds__(256) void iota_kernel(int n, int32_t *__restrict__ out) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) out[i] = i;
}

int bin_sort(const float *points_image, const float *radii, const float *depths, int64_t n,
             int32_t width, int32_t height, int32_t tile_size, int64_t k, int64_t m,
             const void *count_workspace, void *workspace, size_t workspace_bytes,
             int32_t *indexing_offset, int32_t *gaussian_ids_sorted, uint64_t *sorted_keys,
             int32_t *tiles_touched, int32_t *launch_order, hipStream_t stream,
             bool capped = false) {
    if (n < 0 || k < 0 || m < 0 || (!capped && m > k) || width <= 0 || height <= 0 ||
        tile_size <= 0)
        return GS_ERR_INVALID_ARGUMENT;
    if (k > 0x7fffffffLL) return GS_ERR_TOO_MANY_KEYS;
    Grid g;
    if (!make_grid(width, height, tile_size, g)) return GS_ERR_INVALID_ARGUMENT;
    if (!indexing_offset) return GS_ERR_INVALID_ARGUMENT;
    if (g.tiles_x > 65535 || g.tiles_y > 65535)
        return GS_ERR_UNSUPPORTED;  // tile rectangles are staged with 16-bit coordinates
    if ((k == 0) != (m == 0)) return GS_ERR_INVALID_ARGUMENT;
    // the capped sort takes K and M from the count workspace on the device: one-pass
    // level 1 and the tile scan inside l2_prefix_kernel only (grids of at most 256
    // supertiles), no debug outputs
    if (capped && (g.n_super > kRadixMax || g.n_tiles > kFusedTileScanMax || k == 0 ||
                   sorted_keys || tiles_touched))
        return GS_ERR_UNSUPPORTED;
    if (l2_blocks_bound(m, g.n_super) > 0x7fffffffLL) return GS_ERR_TOO_MANY_KEYS;
    const CountWs cw = carve_count(const_cast<void *>(count_workspace), n);
    const BinWs w = carve_bins(workspace, n, m, g);
    if (m > 0 && (!workspace || workspace_bytes < w.bytes)) return GS_ERR_WORKSPACE_TOO_SMALL;
    if (n > 0 && !count_workspace) return GS_ERR_INVALID_ARGUMENT;
    int st;
    if (tiles_touched && n > 0) {
        hipLaunchKernelGGL(tiles_from_rects_kernel, dim3(ceil_div(n, 256)), dim3(256), 0, stream,
                           n, (const uint2 *)cw.rects, tiles_touched);
        st = launch_status();
        if (st) return st;
    }
    if (k == 0) {
        if (launch_order) {
            hipLaunchKernelGGL(iota_kernel, dim3(ceil_div(g.n_tiles, 256)), dim3(256), 0, stream,
                               g.n_tiles, launch_order);
            st = launch_status();
            if (st) return st;
        }
        return zero_bytes(indexing_offset, sizeof(int32_t) * (size_t)g.n_tiles, stream);
    }
    if (!points_image || !radii || !gaussian_ids_sorted || (sorted_keys && !depths) || n == 0)
        return GS_ERR_INVALID_ARGUMENT;

    // level-2 blocks the grids cover: a bound on the chunks of the supertile lists
    const int64_t nb2 = l2_blocks_bound(m, g.n_super);
    // level 1: (supertile, Gaussian) entries in depth order, stably sorted by supertile
    if (g.n_super <= kRadixMax) {  // counts and positions came from gs_bin_count
        L1Args la = l1_args(cw, n, m, g.super_x);
        la.cap_totals = capped ? cw.dev_totals : nullptr;
        hipLaunchKernelGGL(l1_scatter_kernel, dim3(la.nblocks), dim3(kL1Threads), 0, stream, la,
                           (const uint32_t *)cw.l1_hist, (const uint32_t *)cw.l1_totals,
                           g.n_super, w.super_ids, w.super_rects, w.super_off, w.chunk_start,
                           w.block_map, nb2, g.n_tiles, w.tile_counts);
        st = launch_status();
    } else {  // emitted entries sorted by supertile over several radix passes
        EmitArgs a;
        a.rects = cw.rects;
        a.order = cw.dvals_a;  // depth order (even number of depth passes)
        a.offsets = cw.offsets;
        a.n = n;
        a.k = m;
        a.tiles_x = g.super_x;
        st = use_u16_keys(g.super_bits)
                 ? super_sort<uint16_t>(a, w.lvl1, g.super_bits, g.n_super, w.super_off,
                                        w.super_ids, w.super_rects, stream)
                 : super_sort<uint32_t>(a, w.lvl1, g.super_bits, g.n_super, w.super_off,
                                        w.super_ids, w.super_rects, stream);
        if (st) return st;
        // level-2 block plan (the one-pass level 1 writes it itself)
        hipLaunchKernelGGL(l2_plan_kernel, dim3(1), dim3(kPlanThreads), 0, stream, g.n_super, m,
                           w.super_off, w.chunk_start, w.block_map, nb2, g.n_tiles,
                           w.tile_counts);
        st = launch_status();
    }
    if (st) return st;

    // level 2: per-tile counts, tile offsets and block prefixes, scatter
    L2Args l2;
    l2.super_off = w.super_off;
    l2.super_ids = w.super_ids;
    l2.chunk_start = w.chunk_start;
    l2.block_map = w.block_map;
    l2.super_rects = w.super_rects;
    l2.n = n;
    l2.m = m;
    l2.k = k;
    l2.n_super = g.n_super;
    l2.super_x = g.super_x;
    l2.tiles_x = g.tiles_x;
    l2.tiles_y = g.tiles_y;
    l2.width = width;
    l2.height = height;
    l2.tile_size = tile_size;
    l2.nblocks = nb2;
    l2.cap_totals = capped ? cw.dev_totals : nullptr;
    hipLaunchKernelGGL(l2_count_kernel, dim3((unsigned)nb2), dim3(kL2Threads), 0, stream, l2,
                       w.table, w.tile_counts);
    st = launch_status();
    if (st) return st;
    const bool fused_scan = g.n_tiles <= kFusedTileScanMax;
    if (!fused_scan) {
        st = scan_exclusive<uint32_t>(w.tile_counts, reinterpret_cast<uint32_t *>(indexing_offset),
                                      g.n_tiles, (uint32_t *)nullptr, w.scan_ws, stream);
        if (st) return st;
    }
    hipLaunchKernelGGL(l2_prefix_kernel, dim3(g.n_super), dim3(kL2Threads), 0, stream, l2,
                       w.tile_counts, g.n_tiles, fused_scan ? 1 : 0, indexing_offset, w.table);
    st = launch_status();
    if (st) return st;
    const unsigned grid2 = (unsigned)nb2 + (launch_order ? kBinXcds : 0);
    if (k < (1LL << 30))
        hipLaunchKernelGGL(l2_scatter_kernel<true>, dim3(grid2), dim3(kL2Threads), 0, stream, l2,
                           w.table, gaussian_ids_sorted, indexing_offset, launch_order);
    else
        hipLaunchKernelGGL(l2_scatter_kernel<false>, dim3(grid2), dim3(kL2Threads), 0, stream, l2,
                           w.table, gaussian_ids_sorted, indexing_offset, launch_order);
    st = launch_status();
    if (st) return st;
    if (sorted_keys) {
        hipLaunchKernelGGL(keys_from_offsets_kernel, dim3(ceil_div(k, 256)), dim3(256), 0, stream,
                           k, n, g.n_tiles, indexing_offset, gaussian_ids_sorted, depths,
                           sorted_keys);
        st = launch_status();
    }
    return st;
}

}  // namespace gs

extern "C" int gs_bin_sort(const float *points_image, const float *radii, const float *depths,
                           int64_t n, int32_t width, int32_t height, int32_t tile_size,
                           int64_t k, int64_t m, const void *count_workspace, void *workspace,
                           size_t workspace_bytes, int32_t *indexing_offset,
                           int32_t *gaussian_ids_sorted, uint64_t *sorted_keys,
                           int32_t *tiles_touched, hipStream_t stream) {
    return gs::bin_sort(points_image, radii, depths, n, width, height, tile_size, k, m,
                        count_workspace, workspace, workspace_bytes, indexing_offset,
                        gaussian_ids_sorted, sorted_keys, tiles_touched, nullptr, stream);
}

extern "C" int gs_bin_sort_capped(const float *points_image, const float *radii,
                                  const float *depths, int64_t n, int32_t width, int32_t height,
                                  int32_t tile_size, int64_t k_capacity, int64_t m_capacity,
                                  const void *count_workspace, void *workspace,
                                  size_t workspace_bytes, int32_t *indexing_offset,
                                  int32_t *gaussian_ids_sorted, int32_t *launch_order,
                                  hipStream_t stream) {
    if (!launch_order || !count_workspace) return GS_ERR_INVALID_ARGUMENT;
    return gs::bin_sort(points_image, radii, depths, n, width, height, tile_size, k_capacity,
                        m_capacity, count_workspace, workspace, workspace_bytes, indexing_offset,
                        gaussian_ids_sorted, nullptr, nullptr, launch_order, stream, true);
}

extern "C" int gs_bin_sort_ordered(const float *points_image, const float *radii,
                                   const float *depths, int64_t n, int32_t width, int32_t height,
                                   int32_t tile_size, int64_t k, int64_t m,
                                   const void *count_workspace, void *workspace,
                                   size_t workspace_bytes, int32_t *indexing_offset,
                                   int32_t *gaussian_ids_sorted, uint64_t *sorted_keys,
                                   int32_t *tiles_touched, int32_t *launch_order,
                                   hipStream_t stream) {
    if (!launch_order) return GS_ERR_INVALID_ARGUMENT;
    return gs::bin_sort(points_image, radii, depths, n, width, height, tile_size, k, m,
                        count_workspace, workspace, workspace_bytes, indexing_offset,
                        gaussian_ids_sorted, sorted_keys, tiles_touched, launch_order, stream);
}
