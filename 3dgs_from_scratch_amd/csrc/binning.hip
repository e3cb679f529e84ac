// Binning: per-Gaussian tile counts, device scans, LSD radix sort and tile ranges.
//
// The reference (src/cuda/rasterizer.cpp:292-359, src/cuda/kernel.cu:784-914,
// 1341-1388) emits one 64-bit key (tile_id << 32 | depth_bits) per touched tile
// in Gaussian order and stably sorts all 64 bits.  The same order -- (tile,
// depth bits, Gaussian index) -- is produced here with far less sort traffic:
//   1. a stable sort of the N per-Gaussian depth keys (32 bits, N entries),
//   2. the (tile, Gaussian) entries of the Gaussians in that depth order,
//   3. a stable sort of those K entries by tile id (ceil(log2(n_tiles)) bits).
// A stable sort by tile of a sequence already ordered by (depth, index) is
// ordered by (tile, depth, index).
//
// Radix sort: reduce-then-scan LSD passes of <= 8 bits.  A pass is
//   upsweep   per-block digit histogram (wave64 ballot matching, one LDS atomic
//             per distinct digit per wave),
//   scan      exclusive scan of the digit-major histogram table,
//   downsweep stable local ranks from the same ballot matching, a scatter into
//             LDS in digit order, and contiguous runs written to HBM.
// No pass waits on another workgroup, so no launch can deadlock.
//
// The K entries of step 2 are never written unsorted: the first tile pass
// generates each block's 4096 entries on the fly from the depth-ordered
// Gaussians (per-block first Gaussian + a search in LDS), once to build the
// histogram and once to scatter.  Tile ids are stored as 16-bit keys whenever
// n_tiles <= 65536.

#include "wave_ops.h"
#include "preprocess_math.h"

namespace gs {

constexpr int kSortThreads = 256;
constexpr int kSortWaves = kSortThreads / kWave;
constexpr int kRadixMaxBits = 8;
constexpr int kRadixMax = 1 << kRadixMaxBits;
constexpr int kEmitItems = 16;  // entries per thread in the fused first tile pass
constexpr int kEmitTile = kSortThreads * kEmitItems;
constexpr int kDepthItems = 16;  // keys per thread in the depth sort (N-sized)
constexpr int kTileItems = 16;  // keys per thread in later tile passes (K-sized)

constexpr int kScanThreads = 256;
constexpr int kScanItems = 16;
constexpr int kScanTile = kScanThreads * kScanItems;
constexpr int kDirectMaxBlocks = 256;  // passes with <= 256 blocks skip the histogram scan

inline size_t align256(size_t x) { return (x + 255) / 256 * 256; }

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

struct SortLds {
    uint32_t wave_count[kSortWaves][kRadixMax];
    uint32_t global_start[kRadixMax];
    uint32_t local_start[kRadixMax];
    uint32_t skeys[kEmitTile];
    uint32_t svals[kEmitTile];
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
                                                   int nbits, uint32_t *counts) {
    const uint32_t dmask = (1u << nbits) - 1u;
#pragma unroll
    for (int it = 0; it < ITEMS; ++it) {
        const uint32_t d = digit_of(k[it], shift, dmask);
        const uint64_t active = __ballot(valid[it]);
        const uint64_t peers = match_digit(d, nbits, active);
        if (valid[it] && (peers & lanemask_lt()) == 0)
            atomicAdd(&counts[d], (uint32_t)__popcll(peers));
    }
}

// Per-pass histogram tables.  Digit-major (d * nblocks + b) is scanned into
// first output slots by scan_exclusive; block-major (b * radix + d) is summed
// directly by every downsweep block when the pass has <= kDirectMaxBlocks blocks.
template <bool DIRECT>
__device__ __forceinline__ int64_t hist_index(int d, int b, int nblocks, int radix) {
    return DIRECT ? (int64_t)b * radix + d : (int64_t)d * nblocks + b;
}

// Stable rank of the block's keys (registers) by digit, staged through LDS in
// digit order and written to keys_out/vals_out.  `table` is the scanned
// digit-major histogram (first output slot of (digit, block)) or, for DIRECT,
// the raw block-major histogram from which the slots are summed here.  When
// counts_out is set, counts_out[dst] = touched[value] is written as well.
template <typename KeyT, int ITEMS, bool DIRECT>
__device__ __forceinline__ void block_scatter(const uint32_t (&k)[ITEMS],
                                              const uint32_t (&v)[ITEMS],
                                              const bool (&valid)[ITEMS], int shift, int nbits,
                                              int nblocks, const uint32_t *__restrict__ table,
                                              KeyT *__restrict__ keys_out,
                                              uint32_t *__restrict__ vals_out, int64_t n,
                                              bool write_keys, SortLds &s,
                                              const uint32_t *__restrict__ touched = nullptr,
                                              uint64_t *__restrict__ counts_out = nullptr) {
    const int radix = 1 << nbits;
    const uint32_t dmask = (uint32_t)radix - 1u;
    const int wave = threadIdx.x / kWave;
    for (int d = threadIdx.x; d < radix; d += kSortThreads) {
#pragma unroll
        for (int w = 0; w < kSortWaves; ++w) s.wave_count[w][d] = 0;
        if (!DIRECT) s.global_start[d] = table[hist_index<false>(d, blockIdx.x, nblocks, radix)];
    }
    if (DIRECT) {
        uint32_t before = 0, total = 0;
        if ((int)threadIdx.x < radix) {
            // 16 independent loads in flight per round (the rows are L2 resident)
            for (int b0 = 0; b0 < nblocks; b0 += 16) {
                uint32_t h[16];
#pragma unroll
                for (int q = 0; q < 16; ++q)
                    h[q] = b0 + q < nblocks
                               ? table[hist_index<true>(threadIdx.x, b0 + q, nblocks, radix)]
                               : 0u;
#pragma unroll
                for (int q = 0; q < 16; ++q) {
                    total += h[q];
                    before += b0 + q < (int)blockIdx.x ? h[q] : 0u;
                }
            }
        }
        uint32_t grand;
        const uint32_t base =
            block_exclusive_scan<uint32_t, kSortThreads>(total, s.scan_tmp, grand);
        if ((int)threadIdx.x < radix) s.global_start[threadIdx.x] = base + before;
    }
    __syncthreads();
    uint32_t rank[ITEMS];
#pragma unroll
    for (int it = 0; it < ITEMS; ++it) {
        const uint32_t d = digit_of(k[it], shift, dmask);
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
            const uint32_t d = digit_of(k[it], shift, dmask);
            const uint32_t p = s.local_start[d] + s.wave_count[wave][d] + rank[it];
            s.skeys[p] = k[it];
            s.svals[p] = v[it];
        }
    }
    __syncthreads();
    for (uint32_t p = threadIdx.x; p < block_count; p += kSortThreads) {
        const uint32_t key = s.skeys[p];
        const uint32_t d = digit_of(key, shift, dmask);
        const uint32_t dst = s.global_start[d] + (p - s.local_start[d]);
        if (dst < (uint64_t)n) {  // always true for a consistent histogram; guards the store
            const uint32_t val = s.svals[p];
            if (write_keys) keys_out[dst] = (KeyT)key;
            vals_out[dst] = val;
            if (counts_out) counts_out[dst] = val < (uint64_t)n ? touched[val] : 0u;
        }
    }
}

// hist[d * nblocks + block] = number of keys of this block with digit d.
template <typename KeyT, int ITEMS, bool DIRECT>
__global__ __launch_bounds__(kSortThreads) void radix_upsweep_kernel(
    const KeyT *__restrict__ keys, int64_t n, int shift, int nbits, int nblocks,
    uint32_t *__restrict__ hist) {
    __shared__ uint32_t counts[kRadixMax];
    const int radix = 1 << nbits;
    for (int d = threadIdx.x; d < radix; d += kSortThreads) counts[d] = 0;
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
    block_count_digits<ITEMS>(k, valid, shift, nbits, counts);
    __syncthreads();
    for (int d = threadIdx.x; d < radix; d += kSortThreads)
        hist[hist_index<DIRECT>(d, blockIdx.x, nblocks, radix)] = counts[d];
}

template <typename KeyT, int ITEMS, bool DIRECT>
__global__ __launch_bounds__(kSortThreads) void radix_downsweep_kernel(
    const KeyT *__restrict__ keys_in, const uint32_t *__restrict__ vals_in,
    KeyT *__restrict__ keys_out, uint32_t *__restrict__ vals_out, int64_t n, int shift,
    int nbits, int nblocks, const uint32_t *__restrict__ table, int write_keys,
    const uint32_t *__restrict__ touched, uint64_t *__restrict__ counts_out) {
    __shared__ SortLds s;
    const int64_t base = (int64_t)blockIdx.x * (kSortThreads * ITEMS);
    uint32_t k[ITEMS], v[ITEMS];
    bool valid[ITEMS];
#pragma unroll
    for (int it = 0; it < ITEMS; ++it) {
        const int64_t i = base + slot_index<ITEMS>(it);
        valid[it] = i < n;
        k[it] = valid[it] ? (uint32_t)keys_in[i] : 0u;
        v[it] = valid[it] ? vals_in[i] : 0u;
    }
    block_scatter<KeyT, ITEMS, DIRECT>(k, v, valid, shift, nbits, nblocks, table, keys_out,
                                       vals_out, n, write_keys != 0, s, touched, counts_out);
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

template <int ITEMS>
size_t radix_workspace_bytes(int64_t n) {
    const int64_t entries = sort_blocks<ITEMS>(n) * kRadixMax;
    return align256(entries * sizeof(uint32_t)) + scan_workspace_bytes<uint32_t>(entries);
}

// One LSD pass from arrays.  With hist_ready the histogram table of this pass
// (layout by `direct`) was already written into ws by the caller.  With
// counts_out, counts_out[dst] = touched[value] is written next to the values.
template <typename KeyT, int ITEMS>
int radix_pass(const KeyT *kin, const uint32_t *vin, KeyT *kout, uint32_t *vout, int64_t n,
               int shift, int nbits, bool write_keys, void *ws, hipStream_t stream,
               bool hist_ready = false, const uint32_t *touched = nullptr,
               uint64_t *counts_out = nullptr) {
    const int nblocks = (int)sort_blocks<ITEMS>(n);
    const bool direct = nblocks <= kDirectMaxBlocks;
    const int64_t entries = (int64_t)nblocks * kRadixMax;
    uint32_t *hist = reinterpret_cast<uint32_t *>(ws);
    void *scan_ws = reinterpret_cast<char *>(ws) + align256(entries * sizeof(uint32_t));
    int st;
    if (!hist_ready) {
        if (direct)
            hipLaunchKernelGGL((radix_upsweep_kernel<KeyT, ITEMS, true>), dim3(nblocks),
                               dim3(kSortThreads), 0, stream, kin, n, shift, nbits, nblocks, hist);
        else
            hipLaunchKernelGGL((radix_upsweep_kernel<KeyT, ITEMS, false>), dim3(nblocks),
                               dim3(kSortThreads), 0, stream, kin, n, shift, nbits, nblocks, hist);
        st = launch_status();
        if (st) return st;
    }
    if (direct) {
        hipLaunchKernelGGL((radix_downsweep_kernel<KeyT, ITEMS, true>), dim3(nblocks),
                           dim3(kSortThreads), 0, stream, kin, vin, kout, vout, n, shift, nbits,
                           nblocks, hist, write_keys ? 1 : 0, touched, counts_out);
        return launch_status();
    }
    st = scan_exclusive<uint32_t>(hist, hist, (int64_t)nblocks << nbits, (uint32_t *)nullptr,
                                  scan_ws, stream);
    if (st) return st;
    hipLaunchKernelGGL((radix_downsweep_kernel<KeyT, ITEMS, false>), dim3(nblocks),
                       dim3(kSortThreads), 0, stream, kin, vin, kout, vout, n, shift, nbits,
                       nblocks, hist, write_keys ? 1 : 0, touched, counts_out);
    return launch_status();
}

// ------------------------------------------------------------- binning

// tiles_touched and depth sort keys per Gaussian (src/cuda/kernel.cu:784-818),
// fused with the histogram of the first depth-sort pass.  Gaussians without
// tiles get the key 0xFFFFFFFF (sorted last; they emit nothing).
template <int ITEMS, bool DIRECT>
__global__ __launch_bounds__(kSortThreads) void count_tiles_kernel(
    int64_t n, const float *__restrict__ points_image, const float *__restrict__ radii,
    const float *__restrict__ depths, const uint8_t *__restrict__ mask, int width, int height,
    int tile_size, uint32_t *__restrict__ touched, uint32_t *__restrict__ depth_keys,
    uint32_t *__restrict__ ids, int nbits, int nblocks, uint32_t *__restrict__ hist) {
    __shared__ uint32_t counts[kRadixMax];
    const int radix = 1 << nbits;
    for (int d = threadIdx.x; d < radix; d += kSortThreads) counts[d] = 0;
    const int64_t base = (int64_t)blockIdx.x * (kSortThreads * ITEMS);
    uint32_t k[ITEMS];
    bool valid[ITEMS];
#pragma unroll
    for (int it = 0; it < ITEMS; ++it) {
        const int64_t i = base + slot_index<ITEMS>(it);
        valid[it] = i < n;
        k[it] = 0u;
        if (!valid[it]) continue;
        uint32_t cnt = 0;
        if (mask[i]) {
            TileRect r;
            if (tile_rect(points_image[2 * i], points_image[2 * i + 1], radii[2 * i],
                          radii[2 * i + 1], width, height, tile_size, r))
                cnt = (uint32_t)((r.tx1 - r.tx0 + 1) * (r.ty1 - r.ty0 + 1));
        }
        k[it] = cnt ? __float_as_uint(depths[i]) : 0xFFFFFFFFu;
        touched[i] = cnt;
        depth_keys[i] = k[it];
        ids[i] = (uint32_t)i;
    }
    __syncthreads();
    block_count_digits<ITEMS>(k, valid, 0, nbits, counts);
    __syncthreads();
    for (int d = threadIdx.x; d < radix; d += kSortThreads)
        hist[hist_index<DIRECT>(d, blockIdx.x, nblocks, radix)] = counts[d];
}

// block_first[b] = depth-order position of the Gaussian whose entries contain
// entry b * kEmitTile (entries are laid out Gaussian after Gaussian), and
// block_first[ceil(k / kEmitTile)] = the last Gaussian with entries.
__global__ __launch_bounds__(256) void block_first_kernel(int64_t n, int64_t k,
                                                          const uint32_t *__restrict__ order,
                                                          const uint64_t *__restrict__ offsets,
                                                          const uint32_t *__restrict__ touched,
                                                          uint32_t *__restrict__ block_first) {
    const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= n) return;
    const uint32_t g = order[r];
    const uint64_t c = g < (uint64_t)n ? touched[g] : 0u;
    if (c == 0) return;
    const uint64_t off = offsets[r];
    const uint64_t end = off + c < (uint64_t)k ? off + c : (uint64_t)k;
    for (uint64_t b = (off + kEmitTile - 1) / kEmitTile; b * kEmitTile < end; ++b)
        block_first[b] = (uint32_t)r;
    if (off < (uint64_t)k && end == (uint64_t)k)
        block_first[((uint64_t)k + kEmitTile - 1) / kEmitTile] = (uint32_t)r;
}

struct EmitArgs {
    const uint32_t *order;    // Gaussians in depth order
    const uint64_t *offsets;  // first entry of each depth-ordered Gaussian
    const uint32_t *touched;  // tiles per Gaussian (by Gaussian id)
    const uint32_t *block_first;
    const float *points;
    const float *radii;
    int64_t n, k;
    int width, height, tile_size, tiles_x;
};

constexpr int kEmitGroup = 1024;  // depth-ordered Gaussians staged per round (4 per thread)

struct EmitLds {
    int32_t off[kEmitGroup];  // first entry relative to the block start (clamped)
    int32_t end[kEmitGroup];
    uint32_t gid[kEmitGroup];
    uint32_t origin[kEmitGroup];  // tx0 | ty0 << 16 of the tile rectangle
    uint16_t nx[kEmitGroup];      // rectangle width in tiles
};

// Writes the entries [b*kEmitTile, (b+1)*kEmitTile) of the depth-ordered
// (tile, Gaussian) sequence -- entry o of Gaussian r is its o-th tile in
// row-major order -- to keys_out / vals_out, and the block's histogram of the
// low `nbits` tile bits (the first sort pass) to hist.  The block's Gaussians
// block_first[b] .. block_first[b + 1] are staged up to 1024 per round; each
// wave then writes the entries of every 4th staged Gaussian lane-parallel
// (coalesced runs) and counts digits with LDS atomics.
template <typename KeyT, bool DIRECT>
__global__ __launch_bounds__(kSortThreads) void emit_entries_kernel(
    EmitArgs a, int nbits, int nblocks, uint32_t *__restrict__ hist, KeyT *__restrict__ keys_out,
    uint32_t *__restrict__ vals_out) {
    __shared__ EmitLds e;
    __shared__ uint32_t counts[kRadixMax];
    const int radix = 1 << nbits;
    const uint32_t dmask = (uint32_t)radix - 1u;
    for (int d = threadIdx.x; d < radix; d += kSortThreads) counts[d] = 0;
    const int64_t block_base = (int64_t)blockIdx.x * kEmitTile;
    const int64_t left = a.k - block_base;
    const int count = (int)(left < kEmitTile ? left : kEmitTile);
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    KeyT *kout = keys_out + block_base;
    uint32_t *vout = vals_out + block_base;
    int64_t r0 = a.block_first[blockIdx.x];
    const int64_t r_last = a.block_first[blockIdx.x + 1];  // inclusive
    for (;;) {
#pragma unroll
        for (int q = 0; q < kEmitGroup / kSortThreads; ++q) {
            const int j = threadIdx.x + q * kSortThreads;
            const int64_t r = r0 + j;
            int32_t off = 0x7fffffff, end = 0x7fffffff;
            if (r <= r_last && r < a.n) {
                const uint32_t g = a.order[r];
                const uint32_t c = g < (uint64_t)a.n ? a.touched[g] : 0u;
                int64_t o = (int64_t)a.offsets[r] - block_base;
                int64_t oe = o + (int64_t)c;
                o = o > 0x3fffffff ? 0x3fffffff : o;
                oe = oe > 0x3fffffff ? 0x3fffffff : oe;
                off = (int32_t)o;
                end = (int32_t)oe;
                TileRect rect{0, 0, 0, 0};
                if (c > 0)
                    tile_rect(a.points[2 * g], a.points[2 * g + 1], a.radii[2 * g],
                              a.radii[2 * g + 1], a.width, a.height, a.tile_size, rect);
                e.gid[j] = g;
                e.origin[j] = (uint32_t)rect.tx0 | ((uint32_t)rect.ty0 << 16);
                e.nx[j] = (uint16_t)(rect.tx1 - rect.tx0 + 1);
            }
            e.off[j] = off;
            e.end[j] = end;
        }
        __syncthreads();
        for (int j = wave; j < kEmitGroup; j += kSortWaves) {
            const int32_t goff = e.off[j];
            if (goff >= count) break;  // later Gaussians start even later
            const int32_t lo = goff > 0 ? goff : 0;
            const int32_t hi = e.end[j] < count ? e.end[j] : count;
            const int32_t nx = e.nx[j] > 0 ? (int32_t)e.nx[j] : 1;
            const uint32_t origin = e.origin[j];
            const int32_t tx0 = (int32_t)(origin & 0xffffu), ty0 = (int32_t)(origin >> 16);
            const uint32_t g = e.gid[j];
            // row = floor((local + 0.5) / nx): the true quotient is at least 0.5/nx away
            // from an integer and the float error is below that for local < 2^22
            const float rcp = 1.0f / (float)nx;
            for (int32_t idx = lo + lane; idx < hi; idx += kWave) {
                const int32_t local = idx - goff;
                const int32_t row = (int32_t)(((float)local + 0.5f) * rcp);
                const int32_t col = local - row * nx;
                const uint32_t t = (uint32_t)((ty0 + row) * a.tiles_x + tx0 + col);
                kout[idx] = (KeyT)t;
                vout[idx] = g;
                atomicAdd(&counts[t & dmask], 1u);
            }
        }
        const bool more = r0 + kEmitGroup <= r_last;
        __syncthreads();
        if (!more) break;
        r0 += kEmitGroup;
    }
    for (int d = threadIdx.x; d < radix; d += kSortThreads)
        hist[hist_index<DIRECT>(d, blockIdx.x, nblocks, radix)] = counts[d];
}

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

template <typename KeyT>
__global__ __launch_bounds__(256) void sorted_keys_kernel(int64_t k, int64_t n,
                                                          const KeyT *__restrict__ tiles,
                                                          const int32_t *__restrict__ ids,
                                                          const float *__restrict__ depths,
                                                          uint64_t *__restrict__ keys) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= k) return;
    const int32_t g = ids[i];
    const uint32_t bits = (g >= 0 && g < n) ? __float_as_uint(depths[g]) : 0u;
    keys[i] = ((uint64_t)(uint32_t)tiles[i] << 32) | (uint64_t)bits;
}

__global__ __launch_bounds__(256) void copy_u32_to_i32_kernel(int64_t n,
                                                              const uint32_t *__restrict__ in,
                                                              int32_t *__restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = (int32_t)in[i];
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

struct CountWs {
    uint32_t *touched, *dkeys_a, *dvals_a, *dkeys_b, *dvals_b;
    uint64_t *counts, *offsets;
    void *sort_ws, *scan_ws;
    size_t bytes;
};

inline CountWs carve_count(void *base, int64_t n) {
    Carve c{reinterpret_cast<char *>(base)};
    CountWs w;
    w.touched = c.take<uint32_t>(n);
    w.dkeys_a = c.take<uint32_t>(n);
    w.dvals_a = c.take<uint32_t>(n);
    w.dkeys_b = c.take<uint32_t>(n);
    w.dvals_b = c.take<uint32_t>(n);
    w.counts = c.take<uint64_t>(n);
    w.offsets = c.take<uint64_t>(n + 1);
    w.sort_ws = c.take<char>((int64_t)radix_workspace_bytes<kDepthItems>(n));
    w.scan_ws = c.take<char>((int64_t)scan_workspace_bytes<uint64_t>(n));
    w.bytes = align256(c.off);
    return w;
}

// The depth sort is 4 passes of 8 bits, so its result ends in the (a) buffers.
constexpr int kDepthBits = 32;

inline bool use_u16_keys(int tile_bits) { return tile_bits <= 16; }

struct SortWs {
    void *keys_a, *keys_b;  // tile keys (u16 or u32)
    uint32_t *vals_tmp;
    uint32_t *block_first;
    void *pass_ws;  // histogram table + scan scratch of each pass
    size_t bytes;
};

inline SortWs carve_sort(void *base, int64_t k, int tile_bits) {
    Carve c{reinterpret_cast<char *>(base)};
    SortWs w;
    const int64_t kb = use_u16_keys(tile_bits) ? 2 : 4;
    w.keys_a = c.take<char>(k * kb);
    w.keys_b = c.take<char>(k * kb);
    w.vals_tmp = c.take<uint32_t>(k);
    w.block_first = c.take<uint32_t>((k + kEmitTile - 1) / kEmitTile + 1);
    w.pass_ws = c.take<char>((int64_t)radix_workspace_bytes<kTileItems>(k));
    w.bytes = align256(c.off);
    return w;
}

inline int bits_for(int64_t max_value) {
    int b = 0;
    while (b < 63 && (max_value >> b) != 0) ++b;
    return b;
}

// Entry generation (with the first pass's histogram), then the sort passes;
// the last pass writes the caller's gaussian_ids_sorted and the sorted keys
// end in keys_b.
template <typename KeyT>
int tile_sort(const EmitArgs &a, const SortWs &w, int tile_bits, int n_tiles,
              int32_t *indexing_offset, int32_t *ids_out, uint64_t *sorted_keys,
              const float *depths, hipStream_t stream) {
    static_assert(kEmitTile == kSortThreads * kTileItems, "entry blocks must be sort blocks");
    const SortPlan plan = plan_sort(tile_bits);
    const int P = plan.passes;
    const int nblocks = (int)sort_blocks<kTileItems>(a.k);
    const bool direct = nblocks <= kDirectMaxBlocks;
    KeyT *ka = reinterpret_cast<KeyT *>(w.keys_a), *kb = reinterpret_cast<KeyT *>(w.keys_b);
    uint32_t *out = reinterpret_cast<uint32_t *>(ids_out);
    // pass p writes (kb, out) when P-1-p is even, (ka, vals_tmp) otherwise; the
    // entries (pass -1) go to the other set than pass 0
    auto keys_for = [&](int p) { return ((P - 1 - p) % 2 == 0) ? kb : ka; };
    auto vals_for = [&](int p) { return ((P - 1 - p) % 2 == 0) ? out : w.vals_tmp; };

    hipLaunchKernelGGL(block_first_kernel, dim3(ceil_div(a.n, 256)), dim3(256), 0, stream, a.n,
                       a.k, a.order, a.offsets, a.touched, w.block_first);
    int st = launch_status();
    if (st) return st;
    uint32_t *hist = reinterpret_cast<uint32_t *>(w.pass_ws);
    const int nb0 = pass_bits(plan, tile_bits, 0);
    if (direct)
        hipLaunchKernelGGL((emit_entries_kernel<KeyT, true>), dim3(nblocks), dim3(kSortThreads), 0,
                           stream, a, nb0, nblocks, hist, keys_for(-1), vals_for(-1));
    else
        hipLaunchKernelGGL((emit_entries_kernel<KeyT, false>), dim3(nblocks), dim3(kSortThreads),
                           0, stream, a, nb0, nblocks, hist, keys_for(-1), vals_for(-1));
    st = launch_status();
    if (st) return st;
    for (int p = 0; p < P; ++p) {
        st = radix_pass<KeyT, kTileItems>(keys_for(p - 1), vals_for(p - 1), keys_for(p),
                                          vals_for(p), a.k, p * plan.bits_per_pass,
                                          pass_bits(plan, tile_bits, p), true, w.pass_ws, stream,
                                          p == 0);
        if (st) return st;
    }
    hipLaunchKernelGGL(tile_ranges_kernel<KeyT>, dim3(ceil_div(n_tiles, 256)), dim3(256), 0,
                       stream, n_tiles, kb, a.k, indexing_offset);
    st = launch_status();
    if (st) return st;
    if (sorted_keys) {
        hipLaunchKernelGGL(sorted_keys_kernel<KeyT>, dim3(ceil_div(a.k, 256)), dim3(256), 0,
                           stream, a.k, a.n, kb, ids_out, depths, sorted_keys);
        st = launch_status();
    }
    return st;
}

}  // namespace gs

using namespace gs;

extern "C" int gs_bin_count_workspace_size(int64_t n, size_t *bytes) {
    if (n < 0 || !bytes) return GS_ERR_INVALID_ARGUMENT;
    *bytes = carve_count(nullptr, n).bytes;
    return GS_OK;
}

extern "C" int gs_bin_count(const float *points_image, const float *radii, const float *depths,
                            const uint8_t *mask, int64_t n, int32_t width, int32_t height,
                            int32_t tile_size, void *workspace, size_t workspace_bytes,
                            int64_t *total_keys, hipStream_t stream) {
    if (n < 0 || width <= 0 || height <= 0 || tile_size <= 0 || !total_keys)
        return GS_ERR_INVALID_ARGUMENT;
    if (n > 0x7fffffffLL) return GS_ERR_INVALID_ARGUMENT;  // Gaussian ids are int32
    const CountWs w = carve_count(workspace, n);
    if (n > 0 && (!workspace || workspace_bytes < w.bytes)) return GS_ERR_WORKSPACE_TOO_SMALL;
    if (n == 0) return zero_bytes(total_keys, sizeof(int64_t), stream);
    if (!points_image || !radii || !depths || !mask) return GS_ERR_INVALID_ARGUMENT;
    const SortPlan plan = plan_sort(kDepthBits);
    const int nblocks = (int)sort_blocks<kDepthItems>(n);
    const int nb0 = pass_bits(plan, kDepthBits, 0);
    uint32_t *hist = reinterpret_cast<uint32_t *>(w.sort_ws);
    if (nblocks <= kDirectMaxBlocks)
        hipLaunchKernelGGL((count_tiles_kernel<kDepthItems, true>), dim3(nblocks),
                           dim3(kSortThreads), 0, stream, n, points_image, radii, depths, mask,
                           width, height, tile_size, w.touched, w.dkeys_a, w.dvals_a, nb0,
                           nblocks, hist);
    else
        hipLaunchKernelGGL((count_tiles_kernel<kDepthItems, false>), dim3(nblocks),
                           dim3(kSortThreads), 0, stream, n, points_image, radii, depths, mask,
                           width, height, tile_size, w.touched, w.dkeys_a, w.dvals_a, nb0,
                           nblocks, hist);
    int st = launch_status();
    if (st) return st;
    // 4 passes of 8 bits: (a) -> (b) -> (a) -> (b) -> (a); the last pass writes no
    // keys but the tile counts in depth order
    for (int p = 0; p < plan.passes; ++p) {
        const bool from_a = (p % 2) == 0;
        const bool last = p + 1 == plan.passes;
        st = radix_pass<uint32_t, kDepthItems>(
            from_a ? w.dkeys_a : w.dkeys_b, from_a ? w.dvals_a : w.dvals_b,
            from_a ? w.dkeys_b : w.dkeys_a, from_a ? w.dvals_b : w.dvals_a, n,
            p * plan.bits_per_pass, pass_bits(plan, kDepthBits, p), !last, w.sort_ws, stream,
            p == 0, last ? w.touched : nullptr, last ? w.counts : nullptr);
        if (st) return st;
    }
    return scan_exclusive<uint64_t>(w.counts, w.offsets, n,
                                    reinterpret_cast<uint64_t *>(total_keys), w.scan_ws, stream);
}

static int tile_bits_of(int32_t width, int32_t height, int32_t tile_size, int *n_tiles) {
    const int64_t tx = (width + tile_size - 1) / tile_size;
    const int64_t ty = (height + tile_size - 1) / tile_size;
    if (tx * ty > 0x7fffffffLL) return -1;
    *n_tiles = (int)(tx * ty);
    return bits_for((int64_t)*n_tiles - 1);
}

extern "C" int gs_bin_sort_workspace_size(int64_t n, int64_t k, int32_t n_tiles, size_t *bytes) {
    (void)n;
    if (k < 0 || n_tiles < 0 || !bytes) return GS_ERR_INVALID_ARGUMENT;
    *bytes = carve_sort(nullptr, k, bits_for((int64_t)n_tiles - 1)).bytes;
    return GS_OK;
}

extern "C" int gs_bin_sort(const float *points_image, const float *radii, const float *depths,
                           int64_t n, int32_t width, int32_t height, int32_t tile_size,
                           int64_t k, const void *count_workspace, void *workspace,
                           size_t workspace_bytes, int32_t *indexing_offset,
                           int32_t *gaussian_ids_sorted, uint64_t *sorted_keys,
                           int32_t *tiles_touched, hipStream_t stream) {
    if (n < 0 || k < 0 || width <= 0 || height <= 0 || tile_size <= 0)
        return GS_ERR_INVALID_ARGUMENT;
    if (k > 0x7fffffffLL) return GS_ERR_TOO_MANY_KEYS;
    int n_tiles = 0;
    const int tile_bits = tile_bits_of(width, height, tile_size, &n_tiles);
    if (tile_bits < 0) return GS_ERR_INVALID_ARGUMENT;
    if (!indexing_offset) return GS_ERR_INVALID_ARGUMENT;
    if ((width + tile_size - 1) / tile_size > 65535 || (height + tile_size - 1) / tile_size > 65535)
        return GS_ERR_UNSUPPORTED;  // tile rectangles are staged with 16-bit coordinates
    const CountWs cw = carve_count(const_cast<void *>(count_workspace), n);
    const SortWs w = carve_sort(workspace, k, tile_bits);
    if (k > 0 && (!workspace || workspace_bytes < w.bytes)) return GS_ERR_WORKSPACE_TOO_SMALL;
    if (n > 0 && !count_workspace) return GS_ERR_INVALID_ARGUMENT;
    if (tiles_touched && n > 0) {
        hipLaunchKernelGGL(copy_u32_to_i32_kernel, dim3(ceil_div(n, 256)), dim3(256), 0, stream,
                           n, cw.touched, tiles_touched);
        int st = launch_status();
        if (st) return st;
    }
    if (k == 0) return zero_bytes(indexing_offset, sizeof(int32_t) * (size_t)n_tiles, stream);
    if (!points_image || !radii || !gaussian_ids_sorted || (sorted_keys && !depths) || n == 0)
        return GS_ERR_INVALID_ARGUMENT;
    EmitArgs a;
    a.order = cw.dvals_a;  // depth order (even number of depth passes)
    a.offsets = cw.offsets;
    a.touched = cw.touched;
    a.block_first = w.block_first;
    a.points = points_image;
    a.radii = radii;
    a.n = n;
    a.k = k;
    a.width = width;
    a.height = height;
    a.tile_size = tile_size;
    a.tiles_x = (width + tile_size - 1) / tile_size;
    if (use_u16_keys(tile_bits))
        return tile_sort<uint16_t>(a, w, tile_bits, n_tiles, indexing_offset, gaussian_ids_sorted,
                                   sorted_keys, depths, stream);
    return tile_sort<uint32_t>(a, w, tile_bits, n_tiles, indexing_offset, gaussian_ids_sorted,
                               sorted_keys, depths, stream);
}
