// Binning: per-Gaussian tile counts, device scans, LSD radix sort and tile ranges.
//
// The reference (src/cuda/rasterizer.cpp:292-359, src/cuda/kernel.cu:784-914,
// 1341-1388) emits one 64-bit key (tile_id << 32 | depth_bits) per touched tile
// in Gaussian order and stably sorts all 64 bits.  The same order -- (tile,
// depth bits, Gaussian index) -- is produced here with far less sort traffic:
//   1. a stable sort of the N per-Gaussian depth keys (32 bits, N entries),
//   2. key emission in that depth order (tile id only, K entries),
//   3. a stable sort of the K tile ids over ceil(log2(n_tiles)) bits.
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

#include "wave_ops.h"
#include "preprocess_math.h"

namespace gs {

constexpr int kSortThreads = 256;
constexpr int kSortItems = 16;
constexpr int kSortTile = kSortThreads * kSortItems;  // keys per workgroup per pass
constexpr int kSortWaves = kSortThreads / kWave;
constexpr int kRadixMaxBits = 8;
constexpr int kRadixMax = 1 << kRadixMaxBits;

constexpr int kScanThreads = 256;
constexpr int kScanItems = 16;
constexpr int kScanTile = kScanThreads * kScanItems;

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

// Exclusive scan of kScanTile consecutive elements per workgroup, offset by
// `offsets[blockIdx.x]` (or 0 when offsets is null).  In-place safe.  The last
// workgroup writes the grand total to *total when total is not null.
template <typename T>
__global__ __launch_bounds__(kScanThreads) void scan_apply_kernel(
    const T *in, T *out, int64_t n, const T *__restrict__ offsets, T *__restrict__ total) {
    __shared__ T tmp[kScanThreads / kWave + 1];
    const int64_t base = (int64_t)blockIdx.x * kScanTile + (int64_t)threadIdx.x * kScanItems;
    T v[kScanItems];
    T acc = 0;
#pragma unroll
    for (int it = 0; it < kScanItems; ++it) {
        const int64_t i = base + it;
        v[it] = i < n ? in[i] : (T)0;
        acc += v[it];
    }
    T block_total;
    T run = block_exclusive_scan<T, kScanThreads>(acc, tmp, block_total);
    const T off = offsets ? offsets[blockIdx.x] : (T)0;
    run += off;
#pragma unroll
    for (int it = 0; it < kScanItems; ++it) {
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
        bytes += ((nb * sizeof(T) + 255) / 256) * 256;
        n = nb;
    }
    return bytes;
}

// Exclusive scan of n elements (out may alias in).  Writes the total to
// *total (device pointer) when not null.
template <typename T>
int scan_exclusive(const T *in, T *out, int64_t n, T *total, void *ws, hipStream_t stream) {
    if (n <= 0) {
        return total ? zero_bytes(total, sizeof(T), stream) : GS_OK;
    }
    const int64_t nb = (n + kScanTile - 1) / kScanTile;
    if (nb == 1) {
        hipLaunchKernelGGL(scan_apply_kernel<T>, dim3(1), dim3(kScanThreads), 0, stream, in, out,
                           n, (const T *)nullptr, total);
        return launch_status();
    }
    T *sums = reinterpret_cast<T *>(ws);
    void *ws_next = reinterpret_cast<char *>(ws) + ((nb * sizeof(T) + 255) / 256) * 256;
    hipLaunchKernelGGL(scan_reduce_kernel<T>, dim3(nb), dim3(kScanThreads), 0, stream, in, n,
                       sums);
    int st = launch_status();
    if (st) return st;
    st = scan_exclusive<T>(sums, sums, nb, (T *)nullptr, ws_next, stream);
    if (st) return st;
    hipLaunchKernelGGL(scan_apply_kernel<T>, dim3(nb), dim3(kScanThreads), 0, stream, in, out, n,
                       (const T *)sums, total);
    return launch_status();
}

// ------------------------------------------------------------ radix sort

__device__ __forceinline__ uint32_t digit_of(uint32_t key, int shift, uint32_t dmask) {
    return (key >> shift) & dmask;
}

// hist[d * nblocks + block] = number of keys of this block with digit d.
__global__ __launch_bounds__(kSortThreads) void radix_upsweep_kernel(
    const uint32_t *__restrict__ keys, int64_t n, int shift, int nbits, int nblocks,
    uint32_t *__restrict__ hist) {
    __shared__ uint32_t counts[kRadixMax];
    const int radix = 1 << nbits;
    const uint32_t dmask = (uint32_t)radix - 1u;
    for (int d = threadIdx.x; d < radix; d += kSortThreads) counts[d] = 0;
    __syncthreads();
    const int wave = threadIdx.x / kWave;
    const int lane = __lane_id();
    const int64_t base = (int64_t)blockIdx.x * kSortTile + (int64_t)wave * (kSortTile / kSortWaves);
    for (int it = 0; it < kSortItems; ++it) {
        const int64_t i = base + it * kWave + lane;
        const bool valid = i < n;
        const uint32_t d = valid ? digit_of(keys[i], shift, dmask) : 0u;
        const uint64_t active = __ballot(valid);
        const uint64_t peers = match_digit(d, nbits, active);
        if (valid && (peers & lanemask_lt()) == 0) atomicAdd(&counts[d], (uint32_t)__popcll(peers));
    }
    __syncthreads();
    for (int d = threadIdx.x; d < radix; d += kSortThreads)
        hist[(int64_t)d * nblocks + blockIdx.x] = counts[d];
}

// Stable scatter of one pass.  `offsets` is the exclusive scan of the
// histogram table (digit-major), i.e. the first output slot of (digit, block).
__global__ __launch_bounds__(kSortThreads) void radix_downsweep_kernel(
    const uint32_t *__restrict__ keys_in, const uint32_t *__restrict__ vals_in,
    uint32_t *__restrict__ keys_out, uint32_t *__restrict__ vals_out, int64_t n, int shift,
    int nbits, int nblocks, const uint32_t *__restrict__ offsets) {
    __shared__ uint32_t wave_count[kSortWaves][kRadixMax];
    __shared__ uint32_t global_start[kRadixMax];
    __shared__ uint32_t local_start[kRadixMax];
    __shared__ uint32_t skeys[kSortTile];
    __shared__ uint32_t svals[kSortTile];
    __shared__ uint32_t scan_tmp[kSortThreads / kWave + 1];

    const int radix = 1 << nbits;
    const uint32_t dmask = (uint32_t)radix - 1u;
    const int wave = threadIdx.x / kWave;
    const int lane = __lane_id();
    for (int d = threadIdx.x; d < radix; d += kSortThreads) {
#pragma unroll
        for (int w = 0; w < kSortWaves; ++w) wave_count[w][d] = 0;
        global_start[d] = offsets[(int64_t)d * nblocks + blockIdx.x];
    }
    __syncthreads();

    const int64_t block_base = (int64_t)blockIdx.x * kSortTile;
    const int64_t base = block_base + (int64_t)wave * (kSortTile / kSortWaves);
    uint32_t k[kSortItems], v[kSortItems], rank[kSortItems];
#pragma unroll
    for (int it = 0; it < kSortItems; ++it) {
        const int64_t i = base + it * kWave + lane;
        const bool valid = i < n;
        k[it] = valid ? keys_in[i] : 0u;
        v[it] = valid ? vals_in[i] : 0u;
    }
#pragma unroll
    for (int it = 0; it < kSortItems; ++it) {
        const int64_t i = base + it * kWave + lane;
        const bool valid = i < n;
        const uint32_t d = digit_of(k[it], shift, dmask);
        const uint64_t active = __ballot(valid);
        const uint64_t peers = match_digit(d, nbits, active);
        const uint32_t before = valid ? wave_count[wave][d] : 0u;
        const uint32_t r = (uint32_t)__popcll(peers & lanemask_lt());
        if (valid && r == 0) wave_count[wave][d] = before + (uint32_t)__popcll(peers);
        rank[it] = before + r;
    }
    __syncthreads();

    // per-digit exclusive prefix over the waves, then over the digits
    uint32_t digit_total = 0;
    if (threadIdx.x < radix) {
#pragma unroll
        for (int w = 0; w < kSortWaves; ++w) {
            const uint32_t c = wave_count[w][threadIdx.x];
            wave_count[w][threadIdx.x] = digit_total;
            digit_total += c;
        }
    }
    uint32_t block_count;
    const uint32_t ls = block_exclusive_scan<uint32_t, kSortThreads>(digit_total, scan_tmp,
                                                                      block_count);
    if (threadIdx.x < radix) local_start[threadIdx.x] = ls;
    __syncthreads();

#pragma unroll
    for (int it = 0; it < kSortItems; ++it) {
        const int64_t i = base + it * kWave + lane;
        if (i < n) {
            const uint32_t d = digit_of(k[it], shift, dmask);
            const uint32_t p = local_start[d] + wave_count[wave][d] + rank[it];
            skeys[p] = k[it];
            svals[p] = v[it];
        }
    }
    __syncthreads();

    for (uint32_t p = threadIdx.x; p < block_count; p += kSortThreads) {
        const uint32_t key = skeys[p];
        const uint32_t d = digit_of(key, shift, dmask);
        const uint32_t dst = global_start[d] + (p - local_start[d]);
        if (dst < (uint64_t)n) {  // always true for a consistent histogram; guards the store
            keys_out[dst] = key;
            vals_out[dst] = svals[p];
        }
    }
}

struct SortPlan {
    int passes;
    int bits_per_pass;
};

inline SortPlan plan_sort(int total_bits) {
    SortPlan p;
    if (total_bits <= 0) {
        p.passes = 0;
        p.bits_per_pass = 0;
        return p;
    }
    p.passes = (total_bits + kRadixMaxBits - 1) / kRadixMaxBits;
    p.bits_per_pass = (total_bits + p.passes - 1) / p.passes;
    return p;
}

inline size_t align256(size_t x) { return (x + 255) / 256 * 256; }

size_t radix_sort_workspace_bytes(int64_t n) {
    const int64_t nblocks = (n + kSortTile - 1) / kSortTile;
    const int64_t entries = nblocks * kRadixMax;
    return align256(entries * sizeof(uint32_t)) + scan_workspace_bytes<uint32_t>(entries);
}

// Stable LSD sort of (keys, vals) by the low total_bits bits of the keys.
// Ping-pongs between (ka, va) and (kb, vb); the result ends in (ka, va) when
// the pass count is even and in (kb, vb) when odd (*result_in_b says which).
int radix_sort_pairs(uint32_t *ka, uint32_t *va, uint32_t *kb, uint32_t *vb, int64_t n,
                     int total_bits, void *ws, bool *result_in_b, hipStream_t stream) {
    const SortPlan plan = plan_sort(total_bits);
    *result_in_b = (plan.passes % 2) == 1;
    if (n <= 1 || plan.passes == 0) {
        if (*result_in_b && n > 0) {  // keep the documented result location
            hipError_t e = hipMemcpyAsync(kb, ka, n * sizeof(uint32_t), hipMemcpyDeviceToDevice,
                                          stream);
            if (e == hipSuccess)
                e = hipMemcpyAsync(vb, va, n * sizeof(uint32_t), hipMemcpyDeviceToDevice, stream);
            if (e != hipSuccess) return (int)e;
        }
        return GS_OK;
    }
    const int nblocks = (int)((n + kSortTile - 1) / kSortTile);
    const int64_t entries = (int64_t)nblocks * kRadixMax;
    uint32_t *hist = reinterpret_cast<uint32_t *>(ws);
    void *scan_ws = reinterpret_cast<char *>(ws) + align256(entries * sizeof(uint32_t));
    for (int p = 0; p < plan.passes; ++p) {
        const int shift = p * plan.bits_per_pass;
        const int nbits = (total_bits - shift) < plan.bits_per_pass ? (total_bits - shift)
                                                                     : plan.bits_per_pass;
        const bool from_a = (p % 2) == 0;
        uint32_t *kin = from_a ? ka : kb, *vin = from_a ? va : vb;
        uint32_t *kout = from_a ? kb : ka, *vout = from_a ? vb : va;
        hipLaunchKernelGGL(radix_upsweep_kernel, dim3(nblocks), dim3(kSortThreads), 0, stream,
                           kin, n, shift, nbits, nblocks, hist);
        int st = launch_status();
        if (st) return st;
        const int64_t used = (int64_t)nblocks << nbits;
        st = scan_exclusive<uint32_t>(hist, hist, used, (uint32_t *)nullptr, scan_ws, stream);
        if (st) return st;
        hipLaunchKernelGGL(radix_downsweep_kernel, dim3(nblocks), dim3(kSortThreads), 0, stream,
                           kin, vin, kout, vout, n, shift, nbits, nblocks, hist);
        st = launch_status();
        if (st) return st;
    }
    return GS_OK;
}

// ------------------------------------------------------------- binning

// tiles_touched and depth sort keys per Gaussian (src/cuda/kernel.cu:784-818).
// Gaussians without tiles get the key 0xFFFFFFFF (sorted last; they emit nothing).
__global__ __launch_bounds__(256) void count_tiles_kernel(
    int64_t n, const float *__restrict__ points_image, const float *__restrict__ radii,
    const float *__restrict__ depths, const uint8_t *__restrict__ mask, int width, int height,
    int tile_size, uint32_t *__restrict__ touched, uint32_t *__restrict__ depth_keys,
    uint32_t *__restrict__ ids) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    uint32_t cnt = 0;
    if (mask[i]) {
        TileRect r;
        if (tile_rect(points_image[2 * i], points_image[2 * i + 1], radii[2 * i],
                      radii[2 * i + 1], width, height, tile_size, r))
            cnt = (uint32_t)((r.tx1 - r.tx0 + 1) * (r.ty1 - r.ty0 + 1));
    }
    touched[i] = cnt;
    depth_keys[i] = cnt ? __float_as_uint(depths[i]) : 0xFFFFFFFFu;
    ids[i] = (uint32_t)i;
}

__global__ __launch_bounds__(256) void gather_counts_kernel(int64_t n,
                                                            const uint32_t *__restrict__ order,
                                                            const uint32_t *__restrict__ touched,
                                                            uint64_t *__restrict__ counts) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint32_t g = order[i];
    counts[i] = g < (uint64_t)n ? touched[g] : 0u;
}

// One thread per Gaussian in depth order; writes its tiles row-major.
__global__ __launch_bounds__(256) void emit_keys_kernel(
    int64_t n, int64_t k, const uint32_t *__restrict__ order, const uint64_t *__restrict__ offsets,
    const uint32_t *__restrict__ touched, const float *__restrict__ points_image,
    const float *__restrict__ radii, int width, int height, int tile_size, int tiles_x,
    uint32_t *__restrict__ tile_keys, uint32_t *__restrict__ gauss_ids) {
    const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= n) return;
    const uint32_t g = order[r];
    if (g >= (uint64_t)n || touched[g] == 0) return;
    TileRect rect;
    if (!tile_rect(points_image[2 * g], points_image[2 * g + 1], radii[2 * g], radii[2 * g + 1],
                   width, height, tile_size, rect))
        return;
    uint64_t o = offsets[r];
    const uint64_t o_end = o + touched[g];
    for (int ty = rect.ty0; ty <= rect.ty1; ++ty)
        for (int tx = rect.tx0; tx <= rect.tx1; ++tx) {
            if (o >= o_end || o >= (uint64_t)k) return;  // guards the stores
            tile_keys[o] = (uint32_t)(ty * tiles_x + tx);
            gauss_ids[o] = g;
            ++o;
        }
}

// indexing_offset[t] = first sorted position whose tile is >= t.
__global__ __launch_bounds__(256) void tile_ranges_kernel(int n_tiles,
                                                          const uint32_t *__restrict__ tiles,
                                                          int64_t k,
                                                          int32_t *__restrict__ offsets) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n_tiles) return;
    int64_t lo = 0, hi = k;
    while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        if (tiles[mid] < (uint32_t)t)
            lo = mid + 1;
        else
            hi = mid;
    }
    offsets[t] = (int32_t)lo;
}

__global__ __launch_bounds__(256) void sorted_keys_kernel(int64_t k, int64_t n,
                                                          const uint32_t *__restrict__ tiles,
                                                          const int32_t *__restrict__ ids,
                                                          const float *__restrict__ depths,
                                                          uint64_t *__restrict__ keys) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= k) return;
    const int32_t g = ids[i];
    const uint32_t bits = (g >= 0 && g < n) ? __float_as_uint(depths[g]) : 0u;
    keys[i] = ((uint64_t)tiles[i] << 32) | (uint64_t)bits;
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
    w.sort_ws = c.take<char>((int64_t)radix_sort_workspace_bytes(n));
    w.scan_ws = c.take<char>((int64_t)scan_workspace_bytes<uint64_t>(n));
    w.bytes = align256(c.off);
    return w;
}

struct SortWs {
    uint32_t *tkeys_a, *tkeys_b, *tvals_tmp;
    void *sort_ws;
    size_t bytes;
};

inline SortWs carve_sort(void *base, int64_t k) {
    Carve c{reinterpret_cast<char *>(base)};
    SortWs w;
    w.tkeys_a = c.take<uint32_t>(k);
    w.tkeys_b = c.take<uint32_t>(k);
    w.tvals_tmp = c.take<uint32_t>(k);
    w.sort_ws = c.take<char>((int64_t)radix_sort_workspace_bytes(k));
    w.bytes = align256(c.off);
    return w;
}

inline int bits_for(int64_t max_value) {
    int b = 0;
    while (b < 63 && (max_value >> b) != 0) ++b;
    return b;
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
    if (n == 0) {
        return zero_bytes(total_keys, sizeof(int64_t), stream);
    }
    if (!points_image || !radii || !depths || !mask) return GS_ERR_INVALID_ARGUMENT;
    const int grid = ceil_div(n, 256);
    hipLaunchKernelGGL(count_tiles_kernel, dim3(grid), dim3(256), 0, stream, n, points_image,
                       radii, depths, mask, width, height, tile_size, w.touched, w.dkeys_a,
                       w.dvals_a);
    int st = launch_status();
    if (st) return st;
    bool in_b = false;
    st = radix_sort_pairs(w.dkeys_a, w.dvals_a, w.dkeys_b, w.dvals_b, n, 32, w.sort_ws, &in_b,
                          stream);
    if (st) return st;
    const uint32_t *order = in_b ? w.dvals_b : w.dvals_a;
    hipLaunchKernelGGL(gather_counts_kernel, dim3(grid), dim3(256), 0, stream, n, order,
                       w.touched, w.counts);
    st = launch_status();
    if (st) return st;
    return scan_exclusive<uint64_t>(w.counts, w.offsets, n,
                                    reinterpret_cast<uint64_t *>(total_keys), w.scan_ws, stream);
}

extern "C" int gs_bin_sort_workspace_size(int64_t n, int64_t k, int32_t n_tiles, size_t *bytes) {
    (void)n;
    (void)n_tiles;
    if (k < 0 || !bytes) return GS_ERR_INVALID_ARGUMENT;
    *bytes = carve_sort(nullptr, k).bytes;
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
    const int tiles_x = (width + tile_size - 1) / tile_size;
    const int tiles_y = (height + tile_size - 1) / tile_size;
    const int64_t n_tiles64 = (int64_t)tiles_x * tiles_y;
    if (n_tiles64 > 0x7fffffffLL) return GS_ERR_INVALID_ARGUMENT;
    const int n_tiles = (int)n_tiles64;
    if (!indexing_offset) return GS_ERR_INVALID_ARGUMENT;
    const CountWs cw = carve_count(const_cast<void *>(count_workspace), n);
    const SortWs w = carve_sort(workspace, k);
    if (k > 0 && (!workspace || workspace_bytes < w.bytes)) return GS_ERR_WORKSPACE_TOO_SMALL;
    if (n > 0 && !count_workspace) return GS_ERR_INVALID_ARGUMENT;
    if (tiles_touched && n > 0) {
        hipLaunchKernelGGL(copy_u32_to_i32_kernel, dim3(ceil_div(n, 256)), dim3(256), 0, stream,
                           n, cw.touched, tiles_touched);
        int st = launch_status();
        if (st) return st;
    }
    if (k == 0) {
        return zero_bytes(indexing_offset, sizeof(int32_t) * (size_t)n_tiles, stream);
    }
    if (!points_image || !radii || !gaussian_ids_sorted || (sorted_keys && !depths))
        return GS_ERR_INVALID_ARGUMENT;

    const int tile_bits = bits_for((int64_t)n_tiles - 1);
    const SortPlan plan = plan_sort(tile_bits);
    // Values ping-pong between the caller's output and a workspace buffer so
    // that the last pass lands in the caller's output.
    uint32_t *out_vals = reinterpret_cast<uint32_t *>(gaussian_ids_sorted);
    uint32_t *va = (plan.passes % 2 == 0) ? out_vals : w.tvals_tmp;
    uint32_t *vb = (plan.passes % 2 == 0) ? w.tvals_tmp : out_vals;

    // order of Gaussians by depth: result location of the count phase's sort
    const uint32_t *order = (plan_sort(32).passes % 2 == 1) ? cw.dvals_b : cw.dvals_a;
    hipLaunchKernelGGL(emit_keys_kernel, dim3(ceil_div(n, 256)), dim3(256), 0, stream, n, k, order,
                       cw.offsets, cw.touched, points_image, radii, width, height, tile_size,
                       tiles_x, w.tkeys_a, va);
    int st = launch_status();
    if (st) return st;
    bool in_b = false;
    st = radix_sort_pairs(w.tkeys_a, va, w.tkeys_b, vb, k, tile_bits, w.sort_ws, &in_b, stream);
    if (st) return st;
    const uint32_t *sorted_tiles = in_b ? w.tkeys_b : w.tkeys_a;
    hipLaunchKernelGGL(tile_ranges_kernel, dim3(ceil_div(n_tiles, 256)), dim3(256), 0, stream,
                       n_tiles, sorted_tiles, k, indexing_offset);
    st = launch_status();
    if (st) return st;
    if (sorted_keys) {
        hipLaunchKernelGGL(sorted_keys_kernel, dim3(ceil_div(k, 256)), dim3(256), 0, stream, k, n,
                           sorted_tiles, gaussian_ids_sorted, depths, sorted_keys);
        st = launch_status();
    }
    return st;
}
