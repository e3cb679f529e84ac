// Tile blending: front-to-back alpha compositing and its gradient.
//
// One wave64 per 16x16 tile (on grids of at most 1024 tiles, 4 waves per tile:
// see blend_waves).  Lane l owns the four pixels (x0 + l%16, y0 + l/16 + 4s),
// s = 0..3, i.e. one pixel in each 16x4 strip of the tile (with W waves per
// tile, wave w's lanes own strips w*4/W .. and the waves share the staging).  The tile's depth-sorted Gaussian list is walked in batches of 64
// Gaussians (one per lane); at staging each lane computes which strips the
// Gaussian's chi-square / alpha ellipse reaches, and only Gaussians reaching
// the tile are written to LDS (ballot compaction, list order kept) with that
// strip mask and log2 of the opacity (alpha = exp2(E * -log2(e)/2 + log2 o)).
// The wave evaluates only those strips, and it stops once the
// transmittance of all 256 pixels fell below the threshold.  Tiles are assigned to workgroups XCD by XCD (the dispatcher
// places workgroup b on XCD b % 8) so that neighbouring tiles, which share
// Gaussians, run on the same XCD and share its L2.
//
// In the forward, the exponent E and the transmittance T are computed with
// separately rounded ops in the Torch rasterizer's order
// (src/torch_rasterizer.py:255-278) -- this file is compiled with
// -ffp-contract=off -- so the chi-square test (where an entry weighs about
// 0.01 o T) matches the CPU oracle exactly for identical inputs; accumulations
// use explicit fmaf.  alpha = o exp(-E/2) is evaluated as exp2 of an fma with
// the hardware exp2/log2, and the alpha test as the cut-off E < 2 ln(o /
// alpha_thr) on E; both can differ from the oracle's float results in the last
// bits, so an entry within rounding of the alpha threshold (weighing about
// alpha_thr T) may be included differently.  The backward evaluates E with two
// fmas, fewer instructions per (entry, strip); its decisions can differ from
// the forward's only for an E within rounding of a threshold.
//
// The backward walks the list in the same front-to-back order.  With
// S_i = sum_{k>i} w_k (g.c_k) = g.C - sum_{k<=i} w_k (g.c_k), where C is the
// pixel's forward colour, dL/dalpha_i = T_i (g.c_i) - S_i / (1 - alpha_i + eps).
// A lane sums its four pixels' contributions in registers, the wave reduces the
// nine fields with DPP row butterflies plus two permlane swaps, and lane 0
// issues one float atomic per (tile, Gaussian, field) (the reference issues one
// per pixel: src/cuda/kernel.cu:1098-1106).

#include "wave_ops.h"

namespace gs {

constexpr int kTile = 16;
constexpr int kStrips = 4;       // 16x4 strips per tile; one pixel of each per lane
constexpr int kBatch = kWave;    // records staged per batch and wave (one per lane)
constexpr int kGradFields = 9;   // du, dv, dA, dB, dC, dopacity, dr, dg, db
constexpr int kXcds = 8;

// Work units of a tile's walk, counted by the forward and used to launch the
// backward's tiles heaviest first: per staged batch, per staged record (its
// staging and, for nearly all of them, the backward's wave sum and atomics) and
// per evaluated strip, in proportion to the backward's instructions for each.
constexpr uint32_t kCostBatch = 33;
constexpr uint32_t kCostStaged = 11;
constexpr uint32_t kCostStrip = 6;

struct TileSpan {
    int32_t start, end;
};

// [start, end) of a tile's entries, clamped to [0, k] so that malformed
// offsets from a caller can never index outside gaussian_ids_sorted.
__device__ __forceinline__ TileSpan tile_span(const int32_t *__restrict__ offsets, int n_tiles,
                                              int64_t k, int tile) {
    TileSpan s;
    const int32_t kk = (int32_t)k;
    const int32_t a = offsets[tile];
    const int32_t b = tile + 1 < n_tiles ? offsets[tile + 1] : kk;
    s.start = min(max(a, 0), kk);
    s.end = min(max(b, s.start), kk);
    return s;
}

// Checkpoints of the forward walk, which let the backward walk a long tile list
// in up to kCheckpoints + 1 segments on as many workgroups.  Every
// checkpoint_spacing<W>() batches (at most kCheckpoints times) the forward
// saves each pixel's transmittance and accumulated colour before the batch at
// list position pos, where the next segment starts.  A segment's backward walk
// starts from that state: T from the checkpoint and the running colour-gradient
// sum from the accumulated colour (sum_{k<pos} w_k (g.c_k) = g . C_prefix), so
// the segments together make the same front-to-back walk (up to the rounding of
// that one dot product and of the backward's own alpha).  They live in the
// schedule buffer after the per-tile work and launch order (schedule_layout).
constexpr int kCheckpoints = 3;
constexpr int kSegments = kCheckpoints + 1;
// Grids of more tiles keep more workgroups waiting than the GPU holds at once,
// and the dispatcher's start of each as a slot frees already balances the
// walks: there the forward saves no checkpoints (its stores cost more than the
// segments gain: 1M Gaussians at 1920x1080, 8160 tiles, forward 138 -> 153 us,
// backward unchanged) and the schedule is 2 n_tiles int32 (work, order).
// Measured in one process against one workgroup per tile: 200k Gaussians at
// 1280x720 (3600 tiles) backward 227 -> 150 us, 100k at 800x800 (2500 tiles)
// 192 -> 147 us, 10k at 256x256 (256 tiles, 4 waves each) 92 -> 74 us.
constexpr int kCheckpointMaxTiles = 6144;
constexpr int kTilePixels = 256;  // 16 x 16

template <int W>
__device__ __forceinline__ constexpr int checkpoint_spacing() {
    return W == 1 ? 2 : 1;  // batches of W * kBatch records: 128 records with one wave
}

struct Checkpoints {
    float *data;      // [n_tiles * kCheckpoints][4][kTilePixels]: T, r, g, b planes
    int32_t *pos;     // [n_tiles * kCheckpoints] list position where segment i + 1 starts
    uint32_t *work;   // [n_tiles * kCheckpoints] the walk's work units before checkpoint i
    int32_t *count;   // [n_tiles] checkpoints saved by the forward
    int32_t *items;   // [4 n_tiles] per XCD range (at 4 * its first tile): the backward's
                      // segments tile * kSegments + segment, by descending work
    int32_t *n_items; // [kXcds] segments listed per range
};

// Schedule buffer (int32 elements): [0, n) work per tile, [n, 2n) the backward's
// launch order, [2n, 3n) checkpoint counts, [3n, 6n) checkpoint positions,
// [6n, 9n) work before each checkpoint, [9n, 13n) segment lists, [13n, 13n + 8)
// their lengths, then (16-byte aligned) the checkpoint pixels.
__host__ __device__ inline size_t schedule_head_elems(int64_t n_tiles) {
    return (size_t)((13 * n_tiles + 8 + 3) / 4 * 4);
}
__host__ __device__ inline size_t schedule_elems(int64_t n_tiles) {
    return schedule_head_elems(n_tiles) + (size_t)n_tiles * kCheckpoints * kTilePixels * 4;
}
inline Checkpoints schedule_checkpoints(int32_t *schedule, int64_t n_tiles) {
    Checkpoints c;
    c.count = schedule + 2 * n_tiles;
    c.pos = schedule + 3 * n_tiles;
    c.work = reinterpret_cast<uint32_t *>(schedule + 6 * n_tiles);
    c.items = schedule + 9 * n_tiles;
    c.n_items = schedule + 13 * n_tiles;
    c.data = reinterpret_cast<float *>(schedule + schedule_head_elems(n_tiles));
    return c;
}
constexpr Checkpoints kNoCheckpoints{nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
// The checkpoints of a schedule buffer, or none (without one, or on grids of
// more than kCheckpointMaxTiles tiles).
inline Checkpoints schedule_ck(const int32_t *schedule, int64_t n_tiles) {
    if (!schedule || n_tiles <= 0 || n_tiles > kCheckpointMaxTiles) return kNoCheckpoints;
    return schedule_checkpoints(const_cast<int32_t *>(schedule), n_tiles);
}

// Bijection workgroup -> tile giving XCD x the contiguous tile range
// [x*base + min(x, rem), ...) of length base + (x < rem).
__device__ __forceinline__ int tile_of_block(int b, int n_tiles) {
    const int base = n_tiles / kXcds, rem = n_tiles % kXcds;
    const int x = b % kXcds, i = b / kXcds;
    return x * base + min(x, rem) + i;
}

// Exponent cut-off of a Gaussian with log2 opacity log2o: E < chi and
// o exp(-E/2) >= alpha_thr, i.e. E <= 2 ln(o / alpha_thr) = 2 ln2 (log2 o -
// log2 alpha_thr).  Culling tests it with margins well above the error of the
// hardware log; both blend walks' inclusion tests use it as is (an entry within
// that error of the alpha threshold weighs about alpha_thr * T).
__device__ __forceinline__ float effective_chi(float log2o, float chi, float alpha_thr,
                                               float log2_alpha_thr) {
    // o <= 0 (log2 o = -inf) gives -inf: alpha = 0 fails any alpha_thr > 0; a NaN
    // opacity gives NaN, which fminf drops (alpha NaN passes the test, as in the
    // reference)
    float chi_eff = chi;
    if (alpha_thr > 0.0f) chi_eff = fminf(chi_eff, 1.3862943611198906f * (log2o - log2_alpha_thr));
    return chi_eff;
}

// Conservative half-extents of the ellipse {E < chi_eff} of conic (A, B, C).
// Infinite when the conic is not positive definite (no culling).  Hardware
// reciprocal and square root: the extents carry a 1% + 0.01 px margin.
__device__ __forceinline__ void ellipse_extent(float A, float B, float C, float chi_eff,
                                               float &ex, float &ey) {
    const float det = A * C - B * B;
    if (det > 0.0f && A > 0.0f && C > 0.0f && isfinite(chi_eff)) {
        const float s = fmaxf(chi_eff, 0.0f) * __builtin_amdgcn_rcpf(det);
        ex = __builtin_amdgcn_sqrtf(s * C) * 1.01f + 0.01f;
        ey = __builtin_amdgcn_sqrtf(s * A) * 1.01f + 0.01f;
    } else {
        ex = ey = __builtin_inff();
    }
}

// E = A du^2 + 2B du dv + C dv^2 in the oracle's operation order.
__device__ __forceinline__ float conic_exponent(float A, float B2, float C, float du, float dv) {
    return (A * du * du + B2 * du * dv) + C * dv * dv;
}

// alpha = o exp(-E/2) = exp2(E * kNegHalfLog2e + log2(o)): one fma and one
// v_exp_f32 per (entry, pixel).
constexpr float kNegHalfLog2e = -0.72134752044448170f;
// One batch of staged records of a tile worked by W waves (W * kBatch records).
template <int W>
struct BatchLds {
    float4 geo[kBatch * W];  // u, v, A, 2B
    float4 aux[kBatch * W];  // C, E cut-off (chi_eff), strip mask, log2(opacity)
    float4 col[kBatch * W];  // r, g, b, (gaussian id bits)
    float inv_o[kBatch * W];  // 1 / opacity (staged by the backward for its opacity gradient)
    float o_raw[kBatch * W];  // the opacity of a record whose log2 is not finite (see below)
    int wave_count[W];        // W > 1: records each wave stages, and whether one is
    int wave_bad[W];          //   non-finite (the batch then takes the select-based path)
    int wave_flag[W];         // W > 1: per-wave votes of the batch loops (tile_any)
    int wave_flag_once[W];    // W > 1: the backward's one vote before its loop
    uint32_t wave_work[W];    // W > 1: each wave's work so far, summed at a checkpoint
};

// Records whose log2 opacity is not finite -- opacity <= 0, +inf or NaN -- are
// composited as alpha = o exp(-E/2) from the staged raw opacity, with the alpha
// test applied to that value (!(alpha < alpha_thr), so a NaN alpha passes, as in
// the reference), in the select-based path that their batch takes.  They are
// staged only when the alpha test can pass them: with alpha_thr > 0 an opacity
// <= 0 has the cut-off -inf.  Their opacity gradient is sum G dalpha
// (G = exp(-E/2)); the h / o form of the other records would give 0 * inf at
// o = 0, so the backward stages 1 for their 1 / o.
__device__ __forceinline__ bool special_opacity(float log2o) { return !isfinite(log2o); }

// log2(o) for the exponent form of alpha; -inf when o <= 0 and NaN for a NaN
// opacity: such records are composited from their raw opacity (special_opacity).
__device__ __forceinline__ float log2_opacity(float o) {
    return o > 0.0f ? __builtin_amdgcn_logf(o) : (o == o ? -__builtin_inff() : o);
}

__device__ __forceinline__ float alpha_of(float E, float log2o) {
    return __builtin_amdgcn_exp2f(fmaf(E, kNegHalfLog2e, log2o));
}

// One lane's Gaussian record of the next batch, fetched into registers while
// the current batch is processed (id < 0: empty slot).
struct Record {
    float u, v, A, B, C, o, r, g, b;
    int id;
};

__device__ __forceinline__ int32_t fetch_id(int32_t i, int32_t end,
                                            const int32_t *__restrict__ ids) {
    return i < end ? ids[i] : -1;
}

__device__ __forceinline__ Record fetch_record(int32_t g, int64_t n,
                                               const float *__restrict__ points,
                                               const float *__restrict__ conics,
                                               const float *__restrict__ opac,
                                               const float *__restrict__ colors) {
    Record r;
    r.id = -1;
    r.u = r.v = r.A = r.B = r.C = r.o = r.r = r.g = r.b = 0.0f;
    if (g >= 0 && (int64_t)g < n) {
        r.id = g;
        r.u = points[2 * g];
        r.v = points[2 * g + 1];
        r.A = conics[3 * g];
        r.B = conics[3 * g + 1];
        r.C = conics[3 * g + 2];
        r.o = opac[g];
        r.r = colors[3 * g];
        r.g = colors[3 * g + 1];
        r.b = colors[3 * g + 2];
    }
    return r;
}

// Bit s set for each 16x4 strip of the tile with origin (x0, y0) that the box
// |x - u| <= ex, |y - v| <= ey reaches; 0 when it misses the tile.
__device__ __forceinline__ uint32_t strip_mask(float u, float v, float ex, float ey, float x0,
                                               float y0) {
    if (u + ex < x0 || u - ex > x0 + (kTile - 1)) return 0u;
    const float ylo = v - ey - y0, yhi = v + ey - y0;
    if (yhi < 0.0f || ylo > (float)(kTile - 1)) return 0u;
    const int s_lo = ylo <= 0.0f ? 0 : ((int)ylo >> 2);
    const int s_hi = yhi >= (float)(kTile - 1) ? kStrips - 1 : ((int)yhi >> 2);
    return ((2u << s_hi) - 1u) & ~((1u << s_lo) - 1u);
}

// Minimum of E(dx, dy) = A dx^2 + 2B dx dy + C dy^2 (positive definite) over
// the rectangle dx in [ax, bx], dy in [ay, by]: 0 if it contains the origin,
// else the least of the four edge minima (on an edge the quadratic in the free
// coordinate is minimised at its vertex -B dx / C resp. -B dy / A, clamped to
// the edge; nBC = -B / C and nBA = -B / A).
__device__ __forceinline__ float rect_min_exponent(float A, float B, float C, float nBC, float nBA,
                                                   float ax, float bx, float ay, float by) {
    if (ax <= 0.0f && bx >= 0.0f && ay <= 0.0f && by >= 0.0f) return 0.0f;
    auto edge_x = [&](float dx) {  // dx fixed, dy free in [ay, by]
        const float dy = fminf(fmaxf(nBC * dx, ay), by);
        return (A * dx * dx + 2.0f * B * dx * dy) + C * dy * dy;
    };
    auto edge_y = [&](float dy) {  // dy fixed, dx free in [ax, bx]
        const float dx = fminf(fmaxf(nBA * dy, ax), bx);
        return (A * dx * dx + 2.0f * B * dx * dy) + C * dy * dy;
    };
    return fminf(fminf(edge_x(ax), edge_x(bx)), fminf(edge_y(ay), edge_y(by)));
}

// strip_mask refined per strip by the exact ellipse: a strip stays only if the
// minimum of the exponent over its pixel rectangle is below the cut-off
// (chi_eff, with a relative and absolute margin so rounding -- also of the
// hardware reciprocal placing the edge vertices -- never drops a contributing
// pixel).  A non-positive-definite conic keeps the box mask.
__device__ __forceinline__ uint32_t exact_strip_mask(uint32_t box, float u, float v, float A,
                                                     float B, float C, float chi_eff, float x0,
                                                     float y0) {
    if (box == 0u || !(A > 0.0f && C > 0.0f && A * C - B * B > 0.0f) || !(chi_eff < 1e30f))
        return box;
    const float cut = chi_eff * 1.02f + 0.02f;
    const float nBC = -B * __builtin_amdgcn_rcpf(C), nBA = -B * __builtin_amdgcn_rcpf(A);
    const float ax = x0 - u, bx = x0 + (float)(kTile - 1) - u;
    uint32_t m = 0u;
#pragma unroll
    for (int q = 0; q < kStrips; ++q) {
        if (!((box >> q) & 1u)) continue;
        const float ay = y0 + (float)(4 * q) - v, by = ay + 3.0f;
        if (rect_min_exponent(A, B, C, nBC, nBA, ax, bx, ay, by) < cut) m |= 1u << q;
    }
    return m;
}

// Result of staging one batch: the number of staged records, and whether one
// of them has a non-finite colour (the batch then takes the select-based path).
struct Staged {
    int count;
    bool nonfinite;
};

// Stages the thread's record into the next free LDS slot if its ellipse (with
// the chi-square and alpha cut-offs) reaches the tile, keeping thread (= list)
// order, with its E cut-off (effective_chi) in aux.y, its strip mask (all four
// strips of the tile) in aux.z and log2 of its opacity in aux.w.  With W > 1
// waves, wave w's records follow those of waves 0..w-1 (one more barrier).
template <bool kInvO, int W>
__device__ __forceinline__ Staged stage_records(BatchLds<W> &s, const Record &r, float chi,
                                                float alpha_thr, float log2_alpha_thr, float x0,
                                                float y0) {
    uint32_t m = 0u;
    const float log2o = log2_opacity(r.o);
    const float chi_eff = effective_chi(log2o, chi, alpha_thr, log2_alpha_thr);
    if (r.id >= 0) {
        float ex, ey;
        ellipse_extent(r.A, r.B, r.C, chi_eff, ex, ey);
        m = exact_strip_mask(strip_mask(r.u, r.v, ex, ey, x0, y0), r.u, r.v, r.A, r.B, r.C,
                             chi_eff, x0, y0);
    }
    const uint64_t keep = __ballot(m != 0u);
    // a non-finite colour or log2 opacity (o <= 0, +inf or NaN): the batch takes
    // the select-based path (the only one that handles such opacities)
    const bool bad = m != 0u && !(isfinite(r.r) && isfinite(r.g) && isfinite(r.b) &&
                                  isfinite(log2o));
    Staged st;
    int first = 0;  // this wave's first slot
    if constexpr (W == 1) {
        st.count = __popcll(keep);
        st.nonfinite = __ballot(bad) != 0;
    } else {
        const int wave = threadIdx.x / kWave;
        const bool wave_bad = __ballot(bad) != 0;
        if (threadIdx.x % kWave == 0) {
            s.wave_count[wave] = __popcll(keep);
            s.wave_bad[wave] = wave_bad ? 1 : 0;
        }
        __syncthreads();
        st.count = 0;
        st.nonfinite = false;
#pragma unroll
        for (int w = 0; w < W; ++w) {
            const int c = s.wave_count[w];
            first += w < wave ? c : 0;
            st.count += c;
            st.nonfinite = st.nonfinite || s.wave_bad[w] != 0;
        }
    }
    if (m != 0u) {
        const int slot = first + __popcll(keep & lanemask_lt());
        s.geo[slot] = make_float4(r.u, r.v, r.A, r.B + r.B);
        s.aux[slot] = make_float4(r.C, chi_eff, __uint_as_float(m), log2o);
        s.col[slot] = make_float4(r.r, r.g, r.b, __int_as_float(r.id));
        const bool special = special_opacity(log2o);
        if (kInvO) s.inv_o[slot] = special ? 1.0f : __builtin_amdgcn_rcpf(r.o);
        if (special) s.o_raw[slot] = r.o;
    }
    return st;
}

// Software pipeline over a tile's list in batches of kBatch.  With kRecords,
// the ids of batch b+2 and the records of batch b+1 are in flight while batch
// b is processed; without, only the ids of batch b+1 (fewer registers).  The
// backward uses kRecords (2% faster although it costs a wave per SIMD at 93
// VGPRs); the forward does not (4% faster without).
// kInvO: also stage 1 / opacity (the backward).  W waves stage W * kBatch
// records per batch, one per thread.
template <bool kRecords, bool kInvO, int W = 1>
struct BatchPipe {
    int32_t next_id;  // this thread's id in the batch after the next one to stage
    Record rec;       // this thread's record of the next batch to stage (kRecords)

    __device__ __forceinline__ void start(TileSpan span, const int32_t *__restrict__ ids,
                                          int64_t n, const float *__restrict__ points,
                                          const float *__restrict__ conics,
                                          const float *__restrict__ opac,
                                          const float *__restrict__ colors) {
        const int32_t lane = (int32_t)threadIdx.x;
        if (kRecords) {
            const int32_t g0 = fetch_id(span.start + lane, span.end, ids);
            next_id = fetch_id(span.start + kBatch * W + lane, span.end, ids);
            rec = fetch_record(g0, n, points, conics, opac, colors);
        } else {
            next_id = fetch_id(span.start + lane, span.end, ids);
        }
    }

    // Stages the batch starting at b0 (only records reaching the tile) and
    // fetches ahead.
    __device__ __forceinline__ Staged advance(BatchLds<W> &s, int32_t b0, TileSpan span,
                                           const int32_t *__restrict__ ids, int64_t n,
                                           const float *__restrict__ points,
                                           const float *__restrict__ conics,
                                           const float *__restrict__ opac,
                                           const float *__restrict__ colors, float chi,
                                           float alpha_thr, float x0, float y0) {
        const int32_t lane = (int32_t)threadIdx.x;
        if (!kRecords) rec = fetch_record(next_id, n, points, conics, opac, colors);
        __syncthreads();  // previous batch fully read before restaging
        const Staged st =
            stage_records<kInvO, W>(s, rec, chi, alpha_thr, __builtin_amdgcn_logf(alpha_thr), x0,
                                    y0);
        __syncthreads();
        if (kRecords) {
            rec = fetch_record(next_id, n, points, conics, opac, colors);
            next_id = fetch_id(b0 + 2 * kBatch * W + lane, span.end, ids);
        } else {
            next_id = fetch_id(b0 + kBatch * W + lane, span.end, ids);
        }
        return st;
    }
};

// Pixel geometry of one lane: with W waves per tile, wave w's lanes own the
// S = kStrips / W strips w*S .. w*S + S - 1, one pixel of each per lane.
template <int S>
struct LanePixels {
    float fx;       // pixel x
    float fy[S];    // pixel y in the lane's strip s
    float x0, y0;   // tile origin
    bool inside[S];
};

// The wave's index within its tile's workgroup, as a wave-uniform value.
__device__ __forceinline__ int tile_wave() {
    return __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kWave));
}

template <int W>
__device__ __forceinline__ LanePixels<kStrips / W> lane_pixels(int tile, int tiles_x, int width,
                                                               int height) {
    constexpr int S = kStrips / W;
    LanePixels<S> p;
    const int lane = threadIdx.x % kWave;
    const int q0 = W == 1 ? 0 : tile_wave() * S;
    const int tx = tile % tiles_x, ty = tile / tiles_x;
    const int px = tx * kTile + (lane & 15);
    const int py = ty * kTile + (lane >> 4);
    p.fx = (float)px;
    p.x0 = (float)(tx * kTile);
    p.y0 = (float)(ty * kTile);
#pragma unroll
    for (int s = 0; s < S; ++s) {
        p.fy[s] = (float)(py + 4 * (q0 + s));
        p.inside[s] = px < width && py + 4 * (q0 + s) < height;
    }
    return p;
}

__device__ __forceinline__ bool wave_any(bool x) { return __ballot(x) != 0; }

// clamp(x, 0, 1) keeping NaN, as torch.clamp.
__device__ __forceinline__ float clamp01(float x) { return x < 0.0f ? 0.0f : (x > 1.0f ? 1.0f : x); }

// Gradient of display = clamp(image, 0, 1) * 255 w.r.t. image: torch's clamp
// passes it where 0 <= image <= 1.
__device__ __forceinline__ float display_grad(float g, float raw) {
    return (raw >= 0.0f && raw <= 1.0f) ? g * 255.0f : 0.0f;
}

// x / 255 as PyTorch computes it on the GPU for a tensor x and the Python
// scalar 255.0: x times the reciprocal of 255 rounded to float (ATen's true
// division by a CPU scalar multiplies by 1 / b).  The reference's loss divides
// the display image this way (scripts/train.py:187-197: rendered_image / 255.0),
// and the backward of that division divides the gradient the same way.
constexpr float kInv255 = 1.0f / 255.0f;

// Gradient w.r.t. display of scale * |display / 255 - t| (torch's l1_loss: sign
// of the difference, 0 at 0), plus `extra`, a further gradient w.r.t.
// display / 255 (summed there, as autograd sums the two uses of display / 255),
// then the division by 255.
__device__ __forceinline__ float l1_grad(float t, float raw, float scale, float extra) {
    const float x = (clamp01(raw) * 255.0f) * kInv255;
    const float d = x - t;
    const float sgn = d > 0.0f ? 1.0f : (d < 0.0f ? -1.0f : 0.0f);
    return (sgn * scale + extra) * kInv255;
}

// Some pixel of the wave still composites: !(T < T_thr) (NaN stays active).
template <int S>
__device__ __forceinline__ bool any_active(const float (&T)[S], float T_thr) {
    bool a = false;
#pragma unroll
    for (int q = 0; q < S; ++q) a = a || !(T[q] < T_thr);
    return wave_any(a);
}

// OR of a wave-uniform value over the tile's W waves (one barrier when W > 1).
// Every wave of the workgroup must call it; `flag` must not be written again
// before the next barrier.
template <int W>
__device__ __forceinline__ bool tile_any(bool v, int *flag) {
    if constexpr (W == 1) {
        return v;
    } else {
        if (threadIdx.x % kWave == 0) flag[threadIdx.x / kWave] = v ? 1 : 0;
        __syncthreads();
        bool any = false;
#pragma unroll
        for (int w = 0; w < W; ++w) any = any || flag[w] != 0;
        return any;
    }
}

// One staged entry j applied to the lane's four pixels.  Branch-free per
// strip: an entry that fails the chi-square or alpha test gets weight 0, so
// C += 0 * c and T -= 0 leave the pixel unchanged; kSafe (a non-finite colour
// in the batch, where 0 * inf would not be 0) uses selects instead.
// T_{i+1} = T_i - alpha T_i, i.e. T_i (1 - alpha): the 1e-10 of the
// reference's 1 - alpha + 1e-10 is below the float resolution of that factor
// unless alpha is within 1e-7 of 1, where T drops below any threshold either way.
// With W waves per tile, the entry is applied to the wave's own S strips only
// (and skipped when its strip mask misses them).
template <bool kSafe, int W>
__device__ __forceinline__ void blend_entry(const BatchLds<W> &s, int j,
                                            const LanePixels<kStrips / W> &pix, float alpha_thr,
                                            float T_thr, float chi, float (&T)[kStrips / W],
                                            float (&cr)[kStrips / W], float (&cg)[kStrips / W],
                                            float (&cb)[kStrips / W], uint32_t &work) {
    constexpr int S = kStrips / W;
    const float4 aux = s.aux[j];
    uint32_t smask = __builtin_amdgcn_readfirstlane(__float_as_uint(aux.z));
    if constexpr (W > 1) {
        smask = (smask >> (tile_wave() * S)) & ((1u << S) - 1u);
        if (smask == 0u) return;  // uniform: none of this wave's strips
    }
    const float4 geo = s.geo[j];
    const float4 col = s.col[j];
    // uniform: a record with a non-finite log2 opacity (only in the select-based path)
    const bool special =
        kSafe && special_opacity(__uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(aux.w))));
    const float o_sp = special ? s.o_raw[j] : 0.0f;
    const float du = pix.fx - geo.x;
    const float Adudu = (geo.z * du) * du;  // (A du) du, as in the oracle's A*du*du
    const float B2du = geo.w * du;
#pragma unroll
    for (int q = 0; q < S; ++q) {
        if (!((smask >> q) & 1u)) continue;  // uniform
        const float dv = pix.fy[q] - geo.y;
        const float E = (Adudu + B2du * dv) + (aux.x * dv) * dv;
        // the chi-square and alpha tests as one cut-off on E (staged in aux.y)
        bool inc = !(T[q] < T_thr) && (E < aux.y);
        float alpha = 0.0f;
        if (special) {  // alpha = o exp(-E/2) from the raw opacity, alpha test on its value
            alpha = o_sp * __builtin_amdgcn_exp2f(E * kNegHalfLog2e);
            inc = inc && !(alpha < alpha_thr);
        }
        if (!wave_any(inc)) continue;
        work += kCostStrip;
        if (!special) alpha = alpha_of(E, aux.w);
        if (kSafe) {
            const float w = alpha * T[q];
            cr[q] = inc ? fmaf(w, col.x, cr[q]) : cr[q];
            cg[q] = inc ? fmaf(w, col.y, cg[q]) : cg[q];
            cb[q] = inc ? fmaf(w, col.z, cb[q]) : cb[q];
            T[q] = inc ? T[q] - w : T[q];
        } else {
            const float w = (inc ? alpha : 0.0f) * T[q];
            cr[q] = fmaf(w, col.x, cr[q]);
            cg[q] = fmaf(w, col.y, cg[q]);
            cb[q] = fmaf(w, col.z, cb[q]);
            T[q] = T[q] - w;
        }
    }
}

template <bool kSafe, int W>
__device__ __forceinline__ void blend_batch(const BatchLds<W> &s, int cnt,
                                            const LanePixels<kStrips / W> &pix, float alpha_thr,
                                            float T_thr, float chi, float (&T)[kStrips / W],
                                            float (&cr)[kStrips / W], float (&cg)[kStrips / W],
                                            float (&cb)[kStrips / W], uint32_t &work) {
    if (W > 1 && !any_active(T, T_thr)) return;  // this wave's pixels are done
    for (int j = 0; j < cnt; ++j) {
        blend_entry<kSafe, W>(s, j, pix, alpha_thr, T_thr, chi, T, cr, cg, cb, work);
        if ((j & 7) == 7 && !any_active(T, T_thr)) break;
    }
}

// Transmittance of a pixel that takes no part (outside the image, or a zero
// gradient in the backward): inactive for every threshold above -1e30
// (thresholds are clamped there), and finite, so that a zero weight times it
// stays zero.
constexpr float kInactiveT = -3.0e38f;

__device__ __forceinline__ float effective_T_thr(float T_thr) { return fmaxf(T_thr, -1e30f); }

// Front-to-back accumulation of the lane's pixels over the tile's list, the
// tile's W waves sharing each staged batch of W * kBatch records.  Every thread
// of the workgroup must call it (it contains barriers).  `work` counts the
// wave's own strips and, in wave 0 only, the batches and staged records.
// The lane's pixels of checkpoint i of `tile` (local pixel lane + 64 * strip):
// each strip's 64 lanes store 1 KB contiguously.
template <int W>
__device__ __forceinline__ void save_checkpoint(const Checkpoints &ck, int tile, int i,
                                                int32_t pos, uint32_t work,
                                                const float (&T)[kStrips / W],
                                                const float (&cr)[kStrips / W],
                                                const float (&cg)[kStrips / W],
                                                const float (&cb)[kStrips / W]) {
    constexpr int S = kStrips / W;
    // the slot is uniform: a scalar base plus the lane's 32-bit offset
    const int slot = __builtin_amdgcn_readfirstlane(tile * kCheckpoints + i);
    const int q0 = W == 1 ? 0 : tile_wave() * S;
    float *dst = ck.data + (int64_t)slot * (4 * kTilePixels);
    const uint32_t lane = threadIdx.x % kWave;
#pragma unroll
    for (int q = 0; q < S; ++q) {  // four planes: no packing of the values into quads
        const uint32_t p = lane + (uint32_t)(kWave * (q0 + q));
        dst[p] = T[q];
        dst[kTilePixels + p] = cr[q];
        dst[2 * kTilePixels + p] = cg[q];
        dst[3 * kTilePixels + p] = cb[q];
    }
    if (threadIdx.x == 0) {  // thread 0 holds the batch and record work (wave 0)
        ck.pos[slot] = pos;
        ck.work[slot] = work;
    }
}

// With ck.data (the forward of a tile in [0, n_tiles)), saves up to kCheckpoints
// checkpoints and returns their number in n_ck (uniform across the workgroup).
template <int W>
__device__ __forceinline__ void blend_accumulate(
    BatchLds<W> &s, TileSpan span, const int32_t *__restrict__ ids, int64_t n,
    const float *__restrict__ points, const float *__restrict__ conics,
    const float *__restrict__ opac, const float *__restrict__ colors,
    const LanePixels<kStrips / W> &pix, float alpha_thr, float T_thr_in, float chi,
    float (&cr)[kStrips / W], float (&cg)[kStrips / W], float (&cb)[kStrips / W],
    uint32_t &work, const Checkpoints &ck = kNoCheckpoints,
    int tile = 0, int *n_ck = nullptr) {
    constexpr int S = kStrips / W;
    // a pixel is active while !(T < T_thr)
    const float T_thr = effective_T_thr(T_thr_in);
    float T[S];
#pragma unroll
    for (int q = 0; q < S; ++q) {
        T[q] = pix.inside[q] ? 1.0f : kInactiveT;
        cr[q] = cg[q] = cb[q] = 0.0f;
    }
    if (n_ck) *n_ck = 0;
    if (span.end <= span.start) return;
    BatchPipe<false, false, W> pipe;
    pipe.start(span, ids, n, points, conics, opac, colors);
    const bool counter = W == 1 || tile_wave() == 0;
    int batch = 0, saved = 0;
    for (int32_t b0 = span.start; b0 < span.end; b0 += kBatch * W, ++batch) {
        // with W > 1 waves, each one's work joins the vote's barrier, so that a
        // checkpoint records the tile's work so far, not wave 0's
        const bool ck_now = ck.data && batch > 0 && batch % checkpoint_spacing<W>() == 0 &&
                            saved < kCheckpoints;
        if (W > 1 && ck_now && threadIdx.x % kWave == 0) s.wave_work[tile_wave()] = work;
        if (!tile_any<W>(any_active(T, T_thr), s.wave_flag)) break;
        if (ck_now) {
            uint32_t tile_work = work;
            if constexpr (W > 1) {
                tile_work = 0;
#pragma unroll
                for (int w = 0; w < W; ++w) tile_work += s.wave_work[w];
            }
            save_checkpoint<W>(ck, tile, saved, b0, tile_work, T, cr, cg, cb);
            ++saved;
        }
        const Staged st = pipe.advance(s, b0, span, ids, n, points, conics, opac, colors, chi,
                                       alpha_thr, pix.x0, pix.y0);
        if (counter) work += kCostBatch + kCostStaged * (uint32_t)st.count;
        if (st.nonfinite)
            blend_batch<true, W>(s, st.count, pix, alpha_thr, T_thr, chi, T, cr, cg, cb, work);
        else
            blend_batch<false, W>(s, st.count, pix, alpha_thr, T_thr, chi, T, cr, cg, cb, work);
    }
    if (n_ck) *n_ck = saved;
}

// ------------------------------------------------- wave reductions (gfx950)

#define GS_DPP(x, ctrl) \
    __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), (ctrl), 0xF, 0xF, false))

constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // reverse each 8-lane half row
constexpr int kDppMirror = 0x140;     // reverse each 16-lane row
constexpr int kDppRor8 = 0x128;       // rotate each row by 8 lanes

// a + b where the two 32-lane halves are exchanged between them first:
// lanes 0-31 get a[l] + a[l+32], lanes 32-63 get b[l-32] + b[l].
__device__ __forceinline__ float swap32_add(float a, float b) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false,
                                                    false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Rows (16 lanes) r0..r3: result rows are a.r0+a.r1, b.r0+b.r1, a.r2+a.r3, b.r2+b.r3.
__device__ __forceinline__ float swap16_add(float a, float b) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false,
                                                    false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Sum over the 64 lanes, in every lane.
__device__ __forceinline__ float wave_sum(float x) {
    x += GS_DPP(x, kDppXor1);
    x += GS_DPP(x, kDppXor2);
    x += GS_DPP(x, kDppHalfMirror);
    x += GS_DPP(x, kDppMirror);
    x = swap16_add(x, x);
    return swap32_add(x, x);
}

// Lane that holds field f's wave total after wave_sum9 (the others hold partials):
// f0 0, f1 32, f2 16, f3 48, f4 8, f5 40, f6 24, f7 56, f8 4.
__device__ __forceinline__ int sum9_field_of_lane(int lane) {
    switch (lane) {
    case 0: return 0;
    case 32: return 1;
    case 16: return 2;
    case 48: return 3;
    case 8: return 4;
    case 40: return 5;
    case 24: return 6;
    case 56: return 7;
    case 4: return 8;
    default: return -1;
    }
}

// Wave sums of nine per-lane values by transposition: each exchange step halves
// the lanes a field is spread over and doubles the fields a register holds, so
// the nine sums cost 9 swaps/selects and 14 adds instead of nine full
// reductions.  All 64 lanes must be active.
__device__ __forceinline__ float wave_sum9(const float (&f)[kGradFields], bool hi8,
                                           bool f8_lane) {
    const float p0 = swap32_add(f[0], f[1]);  // halves: f0 | f1
    const float p1 = swap32_add(f[2], f[3]);  // f2 | f3
    const float p2 = swap32_add(f[4], f[5]);  // f4 | f5
    const float p3 = swap32_add(f[6], f[7]);  // f6 | f7
    const float p4 = swap32_add(f[8], 0.0f);  // f8 | 0
    const float q0 = swap16_add(p0, p1);      // rows: f0 f2 f1 f3
    const float q1 = swap16_add(p2, p3);      // rows: f4 f6 f5 f7
    float q2 = swap16_add(p4, 0.0f);          // rows: f8 0 0 0
    // low 8 lanes of each row take q0's row field, high 8 lanes q1's
    const float x = hi8 ? q1 : q0, y = hi8 ? q0 : q1;
    float r = x + GS_DPP(y, kDppRor8);
    r += GS_DPP(r, kDppXor1);
    r += GS_DPP(r, kDppXor2);
    r += GS_DPP(r, kDppHalfMirror);
    q2 += GS_DPP(q2, kDppXor1);
    q2 += GS_DPP(q2, kDppXor2);
    q2 += GS_DPP(q2, kDppHalfMirror);
    q2 += GS_DPP(q2, kDppMirror);
    return f8_lane ? q2 : r;
}

// One tile per workgroup of W waves (64 W threads).  Held to 64 VGPRs (8 waves
// per SIMD), which the compiler meets without spilling; the checkpoint stores
// would otherwise take it to 72 (7 waves).
template <int W>
__global__ __launch_bounds__(kWave * W) __attribute__((amdgpu_waves_per_eu(8, 8)))
void blend_forward_kernel(
    const int32_t *__restrict__ offsets, const int32_t *__restrict__ ids, int n_tiles,
    int64_t k, int64_t n, const float *__restrict__ points, const float *__restrict__ conics,
    const float *__restrict__ opac, const float *__restrict__ colors, int tiles_x, int width,
    int height, float alpha_thr, float T_thr, float chi, float *__restrict__ image,
    float *__restrict__ display, const float *__restrict__ target,
    float *__restrict__ tile_loss, float4 *__restrict__ clear4, int64_t clear4_count,
    uint32_t *__restrict__ tile_cost, const int32_t *__restrict__ tile_order, Checkpoints ck) {
    constexpr int S = kStrips / W;
    __shared__ BatchLds<W> s;
    __shared__ float wave_l1[W];
    __shared__ uint32_t wave_work[W];
    if (clear4) {  // this workgroup's share of the buffer to zero (stores overlap the blend)
        const int64_t per = (clear4_count + gridDim.x - 1) / gridDim.x;
        const int64_t c0 = (int64_t)blockIdx.x * per;
        const int64_t c1 = min(c0 + per, clear4_count);
        for (int64_t c = c0 + threadIdx.x; c < c1; c += kWave * W)
            clear4[c] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    // launch position -> tile: the XCD's contiguous range, in the caller's order
    // when given (a permutation of every range, e.g. heaviest first)
    const int slot = tile_of_block(blockIdx.x, n_tiles);
    const int tile = tile_order ? tile_order[slot] : slot;
    if ((unsigned)tile >= (unsigned)n_tiles) return;  // uniform across the workgroup
    const LanePixels<S> pix = lane_pixels<W>(tile, tiles_x, width, height);
    const TileSpan span = tile_span(offsets, n_tiles, k, tile);
    if (n_tiles <= kCheckpointMaxTiles) {
        // Grids whose tiles all start at once end with their longest walks: give
        // the tiles with long lists (their walks' upper bound) more of the SIMDs'
        // issue slots while they share them.  On larger grids the raised
        // priority delays the tiles that start later and the kernel ends later.
        const int64_t mean = (k - (int64_t)offsets[0]) / n_tiles;  // offsets[0]: the capped shift
        const int64_t len = span.end - span.start;
        if (len >= 3 * mean / 2)
            __builtin_amdgcn_s_setprio(3);
        else if (len >= 6 * mean / 5)
            __builtin_amdgcn_s_setprio(2);
        else if (len >= 9 * mean / 10)
            __builtin_amdgcn_s_setprio(1);
    }
    float cr[S], cg[S], cb[S];
    uint32_t work = 0;
    int n_ck = 0;
    blend_accumulate<W>(s, span, ids, n, points, conics, opac, colors, pix, alpha_thr, T_thr, chi,
                        cr, cg, cb, work, ck, tile, &n_ck);
    if (ck.count && threadIdx.x == 0) ck.count[tile] = n_ck;
    float l1 = 0.0f;
#pragma unroll
    for (int q = 0; q < S; ++q) {
        if (!pix.inside[q]) continue;
        const int64_t o = ((int64_t)pix.fy[q] * width + (int64_t)pix.fx) * 3;
        image[o] = cr[q];
        image[o + 1] = cg[q];
        image[o + 2] = cb[q];
        if (display) {  // image.clamp(0, 1) * 255 (src/cuda/wrapper.py:294)
            const float d[3] = {clamp01(cr[q]) * 255.0f, clamp01(cg[q]) * 255.0f,
                                clamp01(cb[q]) * 255.0f};
#pragma unroll
            for (int c = 0; c < 3; ++c) {
                display[o + c] = d[c];
                if (target) l1 += fabsf(d[c] * kInv255 - target[o + c]);  // |display/255 - t|
            }
        }
    }
    if (tile_loss) l1 = wave_sum(l1);  // per-tile sum of the L1 terms (reduced by gs_l1_finish)
    if constexpr (W == 1) {
        if (tile_cost && threadIdx.x == 0) tile_cost[tile] = work;
        if (tile_loss && threadIdx.x == 0) tile_loss[tile] = l1;
    } else {  // the waves' sums in wave order
        if (threadIdx.x % kWave == 0) {
            wave_l1[threadIdx.x / kWave] = l1;
            wave_work[threadIdx.x / kWave] = work;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            float sum = 0.0f;
            uint32_t wsum = 0;
#pragma unroll
            for (int w = 0; w < W; ++w) {
                sum += wave_l1[w];
                wsum += wave_work[w];
            }
            if (tile_cost) tile_cost[tile] = wsum;
            if (tile_loss) tile_loss[tile] = sum;
        }
    }
}

// Destination of the lane's field after wave_sum9:
// out[stride * g] += value * (inv_o ? 1 / o : fa).  stride4 = 4 * stride (bytes).
struct GradTarget {
    float *base;
    uint32_t stride4;
    float fa;
    bool inv_o;
    bool active;
};

__device__ __forceinline__ GradTarget grad_target(int lane, float *g_points, float *g_conics,
                                                  float *g_opac, float *g_colors) {
    GradTarget t;
    const int f = sum9_field_of_lane(lane);
    t.active = f >= 0;
    t.base = g_points;
    int stride = 2;
    t.fa = 1.0f;
    t.inv_o = false;
    switch (f) {
    case 0: t.base = g_points; break;
    case 1: t.base = g_points + 1; break;
    case 2: t.base = g_conics; stride = 3; t.fa = -0.5f; break;
    case 3: t.base = g_conics + 1; stride = 3; t.fa = -1.0f; break;
    case 4: t.base = g_conics + 2; stride = 3; t.fa = -0.5f; break;
    case 5: t.base = g_opac; stride = 1; t.inv_o = true; break;
    case 6: t.base = g_colors; stride = 3; break;
    case 7: t.base = g_colors + 1; stride = 3; break;
    case 8: t.base = g_colors + 2; stride = 3; break;
    default: break;
    }
    t.stride4 = 4u * (uint32_t)stride;
    return t;
}

// Per-lane state of the backward walk: transmittance and the running sum
// acc = sum_{k<=i} w_k (g.c_k) - g.C of the lane's four pixels (minus the
// remaining colour gradient S_i, starting at -g.C), their colour gradients g
// and gC = g.C.
template <int S>
struct BackwardLane {
    float T[S], acc[S];
    float gr[S], gg[S], gb[S], gC[S];
};

// One staged entry j: per-strip gradient terms summed over the lane's pixels,
// then the nine-field wave sum and one atomic per field (lanes of tgt).  With
// W waves per tile each wave sums and adds its own S strips' share.
template <bool kSafe, int W>
__device__ __forceinline__ void backward_entry(const BatchLds<W> &s, int j,
                                               const LanePixels<kStrips / W> &pix,
                                               float alpha_thr, float T_thr, float chi,
                                               BackwardLane<kStrips / W> &L,
                                               const GradTarget &tgt, bool hi8, bool f8_lane) {
    constexpr int S = kStrips / W;
    const float4 aux = s.aux[j];
    uint32_t smask = __builtin_amdgcn_readfirstlane(__float_as_uint(aux.z));
    if constexpr (W > 1) {
        smask = (smask >> (tile_wave() * S)) & ((1u << S) - 1u);
        if (smask == 0u) return;  // uniform: none of this wave's strips
    }
    const float4 geo = s.geo[j];
    // uniform: a record with a non-finite log2 opacity (only in the select-based
    // path); its opacity gradient is summed as G dalpha (its staged 1 / o is 1)
    const bool special =
        kSafe && special_opacity(__uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(aux.w))));
    const float o_sp = special ? s.o_raw[j] : 0.0f;
    float sGd = -0.0f;
    const float4 col = s.col[j];
    const float du = pix.fx - geo.x;
    const float Adudu = (geo.z * du) * du;
    const float B2du = geo.w * du;
    // the alpha test as a cut-off on E, staged in aux.y: alpha = o exp(-E/2) >=
    // alpha_thr iff E <= 2 ln(o / alpha_thr) (up to the rounding of the hardware
    // exp2/log2)
    const float chi_a = aux.y;
    // -0 is the identity of float addition, so the first strip's sums need no add
    float sH = -0.0f, s1 = -0.0f, s2 = -0.0f, sr = -0.0f, sg = -0.0f, sb = -0.0f;
    bool hit = false;  // some strip was evaluated (otherwise every field is -0)
#pragma unroll
    for (int q = 0; q < S; ++q) {
        if (!((smask >> q) & 1u)) continue;  // uniform
        const float dv = pix.fy[q] - geo.y;
        const float E = fmaf(fmaf(aux.x, dv, B2du), dv, Adudu);
        bool inc = !(L.T[q] < T_thr) && (E < chi_a);
        float alpha = 0.0f, G = 0.0f;
        if (special) {  // alpha = o G from the raw opacity, alpha test on its value
            G = __builtin_amdgcn_exp2f(E * kNegHalfLog2e);
            alpha = o_sp * G;
            inc = inc && !(alpha < alpha_thr);
        }
        if (!wave_any(inc)) continue;
        hit = true;
        if (!special) alpha = alpha_of(E, aux.w);
        const float a = kSafe ? alpha : (inc ? alpha : 0.0f);
        const float w = a * L.T[q];
        const float gcol = fmaf(L.gr[q], col.x, fmaf(L.gg[q], col.y, L.gb[q] * col.z));
        const float acc_new = fmaf(w, gcol, L.acc[q]);  // -S_i
        const float one_m = (1.0f - a) + kTransmittanceEps;
        // dalpha = T gcol - S_i / (1 - alpha + eps)
        const float dalpha = fmaf(acc_new, __builtin_amdgcn_rcpf(one_m), L.T[q] * gcol);
        const float h = kSafe ? (inc ? a * dalpha : 0.0f) : a * dalpha;
        const float ws = kSafe ? (inc ? w : 0.0f) : w;
        if (special) sGd += inc ? G * dalpha : 0.0f;
        sH += h;
        const float t = h * dv;
        s1 += t;
        s2 = fmaf(t, dv, s2);
        sr = fmaf(ws, L.gr[q], sr);
        sg = fmaf(ws, L.gg[q], sg);
        sb = fmaf(ws, L.gb[q], sb);
        L.acc[q] = kSafe ? (inc ? acc_new : L.acc[q]) : acc_new;
        L.T[q] = kSafe ? (inc ? L.T[q] - w : L.T[q]) : L.T[q] - w;
    }
    if (hit) {
        const float B = 0.5f * geo.w;
        const float ad = du * sH;
        float f[kGradFields];
        f[0] = fmaf(geo.z, ad, B * s1);  // d/du
        f[1] = fmaf(B, ad, aux.x * s1);  // d/dv
        f[2] = du * ad;                  // d/dA / (-1/2)
        f[3] = du * s1;                  // d/dB / (-1)
        f[4] = s2;                       // d/dC / (-1/2)
        f[5] = special ? sGd : sH;       // d/dopacity * o (special: d/dopacity)
        f[6] = sr;
        f[7] = sg;
        f[8] = sb;
        const float total = wave_sum9(f, hi8, f8_lane);
        // the entry's Gaussian id is uniform (a non-negative int32): one unsigned
        // 32 x 32 -> 64 multiply-add per field address
        const uint32_t g = __builtin_amdgcn_readfirstlane(__float_as_uint(col.w));
        if (tgt.active) {
            const float scale = tgt.inv_o ? s.inv_o[j] : tgt.fa;
            const uint64_t off = (uint64_t)g * (uint64_t)tgt.stride4;
            unsafeAtomicAdd(reinterpret_cast<float *>(reinterpret_cast<char *>(tgt.base) + off),
                            total * scale);
        }
    }
}

template <bool kSafe, int W>
__device__ __forceinline__ void backward_batch(const BatchLds<W> &s, int cnt,
                                               const LanePixels<kStrips / W> &pix,
                                               float alpha_thr, float T_thr, float chi,
                                               BackwardLane<kStrips / W> &L,
                                               const GradTarget &tgt, bool hi8, bool f8_lane) {
    if (W > 1 && !any_active(L.T, T_thr)) return;  // this wave's pixels are done
    for (int j = 0; j < cnt; ++j) {
        backward_entry<kSafe, W>(s, j, pix, alpha_thr, T_thr, chi, L, tgt, hi8, f8_lane);
        if ((j & 7) == 7 && !any_active(L.T, T_thr)) break;
    }
}

// Backward of the front-to-back blend, walking the list in the same order.
// With h = alpha dalpha (= o G dalpha), the per-pixel terms of the gradients are
//   d/du = h (A du + B dv), d/dv = h (B du + C dv),
//   d/dA = -h du^2 / 2, d/dB = -h du dv, d/dC = -h dv^2 / 2,
//   d/do = h / o, d/dc = w g.
// A lane's four pixels share du, so it keeps sH = sum h, s1 = sum h dv,
// s2 = sum h dv^2 and the colour sums, and forms the nine fields once per
// Gaussian (1/o is applied to the opacity field after the wave sum).  An entry
// that fails the chi-square or alpha test gets alpha 0, hence h = 0, w = 0 and
// an unchanged T and partial sum; where that could meet a non-finite value (a
// record's colour, or a gradient or image value of the tile) the update uses
// selects instead.
// kSeed: kSeedImage  grad_image is the gradient of the image;
//        kSeedDisplay grad_image is the gradient of display = clamp(image, 0, 1) * 255
//                     (image required);
//        kSeedL1      the gradient is that of loss = mean(|display / 255 - target|)
//                     times *grad_loss: grad_image holds the target (image required).
enum { kSeedImage = 0, kSeedDisplay = 1, kSeedL1 = 2 };

#define GS_BACKWARD_PARAMS                                                                   \
    const float *__restrict__ grad_image, const float *__restrict__ image,                   \
        const int32_t *__restrict__ offsets, const int32_t *__restrict__ ids, int n_tiles,    \
        int64_t k, int64_t n, const float *__restrict__ points,                               \
        const float *__restrict__ conics, const float *__restrict__ opac,                     \
        const float *__restrict__ colors, int tiles_x, int width, int height, float alpha_thr, \
        float T_thr_in, float chi, float *__restrict__ g_points, float *__restrict__ g_conics, \
        float *__restrict__ g_opac, float *__restrict__ g_colors,                             \
        const float *__restrict__ grad_loss, float inv_count, const float *__restrict__ extra

// The backward walk of `tile`'s list, or (seg >= 0) of its segment seg: from the
// start to checkpoint 0, between checkpoints seg - 1 and seg, or from the last
// checkpoint to the end.  Every thread of the workgroup calls it with the same
// tile and segment (it contains barriers).
template <int kSeed, int W>
__device__ __forceinline__ void backward_tile(BatchLds<W> &s, int tile, int seg,
                                              const Checkpoints &ck, GS_BACKWARD_PARAMS) {
    constexpr int S = kStrips / W;
    const float T_thr = effective_T_thr(T_thr_in);
    if ((unsigned)tile >= (unsigned)n_tiles) return;  // uniform across the workgroup
    const LanePixels<S> pix = lane_pixels<W>(tile, tiles_x, width, height);
    TileSpan span = tile_span(offsets, n_tiles, k, tile);
    int32_t ck_slot = -1;  // the checkpoint this segment starts from (seg > 0)
    if (seg >= 0) {
        // positions clamped into the tile's list: a stale count or position can
        // only make the segments wrong, never reach outside the list
        const int c = min(max(ck.count[tile], 0), kCheckpoints);
        if (seg > c) return;
        const int32_t *pos = ck.pos + (int64_t)tile * kCheckpoints;
        const int32_t a = seg == 0 ? span.start : min(max(pos[seg - 1], span.start), span.end);
        const int32_t b = seg < c ? min(max(pos[seg], a), span.end) : span.end;
        span.start = a;
        span.end = b;
        if (seg > 0) ck_slot = tile * kCheckpoints + seg - 1;
    }
    if (span.end <= span.start) return;  // uniform across the workgroup
    // d loss / d (display / 255) per element, for kSeedL1
    const float l1_scale = kSeed == kSeedL1 ? *grad_loss * inv_count : 0.0f;

    BackwardLane<S> L;
    float cr[S], cg[S], cb[S];
    uint32_t work = 0;  // unused here
    if (!image)
        blend_accumulate<W>(s, span, ids, n, points, conics, opac, colors, pix, alpha_thr,
                            T_thr_in, chi, cr, cg, cb, work);
    bool finite = true;
#pragma unroll
    for (int q = 0; q < S; ++q) {
        float gr = 0.0f, gg = 0.0f, gb = 0.0f;
        if (pix.inside[q]) {
            const int64_t o = ((int64_t)pix.fy[q] * width + (int64_t)pix.fx) * 3;
            gr = grad_image[o];
            gg = grad_image[o + 1];
            gb = grad_image[o + 2];
            if (image) {
                cr[q] = image[o];
                cg[q] = image[o + 1];
                cb[q] = image[o + 2];
            }
            if (kSeed == kSeedL1) {  // sign(display/255 - t) * g / n (+ extra), then / 255
                const bool ex = extra != nullptr;
                gr = l1_grad(gr, cr[q], l1_scale, ex ? extra[o] : 0.0f);
                gg = l1_grad(gg, cg[q], l1_scale, ex ? extra[o + 1] : 0.0f);
                gb = l1_grad(gb, cb[q], l1_scale, ex ? extra[o + 2] : 0.0f);
            }
            if (kSeed != kSeedImage) {
                gr = display_grad(gr, cr[q]);
                gg = display_grad(gg, cg[q]);
                gb = display_grad(gb, cb[q]);
            }
        } else {
            cr[q] = cg[q] = cb[q] = 0.0f;
        }
        L.gr[q] = gr;
        L.gg[q] = gg;
        L.gb[q] = gb;
        L.gC[q] = gr * cr[q] + gg * cg[q] + gb * cb[q];
        L.acc[q] = -L.gC[q];
        finite = finite && isfinite(gr) && isfinite(gg) && isfinite(gb) && isfinite(L.gC[q]);
        // active while !(T < T_thr); pixels outside the image or with a zero
        // gradient (skipped as in src/cuda/kernel.cu:1028-1030) start inactive
        const bool live = pix.inside[q] && !(gr == 0.0f && gg == 0.0f && gb == 0.0f);
        float T0 = 1.0f;
        if (ck_slot >= 0) {  // a later segment: the forward's state at its first entry
            const int q0 = W == 1 ? 0 : tile_wave() * S;
            const float *c = ck.data + (int64_t)ck_slot * (4 * kTilePixels) +
                             (threadIdx.x % kWave) + kWave * (q0 + q);
            T0 = c[0];
            L.acc[q] = fmaf(gr, c[kTilePixels], fmaf(gg, c[2 * kTilePixels],
                                                    gb * c[3 * kTilePixels])) - L.gC[q];
            finite = finite && isfinite(L.acc[q]);
        }
        L.T[q] = live ? T0 : kInactiveT;
    }
    // the zero-weight update needs finite gradients and image values in the tile
    const bool tile_nonfinite = tile_any<W>(__ballot(!finite) != 0, s.wave_flag_once);

    const int lane = threadIdx.x % kWave;
    const bool hi8 = (lane & 8) != 0;
    const bool f8_lane = lane == 4;
    const GradTarget tgt = grad_target(lane, g_points, g_conics, g_opac, g_colors);

    BatchPipe<true, true, W> pipe;
    pipe.start(span, ids, n, points, conics, opac, colors);
    for (int32_t b0 = span.start; b0 < span.end; b0 += kBatch * W) {
        if (!tile_any<W>(any_active(L.T, T_thr), s.wave_flag)) break;
        const Staged st = pipe.advance(s, b0, span, ids, n, points, conics, opac, colors, chi,
                                       alpha_thr, pix.x0, pix.y0);
        if (st.nonfinite || tile_nonfinite)
            backward_batch<true, W>(s, st.count, pix, alpha_thr, T_thr, chi, L, tgt, hi8,
                                    f8_lane);
        else
            backward_batch<false, W>(s, st.count, pix, alpha_thr, T_thr, chi, L, tgt, hi8,
                                     f8_lane);
    }
}

// Without segment lists: one workgroup of W waves per tile slot.  With them:
// kSegments workgroups per tile slot of the largest XCD range, workgroup b
// taking entry b / kXcds of range b % kXcds's list (the dispatcher places
// workgroup b on XCD b % kXcds and launches in order: each XCD works through its
// list heaviest tiles first, a tile's segments side by side); workgroups past
// their range's list end at once.
template <int kSeed, int W>
__global__ __launch_bounds__(kWave * W) void blend_backward_kernel(
    GS_BACKWARD_PARAMS, const int32_t *__restrict__ tile_order, Checkpoints ck) {
    __shared__ BatchLds<W> s;
    int tile, seg = -1;
    if (!ck.items) {
        const int slot = tile_of_block(blockIdx.x, n_tiles);
        tile = tile_order ? tile_order[slot] : slot;
    } else {
        const int base = n_tiles / kXcds, rem = n_tiles % kXcds;
        const int x = (int)blockIdx.x % kXcds, j = (int)blockIdx.x / kXcds;
        const int first = x * base + min(x, rem), len = base + (x < rem ? 1 : 0);
        const int listed = min(ck.n_items[x], kSegments * len);
        if (j >= listed) return;  // uniform across the workgroup
        const int item = ck.items[4 * (int64_t)first + j];
        tile = item / kSegments;
        seg = item % kSegments;
    }
    backward_tile<kSeed, W>(s, tile, seg, ck, grad_image, image, offsets, ids, n_tiles, k, n,
                            points, conics, opac, colors, tiles_x, width, height, alpha_thr,
                            T_thr_in, chi, g_points, g_conics, g_opac, g_colors, grad_loss,
                            inv_count, extra);
}

// ------------------------------------------------ generic tile size path
// One thread per pixel, no staging; used only when tile_size != 16.

__global__ void blend_forward_generic_kernel(
    const int32_t *__restrict__ offsets, const int32_t *__restrict__ ids, int n_tiles,
    int64_t k, int64_t n, const float *__restrict__ points, const float *__restrict__ conics,
    const float *__restrict__ opac, const float *__restrict__ colors, int tiles_x, int width,
    int height, int ts, float alpha_thr, float T_thr, float chi, float *__restrict__ image) {
    const int tile = blockIdx.x;
    const int px = (tile % tiles_x) * ts + (int)threadIdx.x % ts;
    const int py = (tile / tiles_x) * ts + (int)threadIdx.x / ts;
    if (px >= width || py >= height) return;
    const TileSpan span = tile_span(offsets, n_tiles, k, tile);
    float T = 1.0f, cr = 0.f, cg = 0.f, cb = 0.f;
    if (1.0f >= T_thr) {
        for (int32_t i = span.start; i < span.end; ++i) {
            const int g = ids[i];
            if (g < 0 || (int64_t)g >= n) continue;
            const float du = (float)px - points[2 * g], dv = (float)py - points[2 * g + 1];
            const float B = conics[3 * g + 1];
            const float E = conic_exponent(conics[3 * g], B + B, conics[3 * g + 2], du, dv);
            if (!(E < chi)) continue;
            const float alpha = __expf(-0.5f * E) * opac[g];
            if (alpha < alpha_thr) continue;
            const float w = alpha * T;
            cr = fmaf(w, colors[3 * g], cr);
            cg = fmaf(w, colors[3 * g + 1], cg);
            cb = fmaf(w, colors[3 * g + 2], cb);
            T = T * ((1.0f - alpha) + kTransmittanceEps);
            if (T < T_thr) break;
        }
    }
    const int64_t o = ((int64_t)py * width + px) * 3;
    image[o] = cr;
    image[o + 1] = cg;
    image[o + 2] = cb;
}

__global__ void blend_backward_generic_kernel(
    const float *__restrict__ grad_image, const float *__restrict__ image,
    const int32_t *__restrict__ offsets, const int32_t *__restrict__ ids, int n_tiles,
    int64_t k, int64_t n, const float *__restrict__ points, const float *__restrict__ conics,
    const float *__restrict__ opac, const float *__restrict__ colors, int tiles_x, int width,
    int height, int ts, float alpha_thr, float T_thr, float chi, float *__restrict__ g_points,
    float *__restrict__ g_conics, float *__restrict__ g_opac, float *__restrict__ g_colors) {
    const int tile = blockIdx.x;
    const int px = (tile % tiles_x) * ts + (int)threadIdx.x % ts;
    const int py = (tile / tiles_x) * ts + (int)threadIdx.x / ts;
    if (px >= width || py >= height || !(1.0f >= T_thr)) return;
    const TileSpan span = tile_span(offsets, n_tiles, k, tile);
    const int64_t pix = ((int64_t)py * width + px) * 3;
    const float gr = grad_image[pix], gg = grad_image[pix + 1], gb = grad_image[pix + 2];
    if (gr == 0.0f && gg == 0.0f && gb == 0.0f) return;
    float cr = 0.f, cg = 0.f, cb = 0.f;
    if (image) {
        cr = image[pix];
        cg = image[pix + 1];
        cb = image[pix + 2];
    } else {
        float T = 1.0f;
        for (int32_t i = span.start; i < span.end; ++i) {
            const int g = ids[i];
            if (g < 0 || (int64_t)g >= n) continue;
            const float du = (float)px - points[2 * g], dv = (float)py - points[2 * g + 1];
            const float B = conics[3 * g + 1];
            const float E = conic_exponent(conics[3 * g], B + B, conics[3 * g + 2], du, dv);
            if (!(E < chi)) continue;
            const float alpha = __expf(-0.5f * E) * opac[g];
            if (alpha < alpha_thr) continue;
            const float w = alpha * T;
            cr = fmaf(w, colors[3 * g], cr);
            cg = fmaf(w, colors[3 * g + 1], cg);
            cb = fmaf(w, colors[3 * g + 2], cb);
            T = T * ((1.0f - alpha) + kTransmittanceEps);
            if (T < T_thr) break;
        }
    }
    const float gC = gr * cr + gg * cg + gb * cb;
    float T = 1.0f, acc = 0.0f;
    for (int32_t i = span.start; i < span.end; ++i) {
        const int g = ids[i];
        if (g < 0 || (int64_t)g >= n) continue;
        const float u = points[2 * g], vv = points[2 * g + 1];
        const float A = conics[3 * g], B = conics[3 * g + 1], C = conics[3 * g + 2];
        const float du = (float)px - u, dv = (float)py - vv;
        const float E = conic_exponent(A, B + B, C, du, dv);
        if (!(E < chi)) continue;
        const float G = __expf(-0.5f * E);
        const float alpha = G * opac[g];
        if (alpha < alpha_thr) continue;
        const float c0 = colors[3 * g], c1 = colors[3 * g + 1], c2 = colors[3 * g + 2];
        const float w = alpha * T;
        const float gcol = fmaf(gr, c0, fmaf(gg, c1, gb * c2));
        const float acc_new = fmaf(w, gcol, acc);
        const float one_m = (1.0f - alpha) + kTransmittanceEps;
        const float dalpha = T * gcol - (gC - acc_new) / one_m;
        const float h = alpha * dalpha;
        unsafeAtomicAdd(g_points + 2 * g, h * fmaf(A, du, B * dv));
        unsafeAtomicAdd(g_points + 2 * g + 1, h * fmaf(B, du, C * dv));
        unsafeAtomicAdd(g_conics + 3 * g, -0.5f * h * du * du);
        unsafeAtomicAdd(g_conics + 3 * g + 1, -h * du * dv);
        unsafeAtomicAdd(g_conics + 3 * g + 2, -0.5f * h * dv * dv);
        unsafeAtomicAdd(g_opac + g, G * dalpha);
        unsafeAtomicAdd(g_colors + 3 * g, w * gr);
        unsafeAtomicAdd(g_colors + 3 * g + 1, w * gg);
        unsafeAtomicAdd(g_colors + 3 * g + 2, w * gb);
        acc = acc_new;
        T = T * one_m;
        if (T < T_thr) break;
    }
}

// Work of the reference blend loop (src/cuda/kernel.cu:954-982) for the
// roofline: per pixel, the list entries visited until the transmittance test
// stops it (`visited`, including entries culled by the chi-square or alpha
// test) and the entries that were composited (`composited`).  One thread per
// pixel; totals are added to the two counters.
__global__ void blend_work_kernel(const int32_t *__restrict__ offsets,
                                  const int32_t *__restrict__ ids, int n_tiles, int64_t k,
                                  int64_t n, const float *__restrict__ points,
                                  const float *__restrict__ conics,
                                  const float *__restrict__ opac, int tiles_x, int width,
                                  int height, int ts, float alpha_thr, float T_thr, float chi,
                                  unsigned long long *__restrict__ visited,
                                  unsigned long long *__restrict__ composited) {
    const int tile = blockIdx.x;
    const int px = (tile % tiles_x) * ts + (int)threadIdx.x % ts;
    const int py = (tile / tiles_x) * ts + (int)threadIdx.x / ts;
    unsigned long long v = 0, c = 0;
    if (px < width && py < height && 1.0f >= T_thr) {
        const TileSpan span = tile_span(offsets, n_tiles, k, tile);
        float T = 1.0f;
        for (int32_t i = span.start; i < span.end; ++i) {
            ++v;
            const int g = ids[i];
            if (g < 0 || (int64_t)g >= n) continue;
            const float du = (float)px - points[2 * g], dv = (float)py - points[2 * g + 1];
            const float B = conics[3 * g + 1];
            const float E = conic_exponent(conics[3 * g], B + B, conics[3 * g + 2], du, dv);
            if (!(E < chi)) continue;
            const float alpha = __expf(-0.5f * E) * opac[g];
            if (alpha < alpha_thr) continue;
            ++c;
            T = T * ((1.0f - alpha) + kTransmittanceEps);
            if (T < T_thr) break;
        }
    }
    if (v) atomicAdd(visited, v);
    if (c) atomicAdd(composited, c);
}

}  // namespace gs

using namespace gs;

static int check_blend_args(const int32_t *indexing_offset, const int32_t *ids, int32_t n_tiles,
                            int64_t k, int64_t n, int32_t width, int32_t height,
                            int32_t tile_size, float alpha_thr, float T_thr, float chi) {
    if (n < 0 || k < 0 || n_tiles < 0 || width <= 0 || height <= 0 || tile_size <= 0)
        return GS_ERR_INVALID_ARGUMENT;
    // NaN thresholds would make every comparison false (pixels never stop)
    if (alpha_thr != alpha_thr || T_thr != T_thr || chi != chi) return GS_ERR_INVALID_ARGUMENT;
    if (k > 0x7fffffffLL) return GS_ERR_TOO_MANY_KEYS;
    if (tile_size * tile_size > 1024) return GS_ERR_UNSUPPORTED;
    const int64_t tiles_x = (width + tile_size - 1) / tile_size;
    const int64_t tiles_y = (height + tile_size - 1) / tile_size;
    // every grid tile must have an offset entry (the kernels index pixels from the tile id)
    if (n_tiles > tiles_x * tiles_y) return GS_ERR_INVALID_ARGUMENT;
    if (n_tiles > 0 && !indexing_offset) return GS_ERR_INVALID_ARGUMENT;
    if (k > 0 && !ids) return GS_ERR_INVALID_ARGUMENT;
    return GS_OK;
}

// Waves per tile of the 16x16 blend kernels.  A grid with few tiles leaves most
// SIMDs idle, and a kernel then lasts as long as its slowest tile takes on its
// waves: splitting each tile's strips over 2 or 4 waves (which share the staged
// batches) shortens that, at the price of each wave reading the entries that
// reach its strips, and in the backward of a wave sum and atomics per wave and
// entry.  Measured (blend forward / backward, us, 1 -> 2 -> 4 waves):
// 256 tiles 101/155 -> 86/118 -> 73/88; 2500 tiles 140/193 -> 138/247 ->
// 149/352; 3600 tiles 160/210 -> 146/229 -> 152/329; 8160 tiles 159/238 ->
// 173/396 -> 202/712.
// Two waves gain in the forward on mid-size grids and lose in every backward, so
// the backward takes 4 waves up to kFourWaveTiles tiles and 1 above, the forward
// also 2 up to kCheckpointMaxTiles tiles (the forward's checkpoints and the
// backward's segments do not depend on either's wave count).  Per-tile timing of
// the forward with checkpoints (kernel span, us, 1 -> 2 waves): 3600 tiles
// 161.9 -> 140.9, 2500 tiles 129.7 -> 125.6.
constexpr int kFourWaveTiles = 1024;
static int g_blend_waves = 0;  // gs_set_blend_waves: 0 = by tile count

static int blend_waves(int32_t n_tiles) {
    if (g_blend_waves) return g_blend_waves;
    return n_tiles <= kFourWaveTiles ? 4 : 1;
}

static int blend_waves_forward(int32_t n_tiles) {
    if (g_blend_waves) return g_blend_waves;
    return n_tiles <= kFourWaveTiles ? 4 : (n_tiles <= kCheckpointMaxTiles ? 2 : 1);
}

static int rasterize_impl(const int32_t *indexing_offset, const int32_t *gaussian_ids_sorted,
                          int32_t n_tiles, int64_t k, const float *points_image,
                          const float *cov_inv_image, const float *opacities, const float *colors,
                          int64_t n, int32_t width, int32_t height, int32_t tile_size,
                          float alpha_threshold, float transmittance_threshold,
                          float chi_squared_threshold, float *image, float *display,
                          const float *target, float *tile_loss, hipStream_t stream,
                          float *clear = nullptr, int64_t clear_count = 0,
                          uint32_t *tile_cost = nullptr, const int32_t *tile_order = nullptr,
                          Checkpoints ck = kNoCheckpoints) {
    int st = check_blend_args(indexing_offset, gaussian_ids_sorted, n_tiles, k, n, width, height,
                              tile_size, alpha_threshold, transmittance_threshold,
                              chi_squared_threshold);
    if (st) return st;
    if (!image) return GS_ERR_INVALID_ARGUMENT;
    if (display && tile_size != kTile) return GS_ERR_UNSUPPORTED;
    const int tiles_x = (width + tile_size - 1) / tile_size;
    const int tiles_y = (height + tile_size - 1) / tile_size;
    if (n_tiles < tiles_x * tiles_y) {
        // pixels of tiles without an offset entry stay zero (the reference zero-initialises)
        const size_t bytes = (size_t)width * height * 3 * sizeof(float);
        st = zero_bytes(image, bytes, stream);
        if (!st && display) st = zero_bytes(display, bytes, stream);
        if (st) return st;
    }
    if (clear_count < 0 || (clear_count > 0 && !clear)) return GS_ERR_INVALID_ARGUMENT;
    // the forward kernel zeroes `clear` when it is float4-aligned and has tiles to
    // spread it over; otherwise a fill kernel does
    const bool fused_clear = clear_count > 0 && n_tiles > 0 && tile_size == kTile &&
                             (reinterpret_cast<uintptr_t>(clear) & 15) == 0 &&
                             clear_count % 4 == 0;
    if (clear_count > 0 && !fused_clear) {
        st = zero_bytes(clear, (size_t)clear_count * sizeof(float), stream);
        if (st) return st;
    }
    if (n_tiles == 0) return GS_OK;
    if (k > 0 && (!points_image || !cov_inv_image || !opacities || !colors))
        return GS_ERR_INVALID_ARGUMENT;
    if (tile_size == kTile) {
        const int W = blend_waves_forward(n_tiles);
        auto kern = W == 4 ? blend_forward_kernel<4>
                    : W == 2 ? blend_forward_kernel<2>
                             : blend_forward_kernel<1>;
        hipLaunchKernelGGL(kern, dim3(n_tiles), dim3(kWave * W), 0, stream,
                           indexing_offset, gaussian_ids_sorted, n_tiles, k, n, points_image,
                           cov_inv_image, opacities, colors, tiles_x, width, height,
                           alpha_threshold, transmittance_threshold, chi_squared_threshold,
                           image, display, target, tile_loss,
                           fused_clear ? reinterpret_cast<float4 *>(clear) : nullptr,
                           fused_clear ? clear_count / 4 : (int64_t)0, tile_cost, tile_order, ck);
    } else {
        hipLaunchKernelGGL(blend_forward_generic_kernel, dim3(n_tiles),
                           dim3(tile_size * tile_size), 0, stream, indexing_offset,
                           gaussian_ids_sorted, n_tiles, k, n, points_image, cov_inv_image,
                           opacities, colors, tiles_x, width, height, tile_size,
                           alpha_threshold, transmittance_threshold, chi_squared_threshold,
                           image);
    }
    return launch_status();
}

extern "C" int gs_set_blend_waves(int32_t waves) {
    if (waves != 0 && waves != 1 && waves != 2 && waves != 4) return GS_ERR_INVALID_ARGUMENT;
    g_blend_waves = waves;
    return GS_OK;
}

extern "C" int gs_rasterize(const int32_t *indexing_offset, const int32_t *gaussian_ids_sorted,
                            int32_t n_tiles, int64_t k, const float *points_image,
                            const float *cov_inv_image, const float *opacities,
                            const float *colors, int64_t n, int32_t width, int32_t height,
                            int32_t tile_size, float alpha_threshold,
                            float transmittance_threshold, float chi_squared_threshold,
                            float *image, hipStream_t stream) {
    return rasterize_impl(indexing_offset, gaussian_ids_sorted, n_tiles, k, points_image,
                          cov_inv_image, opacities, colors, n, width, height, tile_size,
                          alpha_threshold, transmittance_threshold, chi_squared_threshold, image,
                          nullptr, nullptr, nullptr, stream);
}

static int launch_l1_finish(int32_t n_tiles, const float *tile_loss, float inv_count, float *loss,
                            const uint32_t *tile_cost, int32_t *tile_order, hipStream_t stream,
                            Checkpoints ck = kNoCheckpoints);

extern "C" int gs_rasterize_display(const int32_t *indexing_offset,
                                    const int32_t *gaussian_ids_sorted, int32_t n_tiles,
                                    int64_t k, const float *points_image,
                                    const float *cov_inv_image, const float *opacities,
                                    const float *colors, int64_t n, int32_t width,
                                    int32_t height, int32_t tile_size, float alpha_threshold,
                                    float transmittance_threshold, float chi_squared_threshold,
                                    float *image, float *display, int32_t *tile_schedule,
                                    const int32_t *forward_order, hipStream_t stream) {
    if (!display) return GS_ERR_INVALID_ARGUMENT;
    uint32_t *cost = tile_schedule ? reinterpret_cast<uint32_t *>(tile_schedule) : nullptr;
    const int st = rasterize_impl(indexing_offset, gaussian_ids_sorted, n_tiles, k, points_image,
                                  cov_inv_image, opacities, colors, n, width, height, tile_size,
                                  alpha_threshold, transmittance_threshold, chi_squared_threshold,
                                  image, display, nullptr, nullptr, stream, nullptr, 0, cost,
                                  forward_order, schedule_ck(tile_schedule, n_tiles));
    if (st || !tile_schedule || n_tiles == 0) return st;
    return launch_l1_finish(n_tiles, nullptr, 0.0f, nullptr, cost, tile_schedule + n_tiles,
                            stream, schedule_ck(tile_schedule, n_tiles));
}

extern "C" int gs_rasterize_display_l1(
    const int32_t *indexing_offset, const int32_t *gaussian_ids_sorted, int32_t n_tiles, int64_t k,
    const float *points_image, const float *cov_inv_image, const float *opacities,
    const float *colors, int64_t n, int32_t width, int32_t height, int32_t tile_size,
    float alpha_threshold, float transmittance_threshold, float chi_squared_threshold,
    const float *target, float *image, float *display, float *tile_loss, float *loss,
    int32_t *tile_schedule, float *clear, int64_t clear_count, const int32_t *forward_order,
    hipStream_t stream) {
    if (!display || !target || !tile_loss || tile_size != kTile) return GS_ERR_INVALID_ARGUMENT;
    const int tiles_x = (width + tile_size - 1) / tile_size;
    const int tiles_y = (height + tile_size - 1) / tile_size;
    if (n_tiles != tiles_x * tiles_y) return GS_ERR_INVALID_ARGUMENT;  // every tile's loss
    uint32_t *cost = tile_schedule ? reinterpret_cast<uint32_t *>(tile_schedule) : nullptr;
    int st = rasterize_impl(indexing_offset, gaussian_ids_sorted, n_tiles, k, points_image,
                            cov_inv_image, opacities, colors, n, width, height, tile_size,
                            alpha_threshold, transmittance_threshold, chi_squared_threshold,
                            image, display, target, tile_loss, stream, clear, clear_count, cost,
                            forward_order, schedule_ck(tile_schedule, n_tiles));
    if (st) return st;
    // the loss (when asked for) and the backward's tile order, in one launch
    const double count = (double)width * (double)height * 3.0;
    return launch_l1_finish(n_tiles, tile_loss, (float)(1.0 / count), loss, cost,
                            tile_schedule ? tile_schedule + n_tiles : nullptr, stream,
                            schedule_ck(tile_schedule, n_tiles));
}

// The backward's launch order from the forward's per-tile work: within each
// XCD's contiguous tile range (the range tile_of_block gives XCD x), the tiles by
// descending work, ties by tile, so that an XCD starts its heaviest tiles first
// and the light ones fill the SIMDs as they free up.  order[p] is the tile that
// the workgroup at range position p processes.  Work is compared through a
// 9-bit code, its bit length and the 4 bits below its leading one (16 steps per
// octave, 4% apart), with tiles of equal code in tile order: a stable counting
// sort by one workgroup per range (a histogram, then the range in chunks of
// kFinishThreads tiles, each placed at its code's running start plus its rank
// among the chunk's tiles of that code, by ballot matching and per-wave counts).
constexpr int kFinishThreads = 512;
constexpr int kFinishWaves = kFinishThreads / kWave;
constexpr int kOrderCodes = 512;

// Ascending codes: descending work (0 for the heaviest class, 511 for no work).
__device__ __forceinline__ uint32_t order_code(uint32_t work) {
    if (work == 0u) return kOrderCodes - 1;
    const uint32_t e = 31u - (uint32_t)__clz(work);  // leading one
    const uint32_t m = e >= 4u ? (work >> (e - 4u)) & 15u : (work << (4u - e)) & 15u;
    return (uint32_t)(kOrderCodes - 2) - min(e * 16u + m, (uint32_t)(kOrderCodes - 2));
}


__device__ void order_range(int x, const uint32_t *__restrict__ cost, int n_tiles,
                            int32_t *__restrict__ order, const Checkpoints &ck) {
    __shared__ uint32_t start_of[kOrderCodes];
    __shared__ uint32_t wave_cnt[kFinishWaves][kOrderCodes];
    const int base = n_tiles / kXcds, rem = n_tiles % kXcds;
    const int first = x * base + min(x, rem), len = base + (x < rem ? 1 : 0);
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    // one stable counting sort pass over `codes` codes (a multiple of kWave, at
    // most kOrderCodes) of `bits` bits: the count of each code, their exclusive
    // scan, then the elements in chunks of kFinishThreads (one per thread), each
    // placed at its code's running start plus its rank among the chunk's
    // elements of that code
    auto scan_codes = [&](int codes) {
        if (threadIdx.x < kWave) {  // exclusive scan of the counts by one wave
            const int per = codes / kWave;
            uint32_t c[kOrderCodes / kWave], run = 0;
#pragma unroll
            for (int e = 0; e < kOrderCodes / kWave; ++e) {
                c[e] = e < per ? start_of[lane * per + e] : 0u;
                run += c[e];
            }
            const uint32_t incl = wave_inclusive_scan(run);
            uint32_t at = incl - run;
#pragma unroll
            for (int e = 0; e < kOrderCodes / kWave; ++e) {
                if (e < per) start_of[lane * per + e] = at;
                at += c[e];
            }
        }
    };
    // places one element per thread (valid ones), returns its position (or 0)
    auto place = [&](bool valid, uint32_t d, int codes, int bits) -> uint32_t {
        for (int dd = lane; dd < codes; dd += kWave) wave_cnt[wave][dd] = 0u;
        __syncthreads();
        const uint64_t peers = match_digit(d, bits, __ballot(valid));
        if (valid && (peers & lanemask_lt()) == 0) wave_cnt[wave][d] = (uint32_t)__popcll(peers);
        __syncthreads();
        uint32_t pos = 0;
        if (valid) {
            pos = start_of[d] + (uint32_t)__popcll(peers & lanemask_lt());
            for (int w = 0; w < wave; ++w) pos += wave_cnt[w][d];
        }
        __syncthreads();
        for (int dd = threadIdx.x; dd < codes; dd += kFinishThreads) {
            uint32_t c = 0;
#pragma unroll
            for (int w = 0; w < kFinishWaves; ++w) c += wave_cnt[w][dd];
            start_of[dd] += c;
        }
        __syncthreads();  // counts read before the next chunk clears them
        return pos;
    };

    // the tiles by descending work
    for (int d = threadIdx.x; d < kOrderCodes; d += kFinishThreads) start_of[d] = 0u;
    __syncthreads();
    for (int i = threadIdx.x; i < len; i += kFinishThreads)
        atomicAdd(&start_of[order_code(cost[first + i])], 1u);
    __syncthreads();
    scan_codes(kOrderCodes);
    for (int c0 = 0; c0 < len; c0 += kFinishThreads) {
        const int i = c0 + (int)threadIdx.x;
        const bool valid = i < len;
        const uint32_t d = valid ? order_code(cost[first + i]) : 0u;
        const uint32_t pos = place(valid, d, kOrderCodes, 9);
        if (valid) order[first + (int)pos] = first + i;
    }
    if (!ck.count) return;

    // the segments by descending work (a coarser code, 4 steps per octave: the
    // sort is one of kSegments rounds per chunk): segment q of tile t is worked
    // from checkpoint q - 1 (or the start) to checkpoint q (or the end)
    auto segment_work = [&](int t, int q, int c) -> uint32_t {
        const uint32_t before = q > 0 ? ck.work[t * kCheckpoints + q - 1] : 0u;
        const uint32_t upto = q < c ? ck.work[t * kCheckpoints + q] : cost[t];
        return upto > before ? upto - before : 1u;
    };
    __syncthreads();
    constexpr int kSegCodes = kOrderCodes / 4;
    auto seg_code = [&](int t, int q, int c) { return order_code(segment_work(t, q, c)) >> 2; };
    for (int d = threadIdx.x; d < kSegCodes; d += kFinishThreads) start_of[d] = 0u;
    __syncthreads();
    uint32_t mine = 0;
    for (int i = threadIdx.x; i < len; i += kFinishThreads) {
        const int t = first + i;
        const int c = min(max(ck.count[t], 0), kCheckpoints);
        for (int q = 0; q <= c; ++q) atomicAdd(&start_of[seg_code(t, q, c)], 1u);
        mine += (uint32_t)c + 1u;
    }
    __syncthreads();
    scan_codes(kSegCodes);
    int32_t *items = ck.items + 4 * (int64_t)first;
    for (int c0 = 0; c0 < len; c0 += kFinishThreads) {
        const int i = c0 + (int)threadIdx.x;
        const int t = first + i;
        const int c = i < len ? min(max(ck.count[t], 0), kCheckpoints) : -1;
        for (int q = 0; q < kSegments; ++q) {  // the chunk's q-th segments, one per tile
            const bool valid = q <= c;
            const uint32_t d = valid ? (uint32_t)seg_code(t, q, c) : 0u;
            const uint32_t pos = place(valid, d, kSegCodes, 7);
            if (valid) items[pos] = t * kSegments + q;
        }
    }
    // the list's length: the sum of the tiles' segment counts
    uint32_t total;
    __shared__ uint32_t scan_tmp[kFinishWaves + 1];
    block_exclusive_scan<uint32_t, kFinishThreads>(mine, scan_tmp, total);
    if (threadIdx.x == 0) ck.n_items[x] = (int32_t)total;
}

// Workgroups 0..kXcds-1 (with tile_order) order the backward's tiles (and, with
// checkpoints, list their segments); the last workgroup (with loss) writes
// loss = (sum of the n_tiles partial sums) * inv_count.
__global__ __launch_bounds__(kFinishThreads) void l1_finish_kernel(
    int n_tiles, const float *__restrict__ tile_loss, float inv_count, float *__restrict__ loss,
    const uint32_t *__restrict__ tile_cost, int32_t *__restrict__ tile_order, Checkpoints ck) {
    if (tile_order && (int)blockIdx.x < kXcds) {
        order_range((int)blockIdx.x, tile_cost, n_tiles, tile_order, ck);
        return;
    }
    if (!loss) return;
    __shared__ float tmp[kFinishThreads / kWave];
    // kLossLoads independent loads in flight per thread
    constexpr int kLossLoads = 8;
    float part[kLossLoads];
#pragma unroll
    for (int u = 0; u < kLossLoads; ++u) part[u] = 0.0f;
    for (int t0 = threadIdx.x; t0 < n_tiles; t0 += kFinishThreads * kLossLoads) {
#pragma unroll
        for (int u = 0; u < kLossLoads; ++u) {
            const int t = t0 + u * kFinishThreads;
            if (t < n_tiles) part[u] += tile_loss[t];
        }
    }
    float acc = 0.0f;
#pragma unroll
    for (int u = 0; u < kLossLoads; ++u) acc += part[u];
    acc = wave_sum(acc);
    if (threadIdx.x % kWave == 0) tmp[threadIdx.x / kWave] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        float total = 0.0f;
        for (int w = 0; w < kFinishThreads / kWave; ++w) total += tmp[w];
        *loss = total * inv_count;
    }
}

static int launch_l1_finish(int32_t n_tiles, const float *tile_loss, float inv_count, float *loss,
                            const uint32_t *tile_cost, int32_t *tile_order, hipStream_t stream,
                            Checkpoints ck) {
    const int blocks = (tile_order ? kXcds : 0) + (loss ? 1 : 0);
    if (blocks == 0) return GS_OK;
    hipLaunchKernelGGL(l1_finish_kernel, dim3(blocks), dim3(kFinishThreads), 0, stream, n_tiles,
                       tile_loss, inv_count, loss, tile_cost, tile_order,
                       tile_order ? ck : kNoCheckpoints);
    return launch_status();
}

extern "C" int gs_l1_finish(const float *tile_loss, int32_t n_tiles, int64_t count, float *loss,
                            hipStream_t stream) {
    if (n_tiles < 0 || count <= 0 || !loss || (n_tiles > 0 && !tile_loss))
        return GS_ERR_INVALID_ARGUMENT;
    return launch_l1_finish(n_tiles, tile_loss, (float)(1.0 / (double)count), loss, nullptr,
                            nullptr, stream);
}

static int rasterize_backward_impl(
    const float *grad_image, const float *image, const int32_t *indexing_offset,
    const int32_t *gaussian_ids_sorted, int32_t n_tiles, int64_t k, const float *points_image,
    const float *cov_inv_image, const float *opacities, const float *colors, int64_t n,
    int32_t width, int32_t height, int32_t tile_size, float alpha_threshold,
    float transmittance_threshold, float chi_squared_threshold, float *grad_points_image,
    float *grad_cov_inv_image, float *grad_opacities, float *grad_colors, int32_t accumulate,
    int seed, const float *grad_loss, float inv_count, hipStream_t stream,
    const float *extra = nullptr, const int32_t *tile_order = nullptr,
    Checkpoints ck = kNoCheckpoints) {
    int st = check_blend_args(indexing_offset, gaussian_ids_sorted, n_tiles, k, n, width, height,
                              tile_size, alpha_threshold, transmittance_threshold,
                              chi_squared_threshold);
    if (st) return st;
    if (n > 0 && (!grad_points_image || !grad_cov_inv_image || !grad_opacities || !grad_colors))
        return GS_ERR_INVALID_ARGUMENT;
    if (seed != kSeedImage && (!image || tile_size != kTile)) return GS_ERR_INVALID_ARGUMENT;
    if (seed == kSeedL1 && !grad_loss) return GS_ERR_INVALID_ARGUMENT;
    if (n > 0 && !accumulate) {
        st = zero_bytes(grad_points_image, (size_t)n * 2 * sizeof(float), stream);
        if (!st) st = zero_bytes(grad_cov_inv_image, (size_t)n * 3 * sizeof(float), stream);
        if (!st) st = zero_bytes(grad_opacities, (size_t)n * sizeof(float), stream);
        if (!st) st = zero_bytes(grad_colors, (size_t)n * 3 * sizeof(float), stream);
        if (st) return st;
    }
    if (n_tiles == 0 || k == 0) return GS_OK;
    if (!grad_image || !points_image || !cov_inv_image || !opacities || !colors)
        return GS_ERR_INVALID_ARGUMENT;
    const int tiles_x = (width + tile_size - 1) / tile_size;
    if (tile_size == kTile) {
        const int W = blend_waves(n_tiles);
        auto pick = [&](auto l1, auto disp, auto img) {
            return seed == kSeedL1 ? l1 : (seed == kSeedDisplay ? disp : img);
        };
        auto kern = W == 4 ? pick(blend_backward_kernel<kSeedL1, 4>,
                                  blend_backward_kernel<kSeedDisplay, 4>,
                                  blend_backward_kernel<kSeedImage, 4>)
                    : W == 2 ? pick(blend_backward_kernel<kSeedL1, 2>,
                                    blend_backward_kernel<kSeedDisplay, 2>,
                                    blend_backward_kernel<kSeedImage, 2>)
                             : pick(blend_backward_kernel<kSeedL1, 1>,
                                    blend_backward_kernel<kSeedDisplay, 1>,
                                    blend_backward_kernel<kSeedImage, 1>);
        // segments from the forward's checkpoints need the image (a recomputed
        // forward has none) and the order they came with
        if (!image || !tile_order) ck = kNoCheckpoints;
        // with lists: kSegments workgroups per slot of the largest range, on each XCD
        const int64_t grid =
            ck.items ? (int64_t)kXcds * kSegments * ((n_tiles + kXcds - 1) / kXcds) : n_tiles;
        hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(kWave * W), 0, stream, grad_image,
                           image, indexing_offset, gaussian_ids_sorted, n_tiles, k, n,
                           points_image, cov_inv_image, opacities, colors, tiles_x, width, height,
                           alpha_threshold, transmittance_threshold, chi_squared_threshold,
                           grad_points_image, grad_cov_inv_image, grad_opacities, grad_colors,
                           grad_loss, inv_count, extra, tile_order, ck);
    } else {
        hipLaunchKernelGGL(blend_backward_generic_kernel, dim3(n_tiles),
                           dim3(tile_size * tile_size), 0, stream, grad_image, image,
                           indexing_offset, gaussian_ids_sorted, n_tiles, k, n, points_image,
                           cov_inv_image, opacities, colors, tiles_x, width, height, tile_size,
                           alpha_threshold, transmittance_threshold, chi_squared_threshold,
                           grad_points_image, grad_cov_inv_image, grad_opacities, grad_colors);
    }
    return launch_status();
}

extern "C" int gs_rasterize_backward(
    const float *grad_image, const float *image, const int32_t *indexing_offset,
    const int32_t *gaussian_ids_sorted, int32_t n_tiles, int64_t k, const float *points_image,
    const float *cov_inv_image, const float *opacities, const float *colors, int64_t n,
    int32_t width, int32_t height, int32_t tile_size, float alpha_threshold,
    float transmittance_threshold, float chi_squared_threshold, float *grad_points_image,
    float *grad_cov_inv_image, float *grad_opacities, float *grad_colors, int32_t accumulate,
    hipStream_t stream) {
    return rasterize_backward_impl(grad_image, image, indexing_offset, gaussian_ids_sorted,
                                   n_tiles, k, points_image, cov_inv_image, opacities, colors, n,
                                   width, height, tile_size, alpha_threshold,
                                   transmittance_threshold, chi_squared_threshold,
                                   grad_points_image, grad_cov_inv_image, grad_opacities,
                                   grad_colors, accumulate, kSeedImage, nullptr, 0.0f, stream);
}

extern "C" int gs_rasterize_display_backward(
    const float *grad_display, const float *image, const int32_t *indexing_offset,
    const int32_t *gaussian_ids_sorted, int32_t n_tiles, int64_t k, const float *points_image,
    const float *cov_inv_image, const float *opacities, const float *colors, int64_t n,
    int32_t width, int32_t height, int32_t tile_size, float alpha_threshold,
    float transmittance_threshold, float chi_squared_threshold, float *grad_points_image,
    float *grad_cov_inv_image, float *grad_opacities, float *grad_colors, int32_t accumulate,
    const int32_t *tile_schedule, hipStream_t stream) {
    return rasterize_backward_impl(grad_display, image, indexing_offset, gaussian_ids_sorted,
                                   n_tiles, k, points_image, cov_inv_image, opacities, colors, n,
                                   width, height, tile_size, alpha_threshold,
                                   transmittance_threshold, chi_squared_threshold,
                                   grad_points_image, grad_cov_inv_image, grad_opacities,
                                   grad_colors, accumulate, kSeedDisplay, nullptr, 0.0f, stream,
                                   nullptr, tile_schedule ? tile_schedule + n_tiles : nullptr,
                                   schedule_ck(tile_schedule, n_tiles));
}

extern "C" int gs_rasterize_l1_backward(
    const float *target, const float *grad_loss, const float *image,
    const int32_t *indexing_offset, const int32_t *gaussian_ids_sorted, int32_t n_tiles,
    int64_t k, const float *points_image, const float *cov_inv_image, const float *opacities,
    const float *colors, int64_t n, int32_t width, int32_t height, int32_t tile_size,
    float alpha_threshold, float transmittance_threshold, float chi_squared_threshold,
    float *grad_points_image, float *grad_cov_inv_image, float *grad_opacities,
    float *grad_colors, int32_t accumulate, float loss_scale, const float *grad_display01,
    const int32_t *tile_schedule, hipStream_t stream) {
    if (!target || width <= 0 || height <= 0 || !(loss_scale == loss_scale))
        return GS_ERR_INVALID_ARGUMENT;
    // d loss / d (display / 255) = sign * *grad_loss * loss_scale / (H * W * 3)
    const float inv_count = (float)((double)loss_scale / ((double)width * (double)height * 3.0));
    return rasterize_backward_impl(target, image, indexing_offset, gaussian_ids_sorted, n_tiles,
                                   k, points_image, cov_inv_image, opacities, colors, n, width,
                                   height, tile_size, alpha_threshold, transmittance_threshold,
                                   chi_squared_threshold, grad_points_image, grad_cov_inv_image,
                                   grad_opacities, grad_colors, accumulate, kSeedL1, grad_loss,
                                   inv_count, stream, grad_display01,
                                   tile_schedule ? tile_schedule + n_tiles : nullptr,
                                   schedule_ck(tile_schedule, n_tiles));
}

extern "C" int gs_rasterize_work(const int32_t *indexing_offset,
                                 const int32_t *gaussian_ids_sorted, int32_t n_tiles, int64_t k,
                                 const float *points_image, const float *cov_inv_image,
                                 const float *opacities, int64_t n, int32_t width, int32_t height,
                                 int32_t tile_size, float alpha_threshold,
                                 float transmittance_threshold, float chi_squared_threshold,
                                 uint64_t *visited, uint64_t *composited, hipStream_t stream) {
    int st = check_blend_args(indexing_offset, gaussian_ids_sorted, n_tiles, k, n, width, height,
                              tile_size, alpha_threshold,
                              transmittance_threshold, chi_squared_threshold);
    if (st) return st;
    if (!visited || !composited) return GS_ERR_INVALID_ARGUMENT;
    st = zero_bytes(visited, sizeof(uint64_t), stream);
    if (!st) st = zero_bytes(composited, sizeof(uint64_t), stream);
    if (st || n_tiles == 0 || k == 0) return st;
    if (!points_image || !cov_inv_image || !opacities) return GS_ERR_INVALID_ARGUMENT;
    const int tiles_x = (width + tile_size - 1) / tile_size;
    hipLaunchKernelGGL(blend_work_kernel, dim3(n_tiles), dim3(tile_size * tile_size), 0, stream,
                       indexing_offset, gaussian_ids_sorted, n_tiles, k, n, points_image,
                       cov_inv_image, opacities, tiles_x, width, height, tile_size,
                       alpha_threshold, transmittance_threshold, chi_squared_threshold,
                       reinterpret_cast<unsigned long long *>(visited),
                       reinterpret_cast<unsigned long long *>(composited));
    return launch_status();
}

extern "C" int gs_tile_schedule_size(int32_t n_tiles, size_t *elements) {
    if (n_tiles < 0 || !elements) return GS_ERR_INVALID_ARGUMENT;
    *elements = n_tiles <= 0                              ? 2
                : n_tiles > gs::kCheckpointMaxTiles ? 2 * (size_t)n_tiles
                                                    : gs::schedule_elems(n_tiles);
    return GS_OK;
}
