// SSIM loss term of the training loop for gfx950: the mean structural
// similarity of img1 against img2 and its gradient with respect to img1.
//
// The reference's loss (scripts/train.py:185-205) calls the third-party
// fused_ssim(img1, img2, padding="valid") (fused-ssim==0.0.0,
// environment.yml:56; not vendored).  This file computes the published SSIM of
// Wang et al. (IEEE TIP 2004) that it implements: per (batch, channel) plane,
// local statistics under an 11x11 Gaussian window of standard deviation 1.5
// with zero padding, C1 = 0.01^2, C2 = 0.03^2, averaged over all pixels or
// over the pixels at least 5 from the border.
//
// Layout.  Work is cut into units of 64 columns x 34 rows of outputs of one
// plane, one per wave (lane = output column); a fixed number of workgroups of
// 4 waves (set by the image geometry alone) walk them, each XCD a contiguous
// range.  A wave streams its unit's input rows (10 more than its
// output rows) top to bottom: each row's 74 staged values (and the products
// x^2 + y^2, xy) go to a wave-private LDS line, each lane filters its 11
// neighbours, and the column filter accumulates into an 11-row ring of
// registers, so an output row is complete 10 rows after its first
// contribution; its SSIM and derivatives are formed during the next row's LDS
// reads.  No workgroup barrier inside the walk; input rows are loaded a few
// rows ahead, at wave-uniform row addresses plus per-lane column offsets.
// Both passes sum their 11 taps in ascending order, as a separable 2D filter
// evaluated row pass first does.
// The forward writes per-pixel derivative maps (planar, coalesced) for the
// backward, which filters them back the same way.  The mean is reduced
// deterministically: per-workgroup double partials, then one workgroup.
#include <cmath>
#include <mutex>

#include "gs_common.h"

namespace gs {
namespace {

constexpr int kRadius = 5;
constexpr int kTaps = 2 * kRadius + 1;
constexpr int kTileX = 64;                       // output columns per workgroup (lane = column)
constexpr int kUnitWaves = 4;                    // units (waves) per workgroup
constexpr int kThreads = kUnitWaves * kWave;
constexpr int kWaves = kThreads / kWave;
constexpr int kInX = kTileX + 2 * kRadius;       // staged columns of an input row (74)
constexpr int kRing = kTaps;                     // output rows accumulating at once
constexpr float kC1 = 0.01f * 0.01f;
constexpr float kC2 = 0.03f * 0.03f;

static_assert(kTileX == kWave, "one lane per output column");

// Unit shape of a pass: kRows output rows per unit (kRows + 2 kRadius input
// rows, walked in whole ring turns: the rows past them complete output rows
// past the unit, which are not written), input rows loaded kAheadRows ahead of
// the filtered one.  kRows + 2 kRadius a multiple of kRing walks no rows past
// the unit; taller units re-read fewer halo rows (from L2) but leave fewer
// waves to fill the GPU.
template <int kRows, int kAheadRows>
struct Shape {
    static constexpr int rows = kRows;
    static constexpr int ahead = kAheadRows;
    static constexpr int in_rows = kRows + 2 * kRadius;
    static constexpr int walk = (in_rows + kRing - 1) / kRing * kRing;
    static_assert(kAheadRows > 0 && kAheadRows < kRing, "prefetch within the ring");
};
using FwdShape = Shape<34, 5>;
using BwdShape = Shape<34, 4>;

struct Window {
    float w[kTaps];
};

// Normalised Gaussian taps exp(-k^2 / (2 * 1.5^2)) / sum, k = -5..5, formed in
// double and rounded once.
Window make_window() {
    double e[kTaps], sum = 0.0;
    for (int k = 0; k < kTaps; ++k) {
        const double d = (double)(k - kRadius);
        e[k] = std::exp(-(d * d) / (2.0 * 1.5 * 1.5));
        sum += e[k];
    }
    Window w;
    for (int k = 0; k < kTaps; ++k) w.w[k] = (float)(e[k] / sum);
    return w;
}

struct Planes {
    const float *img1, *img2;
    int64_t s1[2], s2[2];  // element strides of batch and channel
    int r1, c1, r2, c2;    // element strides of row and column (in-plane offsets fit 31 bits)
    int channels, height, width;
    int tiles_x, tiles_y, tiles;
    int valid;             // mean over pixels at least kRadius from the border
    float inv_count;       // 1 / pixels in the mean (all planes)
    float inv1;            // img1 values are its elements * inv1 (1: as stored)
};

// Element of img1 as the SSIM sees it: times inv1 = 1 / divisor rounded to
// float, which is how PyTorch's GPU kernels compute image / divisor for a
// scalar divisor (so the values equal the reference's rendered_image / 255).
__device__ __forceinline__ float img1_value(const Planes &p, float v) {
    return p.inv1 == 1.0f ? v : v * p.inv1;
}

__device__ __forceinline__ bool in_region(const Planes &p, int y, int x) {
    if (!p.valid) return true;
    return y >= kRadius && y < p.height - kRadius && x >= kRadius && x < p.width - kRadius;
}

__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
    for (int o = kWave / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

// Sum over the workgroup, in a fixed order; valid in thread 0.
__device__ __forceinline__ double block_sum(double v, double *tmp) {
    v = wave_sum(v);
    if (threadIdx.x % kWave == 0) tmp[threadIdx.x / kWave] = v;
    __syncthreads();
    double s = 0.0;
    if (threadIdx.x == 0)
#pragma unroll
        for (int w = 0; w < kWaves; ++w) s += tmp[w];
    return s;
}

// Workgroups are dealt to the kXcds XCDs round robin (workgroup w runs on XCD
// w % kXcds), each XCD with its own L2.  xcd_block(w) is the logical workgroup
// whose units w walks: each XCD takes a contiguous range of logical
// workgroups, so the channels of a region, the neighbouring strips whose halo
// columns overlap and the unit rows above and below are read through one L2.
// A bijection of [0, blocks).
constexpr int kXcds = 8;

__device__ __forceinline__ int xcd_block(int w, int blocks) {
    const int base = blocks / kXcds, rem = blocks % kXcds;
    const int x = w % kXcds, i = w / kXcds;
    return x * base + (x < rem ? x : rem) + i;
}

// Unit `t`: units run over (batch, unit row, unit column, channel), channel
// fastest, so the channels of one region -- interleaved in memory for (H, W, C)
// images -- are walked by neighbouring waves at the same time and their rows
// come from one L2.
struct Tile {
    int plane, b, c;
    int ox, oy;  // first output column / row
};

template <int kRows>
__device__ __forceinline__ Tile tile_of(const Planes &p, int t) {
    Tile r;
    r.c = t % p.channels;
    const int rest = t / p.channels;
    const int tx = rest % p.tiles_x;
    const int rest2 = rest / p.tiles_x;
    r.b = rest2 / p.tiles_y;
    r.plane = r.b * p.channels + r.c;
    r.ox = tx * kTileX;
    r.oy = (rest2 % p.tiles_y) * kRows;
    return r;
}

// This lane's staged columns of a unit: ox - kRadius + lane and, for the first
// 2 kRadius lanes, ox - kRadius + kWave + lane (the right halo); with their
// byte offsets, clamped into the image, in a row of img1, of img2 and of a
// planar map, and the byte offsets of the lane's output column (clamped) in a
// row of img1 and img2.  Row starts are wave-uniform pointers (scalar
// registers), so a load adds only these per-lane offsets.
struct Cols {
    int a, b;
    bool has_b;
    uint32_t a1, b1, a2, b2, am, bm;
    uint32_t o1, o2;
};

__device__ __forceinline__ Cols cols_of(const Planes &p, const Tile &t) {
    const int lane = threadIdx.x % kWave;
    Cols c;
    c.a = t.ox - kRadius + lane;
    c.b = t.ox - kRadius + kWave + lane;
    c.has_b = lane < 2 * kRadius;
    const uint32_t ca = (uint32_t)min(max(c.a, 0), p.width - 1);
    const uint32_t cb = (uint32_t)min(c.b, p.width - 1);
    const uint32_t co = (uint32_t)min(t.ox + lane, p.width - 1);
    c.a1 = ca * (uint32_t)p.c1 * 4u;
    c.b1 = cb * (uint32_t)p.c1 * 4u;
    c.a2 = ca * (uint32_t)p.c2 * 4u;
    c.b2 = cb * (uint32_t)p.c2 * 4u;
    c.am = ca * 4u;
    c.bm = cb * 4u;
    c.o1 = co * (uint32_t)p.c1 * 4u;
    c.o2 = co * (uint32_t)p.c2 * 4u;
    return c;
}

// The float `byte_offset` bytes past `row`, a wave-uniform pointer: a raw
// buffer access over the bytes from `row` on, whose base and row offset live in
// scalar registers and whose per-lane offset is the 32-bit value itself (a
// plain access would add a 64-bit vector address per load or store).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t span_of(const float *row) {
    // stride 0, 2^32 - 1 bytes (no range check in practice), gfx9 data format
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(row), (short)0, -1, 0x00020000);
}

__device__ __forceinline__ float load_at(const float *row, uint32_t byte_offset) {
    return __uint_as_float(
        __builtin_amdgcn_raw_buffer_load_b32(span_of(row), (int)byte_offset, 0, 0));
}

__device__ __forceinline__ void store_at(float *row, uint32_t byte_offset, float v) {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), span_of(row), (int)byte_offset, 0,
                                          0);
}

// Image row gy of both images at the lane's staged columns, as stored (loads
// at clamped, in-image positions; the positions outside the image are zeroed
// and the divisor applied when the values are used, some rows later, so that
// no load has to complete before then).
__device__ __forceinline__ void load_image_row(const Planes &p, const float *b1, const float *b2,
                                               int gy, const Cols &c, float &xa, float &ya,
                                               float &xb, float &yb) {
    int y = min(max(gy, 0), p.height - 1);
    asm volatile("" : "+s"(y));  // the loads stay at their row (not hoisted ahead)
    const float *r1 = b1 + y * p.r1, *r2 = b2 + y * p.r2;
    xa = load_at(r1, c.a1);
    ya = load_at(r2, c.a2);
    xb = load_at(r1, c.b1);
    yb = load_at(r2, c.b2);
}

// Whether image row gy's staged columns a and b lie in the image.
__device__ __forceinline__ void row_inside(const Planes &p, int gy, const Cols &c, bool &ina,
                                           bool &inb) {
    const bool row_in = gy >= 0 && gy < p.height;
    ina = row_in && c.a >= 0 && c.a < p.width;
    inb = row_in && c.has_b && c.b < p.width;
}

// Row gy of the three planar maps at the lane's staged columns, as stored
// (clamped loads; zeroed outside the image when used).
__device__ __forceinline__ void load_map_row(const Planes &p, const float *m0, const float *m1,
                                             const float *m2, int64_t base, int gy, const Cols &c,
                                             float (&va)[3], float (&vb)[3]) {
    int y = min(max(gy, 0), p.height - 1);
    asm volatile("" : "+s"(y));  // the loads stay at their row (not hoisted ahead)
    const int64_t o = base + (int64_t)y * p.width;
    va[0] = load_at(m0 + o, c.am);
    va[1] = load_at(m1 + o, c.am);
    va[2] = load_at(m2 + o, c.am);
    vb[0] = load_at(m0 + o, c.bm);
    vb[1] = load_at(m1 + o, c.bm);
    vb[2] = load_at(m2 + o, c.bm);
}

// img1 / img2 at row gy of the lane's output column as stored (clamped load;
// zeroed and divided when used).
__device__ __forceinline__ void load_pixel(const Planes &p, const float *b1, const float *b2,
                                           int gy, const Cols &c, float &x, float &y) {
    int yy = min(max(gy, 0), p.height - 1);
    asm volatile("" : "+s"(yy));  // the loads stay at their row
    x = load_at(b1 + yy * p.r1, c.o1);
    y = load_at(b2 + yy * p.r2, c.o2);
}

typedef float f4v __attribute__((ext_vector_type(4)));

// The wave's LDS line at this lane's 11 taps (line[lane + k], k = 0..10), the
// reads issued together.
__device__ __forceinline__ void read_taps(const float4 *line, f4v (&v)[kTaps]) {
    const int lane = threadIdx.x % kWave;
    const f4v *src = reinterpret_cast<const f4v *>(line) + lane;
#pragma unroll
    for (int k = 0; k < kTaps; ++k) v[k] = src[k];
}

// Waits for all the taps at once, here: left alone, the compiler keeps two
// reads in flight and waits on each pair in turn (and work placed between
// read_taps and this point runs while the reads are in flight).
__device__ __forceinline__ void taps_ready(f4v (&v)[kTaps]) {
    static_assert(kTaps == 11, "one operand per tap");
    asm volatile("" : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]),
                 "+v"(v[6]), "+v"(v[7]), "+v"(v[8]), "+v"(v[9]), "+v"(v[10]));
}

// Horizontal filter at this lane's output column: h[q] = sum_k w[k] v[k].q,
// k ascending.
template <int NQ>
__device__ __forceinline__ void filter_taps(const Window &win, const f4v (&v)[kTaps],
                                            float (&h)[NQ]) {
#pragma unroll
    for (int q = 0; q < NQ; ++q) h[q] = 0.0f;
#pragma unroll
    for (int k = 0; k < kTaps; ++k)
#pragma unroll
        for (int q = 0; q < NQ; ++q) h[q] = fmaf(win.w[k], v[k][q], h[q]);
}

// Makes the wave's LDS line stores visible to the wave's loads that follow
// (and keeps the next row's stores after this row's loads).
__device__ __forceinline__ void line_sync() {
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
}

// One input row ri of a unit in the column filter: the row's filtered values h
// add tap k to output row ri - k (ring slot (ri - k) mod kRing, written as
// (s - k) mod kRing with s = ri mod kRing), rows above the unit (ri - k < 0)
// excluded.  kFirst: ri = s (the first kRing rows; the exclusion is then
// resolved at compile time).
template <int NQ, bool kFirst, int S>
__device__ __forceinline__ void ring_add(const Window &win, int ri, const float (&h)[NQ],
                                         float (&acc)[kRing][NQ]) {
#pragma unroll
    for (int k = 0; k < kTaps; ++k) {
        if (kFirst && S < k) continue;
        (void)ri;
        float(&a)[NQ] = acc[(S - k + kRing) % kRing];
#pragma unroll
        for (int q = 0; q < NQ; ++q) a[q] = fmaf(win.w[k], h[q], a[q]);
    }
    // the ring as it stands after this row, in registers: otherwise the
    // compiler sinks these FMAs to the rows that complete the sums, keeping up
    // to 10 rows of LDS loads live (hundreds of registers)
#pragma unroll
    for (int r = 0; r < kRing; ++r)
#pragma unroll
        for (int q = 0; q < NQ; ++q) asm volatile("" : "+v"(acc[r][q]));
}

// SSIM of one output (statistics mu1, mu2, E[x^2] + E[y^2], E[xy] of its
// window) and its derivatives: S and, with the maps, d mean / d (E[x], E[x^2],
// E[xy]) scaled by g (1 / pixels in the mean, 0 outside the region).
struct SsimOut {
    float S, dm, dxx, dxy;
};

__device__ __forceinline__ SsimOut ssim_point(const float (&a)[4]) {
    const float mu1 = a[0], mu2 = a[1];
    const float s_sum = a[2] - mu1 * mu1 - mu2 * mu2;  // sigma1^2 + sigma2^2
    const float s12 = a[3] - mu1 * mu2;
    const float C = 2.0f * mu1 * mu2 + kC1;
    const float D = 2.0f * s12 + kC2;
    const float A = mu1 * mu1 + mu2 * mu2 + kC1;
    const float B = s_sum + kC2;
    const float rA = __builtin_amdgcn_rcpf(A), rB = __builtin_amdgcn_rcpf(B);
    const float rAB = rA * rB;
    SsimOut o;
    o.S = C * D * rAB;
    // d S / d E[x], d E[x^2], d E[xy] (mu1, E[x^2], E[xy] independent)
    o.dm = 2.0f * mu2 * (D - C) * rAB + 2.0f * mu1 * o.S * (rB - rA);
    o.dxx = -o.S * rB;
    o.dxy = 2.0f * C * rAB;
    return o;
}

// Output row j of a forward unit, complete in ring slot kSlot: its SSIM
// (summed into `local` over the region) and, with d_mu, the derivative maps;
// the slot is then cleared for the output row that starts in it.
template <int kSlot>
__device__ __forceinline__ void forward_out(const Planes &p, const Tile &tl, int j,
                                            float (&acc)[kRing][4], double &local, float *d_mu,
                                            float *d_xx, float *d_xy) {
    const int lane = threadIdx.x % kWave;
    float(&a)[4] = acc[kSlot];
    const int gy = tl.oy + j;
    const int gx = tl.ox + lane;
    if (j < FwdShape::rows && gy < p.height && gx < p.width) {
        const SsimOut o = ssim_point(a);
        const bool in = in_region(p, gy, gx);
        if (in) local += (double)o.S;
        if (d_mu) {
            const float g = in ? p.inv_count : 0.0f;
            int row = gy;
            asm volatile("" : "+s"(row));  // the addresses are formed here, not ahead
            const int64_t at = (int64_t)tl.plane * p.height * p.width + (int64_t)row * p.width;
            const uint32_t col = (uint32_t)gx * 4u;
            store_at(d_mu + at, col, g * o.dm);
            store_at(d_xx + at, col, g * o.dxx);
            store_at(d_xy + at, col, g * o.dxy);
        }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) a[q] = 0.0f;
}

// Forward of one unit: per input row ri, x, y, x^2 + y^2 and xy into the LDS
// line, the horizontal filter, the ring.  Input row ri - 1 completed output row
// ri - 1 - 2 kRadius in slot S (= ri mod kRing); it is emitted while this row's
// taps are read, before tap 0 of this row starts the slot again.
template <bool kFirst, int S>
__device__ __forceinline__ void forward_row(const Planes &p, const Window &win, const Tile &tl,
                                            const Cols &c, const float *b1, const float *b2,
                                            float4 *line, int ri, float (&xa)[kRing],
                                            float (&ya)[kRing], float (&xb)[kRing],
                                            float (&yb)[kRing], float (&acc)[kRing][4],
                                            double &local, float *d_mu, float *d_xx,
                                            float *d_xy) {
    const int lane = threadIdx.x % kWave;
    constexpr int kNext = (S + FwdShape::ahead) % kRing;
    // (rows past the walk load in-image values that are never used)
    load_image_row(p, b1, b2, tl.oy - kRadius + ri + FwdShape::ahead, c, xa[kNext], ya[kNext],
                   xb[kNext], yb[kNext]);
    bool ina, inb;
    row_inside(p, tl.oy - kRadius + ri, c, ina, inb);
    const float x = ina ? img1_value(p, xa[S]) : 0.0f, y = ina ? ya[S] : 0.0f;
    line[lane] = make_float4(x, y, x * x + y * y, x * y);
    if (c.has_b) {
        const float x2 = inb ? img1_value(p, xb[S]) : 0.0f, y2 = inb ? yb[S] : 0.0f;
        line[kWave + lane] = make_float4(x2, y2, x2 * x2 + y2 * y2, x2 * y2);
    }
    line_sync();
    f4v v[kTaps];
    read_taps(line, v);
    // (the first kRing input rows complete no output row before this one)
    if constexpr (!kFirst) forward_out<S>(p, tl, ri - kRing, acc, local, d_mu, d_xx, d_xy);
    taps_ready(v);
    float h[4];
    filter_taps<4>(win, v, h);
    line_sync();
    ring_add<4, kFirst, S>(win, ri, h, acc);
}

template <bool kFirst, int S = 0>
__device__ __forceinline__ void forward_rows(const Planes &p, const Window &win, const Tile &tl,
                                             const Cols &c, const float *b1, const float *b2,
                                             float4 *line, int base, float (&xa)[kRing],
                                             float (&ya)[kRing], float (&xb)[kRing],
                                             float (&yb)[kRing], float (&acc)[kRing][4],
                                             double &local, float *d_mu, float *d_xx,
                                             float *d_xy) {
    if constexpr (S < kRing) {
        forward_row<kFirst, S>(p, win, tl, c, b1, b2, line, base + S, xa, ya, xb, yb, acc, local,
                               d_mu, d_xx, d_xy);
        forward_rows<kFirst, S + 1>(p, win, tl, c, b1, b2, line, base, xa, ya, xb, yb, acc,
                                    local, d_mu, d_xx, d_xy);
    }
}

// Logical workgroup w's waves take units w * kUnitWaves + wave, then every
// gridDim.x * kUnitWaves further; partials[w] = the workgroup's sum of the SSIM
// map over its region pixels (waves in order).
__global__ __launch_bounds__(kThreads) void ssim_forward_kernel(Planes p, Window win,
                                                                 float *__restrict__ d_mu,
                                                                 float *__restrict__ d_xx,
                                                                 float *__restrict__ d_xy,
                                                                 double *__restrict__ partials) {
    __shared__ float4 lines[kUnitWaves][kInX];
    __shared__ double red[kWaves];
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kWave));
    float4 *line = lines[wave];
    const int blk = xcd_block((int)blockIdx.x, (int)gridDim.x);
    double local = 0.0;
    for (int t = blk * kUnitWaves + wave; t < p.tiles;
         t += (int)gridDim.x * kUnitWaves) {
        const Tile tl = tile_of<FwdShape::rows>(p, t);
        const Cols c = cols_of(p, tl);
        const float *b1 = p.img1 + ((int64_t)tl.b * p.s1[0] + (int64_t)tl.c * p.s1[1]);
        const float *b2 = p.img2 + ((int64_t)tl.b * p.s2[0] + (int64_t)tl.c * p.s2[1]);
        float xa[kRing], ya[kRing], xb[kRing], yb[kRing];
        float acc[kRing][4];
#pragma unroll
        for (int r = 0; r < kRing; ++r)
#pragma unroll
            for (int q = 0; q < 4; ++q) acc[r][q] = 0.0f;
#pragma unroll
        for (int d = 0; d < FwdShape::ahead; ++d)
            load_image_row(p, b1, b2, tl.oy - kRadius + d, c, xa[d], ya[d], xb[d], yb[d]);
        forward_rows<true>(p, win, tl, c, b1, b2, line, 0, xa, ya, xb, yb, acc, local, d_mu,
                           d_xx, d_xy);
        for (int base = kRing; base < FwdShape::walk; base += kRing)
            forward_rows<false>(p, win, tl, c, b1, b2, line, base, xa, ya, xb, yb, acc, local,
                                d_mu, d_xx, d_xy);
        // the output row the last input row completed
        forward_out<FwdShape::walk % kRing>(p, tl, FwdShape::walk - kRing, acc, local, d_mu,
                                            d_xx, d_xy);
    }
    const double s = block_sum(local, red);
    if (threadIdx.x == 0) partials[blk] = s;
}

// *mean = (sum of partials, fixed order) * inv_count; NaN for an empty region.
// With loss, also *loss = (1 - lambda) * *other + lambda * (1 - *mean), in
// float as a PyTorch expression of those scalars would round it.
__global__ __launch_bounds__(kThreads) void ssim_mean_kernel(const double *__restrict__ partials,
                                                              int64_t n, double count,
                                                              float *__restrict__ mean,
                                                              const float *__restrict__ other,
                                                              float lambda,
                                                              float *__restrict__ loss) {
    __shared__ double red[kWaves];
    double v = 0.0;
    for (int64_t i = threadIdx.x; i < n; i += kThreads) v += partials[i];
    const double s = block_sum(v, red);
    if (threadIdx.x == 0) {
        const float m = (float)(count > 0.0 ? s / count : __builtin_nan(""));
        *mean = m;
        if (loss) *loss = (1.0f - lambda) * *other + lambda * (1.0f - m);
    }
}

// Backward of one unit: the three maps filtered back the same way; output row
// j's gradient is up * (F[d_mu] + 2 x F[d_xx] + y F[d_xy]) with x, y its pixel
// (loaded BwdShape::ahead rows ahead as well).
struct BwdRows {
    float ma[kRing][3], mb[kRing][3];  // map rows in flight
    float xo[kRing], yo[kRing];        // img1 / img2 at the output row completed `ahead` rows on
};

// Output row j of a backward unit, complete in ring slot kSlot, with its pixel
// in xo / yo slot kPix: its gradient; the slot is then cleared.
template <int kSlot, int kPix>
__device__ __forceinline__ void backward_out(const Planes &p, const Tile &tl, int j,
                                             const BwdRows &r, float (&acc)[kRing][3], float up,
                                             float *bg, int gs2, int gs3) {
    const int gx = tl.ox + (int)(threadIdx.x % kWave);
    float(&a)[3] = acc[kSlot];
    const int gy = tl.oy + j;
    if (j < BwdShape::rows && gy < p.height && gx < p.width) {
        int row = gy;
        asm volatile("" : "+s"(row));  // the address is formed here, not ahead
        const float x = img1_value(p, r.xo[kPix]), y = r.yo[kPix];  // an in-image pixel
        store_at(bg + row * gs2, (uint32_t)gx * (uint32_t)gs3 * 4u,
                 up * (a[0] + 2.0f * x * a[1] + y * a[2]));
    }
#pragma unroll
    for (int q = 0; q < 3; ++q) a[q] = 0.0f;
}

// One input row ri of a backward unit; as in the forward, output row
// ri - 1 - 2 kRadius (complete in slot S, its pixel loaded into slot S - 1) is
// emitted while this row's taps are read.
template <bool kFirst, int S>
__device__ __forceinline__ void backward_row(const Planes &p, const Window &win, const Tile &tl,
                                             const Cols &c, const float *m0, const float *m1,
                                             const float *m2, const float *b1, const float *b2,
                                             float4 *line, int ri, BwdRows &r,
                                             float (&acc)[kRing][3], float up, float *bg,
                                             int gs2, int gs3) {
    const int lane = threadIdx.x % kWave;
    const int64_t base = (int64_t)tl.plane * p.height * p.width;
    constexpr int kNext = (S + BwdShape::ahead) % kRing;
    {  // (rows past the walk load in-image values that are never used)
        load_map_row(p, m0, m1, m2, base, tl.oy - kRadius + ri + BwdShape::ahead, c,
                     r.ma[kNext], r.mb[kNext]);
        // the pixel of the output row that row ri + ahead completes
        load_pixel(p, b1, b2, tl.oy + ri + BwdShape::ahead - 2 * kRadius, c, r.xo[kNext],
                   r.yo[kNext]);
    }
    bool ina, inb;
    row_inside(p, tl.oy - kRadius + ri, c, ina, inb);
    line[lane] = ina ? make_float4(r.ma[S][0], r.ma[S][1], r.ma[S][2], 0.0f)
                     : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (c.has_b)
        line[kWave + lane] = inb ? make_float4(r.mb[S][0], r.mb[S][1], r.mb[S][2], 0.0f)
                                 : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    line_sync();
    f4v v[kTaps];
    read_taps(line, v);
    if constexpr (!kFirst)
        backward_out<S, (S + kRing - 1) % kRing>(p, tl, ri - kRing, r, acc, up, bg, gs2, gs3);
    taps_ready(v);
    float h[3];
    filter_taps<3>(win, v, h);
    line_sync();
    ring_add<3, kFirst, S>(win, ri, h, acc);
}

template <bool kFirst, int S = 0>
__device__ __forceinline__ void backward_rows(const Planes &p, const Window &win, const Tile &tl,
                                              const Cols &c, const float *m0, const float *m1,
                                              const float *m2, const float *b1, const float *b2,
                                              float4 *line, int base, BwdRows &r,
                                              float (&acc)[kRing][3], float up, float *bg,
                                              int gs2, int gs3) {
    if constexpr (S < kRing) {
        backward_row<kFirst, S>(p, win, tl, c, m0, m1, m2, b1, b2, line, base + S, r, acc, up,
                                bg, gs2, gs3);
        backward_rows<kFirst, S + 1>(p, win, tl, c, m0, m1, m2, b1, b2, line, base, r, acc, up,
                                     bg, gs2, gs3);
    }
}

__global__ __launch_bounds__(kThreads) void ssim_backward_kernel(
    Planes p, Window win, const float *__restrict__ grad_mean, const float *__restrict__ d_mu,
    const float *__restrict__ d_xx, const float *__restrict__ d_xy, float *__restrict__ grad,
    int64_t gs0, int64_t gs1, int gs2, int gs3, float grad_scale) {
    __shared__ float4 lines[kUnitWaves][kInX];
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kWave));
    float4 *line = lines[wave];
    const float up = grad_scale * *grad_mean;
    const int blk = xcd_block((int)blockIdx.x, (int)gridDim.x);
    for (int t = blk * kUnitWaves + wave; t < p.tiles;
         t += (int)gridDim.x * kUnitWaves) {
        const Tile tl = tile_of<BwdShape::rows>(p, t);
        const Cols c = cols_of(p, tl);
        const float *b1 = p.img1 + ((int64_t)tl.b * p.s1[0] + (int64_t)tl.c * p.s1[1]);
        const float *b2 = p.img2 + ((int64_t)tl.b * p.s2[0] + (int64_t)tl.c * p.s2[1]);
        float *bg = grad + ((int64_t)tl.b * gs0 + (int64_t)tl.c * gs1);
        const int64_t base = (int64_t)tl.plane * p.height * p.width;
        BwdRows r;
        float acc[kRing][3];
#pragma unroll
        for (int k = 0; k < kRing; ++k)
#pragma unroll
            for (int q = 0; q < 3; ++q) acc[k][q] = 0.0f;
#pragma unroll
        for (int d = 0; d < BwdShape::ahead; ++d) {
            load_map_row(p, d_mu, d_xx, d_xy, base, tl.oy - kRadius + d, c, r.ma[d], r.mb[d]);
            // (row d completes no output row: d < 2 kRadius)
            load_pixel(p, b1, b2, tl.oy + d - 2 * kRadius, c, r.xo[d], r.yo[d]);
        }
        backward_rows<true>(p, win, tl, c, d_mu, d_xx, d_xy, b1, b2, line, 0, r, acc, up, bg,
                            gs2, gs3);
        for (int rb = kRing; rb < BwdShape::walk; rb += kRing)
            backward_rows<false>(p, win, tl, c, d_mu, d_xx, d_xy, b1, b2, line, rb, r, acc, up,
                                 bg, gs2, gs3);
        constexpr int kLast = BwdShape::walk % kRing;  // the last input row's output
        backward_out<kLast, (kLast + kRing - 1) % kRing>(p, tl, BwdShape::walk - kRing, r, acc,
                                                         up, bg, gs2, gs3);
    }
}

// Workgroups: one per kUnitWaves units, at most kMaxBlocks (their waves then
// take several units each).  The count depends on the image geometry alone, so
// the per-workgroup partial sums, and so the mean, do not depend on the device.
constexpr int kMaxBlocks = 1024;

struct Geometry {
    int tiles_x, tiles_y, tiles;
    int blocks;
};

// Units of kRows output rows.
template <int kRows>
bool geometry(int32_t batch, int32_t channels, int32_t height, int32_t width, Geometry &g) {
    if (batch <= 0 || channels <= 0 || height <= 0 || width <= 0) return false;
    const int64_t planes = (int64_t)batch * channels;
    if (planes > 65535) return false;
    g.tiles_x = ceil_div(width, kTileX);
    g.tiles_y = ceil_div(height, kRows);
    const int64_t tiles = planes * g.tiles_x * g.tiles_y;
    if (tiles > 0x7fffffffLL) return false;
    g.tiles = (int)tiles;
    const int per = ceil_div(g.tiles, kUnitWaves);
    g.blocks = per < kMaxBlocks ? per : kMaxBlocks;
    return true;
}

// In-plane offsets are 32-bit: strides must be >= 0, a plane's last element
// offset below 2^31 and a row's last element offset below 2^30 (its byte
// offset, added to a row start, fits 32 bits).
bool plane_fits(const int64_t *s, int32_t height, int32_t width) {
    if (s[0] < 0 || s[1] < 0 || s[2] < 0 || s[3] < 0) return false;
    if (s[3] * (int64_t)(width - 1) >= (1LL << 30)) return false;
    return s[2] * (int64_t)(height - 1) + s[3] * (int64_t)(width - 1) < 0x7fffffffLL;
}

int fill_planes(Planes &p, const Geometry &g, const float *img1, const int64_t *s1,
                const float *img2, const int64_t *s2, int32_t channels, int32_t height,
                int32_t width, int32_t valid) {
    if (!img1 || !img2 || !s1 || !s2) return GS_ERR_INVALID_ARGUMENT;
    if (!plane_fits(s1, height, width) || !plane_fits(s2, height, width) ||
        (int64_t)height * width >= 0x7fffffffLL)
        return GS_ERR_UNSUPPORTED;
    p.img1 = img1;
    p.img2 = img2;
    for (int i = 0; i < 2; ++i) {
        p.s1[i] = s1[i];
        p.s2[i] = s2[i];
    }
    p.r1 = (int)s1[2];
    p.c1 = (int)s1[3];
    p.r2 = (int)s2[2];
    p.c2 = (int)s2[3];
    p.channels = channels;
    p.height = height;
    p.width = width;
    p.tiles_x = g.tiles_x;
    p.tiles_y = g.tiles_y;
    p.tiles = g.tiles;
    p.valid = valid ? 1 : 0;
    p.inv_count = 0.0f;
    p.inv1 = 1.0f;
    return GS_OK;
}

double region_pixels(int32_t batch, int32_t channels, int32_t height, int32_t width,
                     bool valid) {
    const int64_t h = valid ? height - 2 * kRadius : height;
    const int64_t w = valid ? width - 2 * kRadius : width;
    if (h <= 0 || w <= 0) return 0.0;
    return (double)batch * channels * (double)h * (double)w;
}

}  // namespace
}  // namespace gs

using namespace gs;

extern "C" int gs_ssim_workspace_size(int32_t batch, int32_t channels, int32_t height,
                                      int32_t width, size_t *bytes) {
    Geometry g;
    if (!bytes || !geometry<FwdShape::rows>(batch, channels, height, width, g))
        return GS_ERR_INVALID_ARGUMENT;
    *bytes = (size_t)g.blocks * sizeof(double);
    return GS_OK;
}

namespace gs {
namespace {

// gs_ssim_forward with the per-workgroup partials in `partials` (room for
// `capacity` doubles).
int ssim_forward_impl(const float *img1, const int64_t *strides1, const float *img2,
                      const int64_t *strides2, int32_t batch, int32_t channels, int32_t height,
                      int32_t width, int32_t valid_padding, float img1_divisor, float *ssim_mean,
                      float *dm_dmu1, float *dm_dsigma1_sq, float *dm_dsigma12,
                      const float *other_loss, float lambda, float *loss, double *partials,
                      size_t capacity, hipStream_t stream) {
    Geometry g;
    Planes p;
    if (!geometry<FwdShape::rows>(batch, channels, height, width, g) || !ssim_mean ||
        !(img1_divisor > 0.0f))
        return GS_ERR_INVALID_ARGUMENT;
    if (loss && !other_loss) return GS_ERR_INVALID_ARGUMENT;
    int st = fill_planes(p, g, img1, strides1, img2, strides2, channels, height, width,
                         valid_padding);
    if (st) return st;
    p.inv1 = 1.0f / img1_divisor;
    if ((dm_dmu1 != nullptr) != (dm_dsigma1_sq != nullptr) ||
        (dm_dmu1 != nullptr) != (dm_dsigma12 != nullptr))
        return GS_ERR_INVALID_ARGUMENT;
    if (!partials || capacity < (size_t)g.blocks) return GS_ERR_WORKSPACE_TOO_SMALL;
    const double count = region_pixels(batch, channels, height, width, valid_padding != 0);
    p.inv_count = count > 0.0 ? (float)(1.0 / count) : 0.0f;
    hipLaunchKernelGGL(ssim_forward_kernel, dim3(g.blocks), dim3(kThreads), 0, stream, p,
                       make_window(), dm_dmu1, dm_dsigma1_sq, dm_dsigma12, partials);
    st = launch_status();
    if (st) return st;
    hipLaunchKernelGGL(ssim_mean_kernel, dim3(1), dim3(kThreads), 0, stream,
                       (const double *)partials, (int64_t)g.blocks, count, ssim_mean, other_loss,
                       lambda, loss);
    return launch_status();
}

// Scratch of the allocation-free forward: the per-workgroup partials (one
// double per workgroup, at most kMaxBlocks: 8 KiB), in a
// file-scope device array that every GPU the library runs on holds until the
// process ends.  Every forward launch writes all the partials its mean kernel
// reads, so nothing needs clearing between calls; calls that overlap on one GPU
// (different streams) share the array and race.  In host code the array's name
// is not a device address: its address on each device comes from
// hipGetSymbolAddress, taken once per device with that device current.
constexpr int kScratchPartials = kMaxBlocks;
__device__ __align__(256) double scratch[kScratchPartials];

constexpr int kMaxScratchDevices = 64;
std::mutex scratch_mutex;
double *scratch_ptr[kMaxScratchDevices] = {};

// The scratch array's address on the current device, which must be the device
// of `stream`.
int scratch_for_stream(hipStream_t stream, double **out) {
    int dev = -1, stream_dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    e = hipStreamGetDevice(stream, &stream_dev);
    if (e != hipSuccess) return (int)e;
    if (stream_dev != dev) return GS_ERR_INVALID_ARGUMENT;
    if (dev < 0 || dev >= kMaxScratchDevices) return GS_ERR_UNSUPPORTED;
    std::lock_guard<std::mutex> lock(scratch_mutex);
    if (!scratch_ptr[dev]) {
        void *ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return (int)e;
        if (!ptr) return GS_ERR_UNSUPPORTED;
        scratch_ptr[dev] = static_cast<double *>(ptr);
    }
    *out = scratch_ptr[dev];
    return GS_OK;
}

}  // namespace
}  // namespace gs

extern "C" int gs_ssim_forward(const float *img1, const int64_t *strides1, const float *img2,
                               const int64_t *strides2, int32_t batch, int32_t channels,
                               int32_t height, int32_t width, int32_t valid_padding,
                               float img1_divisor, float *ssim_mean, float *dm_dmu1,
                               float *dm_dsigma1_sq, float *dm_dsigma12, const float *other_loss,
                               float lambda, float *loss, void *workspace,
                               size_t workspace_bytes, hipStream_t stream) {
    return ssim_forward_impl(img1, strides1, img2, strides2, batch, channels, height, width,
                             valid_padding, img1_divisor, ssim_mean, dm_dmu1, dm_dsigma1_sq,
                             dm_dsigma12, other_loss, lambda, loss,
                             reinterpret_cast<double *>(workspace),
                             workspace ? workspace_bytes / sizeof(double) : 0, stream);
}

extern "C" int gs_ssim_forward_noalloc(const float *img1, const int64_t *strides1,
                                       const float *img2, const int64_t *strides2, int32_t batch,
                                       int32_t channels, int32_t height, int32_t width,
                                       int32_t valid_padding, float img1_divisor,
                                       float *ssim_mean, float *dm_dmu1, float *dm_dsigma1_sq,
                                       float *dm_dsigma12, const float *other_loss, float lambda,
                                       float *loss, hipStream_t stream) {
    Geometry g;
    if (!geometry<FwdShape::rows>(batch, channels, height, width, g))
        return GS_ERR_INVALID_ARGUMENT;
    // the partials the launch needs must fit the static array (always true:
    // geometry() caps the workgroups at kMaxBlocks)
    if (g.blocks > kScratchPartials) return GS_ERR_WORKSPACE_TOO_SMALL;
    double *partials = nullptr;
    const int st = scratch_for_stream(stream, &partials);
    if (st) return st;
    return ssim_forward_impl(img1, strides1, img2, strides2, batch, channels, height, width,
                             valid_padding, img1_divisor, ssim_mean, dm_dmu1, dm_dsigma1_sq,
                             dm_dsigma12, other_loss, lambda, loss, partials, kScratchPartials,
                             stream);
}

extern "C" int gs_ssim_backward(const float *grad_mean, const float *img1,
                                const int64_t *strides1, const float *img2,
                                const int64_t *strides2, int32_t batch, int32_t channels,
                                int32_t height, int32_t width, float img1_divisor,
                                const float *dm_dmu1, const float *dm_dsigma1_sq,
                                const float *dm_dsigma12, float grad_scale, float *grad_img1,
                                const int64_t *grad_strides, hipStream_t stream) {
    Geometry g;
    Planes p;
    if (!geometry<BwdShape::rows>(batch, channels, height, width, g) || !(img1_divisor > 0.0f))
        return GS_ERR_INVALID_ARGUMENT;
    int st = fill_planes(p, g, img1, strides1, img2, strides2, channels, height, width, 0);
    if (st) return st;
    p.inv1 = 1.0f / img1_divisor;
    if (!grad_mean || !dm_dmu1 || !dm_dsigma1_sq || !dm_dsigma12 || !grad_img1 || !grad_strides)
        return GS_ERR_INVALID_ARGUMENT;
    if (!plane_fits(grad_strides, height, width)) return GS_ERR_UNSUPPORTED;
    hipLaunchKernelGGL(ssim_backward_kernel, dim3(g.blocks), dim3(kThreads), 0, stream, p,
                       make_window(), grad_mean, dm_dmu1, dm_dsigma1_sq, dm_dsigma12, grad_img1,
                       grad_strides[0], grad_strides[1], (int)grad_strides[2],
                       (int)grad_strides[3], grad_scale);
    return launch_status();
}
