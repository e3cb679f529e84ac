// Tile blending: front-to-back alpha compositing and its gradient.
//
// One wave64 per 16x16 tile.  Lane l owns the four pixels
// (x0 + l%16, y0 + l/16 + 4s), s = 0..3, i.e. one pixel in each 16x4 strip of
// the tile.  The tile's depth-sorted Gaussian list is walked in batches of 64
// records staged in LDS (one record per lane); for each Gaussian the wave tests
// (uniformly) which strips its chi-square ellipse reaches and evaluates only
// those, and it stops once the transmittance of all 256 pixels fell below the
// threshold.  Tiles are assigned to workgroups XCD by XCD (the dispatcher
// places workgroup b on XCD b % 8) so that neighbouring tiles, which share
// Gaussians, run on the same XCD and share its L2.
//
// Decision quantities (E, alpha, T) are computed with separately rounded ops in
// the Torch rasterizer's order (src/torch_rasterizer.py:255-278) -- this file
// is compiled with -ffp-contract=off -- so inclusion decisions match the CPU
// oracle for identical inputs; accumulations use explicit fmaf.
//
// The backward walks the list in the same front-to-back order.  With
// S_i = sum_{k>i} w_k (g.c_k) = g.C - sum_{k<=i} w_k (g.c_k), where C is the
// pixel's forward colour, dL/dalpha_i = T_i (g.c_i) - S_i / (1 - alpha_i + eps).
// A lane sums its four pixels' contributions in registers, the wave reduces the
// nine fields with DPP row butterflies plus two permlane swaps, and lane 0
// issues one float atomic per (tile, Gaussian, field) (the reference issues one
// per pixel: src/cuda/kernel.cu:1098-1106).

#include "gs_common.h"

namespace gs {

constexpr int kTile = 16;
constexpr int kStrips = 4;       // 16x4 strips per tile; one pixel of each per lane
constexpr int kBatch = kWave;    // records staged per batch (one per lane)
constexpr int kGradFields = 9;   // du, dv, dA, dB, dC, dopacity, dr, dg, db
constexpr int kXcds = 8;

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

// Bijection workgroup -> tile giving XCD x the contiguous tile range
// [x*base + min(x, rem), ...) of length base + (x < rem).
__device__ __forceinline__ int tile_of_block(int b, int n_tiles) {
    const int base = n_tiles / kXcds, rem = n_tiles % kXcds;
    const int x = b % kXcds, i = b / kXcds;
    return x * base + min(x, rem) + i;
}

// Conservative half-extents of the ellipse {E < chi_eff} of conic (A, B, C),
// where chi_eff also accounts for alpha >= alpha_thr.  Infinite when the conic
// is not positive definite (no culling).
__device__ __forceinline__ void ellipse_extent(float A, float B, float C, float o, float chi,
                                               float alpha_thr, float &ex, float &ey) {
    float chi_eff = chi;
    if (alpha_thr > 0.0f && o > 0.0f) chi_eff = fminf(chi_eff, 2.0f * logf(o / alpha_thr));
    const float det = A * C - B * B;
    if (det > 0.0f && A > 0.0f && C > 0.0f && isfinite(chi_eff)) {
        const float ce = fmaxf(chi_eff, 0.0f);
        ex = sqrtf(ce * C / det) * 1.01f + 0.01f;
        ey = sqrtf(ce * A / det) * 1.01f + 0.01f;
    } else {
        ex = ey = __builtin_inff();
    }
}

// E = A du^2 + 2B du dv + C dv^2 in the oracle's operation order.
__device__ __forceinline__ float conic_exponent(float A, float B2, float C, float du, float dv) {
    return (A * du * du + B2 * du * dv) + C * dv * dv;
}

struct BatchLds {
    float4 geo[kBatch];  // u, v, A, 2B
    float4 aux[kBatch];  // C, opacity, ex, ey
    float4 col[kBatch];  // r, g, b, (gaussian id bits)
};

// Stages Gaussian g into LDS slot `slot`.  An id outside [0, n) stages a record
// that every wave culls (it contributes nothing).
__device__ __forceinline__ void stage_record(BatchLds &s, int slot, int g, int64_t n,
                                             const float *__restrict__ points,
                                             const float *__restrict__ conics,
                                             const float *__restrict__ opac,
                                             const float *__restrict__ colors, float chi,
                                             float alpha_thr) {
    if (g < 0 || (int64_t)g >= n) {
        const float inf = __builtin_inff();
        s.geo[slot] = make_float4(inf, inf, 0.0f, 0.0f);
        s.aux[slot] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        s.col[slot] = make_float4(0.0f, 0.0f, 0.0f, __int_as_float(0));
        return;
    }
    const float u = points[2 * g], v = points[2 * g + 1];
    const float A = conics[3 * g], B = conics[3 * g + 1], C = conics[3 * g + 2];
    const float o = opac[g];
    float ex, ey;
    ellipse_extent(A, B, C, o, chi, alpha_thr, ex, ey);
    s.geo[slot] = make_float4(u, v, A, B + B);
    s.aux[slot] = make_float4(C, o, ex, ey);
    s.col[slot] = make_float4(colors[3 * g], colors[3 * g + 1], colors[3 * g + 2],
                              __int_as_float(g));
}

// Strips [s_lo, s_hi] of the tile reached by the ellipse of record (geo, aux);
// false when the ellipse misses the tile.  Wave-uniform.
__device__ __forceinline__ bool strip_range(float4 geo, float4 aux, float x0, float y0, int &s_lo,
                                            int &s_hi) {
    if (geo.x + aux.z < x0 || geo.x - aux.z > x0 + (kTile - 1)) return false;
    const float ylo = geo.y - aux.w - y0, yhi = geo.y + aux.w - y0;
    if (yhi < 0.0f || ylo > (float)(kTile - 1)) return false;
    s_lo = ylo <= 0.0f ? 0 : ((int)ylo >> 2);
    s_hi = yhi >= (float)(kTile - 1) ? kStrips - 1 : ((int)yhi >> 2);
    return true;
}

// Pixel geometry of one lane.
struct LanePixels {
    float fx;             // pixel x
    float fy0;            // pixel y of strip 0 (strip s adds 4s)
    float x0, y0;         // tile origin
    bool inside[kStrips];
};

__device__ __forceinline__ LanePixels lane_pixels(int tile, int tiles_x, int width, int height) {
    LanePixels p;
    const int lane = threadIdx.x;
    const int tx = tile % tiles_x, ty = tile / tiles_x;
    const int px = tx * kTile + (lane & 15);
    const int py = ty * kTile + (lane >> 4);
    p.fx = (float)px;
    p.fy0 = (float)py;
    p.x0 = (float)(tx * kTile);
    p.y0 = (float)(ty * kTile);
#pragma unroll
    for (int s = 0; s < kStrips; ++s) p.inside[s] = px < width && py + 4 * s < height;
    return p;
}

__device__ __forceinline__ bool wave_all(bool x) { return __ballot(!x) == 0; }

// Front-to-back accumulation of the lane's four pixels over the tile's list.
// All 64 lanes must call it (it contains barriers).
__device__ __forceinline__ void blend_accumulate(
    BatchLds &s, TileSpan span, const int32_t *__restrict__ ids, int64_t n,
    const float *__restrict__ points, const float *__restrict__ conics,
    const float *__restrict__ opac, const float *__restrict__ colors, const LanePixels &pix,
    float alpha_thr, float T_thr, float chi, float (&cr)[kStrips], float (&cg)[kStrips],
    float (&cb)[kStrips]) {
    float T[kStrips];
    bool dn[kStrips];
#pragma unroll
    for (int q = 0; q < kStrips; ++q) {
        T[q] = 1.0f;
        cr[q] = cg[q] = cb[q] = 0.0f;
        dn[q] = !pix.inside[q] || !(1.0f >= T_thr);
    }
    for (int32_t b0 = span.start; b0 < span.end; b0 += kBatch) {
        if (wave_all(dn[0] && dn[1] && dn[2] && dn[3])) break;
        __syncthreads();  // previous batch fully read before restaging
        const int32_t i = b0 + (int32_t)threadIdx.x;
        if (i < span.end)
            stage_record(s, threadIdx.x, ids[i], n, points, conics, opac, colors, chi, alpha_thr);
        __syncthreads();
        const int cnt = min(kBatch, span.end - b0);
        for (int j = 0; j < cnt; ++j) {
            const float4 geo = s.geo[j];
            const float4 aux = s.aux[j];
            int s_lo, s_hi;
            if (!strip_range(geo, aux, pix.x0, pix.y0, s_lo, s_hi)) continue;
            const float4 col = s.col[j];
            const float du = pix.fx - geo.x;
#pragma unroll
            for (int q = 0; q < kStrips; ++q) {
                if (q < s_lo || q > s_hi) continue;  // uniform
                if (dn[q]) continue;
                const float dv = (pix.fy0 + (float)(4 * q)) - geo.y;
                const float E = conic_exponent(geo.z, geo.w, aux.x, du, dv);
                if (!(E < chi)) continue;
                const float alpha = __expf(-0.5f * E) * aux.y;
                if (alpha < alpha_thr) continue;
                const float w = alpha * T[q];
                cr[q] = fmaf(w, col.x, cr[q]);
                cg[q] = fmaf(w, col.y, cg[q]);
                cb[q] = fmaf(w, col.z, cb[q]);
                T[q] = T[q] * ((1.0f - alpha) + kTransmittanceEps);
                if (T[q] < T_thr) dn[q] = true;
            }
            if ((j & 7) == 7 && wave_all(dn[0] && dn[1] && dn[2] && dn[3])) break;
        }
    }
}

__global__ __launch_bounds__(kWave) void blend_forward_kernel(
    const int32_t *__restrict__ offsets, const int32_t *__restrict__ ids, int n_tiles,
    int64_t k, int64_t n, const float *__restrict__ points, const float *__restrict__ conics,
    const float *__restrict__ opac, const float *__restrict__ colors, int tiles_x, int width,
    int height, float alpha_thr, float T_thr, float chi, float *__restrict__ image) {
    __shared__ BatchLds s;
    const int tile = tile_of_block(blockIdx.x, n_tiles);
    const LanePixels pix = lane_pixels(tile, tiles_x, width, height);
    const TileSpan span = tile_span(offsets, n_tiles, k, tile);
    float cr[kStrips], cg[kStrips], cb[kStrips];
    blend_accumulate(s, span, ids, n, points, conics, opac, colors, pix, alpha_thr, T_thr, chi, cr,
                     cg, cb);
#pragma unroll
    for (int q = 0; q < kStrips; ++q) {
        if (!pix.inside[q]) continue;
        const int64_t o = ((int64_t)(pix.fy0 + 4 * q) * width + (int64_t)pix.fx) * 3;
        image[o] = cr[q];
        image[o + 1] = cg[q];
        image[o + 2] = cb[q];
    }
}

// Sum over the 64 lanes, result in every lane: butterflies inside each 16-lane
// row with DPP (xor 1, xor 2, half-mirror, mirror), then the gfx950 permlane
// swaps exchange rows 0<->1, 2<->3 and halves 0-31 <-> 32-63.
__device__ __forceinline__ float wave_sum(float x) {
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xF, 0xF, false));
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xF, 0xF, false));
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x141, 0xF, 0xF, false));
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x140, 0xF, 0xF, false));
    const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x),
                                                      false, false);
    x = __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
    const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                      false, false);
    return __uint_as_float(r32[0]) + __uint_as_float(r32[1]);
}

__global__ __launch_bounds__(kWave) void blend_backward_kernel(
    const float *__restrict__ grad_image, const float *__restrict__ image,
    const int32_t *__restrict__ offsets, const int32_t *__restrict__ ids, int n_tiles,
    int64_t k, int64_t n, const float *__restrict__ points, const float *__restrict__ conics,
    const float *__restrict__ opac, const float *__restrict__ colors, int tiles_x, int width,
    int height, float alpha_thr, float T_thr, float chi, float *__restrict__ g_points,
    float *__restrict__ g_conics, float *__restrict__ g_opac, float *__restrict__ g_colors) {
    __shared__ BatchLds s;
    const int tile = tile_of_block(blockIdx.x, n_tiles);
    const LanePixels pix = lane_pixels(tile, tiles_x, width, height);
    const TileSpan span = tile_span(offsets, n_tiles, k, tile);
    if (span.end <= span.start) return;  // uniform across the workgroup

    float gr[kStrips], gg[kStrips], gb[kStrips], gC[kStrips], T[kStrips], acc[kStrips];
    bool dn[kStrips];
    float cr[kStrips], cg[kStrips], cb[kStrips];
    if (!image)
        blend_accumulate(s, span, ids, n, points, conics, opac, colors, pix, alpha_thr, T_thr,
                         chi, cr, cg, cb);
#pragma unroll
    for (int q = 0; q < kStrips; ++q) {
        gr[q] = gg[q] = gb[q] = 0.0f;
        if (pix.inside[q]) {
            const int64_t o = ((int64_t)(pix.fy0 + 4 * q) * width + (int64_t)pix.fx) * 3;
            gr[q] = grad_image[o];
            gg[q] = grad_image[o + 1];
            gb[q] = grad_image[o + 2];
            if (image) {
                cr[q] = image[o];
                cg[q] = image[o + 1];
                cb[q] = image[o + 2];
            }
        } else {
            cr[q] = cg[q] = cb[q] = 0.0f;
        }
        gC[q] = gr[q] * cr[q] + gg[q] * cg[q] + gb[q] * cb[q];
        T[q] = 1.0f;
        acc[q] = 0.0f;
        dn[q] = !pix.inside[q] || !(1.0f >= T_thr) ||
                (gr[q] == 0.0f && gg[q] == 0.0f && gb[q] == 0.0f);
    }

    for (int32_t b0 = span.start; b0 < span.end; b0 += kBatch) {
        if (wave_all(dn[0] && dn[1] && dn[2] && dn[3])) break;
        __syncthreads();
        const int32_t i = b0 + (int32_t)threadIdx.x;
        if (i < span.end)
            stage_record(s, threadIdx.x, ids[i], n, points, conics, opac, colors, chi, alpha_thr);
        __syncthreads();
        const int cnt = min(kBatch, span.end - b0);
        for (int j = 0; j < cnt; ++j) {
            const float4 geo = s.geo[j];
            const float4 aux = s.aux[j];
            int s_lo, s_hi;
            if (!strip_range(geo, aux, pix.x0, pix.y0, s_lo, s_hi)) continue;
            const float4 col = s.col[j];
            const float du = pix.fx - geo.x;
            const float B = 0.5f * geo.w;
            float v[kGradFields] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            bool hit = false;
#pragma unroll
            for (int q = 0; q < kStrips; ++q) {
                if (q < s_lo || q > s_hi) continue;  // uniform
                if (dn[q]) continue;
                const float dv = (pix.fy0 + (float)(4 * q)) - geo.y;
                const float E = conic_exponent(geo.z, geo.w, aux.x, du, dv);
                if (!(E < chi)) continue;
                const float G = __expf(-0.5f * E);
                const float alpha = G * aux.y;
                if (alpha < alpha_thr) continue;
                hit = true;
                const float w = alpha * T[q];
                const float gcol = fmaf(gr[q], col.x, fmaf(gg[q], col.y, gb[q] * col.z));
                const float acc_new = fmaf(w, gcol, acc[q]);
                const float one_m = (1.0f - alpha) + kTransmittanceEps;
                const float dalpha = T[q] * gcol - (gC[q] - acc_new) / one_m;
                const float h = alpha * dalpha;
                const float hdu = h * du, hdv = h * dv;
                v[0] += hdu;
                v[1] += hdv;
                v[2] = fmaf(hdu, du, v[2]);
                v[3] = fmaf(hdu, dv, v[3]);
                v[4] = fmaf(hdv, dv, v[4]);
                v[5] = fmaf(G, dalpha, v[5]);
                v[6] = fmaf(w, gr[q], v[6]);
                v[7] = fmaf(w, gg[q], v[7]);
                v[8] = fmaf(w, gb[q], v[8]);
                acc[q] = acc_new;
                T[q] = T[q] * one_m;
                if (T[q] < T_thr) dn[q] = true;
            }
            if (__ballot(hit) != 0) {
#pragma unroll
                for (int f = 0; f < kGradFields; ++f) v[f] = wave_sum(v[f]);
                if (threadIdx.x == 0) {
                    const int g = __float_as_int(col.w);
                    // dE/du = -2(A du + B dv): sum h (A du + B dv) = A sum h du + B sum h dv
                    unsafeAtomicAdd(g_points + 2 * g, fmaf(geo.z, v[0], B * v[1]));
                    unsafeAtomicAdd(g_points + 2 * g + 1, fmaf(B, v[0], aux.x * v[1]));
                    unsafeAtomicAdd(g_conics + 3 * g, -0.5f * v[2]);
                    unsafeAtomicAdd(g_conics + 3 * g + 1, -v[3]);
                    unsafeAtomicAdd(g_conics + 3 * g + 2, -0.5f * v[4]);
                    unsafeAtomicAdd(g_opac + g, v[5]);
                    unsafeAtomicAdd(g_colors + 3 * g, v[6]);
                    unsafeAtomicAdd(g_colors + 3 * g + 1, v[7]);
                    unsafeAtomicAdd(g_colors + 3 * g + 2, v[8]);
                }
            }
            if ((j & 7) == 7 && wave_all(dn[0] && dn[1] && dn[2] && dn[3])) break;
        }
    }
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
                            int32_t tile_size) {
    if (n < 0 || k < 0 || n_tiles < 0 || width <= 0 || height <= 0 || tile_size <= 0)
        return GS_ERR_INVALID_ARGUMENT;
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

extern "C" int gs_rasterize(const int32_t *indexing_offset, const int32_t *gaussian_ids_sorted,
                            int32_t n_tiles, int64_t k, const float *points_image,
                            const float *cov_inv_image, const float *opacities,
                            const float *colors, int64_t n, int32_t width, int32_t height,
                            int32_t tile_size, float alpha_threshold,
                            float transmittance_threshold, float chi_squared_threshold,
                            float *image, hipStream_t stream) {
    int st = check_blend_args(indexing_offset, gaussian_ids_sorted, n_tiles, k, n, width, height,
                              tile_size);
    if (st) return st;
    if (!image) return GS_ERR_INVALID_ARGUMENT;
    const int tiles_x = (width + tile_size - 1) / tile_size;
    const int tiles_y = (height + tile_size - 1) / tile_size;
    if (n_tiles < tiles_x * tiles_y) {
        // pixels of tiles without an offset entry stay zero (the reference zero-initialises)
        st = zero_bytes(image, (size_t)width * height * 3 * sizeof(float), stream);
        if (st) return st;
    }
    if (n_tiles == 0) return GS_OK;
    if (k > 0 && (!points_image || !cov_inv_image || !opacities || !colors))
        return GS_ERR_INVALID_ARGUMENT;
    if (tile_size == kTile) {
        hipLaunchKernelGGL(blend_forward_kernel, dim3(n_tiles), dim3(kWave), 0, stream,
                           indexing_offset, gaussian_ids_sorted, n_tiles, k, n, points_image,
                           cov_inv_image, opacities, colors, tiles_x, width, height,
                           alpha_threshold, transmittance_threshold, chi_squared_threshold,
                           image);
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

extern "C" int gs_rasterize_backward(
    const float *grad_image, const float *image, const int32_t *indexing_offset,
    const int32_t *gaussian_ids_sorted, int32_t n_tiles, int64_t k, const float *points_image,
    const float *cov_inv_image, const float *opacities, const float *colors, int64_t n,
    int32_t width, int32_t height, int32_t tile_size, float alpha_threshold,
    float transmittance_threshold, float chi_squared_threshold, float *grad_points_image,
    float *grad_cov_inv_image, float *grad_opacities, float *grad_colors, int32_t accumulate,
    hipStream_t stream) {
    int st = check_blend_args(indexing_offset, gaussian_ids_sorted, n_tiles, k, n, width, height,
                              tile_size);
    if (st) return st;
    if (n > 0 && (!grad_points_image || !grad_cov_inv_image || !grad_opacities || !grad_colors))
        return GS_ERR_INVALID_ARGUMENT;
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
        hipLaunchKernelGGL(blend_backward_kernel, dim3(n_tiles), dim3(kWave), 0, stream,
                           grad_image, image, indexing_offset, gaussian_ids_sorted, n_tiles, k,
                           n, points_image, cov_inv_image, opacities, colors, tiles_x, width, height,
                           alpha_threshold, transmittance_threshold, chi_squared_threshold,
                           grad_points_image, grad_cov_inv_image, grad_opacities, grad_colors);
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

extern "C" int gs_rasterize_work(const int32_t *indexing_offset,
                                 const int32_t *gaussian_ids_sorted, int32_t n_tiles, int64_t k,
                                 const float *points_image, const float *cov_inv_image,
                                 const float *opacities, int64_t n, int32_t width, int32_t height,
                                 int32_t tile_size, float alpha_threshold,
                                 float transmittance_threshold, float chi_squared_threshold,
                                 uint64_t *visited, uint64_t *composited, hipStream_t stream) {
    int st = check_blend_args(indexing_offset, gaussian_ids_sorted, n_tiles, k, n, width, height,
                              tile_size);
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
