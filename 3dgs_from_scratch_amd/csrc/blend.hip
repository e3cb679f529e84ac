// Tile blending: front-to-back alpha compositing and its gradient.
//
// One workgroup per 16x16 tile: 256 threads = 4 wave64s, each wave owning a
// 16x4 strip of pixels (one pixel per lane).  The tile's depth-sorted Gaussian
// list is walked in batches of 256 records staged in LDS; a wave skips a
// Gaussian whose chi-square ellipse misses its strip (uniform branch), and the
// workgroup stops as soon as every pixel's transmittance fell below the
// threshold (__syncthreads_and per batch, per-lane break inside a batch).
//
// Decision quantities (E, alpha, T) are computed with separately rounded ops in
// the Torch rasterizer's order (src/torch_rasterizer.py:255-278) -- this file
// is compiled with -ffp-contract=off -- so inclusion decisions match the CPU
// oracle for identical inputs; accumulations use explicit fmaf.
//
// The backward walks the list in the same front-to-back order.  With
// S_i = sum_{k>i} w_k (g.c_k) = g.C - sum_{k<=i} w_k (g.c_k), where C is the
// pixel's forward colour, dL/dalpha_i = T_i (g.c_i) - S_i / (1 - alpha_i + eps).
// Per-pixel contributions are summed over each wave with a butterfly, the four
// wave partials are combined in LDS, and one float atomic per (tile, Gaussian,
// field) goes to HBM (the reference issues one per pixel: kernel.cu:1098-1106).

#include "gs_common.h"

namespace gs {

constexpr int kTile = 16;
constexpr int kBlendThreads = 256;
constexpr int kBatch = 256;
constexpr int kBlendWaves = kBlendThreads / kWave;
constexpr int kGradFields = 9;  // du, dv, dA, dB, dC, dopacity, dr, dg, db

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

// Front-to-back accumulation of the pixel colour over the tile's list.
// Every thread of the workgroup must call it (it contains barriers).
__device__ __forceinline__ void blend_accumulate(
    BatchLds &s, TileSpan span, const int32_t *__restrict__ ids, int64_t n,
    const float *__restrict__ points, const float *__restrict__ conics,
    const float *__restrict__ opac, const float *__restrict__ colors, float fx, float fy,
    float wx0, float wx1, float wy0, float wy1, bool done, float alpha_thr, float T_thr,
    float chi, float &cr, float &cg, float &cb) {
    float T = 1.0f;
    cr = cg = cb = 0.0f;
    for (int32_t b0 = span.start; b0 < span.end; b0 += kBatch) {
        if (__syncthreads_and(done)) break;
        const int32_t i = b0 + (int32_t)threadIdx.x;
        if (i < span.end)
            stage_record(s, threadIdx.x, ids[i], n, points, conics, opac, colors, chi, alpha_thr);
        __syncthreads();
        const int cnt = min(kBatch, span.end - b0);
        if (!done) {
            for (int j = 0; j < cnt; ++j) {
                const float4 geo = s.geo[j];
                const float4 aux = s.aux[j];
                if (geo.x + aux.z < wx0 || geo.x - aux.z > wx1 || geo.y + aux.w < wy0 ||
                    geo.y - aux.w > wy1)
                    continue;
                const float du = fx - geo.x, dv = fy - geo.y;
                const float E = conic_exponent(geo.z, geo.w, aux.x, du, dv);
                if (!(E < chi)) continue;
                const float alpha = __expf(-0.5f * E) * aux.y;
                if (alpha < alpha_thr) continue;
                const float4 col = s.col[j];
                const float w = alpha * T;
                cr = fmaf(w, col.x, cr);
                cg = fmaf(w, col.y, cg);
                cb = fmaf(w, col.z, cb);
                T = T * ((1.0f - alpha) + kTransmittanceEps);
                if (T < T_thr) {
                    done = true;
                    break;
                }
            }
        }
    }
}

__global__ __launch_bounds__(kBlendThreads) void blend_forward_kernel(
    const int32_t *__restrict__ offsets, const int32_t *__restrict__ ids, int n_tiles,
    int64_t k, int64_t n, const float *__restrict__ points, const float *__restrict__ conics,
    const float *__restrict__ opac, const float *__restrict__ colors, int tiles_x, int width,
    int height, float alpha_thr, float T_thr, float chi, float *__restrict__ image) {
    __shared__ BatchLds s;
    const int tile = blockIdx.x;
    const int tx = tile % tiles_x, ty = tile / tiles_x;
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int px = tx * kTile + (lane & 15);
    const int py = ty * kTile + wave * 4 + (lane >> 4);
    const bool inside = px < width && py < height;
    const float wx0 = (float)(tx * kTile), wx1 = wx0 + (kTile - 1);
    const float wy0 = (float)(ty * kTile + wave * 4), wy1 = wy0 + 3.0f;
    const TileSpan span = tile_span(offsets, n_tiles, k, tile);
    const bool done = !inside || !(1.0f >= T_thr);
    float cr, cg, cb;
    blend_accumulate(s, span, ids, n, points, conics, opac, colors, (float)px, (float)py, wx0,
                     wx1, wy0, wy1, done, alpha_thr, T_thr, chi, cr, cg, cb);
    if (inside) {
        const int64_t o = ((int64_t)py * width + px) * 3;
        image[o] = cr;
        image[o + 1] = cg;
        image[o + 2] = cb;
    }
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o, kWave);
    return x;
}

struct BackLds {
    BatchLds rec;
    float partial[kGradFields][kBlendWaves][kBatch];
};

__global__ __launch_bounds__(kBlendThreads) void blend_backward_kernel(
    const float *__restrict__ grad_image, const float *__restrict__ image,
    const int32_t *__restrict__ offsets, const int32_t *__restrict__ ids, int n_tiles,
    int64_t k, int64_t n, const float *__restrict__ points, const float *__restrict__ conics,
    const float *__restrict__ opac, const float *__restrict__ colors, int tiles_x, int width,
    int height, float alpha_thr, float T_thr, float chi, float *__restrict__ g_points,
    float *__restrict__ g_conics, float *__restrict__ g_opac, float *__restrict__ g_colors) {
    __shared__ BackLds s;
    const int tile = blockIdx.x;
    const int tx = tile % tiles_x, ty = tile / tiles_x;
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int px = tx * kTile + (lane & 15);
    const int py = ty * kTile + wave * 4 + (lane >> 4);
    const bool inside = px < width && py < height;
    const float fx = (float)px, fy = (float)py;
    const float wx0 = (float)(tx * kTile), wx1 = wx0 + (kTile - 1);
    const float wy0 = (float)(ty * kTile + wave * 4), wy1 = wy0 + 3.0f;
    const TileSpan span = tile_span(offsets, n_tiles, k, tile);
    if (span.end <= span.start) return;  // uniform across the workgroup

    float gr = 0.f, gg = 0.f, gb = 0.f, cr = 0.f, cg = 0.f, cb = 0.f;
    const int64_t pix = ((int64_t)py * width + px) * 3;
    if (inside) {
        gr = grad_image[pix];
        gg = grad_image[pix + 1];
        gb = grad_image[pix + 2];
    }
    const bool never = !inside || !(1.0f >= T_thr);
    if (image) {
        if (inside) {
            cr = image[pix];
            cg = image[pix + 1];
            cb = image[pix + 2];
        }
    } else {
        blend_accumulate(s.rec, span, ids, n, points, conics, opac, colors, fx, fy, wx0, wx1,
                         wy0, wy1, never, alpha_thr, T_thr, chi, cr, cg, cb);
    }
    const float gC = gr * cr + gg * cg + gb * cb;
    bool done = never || (gr == 0.0f && gg == 0.0f && gb == 0.0f);
    float T = 1.0f, acc = 0.0f;

    for (int32_t b0 = span.start; b0 < span.end; b0 += kBatch) {
        if (__syncthreads_and(done)) break;
        const int32_t i = b0 + (int32_t)threadIdx.x;
        if (i < span.end)
            stage_record(s.rec, threadIdx.x, ids[i], n, points, conics, opac, colors, chi,
                         alpha_thr);
        {
            float *p = &s.partial[0][0][0];
            for (int q = threadIdx.x; q < kGradFields * kBlendWaves * kBatch; q += kBlendThreads)
                p[q] = 0.0f;
        }
        __syncthreads();
        const int cnt = min(kBatch, span.end - b0);
        for (int j = 0; j < cnt; ++j) {
            if (__ballot(!done) == 0) break;  // whole wave finished
            const float4 geo = s.rec.geo[j];
            const float4 aux = s.rec.aux[j];
            if (geo.x + aux.z < wx0 || geo.x - aux.z > wx1 || geo.y + aux.w < wy0 ||
                geo.y - aux.w > wy1)
                continue;
            float v[kGradFields] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            bool hit = false;
            if (!done) {
                const float du = fx - geo.x, dv = fy - geo.y;
                const float E = conic_exponent(geo.z, geo.w, aux.x, du, dv);
                if (E < chi) {
                    const float G = __expf(-0.5f * E);
                    const float alpha = G * aux.y;
                    if (alpha >= alpha_thr) {
                        hit = true;
                        const float4 col = s.rec.col[j];
                        const float w = alpha * T;
                        const float gcol = fmaf(gr, col.x, fmaf(gg, col.y, gb * col.z));
                        const float acc_new = fmaf(w, gcol, acc);
                        const float suffix = gC - acc_new;
                        const float one_m = (1.0f - alpha) + kTransmittanceEps;
                        const float dalpha = T * gcol - suffix / one_m;
                        const float h = alpha * dalpha;
                        const float B = 0.5f * geo.w;
                        v[0] = h * fmaf(geo.z, du, B * dv);
                        v[1] = h * fmaf(B, du, aux.x * dv);
                        v[2] = -0.5f * h * du * du;
                        v[3] = -h * du * dv;
                        v[4] = -0.5f * h * dv * dv;
                        v[5] = G * dalpha;
                        v[6] = w * gr;
                        v[7] = w * gg;
                        v[8] = w * gb;
                        acc = acc_new;
                        T = T * one_m;
                        if (T < T_thr) done = true;
                    }
                }
            }
            if (__ballot(hit) == 0) continue;
#pragma unroll
            for (int f = 0; f < kGradFields; ++f) {
                const float t = wave_sum(v[f]);
                if (lane == 0) s.partial[f][wave][j] = t;
            }
        }
        __syncthreads();
        for (int q = threadIdx.x; q < kGradFields * cnt; q += kBlendThreads) {
            const int f = q / cnt, j = q % cnt;
            const float t = s.partial[f][0][j] + s.partial[f][1][j] + s.partial[f][2][j] +
                            s.partial[f][3][j];
            if (t != 0.0f) {
                const int g = __float_as_int(s.rec.col[j].w);
                float *dst;
                if (f < 2)
                    dst = g_points + 2 * g + f;
                else if (f < 5)
                    dst = g_conics + 3 * g + (f - 2);
                else if (f == 5)
                    dst = g_opac + g;
                else
                    dst = g_colors + 3 * g + (f - 6);
                unsafeAtomicAdd(dst, t);
            }
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
        hipLaunchKernelGGL(blend_forward_kernel, dim3(n_tiles), dim3(kBlendThreads), 0, stream,
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
    float *grad_cov_inv_image, float *grad_opacities, float *grad_colors, hipStream_t stream) {
    int st = check_blend_args(indexing_offset, gaussian_ids_sorted, n_tiles, k, n, width, height,
                              tile_size);
    if (st) return st;
    if (n > 0 && (!grad_points_image || !grad_cov_inv_image || !grad_opacities || !grad_colors))
        return GS_ERR_INVALID_ARGUMENT;
    if (n > 0) {
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
        hipLaunchKernelGGL(blend_backward_kernel, dim3(n_tiles), dim3(kBlendThreads), 0, stream,
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
