// Preprocess kernels: projection and spherical harmonics, forward and backward.
// One thread per Gaussian; the C entry points mirror the reference extension's
// project_points / project_points_backward / evaluate_spherical_harmonics(_backward)
// (src/cuda/rasterizer.cpp:140-290).
//
// Compiled with -ffp-contract=off: see preprocess_math.h.

#include "preprocess_math.h"

namespace gs {

constexpr int kPreBlock = 256;

__global__ __launch_bounds__(kPreBlock) void project_points_kernel(
    int64_t n, const float *__restrict__ means, const float *__restrict__ scales,
    const float *__restrict__ quats, const float *__restrict__ opacities,
    const float *__restrict__ w2c, const float *__restrict__ K, float near_plane,
    float far_plane, float min_opacity, float min_radius, float max_radius, int width,
    int height, float *__restrict__ points_image, float *__restrict__ depths,
    float *__restrict__ cov_image, float *__restrict__ cov_inv_image,
    float *__restrict__ radii, uint8_t *__restrict__ mask) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const Camera cam = load_camera(w2c, K, width, height);
    const Projection p = project_gaussian(
        cam, means[3 * i], means[3 * i + 1], means[3 * i + 2], scales[3 * i],
        scales[3 * i + 1], scales[3 * i + 2], quats[4 * i], quats[4 * i + 1], quats[4 * i + 2],
        quats[4 * i + 3], opacities[i], near_plane, far_plane, min_opacity, min_radius,
        max_radius, width, height);
    points_image[2 * i] = p.u;
    points_image[2 * i + 1] = p.v;
    depths[i] = p.keep ? p.zc : 0.0f;
    cov_image[3 * i] = p.a;
    cov_image[3 * i + 1] = p.b;
    cov_image[3 * i + 2] = p.c;
    cov_inv_image[3 * i] = p.A;
    cov_inv_image[3 * i + 1] = p.B;
    cov_inv_image[3 * i + 2] = p.C;
    radii[2 * i] = p.ru;
    radii[2 * i + 1] = p.rv;
    mask[i] = p.keep ? 1 : 0;
}

__global__ __launch_bounds__(kPreBlock) void project_points_backward_kernel(
    int64_t n, const float *__restrict__ grad_points_image,
    const float *__restrict__ grad_cov_inv, const float *__restrict__ means,
    const float *__restrict__ scales, const float *__restrict__ quats,
    const float *__restrict__ w2c, const float *__restrict__ K, int width, int height,
    const float *__restrict__ cov_image, const uint8_t *__restrict__ mask,
    float *__restrict__ grad_means, float *__restrict__ grad_scales,
    float *__restrict__ grad_quats) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float gp[3] = {0.f, 0.f, 0.f}, gs_[3] = {0.f, 0.f, 0.f}, gq[4] = {0.f, 0.f, 0.f, 0.f};
    if (mask[i]) {
        const Camera cam = load_camera(w2c, K, width, height);
        project_gaussian_backward(
            cam, means[3 * i], means[3 * i + 1], means[3 * i + 2], scales[3 * i],
            scales[3 * i + 1], scales[3 * i + 2], quats[4 * i], quats[4 * i + 1],
            quats[4 * i + 2], quats[4 * i + 3], cov_image[3 * i], cov_image[3 * i + 1],
            cov_image[3 * i + 2], grad_points_image[2 * i], grad_points_image[2 * i + 1],
            grad_cov_inv[3 * i], grad_cov_inv[3 * i + 1], grad_cov_inv[3 * i + 2], gp[0], gp[1],
            gp[2], gs_[0], gs_[1], gs_[2], gq[0], gq[1], gq[2], gq[3]);
    }
    grad_means[3 * i] = gp[0];
    grad_means[3 * i + 1] = gp[1];
    grad_means[3 * i + 2] = gp[2];
    grad_scales[3 * i] = gs_[0];
    grad_scales[3 * i + 1] = gs_[1];
    grad_scales[3 * i + 2] = gs_[2];
    grad_quats[4 * i] = gq[0];
    grad_quats[4 * i + 1] = gq[1];
    grad_quats[4 * i + 2] = gq[2];
    grad_quats[4 * i + 3] = gq[3];
}

// ---------------------------------------------------------------- SH
// SH evaluation (src/gaussian.py:24-61; data flow of src/cuda/kernel.cu:545-617)
// and its gradient (src/cuda/kernel.cu:619-782), one thread per Gaussian.  The
// backward moves the kShBlock sh_rest rows of its block (45 floats each,
// 180 B) between HBM and LDS with coalesced 16-byte accesses and reads /
// writes them per Gaussian in LDS, so each gradient line is written once
// (per-thread 180-byte row stores write partially filled lines, measured at
// 1.5x the gradient's bytes).  The forward only loads its rows and reads them
// directly (measured faster than staging).
//
// Output modes: kShRaw (the API's raw sum), kShSigmoid (its sigmoid) and
// kShRender (max(raw + 0.5, 0) as render() applies it, src/cuda/wrapper.py:264-265;
// masked rows are then 0.5, as 0 + 0.5 is in the reference).  The camera
// position is either given or computed as -R^T t from world_to_camera.

constexpr int kShBlock = 128;
constexpr int kRest = 45;
enum ShMode { kShRaw = 0, kShSigmoid = 1, kShRender = 2 };

__device__ __forceinline__ void camera_position(const float *__restrict__ cam_pos,
                                                const float *__restrict__ w2c, float &cx,
                                                float &cy, float &cz) {
    if (cam_pos) {
        cx = cam_pos[0];
        cy = cam_pos[1];
        cz = cam_pos[2];
    } else {  // -R^T t, R = rows 0..2 / cols 0..2, t = column 3 (row-major 4x4)
        cx = -(w2c[0] * w2c[3] + w2c[4] * w2c[7] + w2c[8] * w2c[11]);
        cy = -(w2c[1] * w2c[3] + w2c[5] * w2c[7] + w2c[9] * w2c[11]);
        cz = -(w2c[2] * w2c[3] + w2c[6] * w2c[7] + w2c[10] * w2c[11]);
    }
}

// Copies `count` (<= kShBlock * kRest) floats between global memory and LDS with
// the block's threads: every thread issues all its loads before its stores (a
// fully unrolled register stage), 16 bytes per access when the global side is
// 16-byte aligned.  With `rows` (LDS, one flag per kRest-float row), a float4
// whose rows all have flag 0 is not read (its LDS slots get zeros): culled
// Gaussians' SH rows never reach the GPU's caches.
template <bool kToLds>
__device__ __forceinline__ void block_copy(float *__restrict__ lds, float *__restrict__ glob,
                                           int count, const uint8_t *rows = nullptr) {
    constexpr int kMax4 = kShBlock * kRest / 4;
    constexpr int kIters = (kMax4 + kShBlock - 1) / kShBlock;
    static_assert(kShBlock * kRest % 4 == 0, "rows of a block must fill whole float4s");
    const int tid = threadIdx.x;  // count >= kRest, so n4 >= 11 below
    float *src = kToLds ? glob : lds;
    float *dst = kToLds ? lds : glob;
    if ((reinterpret_cast<uintptr_t>(glob) & 15) == 0) {
        const int n4 = count >> 2;
        const float4 *s4 = reinterpret_cast<const float4 *>(src);
        float4 *d4 = reinterpret_cast<float4 *>(dst);
        float4 v[kIters];
#pragma unroll
        for (int it = 0; it < kIters; ++it) {  // clamped loads stay in registers
            const int e = min(tid + it * kShBlock, n4 - 1);
            const bool need = !rows || (rows[(4 * e) / kRest] | rows[(4 * e + 3) / kRest]);
            v[it] = need ? s4[e] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int it = 0; it < kIters; ++it) {
            const int i = tid + it * kShBlock;
            if (i < n4) d4[i] = v[it];
        }
        for (int i = (n4 << 2) + tid; i < count; i += kShBlock) dst[i] = src[i];
    } else {  // misaligned caller view: plain loop
        for (int i = tid; i < count; i += kShBlock) dst[i] = src[i];
    }
}

// View direction of a Gaussian at `mean` from the camera centre (cx, cy, cz)
// and the 15 basis values of degrees 1..3 along it.
struct ShView {
    float x, y, z, norm;
    float b[15];
};

__device__ __forceinline__ ShView sh_view(const float *__restrict__ mean, float cx, float cy,
                                          float cz) {
    ShView v;
    const float dx = mean[0] - cx;
    const float dy = mean[1] - cy;
    const float dz = mean[2] - cz;
    v.norm = sqrtf(dx * dx + dy * dy + dz * dz);
    v.x = dx / v.norm;
    v.y = dy / v.norm;
    v.z = dz / v.norm;
    sh_basis_rest(v.x, v.y, v.z, v.b);
    return v;
}

// Raw colour channel c: C0 dc + sum_k b_k rest_k (rest: 15 x 3 floats).
__device__ __forceinline__ float sh_raw_channel(const ShView &v, const float *__restrict__ dc,
                                                const float *rest, int c) {
    float acc = kShC0 * dc[c];
#pragma unroll
    for (int k = 0; k < 15; ++k) acc += v.b[k] * rest[3 * k + c];
    return acc;
}

// render() colour: max(raw + 0.5, 0) keeping NaN (src/cuda/wrapper.py:264-265).
__device__ __forceinline__ float sh_render_value(float raw) {
    const float v = raw + 0.5f;
    return v < 0.0f ? 0.0f : v;
}

// d raw_c / d mean for the three channels, through the view direction:
// m[c] = (J_c - dir (dir . J_c)) / |d| with J_c = sum_k rest_kc d b_k / d dir
// (dir = d / |d| has the Jacobian (I - dir dir^T) / |d|).  `rest`: 15 x 3.
// Every path that needs the means' colour gradient forms it from these rows
// (sh_mean_grad), in the forward's cache or in the backward, so that the
// cached and the uncached backward agree bit for bit.
// Basis functions whose derivative along x, y or z is identically zero (bit k):
// their terms are left out of J (they would add r * 0).
constexpr uint32_t kShZeroDx = (1u << 0) | (1u << 1) | (1u << 4) | (1u << 5);
constexpr uint32_t kShZeroDy = (1u << 1) | (1u << 2) | (1u << 5) | (1u << 6);
constexpr uint32_t kShZeroDz = (1u << 0) | (1u << 2) | (1u << 3) | (1u << 7) | (1u << 8) |
                               (1u << 14);

__device__ __forceinline__ void sh_mean_rows(const ShView &v, const float *rest,
                                             float (&m)[3][3]) {
    float bx[15], by[15], bz[15];
    sh_basis_rest_grad(v.x, v.y, v.z, bx, by, bz);
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        float jx = 0.f, jy = 0.f, jz = 0.f;
#pragma unroll
        for (int k = 0; k < 15; ++k) {
            const float r = rest[3 * k + c];
            if (!((kShZeroDx >> k) & 1u)) jx += r * bx[k];
            if (!((kShZeroDy >> k) & 1u)) jy += r * by[k];
            if (!((kShZeroDz >> k) & 1u)) jz += r * bz[k];
        }
        const float dot = v.x * jx + v.y * jy + v.z * jz;
        m[c][0] = (jx - v.x * dot) / v.norm;
        m[c][1] = (jy - v.y * dot) / v.norm;
        m[c][2] = (jz - v.z * dot) / v.norm;
    }
}

// The means gradient of the colour gradient g: sum_c g_c m[c].
__device__ __forceinline__ void sh_mean_grad(const float (&m)[3][3], const float (&g)[3],
                                             float (&gm)[3]) {
#pragma unroll
    for (int d = 0; d < 3; ++d) gm[d] = g[0] * m[0][d] + g[1] * m[1][d] + g[2] * m[2][d];
}

// Gradient of the raw colour g (3 channels) into one Gaussian's SH row: the
// row `lrest` (15 x 3, read in full first) is overwritten with its gradient
// b_k g_c, gdc receives the DC gradient and gm the gradient of the mean through
// the view direction.
__device__ __forceinline__ void sh_backward_row(const ShView &v, const float (&g)[3], float *lrest,
                                                float (&gdc)[3], float (&gm)[3]) {
    float m[3][3];
    sh_mean_rows(v, lrest, m);
    sh_mean_grad(m, g, gm);
#pragma unroll
    for (int c = 0; c < 3; ++c) gdc[c] = kShC0 * g[c];
#pragma unroll
    for (int k = 0; k < 15; ++k) {
        lrest[3 * k] = v.b[k] * g[0];
        lrest[3 * k + 1] = v.b[k] * g[1];
        lrest[3 * k + 2] = v.b[k] * g[2];
    }
}

// Colour-gradient cache of one Gaussian, written where the forward computes its
// render() colour so that the backward need not read the 45-float SH row again:
// kShCache floats per Gaussian (rows 8-byte aligned), [0, 9) the rows m of
// sh_mean_rows, [9] the clamp's pass bits as a uint32 (bit c set where
// raw_c + 0.5 >= 0, the condition under which max(raw_c + 0.5, 0) passes the
// gradient).  Rows of Gaussians outside the mask are not written.
constexpr int kShCache = 10;

__device__ __forceinline__ uint32_t sh_pass_bits(const float (&raw)[3]) {
    return (raw[0] + 0.5f >= 0.0f ? 1u : 0u) | (raw[1] + 0.5f >= 0.0f ? 2u : 0u) |
           (raw[2] + 0.5f >= 0.0f ? 4u : 0u);
}

__device__ __forceinline__ void sh_cache_store(float *__restrict__ cache, int64_t i,
                                               const ShView &v, const float *rest,
                                               const float (&raw)[3]) {
    float m[3][3];
    sh_mean_rows(v, rest, m);
    float2 *row = reinterpret_cast<float2 *>(cache + kShCache * i);
    row[0] = make_float2(m[0][0], m[0][1]);
    row[1] = make_float2(m[0][2], m[1][0]);
    row[2] = make_float2(m[1][1], m[1][2]);
    row[3] = make_float2(m[2][0], m[2][1]);
    row[4] = make_float2(m[2][2], __uint_as_float(sh_pass_bits(raw)));  // bits moved, never computed on
}

__device__ __forceinline__ uint32_t sh_cache_load(const float *__restrict__ cache, int64_t i,
                                                  float (&m)[3][3]) {
    const float2 *row = reinterpret_cast<const float2 *>(cache + kShCache * i);
    const float2 r0 = row[0], r1 = row[1], r2 = row[2], r3 = row[3], r4 = row[4];
    m[0][0] = r0.x;
    m[0][1] = r0.y;
    m[0][2] = r1.x;
    m[1][0] = r1.y;
    m[1][1] = r2.x;
    m[1][2] = r2.y;
    m[2][0] = r3.x;
    m[2][1] = r3.y;
    m[2][2] = r4.x;
    return __float_as_uint(r4.y);
}

__global__ __launch_bounds__(kShBlock) void sh_forward_kernel(
    int64_t n, const float *__restrict__ cam_pos, const float *__restrict__ w2c,
    const float *__restrict__ means, const float *__restrict__ sh_dc,
    const float *__restrict__ sh_rest, const uint8_t *__restrict__ mask, int mode,
    float *__restrict__ colors, float *__restrict__ cache) {
    // one Gaussian per thread; a grid smaller than that walks the rest in strides
    for (int64_t i = (int64_t)blockIdx.x * kShBlock + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * kShBlock) {
        float rgb[3] = {0.f, 0.f, 0.f};
        if (mask[i]) {
            float cx, cy, cz;
            camera_position(cam_pos, w2c, cx, cy, cz);
            const ShView v = sh_view(means + 3 * i, cx, cy, cz);
            const float *rest = sh_rest + kRest * i;  // 15 x 12-byte loads per thread
#pragma unroll
            for (int c = 0; c < 3; ++c) rgb[c] = sh_raw_channel(v, sh_dc + 3 * i, rest, c);
            if (cache) sh_cache_store(cache, i, v, rest, rgb);  // kShRender only
        }
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            float v = rgb[c];
            if (mode == kShSigmoid && mask[i]) v = 1.0f / (1.0f + expf(-v));
            if (mode == kShRender) v = sh_render_value(v);
            colors[3 * i + c] = v;
        }
    }
}

__global__ __launch_bounds__(kShBlock) void sh_backward_kernel(
    int64_t n, const float *__restrict__ grad_colors, const float *__restrict__ cam_pos,
    const float *__restrict__ w2c, const float *__restrict__ means,
    const float *__restrict__ sh_dc, const float *__restrict__ sh_rest,
    const float *__restrict__ colors, const uint8_t *__restrict__ mask, int mode,
    int accumulate_means, float *__restrict__ grad_means, float *__restrict__ grad_dc,
    float *__restrict__ grad_rest) {
    __shared__ __align__(16) float rest_lds[kShBlock * kRest];
    __shared__ uint8_t keep[kShBlock];
    const int64_t first = (int64_t)blockIdx.x * kShBlock;
    const int nb = (int)min((int64_t)kShBlock, n - first);
    keep[threadIdx.x] = threadIdx.x < nb ? mask[first + threadIdx.x] : 0;
    __syncthreads();
    block_copy<true>(rest_lds, const_cast<float *>(sh_rest) + kRest * first, kRest * nb, keep);
    __syncthreads();
    const int t = threadIdx.x;
    float *lrest = rest_lds + kRest * t;  // row read in full below, then overwritten by its gradient
    if (t < nb) {
        const int64_t i = first + t;
        float gm[3] = {0.f, 0.f, 0.f}, gdc[3] = {0.f, 0.f, 0.f};
        if (mask[i]) {
            float cx, cy, cz;
            camera_position(cam_pos, w2c, cx, cy, cz);
            const ShView v = sh_view(means + 3 * i, cx, cy, cz);
            float g[3];
#pragma unroll
            for (int c = 0; c < 3; ++c) {
                g[c] = grad_colors[3 * i + c];
                if (mode == kShSigmoid) {
                    const float s = colors[3 * i + c];
                    g[c] *= s * (1.0f - s);
                } else if (mode == kShRender) {
                    // clamp_min(raw + 0.5, 0) passes the gradient where raw + 0.5 >= 0
                    const float raw = sh_raw_channel(v, sh_dc + 3 * i, lrest, c);
                    if (!(raw + 0.5f >= 0.0f)) g[c] = 0.0f;
                }
            }
            sh_backward_row(v, g, lrest, gdc, gm);
        } else {
#pragma unroll
            for (int k = 0; k < kRest; ++k) lrest[k] = 0.0f;
        }
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            grad_means[3 * i + c] = accumulate_means ? grad_means[3 * i + c] + gm[c] : gm[c];
            grad_dc[3 * i + c] = gdc[c];
        }
    }
    __syncthreads();
    block_copy<false>(rest_lds, grad_rest + kRest * first, kRest * nb);
}

// ------------------------------------------------------------- activations
// scripts/train.py:135-143: scales = exp(log_scales), quats = q / max(|q|, 1e-12),
// opacities = sigmoid(logits).

struct Activated {
    float s[3];
    float4 qraw;  // the raw quaternion
    float qn;     // |qraw|
    float q[4];   // the unit quaternion
    float o;      // opacity
};

__device__ __forceinline__ Activated activate_one(const float *__restrict__ log_scales,
                                                  const float *__restrict__ quats_raw,
                                                  const float *__restrict__ logits, int64_t i) {
    Activated a;
#pragma unroll
    for (int c = 0; c < 3; ++c) a.s[c] = expf(log_scales[3 * i + c]);
    const float4 q = reinterpret_cast<const float4 *>(quats_raw)[i];
    a.qraw = q;
    a.qn = sqrtf(q.x * q.x + q.y * q.y + q.z * q.z + q.w * q.w);
    const float r = a.qn < 1e-12f ? 1e-12f : a.qn;  // clamp_min(1e-12)
    a.q[0] = q.x / r;
    a.q[1] = q.y / r;
    a.q[2] = q.z / r;
    a.q[3] = q.w / r;
    a.o = 1.0f / (1.0f + expf(-logits[i]));
    return a;
}

// Gradients of (scales, unit quaternion, opacity) mapped to (log-scales, raw
// quaternion, logit).
__device__ __forceinline__ void activate_backward_one(const Activated &a, const float (&gs)[3],
                                                      float4 g, float go, float (&g_ls)[3],
                                                      float4 &g_qr, float &g_logit) {
#pragma unroll
    for (int c = 0; c < 3; ++c) g_ls[c] = gs[c] * a.s[c];
    const float4 q = a.qraw;
    const float norm = a.qn;
    if (norm < 1e-12f) {  // the clamp holds the divisor constant
        g_qr = make_float4(g.x / 1e-12f, g.y / 1e-12f, g.z / 1e-12f, g.w / 1e-12f);
    } else {  // d(q/|q|) = (g - qhat (qhat . g)) / |q|
        const float hx = q.x / norm, hy = q.y / norm, hz = q.z / norm, hw = q.w / norm;
        const float dot = hx * g.x + hy * g.y + hz * g.z + hw * g.w;
        g_qr = make_float4((g.x - hx * dot) / norm, (g.y - hy * dot) / norm,
                           (g.z - hz * dot) / norm, (g.w - hw * dot) / norm);
    }
    g_logit = go * (a.o * (1.0f - a.o));
}

__global__ __launch_bounds__(256) void activate_kernel(int64_t n,
                                                      const float *__restrict__ log_scales,
                                                      const float *__restrict__ quats_raw,
                                                      const float *__restrict__ logits,
                                                      float *__restrict__ scales,
                                                      float *__restrict__ quats,
                                                      float *__restrict__ opac) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const Activated a = activate_one(log_scales, quats_raw, logits, i);
#pragma unroll
    for (int c = 0; c < 3; ++c) scales[3 * i + c] = a.s[c];
    reinterpret_cast<float4 *>(quats)[i] = make_float4(a.q[0], a.q[1], a.q[2], a.q[3]);
    opac[i] = a.o;
}

// Gradients of activate_kernel's outputs mapped to its inputs; a null gradient
// input counts as zero.  Scales and opacities are the forward's outputs.
__global__ __launch_bounds__(256) void activate_backward_kernel(
    int64_t n, const float *__restrict__ grad_scales, const float *__restrict__ grad_quats,
    const float *__restrict__ grad_opac, const float *__restrict__ scales,
    const float *__restrict__ quats_raw, const float *__restrict__ opac,
    float *__restrict__ grad_log_scales, float *__restrict__ grad_quats_raw,
    float *__restrict__ grad_logits) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    Activated a;
#pragma unroll
    for (int c = 0; c < 3; ++c) a.s[c] = scales[3 * i + c];
    a.qraw = reinterpret_cast<const float4 *>(quats_raw)[i];
    a.qn = sqrtf(a.qraw.x * a.qraw.x + a.qraw.y * a.qraw.y + a.qraw.z * a.qraw.z +
                 a.qraw.w * a.qraw.w);
    a.o = opac[i];
    float gs[3];
#pragma unroll
    for (int c = 0; c < 3; ++c) gs[c] = grad_scales ? grad_scales[3 * i + c] : 0.0f;
    const float4 g = grad_quats ? reinterpret_cast<const float4 *>(grad_quats)[i]
                                : make_float4(0.f, 0.f, 0.f, 0.f);
    float g_ls[3], g_logit;
    float4 g_qr;
    activate_backward_one(a, gs, g, grad_opac ? grad_opac[i] : 0.0f, g_ls, g_qr, g_logit);
#pragma unroll
    for (int c = 0; c < 3; ++c) grad_log_scales[3 * i + c] = grad_scales ? g_ls[c] : 0.0f;
    reinterpret_cast<float4 *>(grad_quats_raw)[i] = g_qr;
    grad_logits[i] = grad_opac ? g_logit : 0.0f;
}

// --------------------------------------------- fused preprocess (training step)
// For the library's training step: activations, projection and the render()
// colour of one Gaussian per thread in one pass over its parameters, and the
// gradients of all three in one pass back.  Values equal the unfused sequence
// activate -> project_points -> SH (render) and SH backward -> project_points
// backward -> activate backward (the same device functions in the same order);
// the forward does not store scales and unit quaternions, the backward
// recomputes them from the raw parameters.

__global__ __launch_bounds__(kShBlock) void preprocess_forward_kernel(
    int64_t n, const float *__restrict__ means, const float *__restrict__ log_scales,
    const float *__restrict__ quats_raw, const float *__restrict__ logits,
    const float *__restrict__ sh_dc, const float *__restrict__ sh_rest,
    const float *__restrict__ w2c, const float *__restrict__ K, float near_plane,
    float far_plane, float min_opacity, float min_radius, float max_radius, int width,
    int height, float *__restrict__ points_image, float *__restrict__ depths,
    float *__restrict__ cov_image, float *__restrict__ cov_inv_image,
    float *__restrict__ radii, uint8_t *__restrict__ mask, float *__restrict__ opacities,
    float *__restrict__ colors, float *__restrict__ sh_cache) {
    const int64_t i = (int64_t)blockIdx.x * kShBlock + threadIdx.x;
    if (i >= n) return;
    const Activated a = activate_one(log_scales, quats_raw, logits, i);
    const Camera cam = load_camera(w2c, K, width, height);
    const Projection p = project_gaussian(
        cam, means[3 * i], means[3 * i + 1], means[3 * i + 2], a.s[0], a.s[1], a.s[2], a.q[0],
        a.q[1], a.q[2], a.q[3], a.o, near_plane, far_plane, min_opacity, min_radius, max_radius,
        width, height);
    points_image[2 * i] = p.u;
    points_image[2 * i + 1] = p.v;
    depths[i] = p.keep ? p.zc : 0.0f;
    cov_image[3 * i] = p.a;
    cov_image[3 * i + 1] = p.b;
    cov_image[3 * i + 2] = p.c;
    cov_inv_image[3 * i] = p.A;
    cov_inv_image[3 * i + 1] = p.B;
    cov_inv_image[3 * i + 2] = p.C;
    radii[2 * i] = p.ru;
    radii[2 * i + 1] = p.rv;
    mask[i] = p.keep ? 1 : 0;
    opacities[i] = a.o;
    if (!colors) return;  // the colours come from another launch
    float rgb[3] = {0.f, 0.f, 0.f};
    if (p.keep) {
        float cx, cy, cz;
        camera_position(nullptr, w2c, cx, cy, cz);
        const ShView v = sh_view(means + 3 * i, cx, cy, cz);
        const float *rest = sh_rest + kRest * i;
#pragma unroll
        for (int c = 0; c < 3; ++c) rgb[c] = sh_raw_channel(v, sh_dc + 3 * i, rest, c);
        if (sh_cache) sh_cache_store(sh_cache, i, v, rest, rgb);
    }
#pragma unroll
    for (int c = 0; c < 3; ++c) colors[3 * i + c] = sh_render_value(rgb[c]);
}

// kRaw: gradients w.r.t. the raw training parameters (log-scales, raw
// quaternions, opacity logits: the activations' backward included).  !kRaw: the
// render() inputs -- scales, quaternions as given (log_scales and quats_raw then
// hold those; logits, grad_opac and grad_logits are unused) -- and the
// gradients of project_points_backward plus evaluate_sh_render_backward, the
// means' two terms summed.
// kCached: sh_cache holds the forward's colour-gradient cache (kShCache floats
// per Gaussian) and sh_dc / sh_rest are not read; LDS then holds each
// Gaussian's 15 basis values and masked colour gradient, the factors of its
// SH-rest gradient row, and the rows are written from them with coalesced
// 12-byte stores (10 KB of LDS per block instead of the 23 KB of staged rows).
constexpr int kBasisStride = 16;  // LDS floats per Gaussian's basis values (15 used)

template <bool kRaw, bool kCached>
__global__ __launch_bounds__(kShBlock) void preprocess_backward_kernel(
    int64_t n, const float *__restrict__ grad_points_image,
    const float *__restrict__ grad_cov_inv, const float *__restrict__ grad_opac,
    const float *__restrict__ grad_colors, const float *__restrict__ means,
    const float *__restrict__ log_scales, const float *__restrict__ quats_raw,
    const float *__restrict__ logits, const float *__restrict__ sh_dc,
    const float *__restrict__ sh_rest, const float *__restrict__ cov_image,
    const uint8_t *__restrict__ mask, const float *__restrict__ w2c,
    const float *__restrict__ K, int width, int height, float *__restrict__ grad_means,
    float *__restrict__ grad_log_scales, float *__restrict__ grad_quats_raw,
    float *__restrict__ grad_logits, float *__restrict__ grad_dc,
    float *__restrict__ grad_rest, const float *__restrict__ sh_cache) {
    constexpr int kLds = kCached ? kShBlock * (kBasisStride + 4) : kShBlock * kRest;
    __shared__ __align__(16) float lds[kLds];
    __shared__ uint8_t keep[kShBlock];
    const int64_t first = (int64_t)blockIdx.x * kShBlock;
    const int nb = (int)min((int64_t)kShBlock, n - first);
    const int t = threadIdx.x;
    if constexpr (!kCached) {
        keep[t] = t < nb ? mask[first + t] : 0;
        __syncthreads();
        block_copy<true>(lds, const_cast<float *>(sh_rest) + kRest * first, kRest * nb, keep);
        __syncthreads();
    }
    float *lrest = lds + kRest * t;                                // !kCached: the row
    float *lbasis = lds + kBasisStride * t;                        // kCached: b_0..b_14
    float *lgrad = lds + kShBlock * kBasisStride + 4 * t;          // kCached: g_0..g_2
    if (t < nb) {
        const int64_t i = first + t;
        Activated a;
        if constexpr (kRaw) {
            a = activate_one(log_scales, quats_raw, logits, i);
        } else {
#pragma unroll
            for (int c = 0; c < 3; ++c) a.s[c] = log_scales[3 * i + c];
#pragma unroll
            for (int c = 0; c < 4; ++c) a.q[c] = quats_raw[4 * i + c];
        }
        float gp[3] = {0.f, 0.f, 0.f}, gs[3] = {0.f, 0.f, 0.f}, gq[4] = {0.f, 0.f, 0.f, 0.f};
        float gm[3] = {0.f, 0.f, 0.f}, gdc[3] = {0.f, 0.f, 0.f};
        if (mask[i]) {
            const Camera cam = load_camera(w2c, K, width, height);
            project_gaussian_backward(
                cam, means[3 * i], means[3 * i + 1], means[3 * i + 2], a.s[0], a.s[1], a.s[2],
                a.q[0], a.q[1], a.q[2], a.q[3], cov_image[3 * i], cov_image[3 * i + 1],
                cov_image[3 * i + 2], grad_points_image[2 * i], grad_points_image[2 * i + 1],
                grad_cov_inv[3 * i], grad_cov_inv[3 * i + 1], grad_cov_inv[3 * i + 2], gp[0],
                gp[1], gp[2], gs[0], gs[1], gs[2], gq[0], gq[1], gq[2], gq[3]);
            float cx, cy, cz;
            camera_position(nullptr, w2c, cx, cy, cz);
            const ShView v = sh_view(means + 3 * i, cx, cy, cz);
            float g[3];
            if constexpr (kCached) {
                float m[3][3];
                const uint32_t pass = sh_cache_load(sh_cache, i, m);
#pragma unroll
                for (int c = 0; c < 3; ++c) {
                    g[c] = grad_colors[3 * i + c];
                    if (!((pass >> c) & 1u)) g[c] = 0.0f;
                }
                sh_mean_grad(m, g, gm);
#pragma unroll
                for (int c = 0; c < 3; ++c) gdc[c] = kShC0 * g[c];
#pragma unroll
                for (int k = 0; k < 15; ++k) lbasis[k] = v.b[k];
#pragma unroll
                for (int c = 0; c < 3; ++c) lgrad[c] = g[c];
            } else {
#pragma unroll
                for (int c = 0; c < 3; ++c) {
                    g[c] = grad_colors[3 * i + c];
                    const float raw = sh_raw_channel(v, sh_dc + 3 * i, lrest, c);
                    if (!(raw + 0.5f >= 0.0f)) g[c] = 0.0f;
                }
                sh_backward_row(v, g, lrest, gdc, gm);
            }
        } else if constexpr (kCached) {  // a zero row: 0 * 0
#pragma unroll
            for (int k = 0; k < 15; ++k) lbasis[k] = 0.0f;
#pragma unroll
            for (int c = 0; c < 3; ++c) lgrad[c] = 0.0f;
        } else {
#pragma unroll
            for (int k = 0; k < kRest; ++k) lrest[k] = 0.0f;
        }
        float g_ls[3], g_logit = 0.0f;
        float4 g_qr;
        if constexpr (kRaw) {
            activate_backward_one(a, gs, make_float4(gq[0], gq[1], gq[2], gq[3]), grad_opac[i],
                                  g_ls, g_qr, g_logit);
        } else {
#pragma unroll
            for (int c = 0; c < 3; ++c) g_ls[c] = gs[c];
            g_qr = make_float4(gq[0], gq[1], gq[2], gq[3]);
        }
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            grad_means[3 * i + c] = gp[c] + gm[c];
            grad_dc[3 * i + c] = gdc[c];
            grad_log_scales[3 * i + c] = g_ls[c];
        }
        if constexpr (kRaw) {
            reinterpret_cast<float4 *>(grad_quats_raw)[i] = g_qr;
            grad_logits[i] = g_logit;
        } else {  // the caller's quaternion gradient need not be 16-byte aligned
            grad_quats_raw[4 * i] = g_qr.x;
            grad_quats_raw[4 * i + 1] = g_qr.y;
            grad_quats_raw[4 * i + 2] = g_qr.z;
            grad_quats_raw[4 * i + 3] = g_qr.w;
        }
    }
    __syncthreads();
    if constexpr (kCached) {
        // entry e = 15 t + k of the block is the triple b_k (g_0, g_1, g_2) of
        // Gaussian t at floats 3e .. 3e + 2 of the block's rows: consecutive
        // lanes write consecutive 12-byte triples
        float *out = grad_rest + kRest * first;
        for (int e = t; e < 15 * nb; e += kShBlock) {
            const int gt = e / 15, k = e - 15 * gt;
            const float b = lds[kBasisStride * gt + k];
            const float *gg = lds + kShBlock * kBasisStride + 4 * gt;
            out[3 * e] = b * gg[0];
            out[3 * e + 1] = b * gg[1];
            out[3 * e + 2] = b * gg[2];
        }
    } else {
        block_copy<false>(lds, grad_rest + kRest * first, kRest * nb);
    }
}

}  // namespace gs


using namespace gs;

extern "C" int gs_project_points(const float *means, const float *scales,
                                 const float *quaternions, const float *opacities,
                                 const float *world_to_camera, const float *intrinsic,
                                 int64_t n, float near_plane, float far_plane,
                                 float min_opacity, float min_radius, float max_radius,
                                 int32_t width, int32_t height, float *points_image,
                                 float *depths, float *cov_image, float *cov_inv_image,
                                 float *radii, uint8_t *mask, hipStream_t stream) {
    if (n < 0 || width <= 0 || height <= 0) return GS_ERR_INVALID_ARGUMENT;
    if (n == 0) return GS_OK;
    if (!means || !scales || !quaternions || !opacities || !world_to_camera || !intrinsic ||
        !points_image || !depths || !cov_image || !cov_inv_image || !radii || !mask)
        return GS_ERR_INVALID_ARGUMENT;
    hipLaunchKernelGGL(project_points_kernel, dim3(ceil_div(n, kPreBlock)), dim3(kPreBlock), 0,
                       stream, n, means, scales, quaternions, opacities, world_to_camera,
                       intrinsic, near_plane, far_plane, min_opacity, min_radius, max_radius,
                       width, height, points_image, depths, cov_image, cov_inv_image, radii,
                       mask);
    return launch_status();
}

extern "C" int gs_project_points_backward(
    const float *grad_points_image, const float *grad_cov_inv_image, const float *means,
    const float *scales, const float *quaternions, const float *opacities,
    const float *world_to_camera, const float *intrinsic, int64_t n, int32_t width,
    int32_t height, const float *cov_image, const uint8_t *mask, float *grad_means,
    float *grad_scales, float *grad_quaternions, hipStream_t stream) {
    (void)opacities;  // part of the reference signature; the gradient does not depend on it
    if (n < 0 || width <= 0 || height <= 0) return GS_ERR_INVALID_ARGUMENT;
    if (n == 0) return GS_OK;
    if (!grad_points_image || !grad_cov_inv_image || !means || !scales || !quaternions ||
        !world_to_camera || !intrinsic || !cov_image || !mask || !grad_means || !grad_scales ||
        !grad_quaternions)
        return GS_ERR_INVALID_ARGUMENT;
    hipLaunchKernelGGL(project_points_backward_kernel, dim3(ceil_div(n, kPreBlock)),
                       dim3(kPreBlock), 0, stream, n, grad_points_image, grad_cov_inv_image,
                       means, scales, quaternions, world_to_camera, intrinsic, width, height,
                       cov_image, mask, grad_means, grad_scales, grad_quaternions);
    return launch_status();
}

// max_blocks > 0 caps the grid (its workgroups then take several Gaussians each).
// cache: null, or the colour-gradient cache to write (kShRender only).
static int launch_sh_forward(const float *camera_pos, const float *w2c, const float *means,
                             const float *sh_dc, const float *sh_rest, const uint8_t *mask,
                             int64_t n, int mode, float *colors, hipStream_t stream,
                             int64_t max_blocks = 0, float *cache = nullptr) {
    if (n < 0 || max_blocks < 0) return GS_ERR_INVALID_ARGUMENT;
    if (n == 0) return GS_OK;
    if ((!camera_pos && !w2c) || !means || !sh_dc || !sh_rest || !mask || !colors ||
        (cache && mode != kShRender) || (reinterpret_cast<uintptr_t>(cache) & 7))
        return GS_ERR_INVALID_ARGUMENT;
    int64_t blocks = ceil_div(n, kShBlock);
    if (max_blocks > 0 && blocks > max_blocks) blocks = max_blocks;
    hipLaunchKernelGGL(sh_forward_kernel, dim3((unsigned)blocks), dim3(kShBlock), 0,
                       stream, n, camera_pos, w2c, means, sh_dc, sh_rest, mask, mode, colors,
                       cache);
    return launch_status();
}

static int launch_sh_backward(const float *grad_colors, const float *camera_pos,
                              const float *w2c, const float *means, const float *sh_dc,
                              const float *sh_rest, const float *colors, const uint8_t *mask,
                              int64_t n, int mode, int accumulate_means, float *grad_means,
                              float *grad_sh_dc, float *grad_sh_rest, hipStream_t stream) {
    if (n < 0) return GS_ERR_INVALID_ARGUMENT;
    if (n == 0) return GS_OK;
    if (!grad_colors || (!camera_pos && !w2c) || !means || !sh_rest || !mask || !grad_means ||
        !grad_sh_dc || !grad_sh_rest || (mode == kShSigmoid && !colors) ||
        (mode == kShRender && !sh_dc))
        return GS_ERR_INVALID_ARGUMENT;
    hipLaunchKernelGGL(sh_backward_kernel, dim3(ceil_div(n, kShBlock)), dim3(kShBlock), 0,
                       stream, n, grad_colors, camera_pos, w2c, means, sh_dc, sh_rest, colors,
                       mask, mode, accumulate_means, grad_means, grad_sh_dc, grad_sh_rest);
    return launch_status();
}

extern "C" int gs_evaluate_sh(const float *camera_pos, const float *means, const float *sh_dc,
                              const float *sh_rest, const uint8_t *mask, int64_t n,
                              int32_t sh_sigmoid, float *colors, hipStream_t stream) {
    if (!camera_pos && n > 0) return GS_ERR_INVALID_ARGUMENT;
    return launch_sh_forward(camera_pos, nullptr, means, sh_dc, sh_rest, mask, n,
                             sh_sigmoid ? kShSigmoid : kShRaw, colors, stream);
}

extern "C" int gs_evaluate_sh_backward(const float *grad_colors, const float *camera_pos,
                                       const float *means, const float *sh_dc,
                                       const float *sh_rest, const float *colors,
                                       const uint8_t *mask, int64_t n, int32_t sh_sigmoid,
                                       float *grad_means, float *grad_sh_dc,
                                       float *grad_sh_rest, hipStream_t stream) {
    if (!camera_pos && n > 0) return GS_ERR_INVALID_ARGUMENT;
    return launch_sh_backward(grad_colors, camera_pos, nullptr, means, sh_dc, sh_rest, colors,
                              mask, n, sh_sigmoid ? kShSigmoid : kShRaw, 0, grad_means,
                              grad_sh_dc, grad_sh_rest, stream);
}

extern "C" int gs_evaluate_sh_render(const float *world_to_camera, const float *means,
                                     const float *sh_dc, const float *sh_rest,
                                     const uint8_t *mask, int64_t n, float *colors,
                                     hipStream_t stream) {
    if (!world_to_camera && n > 0) return GS_ERR_INVALID_ARGUMENT;
    return launch_sh_forward(nullptr, world_to_camera, means, sh_dc, sh_rest, mask, n,
                             kShRender, colors, stream);
}

// Compute units of the current device (cached per device; 0 if unknown).
static int device_cus() {
    static int cus[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    if (cus[dev] == 0) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            return 0;
        cus[dev] = v;
    }
    return cus[dev];
}

// The grid of a colour launch beside other work: one workgroup per compute
// unit (measured at config 3 beside binning: 256 workgroups 0.693 ms per fused
// step, 192 0.698, 320 0.704, 512 0.697, one per 128 Gaussians 0.714), more
// when a thread would take over 32 Gaussians.
static int64_t beside_blocks(int64_t n) {
    const int cus = device_cus();
    int64_t blocks = cus > 0 ? cus : 256;
    const int64_t per32 = (n + 32 * kShBlock - 1) / (32 * kShBlock);
    return per32 > blocks ? per32 : blocks;
}

extern "C" int gs_evaluate_sh_render_beside(const float *world_to_camera, const float *means,
                                            const float *sh_dc, const float *sh_rest,
                                            const uint8_t *mask, int64_t n, float *colors,
                                            hipStream_t stream) {
    if (!world_to_camera && n > 0) return GS_ERR_INVALID_ARGUMENT;
    if (n <= 0) return n < 0 ? GS_ERR_INVALID_ARGUMENT : GS_OK;  // no device query
    return launch_sh_forward(nullptr, world_to_camera, means, sh_dc, sh_rest, mask, n,
                             kShRender, colors, stream, beside_blocks(n));
}

extern "C" int gs_evaluate_sh_render_cache(const float *world_to_camera, const float *means,
                                           const float *sh_dc, const float *sh_rest,
                                           const uint8_t *mask, int64_t n, int32_t beside,
                                           float *colors, float *sh_cache, hipStream_t stream) {
    if ((!world_to_camera || !sh_cache) && n > 0) return GS_ERR_INVALID_ARGUMENT;
    if (n <= 0) return n < 0 ? GS_ERR_INVALID_ARGUMENT : GS_OK;  // no device query
    return launch_sh_forward(nullptr, world_to_camera, means, sh_dc, sh_rest, mask, n,
                             kShRender, colors, stream, beside ? beside_blocks(n) : 0,
                             sh_cache);
}

extern "C" int gs_evaluate_sh_render_backward(const float *grad_colors,
                                              const float *world_to_camera, const float *means,
                                              const float *sh_dc, const float *sh_rest,
                                              const uint8_t *mask, int64_t n,
                                              int32_t accumulate_means, float *grad_means,
                                              float *grad_sh_dc, float *grad_sh_rest,
                                              hipStream_t stream) {
    if (!world_to_camera && n > 0) return GS_ERR_INVALID_ARGUMENT;
    return launch_sh_backward(grad_colors, nullptr, world_to_camera, means, sh_dc, sh_rest,
                              nullptr, mask, n, kShRender, accumulate_means ? 1 : 0, grad_means,
                              grad_sh_dc, grad_sh_rest, stream);
}

extern "C" int gs_activate(const float *log_scales, const float *quats_raw,
                           const float *opacity_logits, int64_t n, float *scales, float *quats,
                           float *opacities, hipStream_t stream) {
    if (n < 0) return GS_ERR_INVALID_ARGUMENT;
    if (n == 0) return GS_OK;
    if (!log_scales || !quats_raw || !opacity_logits || !scales || !quats || !opacities ||
        (reinterpret_cast<uintptr_t>(quats_raw) & 15) || (reinterpret_cast<uintptr_t>(quats) & 15))
        return GS_ERR_INVALID_ARGUMENT;
    hipLaunchKernelGGL(activate_kernel, dim3(ceil_div(n, 256)), dim3(256), 0, stream, n,
                       log_scales, quats_raw, opacity_logits, scales, quats, opacities);
    return launch_status();
}

extern "C" int gs_activate_backward(const float *grad_scales, const float *grad_quats,
                                    const float *grad_opacities, const float *scales,
                                    const float *quats_raw, const float *opacities, int64_t n,
                                    float *grad_log_scales, float *grad_quats_raw,
                                    float *grad_opacity_logits, hipStream_t stream) {
    if (n < 0) return GS_ERR_INVALID_ARGUMENT;
    if (n == 0) return GS_OK;
    if (!scales || !quats_raw || !opacities || !grad_log_scales || !grad_quats_raw ||
        !grad_opacity_logits || (reinterpret_cast<uintptr_t>(quats_raw) & 15) ||
        (reinterpret_cast<uintptr_t>(grad_quats_raw) & 15) ||
        (grad_quats && (reinterpret_cast<uintptr_t>(grad_quats) & 15)))
        return GS_ERR_INVALID_ARGUMENT;
    hipLaunchKernelGGL(activate_backward_kernel, dim3(ceil_div(n, 256)), dim3(256), 0, stream, n,
                       grad_scales, grad_quats, grad_opacities, scales, quats_raw, opacities,
                       grad_log_scales, grad_quats_raw, grad_opacity_logits);
    return launch_status();
}

extern "C" int gs_preprocess_forward(const float *means, const float *log_scales,
                                     const float *quats_raw, const float *opacity_logits,
                                     const float *sh_dc, const float *sh_rest,
                                     const float *world_to_camera, const float *intrinsic,
                                     int64_t n, float near_plane, float far_plane,
                                     float min_opacity, float min_radius, float max_radius,
                                     int32_t width, int32_t height, float *points_image,
                                     float *depths, float *cov_image, float *cov_inv_image,
                                     float *radii, uint8_t *mask, float *opacities,
                                     float *colors, float *sh_cache, hipStream_t stream) {
    if (n < 0 || width <= 0 || height <= 0) return GS_ERR_INVALID_ARGUMENT;
    if (n == 0) return GS_OK;
    if (!means || !log_scales || !quats_raw || !opacity_logits ||
        (colors && (!sh_dc || !sh_rest)) || (sh_cache && !colors) || !world_to_camera ||
        !intrinsic || !points_image || !depths || !cov_image || !cov_inv_image || !radii ||
        !mask || !opacities || (reinterpret_cast<uintptr_t>(quats_raw) & 15) ||
        (reinterpret_cast<uintptr_t>(sh_cache) & 7))
        return GS_ERR_INVALID_ARGUMENT;
    hipLaunchKernelGGL(preprocess_forward_kernel, dim3(ceil_div(n, kShBlock)), dim3(kShBlock), 0,
                       stream, n, means, log_scales, quats_raw, opacity_logits, sh_dc, sh_rest,
                       world_to_camera, intrinsic, near_plane, far_plane, min_opacity,
                       min_radius, max_radius, width, height, points_image, depths, cov_image,
                       cov_inv_image, radii, mask, opacities, colors, sh_cache);
    return launch_status();
}

extern "C" int gs_preprocess_backward(
    const float *grad_points_image, const float *grad_cov_inv_image,
    const float *grad_opacities, const float *grad_colors, const float *means,
    const float *log_scales, const float *quats_raw, const float *opacity_logits,
    const float *sh_dc, const float *sh_rest, const float *cov_image, const uint8_t *mask,
    const float *world_to_camera, const float *intrinsic, int64_t n, int32_t width,
    int32_t height, float *grad_means, float *grad_log_scales, float *grad_quats_raw,
    float *grad_opacity_logits, float *grad_sh_dc, float *grad_sh_rest, const float *sh_cache,
    hipStream_t stream) {
    if (n < 0 || width <= 0 || height <= 0) return GS_ERR_INVALID_ARGUMENT;
    if (n == 0) return GS_OK;
    if (!grad_points_image || !grad_cov_inv_image || !grad_opacities || !grad_colors || !means ||
        !log_scales || !quats_raw || !opacity_logits || (!sh_cache && (!sh_dc || !sh_rest)) ||
        !cov_image || !mask || !world_to_camera || !intrinsic || !grad_means ||
        !grad_log_scales || !grad_quats_raw || !grad_opacity_logits || !grad_sh_dc ||
        !grad_sh_rest || (reinterpret_cast<uintptr_t>(quats_raw) & 15) ||
        (reinterpret_cast<uintptr_t>(grad_quats_raw) & 15) ||
        (reinterpret_cast<uintptr_t>(sh_cache) & 7))
        return GS_ERR_INVALID_ARGUMENT;
    auto kern = sh_cache ? preprocess_backward_kernel<true, true>
                         : preprocess_backward_kernel<true, false>;
    hipLaunchKernelGGL(kern, dim3(ceil_div(n, kShBlock)), dim3(kShBlock), 0, stream, n,
                       grad_points_image, grad_cov_inv_image, grad_opacities, grad_colors, means,
                       log_scales, quats_raw, opacity_logits, sh_dc, sh_rest, cov_image, mask,
                       world_to_camera, intrinsic, width, height, grad_means, grad_log_scales,
                       grad_quats_raw, grad_opacity_logits, grad_sh_dc, grad_sh_rest, sh_cache);
    return launch_status();
}

extern "C" int gs_render_preprocess_backward(
    const float *grad_points_image, const float *grad_cov_inv_image, const float *grad_colors,
    const float *means, const float *scales, const float *quaternions, const float *sh_dc,
    const float *sh_rest, const float *cov_image, const uint8_t *mask,
    const float *world_to_camera, const float *intrinsic, int64_t n, int32_t width,
    int32_t height, float *grad_means, float *grad_scales, float *grad_quaternions,
    float *grad_sh_dc, float *grad_sh_rest, const float *sh_cache, hipStream_t stream) {
    if (n < 0 || width <= 0 || height <= 0) return GS_ERR_INVALID_ARGUMENT;
    if (n == 0) return GS_OK;
    if (!grad_points_image || !grad_cov_inv_image || !grad_colors || !means || !scales ||
        !quaternions || (!sh_cache && (!sh_dc || !sh_rest)) || !cov_image || !mask ||
        !world_to_camera || !intrinsic || !grad_means || !grad_scales || !grad_quaternions ||
        !grad_sh_dc || !grad_sh_rest || (reinterpret_cast<uintptr_t>(sh_cache) & 7))
        return GS_ERR_INVALID_ARGUMENT;
    auto kern = sh_cache ? preprocess_backward_kernel<false, true>
                         : preprocess_backward_kernel<false, false>;
    hipLaunchKernelGGL(kern, dim3(ceil_div(n, kShBlock)), dim3(kShBlock), 0, stream, n,
                       grad_points_image, grad_cov_inv_image, nullptr, grad_colors, means, scales,
                       quaternions, nullptr, sh_dc, sh_rest, cov_image, mask, world_to_camera,
                       intrinsic, width, height, grad_means, grad_scales, grad_quaternions,
                       nullptr, grad_sh_dc, grad_sh_rest, sh_cache);
    return launch_status();
}
