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

// SH evaluation (src/gaussian.py:24-61; data flow of src/cuda/kernel.cu:545-617).
// The API's output is the raw SH sum (or its sigmoid); the caller applies the
// max(c + 0.5, 0) shift (src/cuda/wrapper.py:264-265).
__global__ __launch_bounds__(kPreBlock) void sh_forward_kernel(
    int64_t n, const float *__restrict__ cam_pos, const float *__restrict__ means,
    const float *__restrict__ sh_dc, const float *__restrict__ sh_rest,
    const uint8_t *__restrict__ mask, int sh_sigmoid, float *__restrict__ colors) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float rgb[3] = {0.f, 0.f, 0.f};
    if (mask[i]) {
        const float dx = means[3 * i] - cam_pos[0];
        const float dy = means[3 * i + 1] - cam_pos[1];
        const float dz = means[3 * i + 2] - cam_pos[2];
        const float norm = sqrtf(dx * dx + dy * dy + dz * dz);
        float b[15];
        sh_basis_rest(dx / norm, dy / norm, dz / norm, b);
        const float *rest = sh_rest + 45 * i;
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            float acc = kShC0 * sh_dc[3 * i + c];
#pragma unroll
            for (int k = 0; k < 15; ++k) acc += b[k] * rest[3 * k + c];
            rgb[c] = sh_sigmoid ? 1.0f / (1.0f + expf(-acc)) : acc;
        }
    }
    colors[3 * i] = rgb[0];
    colors[3 * i + 1] = rgb[1];
    colors[3 * i + 2] = rgb[2];
}

// SH gradient (data flow of src/cuda/kernel.cu:619-782).
__global__ __launch_bounds__(kPreBlock) void sh_backward_kernel(
    int64_t n, const float *__restrict__ grad_colors, const float *__restrict__ cam_pos,
    const float *__restrict__ means, const float *__restrict__ sh_rest,
    const float *__restrict__ colors, const uint8_t *__restrict__ mask, int sh_sigmoid,
    float *__restrict__ grad_means, float *__restrict__ grad_dc,
    float *__restrict__ grad_rest) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float *gr = grad_rest + 45 * i;
    if (!mask[i]) {
        grad_means[3 * i] = grad_means[3 * i + 1] = grad_means[3 * i + 2] = 0.0f;
        grad_dc[3 * i] = grad_dc[3 * i + 1] = grad_dc[3 * i + 2] = 0.0f;
#pragma unroll
        for (int k = 0; k < 45; ++k) gr[k] = 0.0f;
        return;
    }
    float g[3];
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        g[c] = grad_colors[3 * i + c];
        if (sh_sigmoid) {
            const float s = colors[3 * i + c];
            g[c] *= s * (1.0f - s);
        }
        grad_dc[3 * i + c] = kShC0 * g[c];
    }
    const float dx = means[3 * i] - cam_pos[0];
    const float dy = means[3 * i + 1] - cam_pos[1];
    const float dz = means[3 * i + 2] - cam_pos[2];
    const float norm = sqrtf(dx * dx + dy * dy + dz * dz);
    const float x = dx / norm, y = dy / norm, z = dz / norm;
    float b[15], bx[15], by[15], bz[15];
    sh_basis_rest(x, y, z, b);
    sh_basis_rest_grad(x, y, z, bx, by, bz);
    const float *rest = sh_rest + 45 * i;
    float gdx = 0.f, gdy = 0.f, gdz = 0.f;
#pragma unroll
    for (int k = 0; k < 15; ++k) {
        gr[3 * k] = b[k] * g[0];
        gr[3 * k + 1] = b[k] * g[1];
        gr[3 * k + 2] = b[k] * g[2];
        const float gk = g[0] * rest[3 * k] + g[1] * rest[3 * k + 1] + g[2] * rest[3 * k + 2];
        gdx += gk * bx[k];
        gdy += gk * by[k];
        gdz += gk * bz[k];
    }
    // dir = d / |d| -> (I - dir dir^T) / |d|
    const float dot = x * gdx + y * gdy + z * gdz;
    grad_means[3 * i] = (gdx - x * dot) / norm;
    grad_means[3 * i + 1] = (gdy - y * dot) / norm;
    grad_means[3 * i + 2] = (gdz - z * dot) / norm;
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

extern "C" int gs_evaluate_sh(const float *camera_pos, const float *means, const float *sh_dc,
                              const float *sh_rest, const uint8_t *mask, int64_t n,
                              int32_t sh_sigmoid, float *colors, hipStream_t stream) {
    if (n < 0) return GS_ERR_INVALID_ARGUMENT;
    if (n == 0) return GS_OK;
    if (!camera_pos || !means || !sh_dc || !sh_rest || !mask || !colors)
        return GS_ERR_INVALID_ARGUMENT;
    hipLaunchKernelGGL(sh_forward_kernel, dim3(ceil_div(n, kPreBlock)), dim3(kPreBlock), 0,
                       stream, n, camera_pos, means, sh_dc, sh_rest, mask, (int)sh_sigmoid,
                       colors);
    return launch_status();
}

extern "C" int gs_evaluate_sh_backward(const float *grad_colors, const float *camera_pos,
                                       const float *means, const float *sh_dc,
                                       const float *sh_rest, const float *colors,
                                       const uint8_t *mask, int64_t n, int32_t sh_sigmoid,
                                       float *grad_means, float *grad_sh_dc,
                                       float *grad_sh_rest, hipStream_t stream) {
    (void)sh_dc;  // the gradient is linear in the coefficients
    if (n < 0) return GS_ERR_INVALID_ARGUMENT;
    if (n == 0) return GS_OK;
    if (!grad_colors || !camera_pos || !means || !sh_rest || !mask || !grad_means ||
        !grad_sh_dc || !grad_sh_rest || (sh_sigmoid && !colors))
        return GS_ERR_INVALID_ARGUMENT;
    hipLaunchKernelGGL(sh_backward_kernel, dim3(ceil_div(n, kPreBlock)), dim3(kPreBlock), 0,
                       stream, n, grad_colors, camera_pos, means, sh_rest, colors, mask,
                       (int)sh_sigmoid, grad_means, grad_sh_dc, grad_sh_rest);
    return launch_status();
}
