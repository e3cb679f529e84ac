"""Autograd glue and `render()`, the counterpart of src/cuda/wrapper.py.

Same three autograd Functions (ProjectPointsFunction, SphericalHarmonicsFunction,
RasterizeFunction) and the same `render` signature and return values
(src/cuda/wrapper.py:12-294): render(...) -> (image[H,W,3] in [0,255],
points_img[N,2], radii[N,2]).  `points_img` is a non-leaf tensor whose
`.grad` (after `retain_grad()`) is dL/d(points_img), as the reference's
densification strategy expects (src/strategy.py:47-68).

Differences from the reference glue (same values and gradients):
- RasterizeFunction saves its forward image and hands it to the backward
  kernel, so the backward does not recompute each pixel's colour
  (src/cuda/kernel.cu:1032-1060 replays the whole forward pass).
- render() uses fused kernels for the glue around the seven functions: the
  camera position, SH and max(c + 0.5, 0) in one kernel, which with the
  projection forms one autograd node whose backward is one kernel
  (RenderPreprocessFunction), and the blend writing clamp(image, 0, 1) * 255
  itself, with the clamp's gradient applied inside the blend backward
  (RenderRasterizeFunction).
- ProjectPointsFunction marks depths, radii and mask non-differentiable, so
  autograd allocates no zero gradients for them.
"""

from __future__ import annotations

import torch

import cuda_rasterizer as _cr


class ProjectPointsFunction(torch.autograd.Function):
    """src/cuda/wrapper.py:12-85."""

    @staticmethod
    def forward(ctx, means, scales, quaternions, opacities, world_to_camera, intrinsic,
                near_plane, far_plane, min_opacity, min_radius, max_radius, width, height):
        points_img, depths, cov_img, cov_inv_img, radii, mask = _cr.project_points(
            means, scales, quaternions, opacities, world_to_camera, intrinsic, near_plane,
            far_plane, min_opacity, min_radius, max_radius, width, height)
        ctx.save_for_backward(means, scales, quaternions, opacities, world_to_camera, intrinsic,
                              cov_img, mask)
        ctx.width = width
        ctx.height = height
        ctx.mark_non_differentiable(depths, radii, mask)
        ctx.set_materialize_grads(False)
        return points_img, depths, cov_inv_img, radii, mask

    @staticmethod
    def backward(ctx, grad_points_img, grad_depths, grad_cov_inv_img, grad_radii, grad_mask):
        means, scales, quaternions, opacities, world_to_camera, intrinsic, cov_img, mask = (
            ctx.saved_tensors)
        if grad_points_img is None and grad_cov_inv_img is None:
            return (None,) * 13
        if grad_points_img is None:
            grad_points_img = torch.zeros((means.shape[0], 2), dtype=means.dtype,
                                          device=means.device)
        if grad_cov_inv_img is None:
            grad_cov_inv_img = torch.zeros((means.shape[0], 3), dtype=means.dtype,
                                           device=means.device)
        g_means, g_scales, g_quats = _cr.project_points_backward(
            grad_points_img, grad_cov_inv_img, means, scales, quaternions, opacities,
            world_to_camera, intrinsic, ctx.width, ctx.height, cov_img, mask)
        return (g_means, g_scales, g_quats) + (None,) * 10


class SphericalHarmonicsFunction(torch.autograd.Function):
    """src/cuda/wrapper.py:88-118."""

    @staticmethod
    def forward(ctx, camera_pos, means, sh_coeffs_dc, sh_coeffs_rest, mask, sh_sigmoid=False):
        colors = _cr.evaluate_spherical_harmonics(camera_pos, means, sh_coeffs_dc,
                                                  sh_coeffs_rest, mask, sh_sigmoid)
        ctx.save_for_backward(camera_pos, means, sh_coeffs_dc, sh_coeffs_rest, colors, mask)
        ctx.sh_sigmoid = sh_sigmoid
        return colors

    @staticmethod
    def backward(ctx, grad_colors):
        camera_pos, means, sh_coeffs_dc, sh_coeffs_rest, colors, mask = ctx.saved_tensors
        g_means, g_dc, g_rest = _cr.evaluate_spherical_harmonics_backward(
            grad_colors, camera_pos, means, sh_coeffs_dc, sh_coeffs_rest, colors, mask,
            ctx.sh_sigmoid)
        return None, g_means, g_dc, g_rest, None, None


class RenderPreprocessFunction(torch.autograd.Function):
    """ProjectPointsFunction and the render() colours (camera position, SH and
    max(c + 0.5, 0); src/cuda/wrapper.py:223-265) as one autograd node: the
    forward runs project_points and the colour kernel (on the calling thread's
    second stream, beside binning, when `beside` is a list: it receives the
    fused.ColorsBeside to wait on), the backward one kernel for both
    (render_preprocess_backward), so the means' two gradient terms are summed in
    it rather than by autograd.  With `with_cache` the colour kernel also writes
    the colour-gradient cache (40 bytes per Gaussian), which the backward reads
    in place of the 180-byte SH rows."""

    @staticmethod
    def forward(ctx, means, scales, quaternions, opacities, world_to_camera, intrinsic,
                sh_coeffs_dc, sh_coeffs_rest, near_plane, far_plane, min_opacity, min_radius,
                max_radius, width, height, beside=None, with_cache=False):
        points_img, depths, cov_img, cov_inv_img, radii, mask = _cr.project_points(
            means, scales, quaternions, opacities, world_to_camera, intrinsic, near_plane,
            far_plane, min_opacity, min_radius, max_radius, width, height)
        if beside is not None:
            from cuda_rasterizer.fused import colors_beside

            pending = colors_beside(world_to_camera, means, sh_coeffs_dc, sh_coeffs_rest, mask,
                                    with_cache=with_cache)
            beside.append(pending)
            colors, cache = pending.colors, pending.sh_cache
        else:
            cache = _cr.sh_cache_empty(means.shape[0], means.device) if with_cache else None
            colors = _cr.evaluate_spherical_harmonics_render(world_to_camera, means,
                                                             sh_coeffs_dc, sh_coeffs_rest, mask,
                                                             sh_cache=cache)
        ctx.save_for_backward(means, scales, quaternions, world_to_camera, intrinsic,
                              sh_coeffs_dc, sh_coeffs_rest, cov_img, mask, cache)
        ctx.width = width
        ctx.height = height
        ctx.mark_non_differentiable(depths, radii, mask)
        ctx.set_materialize_grads(False)
        return points_img, depths, cov_inv_img, radii, mask, colors

    @staticmethod
    def backward(ctx, grad_points_img, grad_depths, grad_cov_inv_img, grad_radii, grad_mask,
                 grad_colors):
        means, scales, quaternions, w2c, K, dc, rest, cov_img, mask, cache = ctx.saved_tensors
        if grad_points_img is None and grad_cov_inv_img is None and grad_colors is None:
            return (None,) * 17
        n = means.shape[0]

        def zeros(w):
            return torch.zeros((n, w), dtype=means.dtype, device=means.device)

        g_means, g_scales, g_quats, g_dc, g_rest = _cr.render_preprocess_backward(
            zeros(2) if grad_points_img is None else grad_points_img,
            zeros(3) if grad_cov_inv_img is None else grad_cov_inv_img,
            zeros(3) if grad_colors is None else grad_colors, means, scales, quaternions, dc,
            rest, cov_img, mask, w2c, K, ctx.width, ctx.height, sh_cache=cache)
        return (g_means, g_scales, g_quats, None, None, None, g_dc, g_rest) + (None,) * 9


class RenderRasterizeFunction(torch.autograd.Function):
    """rasterize followed by clamp(0, 1) * 255 (src/cuda/wrapper.py:268-294) in the
    blend kernels; returns the display image."""

    @staticmethod
    def forward(ctx, indexing_offset, gaussian_ids_sorted, points_img, cov_inv_img, opacities,
                colors, width, height, tile_size, alpha_threshold, transmittance_threshold,
                chi_squared_threshold, grad_mode=True, forward_order=None):
        # the forward's work per tile orders the backward's tiles (heaviest first);
        # not computed when no backward can follow (grad_mode: the caller's
        # torch.is_grad_enabled(), which is always False inside forward)
        grad = grad_mode and any(ctx.needs_input_grad[2:6])
        schedule = _cr.tile_schedule(indexing_offset.shape[0], points_img.device) if grad else None
        image, display = _cr.rasterize_display(
            indexing_offset, gaussian_ids_sorted, points_img, cov_inv_img, opacities, colors,
            width, height, tile_size, alpha_threshold, transmittance_threshold,
            chi_squared_threshold, schedule=schedule, forward_order=forward_order)
        ctx.save_for_backward(indexing_offset, gaussian_ids_sorted, points_img, cov_inv_img,
                              opacities, colors, image, schedule)  # schedule may be None
        ctx.params = (width, height, tile_size, alpha_threshold, transmittance_threshold,
                      chi_squared_threshold)
        return display

    @staticmethod
    def backward(ctx, grad_display):
        offsets, ids, points_img, cov_inv_img, opacities, colors, image, schedule = (
            ctx.saved_tensors)
        g_pts, g_conic, g_opac, g_col = _cr.rasterize_display_backward(
            grad_display, offsets, ids, points_img, cov_inv_img, opacities, colors, *ctx.params,
            rendered_image=image, schedule=schedule)
        return (None, None, g_pts, g_conic, g_opac, g_col, None, None, None, None, None, None,
                None, None)


class RasterizeFunction(torch.autograd.Function):
    """src/cuda/wrapper.py:121-220."""

    @staticmethod
    def forward(ctx, indexing_offset, gaussian_ids_sorted, points_img, cov_inv_img, opacities,
                colors, width, height, tile_size, alpha_threshold, transmittance_threshold,
                chi_squared_threshold):
        image = _cr.rasterize(indexing_offset, gaussian_ids_sorted, points_img, cov_inv_img,
                              opacities, colors, width, height, tile_size, alpha_threshold,
                              transmittance_threshold, chi_squared_threshold)
        ctx.save_for_backward(indexing_offset, gaussian_ids_sorted, points_img, cov_inv_img,
                              opacities, colors, image)
        ctx.params = (width, height, tile_size, alpha_threshold, transmittance_threshold,
                      chi_squared_threshold)
        return image

    @staticmethod
    def backward(ctx, grad_image):
        offsets, ids, points_img, cov_inv_img, opacities, colors, image = ctx.saved_tensors
        g_pts, g_conic, g_opac, g_col = _cr.rasterize_backward(
            grad_image, offsets, ids, points_img, cov_inv_img, opacities, colors, *ctx.params,
            rendered_image=image)
        return None, None, g_pts, g_conic, g_opac, g_col, None, None, None, None, None, None


def render(
    world_to_camera,
    intrinsic,
    width,
    height,
    means,
    scales,
    quaternions,
    opacities,
    sh_coeffs_dc,
    sh_coeffs_rest,
    near_plane=0.01,
    far_plane=100.0,
    min_opacity=1 / 255,
    min_radius=0.5,
    max_radius=128.0,
    alpha_threshold=1e-4,
    transmittance_threshold=1e-4,
    chi_squared_threshold=9.21,  # 99% confidence interval for 2 DOF
    sh_sigmoid=False,
):
    """src/cuda/wrapper.py:223-294.  Returns (image*255 clamped, points_img, radii)."""
    if sh_sigmoid:
        points_img, depths, cov_inv_img, radii, mask = ProjectPointsFunction.apply(
            means, scales, quaternions, opacities, world_to_camera, intrinsic, near_plane,
            far_plane, min_opacity, min_radius, max_radius, width, height)
        camera_pos = -world_to_camera[:3, :3].t() @ world_to_camera[:3, 3]
        colors = SphericalHarmonicsFunction.apply(camera_pos, means, sh_coeffs_dc,
                                                  sh_coeffs_rest, mask, True)
        colors_ready = None
    else:  # projection and max(sh + 0.5, 0) as one node (colours beside binning in training)
        from cuda_rasterizer.fused import BESIDE_MIN_GAUSSIANS

        training = torch.is_grad_enabled()
        sink = [] if training and means.shape[0] >= BESIDE_MIN_GAUSSIANS else None
        # the colour-gradient cache only when the node will have a backward
        with_cache = training and any(
            isinstance(t, torch.Tensor) and t.requires_grad
            for t in (means, scales, quaternions, sh_coeffs_dc, sh_coeffs_rest))
        points_img, depths, cov_inv_img, radii, mask, colors = RenderPreprocessFunction.apply(
            means, scales, quaternions, opacities, world_to_camera, intrinsic, sh_coeffs_dc,
            sh_coeffs_rest, near_plane, far_plane, min_opacity, min_radius, max_radius, width,
            height, sink, with_cache)
        colors_ready = sink[0] if sink else None

    tile_size = 16
    check = None
    try:
        # the tile lists, and a launch order for the blend forward from their lengths;
        # sized by capacities, so no host read of K and M before the blend is queued
        indexing_offset, gaussian_ids_sorted, order, check = _cr.tile_intersection_capped(
            points_img.detach(), radii, depths, mask, width, height, tile_size)
    finally:
        if colors_ready is not None:
            colors_ready.wait()

    def blend():
        return RenderRasterizeFunction.apply(
            indexing_offset, gaussian_ids_sorted, points_img, cov_inv_img, opacities, colors,
            width, height, tile_size, alpha_threshold, transmittance_threshold,
            chi_squared_threshold, torch.is_grad_enabled(), order)

    try:
        display = blend()
    finally:
        fits = check is None or check.ok()
    if not fits:  # the lists outgrew the capacities: bin with exact sizes, blend again
        indexing_offset, gaussian_ids_sorted, order = _cr.compute_tile_intersection_ordered(
            points_img.detach(), radii, depths, mask, width, height, tile_size)
        display = blend()
    return display, points_img, radii


def render_unfused(world_to_camera, intrinsic, width, height, means, scales, quaternions,
                   opacities, sh_coeffs_dc, sh_coeffs_rest, near_plane=0.01, far_plane=100.0,
                   min_opacity=1 / 255, min_radius=0.5, max_radius=128.0, alpha_threshold=1e-4,
                   transmittance_threshold=1e-4, chi_squared_threshold=9.21, sh_sigmoid=False):
    """render() composed of the seven extension functions exactly as the reference's
    own src/cuda/wrapper.py:223-294 composes them: ProjectPointsFunction ->
    camera position and SphericalHarmonicsFunction -> clamp_min(c + 0.5, 0) in
    PyTorch -> compute_tile_intersection -> RasterizeFunction -> clamp(0, 1) * 255
    in PyTorch.  This is the call sequence a caller that keeps the reference's
    wrapper and swaps in this `cuda_rasterizer` module runs; render() gives the
    same values with fused kernels."""
    points_img, depths, cov_inv_img, radii, mask = ProjectPointsFunction.apply(
        means, scales, quaternions, opacities, world_to_camera, intrinsic, near_plane,
        far_plane, min_opacity, min_radius, max_radius, width, height)
    camera_pos = -world_to_camera[:3, :3].t() @ world_to_camera[:3, 3]
    colors = SphericalHarmonicsFunction.apply(camera_pos, means, sh_coeffs_dc, sh_coeffs_rest,
                                              mask, sh_sigmoid)
    if not sh_sigmoid:
        colors = torch.clamp_min(colors + 0.5, 0.0)
    tile_size = 16
    indexing_offset, gaussian_ids_sorted = _cr.compute_tile_intersection(
        points_img.contiguous(), radii.contiguous(), depths.contiguous(), mask.contiguous(),
        width, height, tile_size)
    image = RasterizeFunction.apply(indexing_offset, gaussian_ids_sorted, points_img, cov_inv_img,
                                    opacities, colors, width, height, tile_size, alpha_threshold,
                                    transmittance_threshold, chi_squared_threshold)
    return image.clamp(0, 1) * 255, points_img, radii
