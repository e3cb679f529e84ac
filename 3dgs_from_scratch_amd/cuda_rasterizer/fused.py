"""Fused training step: activations + render + L1 loss as one autograd node.

The reference's training step (scripts/train.py:133-227) applies the
activations in PyTorch (:135-143), calls render() (src/cuda/wrapper.py:223-294)
and computes an L1 loss on the /255 image (:187-191); autograd then runs
separate PyTorch kernels for each of those steps.  `render_l1` computes the
same values with the library's kernels only:

  forward   preprocess (activations and projection: one kernel) -> binning
            -> blend (image, display, per-tile L1 sums) -> loss; the colours
            (SH +0.5 and clamp) run on a second stream beside binning, whose
            chain of small launches leaves most of the GPU idle
  backward  blend backward seeded by the L1 gradient -> preprocess backward
            (projection, SH and activation gradients: one kernel, which reads
            the colour pass's colour-gradient cache instead of the SH rows)

Values equal the unfused sequence up to floating-point summation order (the
loss sum and the gradient atomics); tests/test_gpu_fused.py checks both
against the drop-in path and the CPU oracle.  Only the loss is differentiable;
the display image, points_img and radii are returned for logging.
Densification statistics (src/strategy.py:47-68 reads dL/d points_img, which
this node never materialises as a .grad): pass `densifier`, a
cuda_rasterizer.train.Densifier, and the backward adds the gradient norms in
NDC scale and the visibility counts to it (gs_accumulate_grad2d).

With ssim_lambda > 0 the loss is the reference's full training loss,
(1 - ssim_lambda) * L1 + ssim_lambda * (1 - SSIM(display / 255, target))
(scripts/train.py:185-205; SSIM by cuda_rasterizer.ssim, padding "valid" as
there): the SSIM gradient w.r.t. display / 255 joins the L1 seed inside the
blend backward, as autograd sums the two uses of display / 255.
"""

from __future__ import annotations

import threading

import torch

import cuda_rasterizer as _cr
from cuda_rasterizer import ssim as _ssim


# Gaussians from which the colours run on a second stream beside binning.  Measured
# in one process, fused step: 1M Gaussians (config 3) 0.707 -> 0.689 ms beside
# binning; 200k (config 5) 0.526 -> 0.539 ms and 10k (config 1) 0.417 -> 0.454 ms,
# where the fork and join cost more than the short colour pass saves.
BESIDE_MIN_GAUSSIANS = 600_000

_SIDE: dict = {}


def _side_stream(dev: torch.device):
    """The calling thread's second stream on this device (default priority) and
    the two events that order it against the current stream, created once per
    (thread, device): two host threads rendering on one device never re-record
    each other's events."""
    key = (threading.get_ident(), dev.index)
    s = _SIDE.get(key)
    if s is None:
        s = _SIDE[key] = (torch.cuda.Stream(device=dev), torch.cuda.Event(), torch.cuda.Event())
    return s


class ColorsBeside:
    """Colours being computed on the second stream.  `wait()` queues the current
    stream's wait for them (once; later calls do nothing) and then releases the
    tensors the second stream reads and writes.  Until then they stay referenced
    here, so the caching allocator (whose blocks serve only the stream that
    allocated them, the current one) cannot hand them out again before the
    current stream is ordered after the colour kernel.  Call it before the
    colours are read, and in a `finally` so that an exception between the fork
    and the join leaves no kernel writing into freed memory."""

    __slots__ = ("colors", "sh_cache", "_main", "_join", "_held")

    def __init__(self, colors, sh_cache, main, join, held):
        self.colors, self.sh_cache = colors, sh_cache
        self._main, self._join, self._held = main, join, held

    def wait(self):
        if self._held is not None:
            self._main.wait_event(self._join)
            self._held = None


def colors_beside(world_to_camera, means, sh_dc, sh_rest, mask,
                  with_cache=False) -> ColorsBeside:
    """The render colours max(SH + 0.5, 0) of the Gaussians in `mask`, computed on
    the calling thread's second stream once the current stream has produced
    `mask` (with_cache: and the colour-gradient cache, `sh_cache` of the returned
    object).  Every input is validated and made contiguous on the current stream
    before the fork, so a copy is ordered before the colour kernel reads it.
    The events are reused: each record comes after the previous wait was queued
    (the returned object's wait())."""
    dev = means.device
    main = torch.cuda.current_stream(dev)
    w2c, means, sh_dc, sh_rest, mask = _cr.sh_render_inputs(world_to_camera, means, sh_dc,
                                                            sh_rest, mask)
    colors = torch.empty((means.shape[0], 3), dtype=torch.float32, device=dev)
    cache = _cr.sh_cache_empty(means.shape[0], dev) if with_cache else None
    side, fork, join = _side_stream(dev)
    fork.record(main)
    side.wait_event(fork)
    pending = ColorsBeside(colors, cache, main, join, (w2c, means, sh_dc, sh_rest, mask))
    try:
        _cr.evaluate_spherical_harmonics_render(w2c, means, sh_dc, sh_rest, mask, out=colors,
                                                beside=True, stream=side, sh_cache=cache)
    finally:
        join.record(side)
    return pending


def _chw(img: torch.Tensor) -> torch.Tensor:
    """(H, W, 3) -> the (1, 3, H, W) view the reference hands to fused_ssim."""
    return img.permute(2, 0, 1).unsqueeze(0)


class RenderL1Function(torch.autograd.Function):
    @staticmethod
    def forward(ctx, means, log_scales, quats_raw, opacity_logits, sh_coeffs_dc, sh_coeffs_rest,
                world_to_camera, intrinsic, target, densifier, width, height, near_plane,
                far_plane, min_opacity, min_radius, max_radius, alpha_threshold,
                transmittance_threshold, chi_squared_threshold, ssim_lambda, ssim_padding,
                schedule_cache, view_id):
        beside = means.shape[0] >= BESIDE_MIN_GAUSSIANS
        # the colour pass also writes the colour-gradient cache: the backward then
        # reads 40 bytes per Gaussian instead of its 180-byte SH row
        cache = None if beside else _cr.sh_cache_empty(means.shape[0], means.device)
        pts, depths, cov, conic, radii, mask, opac, colors = _cr.preprocess_forward(
            means, log_scales, quats_raw, opacity_logits, sh_coeffs_dc, sh_coeffs_rest,
            world_to_camera, intrinsic, near_plane, far_plane, min_opacity, min_radius,
            max_radius, width, height, with_colors=not beside, sh_cache=cache)
        pending = colors_beside(world_to_camera, means, sh_coeffs_dc, sh_coeffs_rest,
                                mask, with_cache=True) if beside else None
        check = None
        try:
            # with a launch order for the forward's tiles from the list lengths; sized
            # by capacities, so no host read of K and M before the blend is queued
            off, ids, list_order, check = _cr.tile_intersection_capped(
                pts, radii, depths, mask, width, height, 16)
            # the blend gradients' accumulators, zeroed by the forward blend launch
            acc = _cr.blend_grad_accumulators(means.shape[0], means.device)
            # the forward's work per tile orders the backward's tiles (heaviest first)
            sched = _cr.tile_schedule(off.shape[0], means.device)
        finally:
            if pending is not None:
                pending.wait()
                colors, cache = pending.colors, pending.sh_cache
        # and, kept per view, the next forward of the same view
        previous = None
        if schedule_cache is not None and view_id is not None:
            previous = schedule_cache.get(view_id)
            if (previous is not None and (previous.device != means.device
                                          or previous.numel() != sched.numel())):
                previous = None
        # the forward launches heaviest first by the view's last render when there
        # is one, else in the order from the list lengths
        def blend_forward():
            return _cr.rasterize_display_l1(
                off, ids, pts, conic, opac, colors, width, height, target, alpha_threshold,
                transmittance_threshold, chi_squared_threshold, clear=acc, schedule=sched,
                forward_schedule=previous,
                forward_order=None if previous is not None else list_order)

        try:
            image, display, loss = blend_forward()
        finally:
            fits = check is None or check.ok()
        if not fits:  # the lists outgrew the capacities: bin with exact sizes, blend again
            off, ids, list_order = _cr.compute_tile_intersection_ordered(
                pts, radii, depths, mask, width, height, 16)
            image, display, loss = blend_forward()
        if schedule_cache is not None and view_id is not None:
            schedule_cache[view_id] = sched
        ssim_saved = ()
        if ssim_lambda > 0.0:
            # SSIM of the reference's rendered_image / 255 (its render() returns the
            # display image; the kernels divide on load) on the permuted (1, 3, H, W)
            # views, and the combined loss from the same launches
            _, maps, loss = _ssim.ssim_forward(_chw(display), _chw(target), ssim_padding,
                                               with_maps=True, img1_divisor=255.0,
                                               other_loss=loss, lam=ssim_lambda)
            ssim_saved = (display,) + tuple(maps)
        ctx.save_for_backward(means, log_scales, quats_raw, opacity_logits, sh_coeffs_dc,
                              sh_coeffs_rest, world_to_camera, intrinsic, target, opac, pts, cov,
                              conic, mask, colors, off, ids, image, acc, sched, *ssim_saved)
        ctx.ssim_lambda = ssim_lambda
        ctx.sh_cache = cache  # written by the forward only, read by the backward
        # acc is zeroed once, by the forward launch: only the first backward may add
        # into it (the gradients it returns are views of it)
        ctx.acc_fresh = True
        ctx.densifier = densifier
        ctx.radii = radii if densifier is not None else None
        ctx.params = (width, height, alpha_threshold, transmittance_threshold,
                      chi_squared_threshold)
        ctx.mark_non_differentiable(display, pts, radii)
        ctx.set_materialize_grads(False)  # no zero gradients for the non-differentiable outputs
        return loss.reshape(()), display, pts, radii

    @staticmethod
    def backward(ctx, grad_loss, grad_display, grad_pts, grad_radii):
        saved = ctx.saved_tensors
        (means, log_scales, quats_raw, logits, dc, rest, w2c, K, target, opac, pts, cov, conic,
         mask, colors, off, ids, image, acc, sched) = saved[:20]
        width, height, a_thr, t_thr, chi = ctx.params
        if grad_loss is None:
            return (None,) * 24
        g = grad_loss.reshape(1).to(torch.float32)
        lam = ctx.ssim_lambda
        extra = None
        if lam > 0.0:  # d loss / d SSIM = -lambda g; its gradient w.r.t. display / 255
            display, m1, m2, m3 = saved[20:]
            extra = _ssim.ssim_backward(g, _chw(display), _chw(target), (m1, m2, m3),
                                        img1_divisor=255.0, grad_scale=-lam)
            extra = extra[0].permute(1, 2, 0)  # laid out like display: (H, W, 3) contiguous
        # a later backward over the same graph (retain_graph) gets freshly zeroed
        # buffers, so it neither adds onto nor overwrites the first one's results
        accumulators = acc if ctx.acc_fresh else None
        ctx.acc_fresh = False
        g_pts, g_conic, g_opac, g_col = _cr.rasterize_l1_backward(
            target, g, off, ids, pts, conic, opac, colors, width, height, image, a_thr, t_thr,
            chi, accumulators=accumulators, grad_display01=extra, loss_scale=1.0 - lam,
            schedule=sched)
        if ctx.densifier is not None:
            ctx.densifier.update(g_pts, ctx.radii, width, height)
        g_means, g_ls, g_qr, g_logit, g_dc, g_rest = _cr.preprocess_backward(
            g_pts, g_conic, g_opac, g_col, means, log_scales, quats_raw, logits, dc, rest, cov,
            mask, w2c, K, width, height, sh_cache=ctx.sh_cache)
        return (g_means, g_ls, g_qr, g_logit, g_dc, g_rest) + (None,) * 18


def render_l1(world_to_camera, intrinsic, width, height, means, log_scales, quats_raw,
              opacity_logits, sh_coeffs_dc, sh_coeffs_rest, target, near_plane=0.01,
              far_plane=100.0, min_opacity=1 / 255, min_radius=0.5, max_radius=128.0,
              alpha_threshold=1e-4, transmittance_threshold=1e-4, chi_squared_threshold=9.21,
              densifier=None, ssim_lambda=0.0, ssim_padding="valid", schedule_cache=None,
              view_id=None):
    """loss = l1_loss(render(...activations of the raw parameters...)[0] / 255, target),
    or with ssim_lambda > 0, (1 - ssim_lambda) * that + ssim_lambda * (1 - SSIM).

    Parameters are the raw training leaves of scripts/train.py:135-143
    (log-scales, un-normalised xyzw quaternions, opacity logits); SH colours use
    max(c + 0.5, 0) (render's default).  Returns (loss, display[H,W,3] in
    [0,255], points_img[N,2], radii[N,2]).

    schedule_cache / view_id: a training loop over a fixed set of views (the
    reference's, scripts/train.py:84,146) can pass a dict and the view's key; each
    step then stores its per-tile work there, and the next step of the same view
    launches its forward tiles heaviest first by it (the backward always uses the
    step's own).  Only the launch order changes: the results are the same with
    or without it.
    """
    return RenderL1Function.apply(
        means, log_scales, quats_raw, opacity_logits, sh_coeffs_dc, sh_coeffs_rest,
        world_to_camera, intrinsic, target, densifier, int(width), int(height),
        float(near_plane), float(far_plane), float(min_opacity), float(min_radius),
        float(max_radius), float(alpha_threshold), float(transmittance_threshold),
        float(chi_squared_threshold), float(ssim_lambda), str(ssim_padding), schedule_cache,
        view_id)
