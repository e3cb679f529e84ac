"""GPU parity at BASELINE configurations 2 and 4 at their full sizes.

- Configuration 2 (100k Gaussians, SH3, 800x800, 8 orbit cameras): camera 0 through
  the drop-in render() against the CPU oracle (image max abs error <= 1e-4 on
  [0,1], parameter gradients relative L2 <= 1e-3), and the eight-camera loss
  through the library's fused step against the drop-in path (relative L2 <= 1e-3,
  the drop-in path activates with PyTorch's exp / sigmoid,
  whose last bits differ from the library's, which can flip a handful of the
  discrete decisions -- L1 signs at near-ties, alpha-test boundaries -- over
  15M pixel-channels; one flipped L1 sign moves a gradient by ~1e-3 relative).
  With the drop-in path given the library's activated values instead, the two
  paths agree to 1e-5 (loss to 1e-6): only float summation order differs.
- Configuration 4 (3M Gaussians, 5% of them large, 64M+ tile keys at 1920x1080):
  the GPU's tile layout bit-exact against the numpy oracle on the GPU's own
  projected values.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import bench
import helpers
import cuda_rasterizer as cr
from cuda_rasterizer.fused import render_l1
from cuda_rasterizer.wrapper import render
from oracle import binning
from oracle import render as orender

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def scene2():
    return bench.config2()


def test_config2_camera0_matches_oracle(gpu, scene2):
    p, cam, target = scene2["params"], scene2["cameras"][0], scene2["targets"][0]
    img_g, loss_g, grads_g, _, _ = helpers.forward_backward(render, p, cam, target, gpu)
    img_c, loss_c, grads_c, _, _ = helpers.forward_backward(orender.render, p, cam, target, "cpu")
    assert helpers.max_abs(img_g / 255.0, img_c / 255.0) <= 1e-4
    assert abs(float(loss_g) - float(loss_c)) <= 1e-5
    for k in helpers.PARAMS:
        assert helpers.rel_l2(grads_g[k], grads_c[k]) <= 1e-3, k


def test_config2_eight_cameras_fused_equals_drop_in(gpu, scene2):
    p = scene2["params"]

    def leaves():
        return {k: v.to(gpu).clone().requires_grad_(True) for k, v in p.items()}

    a, b = leaves(), leaves()
    loss_a = loss_b = 0.0
    for cam, target in zip(scene2["cameras"], scene2["targets"]):
        w2c, K, tgt = cam["w2c"].to(gpu), cam["K"].to(gpu), target.to(gpu)
        W, H = cam["width"], cam["height"]
        scales, quats, opac = helpers.activated(a)
        img, _, _ = render(w2c, K, W, H, a["means"], scales, quats, opac, a["sh_dc"],
                           a["sh_rest"])
        loss_a = loss_a + torch.nn.functional.l1_loss(img / 255.0, tgt)
        lb, _, _, _ = render_l1(w2c, K, W, H, b["means"], b["log_scales"], b["quats_raw"],
                                b["opacity_logits"], b["sh_dc"], b["sh_rest"], tgt)
        loss_b = loss_b + lb
    loss_a.backward()
    loss_b.backward()
    assert abs(float(loss_b.detach()) - float(loss_a.detach())) <= 1e-5 * float(loss_a.detach())
    for k in helpers.PARAMS:
        assert helpers.rel_l2(b[k].grad, a[k].grad) <= 1e-3, k


class _LibraryActivate(torch.autograd.Function):
    """The library's activation kernels (gs_activate / gs_activate_backward) as an
    autograd node, to give the drop-in path the fused step's activated values."""

    @staticmethod
    def forward(ctx, log_scales, quats_raw, logits):
        scales, quats, opac = cr.activate(log_scales, quats_raw, logits)
        ctx.save_for_backward(scales, quats_raw, opac)
        return scales, quats, opac

    @staticmethod
    def backward(ctx, g_scales, g_quats, g_opac):
        scales, quats_raw, opac = ctx.saved_tensors
        c = [None if g is None else g.contiguous() for g in (g_scales, g_quats, g_opac)]
        return cr.activate_backward(*c, scales, quats_raw, opac)


def test_config2_eight_cameras_same_activations_agree_closely(gpu, scene2):
    """The cause of the 1e-3 bar above, shown: with the drop-in path given the
    library's activated values (bit-equal to the fused step's), every discrete
    decision matches, and the two paths differ only by float summation order
    (the loss sum and the gradient atomics)."""
    p = scene2["params"]

    def leaves():
        return {k: v.to(gpu).clone().requires_grad_(True) for k, v in p.items()}

    a, b = leaves(), leaves()
    loss_a = loss_b = 0.0
    for cam, target in zip(scene2["cameras"], scene2["targets"]):
        w2c, K, tgt = cam["w2c"].to(gpu), cam["K"].to(gpu), target.to(gpu)
        W, H = cam["width"], cam["height"]
        scales, quats, opac = _LibraryActivate.apply(a["log_scales"], a["quats_raw"],
                                                     a["opacity_logits"])
        img, _, _ = render(w2c, K, W, H, a["means"], scales, quats, opac, a["sh_dc"],
                           a["sh_rest"])
        loss_a = loss_a + torch.nn.functional.l1_loss(img / 255.0, tgt)
        lb, _, _, _ = render_l1(w2c, K, W, H, b["means"], b["log_scales"], b["quats_raw"],
                                b["opacity_logits"], b["sh_dc"], b["sh_rest"], tgt)
        loss_b = loss_b + lb
    loss_a.backward()
    loss_b.backward()
    assert abs(float(loss_b.detach()) - float(loss_a.detach())) <= 1e-6 * float(loss_a.detach())
    for k in helpers.PARAMS:
        assert helpers.rel_l2(b[k].grad, a[k].grad) <= 1e-5, k


def test_config4_layout_bitexact(gpu):
    scene = bench.config4()
    p, cam = scene["params"], scene["camera"]
    scales, quats, opac = helpers.activated(p)
    d = lambda t: t.to(gpu)  # noqa: E731
    g_pts, g_depths, _, _, g_radii, g_mask = cr.project_points(
        d(p["means"]), d(scales), d(quats), d(opac), d(cam["w2c"]), d(cam["K"]), cam["near"],
        100.0, 1 / 255, 0.5, 128.0, cam["width"], cam["height"])
    off, ids = cr.compute_tile_intersection(g_pts, g_radii, g_depths, g_mask, cam["width"],
                                            cam["height"], 16)
    ref_off, ref_ids, _, _ = binning.tile_layout(
        g_pts.cpu().numpy(), g_radii.cpu().numpy(), g_depths.cpu().numpy(),
        g_mask.cpu().numpy(), cam["width"], cam["height"], 16)
    assert len(ref_ids) > 50_000_000  # heavy tile duplication, as the configuration intends
    assert np.array_equal(off.cpu().numpy(), ref_off)
    assert np.array_equal(ids.cpu().numpy(), ref_ids)
