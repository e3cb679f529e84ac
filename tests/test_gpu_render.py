"""GPU parity: render() end to end (forward + backward of an L1 loss).

Against the golden vectors written by the reference's own Torch rasterizer
(tests/golden) and against the CPU oracle on configuration-1 inputs.
Tolerances: image max abs error <= 1e-4 on the [0,1] scale, each parameter
gradient relative L2 <= 1e-3 (north star).
"""

from __future__ import annotations

import pytest
import torch

import helpers
from cuda_rasterizer.wrapper import render
from oracle import render as orender

pytestmark = pytest.mark.gpu

IMG_TOL = 1e-4
GRAD_TOL = 1e-3


@pytest.mark.parametrize("name", ["box_sh0", "orbit_sh3", "sigmoid", "e2e_large"])
def test_render_matches_reference_golden(gpu, name):
    case = helpers.load_golden()[name]
    p, cam, target = helpers.golden_case_tensors(case)
    image, loss, grads, points_img, radii = helpers.forward_backward(
        render, p, cam, target, gpu, loss_kind=str(case["loss_kind"]),
        sh_sigmoid=bool(case["sh_sigmoid"]))
    assert helpers.max_abs(image / 255.0, torch.from_numpy(case["image"]) / 255.0) <= IMG_TOL
    for k in helpers.PARAMS:
        ref = torch.from_numpy(case["grad_" + k])
        if float(ref.norm()) == 0.0:
            assert float(grads[k].norm()) == 0.0, k
        else:
            assert helpers.rel_l2(grads[k], ref) <= GRAD_TOL, k


def test_render_config1_matches_oracle(gpu):
    """10k Gaussians, SH0, 256x256, fx=fy=300, seed 0."""
    import bench

    scene = bench.config1()
    p, cam, target = scene["params"], scene["camera"], scene["target"]
    cam2 = dict(w2c=cam["w2c"], K=cam["K"], width=cam["width"], height=cam["height"])
    img_g, loss_g, grads_g, pts_g, radii_g = helpers.forward_backward(render, p, cam2, target, gpu)
    img_c, loss_c, grads_c, _, _ = helpers.forward_backward(orender.render, p, cam2, target, "cpu")
    assert helpers.max_abs(img_g / 255.0, img_c / 255.0) <= IMG_TOL
    assert abs(float(loss_g) - float(loss_c)) <= 1e-5
    for k in helpers.PARAMS:
        if float(grads_c[k].norm()) == 0.0:
            assert float(grads_g[k].norm()) == 0.0, k
        else:
            assert helpers.rel_l2(grads_g[k], grads_c[k]) <= GRAD_TOL, k


def test_points_img_grad_and_radii(gpu):
    """render() returns points_img whose .grad is dL/d(points_img) and radii whose
    positive rows are the visible Gaussians (what src/strategy.py:47-68 reads)."""
    p, cam, target = helpers.scene_orbit(5_000, 160, 120, 220.0, seed=3, log_scale=(-3.5, 0.5))
    img_g, _, _, pts_g, radii_g = helpers.forward_backward(render, p, cam, target, gpu)
    assert pts_g.grad is not None and pts_g.grad.shape == (5_000, 2)
    leaves = {k: v.clone().requires_grad_(True) for k, v in p.items()}
    scales, quats, opac = helpers.activated(leaves)
    out = orender.render_stages(cam["w2c"], cam["K"], 160, 120, leaves["means"], scales, quats, opac,
                                leaves["sh_dc"], leaves["sh_rest"])
    out["points_image"].retain_grad()
    torch.nn.functional.l1_loss(out["image"] / 255.0, target).backward()
    keep = out["proj"]["keep"]
    assert torch.equal((radii_g.cpu() > 0).all(dim=1), keep)
    ref = torch.where(keep.unsqueeze(1), out["points_image"].grad, 0.0)
    assert helpers.rel_l2(pts_g.grad.cpu() * keep.unsqueeze(1), ref) <= GRAD_TOL


def test_render_empty_frame(gpu):
    """Everything behind the camera: black image, zero gradients, no failure."""
    p, cam, target = helpers.scene_box(500, 64, 64, 75.0, seed=4)
    p["means"][:, 2] = -5.0
    img, loss, grads, _, radii = helpers.forward_backward(render, p, cam, target, gpu)
    assert float(img.abs().max()) == 0.0
    assert float(radii.abs().max()) == 0.0
    assert all(float(g.abs().max()) == 0.0 for g in grads.values())
