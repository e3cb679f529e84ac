"""GPU parity on the reference's own edge cases and the unfused drop-in chain.

- The reference's single-tile blend check (scripts/check_cuda_gradients.py:341-427):
  16 Gaussians in one 16x16 tile with wide conics, alpha and transmittance
  thresholds 0 and chi-square 20 (the staged cut-off and strip culling scale
  with chi-square).  Image <= 1e-4, gradients relative L2 <= 1e-3 against the
  oracle's vectorised tile loop and its per-pixel brute force.
- The reference's radius limits min_radius = 0.1, max_radius = 256
  (check_cuda_gradients.py:226-230), on its own projection case and on a scene
  whose splats reach 128-256 px (up to 33 x 33 tiles): projection and tile
  layout bit-exact, image <= 1e-4, gradients <= 1e-3.
- render_unfused: the seven functions composed as the reference's
  src/cuda/wrapper.py:223-294 composes them, against the reference goldens.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import helpers
import cuda_rasterizer as cr
from cuda_rasterizer.wrapper import render, render_unfused
from oracle import binning, blend, preprocess

pytestmark = pytest.mark.gpu

IMG_TOL = 1e-4
GRAD_TOL = 1e-3
INPUTS = ("points_image", "cov_inv_image", "opacities", "colors")


def _single_tile_case(seed):
    """Inputs of check_rasterize (check_cuda_gradients.py:341-362), drawn with a CPU
    generator: 16 Gaussians at [2, 14]^2 in one tile, A, C ~ U[0.01, 0.04],
    B ~ U[-0.0025, 0.0025], opacity ~ U[0.55, 0.8], colours ~ U[0, 1]."""
    g = torch.Generator().manual_seed(seed)
    count = 16
    pts = torch.rand(count, 2, generator=g) * 12.0 + 2.0
    conic = torch.zeros(count, 3)
    conic[:, 0] = torch.rand(count, generator=g) * 0.03 + 0.01
    conic[:, 1] = (torch.rand(count, generator=g) - 0.5) * 0.005
    conic[:, 2] = torch.rand(count, generator=g) * 0.03 + 0.01
    opac = torch.rand(count, generator=g) * 0.25 + 0.55
    colors = torch.rand(count, 3, generator=g)
    return pts, conic, opac, colors


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_single_tile_chi20_no_thresholds(gpu, seed):
    W = H = 16
    off = torch.tensor([0], dtype=torch.int32)
    ids = torch.arange(16, dtype=torch.int32)
    args = (W, H, 16, 0.0, 0.0, 20.0)
    ins = [t.clone().requires_grad_(True) for t in _single_tile_case(seed)]
    ref = blend.rasterize(off, ids, *ins, *args)
    brute = blend.rasterize_bruteforce(off, ids, *ins, *args)
    assert helpers.max_abs(ref, brute) <= 1e-6
    up = torch.randn(H, W, 3, generator=torch.Generator().manual_seed(seed + 10))
    (ref * up).sum().backward()
    d = [t.detach().to(gpu) for t in ins]
    image = cr.rasterize(off.to(gpu), ids.to(gpu), *d, *args)
    assert helpers.max_abs(image, ref) <= IMG_TOL
    for img in (None, image):  # replayed forward and saved image
        grads = cr.rasterize_backward(up.to(gpu), off.to(gpu), ids.to(gpu), *d, *args,
                                      rendered_image=img)
        for name, a, t in zip(INPUTS, grads, ins):
            assert helpers.rel_l2(a, t.grad) <= GRAD_TOL, name


def test_project_points_reference_radius_case(gpu):
    """check_project_points (check_cuda_gradients.py:196-338): 256 Gaussians of scale
    0.8-1.0 at depth 2-2.5, f = 60, 64x64, min_radius 0.1, max_radius 256 (radii
    of ~70 px, larger than the image).  Outputs bit-exact; gradients <= 1e-3
    against the oracle's autograd."""
    g = torch.Generator().manual_seed(0)
    count, W, H = 256, 64, 64
    w2c = torch.eye(4)
    K = torch.tensor([[60.0, 0.0, W / 2], [0.0, 60.0, H / 2], [0.0, 0.0, 1.0]])
    means = (torch.rand(count, 3, generator=g) - 0.5) * 1.0
    means[:, 2] = torch.rand(count, generator=g) * 0.5 + 2.0
    scales = torch.rand(count, 3, generator=g) * 0.2 + 0.8
    q = torch.randn(count, 4, generator=g)
    q = q / q.norm(dim=1, keepdim=True)
    opac = torch.full((count,), 0.8)
    args = (0.01, 100.0, 1 / 255, 0.1, 256.0, W, H)
    leaves = [t.clone().requires_grad_(True) for t in (means, scales, q)]
    ref = preprocess.project_points(*leaves, opac, w2c, K, *args)
    mask = ref[5]
    assert int(mask.sum()) > 200 and float(ref[4].max()) > 64.0
    d = lambda t: t.detach().to(gpu)  # noqa: E731
    got = cr.project_points(*[d(t) for t in leaves], d(opac), d(w2c), d(K), *args)
    for a, b in zip(got, ref):
        assert helpers.same(a, b)
    up_pts = torch.randn(count, 2, generator=g)
    up_conic = torch.randn(count, 3, generator=g) * 0.1
    ((ref[0] * up_pts).sum() + (ref[3] * up_conic).sum()).backward()
    grads = cr.project_points_backward(d(up_pts), d(up_conic), *[d(t) for t in leaves], d(opac),
                                       d(w2c), d(K), W, H, got[2], got[5])
    m = mask.unsqueeze(1).float()
    for a, t in zip(grads, leaves):
        assert helpers.rel_l2(a.cpu() * m, t.grad * m) <= GRAD_TOL


def _large_splat_scene(n, W, H, seed):
    """Camera-space Gaussians (W2C = I, f = 500) with 10% of scales ~ U[0.15, 0.3] at
    depth 1.6-2.4 -- projected 3-sigma radii of about 90-280 px -- and the rest small."""
    g = torch.Generator().manual_seed(seed)
    means = torch.empty(n, 3)
    means[:, 2] = torch.rand(n, generator=g) * 0.8 + 1.6
    means[:, 0] = (torch.rand(n, generator=g) * 1.6 - 0.8) * means[:, 2] * W / 1000
    means[:, 1] = (torch.rand(n, generator=g) * 1.6 - 0.8) * means[:, 2] * H / 1000
    log_s = torch.randn(n, 3, generator=g) * 0.4 - 4.0
    big = torch.rand(n, generator=g) < 0.1
    log_s[big] = torch.log(torch.rand(int(big.sum()), 3, generator=g) * 0.15 + 0.15)
    p = dict(means=means, log_scales=log_s, quats_raw=torch.randn(n, 4, generator=g),
             opacity_logits=torch.randn(n, generator=g) * 1.5 - 1.0,
             sh_dc=torch.randn(n, 3, generator=g) * 0.3,
             sh_rest=torch.randn(n, 15, 3, generator=g) * 0.05)
    cam = dict(w2c=torch.eye(4), K=helpers.intrinsic(500.0, W, H), width=W, height=H)
    return p, cam


def test_large_splats_radius_limits(gpu):
    """min_radius 0.1 / max_radius 256 with splats of 128-256 px through projection,
    binning and both blend kernels (the drop-in render() path)."""
    W, H = 640, 480
    p, cam = _large_splat_scene(3_000, W, H, seed=5)
    scales, quats, opac = helpers.activated(p)
    args = (cam["w2c"], cam["K"], 0.01, 100.0, 1 / 255, 0.1, 256.0, W, H)
    pts, depths, cov, conic, radii, mask = preprocess.project_points(p["means"], scales, quats,
                                                                     opac, *args)
    r = torch.maximum(radii[:, 0], radii[:, 1])[mask]
    assert int(((r > 128.0) & (r <= 256.0)).sum()) >= 20
    d = lambda t: t.detach().to(gpu)  # noqa: E731
    got = cr.project_points(d(p["means"]), d(scales), d(quats), d(opac), d(args[0]), d(args[1]),
                            *args[2:])
    for a, b in zip(got, (pts, depths, cov, conic, radii, mask)):
        assert helpers.same(a, b)
    ref_off, ref_ids, ref_keys, ref_counts = binning.tile_layout(
        pts.detach().numpy(), radii.detach().numpy(), depths.detach().numpy(), mask.numpy(), W,
        H, 16)
    assert int(ref_counts.max()) >= 17 * 17
    off, ids, keys, touched = cr.compute_tile_intersection_debug(got[0], got[4], got[1], got[5],
                                                                 W, H, 16)
    assert np.array_equal(off.cpu().numpy(), ref_off)
    assert np.array_equal(ids.cpu().numpy(), ref_ids)
    assert np.array_equal(keys.cpu().numpy().view(np.uint64), ref_keys)
    assert np.array_equal(touched.cpu().numpy().astype(np.int64), ref_counts)
    colors = torch.rand(3_000, 3, generator=torch.Generator().manual_seed(6))
    opac_m = torch.where(mask, opac, torch.zeros_like(opac))
    ins = [t.detach().clone().requires_grad_(True) for t in (pts, conic, opac_m, colors)]
    bargs = (W, H, 16, 1e-4, 1e-4, 9.21)
    ref = blend.rasterize(off.cpu(), ids.cpu(), *ins, *bargs)
    up = torch.randn(H, W, 3, generator=torch.Generator().manual_seed(7))
    (ref * up).sum().backward()
    image = cr.rasterize(off, ids, *[d(t) for t in ins], *bargs)
    assert helpers.max_abs(image.clamp(0, 1), ref.clamp(0, 1)) <= IMG_TOL
    grads = cr.rasterize_backward(up.to(gpu), off, ids, *[d(t) for t in ins], *bargs,
                                  rendered_image=image)
    for name, a, t in zip(INPUTS, grads, ins):
        assert helpers.rel_l2(a, t.grad) <= GRAD_TOL, name


def test_large_splats_render_end_to_end(gpu):
    """The same scene through render() and render_unfused() with min_radius 0.1 and
    max_radius 256, fwd + bwd of an L1 loss, against the oracle render."""
    from oracle import render as orender

    W, H = 640, 480
    p, cam = _large_splat_scene(3_000, W, H, seed=8)
    target = torch.rand(H, W, 3, generator=torch.Generator().manual_seed(9))
    kw = dict(min_radius=0.1, max_radius=256.0)
    img_c, _, grads_c, _, _ = helpers.forward_backward(orender.render, p, cam, target, "cpu", **kw)
    for fn in (render, render_unfused):
        img_g, _, grads_g, _, _ = helpers.forward_backward(fn, p, cam, target, gpu, **kw)
        assert helpers.max_abs(img_g / 255.0, img_c / 255.0) <= IMG_TOL
        for k in helpers.PARAMS:
            assert helpers.rel_l2(grads_g[k], grads_c[k]) <= GRAD_TOL, (fn.__name__, k)


@pytest.mark.parametrize("name", ["box_sh0", "orbit_sh3", "sigmoid", "e2e_large"])
def test_render_unfused_matches_reference_golden(gpu, name):
    """The reference's own composition of the seven functions (RasterizeFunction,
    SphericalHarmonicsFunction + clamp_min in PyTorch, clamp * 255 in PyTorch)
    against the goldens written by the reference's Torch rasterizer, and against
    render() (fused glue) on the same inputs."""
    case = helpers.load_golden()[name]
    p, cam, target = helpers.golden_case_tensors(case)
    kind, sig = str(case["loss_kind"]), bool(case["sh_sigmoid"])
    image, _, grads, _, _ = helpers.forward_backward(render_unfused, p, cam, target, gpu,
                                                     loss_kind=kind, sh_sigmoid=sig)
    assert helpers.max_abs(image / 255.0, torch.from_numpy(case["image"]) / 255.0) <= IMG_TOL
    image_f, _, grads_f, _, _ = helpers.forward_backward(render, p, cam, target, gpu,
                                                         loss_kind=kind, sh_sigmoid=sig)
    assert helpers.max_abs(image, image_f) <= 1e-4 * 255
    for k in helpers.PARAMS:
        ref = torch.from_numpy(case["grad_" + k])
        if float(ref.norm()) == 0.0:
            assert float(grads[k].norm()) == 0.0, k
        else:
            assert helpers.rel_l2(grads[k], ref) <= GRAD_TOL, k
            assert helpers.rel_l2(grads[k], grads_f[k]) <= 1e-4, k
