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


def test_render_colours_beside_binning_equal_the_plain_launch(gpu, monkeypatch):
    """With grad enabled (and, here, any scene size) render() computes its
    colours on a second stream while binning runs; without grad on the current
    stream: the same display, and repeated calls (reused fork/join events) stay
    bit-equal."""
    import cuda_rasterizer.fused as fused

    monkeypatch.setattr(fused, "BESIDE_MIN_GAUSSIANS", 0)
    p, cam, _ = helpers.scene_orbit(30_000, 320, 240, 440.0, seed=41)
    dev = gpu
    w2c, K = cam["w2c"].to(dev), cam["K"].to(dev)
    leaves = {k: v.to(dev).requires_grad_(True) for k, v in p.items()}
    scales, quats, opac = helpers.activated(leaves)
    args = (w2c, K, cam["width"], cam["height"], leaves["means"], scales, quats, opac,
            leaves["sh_dc"], leaves["sh_rest"])
    with torch.no_grad():
        plain, _, _ = render(*args)
    for _ in range(3):
        beside, _, _ = render(*args)
        assert beside.requires_grad
        assert torch.equal(beside.detach(), plain)


def test_render_empty_frame(gpu):
    """Everything behind the camera: black image, zero gradients, no failure."""
    p, cam, target = helpers.scene_box(500, 64, 64, 75.0, seed=4)
    p["means"][:, 2] = -5.0
    img, loss, grads, _, radii = helpers.forward_backward(render, p, cam, target, gpu)
    assert float(img.abs().max()) == 0.0
    assert float(radii.abs().max()) == 0.0
    assert all(float(g.abs().max()) == 0.0 for g in grads.values())


def test_fused_colors_equal_unfused_sequence(gpu):
    """evaluate_spherical_harmonics_render == clamp_min(evaluate_sh(-R^T t) + 0.5, 0),
    forward and gradient (autograd through the unfused torch sequence)."""
    import cuda_rasterizer as cr

    p, cam, _ = helpers.scene_orbit(4_000, 160, 120, 220.0, seed=11)
    g = torch.Generator().manual_seed(5)
    n = 4_000
    means = p["means"].to(gpu)
    dc = (torch.randn(n, 3, generator=g) * 2.0).to(gpu)  # many colours below -0.5 (clamped)
    rest = p["sh_rest"].to(gpu)
    mask = (torch.rand(n, generator=g) > 0.2).to(gpu)
    w2c = cam["w2c"].to(gpu)
    fused = cr.evaluate_spherical_harmonics_render(w2c, means, dc, rest, mask)
    cam_pos = -w2c[:3, :3].t() @ w2c[:3, 3]
    raw = cr.evaluate_spherical_harmonics(cam_pos, means, dc, rest, mask)
    unfused = torch.clamp_min(raw + 0.5, 0.0)
    assert float((unfused == 0).float().mean()) > 0.05  # the clamp is exercised
    assert helpers.max_abs(fused, unfused) <= 1e-6
    assert torch.all(fused[~mask] == 0.5)

    up = torch.randn(n, 3, generator=g).to(gpu)
    gm, gdc, grest = cr.evaluate_spherical_harmonics_render_backward(up, w2c, means, dc, rest, mask)
    clamp_grad = up * ((raw + 0.5) >= 0)
    rm, rdc, rrest = cr.evaluate_spherical_harmonics_backward(clamp_grad, cam_pos, means, dc, rest,
                                                              raw, mask, False)
    for a, b in ((gm, rm), (gdc, rdc), (grest, rrest)):
        assert helpers.rel_l2(a, b) <= 1e-5


def test_display_blend_equals_clamp_of_image(gpu):
    """rasterize_display: the image is rasterize()'s, display = clamp(image,0,1)*255
    exactly; its backward equals rasterize_backward of the clamp's gradient."""
    import cuda_rasterizer as cr

    p, cam, _ = helpers.scene_orbit(6_000, 160, 120, 220.0, seed=12, log_scale=(-3.5, 0.5),
                                    opacity_std=3.0)
    scales, quats, opac = helpers.activated(p)
    d = lambda t: t.to(gpu)  # noqa: E731
    pts, depths, _, conic, radii, mask = cr.project_points(
        d(p["means"]), d(scales), d(quats), d(opac), d(cam["w2c"]), d(cam["K"]), 0.01, 100.0,
        1 / 255, 0.5, 128.0, 160, 120)
    colors = (torch.rand(6_000, 3, generator=torch.Generator().manual_seed(2)) * 3.0).to(gpu)
    off, ids = cr.compute_tile_intersection(pts, radii, depths, mask, 160, 120, 16)
    args = (160, 120, 16, 1e-4, 1e-4, 9.21)
    ins = (off, ids, pts, conic, d(opac), colors)
    image = cr.rasterize(*ins, *args)
    image2, display = cr.rasterize_display(*ins, *args)
    assert torch.equal(image, image2)
    assert torch.equal(display, image.clamp(0, 1) * 255)
    assert float((image > 1).float().mean()) > 0.01  # the upper clamp is exercised
    up = torch.randn(120, 160, 3, generator=torch.Generator().manual_seed(3)).to(gpu)
    got = cr.rasterize_display_backward(up, *ins, *args, rendered_image=image)
    want = cr.rasterize_backward(up * 255 * ((image >= 0) & (image <= 1)), *ins, *args,
                                 rendered_image=image)
    for a, b in zip(got, want):
        assert helpers.rel_l2(a, b) <= 1e-6


def test_render_passes_tile_schedule_only_with_grad(gpu, monkeypatch):
    """render() gives the blend forward a tile schedule when a backward can follow
    and hands the same buffer to the blend backward (heaviest tiles first); under
    torch.no_grad() no schedule is computed."""
    import cuda_rasterizer as cr

    seen = {}
    fwd, bwd = cr.rasterize_display, cr.rasterize_display_backward

    def spy_fwd(*args, schedule=None, **kw):
        seen["fwd"] = schedule
        return fwd(*args, schedule=schedule, **kw)

    def spy_bwd(*args, schedule=None, **kw):
        seen["bwd"] = schedule
        return bwd(*args, schedule=schedule, **kw)

    monkeypatch.setattr(cr, "rasterize_display", spy_fwd)
    monkeypatch.setattr(cr, "rasterize_display_backward", spy_bwd)
    p, cam, _ = helpers.scene_box(3000, 96, 80, 110.0, seed=31)
    leaves = {k: v.to(gpu).clone().requires_grad_(True) for k, v in p.items()}

    def run():
        scales, quats, opac = helpers.activated(leaves)
        return render(cam["w2c"].to(gpu), cam["K"].to(gpu), cam["width"], cam["height"],
                      leaves["means"], scales, quats, opac, leaves["sh_dc"], leaves["sh_rest"])[0]

    run().sum().backward()
    assert seen["fwd"] is not None and seen["bwd"] is seen["fwd"]
    seen.clear()
    with torch.no_grad():
        run()
    assert seen["fwd"] is None and "bwd" not in seen


def test_colours_beside_binning_with_non_contiguous_inputs(gpu, monkeypatch):
    """The colour pass on the second stream reads contiguous copies that are made
    on the current stream before the fork and held until the join: a transposed
    world_to_camera, means sliced from a wider array and sh_rest sliced from a
    16-coefficient array give the display and gradients of contiguous inputs,
    in render() and in render_l1, over repeated calls; a failure between the
    fork and the join propagates and the next call is unaffected."""
    import cuda_rasterizer as cr
    import cuda_rasterizer.fused as fused
    from cuda_rasterizer.fused import render_l1

    monkeypatch.setattr(fused, "BESIDE_MIN_GAUSSIANS", 0)
    n, W, H = 30_000, 320, 240
    p, cam, target = helpers.scene_orbit(n, W, H, 440.0, seed=43)
    w2c, K, tgt = cam["w2c"].to(gpu), cam["K"].to(gpu), target.to(gpu)
    w2c_t = w2c.t().contiguous().t()  # the same values, column-major
    assert not w2c_t.is_contiguous()

    def leaves(contiguous):
        out = {k: v.to(gpu).clone().requires_grad_(True) for k, v in p.items()}
        if contiguous:
            return out, out
        wide_means = torch.zeros(n, 5, device=gpu)
        wide_means[:, 1:4] = out["means"].detach()
        wide_means.requires_grad_(True)
        wide_rest = torch.zeros(n, 16, 3, device=gpu)
        wide_rest[:, 1:] = out["sh_rest"].detach()
        wide_rest.requires_grad_(True)
        views = dict(out, means=wide_means[:, 1:4], sh_rest=wide_rest[:, 1:])
        assert not views["means"].is_contiguous() and not views["sh_rest"].is_contiguous()
        return views, dict(out, means=wide_means, sh_rest=wide_rest)

    def grads(roots, contiguous):
        g = {k: t.grad for k, t in roots.items()}
        if not contiguous:  # the wide arrays' gradients, cut to the views
            g["means"], g["sh_rest"] = g["means"][:, 1:4], g["sh_rest"][:, 1:]
        return g

    ref, ref_roots = leaves(True)
    sc, qq, op = helpers.activated(ref)
    disp_ref, _, _ = render(w2c, K, W, H, ref["means"], sc, qq, op, ref["sh_dc"], ref["sh_rest"])
    loss_ref, _, _, _ = render_l1(w2c, K, W, H, ref["means"], ref["log_scales"], ref["quats_raw"],
                                  ref["opacity_logits"], ref["sh_dc"], ref["sh_rest"], tgt)
    loss_ref.backward()
    g_ref = grads(ref_roots, True)
    for _ in range(2):
        v, roots = leaves(False)
        sc, qq, op = helpers.activated(v)
        disp, _, _ = render(w2c_t, K, W, H, v["means"], sc, qq, op, v["sh_dc"], v["sh_rest"])
        assert torch.equal(disp.detach(), disp_ref.detach())
        loss, _, _, _ = render_l1(w2c_t, K, W, H, v["means"], v["log_scales"], v["quats_raw"],
                                  v["opacity_logits"], v["sh_dc"], v["sh_rest"], tgt)
        assert float(loss) == float(loss_ref)
        loss.backward()
        g = grads(roots, False)
        for k in g_ref:
            assert helpers.rel_l2(g[k], g_ref[k]) <= 1e-5, k

    # binning fails after the fork: the error reaches the caller and the wait
    # for the colours is still queued, so the next call is unaffected
    real = cr.tile_intersection_capped

    def failing(*a, **k):
        raise cr.RasterizerError("planted binning failure")

    monkeypatch.setattr(cr, "tile_intersection_capped", failing)
    v, _ = leaves(False)
    with pytest.raises(cr.RasterizerError, match="planted"):
        render_l1(w2c_t, K, W, H, v["means"], v["log_scales"], v["quats_raw"],
                  v["opacity_logits"], v["sh_dc"], v["sh_rest"], tgt)
    monkeypatch.setattr(cr, "tile_intersection_capped", real)
    v, _ = leaves(False)
    loss, _, _, _ = render_l1(w2c_t, K, W, H, v["means"], v["log_scales"], v["quats_raw"],
                              v["opacity_logits"], v["sh_dc"], v["sh_rest"], tgt)
    assert float(loss) == float(loss_ref)


def test_render_preprocess_backward_equals_the_two_entries(gpu):
    """gs_render_preprocess_backward (render()'s projection + colour node backward,
    one kernel) equals project_points_backward and
    evaluate_spherical_harmonics_render_backward bit for bit, the means gradient
    being their sum (as autograd adds the two nodes' gradients)."""
    import cuda_rasterizer as cr

    n = 9_000
    p, cam, _ = helpers.scene_orbit(n, 200, 150, 260.0, seed=17, log_scale=(-3.5, 0.5))
    scales, quats, opac = helpers.activated(p)
    g = torch.Generator().manual_seed(23)
    d = lambda t: t.to(gpu)  # noqa: E731
    w2c, K = d(cam["w2c"]), d(cam["K"])
    means, scales, quats, opac = d(p["means"]), d(scales), d(quats), d(opac)
    dc = d(torch.randn(n, 3, generator=g) * 0.8)  # some colours clamped at 0
    rest = d(p["sh_rest"])
    pts, depths, cov, conic, radii, mask = cr.project_points(means, scales, quats, opac, w2c, K,
                                                             0.01, 100.0, 1 / 255, 0.5, 128.0,
                                                             200, 150)
    assert 0 < int(mask.sum()) < n
    gp = d(torch.randn(n, 2, generator=g))
    gc = d(torch.randn(n, 3, generator=g))
    gcol = d(torch.randn(n, 3, generator=g))
    fm, fs, fq, fdc, frest = cr.render_preprocess_backward(gp, gc, gcol, means, scales, quats, dc,
                                                            rest, cov, mask, w2c, K, 200, 150)
    pm, ps, pq = cr.project_points_backward(gp, gc, means, scales, quats, opac, w2c, K, 200, 150,
                                            cov, mask)
    sm, sdc, srest = cr.evaluate_spherical_harmonics_render_backward(gcol, w2c, means, dc, rest,
                                                                     mask)
    assert torch.equal(fm, pm + sm)
    assert torch.equal(fs, ps) and torch.equal(fq, pq)
    assert torch.equal(fdc, sdc) and torch.equal(frest, srest)
    # from the forward's colour-gradient cache instead of the SH rows: bit-equal
    cache = cr.sh_cache_empty(n, gpu)
    col_c = cr.evaluate_spherical_harmonics_render(w2c, means, dc, rest, mask, sh_cache=cache)
    assert torch.equal(col_c, cr.evaluate_spherical_harmonics_render(w2c, means, dc, rest, mask))
    cached = cr.render_preprocess_backward(gp, gc, gcol, means, scales, quats, None, None, cov,
                                           mask, w2c, K, 200, 150, sh_cache=cache)
    for a, b in zip(cached, (fm, fs, fq, fdc, frest)):
        assert torch.equal(a, b)
    # a quaternion view that is not 16-byte aligned (the entry takes any row start)
    wide = torch.zeros(n * 4 + 1, device=gpu)
    wide[1:] = quats.flatten()
    quats_odd = wide[1:].view(n, 4)
    assert quats_odd.data_ptr() % 16 != 0
    om, os_, oq, odc, orest = cr.render_preprocess_backward(gp, gc, gcol, means, scales, quats_odd,
                                                            dc, rest, cov, mask, w2c, K, 200, 150)
    assert torch.equal(oq, fq) and torch.equal(om, fm)
