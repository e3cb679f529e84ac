"""GPU parity: projection and spherical harmonics vs the CPU oracle.

Forward projection outputs are compared bit-exactly (identical fp32 inputs,
identical operation order); gradients within relative L2 1e-4 (the north-star
bound is 1e-3).
"""

from __future__ import annotations

import pytest
import torch

import helpers
import cuda_rasterizer as cr
from oracle import preprocess

pytestmark = pytest.mark.gpu

NEAR, FAR, MIN_O, MIN_R, MAX_R = 0.01, 100.0, 1 / 255, 0.5, 128.0


def _scenes():
    yield "cfg1", helpers.scene_box(10_000, 256, 256, 300.0, seed=0)
    yield "cfg2cam", helpers.scene_orbit(20_000, 800, 800, 1100.0, seed=1)
    yield "large", helpers.scene_box(3_000, 100, 70, 80.0, seed=2, log_scale=(-1.5, 0.8), z=(0.5, 6.0))


SCENES = dict(_scenes())


def _api_inputs(name):
    p, cam, _ = SCENES[name]
    scales, quats, opac = helpers.activated(p)
    return p["means"], scales, quats, opac, cam


@pytest.mark.parametrize("name", list(SCENES))
def test_project_points_bitexact(gpu, name):
    means, scales, quats, opac, cam = _api_inputs(name)
    args = (cam["w2c"], cam["K"], NEAR, FAR, MIN_O, MIN_R, MAX_R, cam["width"], cam["height"])
    ref = preprocess.project_points(means, scales, quats, opac, *args)
    out = cr.project_points(means.to(gpu), scales.to(gpu), quats.to(gpu), opac.to(gpu),
                            args[0].to(gpu), args[1].to(gpu), *args[2:])
    names = ["points_image", "depths", "cov_image", "cov_inv_image", "radii", "mask"]
    for nm, a, b in zip(names, out, ref):
        assert helpers.same(a, b), nm
    keep = ref[5]
    assert 0 < int(keep.sum()) < means.shape[0]  # culls exercised, something visible


def test_project_points_edge_cases(gpu):
    K = helpers.intrinsic(100.0, 64, 64).to(gpu)
    w2c = torch.eye(4, device=gpu)
    out = cr.project_points(torch.zeros(0, 3, device=gpu), torch.zeros(0, 3, device=gpu),
                            torch.zeros(0, 4, device=gpu), torch.zeros(0, device=gpu), w2c, K,
                            NEAR, FAR, MIN_O, MIN_R, MAX_R, 64, 64)
    assert all(t.shape[0] == 0 for t in out)
    # one Gaussian per cull rule, plus NaN input
    means = torch.tensor([[0.0, 0.0, 2.0], [0.0, 0.0, 0.005], [0.0, 0.0, 200.0], [5.0, 0.0, 2.0],
                          [0.0, 0.0, 2.0], [0.0, 0.0, 2.0], [float("nan"), 0.0, 2.0]])
    scales = torch.tensor([[0.02] * 3] * 5 + [[5.0] * 3] + [[0.02] * 3])
    opac = torch.tensor([0.5, 0.5, 0.5, 0.5, 0.001, 0.5, 0.5])
    quats = torch.tensor([[0.0, 0.0, 0.0, 1.0]] * 7)
    ref = preprocess.project_points(means, scales, quats, opac, w2c.cpu(), K.cpu(), NEAR, FAR,
                                    MIN_O, MIN_R, MAX_R, 64, 64)
    out = cr.project_points(means.to(gpu), scales.to(gpu), quats.to(gpu), opac.to(gpu), w2c, K,
                            NEAR, FAR, MIN_O, MIN_R, MAX_R, 64, 64)
    assert out[5].cpu().tolist() == [True, False, False, False, False, False, False]
    for a, b in zip(out, ref):
        assert helpers.same(a, b)


@pytest.mark.parametrize("name", list(SCENES))
def test_project_points_backward(gpu, name):
    means, scales, quats, opac, cam = _api_inputs(name)
    n = means.shape[0]
    g = torch.Generator().manual_seed(7)
    up_pts = torch.randn(n, 2, generator=g)
    up_conic = torch.randn(n, 3, generator=g) * 0.1
    leaves = [t.clone().requires_grad_(True) for t in (means, scales, quats)]
    p = preprocess.project(*leaves, opac, cam["w2c"], cam["K"], cam["width"], cam["height"], NEAR,
                           FAR, MIN_O, MIN_R, MAX_R)
    keep = p["keep"].float()
    loss = ((p["u"] * up_pts[:, 0] + p["v"] * up_pts[:, 1]) * keep).sum() + (
        (p["A"] * up_conic[:, 0] + p["B"] * up_conic[:, 1] + p["C"] * up_conic[:, 2]) * keep).sum()
    loss.backward()
    ref = [t.grad for t in leaves]

    d = lambda t: t.to(gpu)  # noqa: E731
    fwd = cr.project_points(d(means), d(scales), d(quats), d(opac), d(cam["w2c"]), d(cam["K"]),
                            NEAR, FAR, MIN_O, MIN_R, MAX_R, cam["width"], cam["height"])
    got = cr.project_points_backward(d(up_pts), d(up_conic), d(means), d(scales), d(quats),
                                     d(opac), d(cam["w2c"]), d(cam["K"]), cam["width"],
                                     cam["height"], fwd[2], fwd[5])
    for nm, a, b in zip(["means", "scales", "quats"], got, ref):
        assert helpers.rel_l2(a, b) <= 1e-4, nm
        assert float(a[~p["keep"].to(gpu)].abs().max()) == 0.0


@pytest.mark.parametrize("sh_sigmoid", [False, True])
def test_sh_forward_backward(gpu, sh_sigmoid):
    g = torch.Generator().manual_seed(11)
    n = 5000
    cam_pos = torch.tensor([0.1, -0.2, 0.3])
    means = torch.randn(n, 3, generator=g)
    dc = torch.randn(n, 3, generator=g)
    rest = torch.randn(n, 15, 3, generator=g)
    mask = torch.rand(n, generator=g) > 0.1
    up = torch.randn(n, 3, generator=g)

    leaves = [t.clone().requires_grad_(True) for t in (means, dc, rest)]
    ref_col = preprocess.evaluate_sh_api(cam_pos, leaves[0], leaves[1], leaves[2], mask, sh_sigmoid)
    (ref_col * up).sum().backward()

    d = lambda t: t.to(gpu)  # noqa: E731
    col = cr.evaluate_spherical_harmonics(d(cam_pos), d(means), d(dc), d(rest), d(mask), sh_sigmoid)
    assert helpers.max_abs(col, ref_col) <= 2e-5
    assert float(col[~d(mask)].abs().max()) == 0.0
    got = cr.evaluate_spherical_harmonics_backward(d(up), d(cam_pos), d(means), d(dc), d(rest), col,
                                                   d(mask), sh_sigmoid)
    for nm, a, b in zip(["means", "dc", "rest"], got, [t.grad for t in leaves]):
        assert helpers.rel_l2(a, b) <= 1e-4, nm


def test_sh_cache_rows_and_pass_bits(gpu):
    """The colour-gradient cache the render colour kernel writes: rows 0..2 are
    d raw_c / d mean (through the view direction), checked against float64
    autograd of the oracle's SH evaluation; the pass bits are those of the clamp
    max(raw + 0.5, 0) (set where raw + 0.5 >= 0), checked against the oracle's
    raw colours away from the boundary and against the kernel's own colours."""
    g = torch.Generator().manual_seed(41)
    n = 4000
    w2c = torch.eye(4)
    w2c[:3, 3] = torch.tensor([0.2, -0.1, 3.0])
    means = torch.randn(n, 3, generator=g)
    dc = torch.randn(n, 3, generator=g)
    rest = torch.randn(n, 15, 3, generator=g) * 0.3
    mask = torch.rand(n, generator=g) > 0.1
    d = lambda t: t.to(gpu)  # noqa: E731
    cache = cr.sh_cache_empty(n, gpu)
    col = cr.evaluate_spherical_harmonics_render(d(w2c), d(means), d(dc), d(rest), d(mask),
                                                 sh_cache=cache)
    cache = cache.cpu()
    m = cache[:, :9].reshape(n, 3, 3)[mask].double()
    bits = cache[:, 9].view(torch.int32)[mask]

    cam = preprocess.camera_position(w2c.double())
    mu = means[mask].double().requires_grad_(True)
    raw = preprocess.sh_raw(dc[mask].double(), rest[mask].double(),
                            preprocess.view_directions(mu, cam))
    jac = torch.stack([torch.autograd.grad(raw[:, c].sum(), mu, retain_graph=True)[0]
                       for c in range(3)], dim=1)  # (kept, 3 channels, 3 coords)
    err = (m - jac).norm(dim=2) / jac.norm(dim=2).clamp_min(1e-6)
    assert float(err.max()) <= 1e-4
    raw = raw.detach()
    want = ((raw + 0.5 >= 0).int() * torch.tensor([1, 2, 4])).sum(dim=1).int()
    clear = ((raw + 0.5).abs() > 1e-4).all(dim=1)
    assert int(clear.sum()) > 0.9 * int(mask.sum())
    assert torch.equal(bits[clear], want[clear])
    assert int((bits & ~7).abs().sum()) == 0
    # a positive colour always passes its gradient
    pos = col.cpu()[mask] > 0
    for c in range(3):
        assert bool(((bits[pos[:, c]] >> c) & 1).all())


def test_project_points_bitexact_headline(gpu):
    """BASELINE config 3 at full size (1M Gaussians, 1920x1080, near 0.2): every
    projection output bit-identical to the oracle."""
    import bench

    scene = bench.config3()
    p, cam = scene["params"], scene["camera"]
    scales, quats, opac = helpers.activated(p)
    args = (cam["w2c"], cam["K"], cam["near"], FAR, MIN_O, MIN_R, MAX_R, cam["width"], cam["height"])
    with torch.no_grad():
        ref = preprocess.project_points(p["means"], scales, quats, opac, *args)
    out = cr.project_points(p["means"].to(gpu), scales.to(gpu), quats.to(gpu), opac.to(gpu),
                            args[0].to(gpu), args[1].to(gpu), *args[2:])
    for nm, a, b in zip(["points_image", "depths", "cov_image", "cov_inv_image", "radii", "mask"],
                        out, ref):
        assert helpers.same(a, b), nm
    assert int(ref[5].sum()) > 500_000
