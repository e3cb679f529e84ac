"""Shared test helpers: seeded scenes, parity metrics, golden-file access."""

from __future__ import annotations

import json
import math
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden")
PARAMS = ["means", "log_scales", "quats_raw", "opacity_logits", "sh_dc", "sh_rest"]


def rel_l2(a: torch.Tensor, b: torch.Tensor) -> float:
    """||a - b|| / ||b|| (scripts/check_cuda_gradients.py:37-44)."""
    a = a.detach().double().flatten().cpu()
    b = b.detach().double().flatten().cpu()
    return float((a - b).norm() / max(float(b.norm()), 1e-30))


def cosine(a: torch.Tensor, b: torch.Tensor) -> float:
    a = a.detach().double().flatten().cpu()
    b = b.detach().double().flatten().cpu()
    return float(a.dot(b) / max(float(a.norm() * b.norm()), 1e-30))


def same(a: torch.Tensor, b: torch.Tensor) -> bool:
    """Bit-for-bit equal values, treating NaN == NaN (payloads aside)."""
    a = a.detach().cpu()
    b = b.detach().cpu()
    if a.shape != b.shape or a.dtype != b.dtype:
        return False
    if a.is_floating_point():
        na, nb = torch.isnan(a), torch.isnan(b)
        return bool(torch.equal(na, nb) and torch.equal(a[~na], b[~nb]))
    return bool(torch.equal(a, b))


def max_abs(a: torch.Tensor, b: torch.Tensor) -> float:
    return float((a.detach().double().cpu() - b.detach().double().cpu()).abs().max()) if a.numel() else 0.0


def look_at(azimuth: float, elevation: float, dist: float) -> torch.Tensor:
    """OpenCV world->camera matrix of a camera on a sphere looking at the origin:
    forward f = -c/|c|, right = normalize(f x up) with up = (0,-1,0), down = f x right."""
    c = torch.tensor([dist * math.cos(elevation) * math.cos(azimuth), dist * math.sin(elevation),
                      dist * math.cos(elevation) * math.sin(azimuth)], dtype=torch.float64)
    f = -c / c.norm()
    up = torch.tensor([0.0, -1.0, 0.0], dtype=torch.float64)
    right = torch.linalg.cross(f, up)
    right = right / right.norm()
    down = torch.linalg.cross(f, right)
    R = torch.stack([right, down, f])
    M = torch.eye(4, dtype=torch.float64)
    M[:3, :3] = R
    M[:3, 3] = -R @ c
    return M.float()


def intrinsic(f: float, width: int, height: int) -> torch.Tensor:
    return torch.tensor([[f, 0.0, width / 2], [0.0, f, height / 2], [0.0, 0.0, 1.0]])


def scene_box(n, width, height, f, seed, log_scale=(-4.0, 0.5), sh_degree=0, z=(2.0, 6.0)):
    """Config-1 style scene: camera-space means in [-1,1]^2 x [z0,z1], W2C = I."""
    g = torch.Generator().manual_seed(seed)
    means = torch.empty(n, 3)
    means[:, :2] = torch.rand(n, 2, generator=g) * 2 - 1
    means[:, 2] = torch.rand(n, generator=g) * (z[1] - z[0]) + z[0]
    p = dict(
        means=means,
        log_scales=torch.randn(n, 3, generator=g) * log_scale[1] + log_scale[0],
        quats_raw=torch.randn(n, 4, generator=g),
        opacity_logits=torch.randn(n, generator=g),
        sh_dc=torch.randn(n, 3, generator=g) * 0.3,
        sh_rest=(torch.randn(n, 15, 3, generator=g) * 0.05 if sh_degree else torch.zeros(n, 15, 3)),
    )
    cam = dict(w2c=torch.eye(4), K=intrinsic(f, width, height), width=width, height=height)
    target = torch.rand(height, width, 3, generator=g)
    return p, cam, target


def scene_orbit(n, width, height, f, seed, azimuth=0.7, elevation=0.3, dist=4.0, radius=1.5,
                log_scale=(-4.5, 0.6), opacity_std=1.5):
    """Config-2 style scene: means in a ball of radius 1.5, SH degree 3, camera on an orbit."""
    g = torch.Generator().manual_seed(seed)
    d = torch.randn(n, 3, generator=g)
    d = d / d.norm(dim=1, keepdim=True)
    means = d * radius * torch.rand(n, 1, generator=g) ** (1 / 3)
    p = dict(
        means=means,
        log_scales=torch.randn(n, 3, generator=g) * log_scale[1] + log_scale[0],
        quats_raw=torch.randn(n, 4, generator=g),
        opacity_logits=torch.randn(n, generator=g) * opacity_std,
        sh_dc=torch.randn(n, 3, generator=g) * 0.3,
        sh_rest=torch.randn(n, 15, 3, generator=g) * 0.05,
    )
    cam = dict(w2c=look_at(azimuth, elevation, dist), K=intrinsic(f, width, height), width=width,
               height=height)
    target = torch.rand(height, width, 3, generator=g)
    return p, cam, target


def activated(p: dict):
    """Activations of scripts/train.py:135-143."""
    scales = torch.exp(p["log_scales"])
    q = p["quats_raw"]
    quats = q / torch.norm(q, dim=1, keepdim=True).clamp_min(1e-12)
    opac = torch.sigmoid(p["opacity_logits"])
    return scales, quats, opac


def load_golden() -> dict:
    data = np.load(os.path.join(GOLDEN, "torch_render_golden.npz"), allow_pickle=False)
    cases: dict = {}
    for key in data.files:
        name, field = key.split("/", 1)
        cases.setdefault(name, {})[field] = data[key]
    return cases


def golden_case_tensors(case: dict):
    p = {k: torch.from_numpy(case[k].copy()) for k in PARAMS}
    cam = dict(w2c=torch.from_numpy(case["w2c"].copy()), K=torch.from_numpy(case["K"].copy()),
               width=int(case["width"]), height=int(case["height"]))
    return p, cam, torch.from_numpy(case["target"].copy())


def golden_loss(image: torch.Tensor, target: torch.Tensor, kind: str) -> torch.Tensor:
    if kind == "l1_const64":
        return torch.nn.functional.l1_loss(image, target)
    return torch.nn.functional.l1_loss(image / 255.0, target)


def forward_backward(render_fn, p: dict, cam: dict, target: torch.Tensor, device, loss_kind="l1_target",
                     sh_sigmoid=False, **kw):
    """Render with raw parameters on `device`, L1 loss, backward.  Returns
    (image, loss, {param: grad}, points_img, radii)."""
    leaves = {k: v.to(device).clone().requires_grad_(True) for k, v in p.items()}
    scales, quats, opac = activated(leaves)
    image, points_img, radii = render_fn(cam["w2c"].to(device), cam["K"].to(device), cam["width"],
                                         cam["height"], leaves["means"], scales, quats, opac,
                                         leaves["sh_dc"], leaves["sh_rest"], sh_sigmoid=sh_sigmoid,
                                         **kw)
    if points_img is not None:
        points_img.retain_grad()
    loss = golden_loss(image, target.to(device), loss_kind)
    loss.backward()
    grads = {k: v.grad for k, v in leaves.items()}
    return image.detach(), loss.detach(), grads, points_img, radii


def load_layout_fixtures() -> dict:
    with open(os.path.join(GOLDEN, "layout_fixtures.json")) as fh:
        return json.load(fh)


def fixture_tensors(name: str):
    """Inputs of the reference's constant fixtures as float32 tensors
    (scripts/check_cuda_gradients.py:435-502 and :631-668)."""
    fx = load_layout_fixtures()[name]
    W, H = fx["width"], fx["height"]
    if name == "multitile":
        pts = torch.tensor(fx["points_image"], dtype=torch.float32)
        radii = torch.tensor(fx["radii"], dtype=torch.float32)
        depths = torch.tensor(fx["depths"], dtype=torch.float32)
        conic = torch.tensor(fx["cov_inv_image"], dtype=torch.float32)
        opac = torch.tensor(fx["opacities"], dtype=torch.float32)
        colors = torch.tensor(fx["colors"], dtype=torch.float32)
    else:
        gu = torch.tensor(fx["grid_u"], dtype=torch.float32)
        gv = torch.tensor(fx["grid_v"], dtype=torch.float32)
        pts = torch.cartesian_prod(gu, gv)
        n = pts.shape[0]
        radii = torch.full((n, 2), fx["radius"], dtype=torch.float32)
        depths = torch.linspace(*fx["depth_linspace"], n, dtype=torch.float32)
        conic = torch.stack([torch.linspace(*r, n) for r in fx["cov_inv_linspace"]], dim=1)
        opac = torch.linspace(*fx["opacity_linspace"], n)
        colors = torch.stack([torch.linspace(*r, n) for r in fx["color_linspace"]], dim=-1)
    xs = torch.linspace(-1.0, 1.0, W)
    ys = torch.linspace(-1.0, 1.0, H)
    gy, gx = torch.meshgrid(ys, xs, indexing="ij")
    upstream = torch.stack([cx * gx + cy * gy for cx, cy in fx["upstream_xy_coeffs"]], dim=-1)
    mask = torch.ones(pts.shape[0], dtype=torch.bool)
    return dict(points_image=pts, radii=radii, depths=depths, cov_inv_image=conic,
                opacities=opac, colors=colors, mask=mask, upstream=upstream, width=W, height=H,
                tile_size=fx["tile_size"], alpha_threshold=fx["alpha_threshold"],
                transmittance_threshold=fx["transmittance_threshold"],
                chi_squared_threshold=fx["chi_squared_threshold"],
                expected_indexing_offset=fx["expected_indexing_offset"],
                expected_gaussian_ids_sorted=fx["expected_gaussian_ids_sorted"])
