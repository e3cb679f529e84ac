"""Writes tests/golden/torch_render_golden.npz from the reference's Torch rasterizer.

Runs ONLY in the build container, where the reference checkout is readable
(default /root/reference, override with GS_REFERENCE_DIR).  It imports
src/torch_rasterizer.py::render (with src/gaussian.py) on the CPU, renders a
few small seeded scenes, back-propagates an L1 loss through the reference's
own autograd graph, and stores inputs and outputs as float32 arrays.  Nothing
of the reference is stored: only the numbers it produced.

Cases (key prefix -> scene):
  box_sh0      1000 Gaussians in [-1,1]^2 x [2,6] camera space, SH degree 0,
               64x64, fx=fy=75 (config-1 distributions at a smaller size)
  orbit_sh3    1000 Gaussians in a ball of radius 1.5 seen from distance 4 at
               azimuth 0.7 / elevation 0.3, SH degree 3, 100x70 (partial tiles)
  sigmoid      500 Gaussians, SH degree 3, sh_sigmoid=True, 48x48
  e2e_large    384 Gaussians with scale ~exp(N(0,0.1)) (splats tens of pixels
               wide), 64x64, fx=60, L1 against a constant 64 image -- the
               distributions of scripts/check_cuda_gradients.py:823-912
Loss for the first three: l1(image/255, target), target ~ U[0,1].
Stored per case: w2c, K, width, height, sh_sigmoid, raw parameters (means,
log_scales, quats_raw, opacity_logits, sh_dc, sh_rest), target, image, loss,
and d loss / d raw parameter for each of the six.
"""

from __future__ import annotations

import math
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "torch_render_golden.npz")


def look_at(azimuth: float, elevation: float, dist: float) -> torch.Tensor:
    """OpenCV world->camera matrix of a camera on a sphere looking at the origin."""
    c = torch.tensor([dist * math.cos(elevation) * math.cos(azimuth),
                      dist * math.sin(elevation),
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


def make_cases():
    cases = {}
    g = torch.Generator().manual_seed(1234)

    n, W, H = 1000, 64, 64
    means = torch.empty(n, 3)
    means[:, :2] = torch.rand(n, 2, generator=g) * 2 - 1
    means[:, 2] = torch.rand(n, generator=g) * 4 + 2
    cases["box_sh0"] = dict(
        w2c=torch.eye(4), K=torch.tensor([[75.0, 0, W / 2], [0, 75.0, H / 2], [0, 0, 1]]),
        width=W, height=H, sh_sigmoid=False, means=means,
        log_scales=torch.randn(n, 3, generator=g) * 0.5 - 3.0,
        quats_raw=torch.randn(n, 4, generator=g),
        opacity_logits=torch.randn(n, generator=g),
        sh_dc=torch.randn(n, 3, generator=g) * 0.3,
        sh_rest=torch.zeros(n, 15, 3),
        target=torch.rand(H, W, 3, generator=g), loss="l1_target")

    n, W, H = 1000, 100, 70
    d = torch.randn(n, 3, generator=g)
    d = d / d.norm(dim=1, keepdim=True)
    means = d * 1.5 * torch.rand(n, 1, generator=g) ** (1 / 3)
    cases["orbit_sh3"] = dict(
        w2c=look_at(0.7, 0.3, 4.0), K=torch.tensor([[110.0, 0, W / 2], [0, 110.0, H / 2], [0, 0, 1]]),
        width=W, height=H, sh_sigmoid=False, means=means,
        log_scales=torch.randn(n, 3, generator=g) * 0.6 - 3.5,
        quats_raw=torch.randn(n, 4, generator=g),
        opacity_logits=torch.randn(n, generator=g) * 1.5,
        sh_dc=torch.randn(n, 3, generator=g) * 0.3,
        sh_rest=torch.randn(n, 15, 3, generator=g) * 0.05,
        target=torch.rand(H, W, 3, generator=g), loss="l1_target")

    n, W, H = 500, 48, 48
    means = torch.empty(n, 3)
    means[:, :2] = torch.rand(n, 2, generator=g) * 1.6 - 0.8
    means[:, 2] = torch.rand(n, generator=g) * 2 + 2
    cases["sigmoid"] = dict(
        w2c=torch.eye(4), K=torch.tensor([[60.0, 0, 24.0], [0, 60.0, 24.0], [0, 0, 1]]),
        width=W, height=H, sh_sigmoid=True, means=means,
        log_scales=torch.randn(n, 3, generator=g) * 0.4 - 3.0,
        quats_raw=torch.randn(n, 4, generator=g),
        opacity_logits=torch.randn(n, generator=g),
        sh_dc=torch.randn(n, 3, generator=g) * 0.5,
        sh_rest=torch.randn(n, 15, 3, generator=g) * 0.1,
        target=torch.rand(H, W, 3, generator=g), loss="l1_target")

    n, W, H = 384, 64, 64
    means = (torch.rand(n, 3, generator=g) - 0.5) * 2.0
    means[:, 2] = torch.rand(n, generator=g) * 2.0 + 1.5
    cases["e2e_large"] = dict(
        w2c=torch.eye(4), K=torch.tensor([[60.0, 0, 32.0], [0, 60.0, 32.0], [0, 0, 1]]),
        width=W, height=H, sh_sigmoid=False, means=means,
        log_scales=torch.randn(n, 3, generator=g) * 0.1,
        quats_raw=torch.randn(n, 4, generator=g),
        opacity_logits=torch.randn(n, generator=g) * 0.5,
        sh_dc=torch.randn(n, 3, generator=g) * 0.2,
        sh_rest=torch.randn(n, 15, 3, generator=g) * 0.05,
        target=torch.full((H, W, 3), 64.0), loss="l1_const64")
    return cases


PARAMS = ["means", "log_scales", "quats_raw", "opacity_logits", "sh_dc", "sh_rest"]


def run_render(render_fn, case, **kw):
    """Forward + backward of the case through `render_fn` (reference signature)."""
    p = {k: case[k].clone().requires_grad_(True) for k in PARAMS}
    scales = torch.exp(p["log_scales"])
    quats = p["quats_raw"] / torch.norm(p["quats_raw"], dim=1, keepdim=True)
    opac = torch.sigmoid(p["opacity_logits"])
    image, _, _ = render_fn(case["w2c"], case["K"], case["width"], case["height"], p["means"],
                            scales, quats, opac, p["sh_dc"], p["sh_rest"],
                            sh_sigmoid=case["sh_sigmoid"], **kw)
    if case["loss"] == "l1_const64":
        loss = torch.nn.functional.l1_loss(image, case["target"].to(image.device))
    else:
        loss = torch.nn.functional.l1_loss(image / 255.0, case["target"].to(image.device))
    loss.backward()
    return image.detach(), loss.detach(), {k: p[k].grad for k in PARAMS}


def main():
    ref = os.environ.get("GS_REFERENCE_DIR", "/root/reference")
    if not os.path.isdir(os.path.join(ref, "src")):
        sys.exit(f"reference checkout not found at {ref}; golden vectors are made in the build container")
    sys.path.insert(0, ref)
    from src.torch_rasterizer import render as reference_render  # noqa: E402

    out = {}
    for name, case in make_cases().items():
        image, loss, grads = run_render(reference_render, case, device="cpu")
        for k in ["w2c", "K", "means", "log_scales", "quats_raw", "opacity_logits", "sh_dc",
                  "sh_rest", "target"]:
            out[f"{name}/{k}"] = case[k].numpy().astype(np.float32)
        out[f"{name}/width"] = np.int64(case["width"])
        out[f"{name}/height"] = np.int64(case["height"])
        out[f"{name}/sh_sigmoid"] = np.bool_(case["sh_sigmoid"])
        out[f"{name}/loss_kind"] = np.array(case["loss"])
        out[f"{name}/image"] = image.numpy().astype(np.float32)
        out[f"{name}/loss"] = np.float32(loss.item())
        for k, v in grads.items():
            out[f"{name}/grad_{k}"] = v.numpy().astype(np.float32)
        print(f"{name}: loss={loss.item():.6f}")
    np.savez_compressed(OUT, **out)
    print("wrote", OUT, os.path.getsize(OUT), "bytes")


if __name__ == "__main__":
    main()
