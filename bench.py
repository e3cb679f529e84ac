"""Benchmark of the MI355X Gaussian-splatting rasterizer (BASELINE.json metric).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 3] [--no-cpu-baseline]

One step = activations of the raw parameters, render forward, L1 loss of the
/255 image against a target, and backward through all six parameter groups
(no optimizer step: the metric is "fwd+bwd"), on the headline configuration 3
(1M Gaussians, SH degree 3, 1920x1080, fp32) with synthetic inputs already
resident in HBM.  The timed path is the library's fused step
(cuda_rasterizer.fused.render_l1); the same step written as the reference's
training loop does it (PyTorch activations and l1_loss around the drop-in
render()) is timed beside it ("drop_in").  The configuration-5 training
stress run (2000 steps of render + L1 + backward + Adam with clone / prune
every 100 steps, through the library and through the reference's loop) is
reported in the same line as "train_stress", and the SSIM loss term of the
reference's training loss (fused_ssim at 1920x1080, forward and backward) as
"ssim".  Prints ONE JSON line.

Scene generators for BASELINE configurations 1-5 live here too (tests import
them).  Every tensor is drawn on the CPU with torch.Generator().manual_seed(seed)
in a fixed order -- means, log-scales, quaternions, opacity logits, SH dc, SH
rest, cameras, target -- then copied to the device.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "3dgs_from_scratch_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import torch  # noqa: E402

HBM_PEAK_GBS = 8000.0
# untimed work before each timed region's warm-up: the GPU lowers its clocks
# while idle, and the steps right after an idle pause run up to 10% slower
SETTLE_S = 0.2
FP32_PEAK_TFLOPS = 157.3

METRIC = "fwd+bwd ms/iter at 1M Gaussians 1080p SH3; achieved HBM GB/s vs peak"


# ------------------------------------------------------------------ scenes

def _intrinsic(f, width, height):
    return torch.tensor([[f, 0.0, width / 2], [0.0, f, height / 2], [0.0, 0.0, 1.0]])


def look_at(azimuth: float, elevation: float, dist: float) -> torch.Tensor:
    """OpenCV world->camera matrix for a camera on a sphere looking at the origin."""
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


def _sh(g, n, degree):
    dc = torch.randn(n, 3, generator=g) * 0.3
    rest = torch.randn(n, 15, 3, generator=g) * 0.05 if degree else torch.zeros(n, 15, 3)
    return dc, rest


def config1(seed: int = 0) -> dict:
    """10k Gaussians, SH0, 256x256, fx=fy=300, means U([-1,1]^2 x [2,6]) in camera space."""
    g = torch.Generator().manual_seed(seed)
    n, W, H = 10_000, 256, 256
    means = torch.empty(n, 3)
    means[:, :2] = torch.rand(n, 2, generator=g) * 2 - 1
    means[:, 2] = torch.rand(n, generator=g) * 4 + 2
    log_scales = torch.randn(n, 3, generator=g) * 0.5 - 4.0
    quats = torch.randn(n, 4, generator=g)
    logits = torch.randn(n, generator=g)
    dc, rest = _sh(g, n, 0)
    cam = dict(w2c=torch.eye(4), K=_intrinsic(300.0, W, H), width=W, height=H, near=0.01)
    target = torch.rand(H, W, 3, generator=g)
    return dict(params=dict(means=means, log_scales=log_scales, quats_raw=quats,
                            opacity_logits=logits, sh_dc=dc, sh_rest=rest),
                camera=cam, target=target, name="config1")


def config2(seed: int = 0, n: int = 100_000, cameras: int = 8) -> dict:
    """100k Gaussians in a ball of radius 1.5, SH3, 800x800, fx=fy=1100, 8 orbit cameras
    at distance 4 (azimuth U[0,2pi), elevation U[-pi/3,pi/3])."""
    g = torch.Generator().manual_seed(seed)
    W = H = 800
    d = torch.randn(n, 3, generator=g)
    d = d / d.norm(dim=1, keepdim=True)
    means = d * 1.5 * torch.rand(n, 1, generator=g) ** (1 / 3)
    log_scales = torch.randn(n, 3, generator=g) * 0.6 - 4.5
    quats = torch.randn(n, 4, generator=g)
    logits = torch.randn(n, generator=g) * 1.5
    dc, rest = _sh(g, n, 3)
    az = torch.rand(cameras, generator=g) * 2 * math.pi
    el = (torch.rand(cameras, generator=g) * 2 - 1) * math.pi / 3
    cams = [dict(w2c=look_at(float(a), float(e), 4.0), K=_intrinsic(1100.0, W, H), width=W,
                 height=H, near=0.01) for a, e in zip(az, el)]
    targets = [torch.rand(H, W, 3, generator=g) for _ in range(cameras)]
    return dict(params=dict(means=means, log_scales=log_scales, quats_raw=quats,
                            opacity_logits=logits, sh_dc=dc, sh_rest=rest),
                cameras=cams, targets=targets, camera=cams[0], target=targets[0], name="config2")


def config3(n: int = 1_000_000, seed: int = 0, big_fraction: float = 0.0) -> dict:
    """Headline: 1M Gaussians, SH3, 1920x1080, fx=fy=1400, camera at the origin looking +z,
    near 0.2.  70% clustered (sigma 0.3) around 50 centres inside the frustum
    (z~U[2,10], x~U[-0.6,0.6]z, y~U[-0.35,0.35]z), 30% uniform in [-10,10]^3.
    log-scale ~ N(-3.5, 0.8) (a `big_fraction` of them ~ N(-1, 0.3): config 4),
    opacity logit ~ N(0, 1.5)."""
    g = torch.Generator().manual_seed(seed)
    W, H = 1920, 1080
    n_cl = int(round(0.7 * n))
    cz = torch.rand(50, generator=g) * 8 + 2
    cx = (torch.rand(50, generator=g) * 1.2 - 0.6) * cz
    cy = (torch.rand(50, generator=g) * 0.7 - 0.35) * cz
    centres = torch.stack([cx, cy, cz], dim=1)
    which = torch.randint(0, 50, (n_cl,), generator=g)
    clustered = centres[which] + torch.randn(n_cl, 3, generator=g) * 0.3
    uniform = torch.rand(n - n_cl, 3, generator=g) * 20 - 10
    means = torch.cat([clustered, uniform], dim=0)
    log_scales = torch.randn(n, 3, generator=g) * 0.8 - 3.5
    if big_fraction > 0:
        big = torch.rand(n, generator=g) < big_fraction
        log_scales[big] = torch.randn(int(big.sum()), 3, generator=g) * 0.3 - 1.0
    quats = torch.randn(n, 4, generator=g)
    logits = torch.randn(n, generator=g) * 1.5
    dc, rest = _sh(g, n, 3)
    cam = dict(w2c=torch.eye(4), K=_intrinsic(1400.0, W, H), width=W, height=H, near=0.2)
    target = torch.rand(H, W, 3, generator=g)
    return dict(params=dict(means=means, log_scales=log_scales, quats_raw=quats,
                            opacity_logits=logits, sh_dc=dc, sh_rest=rest),
                camera=cam, target=target, name="config3" if big_fraction == 0 else "config4")


def config4(seed: int = 0) -> dict:
    """3M Gaussians, configuration-3 distributions with 5% log-scales ~ N(-1, 0.3)."""
    return config3(n=3_000_000, seed=seed, big_fraction=0.05)


def config5(seed: int = 0, n: int = 100_000 * 2, steps: int = 2000, n_targets: int = 16) -> dict:
    """Training-loop stress run: 200k Gaussians with configuration-2 distributions,
    1280x720 with fx=fy=1000, one orbit camera per step (distance 4, azimuth
    U[0,2pi), elevation U[-pi/3,pi/3]) and a bank of 16 fixed random targets
    used round-robin (step % 16)."""
    g = torch.Generator().manual_seed(seed)
    W, H = 1280, 720
    d = torch.randn(n, 3, generator=g)
    d = d / d.norm(dim=1, keepdim=True)
    means = d * 1.5 * torch.rand(n, 1, generator=g) ** (1 / 3)
    log_scales = torch.randn(n, 3, generator=g) * 0.6 - 4.5
    quats = torch.randn(n, 4, generator=g)
    logits = torch.randn(n, generator=g) * 1.5
    dc, rest = _sh(g, n, 3)
    az = torch.rand(steps, generator=g) * 2 * math.pi
    el = (torch.rand(steps, generator=g) * 2 - 1) * math.pi / 3
    w2c = torch.stack([look_at(float(a), float(e), 4.0) for a, e in zip(az, el)])
    targets = torch.rand(n_targets, H, W, 3, generator=g)
    cam = dict(w2c=w2c[0], K=_intrinsic(1000.0, W, H), width=W, height=H, near=0.01)
    return dict(params=dict(means=means, log_scales=log_scales, quats_raw=quats,
                            opacity_logits=logits, sh_dc=dc, sh_rest=rest),
                w2c_per_step=w2c, targets=targets, camera=cam, target=targets[0], name="config5")


CONFIGS = {1: config1, 2: config2, 3: config3, 4: config4, 5: config5}


# --------------------------------------------------------------- GPU leg

def activated(p: dict):
    """scripts/train.py:135-143."""
    scales = torch.exp(p["log_scales"])
    q = p["quats_raw"]
    quats = q / torch.norm(q, dim=1, keepdim=True).clamp_min(1e-12)
    opac = torch.sigmoid(p["opacity_logits"])
    return scales, quats, opac


def gpu_step(render, leaves: dict, cam: dict, target: torch.Tensor):
    """render + L1 loss + backward; returns (loss, image, points_img)."""
    for t in leaves.values():
        t.grad = None
    scales, quats, opac = activated(leaves)
    image, points_img, radii = render(cam["w2c"], cam["K"], cam["width"], cam["height"],
                                      leaves["means"], scales, quats, opac, leaves["sh_dc"],
                                      leaves["sh_rest"], near_plane=cam["near"])
    loss = torch.nn.functional.l1_loss(image / 255.0, target)
    loss.backward()
    return loss, image


def fused_step(leaves: dict, cam: dict, target: torch.Tensor, ssim_lambda: float = 0.0,
               schedule_cache: dict | None = None):
    """The same step through cuda_rasterizer.fused.render_l1 (activations, render and
    L1 loss -- plus the SSIM term with ssim_lambda > 0 -- as one autograd node of
    library kernels).  With `schedule_cache`, the step passes it with the scene's
    one view id (a training loop revisiting the view)."""
    from cuda_rasterizer.fused import render_l1

    for t in leaves.values():
        t.grad = None
    loss, image, _, _ = render_l1(cam["w2c"], cam["K"], cam["width"], cam["height"],
                                  leaves["means"], leaves["log_scales"], leaves["quats_raw"],
                                  leaves["opacity_logits"], leaves["sh_dc"], leaves["sh_rest"],
                                  target, near_plane=cam["near"], ssim_lambda=ssim_lambda,
                                  schedule_cache=schedule_cache,
                                  view_id=None if schedule_cache is None else "view0")
    loss.backward()
    return loss, image


def device_time(step, steps: int):
    """Kernel time per step in ms over `steps` calls of `step`, summed over every
    stream (the fused step's colours run beside binning on a second stream), from
    torch.profiler's device activity; None when the profiler reports none."""
    try:
        from torch.profiler import ProfilerActivity, profile

        torch.cuda.synchronize()
        with profile(activities=[ProfilerActivity.CUDA]) as prof:
            for _ in range(steps):
                step()
            torch.cuda.synchronize()
        total_us = sum(e.self_device_time_total for e in prof.key_averages())
    except Exception:  # noqa: BLE001 -- the profiler is optional here
        return None
    return total_us / steps / 1e3 if total_us > 0 else None


def busy(device_ms, wall_ms: float):
    """{"device_ms", "busy"}: kernel time per step and its share of the wall time
    per step (above 1 where streams overlap); None without a device time."""
    if device_ms is None:
        return None
    return {"device_ms": round(device_ms, 4), "busy": round(device_ms / wall_ms, 3)}


def settle(step, seconds: float = SETTLE_S, wait_each: bool = False) -> int:
    """Untimed calls of `step` for at least `seconds` of wall time, after which the
    GPU runs at its working clocks; returns the number of calls.  An eager step
    waits on the device within each call (the capped sort's check), so the host
    stays at most a step ahead; a graph replay does not, and is waited for after
    each call (`wait_each`) so that the loop does not queue thousands."""
    n = 0
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end:
        step()
        if wait_each:
            torch.cuda.synchronize()
        n += 1
    torch.cuda.synchronize()
    return n


def run_gpu(scene: dict, steps: int, warmup: int, path: str = "fused",
            schedule_cache: bool = False) -> dict:
    """Runs `warmup` steps, the profiler's kernel time (`steps` steps), untimed
    steps for SETTLE_S seconds (so that the timed region's warm-up follows GPU
    work, not a GPU idling at low clocks), `warmup` steps, times `steps` steps,
    then the per-stage breakdown (`steps` steps).  path: "fused" (fused_step) or "drop-in"
    (gpu_step: PyTorch activations and loss around the drop-in render()).
    schedule_cache: the fused step with a per-view schedule cache (the view
    repeats every step, as a training view does every epoch)."""
    from cuda_rasterizer import _lib
    from cuda_rasterizer.wrapper import render

    dev = torch.device("cuda:0")
    leaves = {k: v.to(dev).requires_grad_(True) for k, v in scene["params"].items()}
    cam = dict(scene["camera"])
    cam["w2c"] = cam["w2c"].to(dev)
    cam["K"] = cam["K"].to(dev)
    target = scene["target"].to(dev)
    cache = {} if schedule_cache else None
    if path == "fused":
        step = lambda: fused_step(leaves, cam, target, schedule_cache=cache)  # noqa: E731
    else:
        step = lambda: gpu_step(render, leaves, cam, target)  # noqa: E731
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()

    # the kernel time per step from the profiler first; then untimed steps for a
    # while, since the GPU's clocks drop while it idles (the profiler's host-side
    # processing, the uploads) and the steps after such a pause run up to 10%
    # slower until they are back up; then the timed region's warm-up
    device_ms = device_time(step, steps)
    settle(step)
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()

    # timed region: wall clock with a synchronize on both sides, plus HIP events
    # around the blend backward (the dominant kernel) on the stream it runs on, on
    # every other step: each event pair adds about 3 us to its step, and the
    # sampled launches' average is the kernel's launch duration
    _lib.timer.reset()
    _lib.timer.only = DOMINANT_STAGES
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        _lib.timer.enabled = i % 2 == 0
        loss, image = step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    _lib.timer.enabled = False
    main_stages = _lib.timer.summary()
    ms = (t1 - t0) * 1e3 / steps

    # per-stage breakdown: the same steps again with events around every entry point
    _lib.timer.reset()
    _lib.timer.only = None
    _lib.timer.enabled = True
    for _ in range(steps):
        step()
    _lib.timer.enabled = False
    stages = _lib.timer.summary()

    # workload statistics of one step
    from cuda_rasterizer import compute_tile_intersection, project_points, rasterize_work
    with torch.no_grad():
        scales, quats, opac = activated(leaves)
        pts, depths, _, conic, radii, mask = project_points(
            leaves["means"], scales, quats, opac, cam["w2c"], cam["K"], cam["near"], 100.0,
            1 / 255, 0.5, 128.0, cam["width"], cam["height"])
        off, ids = compute_tile_intersection(pts, radii, depths, mask, cam["width"], cam["height"], 16)
        visited, composited = rasterize_work(off, ids, pts, conic, opac, cam["width"],
                                             cam["height"], 16, 1e-4, 1e-4, 9.21)
    return dict(ms=ms, stages={k: (c, t / steps) for k, (c, t) in stages.items()},
                main_launch_ms={k: t / c for k, (c, t) in main_stages.items() if c}, steps=steps,
                n=scene["params"]["means"].shape[0], n_visible=int(mask.sum()), keys=int(ids.numel()),
                n_tiles=int(off.numel()), visited=visited, composited=composited,
                loss=float(loss.detach()), width=cam["width"], height=cam["height"],
                device_busy=busy(device_ms, ms))


def run_full_loss(scene: dict, steps: int, warmup: int, ssim_lambda: float = 0.2) -> dict:
    """The fused step with the reference's full training loss,
    (1 - lambda) L1 + lambda (1 - SSIM), lambda = 0.2 (scripts/train.py:185-205 after
    its warm-up): wall clock over `steps` steps, synchronised on both sides."""
    dev = torch.device("cuda:0")
    leaves = {k: v.to(dev).requires_grad_(True) for k, v in scene["params"].items()}
    cam = dict(scene["camera"])
    cam["w2c"] = cam["w2c"].to(dev)
    cam["K"] = cam["K"].to(dev)
    target = scene["target"].to(dev)
    settle(lambda: fused_step(leaves, cam, target, ssim_lambda))  # as in run_gpu
    for _ in range(warmup):
        fused_step(leaves, cam, target, ssim_lambda)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        loss, _ = fused_step(leaves, cam, target, ssim_lambda)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    return {"ssim_lambda": ssim_lambda, "ms_per_step": round(ms, 4),
            "loss": round(float(loss.detach()), 6)}


def run_ssim(scene: dict, steps: int, warmup: int) -> dict:
    """The reference's SSIM loss term (scripts/train.py:193-197) at the scene's
    resolution: fused_ssim(img.permute(2, 0, 1)[None], target.permute(2, 0, 1)[None],
    padding="valid") on (H, W, 3) float32 images resident in HBM.  Warm-up steps
    run forward and backward through autograd; the timed part queues `steps`
    forward calls, then `steps` backward calls, back to back, with HIP events
    around each run (device time per call; the forward includes its mean
    kernel).  Algorithmic HBM bytes: forward reads both images and writes three
    derivative maps (5 images' worth), backward reads the maps and both images
    and writes the gradient (6)."""
    from cuda_rasterizer import fused_ssim
    from cuda_rasterizer.ssim import ssim_backward, ssim_forward

    dev = torch.device("cuda:0")
    W, H = scene["camera"]["width"], scene["camera"]["height"]
    g = torch.Generator().manual_seed(5)
    target = scene["target"].to(dev)
    img = (scene["target"] + 0.1 * torch.randn(scene["target"].shape, generator=g)).clamp(0, 1).to(dev)
    img.requires_grad_(True)
    x1 = img.detach().permute(2, 0, 1).unsqueeze(0)
    x2 = target.permute(2, 0, 1).unsqueeze(0)

    def loss_term():
        img.grad = None
        v = 1.0 - fused_ssim(img.permute(2, 0, 1).unsqueeze(0), x2, padding="valid")
        v.backward()
        return v

    settle(loss_term)
    v = None
    for _ in range(max(warmup, 1)):
        v = loss_term()
    mean, maps = ssim_forward(x1, x2, "valid")
    grad_mean = torch.ones((), device=dev)
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
    ev[0].record()
    for _ in range(steps):
        ssim_forward(x1, x2, "valid")
    ev[1].record()
    for _ in range(steps):
        ssim_backward(grad_mean, x1, x2, maps)
    ev[2].record()
    torch.cuda.synchronize()
    image_bytes = H * W * 3 * 4
    out = {"workload": f"{W}x{H}x3 (H, W, C) permuted to (1, 3, H, W), padding valid",
           "ssim": round(1.0 - float(v.detach()), 6),
           "timing": f"{steps} calls of each entry point back to back, HIP events around each run"}
    for name, mult, (e0, e1) in (("ssim_forward", 5, (ev[0], ev[1])),
                                 ("ssim_backward", 6, (ev[1], ev[2]))):
        ms = e0.elapsed_time(e1) / steps
        gbs = mult * image_bytes / (ms * 1e-3) / 1e9
        out[name] = {"ms": round(ms, 4), "gbs": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
                     "bytes": mult * image_bytes}
    return out


def run_cameras(scene: dict, steps: int, warmup: int) -> dict:
    """Configuration 2: one iteration is the fused step (render_l1) on every one
    of the scene's cameras against its own target, the loss being the mean of
    the per-camera L1 terms, so the parameter gradients accumulate over the
    cameras.  Wall clock over `steps` iterations, synchronised on both sides."""
    from cuda_rasterizer.fused import render_l1

    dev = torch.device("cuda:0")
    leaves = {k: v.to(dev).requires_grad_(True) for k, v in scene["params"].items()}
    cams = [dict(c, w2c=c["w2c"].to(dev), K=c["K"].to(dev)) for c in scene["cameras"]]
    targets = [t.to(dev) for t in scene["targets"]]
    weight = 1.0 / len(cams)

    def step():
        for t in leaves.values():
            t.grad = None
        total = 0.0
        for cam, target in zip(cams, targets):
            loss, _, _, _ = render_l1(cam["w2c"], cam["K"], cam["width"], cam["height"],
                                      leaves["means"], leaves["log_scales"], leaves["quats_raw"],
                                      leaves["opacity_logits"], leaves["sh_dc"], leaves["sh_rest"],
                                      target, near_plane=cam["near"])
            (loss * weight).backward()
            total = total + loss.detach() * weight
        return total

    settle(step)
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        loss = step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    n = scene["params"]["means"].shape[0]
    params = [leaves[k] for k in ("means", "log_scales", "quats_raw", "opacity_logits",
                                  "sh_dc", "sh_rest")]

    def view(cam, target):  # one camera's weighted loss and its parameter gradients
        def f():
            loss, _, _, _ = render_l1(cam["w2c"], cam["K"], cam["width"], cam["height"], *params,
                                      target, near_plane=cam["near"])
            return (loss.detach() * weight,) + tuple(torch.autograd.grad(loss * weight, params))
        return f

    return {"ms_per_step": round(ms, 4), "cameras": len(cams),
            "gaussians_per_s": round(n / (ms * 1e-3), 1), "loss": round(float(loss), 6),
            "device_busy": busy(device_time(step, steps), ms),
            "graph": run_graph(step, steps, warmup, float(loss)),
            "graph_views": run_views([view(c, t) for c, t in zip(cams, targets)], steps, warmup,
                                     float(loss))}


def run_views(fns, steps: int, warmup: int, eager_loss: float, streams: int = 4) -> dict:
    """The cameras of one step each captured into a HIP graph and replayed on
    `streams` streams at once (cuda_rasterizer.graphs.ConcurrentSteps), their losses
    and gradients summed by a further graph: wall clock over `steps` replays after
    `warmup`, then the capacity check and the loss against the eager step's."""
    from cuda_rasterizer.graphs import ConcurrentSteps

    views = ConcurrentSteps(fns, streams=streams, warmup=max(warmup, 1))
    settle(views.replay, wait_each=True)
    for _ in range(warmup):
        views.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        out = views.replay()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    if not views.ok():
        raise RuntimeError("bench: a replay's tile lists outgrew the captured capacities")
    loss = float(out[0])
    if abs(loss - eager_loss) > 1e-5 * abs(eager_loss):
        raise RuntimeError(f"bench: concurrent replay loss {loss} != eager loss {eager_loss}")
    return {"ms_per_step": round(ms, 4), "streams": streams, "loss": round(loss, 6),
            "device_busy": busy(device_time(views.replay, steps), ms)}


def run_graph(step, steps: int, warmup: int, eager_loss: float) -> dict:
    """The same step captured into a HIP graph (cuda_rasterizer.graphs.CapturedStep)
    and replayed: wall clock over `steps` replays after `warmup` (which follow the
    profiler's replays and SETTLE_S seconds of untimed ones), synchronised on both
    sides; every capped sort of the last replay is checked against its
    capacities afterwards, and its loss against the eager step's (the parameters
    do not change between steps, so the two agree up to float summation order)."""
    from cuda_rasterizer.graphs import CapturedStep

    captured = CapturedStep(step, warmup=max(warmup, 1))
    # the profiler's kernel time first, then untimed replays that keep the GPU at
    # its working clocks up to the timed region's warm-up (as in run_gpu)
    device_ms = device_time(captured.replay, steps)
    settle(captured.replay, wait_each=True)
    for _ in range(warmup):
        captured.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        captured.replay()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    if not captured.ok():
        raise RuntimeError("bench: a replay's tile lists outgrew the captured capacities")
    out = captured.output
    loss = float((out[0] if isinstance(out, tuple) else out).detach())
    if abs(loss - eager_loss) > 1e-5 * abs(eager_loss):
        raise RuntimeError(f"bench: graph replay loss {loss} != eager loss {eager_loss}")
    return {"ms_per_step": round(ms, 4), "loss": round(loss, 6),
            "device_busy": busy(device_ms, ms)}


def run_small_configs(steps: int, warmup: int, cpu: bool) -> dict:
    """Configurations 1 and 2 on the GPU (fused fwd+bwd; configuration 2 over its 8
    cameras) and, with `cpu`, the oracle on the host CPU over the whole of each
    workload (configuration 2: its first camera)."""
    out = {}
    s1 = config1()
    r = run_gpu(s1, steps, warmup, "fused")
    dev = torch.device("cuda:0")
    leaves = {k: v.to(dev).requires_grad_(True) for k, v in s1["params"].items()}
    cam = dict(s1["camera"], w2c=s1["camera"]["w2c"].to(dev), K=s1["camera"]["K"].to(dev))
    target = s1["target"].to(dev)
    out["config1"] = {"workload": f"{r['n']} Gaussians SH0 {r['width']}x{r['height']} fwd+bwd L1",
                      "ms_per_step": round(r["ms"], 4), "keys": r["keys"],
                      "gaussians_per_s": round(r["n"] / (r["ms"] * 1e-3), 1),
                      "device_busy": r["device_busy"],
                      "graph": run_graph(lambda: fused_step(leaves, cam, target), steps, warmup,
                                         r["loss"])}
    s2 = config2()
    c2 = run_cameras(s2, steps, warmup)
    out["config2"] = dict(workload=f"{s2['params']['means'].shape[0]} Gaussians SH3 800x800 "
                                   f"fwd+bwd L1 over {c2['cameras']} cameras", **c2)
    if cpu:
        out["config1"]["cpu_baseline"] = cpu_baseline(s1, budget_s=float("inf"))
        out["config2"]["cpu_baseline"] = cpu_baseline(s2, budget_s=float("inf"))
        out["config2"]["cpu_baseline"]["sample"] += " (first camera only)"
    return out


def run_forward(scene: dict, steps: int, warmup: int) -> dict:
    """Configuration 4: forward-only render() (no autograd) of the scene, with
    HIP events around every entry point.  Reports the binning's keys per second
    (K over the count + sort time) and the blend's pixels per second."""
    from cuda_rasterizer import _lib
    from cuda_rasterizer.wrapper import render

    dev = torch.device("cuda:0")
    p = {k: v.to(dev) for k, v in scene["params"].items()}
    cam = scene["camera"]
    w2c, K = cam["w2c"].to(dev), cam["K"].to(dev)
    W, H = cam["width"], cam["height"]
    with torch.no_grad():
        scales, quats, opac = activated(p)

        def step():
            return render(w2c, K, W, H, p["means"], scales, quats, opac, p["sh_dc"],
                          p["sh_rest"], near_plane=cam["near"])

        settle(step)
        for _ in range(warmup):
            step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            step()
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / steps
        _lib.timer.reset()
        _lib.timer.only = None
        _lib.timer.enabled = True
        for _ in range(steps):
            step()
        _lib.timer.enabled = False
        st = {k: t / steps for k, (c, t) in _lib.timer.summary().items()}
        from cuda_rasterizer import compute_tile_intersection, project_points
        pts, depths, _, _, radii, mask = project_points(
            p["means"], scales, quats, opac, w2c, K, cam["near"], 100.0, 1 / 255, 0.5, 128.0, W, H)
        _, ids = compute_tile_intersection(pts, radii, depths, mask, W, H, 16)
    keys = int(ids.numel())
    bin_ms = st["bin_count"] + st["bin_sort"]
    blend_ms = st["rasterize_display"]
    return {"metric": "forward ms/iter; binning keys/s; blend pixels/s",
            "workload": f"{scene['name']}: {scene['params']['means'].shape[0]} Gaussians SH3 "
                        f"{W}x{H} forward-only render()",
            "ms_per_step": round(ms, 4), "keys": keys,
            "binning_keys_per_s": round(keys / (bin_ms * 1e-3), 1),
            "blend_pixels_per_s": round(W * H / (blend_ms * 1e-3), 1),
            "stages_ms": {k: round(v, 4) for k, v in st.items()}}


# ------------------------------------------------- configuration 5 (training)

def _torch_clone_top_and_prune(leaves: dict, optims: dict, grads: torch.Tensor, fraction: float,
                               jitter: float, prune_opacity: float = 0.005, generator=None):
    """The configuration-5 rule written the way src/strategy.py:71-229 rebuilds
    parameters and Adam state (index / cat per tensor, state moved to the new leaf).
    The rows to clone are chosen as cuda_rasterizer.train.top_rows chooses them.
    The jitter is drawn from `generator` as Densifier.clone_top_and_prune draws it."""
    opac = torch.sigmoid(leaves["opacity_logits"])
    keep = torch.where(~(opac < prune_opacity))[0]
    n_top = int(round(fraction * grads.shape[0]))
    from cuda_rasterizer.train import top_rows

    top = top_rows(grads, n_top)  # the library's rule: largest first, ties by index
    for name, p in list(leaves.items()):
        extra = p[top]
        if name == "means":
            extra = extra + torch.randn(extra.shape, device=extra.device,
                                        generator=generator) * jitter
        new = torch.cat([p[keep], extra]).detach().requires_grad_(True)
        opt = optims[name]
        state = opt.state.pop(p)
        for key in ("exp_avg", "exp_avg_sq"):
            s = state[key]
            state[key] = torch.cat([s[keep], torch.zeros((n_top,) + s.shape[1:], device=s.device)])
        opt.param_groups[0]["params"] = [new]
        opt.state[new] = state
        leaves[name] = new
    return int(opac.numel() - keep.numel()), n_top


def run_train(scene: dict, path: str = "fused", steps: int | None = None, every: int = 100,
              fraction: float = 0.05, jitter: float = 0.01) -> dict:
    """Configuration 5: `steps` training steps (render + L1 + backward + Adam), and
    every `every` steps clone the top `fraction` by accumulated |dL/d points_img|
    (in NDC scale, over visible steps: src/strategy.py:47-68) (means jittered by
    N(0, jitter)) and prune opacity < 0.005.

    path "fused": render_l1 + FusedAdam + Densifier (library kernels only);
    path "drop-in": the reference's loop -- PyTorch activations and l1_loss
    around the drop-in render(), one torch.optim.Adam per group
    (scripts/train.py:17-44), index/cat rebuilds.  Reports the average step
    time over the whole run (densification included) and peak HBM."""
    from cuda_rasterizer.fused import render_l1
    from cuda_rasterizer.train import Densifier, FusedAdam
    from cuda_rasterizer.wrapper import render

    dev = torch.device("cuda:0")
    w2c_all = scene["w2c_per_step"].to(dev)
    steps = steps or w2c_all.shape[0]
    targets = scene["targets"].to(dev)
    cam = scene["camera"]
    K = cam["K"].to(dev)
    W, H = cam["width"], cam["height"]
    leaves = {k: v.to(dev).requires_grad_(True) for k, v in scene["params"].items()}
    gen = torch.Generator(device=dev).manual_seed(0)
    if path == "fused":
        opt = FusedAdam(leaves, means_decay_steps=steps)
        dens = Densifier(leaves["means"].shape[0], dev)
    else:
        from cuda_rasterizer.train import DEFAULT_LR

        optims = {k: torch.optim.Adam([{"params": [p], "lr": DEFAULT_LR[k]}], eps=1e-15,
                                      betas=(0.9, 0.999)) for k, p in leaves.items()}
        sched = torch.optim.lr_scheduler.ExponentialLR(optims["means"], gamma=0.01 ** (1 / steps))
        grads = torch.zeros(leaves["means"].shape[0], device=dev)
    losses, sizes = [], []
    state = {"grads": None if path == "fused" else grads}

    def one_step(step, densify=True):
        target = targets[step % targets.shape[0]]
        if path == "fused":
            loss, _, _, _ = render_l1(w2c_all[step], K, W, H, leaves["means"], leaves["log_scales"],
                                      leaves["quats_raw"], leaves["opacity_logits"], leaves["sh_dc"],
                                      leaves["sh_rest"], target, near_plane=cam["near"],
                                      densifier=dens)
            loss.backward()
            opt.step()
            opt.zero_grad()
            if densify and (step + 1) % every == 0:
                dens.clone_top_and_prune(leaves, opt, fraction, jitter, generator=gen)
                sizes.append(leaves["means"].shape[0])
        else:
            grads = state["grads"]
            scales, quats, opac = activated(leaves)
            image, pts, radii = render(w2c_all[step], K, W, H, leaves["means"], scales, quats,
                                       opac, leaves["sh_dc"], leaves["sh_rest"],
                                       near_plane=cam["near"])
            pts.retain_grad()
            loss = torch.nn.functional.l1_loss(image / 255.0, target)
            loss.backward()
            with torch.no_grad():  # src/strategy.py:47-68
                g = pts.grad.clone()
                g[:, 0] *= W / 2.0
                g[:, 1] *= H / 2.0
                sel = torch.where((radii > 0.0).all(dim=1))[0]
                grads.index_add_(0, sel, g[sel].norm(dim=1))
            for o in optims.values():
                o.step()
                o.zero_grad(set_to_none=True)
            sched.step()
            if densify and (step + 1) % every == 0:
                with torch.no_grad():
                    _torch_clone_top_and_prune(leaves, optims, grads, fraction, jitter,
                                               generator=gen)
                state["grads"] = torch.zeros(leaves["means"].shape[0], device=dev)
                sizes.append(leaves["means"].shape[0])
        return loss

    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats(dev)
    base = torch.cuda.memory_allocated(dev)
    t0 = time.perf_counter()
    for step in range(steps):
        loss = one_step(step)
        if step % 100 == 0 or step == steps - 1:
            losses.append(loss.detach())
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    peak = torch.cuda.max_memory_allocated(dev)
    # device busy over a window of steps at the final size (no densification):
    # wall clock, then the same steps under the profiler
    window = 20
    cams = iter(range(window * 2))
    t2 = time.perf_counter()
    for _ in range(window):
        one_step(next(cams) % steps, densify=False)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t2) * 1e3 / window
    dev_ms = device_time(lambda: one_step(next(cams) % steps, densify=False), window)
    return dict(ms=(t1 - t0) * 1e3 / steps, steps=steps, peak_hbm_bytes=int(peak),
                peak_hbm_above_inputs_bytes=int(peak - base), n_start=scene["params"]["means"].shape[0],
                n_end=leaves["means"].shape[0], sizes=sizes,
                loss_first=float(losses[0]), loss_last=float(losses[-1]), width=W, height=H,
                device_busy=dict(busy(dev_ms, wall) or {}, window_ms_per_step=round(wall, 4),
                                 window=f"{window} steps at the final size, no densification"))


def train_stress(steps: int = 2000, which: str = "both") -> dict:
    """Configuration 5 through the library (fused) and through the reference's
    loop around the drop-in render() (drop-in), same scene and schedule."""
    scene = config5(steps=steps)
    out = {"workload": f"config5: {steps} steps from {scene['params']['means'].shape[0]} Gaussians "
                       f"SH3 1280x720, clone top 5% / prune every 100 steps"}
    for path in ("fused", "drop-in"):
        if which not in ("both", path):
            continue
        r = run_train(scene, path)
        out[path] = {"ms_per_step": round(r["ms"], 4), "peak_hbm_gib": round(r["peak_hbm_bytes"] / 2**30, 3),
                     "n_end": r["n_end"], "sizes": r["sizes"], "loss_first": round(r["loss_first"], 5),
                     "loss_last": round(r["loss_last"], 5), "device_busy": r["device_busy"]}
    return out


# ----------------------------------------------------------- roofline

# FP32 flops per evaluated (pixel, list entry) pair of the reference blend loop
# (src/cuda/kernel.cu:954-982 forward; :1063-1106 backward), exp counted as one
BLEND_FLOP_PER_PAIR = {"rasterize": 22.0, "rasterize_backward": 70.0, "rasterize_display": 22.0,
                       "rasterize_display_backward": 70.0, "rasterize_display_l1": 22.0,
                       "rasterize_l1_backward": 70.0}
HBM_STAGES = ("activate", "project_points", "evaluate_sh", "evaluate_sh_render", "bin_count",
              "bin_sort", "evaluate_sh_backward", "evaluate_sh_render_backward",
              "project_points_backward", "activate_backward", "preprocess_forward",
              "preprocess_project", "preprocess_backward")
# stages of the fused step that run on a second stream beside binning: their bytes
# count in the HBM stages, their time does not (it overlaps bin_count and bin_sort)
SIDE_STAGES = {"preprocess_project": ("evaluate_sh_render",)}


def sort_passes(n_tiles: int) -> int:
    """8-bit digit passes a 64-bit (tile << 32 | depth) radix sort needs: ceil((32 + bits(T)) / 8)."""
    return math.ceil((32 + math.ceil(math.log2(max(n_tiles, 2)))) / 8)


def sort_convention_bytes(n: int, k: int, n_tiles: int) -> float:
    """Bytes the reference's binning algorithm moves (count + scan 33 B/G, emit
    12 B/key, P 8-bit radix passes of 24 B/key over 64-bit keys, ranges 8 B/key +
    4 B/tile).  Reported beside the timing as work done per second; it is not
    traffic (this build sorts N depth keys and M supertile entries instead)."""
    return n * 33 + k * 12 + 24 * k * sort_passes(n_tiles) + k * 8 + 4 * n_tiles


def algorithmic_bytes(stage: str, n: int, k: int, n_tiles: int, hw: int) -> float:
    """Bytes one call of an entry point must move: every API tensor read once and
    written once at full size (compute_tile_intersection: points, radii, depths
    and mask in; the tile offsets and the K ids out)."""
    if stage == "project_points":  # means, scales, quats, opac -> uv, z, cov, conic, radii, mask
        return n * (12 + 12 + 16 + 4) + n * (8 + 4 + 12 + 12 + 8 + 1)
    if stage in ("evaluate_sh", "evaluate_sh_render"):  # means, dc, rest, mask -> colours
        return n * (12 + 12 + 180 + 1) + n * 12
    if stage == "evaluate_sh_backward":  # grad, means, rest, colours, mask -> grads of means, dc, rest
        return n * (12 + 12 + 180 + 12 + 1) + n * (12 + 12 + 180)
    if stage == "evaluate_sh_render_backward":  # grad, means, dc, rest, mask -> the same grads
        return n * (12 + 12 + 12 + 180 + 1) + n * (12 + 12 + 180)
    if stage == "project_points_backward":  # grads uv/conic, means, scales, quats, cov, mask -> 3 grads
        return n * (8 + 12 + 12 + 12 + 16 + 12 + 1) + n * (12 + 12 + 16)
    if stage == "bin_count":
        return n * 21
    if stage == "bin_sort":
        return k * 4 + 4 * n_tiles
    if stage == "rasterize":
        return k * 40 + 12 * hw
    if stage == "rasterize_display":  # + the clamped x255 image
        return k * 40 + 24 * hw
    if stage == "rasterize_display_l1":  # + the target read, per-tile loss sums
        return k * 40 + 36 * hw
    if stage in ("rasterize_backward", "rasterize_display_backward"):
        return 12 * hw + k * 76 + 36 * n
    if stage == "rasterize_l1_backward":  # image + target read instead of a gradient image
        return 24 * hw + k * 76 + 36 * n
    if stage == "preprocess_forward":  # raw parameters + SH -> projection, opacity, colours
        return n * (12 + 12 + 16 + 4 + 12 + 180) + n * (8 + 4 + 12 + 12 + 8 + 1 + 4 + 12)
    if stage == "preprocess_project":  # raw parameters -> projection, opacity (no colours)
        return n * (12 + 12 + 16 + 4) + n * (8 + 4 + 12 + 12 + 8 + 1 + 4)
    if stage == "preprocess_backward":  # 4 gradients, raw parameters, SH, cov, mask -> 6 gradients
        # (the API's tensors, as every stage here; the kernel reads the forward's 40-byte
        # colour-gradient cache instead of the 192 bytes of SH, so it moves fewer: the
        # counters' figure is hbm_stages.counter_achieved)
        return n * (8 + 12 + 4 + 12 + 12 + 12 + 16 + 4 + 12 + 180 + 12 + 1) + \
            n * (12 + 12 + 16 + 4 + 12 + 180)
    if stage == "activate":  # log-scales, quaternions, logits -> scales, unit quaternions, opacity
        return n * (12 + 16 + 4) * 2
    if stage == "activate_backward":  # 3 gradients + scales, quaternions, opacity -> 3 gradients
        return n * (12 + 16 + 4) * 3
    return 0.0


# the blend backward entry points: timed with HIP events inside the timed loop
DOMINANT_STAGES = {"rasterize_backward", "rasterize_display_backward", "rasterize_l1_backward"}

# kernel that implements each single-kernel entry point
STAGE_KERNEL = {"rasterize": "blend_forward_kernel", "rasterize_display": "blend_forward_kernel",
                "rasterize_display_l1": "blend_forward_kernel",
                "rasterize_backward": "blend_backward_kernel<0>",
                "rasterize_display_backward": "blend_backward_kernel<1>",
                "rasterize_l1_backward": "blend_backward_kernel<2>",
                "project_points": "project_points_kernel", "evaluate_sh": "sh_forward_kernel",
                "evaluate_sh_render": "sh_forward_kernel",
                "evaluate_sh_backward": "sh_backward_kernel",
                "evaluate_sh_render_backward": "sh_backward_kernel",
                "project_points_backward": "project_points_backward_kernel",
                "preprocess_forward": "preprocess_forward_kernel",
                "preprocess_project": "preprocess_forward_kernel",
                "preprocess_backward": "preprocess_backward_kernel"}


def kernel_base(name: str) -> str:
    """A profiled kernel name without the blend kernels' waves-per-tile template
    argument: blend_forward_kernel<1> -> blend_forward_kernel,
    blend_backward_kernel<2, 1> -> blend_backward_kernel<2>."""
    import re

    m = re.fullmatch(r"(blend_forward_kernel)<\d+>", name)
    if m:
        return m.group(1)
    m = re.fullmatch(r"(blend_backward_kernel<\d+), \d+>", name)
    return m.group(1) + ">" if m else name


def profiled_traffic(stage: str, workload: str):
    """HBM bytes per launch of `stage`'s kernel for `workload`, from the committed
    rocprofv3 FETCH_SIZE/WRITE_SIZE summary profiles/hbm_traffic_<workload>.md
    (line `traffic_bytes_per_launch[<kernel>]: <bytes>`), or None without one."""
    import re

    path = os.path.join(ROOT, "profiles", f"hbm_traffic_{workload}.md")
    kernel = STAGE_KERNEL.get(stage)
    if kernel is None or not os.path.exists(path):
        return None
    for name, nbytes in re.findall(r"^traffic_bytes_per_launch\[(.+?)\]:\s*([0-9.eE+]+)",
                                   open(path).read(), re.M):
        if kernel_base(name) == kernel:
            return float(nbytes)
    return None


# kernels of the HBM-bound stages (preprocess, the colours, binning, preprocess backward)
# of the fused step, by name prefix
HBM_STAGE_KERNELS = ("preprocess_forward_kernel", "sh_forward_kernel", "count_tiles_kernel",
                     "depth_upsweep0_kernel", "radix_upsweep_kernel", "radix_downsweep_kernel",
                     "digit_scan_kernel", "segment_sort_kernel",
                     "l1_scatter_kernel", "l2_count_kernel", "l2_prefix_kernel",
                     "l2_scatter_kernel", "preprocess_backward_kernel")


def counter_stage_bytes(workload: str) -> float | None:
    """HBM bytes per fused step of the HBM-stage kernels by the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE profile (launches per step x bytes per launch), or None
    without the profile."""
    import re

    path = os.path.join(ROOT, "profiles", f"hbm_traffic_{workload}.md")
    if not os.path.exists(path):
        return None
    rows = re.findall(r"^step_kernel\[(.+?)\]:\s*([0-9.eE+]+)\s+([0-9.eE+]+)\s*$",
                      open(path).read(), re.M)
    total = sum(float(launches) * float(nbytes) for name, launches, nbytes in rows
                if name.split("<")[0] in HBM_STAGE_KERNELS)
    return total or None


def roofline(res: dict, workload: str) -> dict:
    n, k, nt = res["n"], res["keys"], res["n_tiles"]
    hw = res["width"] * res["height"]
    steps = res["steps"]
    per_stage = {}
    for stage, (calls, ms) in res["stages"].items():
        b = algorithmic_bytes(stage, n, k, nt, hw)
        per_call = ms / max(calls / steps, 1)
        row = dict(ms=round(ms, 4), calls_per_step=calls // steps)
        if b and ms > 0:
            row["gbs"] = round(b / (per_call * 1e-3) / 1e9, 1)
        if stage in BLEND_FLOP_PER_PAIR and ms > 0:
            row["tflops"] = round(res["visited"] * BLEND_FLOP_PER_PAIR[stage] / (per_call * 1e-3) / 1e12, 2)
        per_stage[stage] = row

    dominant = max(res["stages"].items(), key=lambda kv: kv[1][1])[0]
    # the timed loop's own events when they cover the dominant stage
    launch_ms = res.get("main_launch_ms", {}).get(dominant)
    if launch_ms is None:
        calls, ms = res["stages"][dominant]
        launch_ms = ms / max(calls / steps, 1)
    per_launch_s = launch_ms * 1e-3
    traffic = profiled_traffic(dominant, workload)
    if dominant in BLEND_FLOP_PER_PAIR:
        achieved = res["visited"] * BLEND_FLOP_PER_PAIR[dominant] / per_launch_s / 1e12
        main = dict(bound="valu", achieved=round(achieved, 3), peak=FP32_PEAK_TFLOPS,
                    unit="TFLOP/s", frac=round(achieved / FP32_PEAK_TFLOPS, 4), traffic=traffic,
                    kernel=dominant, launch_ms=round(per_launch_s * 1e3, 4),
                    work=f"{res['visited']} evaluated (pixel, entry) pairs x "
                         f"{BLEND_FLOP_PER_PAIR[dominant]:g} flop")
    else:
        achieved = algorithmic_bytes(dominant, n, k, nt, hw) / per_launch_s / 1e9
        main = dict(bound="hbm", achieved=round(achieved, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                    frac=round(achieved / HBM_PEAK_GBS, 4), traffic=traffic, kernel=dominant,
                    launch_ms=round(per_launch_s * 1e3, 4))

    # HBM-bound stages together (preprocess fwd/bwd, binning and sort)
    hb = sum(algorithmic_bytes(s, n, k, nt, hw) * res["stages"][s][0] / steps
             for s in HBM_STAGES if s in res["stages"])
    beside = {b for s, bs in SIDE_STAGES.items() if s in res["stages"] for b in bs}
    ht = sum(res["stages"][s][1] for s in HBM_STAGES
             if s in res["stages"] and s not in beside) * 1e-3
    hbm = dict(achieved=round(hb / ht / 1e9, 1) if ht else None, peak=HBM_PEAK_GBS, unit="GB/s",
               frac=round(hb / ht / 1e9 / HBM_PEAK_GBS, 4) if ht else None, bytes=int(hb),
               ms=round(ht * 1e3, 4))
    if beside:
        hbm["beside_binning"] = sorted(beside)
    # the same window with the bytes the counters measured for those stages' kernels
    # (FETCH_SIZE + WRITE_SIZE per launch, profiles/hbm_traffic_<workload>.md): wasted
    # re-reads count here, so it is the DRAM traffic rate, not algorithmic work
    counted = counter_stage_bytes(workload)
    if counted and ht:
        hbm["counter_bytes"] = int(counted)
        hbm["counter_achieved"] = round(counted / ht / 1e9, 1)
        hbm["counter_frac"] = round(counted / ht / 1e9 / HBM_PEAK_GBS, 4)
    # the reference binning algorithm's bytes per second of this build's binning
    bt = sum(res["stages"][s][1] for s in ("bin_count", "bin_sort") if s in res["stages"]) * 1e-3
    if bt:
        hbm["binning_reference_algorithm_gbs"] = round(sort_convention_bytes(n, k, nt) / bt / 1e9, 1)
    return dict(dominant=dominant, roofline=main, hbm_stages=hbm, per_stage=per_stage)


def step_roofline(res: dict, workload: str) -> dict | None:
    """Speed-of-light fraction of the whole fused step.  Every kernel one step
    launches -- launches per step and HBM bytes per launch from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE profile of the same step
    (profiles/hbm_traffic_<workload>.md, lines `step_kernel[<kernel>]:
    <launches per step> <bytes per launch>`) -- is priced at its bound: its bytes
    at the HBM peak, and for the two blend kernels the larger of that and their
    flops (evaluated pairs x flop per pair) at the fp32 peak.  The sum of the
    bound times over the measured ms per step; None without the profile."""
    import re

    path = os.path.join(ROOT, "profiles", f"hbm_traffic_{workload}.md")
    if not os.path.exists(path):
        return None
    rows = re.findall(r"^step_kernel\[(.+?)\]:\s*([0-9.eE+]+)\s+([0-9.eE+]+)\s*$",
                      open(path).read(), re.M)
    if not rows:
        return None
    flop = {"blend_forward_kernel": BLEND_FLOP_PER_PAIR["rasterize_display_l1"],
            "blend_backward_kernel<2>": BLEND_FLOP_PER_PAIR["rasterize_l1_backward"]}
    bound_s, hbm_s, valu_s = 0.0, 0.0, 0.0
    for name, launches, nbytes in rows:
        t_hbm = float(nbytes) / (HBM_PEAK_GBS * 1e9)
        base = kernel_base(name)
        t_valu = res["visited"] * flop[base] / (FP32_PEAK_TFLOPS * 1e12) if base in flop else 0.0
        bound_s += float(launches) * max(t_hbm, t_valu)
        hbm_s += float(launches) * t_hbm
        valu_s += float(launches) * t_valu
    step_s = res["ms"] * 1e-3
    return dict(frac=round(bound_s / step_s, 4), bound_ms=round(bound_s * 1e3, 4),
                hbm_ms=round(hbm_s * 1e3, 4), valu_ms=round(valu_s * 1e3, 4),
                ms_per_step=round(res["ms"], 4), kernels=len(rows),
                source=os.path.relpath(path, ROOT))


# -------------------------------------------------------------- CPU leg

def cpu_baseline(scene: dict, budget_s: float = 12.0, batch_tiles: int = 128, seed: int = 0) -> dict:
    """The oracle (a restatement of src/torch_rasterizer.py) timed on the host CPU.

    Full fwd+bwd at the headline size does not fit in host RAM (autograd keeps
    ~15 KB per (tile, Gaussian) key), so the run is bounded: the whole
    preprocess + binning forward for all N Gaussians, then fwd+bwd of the blend
    over batches of randomly chosen non-empty tiles until `budget_s` seconds of
    blend work have run (blend inputs are detached leaves, so each batch's
    backward stops there), then the preprocess backward once from the
    accumulated gradients.  The blend time per tile is scaled to all non-empty
    tiles.  Reports ms per full iteration.
    """
    import numpy as np

    from oracle import blend
    from oracle import render as orender

    # the host's CPU share when the environment states it (OMP_NUM_THREADS), else every core
    torch.set_num_threads(max(1, int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
                              or os.cpu_count() or 1))
    leaves = {k: v.clone().requires_grad_(True) for k, v in scene["params"].items()}
    cam = scene["camera"]
    W, H = cam["width"], cam["height"]
    t0 = time.perf_counter()
    scales, quats, opac = activated(leaves)
    out = orender.render_stages(cam["w2c"], cam["K"], W, H, leaves["means"], scales, quats, opac,
                                leaves["sh_dc"], leaves["sh_rest"], near_plane=cam["near"], tiles=[])
    keep = out["proj"]["keep"]
    blend_in = [out["points_image"], out["conic"], torch.where(keep, opac, torch.zeros_like(opac)),
                out["colors"]]
    t_pre = time.perf_counter() - t0

    off = out["indexing_offset"].numpy()
    k = int(out["gaussian_ids_sorted"].numel())
    ends = np.append(off[1:], k)
    nonempty = np.nonzero(ends > off)[0]
    order = np.random.default_rng(seed).permutation(nonempty)
    sub = [t.detach().requires_grad_(True) for t in blend_in]
    done, t_tiles = 0, 0.0
    while done < len(order) and t_tiles < budget_s:
        batch = sorted(order[done:done + batch_tiles].tolist())
        t1 = time.perf_counter()
        raw = blend.rasterize(out["indexing_offset"], out["gaussian_ids_sorted"], *sub, W, H, 16,
                              1e-4, 1e-4, 9.21, tiles=batch)
        torch.nn.functional.l1_loss(raw.clamp(0, 1), scene["target"]).backward()
        t_tiles += time.perf_counter() - t1
        done += len(batch)

    t2 = time.perf_counter()
    torch.autograd.backward(blend_in, [t.grad for t in sub])
    t_pre_bwd = time.perf_counter() - t2
    total_s = t_pre + t_pre_bwd + t_tiles * len(nonempty) / max(done, 1)
    return dict(value=round(total_s * 1e3, 1), unit="ms/iter", cores=torch.get_num_threads(),
                kind="port",
                sample=(f"oracle (restated src/torch_rasterizer.py) on the same {scene['name']} inputs: "
                        f"preprocess+binning forward of all {scene['params']['means'].shape[0]} "
                        f"Gaussians ({t_pre:.1f} s), blend fwd+bwd of {done} random non-empty tiles "
                        f"({t_tiles:.1f} s) scaled to all {len(nonempty)} non-empty tiles, "
                        f"preprocess backward ({t_pre_bwd:.1f} s); cpu={cpu_model()}"))


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


# ------------------------------------------------------------------- main

def profile_step(scene: dict, steps: int) -> int:
    """`steps` fused steps and nothing else on the GPU after the inputs are copied
    (the copies are the only other dispatches), so that a rocprofv3 run's
    dispatch counts divided by `steps` are launches per step."""
    dev = torch.device("cuda:0")
    leaves = {k: v.to(dev).requires_grad_(True) for k, v in scene["params"].items()}
    cam = dict(scene["camera"], w2c=scene["camera"]["w2c"].to(dev), K=scene["camera"]["K"].to(dev))
    target = scene["target"].to(dev)
    torch.cuda.synchronize()
    for _ in range(steps):
        loss, _ = fused_step(leaves, cam, target)
    torch.cuda.synchronize()
    print(json.dumps({"profiled_steps": steps, "workload": scene["name"],
                      "loss": round(float(loss.detach()), 6)}), flush=True)
    return 0


def profile_ssim(scene: dict, steps: int) -> int:
    """`steps` SSIM loss terms (forward and backward, as run_ssim times them) and
    nothing else on the GPU after the inputs are copied, for rocprofv3 counter
    runs over the SSIM kernels alone."""
    from cuda_rasterizer import fused_ssim

    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(5)
    target = scene["target"].to(dev)
    img = (scene["target"] + 0.1 * torch.randn(scene["target"].shape, generator=g)).clamp(0, 1).to(dev)
    img.requires_grad_(True)
    torch.cuda.synchronize()
    for _ in range(steps):
        img.grad = None
        v = 1.0 - fused_ssim(img.permute(2, 0, 1).unsqueeze(0), target.permute(2, 0, 1).unsqueeze(0),
                             padding="valid")
        v.backward()
    torch.cuda.synchronize()
    W, H = scene["camera"]["width"], scene["camera"]["height"]
    print(json.dumps({"profiled_ssim_steps": steps, "workload": f"{W}x{H}x3 padding valid",
                      "ssim": round(1.0 - float(v.detach()), 6)}), flush=True)
    return 0


def copy_calibration(mib: int) -> int:
    """A plain device copy of known size: under rocprofv3 --pmc its FETCH_SIZE and
    WRITE_SIZE per dispatch give the counters' scale (expected: mib * 1024 KiB each)."""
    src = torch.full((mib * 2**18,), 1.5, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(4):  # an elementwise kernel (not a DMA copy): reads and writes mib MiB
        torch.mul(src, 1.0, out=dst)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": src.numel() * 4, "launches": 4}), flush=True)
    return 0


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", type=int, default=3, choices=[1, 2, 3, 4, 5],
                    help="3 (headline, default) or 1; 2 prints only the 8-camera step, 4 only "
                         "the forward-only sort and blend rates, 5 only the training stress run")
    ap.add_argument("--profile-step", action="store_true",
                    help="only run warmup + steps fused steps of the chosen configuration's first "
                         "view (for rocprofv3: every dispatch then belongs to a step) and print "
                         "the count")
    ap.add_argument("--profile-ssim", action="store_true",
                    help="only run warmup + steps SSIM loss terms (forward and backward) at the "
                         "chosen configuration's resolution (for rocprofv3 counter runs)")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip configurations 1, 2 and 4 beside the headline")
    ap.add_argument("--path", choices=["fused", "drop-in"], default="fused",
                    help="the timed step: fused render_l1 (default) or PyTorch glue around render()")
    ap.add_argument("--no-drop-in", action="store_true",
                    help="skip timing the drop-in path beside the fused one")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-train", action="store_true",
                    help="skip the configuration-5 training stress run beside the headline")
    ap.add_argument("--no-ssim", action="store_true",
                    help="skip timing the SSIM loss term at the headline resolution")
    ap.add_argument("--train-steps", type=int, default=2000)
    ap.add_argument("--train-path", choices=["both", "fused", "drop-in"], default="both",
                    help="which loops the training stress run times")
    ap.add_argument("--cpu-budget", type=float, default=12.0,
                    help="seconds of CPU blend work in the cpu_baseline sample")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run 4 device copies of MIB MiB (scales FETCH_SIZE/WRITE_SIZE counters)")
    args = ap.parse_args(argv)

    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(the multi-GPU design is documented but not built)", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py: no HIP device visible", file=sys.stderr)
        return 2

    if args.copy_calibration:
        return copy_calibration(args.copy_calibration)

    if args.profile_step:  # any configuration: its first view
        return profile_step(CONFIGS[args.config](), args.steps + args.warmup)
    if args.profile_ssim:
        return profile_ssim(CONFIGS[args.config](), args.steps + args.warmup)
    if args.config == 5:
        print(json.dumps(train_stress(args.train_steps, args.train_path)), flush=True)
        return 0
    if args.config == 4:
        print(json.dumps(run_forward(CONFIGS[4](), args.steps, args.warmup)), flush=True)
        return 0
    if args.config == 2:
        print(json.dumps(run_cameras(CONFIGS[2](), args.steps, args.warmup)), flush=True)
        return 0

    scene = CONFIGS[args.config]()
    res = run_gpu(scene, args.steps, args.warmup, args.path)
    rl = roofline(res, scene["name"])
    drop_in = None
    if args.path == "fused" and not args.no_drop_in:
        d = run_gpu(scene, args.steps, args.warmup, "drop-in")
        drop_in = {"ms_per_step": round(d["ms"], 3), "loss": d["loss"],
                   "device_busy": d["device_busy"],
                   "stages": roofline(d, scene["name"])["per_stage"]}
    graph = None
    if args.path == "fused":  # the same step captured once and replayed from a HIP graph
        dev = torch.device("cuda:0")
        leaves = {k: v.to(dev).requires_grad_(True) for k, v in scene["params"].items()}
        cam = dict(scene["camera"], w2c=scene["camera"]["w2c"].to(dev),
                   K=scene["camera"]["K"].to(dev))
        target = scene["target"].to(dev)
        graph = run_graph(lambda: fused_step(leaves, cam, target), args.steps, args.warmup,
                          res["loss"])
        del leaves, target
    view_cache = None
    if args.path == "fused":
        v = run_gpu(scene, args.steps, args.warmup, "fused", schedule_cache=True)
        view_cache = {"ms_per_step": round(v["ms"], 4),
                      "rasterize_display_l1_ms": round(v["stages"]["rasterize_display_l1"][1], 4),
                      "note": "the fused step with a per-view tile schedule cache: the forward "
                              "launches its tiles heaviest first by the last render of the same "
                              "view (a training view recurs every epoch; here every step)"}
    ssim = None if args.no_ssim else run_ssim(scene, args.steps, args.warmup)
    if ssim is not None and args.path == "fused":
        ssim["fused_step_l1_ssim"] = run_full_loss(scene, args.steps, args.warmup)
    train = None
    if not args.no_train and args.path == "fused":
        train = train_stress(args.train_steps, args.train_path)
    configs = None
    if not args.no_configs and args.config == 3:
        configs = run_small_configs(args.steps, args.warmup, not args.no_cpu_baseline)
        configs["config4"] = run_forward(config4(), args.steps, args.warmup)
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(scene, args.cpu_budget)
    line = {
        "metric": METRIC,
        "value": round(res["ms"], 3),
        "unit": "ms/iter",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(res["ms"], 3),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": f"{scene['name']}: {res['n']} Gaussians SH3 "
                               f"{res['width']}x{res['height']} fwd+bwd L1",
                   "path": args.path, "gaussians": res["n"], "visible": res["n_visible"],
                   "keys": res["keys"], "resolution": [res["width"], res["height"]]},
        "gaussians_per_s": round(res["n"] / (res["ms"] * 1e-3), 1),
        "device_busy": res["device_busy"],
        "roofline": rl["roofline"],
        "step_roofline": step_roofline(res, scene["name"]) if args.path == "fused" else None,
        "hbm_stages": rl["hbm_stages"],
        "blend_pairs": {"visited": res["visited"], "composited": res["composited"]},
        "stages": rl["per_stage"],
        "loss": res["loss"],
        "drop_in": drop_in,
        "graph": graph,
        "view_schedule_cache": view_cache,
        "ssim": ssim,
        "train_stress": train,
        "configs": configs,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
