"""Steps captured into HIP graphs (cuda_rasterizer.graphs.CapturedStep): the
fused step (render_l1 forward + backward) and the drop-in step (PyTorch
activations, render(), backward from a fixed gradient of the display image),
replayed.

Each replay is checked against an eager call on the same parameter values, with
in-place parameter updates, eager work and synchronisations between the
replays: the replay must read the updated parameters.  Loss and display are
bit-equal (the same kernels on the same inputs; the capped lists do not depend
on the capacity); gradients within relative L2 1e-5, 5e-5 for the raw
quaternions (the blend backward's float atomics land in a different order, and
the quaternion normalisation's backward cancels: the bar of the configuration-3
fused-vs-drop-in test for the same reason).  A replay
whose lists outgrow the capacities fixed at capture is reported by ok(), and a
recapture after an eager call covers the larger lists.

The drop-in step leaves PyTorch's l1_loss out of the graph: its multi-block
mean clears a semaphore with a memset node, and such replays gave a loss of 0
after the first one here.  The fused step's loss is reduced by the library's
own kernel, which clears nothing with memsets.
"""

from __future__ import annotations

import pytest
import torch

import helpers
from cuda_rasterizer.fused import render_l1
from cuda_rasterizer.graphs import CapturedStep
from cuda_rasterizer.wrapper import render

pytestmark = pytest.mark.gpu

W, H = 256, 192
ORDER_BAR = {k: 5e-5 if k == "quats_raw" else 1e-5 for k in helpers.PARAMS}


def _scene(gpu):
    p, cam, target = helpers.scene_orbit(20_000, W, H, 300.0, seed=41)
    return p, cam["w2c"].to(gpu), cam["K"].to(gpu), target.to(gpu)


def _leaves(p, gpu):
    return {k: v.clone().to(gpu).requires_grad_(True) for k, v in p.items()}


def _step_fn(path, leaves, w2c, K, target):
    def fused():
        for t in leaves.values():
            t.grad = None
        loss, display, _, _ = render_l1(w2c, K, W, H, leaves["means"], leaves["log_scales"],
                                        leaves["quats_raw"], leaves["opacity_logits"],
                                        leaves["sh_dc"], leaves["sh_rest"], target)
        loss.backward()
        return loss, display

    seed = (target - 0.5) / (W * H)  # a fixed gradient of the display image

    def drop_in():
        for t in leaves.values():
            t.grad = None
        scales, quats, opac = helpers.activated(leaves)
        display, _, _ = render(w2c, K, W, H, leaves["means"], scales, quats, opac,
                               leaves["sh_dc"], leaves["sh_rest"])
        display.backward(seed)
        return display[0, 0, 0].detach(), display

    return fused if path == "fused" else drop_in


def _perturb(leaves_list, step):
    g = torch.Generator().manual_seed(100 + step)
    noise = torch.randn(leaves_list[0]["means"].shape, generator=g) * 0.01
    for lv in leaves_list:
        with torch.no_grad():
            lv["means"].add_(noise.to(lv["means"].device))
            lv["opacity_logits"].mul_(0.99)


@pytest.mark.parametrize("path", ["fused", "drop-in"])
def test_captured_step_replays_match_eager(gpu, path):
    p, w2c, K, target = _scene(gpu)
    b, e = _leaves(p, gpu), _leaves(p, gpu)
    step = CapturedStep(_step_fn(path, b, w2c, K, target))
    eager = _step_fn(path, e, w2c, K, target)
    for i in range(3):
        _perturb([b, e], i)
        step.replay()
        loss_e, disp_e = eager()  # eager work on the same stream between replays
        assert step.ok(), i
        loss_g, disp_g = step.output
        assert float(loss_g) == float(loss_e), (path, i)
        assert torch.equal(disp_g, disp_e), (path, i)
        for k in helpers.PARAMS:
            assert helpers.rel_l2(b[k].grad, e[k].grad) <= ORDER_BAR[k], (path, i, k)
        torch.cuda.synchronize()


def test_captured_step_reports_outgrown_lists(gpu):
    p, w2c, K, target = _scene(gpu)
    b, e = _leaves(p, gpu), _leaves(p, gpu)
    step = CapturedStep(_step_fn("fused", b, w2c, K, target))
    step.replay()
    assert step.ok()
    # larger splats: more tiles per Gaussian than the capacities fixed at capture
    for lv in (b, e):
        with torch.no_grad():
            lv["log_scales"].add_(1.0)
    step.replay()
    assert not step.ok()
    # an eager call bins with exact sizes and raises the capacities; recapture
    eager = _step_fn("fused", e, w2c, K, target)
    loss_e, disp_e = eager()
    step.recapture()
    step.replay()
    assert step.ok()
    loss_e, disp_e = eager()
    loss_g, disp_g = step.output
    assert float(loss_g) == float(loss_e)
    assert torch.equal(disp_g, disp_e)
    for k in helpers.PARAMS:
        assert helpers.rel_l2(b[k].grad, e[k].grad) <= ORDER_BAR[k], k


def test_concurrent_views_match_the_sequential_step(gpu):
    """ConcurrentSteps: three views of one scene, each captured into its own graph
    (loss and torch.autograd.grad of the parameters) and replayed on two streams at
    once, summed by a further graph.  Against the sequential eager step (each
    view's weighted loss backward into the leaves' .grad), with in-place parameter
    updates between replays: loss within 1e-6 relative (the sum's order), gradients
    within the summation-order bars."""
    from cuda_rasterizer.graphs import ConcurrentSteps

    views = []
    for az in (0.7, 2.2, 4.1):
        p, cam, target = helpers.scene_orbit(20_000, W, H, 300.0, seed=41, azimuth=az)
        views.append((cam["w2c"].to(gpu), cam["K"].to(gpu), target.to(gpu)))
    b, e = _leaves(p, gpu), _leaves(p, gpu)
    params = [b[k] for k in helpers.PARAMS]
    weight = 1.0 / len(views)

    def view_fn(w2c, K, target):
        def f():
            loss, _, _, _ = render_l1(w2c, K, W, H, *params, target)
            grads = torch.autograd.grad(loss * weight, params)
            return (loss.detach() * weight,) + tuple(grads)
        return f

    steps = ConcurrentSteps([view_fn(*v) for v in views], streams=2)

    def eager():
        for t in e.values():
            t.grad = None
        total = 0.0
        for w2c, K, target in views:
            loss, _, _, _ = render_l1(w2c, K, W, H, *[e[k] for k in helpers.PARAMS], target)
            (loss * weight).backward()
            total = total + float(loss) * weight
        return total

    for i in range(3):
        _perturb([b, e], i)
        out = steps.replay()
        loss_e = eager()
        assert steps.ok(), i
        assert abs(float(out[0]) - loss_e) <= 1e-6 * loss_e, i
        for j, k in enumerate(helpers.PARAMS):
            assert helpers.rel_l2(out[1 + j], e[k].grad) <= ORDER_BAR[k], (i, k)
        torch.cuda.synchronize()
