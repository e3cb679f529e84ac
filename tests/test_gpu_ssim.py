"""GPU parity: fused_ssim (gs_ssim_forward / gs_ssim_backward) against the SSIM
oracle (oracle/ssim.py, float64).

Tolerances (float32 statistics against float64): mean SSIM abs error <= 2e-6,
gradient relative L2 <= 1e-4 and max abs error <= 1e-4 * max |gradient|.
The full-size case is the reference's training call at configuration 3's
resolution: a (1080, 1920, 3) image permuted to (1, 3, 1080, 1920),
padding="valid" (scripts/train.py:193-197).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import helpers
from cuda_rasterizer import fused_ssim
from cuda_rasterizer.ssim import ssim_backward, ssim_forward
from oracle import ssim as ossim

pytestmark = pytest.mark.gpu

MEAN_TOL = 2e-6
GRAD_REL = 1e-4


def images(shape, seed, noise=0.2):
    g = torch.Generator().manual_seed(seed)
    a = torch.rand(shape, generator=g)
    b = (a + noise * torch.randn(shape, generator=g)).clamp(0.0, 1.0)
    return a, b


def run(img1, img2, padding, grad_out=1.0):
    x = img1.clone().requires_grad_(True)
    val = fused_ssim(x, img2, padding=padding)
    (val * grad_out).backward()
    return val.detach(), x.grad


def check_against_oracle(a, b, padding, val, grad, grad_out=1.0):
    an = a.detach().double().cpu().numpy()
    bn = b.detach().double().cpu().numpy()
    want = ossim.ssim(an, bn, padding)
    want_g = torch.from_numpy(ossim.ssim_backward(an, bn, padding, grad_out=grad_out))
    assert abs(float(val) - want) <= MEAN_TOL, (float(val), want)
    assert helpers.rel_l2(grad, want_g) <= GRAD_REL
    assert helpers.max_abs(grad, want_g) <= 1e-4 * float(want_g.abs().max())


@pytest.mark.parametrize("padding", ["same", "valid"])
@pytest.mark.parametrize("shape", [(2, 3, 37, 70), (1, 1, 11, 11), (1, 2, 64, 32), (3, 1, 97, 129)])
def test_ssim_matches_oracle(gpu, shape, padding):
    a, b = images(shape, seed=sum(shape))
    val, grad = run(a.to(gpu), b.to(gpu), padding, grad_out=0.37)
    check_against_oracle(a, b, padding, val, grad, grad_out=0.37)


def test_reference_call_layout_full_size(gpu):
    """(H, W, 3) images permuted to (1, 3, H, W) as the reference does, at
    1920x1080: same values as the contiguous call, gradient laid out like img1."""
    h, w = 1080, 1920
    a, b = images((h, w, 3), seed=11, noise=0.1)
    x = a.to(gpu).requires_grad_(True)
    y = b.to(gpu)
    val = 1.0 - fused_ssim(x.permute(2, 0, 1).unsqueeze(0), y.permute(2, 0, 1).unsqueeze(0),
                           padding="valid")
    val.backward()
    assert x.grad.shape == (h, w, 3) and x.grad.is_contiguous()
    a4 = a.permute(2, 0, 1).unsqueeze(0).contiguous()
    b4 = b.permute(2, 0, 1).unsqueeze(0).contiguous()
    val_c, grad_c = run(a4.to(gpu), b4.to(gpu), "valid", grad_out=-1.0)
    # the arithmetic does not depend on the strides: bit-equal results
    assert helpers.same(val.detach(), 1.0 - val_c)
    assert helpers.same(x.grad.permute(2, 0, 1).unsqueeze(0), grad_c)
    check_against_oracle(a4, b4, "valid", val_c, grad_c, grad_out=-1.0)


def test_identical_images_give_one(gpu):
    a, _ = images((1, 3, 50, 60), seed=3)
    val, grad = run(a.to(gpu), a.to(gpu), "valid")
    assert abs(float(val) - 1.0) <= 1e-6
    assert float(grad.abs().max()) <= 1e-6


def test_deterministic(gpu):
    a, b = images((1, 3, 200, 300), seed=4)
    v1, g1 = run(a.to(gpu), b.to(gpu), "valid")
    v2, g2 = run(a.to(gpu), b.to(gpu), "valid")
    assert helpers.same(v1, v2) and helpers.same(g1, g2)


def test_empty_valid_region(gpu):
    a, b = images((1, 3, 10, 40), seed=5)
    val, grad = run(a.to(gpu), b.to(gpu), "valid")
    assert torch.isnan(val)
    assert float(grad.abs().max()) == 0.0


def test_no_maps_without_grad(gpu):
    a, b = images((1, 3, 20, 20), seed=6)
    mean, maps = ssim_forward(a.to(gpu), b.to(gpu), "same", with_maps=False)
    assert maps == (None, None, None)
    assert abs(float(mean) - ossim.ssim(a.double().numpy(), b.double().numpy(), "same")) <= MEAN_TOL
    with torch.no_grad():
        v = fused_ssim(a.to(gpu), b.to(gpu), train=False)
    assert helpers.same(v, mean)
    x = a.to(gpu).requires_grad_(True)
    with pytest.raises(RuntimeError):
        fused_ssim(x, b.to(gpu), train=False).backward()


def test_argument_errors(gpu):
    a, b = images((1, 3, 20, 20), seed=7)
    with pytest.raises(ValueError):
        fused_ssim(a.to(gpu), b.to(gpu), padding="full")
    with pytest.raises(RuntimeError, match="float32"):
        fused_ssim(a.to(gpu).double(), b.to(gpu).double())
    with pytest.raises(RuntimeError, match="shapes"):
        fused_ssim(a.to(gpu), b[..., :10].to(gpu))


def test_training_loss_through_render(gpu):
    """The reference's loss 0.8 * L1 + 0.2 * (1 - SSIM_valid) on a rendered image
    (scripts/check_cuda_gradients.py:975-981): parameter gradients through the
    drop-in render match the oracle render with the oracle's SSIM gradient
    injected at the image."""
    from cuda_rasterizer.wrapper import render
    from oracle import render as orender

    p, cam, target = helpers.scene_orbit(3000, 96, 80, 110.0, seed=21)

    def loss_grads(render_fn, device, ssim_fn):
        leaves = {k: v.to(device).clone().requires_grad_(True) for k, v in p.items()}
        scales, quats, opac = helpers.activated(leaves)
        image, _, _ = render_fn(cam["w2c"].to(device), cam["K"].to(device), cam["width"],
                                cam["height"], leaves["means"], scales, quats, opac,
                                leaves["sh_dc"], leaves["sh_rest"])
        img = image / 255.0
        tgt = target.to(device)
        loss = 0.8 * torch.nn.functional.l1_loss(img, tgt) + 0.2 * (1.0 - ssim_fn(img, tgt))
        loss.backward()
        return image.detach(), loss.detach(), {k: v.grad for k, v in leaves.items()}

    def gpu_ssim(img, tgt):
        return fused_ssim(img.permute(2, 0, 1).unsqueeze(0), tgt.permute(2, 0, 1).unsqueeze(0),
                          padding="valid")

    class OracleSSIM(torch.autograd.Function):
        @staticmethod
        def forward(ctx, img, tgt):
            a = img.detach().permute(2, 0, 1).unsqueeze(0).double().numpy()
            b = tgt.detach().permute(2, 0, 1).unsqueeze(0).double().numpy()
            ctx.g = ossim.ssim_backward(a, b, "valid")
            return torch.tensor(ossim.ssim(a, b, "valid"), dtype=img.dtype)

        @staticmethod
        def backward(ctx, go):
            g = torch.from_numpy(ctx.g[0]).permute(1, 2, 0).float()
            return go * g, None

    img_g, loss_g, grads_g = loss_grads(render, gpu, gpu_ssim)
    img_c, loss_c, grads_c = loss_grads(orender.render, "cpu", OracleSSIM.apply)
    assert helpers.max_abs(img_g / 255.0, img_c / 255.0) <= 1e-4
    assert abs(float(loss_g) - float(loss_c)) <= 1e-5
    for k in helpers.PARAMS:
        assert helpers.rel_l2(grads_g[k], grads_c[k]) <= 1e-3, k


def test_backward_entry_scales_by_grad_mean(gpu):
    a, b = images((1, 2, 30, 40), seed=8)
    a, b = a.to(gpu), b.to(gpu)
    _, maps = ssim_forward(a, b, "valid")
    g1 = ssim_backward(torch.ones(1, device=gpu), a, b, maps)
    g3 = ssim_backward(torch.full((1,), -3.0, device=gpu), a, b, maps)
    torch.testing.assert_close(g3, -3.0 * g1, rtol=1e-6, atol=0)
    want = ossim.ssim_backward(a.double().cpu().numpy(), b.double().cpu().numpy(), "valid")
    assert helpers.rel_l2(g1, torch.from_numpy(want)) <= GRAD_REL


def test_divisor_combined_loss_and_grad_scale(gpu):
    """img1_divisor = 255 on a [0, 255] image equals the plain call on image / 255
    (the same true division); the combined loss is (1 - lam) * other + lam * (1 - mean);
    grad_scale multiplies the upstream gradient."""
    a, b = images((1, 3, 40, 50), seed=9)
    a255, b = (a * 255.0).to(gpu), b.to(gpu)
    other = torch.full((1,), 0.3, device=gpu)
    mean_d, maps_d, loss = ssim_forward(a255, b, "valid", with_maps=True, img1_divisor=255.0,
                                        other_loss=other, lam=0.2)
    mean_p, maps_p = ssim_forward(a255 / 255.0, b, "valid", with_maps=True)
    assert helpers.same(mean_d, mean_p)
    for x, y in zip(maps_d, maps_p):
        assert helpers.same(x, y)
    want = (1.0 - 0.2) * 0.3 + 0.2 * (1.0 - float(mean_p))
    assert abs(float(loss) - want) <= 1e-6
    g = torch.full((1,), 1.5, device=gpu)
    gd = ssim_backward(g, a255, b, maps_d, img1_divisor=255.0, grad_scale=-0.2)
    gp = ssim_backward(g * -0.2, a255 / 255.0, b, maps_p)
    torch.testing.assert_close(gd, gp, rtol=1e-6, atol=0)
