"""fused_ssim -- drop-in for the SSIM loss the reference's training loop calls.

The reference computes its loss as
    0.8 * L1 + 0.2 * (1 - fused_ssim(img1, img2, padding="valid"))
(scripts/train.py:185-205, scripts/check_cuda_gradients.py:975-980), importing
`fused_ssim` from the third-party package fused-ssim (environment.yml:56, not
vendored).  This module gives the same call, `fused_ssim(img1, img2,
padding="same", train=True)`, on the library's gfx950 kernels
(gs_ssim_forward / gs_ssim_backward): the mean SSIM of (B, C, H, W) float32
images in [0, 1] (11x11 Gaussian window, sigma 1.5, zero padding,
C1 = 0.01^2, C2 = 0.03^2), averaged over every pixel ("same") or over the
pixels at least 5 from the border ("valid"), differentiable with respect to
img1 only.  Inputs may have any strides (the reference passes permuted
(H, W, C) images); the gradient has img1's strides.  With train=False, or when
img1 does not require a gradient, no derivative maps are kept.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib

C1 = 0.01 ** 2
C2 = 0.03 ** 2


def _strides(t: torch.Tensor):
    return (ctypes.c_int64 * 4)(*t.stride())


def _sp(arr) -> int:
    return ctypes.cast(arr, ctypes.c_void_p).value


def _check(img1: torch.Tensor, img2: torch.Tensor):
    for name, t in (("img1", img1), ("img2", img2)):
        if not isinstance(t, torch.Tensor):
            raise RuntimeError(f"fused_ssim: {name} must be a torch.Tensor")
        if t.device.type != "cuda":
            raise RuntimeError(f"fused_ssim runs on the GPU only; {name} is on {t.device} "
                               "(there is no CPU fallback)")
        if t.dtype != torch.float32:
            raise RuntimeError(f"fused_ssim: {name} must be float32, got {t.dtype}")
        if t.dim() != 4:
            raise RuntimeError(f"fused_ssim: {name} must be (B, C, H, W), got {tuple(t.shape)}")
    if img1.shape != img2.shape or img1.device != img2.device:
        raise RuntimeError(f"fused_ssim: shapes/devices differ: {tuple(img1.shape)} on "
                           f"{img1.device} vs {tuple(img2.shape)} on {img2.device}")


def ssim_forward(img1: torch.Tensor, img2: torch.Tensor, padding: str = "same",
                 with_maps: bool = True, img1_divisor: float = 1.0,
                 other_loss: torch.Tensor | None = None, lam: float = 0.0):
    """Mean SSIM (0-d float32 device tensor), with_maps the three (B*C, H, W)
    derivative maps that ssim_backward reads, and -- with other_loss (a 1-element
    float32 device tensor) -- the combined loss (1 - lam) * other_loss +
    lam * (1 - mean) (else None), all from one launch pair.  The SSIM sees
    img1 / img1_divisor as PyTorch's GPU kernels compute it (times the float
    reciprocal), so a display image with divisor 255 equals display / 255.0."""
    _check(img1, img2)
    if padding not in ("same", "valid"):
        raise ValueError(f"fused_ssim: padding must be 'same' or 'valid', got {padding!r}")
    dev = img1.device
    b, c, h, w = (int(x) for x in img1.shape)
    lib = _lib.load()
    sz = ctypes.c_size_t(0)
    _lib.check(lib.gs_ssim_workspace_size(b, c, h, w, ctypes.byref(sz)), "ssim_workspace_size")
    ws = torch.empty(max(int(sz.value), 8), dtype=torch.uint8, device=dev)
    mean = torch.empty((), dtype=torch.float32, device=dev)
    loss = None if other_loss is None else torch.empty((), dtype=torch.float32, device=dev)
    maps = (tuple(torch.empty((b * c, h, w), dtype=torch.float32, device=dev) for _ in range(3))
            if with_maps else (None, None, None))
    s1, s2 = _strides(img1), _strides(img2)
    with torch.cuda.device(dev):
        ev = _lib.timer.record("ssim_forward", dev)
        _lib.check(lib.gs_ssim_forward(
            img1.data_ptr(), _sp(s1), img2.data_ptr(), _sp(s2), b, c, h, w,
            1 if padding == "valid" else 0, float(img1_divisor), mean.data_ptr(),
            *(None if m is None else m.data_ptr() for m in maps),
            None if other_loss is None else other_loss.data_ptr(), float(lam),
            None if loss is None else loss.data_ptr(), ws.data_ptr(), int(sz.value),
            torch.cuda.current_stream(dev).cuda_stream), "ssim_forward")
        _lib.timer.stop(ev, dev)
    if other_loss is not None:
        return mean, maps, loss
    return mean, maps


def ssim_backward(grad_mean: torch.Tensor, img1: torch.Tensor, img2: torch.Tensor, maps,
                  img1_divisor: float = 1.0, grad_scale: float = 1.0):
    """grad_scale * grad_mean (a 1-element float32 device tensor) times
    d(mean SSIM)/d x, x = img1 / img1_divisor; laid out like img1 when img1 is
    dense, else contiguous."""
    _check(img1, img2)
    dev = img1.device
    b, c, h, w = (int(x) for x in img1.shape)
    g = grad_mean.reshape(1).to(device=dev, dtype=torch.float32).contiguous()
    grad = torch.empty_like(img1)
    s1, s2, sg = _strides(img1), _strides(img2), _strides(grad)
    with torch.cuda.device(dev):
        ev = _lib.timer.record("ssim_backward", dev)
        _lib.check(_lib.load().gs_ssim_backward(
            g.data_ptr(), img1.data_ptr(), _sp(s1), img2.data_ptr(), _sp(s2), b, c, h, w,
            float(img1_divisor), *(m.data_ptr() for m in maps), float(grad_scale),
            grad.data_ptr(), _sp(sg), torch.cuda.current_stream(dev).cuda_stream),
            "ssim_backward")
        _lib.timer.stop(ev, dev)
    return grad


class _FusedSSIM(torch.autograd.Function):
    @staticmethod
    def forward(ctx, img1, img2, padding, train):
        keep = bool(train) and ctx.needs_input_grad[0]
        mean, maps = ssim_forward(img1.detach(), img2.detach(), padding, with_maps=keep)
        if keep:
            ctx.save_for_backward(img1.detach(), img2.detach(), *maps)
        return mean

    @staticmethod
    def backward(ctx, grad_mean):
        if not ctx.saved_tensors:
            raise RuntimeError("fused_ssim: backward needs train=True in the forward call")
        img1, img2, m1, m2, m3 = ctx.saved_tensors
        return ssim_backward(grad_mean, img1, img2, (m1, m2, m3)), None, None, None


def fused_ssim(img1: torch.Tensor, img2: torch.Tensor, padding: str = "same",
               train: bool = True) -> torch.Tensor:
    """Mean SSIM of img1 against img2 ((B, C, H, W) float32 on the GPU, values in
    [0, 1]); differentiable with respect to img1."""
    if padding not in ("same", "valid"):
        raise ValueError(f"fused_ssim: padding must be 'same' or 'valid', got {padding!r}")
    return _FusedSSIM.apply(img1, img2, padding, train)
