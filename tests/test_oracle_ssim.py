"""CPU pinning of the SSIM oracle (oracle/ssim.py).

The third-party fused_ssim used by the reference's loss is absent, so the oracle
is pinned by what the mathematics fixes, each check chosen so that a plausible
slip fails it:
  * the window against scipy.signal.windows.gaussian (a wrong sigma, length or
    normalisation fails);
  * the separable blur against scipy.ndimage.correlate with the 2-D outer-product
    window and zero padding (a transposed axis, a shifted tap or another border
    rule fails);
  * SSIM(x, x) = 1 with a zero gradient, SSIM of constant images in closed form
    (a wrong C1 or luminance term fails), and SSIM(x, x + c) = the luminance term
    alone, the contrast-structure factor being exactly 1 (a wrong sigma term,
    C2 or sign fails);
  * the gradient against central finite differences of the oracle's own mean
    and against torch autograd of an independent F.conv2d formulation (a wrong
    derivative term, factor 2 or border fails);
  * the "valid" region, by a planted disturbance in the border that only "same"
    sees.
"""

from __future__ import annotations

import numpy as np
import pytest
import scipy.ndimage
import scipy.signal
import torch

from oracle import ssim as ossim


def rand_images(shape, seed):
    rng = np.random.default_rng(seed)
    a = rng.random(shape)
    b = np.clip(a + 0.2 * rng.standard_normal(shape), 0.0, 1.0)
    return a, b


def test_window_matches_scipy_gaussian():
    w = ossim.gaussian_window()
    ref = scipy.signal.windows.gaussian(11, 1.5)
    np.testing.assert_allclose(w, ref / ref.sum(), rtol=0, atol=1e-15)
    assert abs(w.sum() - 1.0) < 1e-15 and len(w) == 11


def test_blur_matches_scipy_2d_correlation():
    rng = np.random.default_rng(1)
    a = rng.standard_normal((2, 3, 17, 23))
    w = ossim.gaussian_window()
    w2 = np.outer(w, w)
    ref = np.stack([np.stack([scipy.ndimage.correlate(a[b, c], w2, mode="constant", cval=0.0)
                              for c in range(3)]) for b in range(2)])
    np.testing.assert_allclose(ossim.blur(a), ref, rtol=0, atol=1e-13)
    # a non-square, non-symmetric input detects a transposed axis
    assert not np.allclose(ossim.blur(a[..., :17, :17]), ossim.blur(a[..., :17, :17].swapaxes(-1, -2)))


@pytest.mark.parametrize("padding", ["same", "valid"])
def test_identical_images(padding):
    a, _ = rand_images((1, 3, 20, 24), 2)
    assert abs(ossim.ssim(a, a, padding) - 1.0) < 1e-12
    assert np.abs(ossim.ssim_backward(a, a, padding)).max() < 1e-12


def test_constant_images_closed_form():
    x, y = 0.3, 0.7
    a = np.full((1, 1, 16, 16), x)
    b = np.full((1, 1, 16, 16), y)
    want = (2 * x * y + ossim.C1) / (x * x + y * y + ossim.C1)
    assert abs(ossim.ssim(a, b, "valid") - want) < 1e-12


def test_shifted_image_is_luminance_only():
    """y = x + c: sigma2^2 = sigma12 = sigma1^2 inside the region, so the map is
    (2 mu1 mu2 + C1) / (mu1^2 + mu2^2 + C1) with mu2 = mu1 + c."""
    a, _ = rand_images((1, 2, 22, 19), 3)
    c = 0.15
    w2 = np.outer(ossim.gaussian_window(), ossim.gaussian_window())
    mu1 = np.stack([scipy.ndimage.correlate(a[0, k], w2, mode="constant") for k in range(2)])[None]
    ones = scipy.ndimage.correlate(np.ones(a.shape[-2:]), w2, mode="constant")
    mu2 = mu1 + c * ones  # the zero padding scales the shift near the border
    lum = (2 * mu1 * mu2 + ossim.C1) / (mu1 ** 2 + mu2 ** 2 + ossim.C1)
    m = ossim.region_mask(22, 19, "valid")
    assert abs(ossim.ssim(a, a + c, "valid") - lum[..., m].mean()) < 1e-12


@pytest.mark.parametrize("padding", ["same", "valid"])
def test_gradient_matches_finite_differences(padding):
    a, b = rand_images((1, 2, 13, 14), 4)
    g = ossim.ssim_backward(a, b, padding, grad_out=1.0)
    rng = np.random.default_rng(5)
    h = 1e-6
    for _ in range(12):
        idx = (0, rng.integers(2), rng.integers(13), rng.integers(14))
        ap, am = a.copy(), a.copy()
        ap[idx] += h
        am[idx] -= h
        fd = (ossim.ssim(ap, b, padding) - ossim.ssim(am, b, padding)) / (2 * h)
        assert abs(fd - g[idx]) < 1e-8 + 1e-5 * abs(fd), (idx, fd, g[idx])


def torch_ssim(x, y, padding):
    """Independent formulation: conv2d with the 2-D window, autograd for the gradient."""
    w = torch.tensor(ossim.gaussian_window(), dtype=torch.float64)
    w2 = torch.outer(w, w)[None, None].repeat(x.shape[1], 1, 1, 1)

    def f(z):
        return torch.nn.functional.conv2d(z, w2, padding=5, groups=x.shape[1])

    mu1, mu2 = f(x), f(y)
    s11 = f(x * x) - mu1 ** 2
    s22 = f(y * y) - mu2 ** 2
    s12 = f(x * y) - mu1 * mu2
    smap = ((2 * mu1 * mu2 + 1e-4) * (2 * s12 + 9e-4)) / ((mu1 ** 2 + mu2 ** 2 + 1e-4) * (s11 + s22 + 9e-4))
    if padding == "valid":
        smap = smap[:, :, 5:-5, 5:-5]
    return smap.mean()


@pytest.mark.parametrize("padding", ["same", "valid"])
def test_gradient_matches_torch_autograd(padding):
    a, b = rand_images((2, 3, 21, 18), 6)
    xt = torch.tensor(a, requires_grad=True)
    val = torch_ssim(xt, torch.tensor(b), padding)
    (val * 0.7).backward()
    assert abs(val.item() - ossim.ssim(a, b, padding)) < 1e-12
    np.testing.assert_allclose(ossim.ssim_backward(a, b, padding, grad_out=0.7), xt.grad.numpy(),
                               rtol=0, atol=1e-12)


def test_valid_region_ignores_the_border():
    a, b = rand_images((1, 1, 24, 24), 7)
    b2 = b.copy()
    b2[..., 0, :] = 1.0 - b2[..., 0, :]  # disturb row 0 only
    # row 0 reaches statistics of rows 0..5; "valid" keeps rows >= 5 whose window
    # reaches row 0 only from row 5, so row 5's map changes and row 6's does not
    t1 = ossim.ssim_terms(a, b)["map"]
    t2 = ossim.ssim_terms(a, b2)["map"]
    assert not np.allclose(t1[..., 5, 5:-5], t2[..., 5, 5:-5])
    np.testing.assert_allclose(t1[..., 6:, :], t2[..., 6:, :], rtol=0, atol=1e-15)
    assert ossim.ssim(a, b, "same") != ossim.ssim(a, b2, "same")


def test_empty_valid_region_is_nan():
    a, b = rand_images((1, 1, 10, 30), 8)
    assert np.isnan(ossim.ssim(a, b, "valid"))
    assert not np.any(ossim.ssim_backward(a, b, "valid"))
    with pytest.raises(ValueError):
        ossim.region_mask(4, 4, "full")
