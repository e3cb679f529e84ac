"""CPU oracle for the SSIM loss term -- TEST INFRASTRUCTURE ONLY.

The reference's training loss (scripts/train.py:185-205, and the end-to-end check
scripts/check_cuda_gradients.py:975-980) is
    0.8 * L1 + 0.2 * (1 - fused_ssim(img1, img2, padding="valid"))
with img1 = the rendered image and img2 = the target, both (H, W, C) / 255
permuted to (1, C, H, W).  `fused_ssim` is the third-party package fused-ssim,
pinned as fused-ssim==0.0.0 (a source install, environment.yml:56); it is not
vendored in the reference and not importable here.  This module restates, in
float64 numpy, the published algorithm that package computes: the structural
similarity index of Wang, Bovik, Sheikh and Simoncelli (IEEE Trans. Image
Processing 13(4), 2004) with

  * an 11 x 11 Gaussian window of standard deviation 1.5, normalised to sum 1,
    applied separably to every (batch, channel) plane,
  * zero padding at the image border (statistics for every pixel),
  * C1 = 0.01 ** 2 and C2 = 0.03 ** 2 (images in [0, 1]),
  * the mean of the SSIM map over all pixels (padding="same") or over the map
    without its 5-pixel border (padding="valid"),

and its gradient with respect to img1 (img2 gets none):

  gaussian_window   the normalised 11-tap window
  blur              separable zero-padded filtering of every plane
  ssim_terms        local statistics and the SSIM map
  ssim              the mean SSIM
  ssim_backward     d(mean SSIM)/d img1, from the map's partial derivatives with
                    respect to mu1, E[x^2] and E[xy], filtered back

Only tests/ (and __graft_entry__.smoke / bench.py's CPU baseline) use it.
"""

from __future__ import annotations

import numpy as np

RADIUS = 5
SIGMA = 1.5
C1 = 0.01 ** 2
C2 = 0.03 ** 2


def gaussian_window(radius: int = RADIUS, sigma: float = SIGMA) -> np.ndarray:
    """Normalised 1-D Gaussian window of 2 * radius + 1 taps."""
    k = np.arange(-radius, radius + 1, dtype=np.float64)
    w = np.exp(-(k * k) / (2.0 * sigma * sigma))
    return w / w.sum()


def _filter_axis(a: np.ndarray, w: np.ndarray, axis: int) -> np.ndarray:
    """Zero-padded correlation of `a` with the odd-length window `w` along `axis`
    (output has the input's shape)."""
    r = (len(w) - 1) // 2
    a = np.moveaxis(a, axis, -1)
    n = a.shape[-1]
    padded = np.zeros(a.shape[:-1] + (n + 2 * r,), dtype=np.float64)
    padded[..., r:r + n] = a
    out = np.zeros(a.shape, dtype=np.float64)
    for t in range(len(w)):
        out += w[t] * padded[..., t:t + n]
    return np.moveaxis(out, -1, axis)


def blur(a: np.ndarray, w: np.ndarray | None = None) -> np.ndarray:
    """Separable zero-padded Gaussian filter over the last two axes (H, W)."""
    w = gaussian_window() if w is None else w
    return _filter_axis(_filter_axis(np.asarray(a, np.float64), w, -1), w, -2)


def ssim_terms(img1, img2, c1: float = C1, c2: float = C2):
    """Local statistics of (B, C, H, W) images and the SSIM map.

    Returns a dict with mu1, mu2, sigma1_sq, sigma2_sq, sigma12 and map, all
    (B, C, H, W) float64."""
    x = np.asarray(img1, np.float64)
    y = np.asarray(img2, np.float64)
    mu1, mu2 = blur(x), blur(y)
    s11 = blur(x * x) - mu1 * mu1
    s22 = blur(y * y) - mu2 * mu2
    s12 = blur(x * y) - mu1 * mu2
    num = (2.0 * mu1 * mu2 + c1) * (2.0 * s12 + c2)
    den = (mu1 * mu1 + mu2 * mu2 + c1) * (s11 + s22 + c2)
    return dict(mu1=mu1, mu2=mu2, sigma1_sq=s11, sigma2_sq=s22, sigma12=s12, map=num / den)


def region_mask(height: int, width: int, padding: str) -> np.ndarray:
    """Pixels the mean runs over: all ("same") or all but a RADIUS border ("valid")."""
    if padding not in ("same", "valid"):
        raise ValueError(f"padding must be 'same' or 'valid', got {padding!r}")
    m = np.zeros((height, width), dtype=bool)
    if padding == "same":
        m[:, :] = True
    elif height > 2 * RADIUS and width > 2 * RADIUS:
        m[RADIUS:height - RADIUS, RADIUS:width - RADIUS] = True
    return m


def ssim(img1, img2, padding: str = "same") -> float:
    """Mean SSIM of (B, C, H, W) images (nan when the region is empty)."""
    t = ssim_terms(img1, img2)
    m = region_mask(t["map"].shape[-2], t["map"].shape[-1], padding)
    sel = t["map"][..., m]
    return float(sel.mean()) if sel.size else float("nan")


def ssim_backward(img1, img2, padding: str = "same", grad_out: float = 1.0) -> np.ndarray:
    """grad_out * d(mean SSIM)/d img1, (B, C, H, W) float64.

    With A = mu1^2 + mu2^2 + C1, B = sigma1^2 + sigma2^2 + C2, C = 2 mu1 mu2 + C1
    and D = 2 sigma12 + C2 the map is S = C D / (A B).  Taking mu1 = E[x],
    E[x^2] and E[xy] as the independent local statistics (sigma1^2 = E[x^2] -
    mu1^2, sigma12 = E[xy] - mu1 mu2):
        dS/dE[x]   = 2 mu2 (D - C) / (A B) + 2 mu1 S (1/B - 1/A)
        dS/dE[x^2] = -S / B
        dS/dE[xy]  = 2 C / (A B)
    and every statistic is a window sum w(q - p) over pixels p, so
        d/dx_p = sum_q w(q - p) g_q [dS/dE[x] + 2 x_p dS/dE[x^2] + y_p dS/dE[xy]]_q
    with g_q = grad_out / (pixels in the region) inside the region, else 0.  The
    window is symmetric, so the back-filter is the same zero-padded blur."""
    x = np.asarray(img1, np.float64)
    y = np.asarray(img2, np.float64)
    t = ssim_terms(x, y)
    mu1, mu2 = t["mu1"], t["mu2"]
    A = mu1 * mu1 + mu2 * mu2 + C1
    B = t["sigma1_sq"] + t["sigma2_sq"] + C2
    C = 2.0 * mu1 * mu2 + C1
    D = 2.0 * t["sigma12"] + C2
    S = t["map"]
    d_mu = 2.0 * mu2 * (D - C) / (A * B) + 2.0 * mu1 * S * (1.0 / B - 1.0 / A)
    d_xx = -S / B
    d_xy = 2.0 * C / (A * B)
    m = region_mask(x.shape[-2], x.shape[-1], padding)
    count = int(m.sum()) * int(np.prod(x.shape[:-2]))
    g = np.where(m, grad_out / count, 0.0) if count else np.zeros(m.shape)
    return blur(g * d_mu) + 2.0 * x * blur(g * d_xx) + y * blur(g * d_xy)
