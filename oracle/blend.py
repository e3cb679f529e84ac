"""Oracle blending: per-tile vectorised compositing and a brute-force pixel loop.

Test infrastructure only (see oracle/__init__.py).

`rasterize` restates the Torch rasterizer's tile loop
(src/torch_rasterizer.py:228-284): for each non-empty tile, (G, h, w) tensors of
exponents, alphas and a cumprod transmittance; gradients come from autograd.
Inclusion rules: E < chi, alpha >= alpha_threshold, transmittance before the
Gaussian >= transmittance_threshold, transmittance factor 1 - alpha + 1e-10.

`rasterize_bruteforce` restates the reference test's per-pixel oracle
(scripts/check_cuda_gradients.py:134-193) with the same inclusion rules (the
test itself skips E > chi, keeping E == chi, and omits the 1e-10; the Torch
rasterizer, this repository's reference semantics, keeps E < chi).
"""

from __future__ import annotations

import torch

TRANSMITTANCE_EPS = 1e-10  # src/torch_rasterizer.py:271


def rasterize(indexing_offset, gaussian_ids_sorted, points_image, cov_inv_image, opacities,
              colors, width, height, tile_size, alpha_threshold, transmittance_threshold,
              chi_squared_threshold, tiles=None):
    """Differentiable in points_image, cov_inv_image, opacities, colors.

    indexing_offset / gaussian_ids_sorted as produced by compute_tile_intersection.
    `tiles` optionally restricts the loop to a subset of tile ids (timing samples).
    Returns the un-clamped (H, W, 3) image.
    """
    device = points_image.device
    n_tiles = int(indexing_offset.shape[0])
    k = int(gaussian_ids_sorted.shape[0])
    tiles_x = (width + tile_size - 1) // tile_size
    off = indexing_offset.tolist()
    ids = gaussian_ids_sorted.long()
    image = torch.zeros((height, width, 3), dtype=torch.float32, device=device)
    tile_iter = range(n_tiles) if tiles is None else tiles
    for t in tile_iter:
        start = off[t]
        end = off[t + 1] if t + 1 < n_tiles else k
        if end <= start:
            continue
        tu, tv = t % tiles_x, t // tiles_x
        u0, v0 = tu * tile_size, tv * tile_size
        u1, v1 = min(u0 + tile_size, width), min(v0 + tile_size, height)
        if u1 <= u0 or v1 <= v0:
            continue
        g = ids[start:end]
        gs_u = points_image[g, 0]
        gs_v = points_image[g, 1]
        A = cov_inv_image[g, 0].view(-1, 1, 1)
        B = cov_inv_image[g, 1].view(-1, 1, 1)
        C = cov_inv_image[g, 2].view(-1, 1, 1)
        o = opacities[g].view(-1, 1, 1)
        col = colors[g]
        su, sv = u1 - u0, v1 - v0
        pu, pv = torch.meshgrid(torch.arange(u0, u1, device=device),
                                torch.arange(v0, v1, device=device), indexing="xy")
        du = pu.view(-1, sv, su) - gs_u.view(-1, 1, 1)
        dv = pv.view(-1, sv, su) - gs_v.view(-1, 1, 1)
        exponent = A * du * du + (B + B) * du * dv + C * dv * dv
        chi_mask = (exponent < chi_squared_threshold).float()
        density = torch.exp(-0.5 * exponent) * chi_mask
        alpha = density * o
        alpha = torch.where(alpha < alpha_threshold, torch.zeros_like(alpha), alpha)
        one_minus_alpha = 1 - alpha + TRANSMITTANCE_EPS
        transmittance = torch.ones_like(one_minus_alpha)
        transmittance[1:] = torch.cumprod(one_minus_alpha[:-1], dim=0)
        transmittance = torch.where(transmittance < transmittance_threshold,
                                    torch.zeros_like(transmittance), transmittance)
        contribution = ((transmittance * alpha).unsqueeze(-1) * col.view(-1, 1, 1, 3)).sum(dim=0)
        image[v0:v1, u0:u1, :] = contribution
    return image


def rasterize_bruteforce(indexing_offset, gaussian_ids_sorted, points_image, cov_inv_image,
                         opacities, colors, width, height, tile_size, alpha_threshold,
                         transmittance_threshold, chi_squared_threshold):
    """Per-pixel loop (scripts/check_cuda_gradients.py:134-193), differentiable.
    Small inputs only."""
    n_tiles = int(indexing_offset.shape[0])
    k = int(gaussian_ids_sorted.shape[0])
    tiles_x = (width + tile_size - 1) // tile_size
    out = torch.zeros((height, width, 3), dtype=points_image.dtype)
    for t in range(n_tiles):
        row, col = t // tiles_x, t % tiles_x
        start = int(indexing_offset[t])
        end = int(indexing_offset[t + 1]) if t + 1 < n_tiles else k
        for p in range(tile_size * tile_size):
            u = col * tile_size + p % tile_size
            v = row * tile_size + p // tile_size
            if u >= width or v >= height:
                continue
            T = torch.tensor(1.0)
            pix = torch.zeros(3)
            if not (1.0 >= transmittance_threshold):
                continue
            for i in range(start, end):
                g = int(gaussian_ids_sorted[i])
                du = u - points_image[g, 0]
                dv = v - points_image[g, 1]
                B = cov_inv_image[g, 1]
                E = cov_inv_image[g, 0] * du * du + (B + B) * du * dv + cov_inv_image[g, 2] * dv * dv
                if not (E.item() < chi_squared_threshold):
                    continue
                alpha = torch.exp(-0.5 * E) * opacities[g]
                if alpha.item() < alpha_threshold:
                    continue
                pix = pix + (alpha * T) * colors[g]
                T = T * (1.0 - alpha + TRANSMITTANCE_EPS)
                if T.item() < transmittance_threshold:
                    break
            out[v, u] = pix
    return out
