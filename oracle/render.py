"""Oracle render: the reference's pure-Torch rasterizer pipeline on the CPU.

Test infrastructure only (see oracle/__init__.py).

Restates src/torch_rasterizer.py:9-290: project and cull, SH colours, global
depth order, tile expansion with keys tile*(L+1)+rank, per-tile vectorised
compositing, clamp(0,1)*255.  Gradients come from autograd.  Two deliberate
differences, both explained in oracle/preprocess.py and below:
- the projection is element-wise in the GPU kernel's operation order (bit-exact
  u, v, covariance, conic) instead of batched matmuls;
- the global depth order is a stable sort of the fp32 depth bit patterns
  (ties by Gaussian index), which is the order the reference's CUDA binning
  defines (src/cuda/kernel.cu:857-868 with a stable sort) and which
  argsort(z) (src/torch_rasterizer.py:147) leaves unspecified for ties.
"""

from __future__ import annotations

import numpy as np
import torch

from . import blend, preprocess


def render_stages(world_to_camera, intrinsic, width, height, means, scales, quaternions,
                  opacities, sh_coeffs_dc, sh_coeffs_rest, near_plane=0.01, far_plane=100.0,
                  min_opacity=1 / 255, min_radius=0.5, max_radius=128.0, alpha_threshold=1e-4,
                  transmittance_threshold=1e-4, chi_squared_threshold=9.21, sh_sigmoid=False,
                  tile_size=16, tiles=None):
    """Full pipeline, returning a dict with the image and every intermediate.

    Keys: image (clamped*255), raw_image (un-clamped), proj (see
    preprocess.project), colors (N,3 for visible rows, 0 elsewhere), points_image,
    conic, indexing_offset, gaussian_ids_sorted (indices into the N Gaussians).
    """
    N = means.shape[0]
    proj = preprocess.project(means, scales, quaternions, opacities, world_to_camera,
                              intrinsic, width, height, near_plane, far_plane, min_opacity,
                              min_radius, max_radius)
    keep = proj["keep"]

    # SH colours along the view direction (src/torch_rasterizer.py:59-65)
    cam_pos = preprocess.camera_position(world_to_camera.to(torch.float32))
    dirs = preprocess.view_directions(means, cam_pos)
    colors_all = preprocess.evaluate_spherical_harmonics(sh_coeffs_dc, sh_coeffs_rest, dirs,
                                                         sh_sigmoid)
    zeros3 = torch.zeros_like(colors_all)
    colors = torch.where(keep.unsqueeze(1), colors_all, zeros3)

    points_image = torch.stack([proj["u"], proj["v"]], dim=1)
    conic = torch.stack([proj["A"], proj["B"], proj["C"]], dim=1)
    radii = torch.stack([proj["ru"], proj["rv"]], dim=1)
    keep_np = keep.numpy()
    vis = np.nonzero(keep_np)[0]
    L = len(vis)
    n_tiles = ((width + tile_size - 1) // tile_size) * ((height + tile_size - 1) // tile_size)
    if L == 0:
        raw = torch.zeros((height, width, 3), dtype=torch.float32)
        return dict(image=raw * 255, raw_image=raw, proj=proj, colors=colors,
                    points_image=points_image, conic=conic, radii=radii,
                    indexing_offset=torch.zeros(n_tiles, dtype=torch.int32),
                    gaussian_ids_sorted=torch.zeros(0, dtype=torch.int32))

    # global depth order (src/torch_rasterizer.py:146-152), stable on the depth bits
    z_bits = proj["zc"].detach().numpy().astype(np.float32)[vis].view(np.uint32)
    order = vis[np.argsort(z_bits, kind="stable")]

    # tile expansion (src/torch_rasterizer.py:154-211)
    pts_np = points_image.detach().numpy()[order]
    rad_np = radii.detach().numpy()[order]
    tx0, tx1, ty0, ty1, _ = _rects(pts_np, rad_np, width, height, tile_size)
    tiles_x = (width + tile_size - 1) // tile_size
    counts = (tx1 - tx0 + 1) * (ty1 - ty0 + 1)
    rank = np.repeat(np.arange(L, dtype=np.int64), counts)
    starts = np.cumsum(counts) - counts
    local = np.arange(int(counts.sum()), dtype=np.int64) - np.repeat(starts, counts)
    nx = (tx1 - tx0 + 1)[rank]
    tile_ids = (ty0[rank] + local // nx) * tiles_x + (tx0[rank] + local % nx)
    scaled = tile_ids * (L + 1) + rank
    perm = np.argsort(scaled, kind="stable")
    sorted_tiles = scaled[perm] // (L + 1)
    ids_sorted = order[rank[perm]]
    offsets = np.searchsorted(sorted_tiles, np.arange(n_tiles), side="left")

    indexing_offset = torch.from_numpy(offsets.astype(np.int32))
    gaussian_ids_sorted = torch.from_numpy(ids_sorted.astype(np.int32))
    opac_vis = torch.where(keep, opacities, torch.zeros_like(opacities))
    raw = blend.rasterize(indexing_offset, gaussian_ids_sorted, points_image, conic, opac_vis,
                          colors, width, height, tile_size, alpha_threshold,
                          transmittance_threshold, chi_squared_threshold, tiles=tiles)
    return dict(image=raw.clamp(0, 1) * 255, raw_image=raw, proj=proj, colors=colors,
                points_image=points_image, conic=conic, radii=radii,
                indexing_offset=indexing_offset, gaussian_ids_sorted=gaussian_ids_sorted)


def _rects(pts, rad, width, height, tile_size):
    from .binning import tile_rects

    return tile_rects(pts, rad, width, height, tile_size)


def render(world_to_camera, intrinsic, width, height, means, scales, quaternions, opacities,
           sh_coeffs_dc, sh_coeffs_rest, near_plane=0.01, far_plane=100.0,
           min_opacity=1 / 255, min_radius=0.5, max_radius=128.0, alpha_threshold=1e-4,
           transmittance_threshold=1e-4, chi_squared_threshold=9.21, device="cpu",
           sh_sigmoid=False):
    """Same signature and returns as src/torch_rasterizer.py:9-30,286-290:
    (image*255 clamped, None, None).  Runs on the CPU."""
    if device not in ("cpu", torch.device("cpu")):
        raise ValueError("the oracle runs on the CPU only")
    out = render_stages(world_to_camera, intrinsic, width, height, means, scales, quaternions,
                        opacities, sh_coeffs_dc, sh_coeffs_rest, near_plane, far_plane,
                        min_opacity, min_radius, max_radius, alpha_threshold,
                        transmittance_threshold, chi_squared_threshold, sh_sigmoid)
    return out["image"], None, None
