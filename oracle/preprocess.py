"""Oracle preprocess: projection and spherical harmonics (CPU, PyTorch).

Test infrastructure only (see oracle/__init__.py).

The projection restates src/torch_rasterizer.py:41-144 (camera transform,
depth cull, u/v, EWA covariance with the frustum-clamped Jacobian, low-pass
filter, symmetrisation, finite / radius / image-bound culls) and the conic of
src/torch_rasterizer.py:213-226.  It is written element-wise, one rounded fp32
operation at a time, in the same order as the GPU kernel
(3dgs_from_scratch_amd/csrc/preprocess_math.h), instead of the reference's
batched matmuls, so that u, v, the covariance and the conic are bit-identical
to the kernel's for identical inputs.  The mathematics is the reference's:
Sigma_2D = J W Sigma_w W^T J^T computed as T Sigma_w T^T with T = J W.
"""

from __future__ import annotations

import torch

# src/torch_rasterizer.py:5-6
LOW_PASS_FILTER = 0.3
FRUSTUM_CLAMP_FACTOR = 1.3
SIGMA_EXTENT = 3.0  # src/torch_rasterizer.py:118

# src/gaussian.py:6-21
SH_C0 = 0.28209479177387814
SH_C1 = 0.4886025119029199
SH_C2_xy = 1.0925484305920792
SH_C2_zz = 0.31539156525252005
SH_C2_xx_yy = 0.5462742152960396
SH_C3_yxx_yyy = 0.5900435899266435
SH_C3_xyz = 2.890611442640554
SH_C3_yzz = 0.4570457994644658
SH_C3_zzz = 0.3731763325901154
SH_C3_xzz = 0.4570457994644658
SH_C3_zxx_zyy = 1.445305721320277
SH_C3_xxx_xyy = 0.5900435899266435

F32 = torch.float32


def _s(x) -> torch.Tensor:
    """fp32 0-d tensor."""
    return torch.as_tensor(x, dtype=F32)


def quaternion_to_rotation_matrix(q: torch.Tensor) -> torch.Tensor:
    """(N,4) xyzw -> (N,3,3).  src/gaussian.py:64-79."""
    x, y, z, w = q.unbind(dim=1)
    rows = quat_rows(x, y, z, w)
    return torch.stack(rows, dim=1).reshape(-1, 3, 3)


def quat_rows(x, y, z, w):
    """The nine entries of R(q), row-major (src/gaussian.py:69-77)."""
    return [
        1.0 - 2.0 * (y * y + z * z),
        2.0 * (x * y - z * w),
        2.0 * (x * z + y * w),
        2.0 * (x * y + z * w),
        1.0 - 2.0 * (x * x + z * z),
        2.0 * (y * z - x * w),
        2.0 * (x * z - y * w),
        2.0 * (y * z + x * w),
        1.0 - 2.0 * (x * x + y * y),
    ]


def sh_basis_rest(dirs: torch.Tensor) -> torch.Tensor:
    """(N,3) unit directions -> (N,15) basis of degrees 1..3.  src/gaussian.py:29-52."""
    x, y, z = dirs.unbind(dim=1)
    xx, yy, zz = x * x, y * y, z * z
    xy, xz, yz = x * y, x * z, y * z
    return torch.stack(
        [
            -SH_C1 * y,
            SH_C1 * z,
            -SH_C1 * x,
            SH_C2_xy * xy,
            SH_C2_xy * yz,
            SH_C2_zz * (3 * zz - 1),
            SH_C2_xy * xz,
            SH_C2_xx_yy * (xx - yy),
            SH_C3_yxx_yyy * y * (xx - yy),
            SH_C3_xyz * (x * y * z),
            SH_C3_yzz * y * (4 * zz - xx - yy),
            SH_C3_zzz * z * (2 * zz - 3 * xx - 3 * yy),
            SH_C3_xzz * x * (4 * zz - xx - yy),
            SH_C3_zxx_zyy * z * (xx - yy),
            SH_C3_xxx_xyy * x * (xx - 3 * yy),
        ],
        dim=1,
    )


def sh_raw(sh_dc: torch.Tensor, sh_rest: torch.Tensor, dirs: torch.Tensor) -> torch.Tensor:
    """C0*dc + sum_k basis_k * rest_k (before the shift/sigmoid).  src/gaussian.py:54-56."""
    return sh_dc * SH_C0 + (sh_rest * sh_basis_rest(dirs).unsqueeze(-1)).sum(dim=1)


def evaluate_spherical_harmonics(sh_dc, sh_rest, dirs, sh_sigmoid=False):
    """src/gaussian.py:24-61: sigmoid(sh) or max(sh + 0.5, 0)."""
    sh = sh_raw(sh_dc, sh_rest, dirs)
    if sh_sigmoid:
        return torch.sigmoid(sh)
    return torch.clamp_min(sh + 0.5, 0.0)


def view_directions(means: torch.Tensor, camera_pos: torch.Tensor) -> torch.Tensor:
    """normalize(mean - camera_pos).  src/torch_rasterizer.py:60-62."""
    d = means - camera_pos.unsqueeze(0)
    return d / torch.norm(d, dim=1, keepdim=True)


def sqrt_rn(x: torch.Tensor) -> torch.Tensor:
    """IEEE correctly rounded fp32 square root (torch's CPU float32 sqrt goes
    through MKL VML and is not correctly rounded for large tensors; the float64
    root rounded once to float32 is, since 53 >= 2*24 + 2)."""
    return torch.sqrt(x.double()).float()


def camera_position(world_to_camera: torch.Tensor) -> torch.Tensor:
    """-R^T t.  src/torch_rasterizer.py:60, src/cuda/wrapper.py:260."""
    return -world_to_camera[:3, :3].t() @ world_to_camera[:3, 3]


class Camera:
    """fp32 scalars of a pinhole camera (world_to_camera rows 0..2, fx, fy, cx, cy)."""

    def __init__(self, world_to_camera: torch.Tensor, intrinsic: torch.Tensor, width: int,
                 height: int):
        W = world_to_camera.detach().to(F32).cpu()
        K = intrinsic.detach().to(F32).cpu()
        self.w = [W[i // 4, i % 4].clone() for i in range(12)]
        self.fx, self.cx, self.fy, self.cy = K[0, 0], K[0, 2], K[1, 1], K[1, 2]
        # src/torch_rasterizer.py:87-88
        self.lim_x = (_s(FRUSTUM_CLAMP_FACTOR) * torch.maximum(self.cx, _s(float(width)) - self.cx)) / self.fx
        self.lim_y = (_s(FRUSTUM_CLAMP_FACTOR) * torch.maximum(self.cy, _s(float(height)) - self.cy)) / self.fy


def project(means, scales, quaternions, opacities, world_to_camera, intrinsic, width, height,
            near_plane=0.01, far_plane=100.0, min_opacity=1 / 255, min_radius=0.5,
            max_radius=128.0):
    """Projection of every Gaussian.  Differentiable in means, scales, quaternions.

    Returns a dict of (N,) tensors: xc, yc, zc, u, v, a, b, c (2D covariance incl.
    low-pass), A, B, C (conic), ru, rv (3-sigma radii), and boolean masks
    pre (passed opacity and depth culls: covariance computed) and keep (visible).
    src/torch_rasterizer.py:41-144 and :213-226.
    """
    cam = Camera(world_to_camera, intrinsic, width, height)
    w = cam.w
    px, py, pz = means.unbind(1)
    xc = w[0] * px + w[1] * py + w[2] * pz + w[3]
    yc = w[4] * px + w[5] * py + w[6] * pz + w[7]
    zc = w[8] * px + w[9] * py + w[10] * pz + w[11]
    with torch.no_grad():
        pre = (opacities >= min_opacity) & (zc > near_plane) & (zc < far_plane)

    u = (cam.fx * xc) / zc + cam.cx
    v = (cam.fy * yc) / zc + cam.cy

    qx, qy, qz, qw = quaternions.unbind(1)
    R = quat_rows(qx, qy, qz, qw)
    sx, sy, sz = scales.unbind(1)
    m = [R[0] * sx, R[1] * sy, R[2] * sz,
         R[3] * sx, R[4] * sy, R[5] * sz,
         R[6] * sx, R[7] * sy, R[8] * sz]

    def dot_rows(i, j):
        return m[3 * i] * m[3 * j] + m[3 * i + 1] * m[3 * j + 1] + m[3 * i + 2] * m[3 * j + 2]

    s00, s01, s02 = dot_rows(0, 0), dot_rows(0, 1), dot_rows(0, 2)
    s11, s12, s22 = dot_rows(1, 1), dot_rows(1, 2), dot_rows(2, 2)

    invz = 1.0 / zc
    xn = xc * invz
    yn = yc * invz
    # src/torch_rasterizer.py:91-94: the clamped value is a constant for autograd
    x_free = torch.abs(xn) <= cam.lim_x
    y_free = torch.abs(yn) <= cam.lim_y
    xcl = torch.where(x_free, xn, xn.clamp(min=-cam.lim_x, max=cam.lim_x).detach())
    ycl = torch.where(y_free, yn, yn.clamp(min=-cam.lim_y, max=cam.lim_y).detach())
    j00 = cam.fx * invz
    j02 = (-cam.fx * xcl) * invz
    j11 = cam.fy * invz
    j12 = (-cam.fy * ycl) * invz

    t00 = j00 * w[0] + j02 * w[8]
    t01 = j00 * w[1] + j02 * w[9]
    t02 = j00 * w[2] + j02 * w[10]
    t10 = j11 * w[4] + j12 * w[8]
    t11 = j11 * w[5] + j12 * w[9]
    t12 = j11 * w[6] + j12 * w[10]
    q00 = t00 * s00 + t01 * s01 + t02 * s02
    q01 = t00 * s01 + t01 * s11 + t02 * s12
    q02 = t00 * s02 + t01 * s12 + t02 * s22
    q10 = t10 * s00 + t11 * s01 + t12 * s02
    q11 = t10 * s01 + t11 * s11 + t12 * s12
    q12 = t10 * s02 + t11 * s12 + t12 * s22
    a = (q00 * t00 + q01 * t01 + q02 * t02) + LOW_PASS_FILTER
    b = q00 * t10 + q01 * t11 + q02 * t12
    c = (q10 * t10 + q11 * t11 + q12 * t12) + LOW_PASS_FILTER

    det = a * c - b * b
    inv_det = 1.0 / torch.clamp_min(det, 1e-12)
    A = c * inv_det
    B = -b * inv_det
    C = a * inv_det
    ru = sqrt_rn(torch.clamp_min(a, 1e-12)) * SIGMA_EXTENT
    rv = sqrt_rn(torch.clamp_min(c, 1e-12)) * SIGMA_EXTENT
    with torch.no_grad():
        r = torch.maximum(ru, rv)
        finite = torch.isfinite(a) & torch.isfinite(b) & torch.isfinite(c)
        keep = (pre & finite & torch.isfinite(ru) & torch.isfinite(rv) & (r >= min_radius)
                & (r <= max_radius) & (u > -ru) & (u < width + ru) & (v > -rv)
                & (v < height + rv))
    return dict(xc=xc, yc=yc, zc=zc, u=u, v=v, a=a, b=b, c=c, A=A, B=B, C=C, ru=ru, rv=rv,
                pre=pre, keep=keep)


def project_points(means, scales, quaternions, opacities, world_to_camera, intrinsic,
                   near_plane, far_plane, min_opacity, min_radius, max_radius, width, height):
    """The seven-function API's project_points (src/cuda/rasterizer.cpp:140-191) with the
    Torch rasterizer's culls: (points_image, depths, cov_image, cov_inv_image, radii, mask),
    zero where culled (cov_image kept for Gaussians culled after it was computed)."""
    p = project(means, scales, quaternions, opacities, world_to_camera, intrinsic, width,
                height, near_plane, far_plane, min_opacity, min_radius, max_radius)
    keep = p["keep"]
    pre = p["pre"]
    z = torch.zeros_like(p["u"])

    def sel(m, x):
        return torch.where(m, x, z)

    points_image = torch.stack([sel(keep, p["u"]), sel(keep, p["v"])], dim=1)
    depths = sel(keep, p["zc"])
    cov_image = torch.stack([sel(pre, p["a"]), sel(pre, p["b"]), sel(pre, p["c"])], dim=1)
    cov_inv = torch.stack([sel(keep, p["A"]), sel(keep, p["B"]), sel(keep, p["C"])], dim=1)
    radii = torch.stack([sel(keep, p["ru"]), sel(keep, p["rv"])], dim=1)
    return points_image, depths, cov_image, cov_inv, radii, keep.clone()


def evaluate_sh_api(camera_pos, means, sh_dc, sh_rest, mask, sh_sigmoid=False):
    """The API's evaluate_spherical_harmonics (src/cuda/rasterizer.cpp:234-257): raw SH sum
    (or its sigmoid) with masked rows 0; the caller applies max(c + 0.5, 0)."""
    dirs = view_directions(means, camera_pos)
    sh = sh_raw(sh_dc, sh_rest, dirs)
    if sh_sigmoid:
        sh = torch.sigmoid(sh)
    return torch.where(mask.unsqueeze(1), sh, torch.zeros_like(sh))
