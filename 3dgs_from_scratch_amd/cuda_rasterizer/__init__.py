"""`cuda_rasterizer` -- drop-in for the reference extension module of the same name.

The reference builds a pybind11 module with seven functions
(src/cuda/rasterizer.cpp:442-464) that src/cuda/wrapper.py imports.  This
package exposes the same seven functions with the same positional signatures,
tensor layouts and return tuples, implemented by hand-written gfx950 HIP
kernels behind a C ABI (libgsraster.so, include/gs_rasterizer.h).  Outputs are
allocated with PyTorch on the first input's device; kernels run on the current
HIP stream of that device.

Behavioural notes relative to the reference:
- Culling and blending inclusion follow the reference's Torch rasterizer
  (src/torch_rasterizer.py), the repository's correctness oracle: strict
  near/far and image-bound tests, non-finite covariances culled,
  E < chi_squared_threshold.
- project_points_backward returns the exact derivative (the reference kernel
  doubles the Jacobian off-diagonal term, src/cuda/kernel.cu:384-394).
- Inputs are made contiguous; wrong dtype, device or shape raises RuntimeError
  (the reference raises only on dtype).
- rasterize_backward accepts an optional `rendered_image` (the forward output)
  to skip recomputing each pixel's colour.
"""

from __future__ import annotations

import ctypes
import threading
import time

import torch

from . import _lib
from ._lib import RasterizerError
from .ssim import fused_ssim

__all__ = [
    "project_points",
    "project_points_backward",
    "evaluate_spherical_harmonics",
    "evaluate_spherical_harmonics_backward",
    "compute_tile_intersection",
    "compute_tile_intersection_debug",
    "compute_tile_intersection_ordered",
    "tile_intersection_capped",
    "CappedCheck",
    "CapturedChecks",
    "rasterize",
    "rasterize_backward",
    "rasterize_work",
    "evaluate_spherical_harmonics_render",
    "sh_cache_empty",
    "evaluate_spherical_harmonics_render_backward",
    "rasterize_display",
    "rasterize_display_backward",
    "activate",
    "activate_backward",
    "preprocess_forward",
    "preprocess_backward",
    "render_preprocess_backward",
    "rasterize_display_l1",
    "rasterize_l1_backward",
    "blend_grad_accumulators",
    "tile_schedule",
    "schedule_size",
    "set_blend_waves",
    "check_forward_order",
    "fused_ssim",
    "RasterizerError",
]


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _prep(t: torch.Tensor, name: str, dtype: torch.dtype, shape: tuple, device) -> torch.Tensor:
    if not isinstance(t, torch.Tensor):
        raise RuntimeError(f"{name}: expected a torch.Tensor, got {type(t).__name__}")
    if t.dtype != dtype:
        raise RuntimeError(f"{name}: expected dtype {dtype}, got {t.dtype}")
    if device is not None and t.device != device:
        raise RuntimeError(f"{name}: expected device {device}, got {t.device}")
    if tuple(t.shape) != tuple(shape):
        raise RuntimeError(f"{name}: expected shape {tuple(shape)}, got {tuple(t.shape)}")
    return t.contiguous()


def _device_of(t: torch.Tensor) -> torch.device:
    if not isinstance(t, torch.Tensor):
        raise RuntimeError(f"expected a torch.Tensor, got {type(t).__name__}")
    if t.device.type != "cuda":
        raise RuntimeError(
            f"cuda_rasterizer runs on the GPU only; got a tensor on {t.device} "
            "(there is no CPU fallback)"
        )
    return t.device


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def project_points(
    points_world,
    scales,
    quaternions,
    opacities,
    world_to_camera,
    intrinsic,
    near_plane,
    far_plane,
    min_opacity,
    min_radius,
    max_radius,
    width,
    height,
):
    """Reference: src/cuda/rasterizer.cpp:140-191.

    Returns (points_image[N,2], depths[N], cov_image[N,3], cov_inv_image[N,3],
    radii[N,2] float32, mask[N] bool).
    """
    dev = _device_of(points_world)
    n = points_world.shape[0]
    f32 = torch.float32
    points_world = _prep(points_world, "points_world", f32, (n, 3), dev)
    scales = _prep(scales, "scales", f32, (n, 3), dev)
    quaternions = _prep(quaternions, "quaternions", f32, (n, 4), dev)
    opacities = _prep(opacities, "opacities", f32, (n,), dev)
    world_to_camera = _prep(world_to_camera, "world_to_camera", f32, (4, 4), dev)
    intrinsic = _prep(intrinsic, "intrinsic", f32, (3, 3), dev)
    points_image = torch.empty((n, 2), dtype=f32, device=dev)
    depths = torch.empty((n,), dtype=f32, device=dev)
    cov_image = torch.empty((n, 3), dtype=f32, device=dev)
    cov_inv_image = torch.empty((n, 3), dtype=f32, device=dev)
    radii = torch.empty((n, 2), dtype=f32, device=dev)
    mask = torch.empty((n,), dtype=torch.bool, device=dev)
    with torch.cuda.device(dev):
        ev = _lib.timer.record("project_points", dev)
        _lib.check(
            _lib.load().gs_project_points(
                _ptr(points_world), _ptr(scales), _ptr(quaternions), _ptr(opacities),
                _ptr(world_to_camera), _ptr(intrinsic), n, float(near_plane), float(far_plane),
                float(min_opacity), float(min_radius), float(max_radius), int(width), int(height),
                _ptr(points_image), _ptr(depths), _ptr(cov_image), _ptr(cov_inv_image),
                _ptr(radii), _ptr(mask), _stream(dev),
            ),
            "project_points",
        )
        _lib.timer.stop(ev, dev)
    return points_image, depths, cov_image, cov_inv_image, radii, mask


def project_points_backward(
    grad_points_image,
    grad_cov_inv_image,
    points_world,
    scales,
    quaternions,
    opacities,
    world_to_camera,
    intrinsic,
    width,
    height,
    cov_image,
    mask,
):
    """Reference: src/cuda/rasterizer.cpp:193-232.

    Returns (grad_points_world[N,3], grad_scales[N,3], grad_quaternions[N,4]).
    """
    dev = _device_of(points_world)
    n = points_world.shape[0]
    f32 = torch.float32
    grad_points_image = _prep(grad_points_image, "grad_points_image", f32, (n, 2), dev)
    grad_cov_inv_image = _prep(grad_cov_inv_image, "grad_cov_inv_image", f32, (n, 3), dev)
    points_world = _prep(points_world, "points_world", f32, (n, 3), dev)
    scales = _prep(scales, "scales", f32, (n, 3), dev)
    quaternions = _prep(quaternions, "quaternions", f32, (n, 4), dev)
    opacities = _prep(opacities, "opacities", f32, (n,), dev)
    world_to_camera = _prep(world_to_camera, "world_to_camera", f32, (4, 4), dev)
    intrinsic = _prep(intrinsic, "intrinsic", f32, (3, 3), dev)
    cov_image = _prep(cov_image, "cov_image", f32, (n, 3), dev)
    mask = _prep(mask, "mask", torch.bool, (n,), dev)
    g_means = torch.empty((n, 3), dtype=f32, device=dev)
    g_scales = torch.empty((n, 3), dtype=f32, device=dev)
    g_quats = torch.empty((n, 4), dtype=f32, device=dev)
    with torch.cuda.device(dev):
        ev = _lib.timer.record("project_points_backward", dev)
        _lib.check(
            _lib.load().gs_project_points_backward(
                _ptr(grad_points_image), _ptr(grad_cov_inv_image), _ptr(points_world),
                _ptr(scales), _ptr(quaternions), _ptr(opacities), _ptr(world_to_camera),
                _ptr(intrinsic), n, int(width), int(height), _ptr(cov_image), _ptr(mask),
                _ptr(g_means), _ptr(g_scales), _ptr(g_quats), _stream(dev),
            ),
            "project_points_backward",
        )
        _lib.timer.stop(ev, dev)
    return g_means, g_scales, g_quats


def evaluate_spherical_harmonics(
    camera_pos, points_world, sh_coeffs_dc, sh_coeffs_rest, mask, sh_sigmoid=False
):
    """Reference: src/cuda/rasterizer.cpp:234-257.  Returns colors[N,3] (0 where masked)."""
    dev = _device_of(points_world)
    n = points_world.shape[0]
    f32 = torch.float32
    camera_pos = _prep(camera_pos, "camera_pos", f32, (3,), dev)
    points_world = _prep(points_world, "points_world", f32, (n, 3), dev)
    sh_coeffs_dc = _prep(sh_coeffs_dc, "sh_coeffs_dc", f32, (n, 3), dev)
    sh_coeffs_rest = _prep(sh_coeffs_rest, "sh_coeffs_rest", f32, (n, 15, 3), dev)
    mask = _prep(mask, "mask", torch.bool, (n,), dev)
    colors = torch.empty((n, 3), dtype=f32, device=dev)
    with torch.cuda.device(dev):
        ev = _lib.timer.record("evaluate_sh", dev)
        _lib.check(
            _lib.load().gs_evaluate_sh(
                _ptr(camera_pos), _ptr(points_world), _ptr(sh_coeffs_dc), _ptr(sh_coeffs_rest),
                _ptr(mask), n, 1 if sh_sigmoid else 0, _ptr(colors), _stream(dev),
            ),
            "evaluate_spherical_harmonics",
        )
        _lib.timer.stop(ev, dev)
    return colors


def evaluate_spherical_harmonics_backward(
    grad_colors,
    camera_pos,
    points_world,
    sh_coeffs_dc,
    sh_coeffs_rest,
    colors,
    mask,
    sh_sigmoid,
):
    """Reference: src/cuda/rasterizer.cpp:259-290.

    Returns (grad_points_world[N,3], grad_sh_coeffs_dc[N,3], grad_sh_coeffs_rest[N,15,3]).
    """
    dev = _device_of(points_world)
    n = points_world.shape[0]
    f32 = torch.float32
    grad_colors = _prep(grad_colors, "grad_colors", f32, (n, 3), dev)
    camera_pos = _prep(camera_pos, "camera_pos", f32, (3,), dev)
    points_world = _prep(points_world, "points_world", f32, (n, 3), dev)
    sh_coeffs_dc = _prep(sh_coeffs_dc, "sh_coeffs_dc", f32, (n, 3), dev)
    sh_coeffs_rest = _prep(sh_coeffs_rest, "sh_coeffs_rest", f32, (n, 15, 3), dev)
    colors = _prep(colors, "colors", f32, (n, 3), dev)
    mask = _prep(mask, "mask", torch.bool, (n,), dev)
    g_means = torch.empty((n, 3), dtype=f32, device=dev)
    g_dc = torch.empty((n, 3), dtype=f32, device=dev)
    g_rest = torch.empty((n, 15, 3), dtype=f32, device=dev)
    with torch.cuda.device(dev):
        ev = _lib.timer.record("evaluate_sh_backward", dev)
        _lib.check(
            _lib.load().gs_evaluate_sh_backward(
                _ptr(grad_colors), _ptr(camera_pos), _ptr(points_world), _ptr(sh_coeffs_dc),
                _ptr(sh_coeffs_rest), _ptr(colors), _ptr(mask), n, 1 if sh_sigmoid else 0,
                _ptr(g_means), _ptr(g_dc), _ptr(g_rest), _stream(dev),
            ),
            "evaluate_spherical_harmonics_backward",
        )
        _lib.timer.stop(ev, dev)
    return g_means, g_dc, g_rest


def _pinned_device_pointer(t: torch.Tensor):
    """The device address of a pinned host tensor (gs_host_device_pointer), or
    None when the memory is not mapped for the current device."""
    out = ctypes.c_void_p(0)
    if _lib.load().gs_host_device_pointer(_ptr(t), ctypes.byref(out)) != 0 or not out.value:
        return None
    return out.value


# The host waits for K and M by polling the event (hipEventQuery) for up to
# SPIN_WAIT_S seconds, then blocks: the count's second phase runs on the GPU
# meanwhile and the sort is queued behind it, so a wake-up later than that phase
# leaves the GPU idle.
SPIN_WAIT_S = 500e-6


def _wait(event) -> None:
    t_end = time.perf_counter() + SPIN_WAIT_S
    while not event.query():
        if time.perf_counter() > t_end:
            event.synchronize()
            return


# The depth sort's bucket transform is taken from the previous call's least and
# greatest depth key on the same device (gs_bin_count_begin_hinted), widened by
# an eighth of the span on each side: consecutive renders of a scene (training
# steps, camera paths) cover nearly the same depths.  The outputs never depend
# on it; a poor hint only crowds keys into few buckets.  DEPTH_HINTS = False
# derives the transform on the device instead (one more launch).
DEPTH_HINTS = True
_DEPTH_RANGE: dict = {}
_FORCED_DEPTH_HINT = None  # (kmin, shift): tests force a hint


def _depth_hint(dev) -> tuple:
    """(hint_kmin, hint_shift) for gs_bin_count_begin_hinted; shift -1: none."""
    if _FORCED_DEPTH_HINT is not None:
        return _FORCED_DEPTH_HINT
    r = _DEPTH_RANGE.get(dev.index) if DEPTH_HINTS else None
    if r is None or r[0] > r[1]:
        return 0, -1
    lo, hi = r
    span = hi - lo
    lo, hi = max(lo - span // 8, 0), min(hi + span // 8, 0xFFFFFFFE)
    return lo, max((hi - lo).bit_length() - 16, 0)  # 16 bucket bits cover hi - lo


def _tile_intersection(points_image, radii, depths, mask, width, height, tile_size, debug,
                       ordered=False):
    dev = _device_of(points_image)
    n = points_image.shape[0]
    f32 = torch.float32
    points_image = _prep(points_image, "points_image", f32, (n, 2), dev)
    radii = _prep(radii, "radii", f32, (n, 2), dev)
    depths = _prep(depths, "depths", f32, (n,), dev)
    mask = _prep(mask, "mask", torch.bool, (n,), dev)
    width, height, tile_size = int(width), int(height), int(tile_size)
    if tile_size <= 0 or width <= 0 or height <= 0:
        raise RuntimeError("compute_tile_intersection: width, height and tile_size must be > 0")
    n_tiles = ((width + tile_size - 1) // tile_size) * ((height + tile_size - 1) // tile_size)
    if torch.cuda.is_current_stream_capturing():
        raise RuntimeError("compute_tile_intersection: the list sizes are read on the host, "
                           "which a graph capture cannot wait for (render through "
                           "render_l1 or render(), whose capped sort needs no host read)")
    lib = _lib.load()
    with torch.cuda.device(dev):
        stream = _stream(dev)
        sz = ctypes.c_size_t(0)
        _lib.check(lib.gs_bin_count_workspace_size(n, ctypes.byref(sz)), "workspace query")
        ws_count = torch.empty((max(sz.value, 1),), dtype=torch.uint8, device=dev)
        # the one host read (src/cuda/rasterizer.cpp:322): K keys and M supertile
        # entries, final after the first phase and written by the device straight
        # into pinned host memory (no copy); waited for after the second phase is
        # queued, so the GPU keeps working.  Device memory and a copy instead when
        # the pinned memory is not mapped for the device, and for n = 0 (the
        # library then zeroes them with a memset)
        # four totals: K, M and the least and greatest depth key (the next call's hint)
        host_totals = torch.empty((4,), dtype=torch.int64, pin_memory=n > 0)
        totals_ptr = _pinned_device_pointer(host_totals) if n > 0 else None
        totals = None
        if totals_ptr is None:  # device memory and a copy
            totals = torch.empty((4,), dtype=torch.int64, device=dev)
            totals_ptr = _ptr(totals)
        args = (_ptr(points_image), _ptr(radii), _ptr(depths), _ptr(mask), n, width, height,
                tile_size, _ptr(ws_count), sz.value, totals_ptr, stream)
        hint_kmin, hint_shift = _depth_hint(dev)
        # the outputs whose size does not depend on K or M, allocated before the wait
        indexing_offset = torch.empty((n_tiles,), dtype=torch.int32, device=dev)
        tiles_touched = torch.empty((n,), dtype=torch.int32, device=dev) if debug else None
        order = torch.empty((n_tiles,), dtype=torch.int32, device=dev) if ordered else None
        ev = _lib.timer.record("bin_count", dev)
        ready = None
        try:
            _lib.check(lib.gs_bin_count_begin_hinted(*args[:10], hint_kmin, hint_shift,
                                                     *args[10:]),
                       "compute_tile_intersection (count)")
            if totals is not None and n > 0:
                host_totals.copy_(totals, non_blocking=True)
            ready = torch.cuda.Event()
            ready.record(torch.cuda.current_stream(dev))
            _lib.check(lib.gs_bin_count_finish(*args), "compute_tile_intersection (count)")
            _lib.timer.stop(ev, dev)
        finally:
            # the pinned block is the caching host allocator's, which does not know
            # that the device writes it: it is released only once those writes are
            # done, also when a call above raised
            if ready is not None:
                _wait(ready)
            else:
                torch.cuda.current_stream(dev).synchronize()
        k, m, kmin, kmax = (int(v) for v in (host_totals if n > 0 else totals.cpu()).tolist())
        if n > 0:
            _DEPTH_RANGE[dev.index] = (kmin, kmax)
            _set_capacity((dev.index, width, height, tile_size), k, m)
        if k > 2**31 - 1:
            raise RasterizerError(f"compute_tile_intersection: {k} keys exceed the int32 range")
        sz2 = ctypes.c_size_t(0)
        _lib.check(lib.gs_bin_sort_workspace_size(n, k, m, width, height, tile_size,
                                                  ctypes.byref(sz2)), "workspace query")
        ws_sort = torch.empty((max(sz2.value, 1),), dtype=torch.uint8, device=dev)
        gaussian_ids_sorted = torch.empty((k,), dtype=torch.int32, device=dev)
        sorted_keys = torch.empty((k,), dtype=torch.int64, device=dev) if debug else None
        sort_args = (_ptr(points_image), _ptr(radii), _ptr(depths), n, width, height, tile_size,
                     k, m, _ptr(ws_count), _ptr(ws_sort), sz2.value, _ptr(indexing_offset),
                     _ptr(gaussian_ids_sorted), _ptr(sorted_keys), _ptr(tiles_touched))
        ev = _lib.timer.record("bin_sort", dev)
        if ordered:
            _lib.check(lib.gs_bin_sort_ordered(*sort_args, _ptr(order), stream),
                       "compute_tile_intersection (sort)")
        else:
            _lib.check(lib.gs_bin_sort(*sort_args, stream), "compute_tile_intersection (sort)")
        _lib.timer.stop(ev, dev)
    if debug:
        return indexing_offset, gaussian_ids_sorted, sorted_keys, tiles_touched
    if ordered:
        return indexing_offset, gaussian_ids_sorted, order
    return indexing_offset, gaussian_ids_sorted


def compute_tile_intersection(points_image, radii, depths, mask, width, height, tile_size=16):
    """Reference: src/cuda/rasterizer.cpp:292-359.

    Returns (indexing_offset[T] int32, gaussian_ids_sorted[K] int32) with
    T = ceil(W/ts)*ceil(H/ts): entries ordered by (tile, depth bits, Gaussian
    index); indexing_offset[t] = number of entries whose tile is < t.
    """
    return _tile_intersection(points_image, radii, depths, mask, width, height, tile_size, False)


def compute_tile_intersection_ordered(points_image, radii, depths, mask, width, height,
                                      tile_size=16):
    """compute_tile_intersection plus a blend launch order (n_tiles int32) for
    rasterize_display_l1(forward_order=...): in each XCD's tile range, the tiles by
    ascending bit length of their list length, tile order within a bucket
    (gs_bin_sort_ordered).  Returns (indexing_offset, gaussian_ids_sorted, order)."""
    return _tile_intersection(points_image, radii, depths, mask, width, height, tile_size, False,
                              ordered=True)


# Capacities of the capped sort per (device, image and tile size): K and M of
# the last lists binned there, plus a quarter and a constant (a scene's K varies
# from view to view and grows with densification).  Taken from the last call,
# not the largest, so that a smaller scene at the same resolution does not keep
# an oversized sort.  CAPPED_BINNING = False makes tile_intersection_capped bin
# with exact sizes.
CAPPED_BINNING = True
_CAPACITY: dict = {}


def _set_capacity(key, k: int, m: int) -> None:
    _CAPACITY[key] = (k + k // 4 + 4096, m + m // 4 + 1024)


# Checks of capped sorts queued while the calling thread captures a HIP graph:
# CapturedChecks collects them so that the graph's owner can test every replay.
_CAPTURE = threading.local()


class CapturedChecks:
    """Context manager that collects the capped-sort checks queued by the calling
    thread inside it (while it captures a graph): `.checks` afterwards."""

    def __init__(self):
        self.checks = []

    def __enter__(self):
        self._outer = getattr(_CAPTURE, "sink", None)
        _CAPTURE.sink = self.checks
        return self

    def __exit__(self, *exc):
        _CAPTURE.sink = self._outer
        return False


class CappedCheck:
    """The pending check of a capped sort (tile_intersection_capped): ok() waits
    for the sort's launches (after which the count's totals, K, M and the depth
    key range, are final; the GPU has usually run them long before), records
    the totals for the next call's depth hint and capacities, and returns
    whether the lists fit the capacities -- if not, no list was written and the
    caller bins again with exact sizes.  The pinned totals are released only
    after that wait.

    A check queued during a graph capture (no `ready` event; the totals in
    device memory of the graph's pool) cannot wait: ok() returns True and hands
    the check to the enclosing CapturedChecks, and replayed_ok() tells, once a
    replay has completed, whether that replay's lists fit."""

    __slots__ = ("_ready", "_host", "_dev_totals", "_caps", "_key", "_result")

    def __init__(self, ready, host_totals, dev_totals, caps, key):
        self._ready, self._host, self._dev_totals = ready, host_totals, dev_totals
        self._caps, self._key, self._result = caps, key, None

    @property
    def captured(self) -> bool:
        return self._ready is None

    def ok(self) -> bool:
        if self.captured:
            sink = getattr(_CAPTURE, "sink", None)
            if sink is not None and not any(c is self for c in sink):
                sink.append(self)
            return True
        if self._result is None:
            _wait(self._ready)
            src = self._host if self._dev_totals is None else self._dev_totals.cpu()
            self._result = self._record(src)
            self._host = self._dev_totals = None
        return self._result

    def _record(self, src) -> bool:
        k, m, kmin, kmax = (int(v) for v in src.tolist())
        _DEPTH_RANGE[self._key[0]] = (kmin, kmax)
        _set_capacity(self._key, k, m)
        return k <= self._caps[0] and m <= self._caps[1]

    def replayed_ok(self) -> bool:
        """A captured check, after a replay of its graph has completed (the caller
        synchronised): whether that replay's lists fit the capacities fixed at
        capture.  Also records the replay's totals for later eager calls."""
        if not self.captured:
            raise RuntimeError("replayed_ok: the check was not queued during a graph capture")
        return self._record(self._dev_totals.cpu())

    def __del__(self):
        if self._result is None and self._ready is not None:
            self._ready.synchronize()


def tile_intersection_capped(points_image, radii, depths, mask, width, height, tile_size=16):
    """compute_tile_intersection_ordered without the host read between the
    count and the sort (gs_bin_sort_capped): the lists are sized by this
    device's capacities, K and M stay on the device, and the lists end at the
    capacity (indexing_offset shifted by capacity - K; the result is a valid
    blend input with k = gaussian_ids_sorted.numel()).  Returns (indexing_offset,
    gaussian_ids_sorted, launch_order, check): call check.ok() after queueing
    the work that reads the lists; False means they did not fit (every tile is
    then empty) and must be binned again, e.g. by
    compute_tile_intersection_ordered, which also grows the capacities.  check is
    None when the lists were binned with exact sizes: the first call on a device,
    grids of more than 256 supertiles (16384 tiles), or no Gaussians."""
    dev = _device_of(points_image)
    n = points_image.shape[0]
    f32 = torch.float32
    width, height, tile_size = int(width), int(height), int(tile_size)
    if tile_size <= 0 or width <= 0 or height <= 0:
        raise RuntimeError("compute_tile_intersection: width, height and tile_size must be > 0")
    tiles_x = (width + tile_size - 1) // tile_size
    tiles_y = (height + tile_size - 1) // tile_size
    n_tiles = tiles_x * tiles_y
    n_super = ((tiles_x + 7) // 8) * ((tiles_y + 7) // 8)
    key = (dev.index, width, height, tile_size)
    caps = _CAPACITY.get(key)
    capturing = torch.cuda.is_current_stream_capturing()
    if not CAPPED_BINNING or caps is None or n == 0 or n_super > 256 or n_tiles > 16384:
        if capturing:  # the exact sizes need a host read, which a capture cannot wait for
            raise RuntimeError(
                "compute_tile_intersection: a graph capture needs the capped sort: render "
                "once at this resolution before capturing (the capacities come from that "
                f"call), with at least one visible Gaussian and at most 16384 tiles "
                f"(n={n}, {n_tiles} tiles, capacities {'set' if caps else 'unset'}, "
                f"CAPPED_BINNING={CAPPED_BINNING})")
        off, ids, order = _tile_intersection(points_image, radii, depths, mask, width, height,
                                             tile_size, False, ordered=True)
        return off, ids, order, None
    points_image = _prep(points_image, "points_image", f32, (n, 2), dev)
    radii = _prep(radii, "radii", f32, (n, 2), dev)
    depths = _prep(depths, "depths", f32, (n,), dev)
    mask = _prep(mask, "mask", torch.bool, (n,), dev)
    lib = _lib.load()
    k_cap, m_cap = caps
    with torch.cuda.device(dev):
        stream = _stream(dev)
        sz = ctypes.c_size_t(0)
        _lib.check(lib.gs_bin_count_workspace_size(n, ctypes.byref(sz)), "workspace query")
        ws_count = torch.empty((max(sz.value, 1),), dtype=torch.uint8, device=dev)
        sz2 = ctypes.c_size_t(0)
        _lib.check(lib.gs_bin_sort_workspace_size(n, k_cap, m_cap, width, height, tile_size,
                                                  ctypes.byref(sz2)), "workspace query")
        ws_sort = torch.empty((max(sz2.value, 1),), dtype=torch.uint8, device=dev)
        indexing_offset = torch.empty((n_tiles,), dtype=torch.int32, device=dev)
        order = torch.empty((n_tiles,), dtype=torch.int32, device=dev)
        ids = torch.empty((k_cap,), dtype=torch.int32, device=dev)
        # the totals go to mapped pinned memory, or (when it is not mapped, and in a
        # graph capture, where the graph's pool holds them for every replay) to
        # device memory read with a copy
        host_totals = dev_totals = totals_ptr = None
        if not capturing:
            host_totals = torch.empty((4,), dtype=torch.int64, pin_memory=True)
            totals_ptr = _pinned_device_pointer(host_totals)
        if totals_ptr is None:
            host_totals = None
            dev_totals = torch.empty((4,), dtype=torch.int64, device=dev)
            totals_ptr = _ptr(dev_totals)
        args = (_ptr(points_image), _ptr(radii), _ptr(depths), _ptr(mask), n, width, height,
                tile_size, _ptr(ws_count), sz.value, totals_ptr, stream)
        hint_kmin, hint_shift = _depth_hint(dev)
        ev = _lib.timer.record("bin_count", dev)
        # the totals are final once the first count phase has run; the event the
        # check waits on is recorded after the sort, so that no marker sits between
        # the binning kernels (the check runs after the blend is queued anyway:
        # bin_count 113 -> 110 us at config 3, 56 -> 53 us at config 1)
        ready = None if capturing else torch.cuda.Event()
        check = None
        recorded = False
        try:
            _lib.check(lib.gs_bin_count_begin_hinted(*args[:10], hint_kmin, hint_shift,
                                                     *args[10:]),
                       "compute_tile_intersection (count)")
            check = CappedCheck(ready, host_totals, dev_totals, caps, key)
            _lib.check(lib.gs_bin_count_finish(*args), "compute_tile_intersection (count)")
            _lib.timer.stop(ev, dev)
            ev = _lib.timer.record("bin_sort", dev)
            _lib.check(lib.gs_bin_sort_capped(
                _ptr(points_image), _ptr(radii), _ptr(depths), n, width, height, tile_size,
                k_cap, m_cap, _ptr(ws_count), _ptr(ws_sort), sz2.value, _ptr(indexing_offset),
                _ptr(ids), _ptr(order), stream), "compute_tile_intersection (sort)")
            _lib.timer.stop(ev, dev)
            if ready is not None:
                ready.record(torch.cuda.current_stream(dev))
                recorded = True
        except BaseException:
            # the device may still write the pinned totals: wait before releasing them
            if capturing:
                pass  # nothing ran yet; the capture itself is invalid now
            elif check is not None:
                if not recorded:
                    ready.record(torch.cuda.current_stream(dev))
                check.ok()
            else:
                torch.cuda.current_stream(dev).synchronize()
            raise
    return indexing_offset, ids, order, check


def compute_tile_intersection_debug(points_image, radii, depths, mask, width, height, tile_size=16):
    """compute_tile_intersection plus the sorted 64-bit keys (tile << 32 | depth bits,
    as int64) and tiles_touched per Gaussian (int32), for parity checks."""
    return _tile_intersection(points_image, radii, depths, mask, width, height, tile_size, True)


def _blend_inputs(indexing_offset, gaussian_ids_sorted, points_image, cov_inv_image, opacities,
                  colors):
    dev = _device_of(points_image)
    n = points_image.shape[0]
    f32 = torch.float32
    indexing_offset = _prep(indexing_offset, "indexing_offset", torch.int32,
                            (indexing_offset.shape[0],), dev)
    gaussian_ids_sorted = _prep(gaussian_ids_sorted, "gaussian_ids_sorted", torch.int32,
                                (gaussian_ids_sorted.shape[0],), dev)
    points_image = _prep(points_image, "points_image", f32, (n, 2), dev)
    cov_inv_image = _prep(cov_inv_image, "cov_inv_image", f32, (n, 3), dev)
    opacities = _prep(opacities, "opacities", f32, (n,), dev)
    colors = _prep(colors, "colors", f32, (n, 3), dev)
    return dev, n, indexing_offset, gaussian_ids_sorted, points_image, cov_inv_image, opacities, colors


def rasterize(
    indexing_offset,
    gaussian_ids_sorted,
    points_image,
    cov_inv_image,
    opacities,
    colors,
    width,
    height,
    tile_size,
    alpha_threshold,
    transmittance_threshold,
    chi_squared_threshold,
):
    """Reference: src/cuda/rasterizer.cpp:361-395.  Returns image[H,W,3] (un-clamped)."""
    dev, n, off, ids, pts, conic, opac, col = _blend_inputs(
        indexing_offset, gaussian_ids_sorted, points_image, cov_inv_image, opacities, colors)
    width, height = int(width), int(height)
    image = torch.empty((height, width, 3), dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        ev = _lib.timer.record("rasterize", dev)
        _lib.check(
            _lib.load().gs_rasterize(
                _ptr(off), _ptr(ids), off.shape[0], ids.shape[0], _ptr(pts), _ptr(conic),
                _ptr(opac), _ptr(col), n, width, height, int(tile_size), float(alpha_threshold),
                float(transmittance_threshold), float(chi_squared_threshold), _ptr(image),
                _stream(dev),
            ),
            "rasterize",
        )
        _lib.timer.stop(ev, dev)
    return image


def _blend_grad_views(buf, n):
    """The four gradient outputs (N,2), (N,3), (N,), (N,3) carved from one 9N buffer."""
    return (buf[: 2 * n].view(n, 2), buf[2 * n : 5 * n].view(n, 3), buf[5 * n : 6 * n],
            buf[6 * n :].view(n, 3))


def _zeroed_blend_grads(n, dev):
    """Four zeroed gradient outputs (N,2), (N,3), (N,), (N,3) carved from one buffer."""
    return _blend_grad_views(torch.zeros((9 * n,), dtype=torch.float32, device=dev), n)


def blend_grad_accumulators(n, device):
    """An uninitialised 9N fp32 buffer for the blend gradients: pass it as
    rasterize_display_l1(clear=...) (which zeroes it) and then as
    rasterize_l1_backward(accumulators=...)."""
    return torch.empty((9 * int(n),), dtype=torch.float32, device=device)


def set_blend_waves(waves: int = 0) -> None:
    """Waves per 16x16 tile of the blend kernels (gs_set_blend_waves): 0 = by the
    tile count (the default), or 1, 2, 4.  Process-wide."""
    _lib.check(_lib.load().gs_set_blend_waves(int(waves)), "set_blend_waves")


def schedule_size(n_tiles) -> int:
    """int32 elements of a tile schedule for n_tiles tiles (gs_tile_schedule_size)."""
    out = ctypes.c_size_t(0)
    _lib.check(_lib.load().gs_tile_schedule_size(int(n_tiles), ctypes.byref(out)),
               "tile_schedule_size")
    return int(out.value)


def tile_schedule(n_tiles, device):
    """An uninitialised int32 buffer of schedule_size(n_tiles) elements: pass it as
    rasterize_display_l1(schedule=...) or rasterize_display(schedule=...), which
    fill it (the work of each tile, the backward's launch order, and the
    transmittance and colour checkpoints of the long tiles' walks), and then as
    the backward's schedule, which launches those tiles in segments."""
    return torch.empty((max(schedule_size(n_tiles), 2),), dtype=torch.int32, device=device)


def _check_schedule(schedule, n_tiles, dev, who):
    need = schedule_size(n_tiles)
    if (not isinstance(schedule, torch.Tensor) or schedule.dtype != torch.int32
            or schedule.device != dev or not schedule.is_contiguous()
            or schedule.numel() < need):
        raise RuntimeError(f"{who}: schedule must be a contiguous int32 tensor of at least "
                           f"{need} elements on {dev} (tile_schedule)")


# Set True (tests do) to verify every forward launch order as a permutation of
# each XCD range before the launch: a device sort and one host read per call.
CHECK_FORWARD_ORDERS = False

_XCDS = 8  # the blend kernels' tile ranges: launch slot p of XCD x is in range x


def check_forward_order(order, n_tiles):
    """Raise RasterizerError unless order[:n_tiles] permutes every XCD range.

    The blend forward launches the tiles of each XCD's contiguous range
    [x*b + min(x, r), (x+1)*b + min(x+1, r)), b, r = divmod(n_tiles, 8), in the
    order's sequence: slot p launches tile order[p], which must lie in p's range,
    and every tile must appear once.  An order that breaks this leaves some tiles'
    image, display and loss entries unwritten (nothing faults: the kernel skips
    tiles out of range)."""
    n_tiles = int(n_tiles)
    if n_tiles == 0:
        return
    o = order[:n_tiles].to(torch.int64)
    b, r = divmod(n_tiles, _XCDS)

    def range_of(t):
        big = r * (b + 1)  # the first r ranges hold b + 1 tiles
        return torch.where(t < big, t // (b + 1), r + (t - big) // max(b, 1))

    slots = torch.arange(n_tiles, device=o.device)
    in_range = bool(((o >= 0) & (o < n_tiles)).all())
    if not in_range or not bool((range_of(o) == range_of(slots)).all()) or not torch.equal(
            torch.sort(o).values, slots):
        raise RasterizerError("forward_order is not a permutation of every XCD tile range")


def _check_order(order, schedule, n_tiles, dev, who):
    """A forward launch order: n_tiles int32 on the device, not inside `schedule`
    (a permutation of every XCD range, see check_forward_order; verified only
    with CHECK_FORWARD_ORDERS, and not during a graph capture, which cannot read
    it on the host)."""
    if order is None:
        return
    if (not isinstance(order, torch.Tensor) or order.dtype != torch.int32
            or order.device != dev or not order.is_contiguous() or order.numel() < n_tiles):
        raise RuntimeError(f"{who}: forward_order must be a contiguous int32 tensor of at "
                           f"least {n_tiles} elements on {dev}")
    if schedule is not None and (
            schedule.data_ptr() <= order.data_ptr() < schedule.data_ptr() + schedule.numel() * 4):
        raise RasterizerError(f"{who}: forward_order must not lie in the schedule this call "
                              "writes")
    if CHECK_FORWARD_ORDERS and not torch.cuda.is_current_stream_capturing():
        check_forward_order(order, n_tiles)


def rasterize_backward(
    grad_rendered_image,
    indexing_offset,
    gaussian_ids_sorted,
    points_image,
    cov_inv_image,
    opacities,
    colors,
    width,
    height,
    tile_size,
    alpha_threshold,
    transmittance_threshold,
    chi_squared_threshold,
    rendered_image=None,
):
    """Reference: src/cuda/rasterizer.cpp:397-440.

    Returns (grad_points_image[N,2], grad_cov_inv_image[N,3], grad_opacities[N],
    grad_colors[N,3]).  `rendered_image`, if given, must be rasterize()'s
    output for the same inputs.
    """
    dev, n, off, ids, pts, conic, opac, col = _blend_inputs(
        indexing_offset, gaussian_ids_sorted, points_image, cov_inv_image, opacities, colors)
    width, height = int(width), int(height)
    f32 = torch.float32
    grad = _prep(grad_rendered_image, "grad_rendered_image", f32, (height, width, 3), dev)
    img = None
    if rendered_image is not None:
        img = _prep(rendered_image, "rendered_image", f32, (height, width, 3), dev)
    # zeroed here (one fill) so that the library call and its timing events are the
    # blend kernel alone
    g_pts, g_conic, g_opac, g_col = _zeroed_blend_grads(n, dev)
    with torch.cuda.device(dev):
        ev = _lib.timer.record("rasterize_backward", dev)
        _lib.check(
            _lib.load().gs_rasterize_backward(
                _ptr(grad), _ptr(img), _ptr(off), _ptr(ids), off.shape[0], ids.shape[0],
                _ptr(pts), _ptr(conic), _ptr(opac), _ptr(col), n, width, height, int(tile_size),
                float(alpha_threshold), float(transmittance_threshold),
                float(chi_squared_threshold), _ptr(g_pts), _ptr(g_conic), _ptr(g_opac),
                _ptr(g_col), 1, _stream(dev),
            ),
            "rasterize_backward",
        )
        _lib.timer.stop(ev, dev)
    return g_pts, g_conic, g_opac, g_col


def rasterize_work(indexing_offset, gaussian_ids_sorted, points_image, cov_inv_image, opacities,
                   width, height, tile_size, alpha_threshold, transmittance_threshold,
                   chi_squared_threshold):
    """Work of the reference blend loop for these inputs (measurement helper):
    returns (visited, composited) -- (pixel, list entry) pairs walked before each
    pixel's transmittance test stopped it, and pairs actually blended."""
    colors = torch.zeros((points_image.shape[0], 3), dtype=torch.float32, device=points_image.device)
    dev, n, off, ids, pts, conic, opac, _ = _blend_inputs(
        indexing_offset, gaussian_ids_sorted, points_image, cov_inv_image, opacities, colors)
    counters = torch.empty((2,), dtype=torch.int64, device=dev)
    with torch.cuda.device(dev):
        _lib.check(
            _lib.load().gs_rasterize_work(
                _ptr(off), _ptr(ids), off.shape[0], ids.shape[0], _ptr(pts), _ptr(conic),
                _ptr(opac), n, int(width), int(height), int(tile_size), float(alpha_threshold),
                float(transmittance_threshold), float(chi_squared_threshold), _ptr(counters),
                counters.data_ptr() + 8, _stream(dev),
            ),
            "rasterize_work",
        )
    visited, composited = counters.tolist()
    return visited, composited


# ------------------------------------------------------------- render() fusions
# Fused forms of the glue render() puts around the seven functions
# (src/cuda/wrapper.py:223-294).  Results equal the unfused sequence; used by
# cuda_rasterizer.wrapper.render.


def sh_render_inputs(world_to_camera, points_world, sh_coeffs_dc, sh_coeffs_rest, mask):
    """evaluate_spherical_harmonics_render's inputs validated (dtype, device, shape)
    and made contiguous, on the current stream.  A caller that launches the
    colours on another stream calls this first, so that any copy is queued
    before its fork."""
    dev = _device_of(points_world)
    n = points_world.shape[0]
    f32 = torch.float32
    return (_prep(world_to_camera, "world_to_camera", f32, (4, 4), dev),
            _prep(points_world, "points_world", f32, (n, 3), dev),
            _prep(sh_coeffs_dc, "sh_coeffs_dc", f32, (n, 3), dev),
            _prep(sh_coeffs_rest, "sh_coeffs_rest", f32, (n, 15, 3), dev),
            _prep(mask, "mask", torch.bool, (n,), dev))


SH_CACHE_FLOATS = 10


def sh_cache_empty(n: int, device) -> torch.Tensor:
    """An uninitialised colour-gradient cache for n Gaussians: (N, 10) float32,
    written by evaluate_spherical_harmonics_render(sh_cache=...) or
    preprocess_forward(sh_cache=...) for the Gaussians in their mask."""
    return torch.empty((n, SH_CACHE_FLOATS), dtype=torch.float32, device=device)


def _check_sh_cache(sh_cache, n, dev, who):
    if (not isinstance(sh_cache, torch.Tensor) or sh_cache.dtype != torch.float32
            or sh_cache.shape != (n, SH_CACHE_FLOATS) or sh_cache.device != dev
            or not sh_cache.is_contiguous() or sh_cache.data_ptr() % 8):
        raise RuntimeError(f"{who}: sh_cache must be a contiguous ({n}, {SH_CACHE_FLOATS}) "
                           f"float32 tensor on {dev} (sh_cache_empty)")
    return sh_cache


def evaluate_spherical_harmonics_render(world_to_camera, points_world, sh_coeffs_dc,
                                        sh_coeffs_rest, mask, out=None, beside=False,
                                        stream=None, sh_cache=None):
    """max(evaluate_spherical_harmonics(-R^T t, ...) + 0.5, 0) in one kernel
    (src/cuda/wrapper.py:260-265).  Masked rows are 0.5.  out: a contiguous
    (N, 3) float32 tensor to write instead of a new one.  beside: launch it for a
    stream that runs beside other work (gs_evaluate_sh_render_beside: one
    workgroup per compute unit; the same values).  stream: a torch.cuda.Stream
    of the tensors' device to launch on (default: the current stream); the
    caller orders it against the producers and consumers of the tensors.
    sh_cache: an (N, 10) float32 tensor (sh_cache_empty) that also receives the
    colour-gradient cache (gs_evaluate_sh_render_cache), which
    render_preprocess_backward and preprocess_backward take in place of the SH
    coefficients."""
    dev = _device_of(points_world)
    n = points_world.shape[0]
    f32 = torch.float32
    world_to_camera, points_world, sh_coeffs_dc, sh_coeffs_rest, mask = sh_render_inputs(
        world_to_camera, points_world, sh_coeffs_dc, sh_coeffs_rest, mask)
    if out is None:
        colors = torch.empty((n, 3), dtype=f32, device=dev)
    else:
        if (not isinstance(out, torch.Tensor) or out.dtype != f32 or out.shape != (n, 3)
                or out.device != dev or not out.is_contiguous()):
            raise RuntimeError("evaluate_spherical_harmonics_render: out must be a contiguous "
                               f"({n}, 3) float32 tensor on {dev}")
        colors = out
    if sh_cache is not None:
        _check_sh_cache(sh_cache, n, dev, "evaluate_spherical_harmonics_render")
    with torch.cuda.device(dev):
        ev = _lib.timer.record("evaluate_sh_render", dev, stream)
        lib = _lib.load()
        launch = _stream(dev) if stream is None else stream.cuda_stream
        if sh_cache is not None:
            status = lib.gs_evaluate_sh_render_cache(
                _ptr(world_to_camera), _ptr(points_world), _ptr(sh_coeffs_dc),
                _ptr(sh_coeffs_rest), _ptr(mask), n, 1 if beside else 0, _ptr(colors),
                _ptr(sh_cache), launch)
        else:
            fn = lib.gs_evaluate_sh_render_beside if beside else lib.gs_evaluate_sh_render
            status = fn(_ptr(world_to_camera), _ptr(points_world), _ptr(sh_coeffs_dc),
                        _ptr(sh_coeffs_rest), _ptr(mask), n, _ptr(colors), launch)
        _lib.check(status, "evaluate_spherical_harmonics_render")
        _lib.timer.stop(ev, dev, stream)
    return colors


def evaluate_spherical_harmonics_render_backward(grad_colors, world_to_camera, points_world,
                                                 sh_coeffs_dc, sh_coeffs_rest, mask,
                                                 accumulate_means=None):
    """Gradient of evaluate_spherical_harmonics_render.  Returns
    (grad_points_world[N,3], grad_sh_coeffs_dc[N,3], grad_sh_coeffs_rest[N,15,3]).
    With `accumulate_means` (an (N,3) fp32 tensor on the device), the means
    gradient is added to it in place and it is returned as the first element."""
    dev = _device_of(points_world)
    n = points_world.shape[0]
    f32 = torch.float32
    grad_colors = _prep(grad_colors, "grad_colors", f32, (n, 3), dev)
    world_to_camera = _prep(world_to_camera, "world_to_camera", f32, (4, 4), dev)
    points_world = _prep(points_world, "points_world", f32, (n, 3), dev)
    sh_coeffs_dc = _prep(sh_coeffs_dc, "sh_coeffs_dc", f32, (n, 3), dev)
    sh_coeffs_rest = _prep(sh_coeffs_rest, "sh_coeffs_rest", f32, (n, 15, 3), dev)
    mask = _prep(mask, "mask", torch.bool, (n,), dev)
    if accumulate_means is not None:
        if (accumulate_means.dtype != f32 or accumulate_means.shape != (n, 3)
                or not accumulate_means.is_contiguous() or accumulate_means.device != dev):
            raise RuntimeError("accumulate_means must be a contiguous (N,3) fp32 tensor on "
                               f"{dev}")
        g_means = accumulate_means
    else:
        g_means = torch.empty((n, 3), dtype=f32, device=dev)
    g_dc = torch.empty((n, 3), dtype=f32, device=dev)
    g_rest = torch.empty((n, 15, 3), dtype=f32, device=dev)
    with torch.cuda.device(dev):
        ev = _lib.timer.record("evaluate_sh_render_backward", dev)
        _lib.check(
            _lib.load().gs_evaluate_sh_render_backward(
                _ptr(grad_colors), _ptr(world_to_camera), _ptr(points_world), _ptr(sh_coeffs_dc),
                _ptr(sh_coeffs_rest), _ptr(mask), n, 1 if accumulate_means is not None else 0,
                _ptr(g_means), _ptr(g_dc), _ptr(g_rest), _stream(dev),
            ),
            "evaluate_spherical_harmonics_render_backward",
        )
        _lib.timer.stop(ev, dev)
    return g_means, g_dc, g_rest


def rasterize_display(indexing_offset, gaussian_ids_sorted, points_image, cov_inv_image,
                      opacities, colors, width, height, tile_size, alpha_threshold,
                      transmittance_threshold, chi_squared_threshold, schedule=None,
                      forward_order=None):
    """rasterize() that also returns clamp(image, 0, 1) * 255 (src/cuda/wrapper.py:294).
    Returns (image[H,W,3] un-clamped, display[H,W,3]).  `schedule` (see
    tile_schedule) receives the work per tile and the order in which
    rasterize_display_backward, given it, launches the tiles.  `forward_order`:
    a launch order for this forward (compute_tile_intersection_ordered's).  It
    must permute every XCD tile range (check_forward_order states the ranges):
    tiles it leaves out are not written."""
    dev, n, off, ids, pts, conic, opac, col = _blend_inputs(
        indexing_offset, gaussian_ids_sorted, points_image, cov_inv_image, opacities, colors)
    width, height = int(width), int(height)
    if schedule is not None:
        _check_schedule(schedule, off.shape[0], dev, "rasterize_display")
    _check_order(forward_order, schedule, off.shape[0], dev, "rasterize_display")
    image = torch.empty((height, width, 3), dtype=torch.float32, device=dev)
    display = torch.empty((height, width, 3), dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        ev = _lib.timer.record("rasterize_display", dev)
        _lib.check(
            _lib.load().gs_rasterize_display(
                _ptr(off), _ptr(ids), off.shape[0], ids.shape[0], _ptr(pts), _ptr(conic),
                _ptr(opac), _ptr(col), n, width, height, int(tile_size), float(alpha_threshold),
                float(transmittance_threshold), float(chi_squared_threshold), _ptr(image),
                _ptr(display), _ptr(schedule), _ptr(forward_order), _stream(dev),
            ),
            "rasterize_display",
        )
        _lib.timer.stop(ev, dev)
    return image, display


def rasterize_display_backward(grad_display, indexing_offset, gaussian_ids_sorted, points_image,
                               cov_inv_image, opacities, colors, width, height, tile_size,
                               alpha_threshold, transmittance_threshold, chi_squared_threshold,
                               rendered_image, schedule=None):
    """Gradient of rasterize_display's display output; `rendered_image` (its
    un-clamped image) is required.  Returns the four gradients of rasterize_backward.
    `schedule`: the tensor rasterize_display filled for the same layout."""
    dev, n, off, ids, pts, conic, opac, col = _blend_inputs(
        indexing_offset, gaussian_ids_sorted, points_image, cov_inv_image, opacities, colors)
    width, height = int(width), int(height)
    if schedule is not None:
        _check_schedule(schedule, off.shape[0], dev, "rasterize_display_backward")
    f32 = torch.float32
    grad = _prep(grad_display, "grad_display", f32, (height, width, 3), dev)
    img = _prep(rendered_image, "rendered_image", f32, (height, width, 3), dev)
    g_pts, g_conic, g_opac, g_col = _zeroed_blend_grads(n, dev)
    with torch.cuda.device(dev):
        ev = _lib.timer.record("rasterize_display_backward", dev)
        _lib.check(
            _lib.load().gs_rasterize_display_backward(
                _ptr(grad), _ptr(img), _ptr(off), _ptr(ids), off.shape[0], ids.shape[0],
                _ptr(pts), _ptr(conic), _ptr(opac), _ptr(col), n, width, height, int(tile_size),
                float(alpha_threshold), float(transmittance_threshold),
                float(chi_squared_threshold), _ptr(g_pts), _ptr(g_conic), _ptr(g_opac),
                _ptr(g_col), 1, _ptr(schedule), _stream(dev),
            ),
            "rasterize_display_backward",
        )
        _lib.timer.stop(ev, dev)
    return g_pts, g_conic, g_opac, g_col


# ------------------------------------------------------ fused training step
# Kernels for the caller-side glue of a training step (activations and the L1
# loss, scripts/train.py:135-143,187-191); cuda_rasterizer.fused chains them.


def activate(log_scales, quats_raw, opacity_logits):
    """(exp(log_scales), q / max(|q|, 1e-12), sigmoid(logits)) in one kernel."""
    dev = _device_of(log_scales)
    n = log_scales.shape[0]
    f32 = torch.float32
    log_scales = _prep(log_scales, "log_scales", f32, (n, 3), dev)
    quats_raw = _prep(quats_raw, "quats_raw", f32, (n, 4), dev)
    opacity_logits = _prep(opacity_logits, "opacity_logits", f32, (n,), dev)
    scales = torch.empty((n, 3), dtype=f32, device=dev)
    quats = torch.empty((n, 4), dtype=f32, device=dev)
    opac = torch.empty((n,), dtype=f32, device=dev)
    with torch.cuda.device(dev):
        ev = _lib.timer.record("activate", dev)
        _lib.check(_lib.load().gs_activate(_ptr(log_scales), _ptr(quats_raw), _ptr(opacity_logits),
                                           n, _ptr(scales), _ptr(quats), _ptr(opac), _stream(dev)),
                   "activate")
        _lib.timer.stop(ev, dev)
    return scales, quats, opac


def activate_backward(grad_scales, grad_quats, grad_opacities, scales, quats_raw, opacities):
    """Gradients of activate's outputs (None = zero) -> (d log_scales, d quats_raw, d logits)."""
    dev = _device_of(scales)
    n = scales.shape[0]
    f32 = torch.float32
    gs_ = None if grad_scales is None else _prep(grad_scales, "grad_scales", f32, (n, 3), dev)
    gq = None if grad_quats is None else _prep(grad_quats, "grad_quats", f32, (n, 4), dev)
    go = None if grad_opacities is None else _prep(grad_opacities, "grad_opacities", f32, (n,), dev)
    scales = _prep(scales, "scales", f32, (n, 3), dev)
    quats_raw = _prep(quats_raw, "quats_raw", f32, (n, 4), dev)
    opacities = _prep(opacities, "opacities", f32, (n,), dev)
    g_ls = torch.empty((n, 3), dtype=f32, device=dev)
    g_q = torch.empty((n, 4), dtype=f32, device=dev)
    g_l = torch.empty((n,), dtype=f32, device=dev)
    with torch.cuda.device(dev):
        ev = _lib.timer.record("activate_backward", dev)
        _lib.check(_lib.load().gs_activate_backward(
            _ptr(gs_), _ptr(gq), _ptr(go), _ptr(scales), _ptr(quats_raw), _ptr(opacities), n,
            _ptr(g_ls), _ptr(g_q), _ptr(g_l), _stream(dev)), "activate_backward")
        _lib.timer.stop(ev, dev)
    return g_ls, g_q, g_l


def preprocess_forward(means, log_scales, quats_raw, opacity_logits, sh_coeffs_dc,
                       sh_coeffs_rest, world_to_camera, intrinsic, near_plane, far_plane,
                       min_opacity, min_radius, max_radius, width, height, with_colors=True,
                       sh_cache=None):
    """activate -> project_points -> evaluate_spherical_harmonics_render in one kernel
    (gs_preprocess_forward).  Returns (points_image, depths, cov_image, cov_inv_image,
    radii, mask, opacities, colors); with_colors=False skips the colours (None;
    evaluate_spherical_harmonics_render gives the same values).  sh_cache (with
    the colours): an (N, 10) float32 tensor (sh_cache_empty) that also receives
    the colour-gradient cache for preprocess_backward."""
    dev = _device_of(means)
    n = means.shape[0]
    f32 = torch.float32
    means = _prep(means, "means", f32, (n, 3), dev)
    log_scales = _prep(log_scales, "log_scales", f32, (n, 3), dev)
    quats_raw = _prep(quats_raw, "quats_raw", f32, (n, 4), dev)
    opacity_logits = _prep(opacity_logits, "opacity_logits", f32, (n,), dev)
    dc = rest = colors = None
    if with_colors:
        dc = _prep(sh_coeffs_dc, "sh_coeffs_dc", f32, (n, 3), dev)
        rest = _prep(sh_coeffs_rest, "sh_coeffs_rest", f32, (n, 15, 3), dev)
        colors = torch.empty((n, 3), dtype=f32, device=dev)
    if sh_cache is not None:
        if not with_colors:
            raise RuntimeError("preprocess_forward: sh_cache is written with the colours only")
        _check_sh_cache(sh_cache, n, dev, "preprocess_forward")
    world_to_camera = _prep(world_to_camera, "world_to_camera", f32, (4, 4), dev)
    intrinsic = _prep(intrinsic, "intrinsic", f32, (3, 3), dev)
    out = [torch.empty(shape, dtype=f32, device=dev)
           for shape in ((n, 2), (n,), (n, 3), (n, 3), (n, 2))]
    mask = torch.empty((n,), dtype=torch.bool, device=dev)
    opac = torch.empty((n,), dtype=f32, device=dev)
    with torch.cuda.device(dev):
        ev = _lib.timer.record("preprocess_forward" if with_colors else "preprocess_project", dev)
        _lib.check(_lib.load().gs_preprocess_forward(
            _ptr(means), _ptr(log_scales), _ptr(quats_raw), _ptr(opacity_logits), _ptr(dc),
            _ptr(rest), _ptr(world_to_camera), _ptr(intrinsic), n, float(near_plane),
            float(far_plane), float(min_opacity), float(min_radius), float(max_radius), int(width),
            int(height), *[_ptr(t) for t in out], _ptr(mask), _ptr(opac), _ptr(colors),
            _ptr(sh_cache), _stream(dev)), "preprocess_forward")
        _lib.timer.stop(ev, dev)
    return (*out, mask, opac, colors)


def _sh_or_cache(sh_coeffs_dc, sh_coeffs_rest, sh_cache, n, dev, who):
    """The SH coefficients a backward reads, or (None, None) with a valid cache."""
    if sh_cache is not None:
        _check_sh_cache(sh_cache, n, dev, who)
        return None, None
    f32 = torch.float32
    return (_prep(sh_coeffs_dc, "sh_coeffs_dc", f32, (n, 3), dev),
            _prep(sh_coeffs_rest, "sh_coeffs_rest", f32, (n, 15, 3), dev))


def preprocess_backward(grad_points_image, grad_cov_inv_image, grad_opacities, grad_colors,
                        means, log_scales, quats_raw, opacity_logits, sh_coeffs_dc,
                        sh_coeffs_rest, cov_image, mask, world_to_camera, intrinsic, width,
                        height, sh_cache=None):
    """Gradients of preprocess_forward's points_image, cov_inv_image, opacities and
    colors w.r.t. the raw parameters (gs_preprocess_backward).  Returns (d means,
    d log_scales, d quats_raw, d logits, d sh_dc, d sh_rest).  sh_cache: the
    forward's colour-gradient cache; the SH coefficients are then not read (and
    may be None), the results are the same bit for bit."""
    dev = _device_of(means)
    n = means.shape[0]
    f32 = torch.float32
    g_pts = _prep(grad_points_image, "grad_points_image", f32, (n, 2), dev)
    g_conic = _prep(grad_cov_inv_image, "grad_cov_inv_image", f32, (n, 3), dev)
    g_opac = _prep(grad_opacities, "grad_opacities", f32, (n,), dev)
    g_col = _prep(grad_colors, "grad_colors", f32, (n, 3), dev)
    means = _prep(means, "means", f32, (n, 3), dev)
    log_scales = _prep(log_scales, "log_scales", f32, (n, 3), dev)
    quats_raw = _prep(quats_raw, "quats_raw", f32, (n, 4), dev)
    opacity_logits = _prep(opacity_logits, "opacity_logits", f32, (n,), dev)
    dc, rest = _sh_or_cache(sh_coeffs_dc, sh_coeffs_rest, sh_cache, n, dev,
                            "preprocess_backward")
    cov_image = _prep(cov_image, "cov_image", f32, (n, 3), dev)
    mask = _prep(mask, "mask", torch.bool, (n,), dev)
    world_to_camera = _prep(world_to_camera, "world_to_camera", f32, (4, 4), dev)
    intrinsic = _prep(intrinsic, "intrinsic", f32, (3, 3), dev)
    outs = [torch.empty(shape, dtype=f32, device=dev)
            for shape in ((n, 3), (n, 3), (n, 4), (n,), (n, 3), (n, 15, 3))]
    with torch.cuda.device(dev):
        ev = _lib.timer.record("preprocess_backward", dev)
        _lib.check(_lib.load().gs_preprocess_backward(
            _ptr(g_pts), _ptr(g_conic), _ptr(g_opac), _ptr(g_col), _ptr(means), _ptr(log_scales),
            _ptr(quats_raw), _ptr(opacity_logits), _ptr(dc), _ptr(rest), _ptr(cov_image),
            _ptr(mask), _ptr(world_to_camera), _ptr(intrinsic), n, int(width), int(height),
            *[_ptr(t) for t in outs], _ptr(sh_cache), _stream(dev)), "preprocess_backward")
        _lib.timer.stop(ev, dev)
    return tuple(outs)


def render_preprocess_backward(grad_points_image, grad_cov_inv_image, grad_colors, means, scales,
                               quaternions, sh_coeffs_dc, sh_coeffs_rest, cov_image, mask,
                               world_to_camera, intrinsic, width, height, sh_cache=None):
    """project_points_backward and evaluate_sh_render_backward in one kernel
    (gs_render_preprocess_backward): gradients of render()'s points_image,
    cov_inv_image and colours w.r.t. (means, scales, quaternions, sh_dc,
    sh_rest), the means' two terms summed.  Returns those five tensors.
    sh_cache: the colour-gradient cache evaluate_spherical_harmonics_render
    wrote for the same inputs; the SH coefficients are then not read (and may be
    None), the results are the same bit for bit."""
    dev = _device_of(means)
    n = means.shape[0]
    f32 = torch.float32
    g_pts = _prep(grad_points_image, "grad_points_image", f32, (n, 2), dev)
    g_conic = _prep(grad_cov_inv_image, "grad_cov_inv_image", f32, (n, 3), dev)
    g_col = _prep(grad_colors, "grad_colors", f32, (n, 3), dev)
    means = _prep(means, "means", f32, (n, 3), dev)
    scales = _prep(scales, "scales", f32, (n, 3), dev)
    quaternions = _prep(quaternions, "quaternions", f32, (n, 4), dev)
    dc, rest = _sh_or_cache(sh_coeffs_dc, sh_coeffs_rest, sh_cache, n, dev,
                            "render_preprocess_backward")
    cov_image = _prep(cov_image, "cov_image", f32, (n, 3), dev)
    mask = _prep(mask, "mask", torch.bool, (n,), dev)
    world_to_camera = _prep(world_to_camera, "world_to_camera", f32, (4, 4), dev)
    intrinsic = _prep(intrinsic, "intrinsic", f32, (3, 3), dev)
    outs = [torch.empty(shape, dtype=f32, device=dev)
            for shape in ((n, 3), (n, 3), (n, 4), (n, 3), (n, 15, 3))]
    with torch.cuda.device(dev):
        ev = _lib.timer.record("render_preprocess_backward", dev)
        _lib.check(_lib.load().gs_render_preprocess_backward(
            _ptr(g_pts), _ptr(g_conic), _ptr(g_col), _ptr(means), _ptr(scales),
            _ptr(quaternions), _ptr(dc), _ptr(rest), _ptr(cov_image), _ptr(mask),
            _ptr(world_to_camera), _ptr(intrinsic), n, int(width), int(height),
            *[_ptr(t) for t in outs], _ptr(sh_cache), _stream(dev)), "render_preprocess_backward")
        _lib.timer.stop(ev, dev)
    return tuple(outs)


def rasterize_display_l1(indexing_offset, gaussian_ids_sorted, points_image, cov_inv_image,
                         opacities, colors, width, height, target, alpha_threshold=1e-4,
                         transmittance_threshold=1e-4, chi_squared_threshold=9.21, clear=None,
                         schedule=None, forward_schedule=None, forward_order=None):
    """rasterize_display with tile size 16 plus loss = mean(|display / 255 - target|).
    Returns (image, display, loss[1] fp32).  `clear` (an fp32 device tensor, e.g.
    from blend_grad_accumulators) is zeroed by the same launch.  `schedule` (an
    int32 device tensor from tile_schedule) receives the work per tile, the order
    in which rasterize_l1_backward, given it, launches the tiles (heaviest first)
    and the checkpoints that let it walk long tiles in segments.  `forward_schedule`: a schedule an earlier call filled
    for the same image size (not this call's `schedule`); this forward then
    launches its tiles in that order (results do not depend on it).
    `forward_order`: instead of forward_schedule, any per-XCD-range launch order
    of n_tiles int32 (e.g. compute_tile_intersection_ordered's).  Either order must
    permute every XCD tile range (check_forward_order states the ranges): tiles
    it leaves out are not written, and the loss then sums unwritten entries."""
    dev, n, off, ids, pts, conic, opac, col = _blend_inputs(
        indexing_offset, gaussian_ids_sorted, points_image, cov_inv_image, opacities, colors)
    width, height = int(width), int(height)
    f32 = torch.float32
    target = _prep(target, "target", f32, (height, width, 3), dev)
    image = torch.empty((height, width, 3), dtype=f32, device=dev)
    display = torch.empty((height, width, 3), dtype=f32, device=dev)
    n_tiles = off.shape[0]
    tile_loss = torch.empty((max(n_tiles, 1),), dtype=f32, device=dev)
    loss = torch.empty((1,), dtype=f32, device=dev)
    if schedule is not None:
        _check_schedule(schedule, n_tiles, dev, "rasterize_display_l1")
    fwd_order = None
    if forward_schedule is not None:
        _check_schedule(forward_schedule, n_tiles, dev, "rasterize_display_l1")
        if schedule is not None and forward_schedule.data_ptr() == schedule.data_ptr():
            raise RasterizerError("rasterize_display_l1: forward_schedule must be an earlier "
                                  "call's schedule, not the one this call writes")
        fwd_order = forward_schedule[n_tiles:]
        if CHECK_FORWARD_ORDERS and not torch.cuda.is_current_stream_capturing():
            check_forward_order(fwd_order, n_tiles)
    if forward_order is not None:
        if forward_schedule is not None:
            raise RasterizerError("rasterize_display_l1: pass forward_schedule or forward_order, "
                                  "not both")
        _check_order(forward_order, schedule, n_tiles, dev, "rasterize_display_l1")
        fwd_order = forward_order
    lib = _lib.load()
    with torch.cuda.device(dev):
        ev = _lib.timer.record("rasterize_display_l1", dev)
        _lib.check(lib.gs_rasterize_display_l1(
            _ptr(off), _ptr(ids), n_tiles, ids.shape[0], _ptr(pts), _ptr(conic), _ptr(opac),
            _ptr(col), n, width, height, 16, float(alpha_threshold), float(transmittance_threshold),
            float(chi_squared_threshold), _ptr(target), _ptr(image), _ptr(display), _ptr(tile_loss),
            _ptr(loss), _ptr(schedule), _ptr(clear), 0 if clear is None else clear.numel(),
            _ptr(fwd_order), _stream(dev)), "rasterize_display_l1")
        _lib.timer.stop(ev, dev)
    return image, display, loss


def rasterize_l1_backward(target, grad_loss, indexing_offset, gaussian_ids_sorted, points_image,
                          cov_inv_image, opacities, colors, width, height, rendered_image,
                          alpha_threshold=1e-4, transmittance_threshold=1e-4,
                          chi_squared_threshold=9.21, accumulators=None, grad_display01=None,
                          loss_scale=1.0, schedule=None):
    """Gradient of rasterize_display_l1's loss (times grad_loss, a 1-element fp32
    device tensor) w.r.t. the four blend inputs.  `accumulators`: a 9N buffer
    already zeroed (rasterize_display_l1's `clear`) that the gradients are added
    into; otherwise a zeroed one is allocated.  `grad_display01`: an (H, W, 3)
    further gradient w.r.t. display / 255 (an SSIM term's), added to the L1 one;
    `loss_scale` weights the L1 term (1 - lambda in an L1 + SSIM loss).
    `schedule`: the tensor rasterize_display_l1 filled for the same layout (the
    tiles then start heaviest first; the gradients do not depend on it)."""
    dev, n, off, ids, pts, conic, opac, col = _blend_inputs(
        indexing_offset, gaussian_ids_sorted, points_image, cov_inv_image, opacities, colors)
    width, height = int(width), int(height)
    f32 = torch.float32
    target = _prep(target, "target", f32, (height, width, 3), dev)
    img = _prep(rendered_image, "rendered_image", f32, (height, width, 3), dev)
    gl = _prep(grad_loss.reshape(1), "grad_loss", f32, (1,), dev)
    extra = (None if grad_display01 is None
             else _prep(grad_display01, "grad_display01", f32, (height, width, 3), dev))
    if accumulators is None:
        g_pts, g_conic, g_opac, g_col = _zeroed_blend_grads(n, dev)
    else:
        if (accumulators.dtype != f32 or accumulators.device != dev
                or accumulators.numel() != 9 * n or not accumulators.is_contiguous()):
            raise RuntimeError("rasterize_l1_backward: accumulators must be a contiguous fp32 "
                               f"tensor of {9 * n} elements on {dev}")
        g_pts, g_conic, g_opac, g_col = _blend_grad_views(accumulators, n)
    if schedule is not None:
        _check_schedule(schedule, off.shape[0], dev, "rasterize_l1_backward")
    with torch.cuda.device(dev):
        ev = _lib.timer.record("rasterize_l1_backward", dev)
        _lib.check(_lib.load().gs_rasterize_l1_backward(
            _ptr(target), _ptr(gl), _ptr(img), _ptr(off), _ptr(ids), off.shape[0], ids.shape[0],
            _ptr(pts), _ptr(conic), _ptr(opac), _ptr(col), n, width, height, 16,
            float(alpha_threshold), float(transmittance_threshold), float(chi_squared_threshold),
            _ptr(g_pts), _ptr(g_conic), _ptr(g_opac), _ptr(g_col), 1, float(loss_scale),
            _ptr(extra), _ptr(schedule), _stream(dev)),
            "rasterize_l1_backward")
        _lib.timer.stop(ev, dev)
    return g_pts, g_conic, g_opac, g_col
