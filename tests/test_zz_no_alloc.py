"""GPU test of the allocation-free entry point gs_ssim_forward_noalloc, through
the C ABI.

It runs gs_ssim_forward's kernels with the per-workgroup partials in a static
device array instead of a caller workspace, so its outputs -- the mean, the
three derivative maps and the combined loss -- must equal gs_ssim_forward's bit
for bit (the mean is reduced in a fixed order).  Checked on two calls in a row,
each with a smaller input than the one before (the array then still holds
the earlier call's partials past the later call's workgroup count; the first
fills all 1024), in both orders of the two entry points, and its argument
checks.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

import helpers
from cuda_rasterizer import _lib

pytestmark = pytest.mark.gpu


def _strides(t):
    arr = (ctypes.c_int64 * 4)(*t.stride())
    return arr, ctypes.cast(arr, ctypes.c_void_p).value


def _forward(gpu, img1, img2, valid, divisor, other, lam, noalloc):
    """One call of either entry point; returns (mean, maps, loss) on the host."""
    lib = _lib.load()
    b, c, h, w = (int(x) for x in img1.shape)
    mean = torch.full((1,), float("nan"), device=gpu)
    loss = torch.full((1,), float("nan"), device=gpu)
    maps = [torch.full((b * c, h, w), float("nan"), device=gpu) for _ in range(3)]
    a1, s1 = _strides(img1)
    a2, s2 = _strides(img2)
    stream = torch.cuda.current_stream(gpu).cuda_stream
    args = [img1.data_ptr(), s1, img2.data_ptr(), s2, b, c, h, w, valid, divisor,
            mean.data_ptr(), *[m.data_ptr() for m in maps], other.data_ptr(), lam,
            loss.data_ptr()]
    with torch.cuda.device(gpu):
        if noalloc:
            st = lib.gs_ssim_forward_noalloc(*args, stream)
        else:
            sz = ctypes.c_size_t(0)
            assert lib.gs_ssim_workspace_size(b, c, h, w, ctypes.byref(sz)) == 0
            ws = torch.full((sz.value,), 0xAB, dtype=torch.uint8, device=gpu)
            st = lib.gs_ssim_forward(*args, ws.data_ptr(), sz.value, stream)
    assert st == 0, _lib.load().gs_status_string(st)
    torch.cuda.synchronize()
    return mean.cpu(), [m.cpu() for m in maps], loss.cpu()


def _inputs(shape_hwc, seed, permuted, gpu):
    g = torch.Generator().manual_seed(seed)
    h, w, c = shape_hwc
    x = torch.rand(h, w, c, generator=g) * 255.0
    y = torch.rand(h, w, c, generator=g)
    if permuted:  # the reference's (H, W, C) images permuted to (1, C, H, W)
        return (x.to(gpu).permute(2, 0, 1).unsqueeze(0), y.to(gpu).permute(2, 0, 1).unsqueeze(0))
    return (x.permute(2, 0, 1).contiguous().unsqueeze(0).to(gpu),
            y.permute(2, 0, 1).contiguous().unsqueeze(0).to(gpu))


# Units of 64 columns x 34 output rows per plane, 4 per workgroup, at most 1024
# workgroups (the static array's size).  2160x3840x3: 60 x 64 x 3 = 11520 units,
# 2880 workgroups capped at 1024, so the array is filled to capacity; then
# 720x1280x3: 20 x 22 x 3 = 1320 units, 330 workgroups; then 32x96x3: 2 x 1 x 3 =
# 6 units, 2 workgroups (every partial past the second still holds an earlier
# call's value)
CALLS = [((2160, 3840, 3), 4, True, 0, 255.0), ((720, 1280, 3), 1, True, 1, 255.0),
         ((32, 96, 3), 2, False, 0, 255.0)]


@pytest.mark.parametrize("noalloc_first", [True, False])
def test_noalloc_equals_workspace_entry(gpu, noalloc_first):
    other = torch.tensor([0.25], device=gpu)
    for shape, seed, permuted, valid, divisor in CALLS:
        img1, img2 = _inputs(shape, seed, permuted, gpu)
        order = (True, False) if noalloc_first else (False, True)
        out = {na: _forward(gpu, img1, img2, valid, divisor, other, 0.2, na) for na in order}
        (m_a, maps_a, l_a), (m_b, maps_b, l_b) = out[True], out[False]
        assert torch.isfinite(m_a).all() and torch.isfinite(maps_a[0]).all()
        assert helpers.same(m_a, m_b) and helpers.same(l_a, l_b)
        for x, y in zip(maps_a, maps_b):
            assert helpers.same(x, y)
        assert abs(float(l_a) - (0.8 * 0.25 + 0.2 * (1.0 - float(m_a)))) <= 1e-6


def test_noalloc_argument_checks(gpu):
    lib = _lib.load()
    img1, img2 = _inputs((32, 48, 3), 3, False, gpu)
    a1, s1 = _strides(img1)
    a2, s2 = _strides(img2)
    mean = torch.empty(1, device=gpu)
    stream = torch.cuda.current_stream(gpu).cuda_stream
    with torch.cuda.device(gpu):
        # empty batch, a non-positive divisor, a missing mean: rejected before any launch
        assert lib.gs_ssim_forward_noalloc(img1.data_ptr(), s1, img2.data_ptr(), s2, 0, 3, 32,
                                           48, 0, 1.0, mean.data_ptr(), None, None, None, None,
                                           0.0, None, stream) == -1
        assert lib.gs_ssim_forward_noalloc(img1.data_ptr(), s1, img2.data_ptr(), s2, 1, 3, 32,
                                           48, 0, 0.0, mean.data_ptr(), None, None, None, None,
                                           0.0, None, stream) == -1
        assert lib.gs_ssim_forward_noalloc(img1.data_ptr(), s1, img2.data_ptr(), s2, 1, 3, 32,
                                           48, 0, 1.0, None, None, None, None, None, 0.0, None,
                                           stream) == -1
        # past the limits: more than 65535 planes
        assert lib.gs_ssim_forward_noalloc(img1.data_ptr(), s1, img2.data_ptr(), s2, 65536, 1,
                                           32, 48, 0, 1.0, mean.data_ptr(), None, None, None,
                                           None, 0.0, None, stream) == -1
        # only some of the three maps
        maps = torch.empty((3, 32, 48), device=gpu)
        assert lib.gs_ssim_forward_noalloc(img1.data_ptr(), s1, img2.data_ptr(), s2, 1, 3, 32,
                                           48, 0, 1.0, mean.data_ptr(), maps.data_ptr(), None,
                                           None, None, 0.0, None, stream) == -1
        # without maps: the mean alone, as gs_ssim_forward gives it
        assert lib.gs_ssim_forward_noalloc(img1.data_ptr(), s1, img2.data_ptr(), s2, 1, 3, 32,
                                           48, 0, 1.0, mean.data_ptr(), None, None, None, None,
                                           0.0, None, stream) == 0
    torch.cuda.synchronize()
    m_ref, _, _ = _forward(gpu, img1, img2, 0, 1.0, torch.zeros(1, device=gpu), 0.0, False)
    assert helpers.same(mean.cpu(), m_ref)
