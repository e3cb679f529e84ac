"""CPU tests of the C-ABI library and the Python host layer (no GPU calls)."""

from __future__ import annotations

import ctypes
import os
import re

import pytest
import torch

import helpers  # noqa: F401  (sets sys.path via conftest)
import cuda_rasterizer
from cuda_rasterizer import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "gs_rasterizer.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gs_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail(f"{_lib.LIB_PATH} missing: run __graft_entry__.build() first")
    return _lib.load()


def test_header_declares_the_seven_reference_stages():
    names = declared_functions()
    for required in ["gs_project_points", "gs_project_points_backward", "gs_evaluate_sh",
                     "gs_evaluate_sh_backward", "gs_bin_count", "gs_bin_sort", "gs_rasterize",
                     "gs_rasterize_backward"]:
        assert required in names


def test_library_exports_every_declared_symbol(lib):
    raw = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(raw, n)]
    assert not missing, missing
    assert set(_lib.SIGNATURES) | {"gs_status_string"} >= set(declared_functions())


def test_abi_version_and_status_strings(lib):
    assert lib.gs_abi_version() == 20
    assert lib.gs_status_string(0) == b"success"
    for code in (-1, -2, -3, -4):
        assert lib.gs_status_string(code) not in (b"", b"unknown status")
    assert lib.gs_status_string(-99) == b"unknown status"


def test_host_device_pointer_rejects_null(lib):
    out = ctypes.c_void_p(123)
    assert lib.gs_host_device_pointer(None, ctypes.byref(out)) == -1
    assert lib.gs_host_device_pointer(ctypes.c_void_p(256), None) == -1


def test_workspace_queries(lib):
    sz = ctypes.c_size_t(0)
    assert lib.gs_bin_count_workspace_size(0, ctypes.byref(sz)) == 0
    small = sz.value
    assert lib.gs_bin_count_workspace_size(1_000_000, ctypes.byref(sz)) == 0
    assert sz.value >= 1_000_000 * 36 and sz.value > small
    # the sort workspace scales with the supertile entries M, not with the keys K:
    # two 16-bit key buffers + two 32-bit id buffers per entry, plus 64 counters
    # per 256 entries
    assert lib.gs_bin_sort_workspace_size(1000, 20_000_000, 1_000_000, 1920, 1080, 16,
                                          ctypes.byref(sz)) == 0
    assert 1_000_000 * 12 <= sz.value < 20_000_000 * 4
    assert lib.gs_bin_sort_workspace_size(1000, 20_000_000, 1_000_000, 1920, 0, 16,
                                          ctypes.byref(sz)) == -1
    assert lib.gs_bin_count_workspace_size(-1, ctypes.byref(sz)) == -1


def test_invalid_arguments_rejected_on_host(lib):
    null = None
    # negative sizes / bad image sizes never reach the device
    assert lib.gs_project_points(*([null] * 6), -1, 0.01, 100.0, 0.0, 0.5, 128.0, 64, 64,
                                 *([null] * 6), null) == -1
    assert lib.gs_project_points(*([null] * 6), 10, 0.01, 100.0, 0.0, 0.5, 128.0, 0, 64,
                                 *([null] * 6), null) == -1
    assert lib.gs_project_points(*([null] * 6), 10, 0.01, 100.0, 0.0, 0.5, 128.0, 64, 64,
                                 *([null] * 6), null) == -1  # null buffers
    assert lib.gs_evaluate_sh(*([null] * 5), -3, 0, null, null) == -1
    # the colour launch for a second stream: the same checks as gs_evaluate_sh_render
    assert lib.gs_evaluate_sh_render_beside(*([null] * 5), 10, null, null) == -1
    assert lib.gs_evaluate_sh_render_beside(*([null] * 5), -1, null, null) == -1
    assert lib.gs_evaluate_sh_render_beside(*([null] * 5), 0, null, null) == 0  # nothing to do
    # the colour launch that also writes the colour-gradient cache: the cache is
    # required and must be 8-byte aligned (rows of 10 floats read as float2)
    some = ctypes.c_void_p(4096)  # never dereferenced: every call below is rejected first
    assert lib.gs_evaluate_sh_render_cache(*([some] * 5), 10, 0, some, null, null) == -1
    assert lib.gs_evaluate_sh_render_cache(*([some] * 5), 10, 0, some,
                                           ctypes.c_void_p(4100), null) == -1
    assert lib.gs_evaluate_sh_render_cache(*([null] * 5), 0, 1, null, null, null) == 0
    assert lib.gs_evaluate_sh_render_cache(*([null] * 5), -1, 0, null, null, null) == -1
    assert lib.gs_rasterize(null, null, 4, 10, *([null] * 4), 10, 32, 32, 16, 1e-4, 1e-4, 9.21,
                            null, null) == -1
    assert lib.gs_rasterize(null, null, 4, 2**31, *([null] * 4), 10, 32, 32, 16, 1e-4, 1e-4,
                            9.21, null, null) == -3
    assert lib.gs_rasterize(null, null, 4, 10, *([null] * 4), 10, 64, 64, 64, 1e-4, 1e-4, 9.21,
                            null, null) == -4  # 64x64 tile: more than 1024 threads
    assert lib.gs_rasterize(null, null, 4, 10, *([null] * 4), 10, 32, 32, 16, 1e-4,
                            float("nan"), 9.21, null, null) == -1  # NaN threshold
    # more offset entries than the image has tiles
    assert lib.gs_rasterize(null, null, 5, 0, *([null] * 4), 0, 32, 32, 16, 1e-4, 1e-4, 9.21,
                            null, null) == -1
    assert lib.gs_bin_sort(null, null, null, 10, 64, 64, 16, 2**31, 5, null, null, 0, null, null,
                           null, null, null) == -3
    assert lib.gs_bin_sort(null, null, null, 10, 64, 64, 16, 5, 6, null, null, 0, null, null,
                           null, null, null) == -1  # more supertile entries than keys
    assert lib.gs_bin_sort_ordered(null, null, null, 10, 64, 64, 16, 5, 5, null, null, 0, null,
                                   null, null, null, null, null) == -1  # launch_order required
    fake = ctypes.c_void_p(256)  # never dereferenced: the key count is rejected first
    assert lib.gs_bin_sort_ordered(null, null, null, 10, 64, 64, 16, 2**31, 5, null, null, 0,
                                   null, null, null, null, fake, null) == -3
    sz = ctypes.c_size_t(0)
    assert lib.gs_bin_count(null, null, null, null, 10, 64, 64, 16, null, 0, null, null) == -1
    # training-loop entries: bad hyper-parameters, missing buffers, bad widths
    t = _lib.GsAdamTensor(None, None, None, None, 10, 0.1, 1.0)
    assert lib.gs_adam_step(ctypes.byref(t), 1, 0.9, 0.999, 1e-15, null) == -1  # null param
    assert lib.gs_adam_step(None, 0, 1.0, 0.999, 1e-15, null) == -1  # beta1 = 1
    assert lib.gs_adam_step(None, 0, 0.9, float("nan"), 1e-15, null) == -1
    assert lib.gs_adam_step(None, 0, 0.9, 0.999, 1e-15, null) == 0  # empty list
    assert lib.gs_accumulate_grad2d(null, null, 10, 0, 64, null, null, null) == -1
    assert lib.gs_accumulate_grad2d(null, null, 10, 64, 64, null, null, null) == -1
    g = _lib.GsGatherTensor(None, None, None, 0, 0)
    assert lib.gs_gather_rows(10, None, None, ctypes.byref(g), 1, null) == -1
    assert lib.gs_gather_rows(-1, None, None, None, 0, null) == -1
    # SSIM entries: sizes, plane limit, null buffers, partial map sets
    assert lib.gs_ssim_workspace_size(1, 3, 64, 64, ctypes.byref(sz)) == 0 and sz.value > 0
    assert lib.gs_ssim_workspace_size(0, 3, 64, 64, ctypes.byref(sz)) == -1
    assert lib.gs_ssim_workspace_size(256, 256, 64, 64, ctypes.byref(sz)) == -1  # > 65535 planes
    st = (ctypes.c_int64 * 4)(3 * 64 * 64, 64 * 64, 64, 1)
    assert lib.gs_ssim_forward(null, st, null, st, 1, 3, 64, 64, 1, 1.0, null, null, null, null,
                               null, 0.0, null, null, 0, null) == -1
    fake = ctypes.c_void_p(256)  # never dereferenced: the host checks fail first
    assert lib.gs_ssim_forward(fake, st, fake, st, 1, 3, 64, 64, 1, 1.0, fake, fake, null, null,
                               null, 0.0, null, fake, 1 << 20, null) == -1  # maps all or none
    assert lib.gs_ssim_forward(fake, st, fake, st, 1, 3, 64, 64, 1, 0.0, fake, null, null, null,
                               null, 0.0, null, fake, 1 << 20, null) == -1  # divisor 0
    assert lib.gs_ssim_forward(fake, st, fake, st, 1, 3, 64, 64, 1, 1.0, fake, null, null, null,
                               null, 0.2, fake, fake, 1 << 20, null) == -1  # loss without other
    assert lib.gs_ssim_forward(fake, st, fake, st, 1, 3, 64, 64, 1, 1.0, fake, null, null, null,
                               null, 0.0, null, fake, 0, null) == -2  # workspace too small
    # a row whose last element lies 2^30 or more elements past its first: unsupported (-4)
    # (a 33-column row with column stride 2^25, within the 2^31 plane limit)
    wide = (ctypes.c_int64 * 4)(3 * 64 * 64, 64 * 64, 64, 1 << 25)
    assert lib.gs_ssim_forward(fake, wide, fake, st, 1, 3, 64, 33, 1, 1.0, fake, null, null, null,
                               null, 0.0, null, fake, 1 << 20, null) == -4
    assert lib.gs_ssim_backward(fake, fake, st, fake, st, 1, 3, 64, 64, 1.0, fake, fake, null,
                                1.0, fake, st, null) == -1
    # fused blend entries: missing display / target / tile sums, grids not covering the image,
    # a NaN loss weight
    blend_args = (null, null, 16, 10, *([null] * 4), 10, 64, 64, 16, 1e-4, 1e-4, 9.21)
    assert lib.gs_rasterize_display_l1(*blend_args, fake, fake, null, fake, null, null, null, 0,
                                       null, null) == -1  # no display
    assert lib.gs_rasterize_display_l1(null, null, 15, 10, *([null] * 4), 10, 64, 64, 16, 1e-4,
                                       1e-4, 9.21, fake, fake, fake, fake, null, null, null, 0,
                                       null, null) == -1  # 15 offsets for a 16-tile image
    assert lib.gs_l1_finish(fake, 16, 0, fake, null) == -1
    assert lib.gs_rasterize_l1_backward(fake, fake, fake, *blend_args, *([fake] * 4), 1,
                                        float("nan"), null, null, null) == -1


def test_python_layer_refuses_cpu_tensors():
    """No CPU fallback: the product path raises on host tensors."""
    n = 4
    with pytest.raises(RuntimeError, match="GPU only"):
        cuda_rasterizer.project_points(torch.zeros(n, 3), torch.ones(n, 3), torch.zeros(n, 4),
                                       torch.ones(n), torch.eye(4), torch.eye(3), 0.01, 100.0,
                                       1 / 255, 0.5, 128.0, 16, 16)
    with pytest.raises(RuntimeError, match="GPU only"):
        cuda_rasterizer.compute_tile_intersection(torch.zeros(n, 2), torch.ones(n, 2),
                                                  torch.ones(n), torch.ones(n, dtype=torch.bool),
                                                  16, 16, 16)


def test_tile_schedule_buffers_are_checked():
    """The schedule buffer must be a contiguous int32 tensor of at least
    gs_tile_schedule_size(n_tiles) elements: per tile its work, launch slot,
    checkpoint count, 3 checkpoint positions, 3 work counts and 4 segment-list
    entries, 8 list lengths (padded to 16 bytes), then 3 checkpoints of 256
    (T, r, g, b) pixels per tile."""
    need = cuda_rasterizer.schedule_size(8)
    assert need == 112 + 8 * 3 * 256 * 4
    assert cuda_rasterizer.schedule_size(7) == 100 + 7 * 3 * 256 * 4  # 99 padded to 100
    assert cuda_rasterizer.schedule_size(0) == 2
    assert cuda_rasterizer.schedule_size(6144) == (13 * 6144 + 8 + 3) // 4 * 4 + 6144 * 3072
    assert cuda_rasterizer.schedule_size(6145) == 2 * 6145  # no checkpoints on larger grids
    out = ctypes.c_size_t(0)
    assert _lib.load().gs_tile_schedule_size(-1, ctypes.byref(out)) != 0
    assert _lib.load().gs_tile_schedule_size(8, None) != 0
    cpu = torch.device("cpu")
    cuda_rasterizer._check_schedule(torch.zeros(need, dtype=torch.int32), 8, cpu, "probe")
    for bad in (torch.zeros(need - 1, dtype=torch.int32), torch.zeros(need, dtype=torch.int64),
                torch.zeros(2 * need, dtype=torch.int32)[::2], [0] * need):
        with pytest.raises(RuntimeError, match="schedule"):
            cuda_rasterizer._check_schedule(bad, 8, cpu, "probe")


def test_status_to_exception():
    with pytest.raises(_lib.RasterizerError, match="invalid argument"):
        _lib.check(-1, "probe")


@pytest.mark.parametrize("n_tiles", [1, 7, 8, 256, 2500, 8160, 8163])
def test_check_forward_order_accepts_range_permutations(n_tiles):
    """Each XCD range [x*b + min(x, r), ...) of b, r = divmod(n_tiles, 8), shuffled
    within itself, is a valid launch order; the identity too."""
    g = torch.Generator().manual_seed(n_tiles)
    b, r = divmod(n_tiles, 8)
    starts = [x * b + min(x, r) for x in range(9)]
    parts = [starts[x] + torch.randperm(starts[x + 1] - starts[x], generator=g)
             for x in range(8)]
    order = torch.cat(parts).to(torch.int32)
    cuda_rasterizer.check_forward_order(order, n_tiles)
    cuda_rasterizer.check_forward_order(torch.arange(n_tiles, dtype=torch.int32), n_tiles)


@pytest.mark.parametrize("n_tiles", [16, 2500, 8160])
def test_check_forward_order_rejects_broken_orders(n_tiles):
    ident = torch.arange(n_tiles, dtype=torch.int32)
    dup = ident.clone()
    dup[1] = dup[0]  # a tile twice, another never
    across = ident.clone()
    b, r = divmod(n_tiles, 8)
    first_end = b + (1 if r else 0)
    across[0], across[first_end] = across[first_end].item(), across[0].item()  # swaps two ranges
    out = ident.clone()
    out[-1] = n_tiles  # past the grid
    neg = ident.clone()
    neg[0] = -1
    for bad in (dup, across, out, neg):
        with pytest.raises(cuda_rasterizer.RasterizerError):
            cuda_rasterizer.check_forward_order(bad, n_tiles)
