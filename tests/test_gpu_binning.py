"""GPU parity: compute_tile_intersection vs the numpy oracle, bit-exact.

Checked: indexing_offset, gaussian_ids_sorted, the sorted 64-bit keys
(tile << 32 | depth bits) and tiles_touched.  Cases: random splats with depth
ties, image sizes that are not tile multiples, tile sizes 8/16/32, the
reference's two constant fixtures (hand-derived layouts), empty inputs, a
fully culled frame, and the headline configuration's full size (1M Gaussians
at 1920x1080).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import helpers
import cuda_rasterizer as cr
from oracle import binning, preprocess

pytestmark = pytest.mark.gpu


def _random_splats(n, width, height, seed, rmax=40.0):
    g = np.random.default_rng(seed)
    pts = np.stack([g.uniform(-30, width + 30, n), g.uniform(-30, height + 30, n)], 1).astype(np.float32)
    radii = g.uniform(0.5, rmax, (n, 2)).astype(np.float32)
    depths = g.uniform(0.2, 10.0, n).astype(np.float32)
    if n > 3:
        depths[::5] = depths[3]  # many exact depth ties
    mask = g.uniform(size=n) > 0.15
    return pts, radii, depths, mask


def _check(gpu, pts, radii, depths, mask, width, height, tile):
    ref_off, ref_ids, ref_keys, ref_counts = binning.tile_layout(pts, radii, depths, mask, width,
                                                                 height, tile)
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)  # noqa: E731
    off, ids, keys, touched = cr.compute_tile_intersection_debug(d(pts), d(radii), d(depths),
                                                                 d(mask), width, height, tile)
    assert np.array_equal(off.cpu().numpy(), ref_off)
    assert np.array_equal(ids.cpu().numpy(), ref_ids)
    assert np.array_equal(keys.cpu().numpy().view(np.uint64), ref_keys)
    assert np.array_equal(touched.cpu().numpy().astype(np.int64), ref_counts)
    off2, ids2 = cr.compute_tile_intersection(d(pts), d(radii), d(depths), d(mask), width, height,
                                              tile)
    assert torch.equal(off2, off) and torch.equal(ids2, ids)
    return len(ref_ids)


@pytest.mark.parametrize("n,width,height,tile", [
    (1, 64, 64, 16),
    (1000, 64, 48, 16),
    (5000, 100, 37, 16),
    (20000, 256, 256, 16),
    (3000, 64, 64, 8),
    (3000, 200, 90, 32),
    (50000, 800, 800, 16),
    (30000, 2048, 2048, 16),  # 16384 tiles: the largest grid the fused tile scan takes
    (30000, 2048, 2064, 16),  # 16512 tiles: one tile row past it (separate scan)
])
def test_layout_random_bitexact(gpu, n, width, height, tile):
    pts, radii, depths, mask = _random_splats(n, width, height, seed=n + width)
    k = _check(gpu, pts, radii, depths, mask, width, height, tile)
    assert k > 0


@pytest.mark.parametrize("width,height,tile", [(256, 256, 16), (2560, 1600, 8)])
def test_totals_copy_fallback_bitexact(gpu, monkeypatch, width, height, tile):
    """The host layer reads K and M from pinned host memory the device writes;
    where that memory is not mapped for the device it keeps them in device
    memory and copies them.  Both give the same layouts (one-pass and general
    level 1)."""
    pts, radii, depths, mask = _random_splats(20000, width, height, seed=width + tile)
    monkeypatch.setattr(cr, "_pinned_device_pointer", lambda t: None)
    assert _check(gpu, pts, radii, depths, mask, width, height, tile) > 0


def test_layout_many_supertiles_bitexact(gpu):
    """A grid of more than 256 supertiles (40 x 25 at 2560x1600, tile 8): the
    level-1 sort over several radix passes instead of the one-pass count."""
    n, width, height, tile = 20000, 2560, 1600, 8
    pts, radii, depths, mask = _random_splats(n, width, height, seed=7, rmax=24.0)
    assert _check(gpu, pts, radii, depths, mask, width, height, tile) > 0


@pytest.mark.parametrize("name", ["multitile", "truncated"])
def test_layout_reference_fixtures(gpu, name):
    f = helpers.fixture_tensors(name)
    off, ids = cr.compute_tile_intersection(f["points_image"].to(gpu), f["radii"].to(gpu),
                                            f["depths"].to(gpu), f["mask"].to(gpu), f["width"],
                                            f["height"], f["tile_size"])
    assert off.cpu().tolist() == f["expected_indexing_offset"]
    assert ids.cpu().tolist() == f["expected_gaussian_ids_sorted"]


def test_layout_empty_inputs(gpu):
    z2 = torch.zeros(0, 2, device=gpu)
    off, ids = cr.compute_tile_intersection(z2, z2, torch.zeros(0, device=gpu),
                                            torch.zeros(0, dtype=torch.bool, device=gpu), 40, 40, 16)
    assert off.cpu().tolist() == [0] * 9 and ids.numel() == 0
    pts, radii, depths, _ = _random_splats(100, 40, 40, seed=3)
    none = np.zeros(100, dtype=bool)
    k = _check(gpu, pts, radii, depths, none, 40, 40, 16)
    assert k == 0


def test_layout_from_projection_end_to_end(gpu):
    """Projection on the GPU then binning on the GPU equals the oracle's chain
    (the projection is bit-exact, so the integer layout must be too)."""
    p, cam, _ = helpers.scene_orbit(30_000, 800, 800, 1100.0, seed=4)
    scales, quats, opac = helpers.activated(p)
    args = (cam["w2c"], cam["K"], 0.01, 100.0, 1 / 255, 0.5, 128.0, cam["width"], cam["height"])
    pts, depths, _, _, radii, mask = preprocess.project_points(p["means"], scales, quats, opac, *args)
    ref = binning.tile_layout(pts.detach().numpy(), radii.detach().numpy(), depths.detach().numpy(),
                              mask.numpy(), 800, 800, 16)
    d = lambda t: t.to(gpu)  # noqa: E731
    g_pts, g_depths, _, _, g_radii, g_mask = cr.project_points(
        d(p["means"]), d(scales), d(quats), d(opac), d(args[0]), d(args[1]), *args[2:])
    off, ids, keys, touched = cr.compute_tile_intersection_debug(g_pts, g_radii, g_depths, g_mask,
                                                                 800, 800, 16)
    assert np.array_equal(off.cpu().numpy(), ref[0])
    assert np.array_equal(ids.cpu().numpy(), ref[1])
    assert np.array_equal(keys.cpu().numpy().view(np.uint64), ref[2])


def test_layout_headline_size_bitexact(gpu):
    """Full-size check at the headline configuration (1M
    Gaussians, 1920x1080): projection on the GPU, then the GPU layout against the
    numpy oracle on the GPU's own projected values."""
    import bench

    scene = bench.config3()
    p = scene["params"]
    scales, quats, opac = helpers.activated(p)
    cam = scene["camera"]
    d = lambda t: t.to(gpu)  # noqa: E731
    g_pts, g_depths, _, _, g_radii, g_mask = cr.project_points(
        d(p["means"]), d(scales), d(quats), d(opac), d(cam["w2c"]), d(cam["K"]), cam["near"], 100.0,
        1 / 255, 0.5, 128.0, cam["width"], cam["height"])
    pts, radii, depths, mask = (t.cpu().numpy() for t in (g_pts, g_radii, g_depths, g_mask))
    k = _check(gpu, pts, radii, depths, mask, cam["width"], cam["height"], 16)
    assert k > 5_000_000


@pytest.mark.parametrize("width,height", [(640, 480), (2560, 1600)])
def test_single_call_count_equals_two_phases(gpu, width, height):
    """gs_bin_count (one call) leaves the same workspace state and totals as
    gs_bin_count_begin + gs_bin_count_finish, which compute_tile_intersection
    uses: gs_bin_sort after it gives the identical layout (one-pass and general
    level 1)."""
    import ctypes

    from cuda_rasterizer import _lib

    pts, radii, depths, mask = (torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
                                for a in _random_splats(20000, width, height, seed=9))
    off2, ids2 = cr.compute_tile_intersection(pts, radii, depths, mask, width, height, 16)
    lib = _lib.load()
    n = pts.shape[0]
    sz = ctypes.c_size_t(0)
    assert lib.gs_bin_count_workspace_size(n, ctypes.byref(sz)) == 0
    ws = torch.empty(sz.value, dtype=torch.uint8, device=gpu)
    totals = torch.empty(2, dtype=torch.int64, device=gpu)
    stream = torch.cuda.current_stream(gpu).cuda_stream
    assert lib.gs_bin_count(pts.data_ptr(), radii.data_ptr(), depths.data_ptr(), mask.data_ptr(),
                            n, width, height, 16, ws.data_ptr(), sz.value, totals.data_ptr(),
                            stream) == 0
    k, m = (int(v) for v in totals.tolist())
    assert k == ids2.numel()
    sz2 = ctypes.c_size_t(0)
    assert lib.gs_bin_sort_workspace_size(n, k, m, width, height, 16, ctypes.byref(sz2)) == 0
    ws2 = torch.empty(max(sz2.value, 1), dtype=torch.uint8, device=gpu)
    off = torch.empty_like(off2)
    ids = torch.empty(k, dtype=torch.int32, device=gpu)
    assert lib.gs_bin_sort(pts.data_ptr(), radii.data_ptr(), depths.data_ptr(), n, width, height,
                           16, k, m, ws.data_ptr(), ws2.data_ptr(), sz2.value, off.data_ptr(),
                           ids.data_ptr(), None, None, stream) == 0
    assert torch.equal(off, off2) and torch.equal(ids, ids2)


def _launch_order_ref(off, k, n_tiles):
    """Per XCD range (8 ranges: base + (x < rem) tiles from x * base + min(x, rem)),
    the tiles by (bit length of the list length, tile)."""
    lens = np.diff(np.append(off.astype(np.int64), k))
    bits = np.array([int(v).bit_length() for v in lens], dtype=np.int64)
    out = np.empty(n_tiles, dtype=np.int64)
    base, rem = divmod(n_tiles, 8)
    for x in range(8):
        st, ln = x * base + min(x, rem), base + (1 if x < rem else 0)
        t = np.arange(st, st + ln)
        out[st:st + ln] = t[np.lexsort((t, bits[t]))]
    return out


@pytest.mark.parametrize("n,width,height,tile,culled", [
    (1, 32, 32, 16, False),        # 4 tiles: ranges of 0 and 1 tiles
    (3000, 64, 64, 16, False),     # 16 tiles
    (3000, 64, 64, 8, False),
    (50000, 800, 800, 16, False),
    (200000, 1920, 1080, 16, False),  # 1020 tiles per range: two chunks of 512
    (100000, 3840, 2160, 16, False),  # 4050 tiles per range
    (5000, 640, 480, 16, True),    # K = 0: tile order
])
def test_launch_order(gpu, n, width, height, tile, culled):
    """gs_bin_sort_ordered: the same layout as gs_bin_sort, and a launch order that
    sorts each XCD range stably by the bit length of its tiles' list lengths."""
    pts, radii, depths, mask = _random_splats(n, width, height, seed=n + width)
    if culled:
        mask[:] = False
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)  # noqa: E731
    off, ids, order = cr.compute_tile_intersection_ordered(d(pts), d(radii), d(depths), d(mask),
                                                           width, height, tile)
    off2, ids2 = cr.compute_tile_intersection(d(pts), d(radii), d(depths), d(mask), width, height,
                                              tile)
    assert torch.equal(off, off2) and torch.equal(ids, ids2)
    n_tiles = off.shape[0]
    ref = _launch_order_ref(off.cpu().numpy(), ids.shape[0], n_tiles)
    assert np.array_equal(order.cpu().numpy().astype(np.int64), ref)
    if culled:
        assert ids.shape[0] == 0 and np.array_equal(ref, np.arange(n_tiles))
    elif n >= 1000:  # lists of many lengths, so the order is not trivial
        assert len(set(np.diff(np.append(off.cpu().numpy(), ids.shape[0])).tolist())) > 3


def _key_range(depths, mask):
    bits = depths.view(np.uint32)
    live = bits[mask]
    return int(live.min()), int(live.max())


@pytest.mark.parametrize("case", ["derived", "previous", "below", "above", "narrow", "shift0",
                                  "top"])
@pytest.mark.parametrize("width,height,tile", [(256, 256, 16), (2560, 1600, 8)])
def test_depth_hint_layouts_bitexact(gpu, monkeypatch, case, width, height, tile):
    """The depth sort's bucket transform (gs_bin_count_begin_hinted): derived on
    the device, taken from the previous call's key range, or forced far from the
    keys -- a range below every key (all in the last bucket), above every key
    (all in bucket 0), one covering a tenth of the span (both clamps), shift 0
    (a 16-bit window of single key values) and the top of the key space.  Every
    transform gives the oracle's layout bit for bit; the crowded buckets run the
    segment sort's global-memory path.  Both level-1 paths (one pass and, at
    2560x1600 with 8-pixel tiles, general)."""
    pts, radii, depths, mask = _random_splats(30000, width, height, seed=7 + width)
    kmin, kmax = _key_range(depths, mask)
    span = kmax - kmin
    forced = {"below": (max(kmin - 2 * span - 100, 0), 0),
              "above": (kmax + 1, 4),
              "narrow": (kmin + span // 2, max((span // 10).bit_length() - 16, 0)),
              "shift0": (kmin + span // 3, 0),
              "top": (0xFFFFFF00, 16)}
    if case == "derived":
        monkeypatch.setattr(cr, "DEPTH_HINTS", False)
    elif case == "previous":
        _check(gpu, pts, radii, depths, mask, width, height, tile)  # leaves this range as hint
        assert cr._DEPTH_RANGE[gpu.index] == (kmin, kmax)
    else:
        monkeypatch.setattr(cr, "_FORCED_DEPTH_HINT", forced[case])
    assert _check(gpu, pts, radii, depths, mask, width, height, tile) > 0
    if case != "derived":
        assert cr._DEPTH_RANGE[gpu.index] == (kmin, kmax)  # the totals report the key range


def test_depth_hint_rejects_wide_shift(gpu, monkeypatch):
    """A hint shift above 16 is rejected before any launch."""
    pts, radii, depths, mask = _random_splats(100, 64, 64, seed=3)
    monkeypatch.setattr(cr, "_FORCED_DEPTH_HINT", (0, 17))
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)  # noqa: E731
    with pytest.raises(cr.RasterizerError):
        cr.compute_tile_intersection(d(pts), d(radii), d(depths), d(mask), 64, 64, 16)


def _capped(gpu, pts, radii, depths, mask, width, height, caps):
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)  # noqa: E731
    cr._CAPACITY[(gpu.index, width, height, 16)] = caps
    out = cr.tile_intersection_capped(d(pts), d(radii), d(depths), d(mask), width, height, 16)
    ok = out[3].ok() if out[3] is not None else None
    return out[:3], ok


@pytest.mark.parametrize("width,height", [(256, 256), (800, 600), (2048, 2048)])
def test_capped_sort_equals_exact_lists_shifted(gpu, monkeypatch, width, height):
    """gs_bin_sort_capped, queued before the host reads K and M: with room to
    spare, each tile's list is the exact one and the offsets are the exact ones
    shifted by capacity - K, so the lists end at the capacity; the launch order
    is the same.  Also with capacities exactly K and M (no spare room)."""
    monkeypatch.setattr(cr, "_CAPACITY", dict(cr._CAPACITY))
    pts, radii, depths, mask = _random_splats(40000, width, height, seed=width + 1)
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)  # noqa: E731
    off, ids, order = cr.compute_tile_intersection_ordered(d(pts), d(radii), d(depths), d(mask),
                                                           width, height, 16)
    k = ids.numel()
    ref_off, ref_ids, _, _ = binning.tile_layout(pts, radii, depths, mask, width, height, 16)
    assert np.array_equal(ids.cpu().numpy(), ref_ids)
    for caps in [(k + 12345, 10**7), (k, None)]:
        if caps[1] is None:  # the exact M: the smallest capacity that fits
            lo, hi = 1, 10**7
            while lo < hi:  # M from the capped call's own check
                mid = (lo + hi) // 2
                _, fits = _capped(gpu, pts, radii, depths, mask, width, height, (k, mid))
                lo, hi = (lo, mid) if fits else (mid + 1, hi)
            caps = (k, lo)
            _, fits = _capped(gpu, pts, radii, depths, mask, width, height, (k, lo - 1))
            assert not fits
        (c_off, c_ids, c_order), fits = _capped(gpu, pts, radii, depths, mask, width, height,
                                                caps)
        assert fits
        shift = caps[0] - k
        assert c_ids.numel() == caps[0]
        assert torch.equal(c_off.cpu() - shift, off.cpu())
        assert torch.equal(c_ids[shift:].cpu(), ids.cpu())
        assert torch.equal(c_order, order)


def test_capped_sort_overflow_leaves_empty_lists(gpu, monkeypatch):
    """Capacities below K (or M): check.ok() is False and every tile is empty at
    the capacity, so a blend over the result reads nothing; the next exact call
    grows the capacities so that a capped call fits again."""
    monkeypatch.setattr(cr, "_CAPACITY", dict(cr._CAPACITY))
    pts, radii, depths, mask = _random_splats(20000, 320, 240, seed=5)
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)  # noqa: E731
    off, ids, _ = cr.compute_tile_intersection_ordered(d(pts), d(radii), d(depths), d(mask), 320,
                                                       240, 16)
    k = ids.numel()
    for caps in [(k - 1, 10**7), (k + 10, 1)]:
        (c_off, c_ids, c_order), fits = _capped(gpu, pts, radii, depths, mask, 320, 240, caps)
        assert fits is False
        assert bool((c_off == caps[0]).all())
        cr.check_forward_order(c_order, c_off.numel())
    cr._CAPACITY.pop((gpu.index, 320, 240, 16))
    out = cr.tile_intersection_capped(d(pts), d(radii), d(depths), d(mask), 320, 240, 16)
    assert out[3] is None and torch.equal(out[1], ids)  # first call: exact sizes
    out = cr.tile_intersection_capped(d(pts), d(radii), d(depths), d(mask), 320, 240, 16)
    assert out[3] is not None and out[3].ok()
    shift = out[1].numel() - k
    assert shift > 0 and torch.equal(out[1][shift:], ids) and torch.equal(out[0] - shift, off)
