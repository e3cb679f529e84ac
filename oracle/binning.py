"""Oracle binning: tile rectangles, 64-bit keys, stable sort, tile ranges (numpy).

Test infrastructure only (see oracle/__init__.py).

Integer semantics of compute_tile_intersection (src/cuda/rasterizer.cpp:292-359,
src/cuda/kernel.cu:784-914) as pinned by the reference's layout test
(scripts/check_cuda_gradients.py:57-131):
  u_min = clamp(floor(u - r_u), 0, W-1), u_max = clamp(floor(u + r_u), 0, W-1)
  (v likewise), tile rect [u_min/ts .. u_max/ts] x [v_min/ts .. v_max/ts],
  key = tile_id << 32 | bits(depth), entries in Gaussian order with row-major
  tiles, stable ascending sort (ties by Gaussian index),
  indexing_offset[t] = number of entries with tile < t.
"""

from __future__ import annotations

import numpy as np


def tile_rects(points_image: np.ndarray, radii: np.ndarray, width: int, height: int,
               tile_size: int):
    """Per-Gaussian inclusive tile bounds (tx0, tx1, ty0, ty1) and a validity flag.
    fp32 arithmetic as in src/cuda/kernel.cu:795-817 / src/torch_rasterizer.py:160-169."""
    p = np.asarray(points_image, dtype=np.float32)
    r = np.asarray(radii, dtype=np.float32)
    u, v = p[:, 0], p[:, 1]
    ru, rv = r[:, 0], r[:, 1]
    with np.errstate(invalid="ignore"):
        u0 = np.clip(np.floor(u - ru), 0, width - 1).astype(np.int64)
        u1 = np.clip(np.floor(u + ru), 0, width - 1).astype(np.int64)
        v0 = np.clip(np.floor(v - rv), 0, height - 1).astype(np.int64)
        v1 = np.clip(np.floor(v + rv), 0, height - 1).astype(np.int64)
    ok = (u0 <= u1) & (v0 <= v1)
    return u0 // tile_size, u1 // tile_size, v0 // tile_size, v1 // tile_size, ok


def tiles_touched(points_image, radii, mask, width, height, tile_size) -> np.ndarray:
    """count_tiles_kernel (src/cuda/kernel.cu:784-818)."""
    tx0, tx1, ty0, ty1, ok = tile_rects(points_image, radii, width, height, tile_size)
    n = (tx1 - tx0 + 1) * (ty1 - ty0 + 1)
    return np.where(np.asarray(mask, dtype=bool) & ok, n, 0).astype(np.int64)


def depth_bits(depths) -> np.ndarray:
    """Zero-extended fp32 bit pattern (src/cuda/kernel.cu:857-859)."""
    return np.asarray(depths, dtype=np.float32).view(np.uint32).astype(np.uint64)


def tile_layout(points_image, radii, depths, mask, width, height, tile_size=16):
    """Vectorised compute_tile_intersection.

    Returns (indexing_offset int32[T], gaussian_ids_sorted int32[K],
    sorted_keys uint64[K], tiles_touched int64[N]).
    """
    tiles_x = (width + tile_size - 1) // tile_size
    tiles_y = (height + tile_size - 1) // tile_size
    n_tiles = tiles_x * tiles_y
    tx0, tx1, ty0, ty1, ok = tile_rects(points_image, radii, width, height, tile_size)
    counts = tiles_touched(points_image, radii, mask, width, height, tile_size)
    total = int(counts.sum())
    gid = np.repeat(np.arange(len(counts), dtype=np.int64), counts)
    # position of each entry inside its Gaussian's rectangle (row-major)
    starts = np.cumsum(counts) - counts
    local = np.arange(total, dtype=np.int64) - np.repeat(starts, counts)
    nx = (tx1 - tx0 + 1)[gid]
    tx = tx0[gid] + local % nx
    ty = ty0[gid] + local // nx
    tile = ty * tiles_x + tx
    keys = (tile.astype(np.uint64) << np.uint64(32)) | depth_bits(depths)[gid]
    order = np.argsort(keys, kind="stable")  # stable: ties keep Gaussian order
    keys_sorted = keys[order]
    ids_sorted = gid[order].astype(np.int32)
    tiles_sorted = (keys_sorted >> np.uint64(32)).astype(np.int64)
    offsets = np.searchsorted(tiles_sorted, np.arange(n_tiles), side="left").astype(np.int32)
    return offsets, ids_sorted, keys_sorted, counts


def tile_layout_loop(points_image, radii, depths, mask, width, height, tile_size=16):
    """Pure-Python restatement of build_reference_tile_layout
    (scripts/check_cuda_gradients.py:57-131), for small inputs.  Returns
    (indexing_offset list[int], gaussian_ids_sorted list[int])."""
    import math
    import struct

    def f32(x):
        return struct.unpack("f", struct.pack("f", x))[0]

    tiles_x = (width + tile_size - 1) // tile_size
    tiles_y = (height + tile_size - 1) // tile_size
    unique_tiles = tiles_x * tiles_y
    entries = []
    for g in range(len(points_image)):
        if not bool(mask[g]):
            continue
        u, v = float(points_image[g][0]), float(points_image[g][1])
        ru, rv = float(radii[g][0]), float(radii[g][1])
        u0 = min(max(0, math.floor(f32(u - ru))), width - 1)
        u1 = min(max(0, math.floor(f32(u + ru))), width - 1)
        v0 = min(max(0, math.floor(f32(v - rv))), height - 1)
        v1 = min(max(0, math.floor(f32(v + rv))), height - 1)
        if u0 > u1 or v0 > v1:
            continue
        bits = struct.unpack("I", struct.pack("f", float(depths[g])))[0]
        for ty in range(v0 // tile_size, v1 // tile_size + 1):
            for tx in range(u0 // tile_size, u1 // tile_size + 1):
                entries.append((ty * tiles_x + tx, bits, g))
    entries.sort(key=lambda e: (e[0], e[1]))  # Python's sort is stable
    total = len(entries)
    offsets = [total] * unique_tiles
    if total == 0:
        return [0] * unique_tiles, []
    prev = None
    for idx, (tile, _, _) in enumerate(entries):
        if prev is None:
            for t in range(tile + 1):
                offsets[t] = 0
            prev = tile
        elif tile != prev:
            for t in range(prev + 1, tile + 1):
                offsets[t] = idx
            prev = tile
    for t in range(prev + 1, unique_tiles):
        offsets[t] = total
    return offsets, [e[2] for e in entries]
