"""GPU parity of the fused training step (cuda_rasterizer.fused.render_l1) and
its kernels: activations, L1 loss in the blend, L1-seeded blend backward.

References: the drop-in path (PyTorch activations of scripts/train.py:135-143,
render(), PyTorch l1_loss on the /255 image) on the GPU, and the CPU oracle.
Tolerances: activations within 2 ulp-level relative error (device expf/sqrt vs
PyTorch's); loss relative 1e-5 (summation order); image max abs error 1e-4 on
the [0,1] scale; gradients relative L2 <= 1e-4 against the drop-in path (same
kernels, different float summation order and activation rounding) and <= 1e-3
against the oracle (north star).
"""

from __future__ import annotations

import pytest
import torch

import helpers
import cuda_rasterizer as cr
from cuda_rasterizer.fused import render_l1
from cuda_rasterizer.train import Densifier
from cuda_rasterizer.wrapper import render
from oracle import render as orender
from oracle import train as otrain

pytestmark = pytest.mark.gpu


def _raw_leaves(p, dev):
    return {k: v.clone().to(dev).requires_grad_(True) for k, v in p.items()}


def test_activate_matches_torch(gpu):
    g = torch.Generator().manual_seed(0)
    n = 5000
    ls = torch.randn(n, 3, generator=g) - 3.0
    q = torch.randn(n, 4, generator=g)
    q[7] = 0.0  # the clamp_min(1e-12) branch
    q[8] = 1e-14
    lo = torch.randn(n, generator=g) * 3.0
    leaves = [t.to(gpu).requires_grad_(True) for t in (ls, q, lo)]
    scales, quats, opac = helpers.activated(dict(log_scales=leaves[0], quats_raw=leaves[1],
                                                 opacity_logits=leaves[2]))
    s2, q2, o2 = cr.activate(*[t.detach() for t in leaves])
    assert helpers.max_abs(s2 / scales.detach(), torch.ones_like(s2)) <= 1e-6
    assert helpers.max_abs(q2, quats) <= 1e-6
    assert helpers.max_abs(o2, opac) <= 1e-6
    ups = [torch.randn(t.shape, generator=g).to(gpu) for t in (scales, quats, opac)]
    torch.autograd.backward([scales, quats, opac], ups)
    got = cr.activate_backward(*ups, s2, leaves[1].detach(), o2)
    for a, t in zip(got, leaves):
        assert helpers.rel_l2(a, t.grad) <= 1e-5
    # absent gradients count as zero
    g_ls, g_q, g_l = cr.activate_backward(None, None, ups[2], s2, leaves[1].detach(), o2)
    assert float(g_ls.abs().max()) == 0.0 and float(g_q.abs().max()) == 0.0
    assert helpers.rel_l2(g_l, leaves[2].grad) <= 1e-5


def test_fused_preprocess_equals_unfused_sequence(gpu):
    """gs_preprocess_forward/backward run the same device functions in the same
    order as activate -> project -> SH render and their backward: bit-equal."""
    p, cam, _ = helpers.scene_orbit(6_000, 160, 120, 220.0, seed=31)
    g = torch.Generator().manual_seed(32)
    n = p["means"].shape[0]
    dev = gpu
    w2c, K = cam["w2c"].to(dev), cam["K"].to(dev)
    W, H = cam["width"], cam["height"]
    raw = {k: v.to(dev) for k, v in p.items()}
    raw["quats_raw"][5] = 0.0  # the clamp_min(1e-12) branch
    args = (0.01, 100.0, 1 / 255, 0.5, 128.0, W, H)
    fwd = cr.preprocess_forward(raw["means"], raw["log_scales"], raw["quats_raw"],
                                raw["opacity_logits"], raw["sh_dc"], raw["sh_rest"], w2c, K, *args)
    s, q, o = cr.activate(raw["log_scales"], raw["quats_raw"], raw["opacity_logits"])
    ref = cr.project_points(raw["means"], s, q, o, w2c, K, *args)
    col = cr.evaluate_spherical_harmonics_render(w2c, raw["means"], raw["sh_dc"], raw["sh_rest"],
                                                 ref[5])
    for a, b in zip(fwd[:6], ref):
        assert torch.equal(a, b)
    assert torch.equal(fwd[6], o) and torch.equal(fwd[7], col)
    assert 0 < int(ref[5].sum()) < n
    # without colours (the fused step's launch): the same projection; the colours
    # from the grid-capped launch meant for a second stream are bit-equal too
    proj = cr.preprocess_forward(raw["means"], raw["log_scales"], raw["quats_raw"],
                                 raw["opacity_logits"], raw["sh_dc"], raw["sh_rest"], w2c, K,
                                 *args, with_colors=False)
    assert proj[7] is None
    for a, b in zip(proj[:7], fwd[:7]):
        assert torch.equal(a, b)
    out = torch.full((n, 3), float("nan"), device=dev)
    beside = cr.evaluate_spherical_harmonics_render(w2c, raw["means"], raw["sh_dc"],
                                                    raw["sh_rest"], ref[5], out=out, beside=True)
    assert beside is out and torch.equal(beside, col)
    ups = [torch.randn(shape, generator=g).to(dev) for shape in ((n, 2), (n, 3), (n,), (n, 3))]
    got = cr.preprocess_backward(*ups, raw["means"], raw["log_scales"], raw["quats_raw"],
                                 raw["opacity_logits"], raw["sh_dc"], raw["sh_rest"], ref[2],
                                 ref[5], w2c, K, W, H)
    gm, gsc, gq = cr.project_points_backward(ups[0], ups[1], raw["means"], s, q, o, w2c, K, W, H,
                                             ref[2], ref[5])
    _, gdc, grest = cr.evaluate_spherical_harmonics_render_backward(
        ups[3], w2c, raw["means"], raw["sh_dc"], raw["sh_rest"], ref[5], accumulate_means=gm)
    gls, gqr, glog = cr.activate_backward(gsc, gq, ups[2], s, raw["quats_raw"], o)
    for a, b in zip(got, (gm, gls, gqr, glog, gdc, grest)):
        assert torch.equal(a, b)
    # the colour-gradient cache, written by the joint forward or the grid-capped
    # colour launch (identical rows), replaces the SH rows in the backward: the
    # same gradients, bit for bit, without reading sh_dc / sh_rest
    keep = ref[5]
    cache = torch.full((n, 10), float("nan"), device=dev)
    fwd_c = cr.preprocess_forward(raw["means"], raw["log_scales"], raw["quats_raw"],
                                  raw["opacity_logits"], raw["sh_dc"], raw["sh_rest"], w2c, K,
                                  *args, sh_cache=cache)
    for a, b in zip(fwd_c, fwd):
        assert torch.equal(a, b)
    cache_b = torch.full((n, 10), float("nan"), device=dev)
    col_b = cr.evaluate_spherical_harmonics_render(w2c, raw["means"], raw["sh_dc"],
                                                   raw["sh_rest"], keep, beside=True,
                                                   sh_cache=cache_b)
    assert torch.equal(col_b, col)
    assert torch.equal(cache[keep].view(torch.int32), cache_b[keep].view(torch.int32))
    assert bool(torch.isnan(cache[~keep]).all())  # rows outside the mask are not written
    got_c = cr.preprocess_backward(*ups, raw["means"], raw["log_scales"], raw["quats_raw"],
                                   raw["opacity_logits"], None, None, ref[2], keep, w2c, K, W,
                                   H, sh_cache=cache)
    for a, b in zip(got_c, got):
        assert torch.equal(a, b)
    with pytest.raises(RuntimeError, match="sh_cache"):
        cr.preprocess_forward(raw["means"], raw["log_scales"], raw["quats_raw"],
                              raw["opacity_logits"], raw["sh_dc"], raw["sh_rest"], w2c, K, *args,
                              with_colors=False, sh_cache=cache)


def _written_schedule(sched, n_tiles):
    """The parts of a schedule a forward writes: work, backward order and
    checkpoint counts of every tile, the position, work and pixels of each saved
    checkpoint (the slots past a tile's count keep whatever they held), and each
    XCD range's segment list; on grids of more than 6144 tiles, which take no
    checkpoints, the work and order."""
    s = sched.cpu()
    n = n_tiles
    if n > 6144:  # larger grids: work and order only
        assert s.numel() == 2 * n
        return s.tolist()
    counts = s[2 * n:3 * n].long()
    assert int(counts.min()) >= 0 and int(counts.max()) <= 3
    used = torch.arange(3).unsqueeze(0) < counts.unsqueeze(1)  # (n_tiles, 3)
    pos = s[3 * n:6 * n].view(n, 3)[used]
    work = s[6 * n:9 * n].view(n, 3)[used]
    head = (13 * n + 8 + 3) // 4 * 4
    pix = s[head:head + n * 3 * 1024].view(n, 3, 1024)[used]
    lengths = s[13 * n:13 * n + 8].tolist()
    items = [s[9 * n + 4 * a:9 * n + 4 * a + m].tolist() for a, m in zip(_xcd_firsts(n), lengths)]
    assert sum(lengths) == int(counts.sum()) + n
    return (s[:3 * n].tolist(), pos.tolist(), work.tolist(), pix.view(torch.float32).tolist(),
            items)


def _xcd_firsts(n_tiles):
    b, r = divmod(n_tiles, 8)
    return [x * b + min(x, r) for x in range(8)]


def test_forward_tile_order_changes_nothing_but_the_launch_order(gpu):
    """rasterize_display_l1 with an earlier call's schedule as forward_schedule (its
    tiles launched heaviest first): image, display, loss and this call's schedule
    (work per tile and backward order) are bit-equal to the plain launch; a
    reversed order (any per-range permutation is allowed) likewise."""
    p, cam, target = helpers.scene_orbit(20_000, 320, 240, 440.0, seed=23)
    W, H = cam["width"], cam["height"]
    raw = {k: v.to(gpu) for k, v in p.items()}
    w2c, K, tgt = cam["w2c"].to(gpu), cam["K"].to(gpu), target.to(gpu)
    pts, depths, _, conic, radii, mask, opac, colors = cr.preprocess_forward(
        raw["means"], raw["log_scales"], raw["quats_raw"], raw["opacity_logits"], raw["sh_dc"],
        raw["sh_rest"], w2c, K, 0.01, 100.0, 1 / 255, 0.5, 128.0, W, H)
    off, ids = cr.compute_tile_intersection(pts, radii, depths, mask, W, H, 16)
    nt = off.shape[0]
    args = (off, ids, pts, conic, opac, colors, W, H, tgt)
    first = cr.tile_schedule(nt, gpu)
    ref = cr.rasterize_display_l1(*args, schedule=first)
    reversed_sched = first.clone()
    base, rem = divmod(nt, 8)
    for x in range(8):  # each XCD range reversed: another permutation of every range
        s0 = x * base + min(x, rem)
        ln = base + (1 if x < rem else 0)
        reversed_sched[nt + s0:nt + s0 + ln] = torch.arange(s0 + ln - 1, s0 - 1, -1,
                                                           dtype=torch.int32, device=gpu)
    for prev in (first, reversed_sched):
        second = cr.tile_schedule(nt, gpu)
        got = cr.rasterize_display_l1(*args, schedule=second, forward_schedule=prev)
        for a, b in zip(got, ref):
            assert torch.equal(a, b)
        assert _written_schedule(second, nt) == _written_schedule(first, nt)
    with pytest.raises(cr.RasterizerError):
        cr.rasterize_display_l1(*args, schedule=first, forward_schedule=first)


def test_render_l1_waves_per_tile(gpu):
    """The fused step with each tile on 1, 2 or 4 waves: display bit-equal, the loss
    within 1e-6 (summation order of the per-tile sums) and the gradients within
    1e-5 of one wave.  (The per-tile work counts differ: a batch is 64 records per
    wave, so the tiles' batch counts differ.)"""
    p, cam, target = helpers.scene_orbit(20_000, 320, 240, 440.0, seed=27)
    W, H = cam["width"], cam["height"]
    w2c, K, tgt = cam["w2c"].to(gpu), cam["K"].to(gpu), target.to(gpu)
    runs = {}
    try:
        for waves in (1, 2, 4):
            cr.set_blend_waves(waves)
            a = _raw_leaves(p, gpu)
            cache = {}
            loss, disp, _, _ = render_l1(w2c, K, W, H, a["means"], a["log_scales"],
                                         a["quats_raw"], a["opacity_logits"], a["sh_dc"],
                                         a["sh_rest"], tgt, schedule_cache=cache, view_id="v")
            loss.backward()
            runs[waves] = (loss.detach(), disp, {k: a[k].grad for k in helpers.PARAMS},
                           cache["v"][:cache["v"].numel() // 2].clone())
    finally:
        cr.set_blend_waves(0)
    l1, d1, g1, w1 = runs[1]
    for waves in (2, 4):
        loss, disp, grads, work = runs[waves]
        assert torch.equal(disp, d1)
        assert work.shape == w1.shape and bool((work > 0).any())
        assert abs(float(loss) - float(l1)) <= 1e-6 * abs(float(l1))
        for k in helpers.PARAMS:
            assert helpers.rel_l2(grads[k], g1[k]) <= 1e-5, (waves, k)


def test_render_l1_view_schedule_cache(gpu):
    """render_l1 with a per-view schedule cache: the first step of a view fills
    it, the next launches its forward in that order; loss and display are
    bit-equal to the uncached step, gradients equal up to the float-atomic order."""
    p, cam, target = helpers.scene_orbit(20_000, 320, 240, 440.0, seed=24)
    W, H = cam["width"], cam["height"]
    w2c, K, tgt = cam["w2c"].to(gpu), cam["K"].to(gpu), target.to(gpu)
    cache = {}
    runs = []
    for use_cache in (False, True, True):
        a = _raw_leaves(p, gpu)
        loss, disp, _, _ = render_l1(w2c, K, W, H, a["means"], a["log_scales"], a["quats_raw"],
                                     a["opacity_logits"], a["sh_dc"], a["sh_rest"], tgt,
                                     schedule_cache=cache if use_cache else None, view_id="v0")
        loss.backward()
        runs.append((loss.detach(), disp, {k: a[k].grad for k in helpers.PARAMS}))
    assert list(cache) == ["v0"] and cache["v0"].dtype == torch.int32
    for loss, disp, grads in runs[1:]:
        assert torch.equal(loss, runs[0][0]) and torch.equal(disp, runs[0][1])
        for k in helpers.PARAMS:
            assert helpers.rel_l2(grads[k], runs[0][2][k]) <= 1e-5, k


@pytest.mark.parametrize("scene", ["orbit", "box"])
def test_render_l1_matches_drop_in_path(gpu, scene):
    if scene == "orbit":
        p, cam, target = helpers.scene_orbit(20_000, 320, 240, 440.0, seed=21)
    else:
        p, cam, target = helpers.scene_box(8_000, 200, 130, 220.0, seed=22, log_scale=(-3.5, 0.6))
    W, H = cam["width"], cam["height"]
    w2c, K, tgt = cam["w2c"].to(gpu), cam["K"].to(gpu), target.to(gpu)
    # drop-in path
    a = _raw_leaves(p, gpu)
    scales, quats, opac = helpers.activated(a)
    img, pts, radii = render(w2c, K, W, H, a["means"], scales, quats, opac, a["sh_dc"],
                             a["sh_rest"])
    pts.retain_grad()
    loss_a = torch.nn.functional.l1_loss(img / 255.0, tgt)
    loss_a.backward()
    # fused path, densification statistics through a Densifier
    b = _raw_leaves(p, gpu)
    n = p["means"].shape[0]
    dens = Densifier(n, gpu)
    loss_b, disp, pts_b, radii_b = render_l1(w2c, K, W, H, b["means"], b["log_scales"],
                                             b["quats_raw"], b["opacity_logits"], b["sh_dc"],
                                             b["sh_rest"], tgt, densifier=dens)
    loss_b.backward()
    assert loss_b.shape == ()
    assert abs(float(loss_b.detach()) - float(loss_a.detach())) <= 1e-5 * float(loss_a.detach())
    assert helpers.max_abs(disp / 255.0, img.detach() / 255.0) <= 1e-4
    for k in helpers.PARAMS:
        assert helpers.rel_l2(b[k].grad, a[k].grad) <= 1e-4, k
    # src/strategy.py:47-68 applied to the drop-in path's points_img.grad
    want_g, want_c = otrain.accumulate_grad2d(torch.zeros(n), torch.zeros(n), pts.grad.cpu(),
                                              radii.detach().cpu(), W, H)
    assert helpers.rel_l2(dens.grads, want_g) <= 1e-4
    assert torch.equal(dens.count.cpu(), want_c)
    assert torch.equal(pts_b, pts.detach()) or helpers.max_abs(pts_b, pts.detach()) <= 1e-4


def test_render_l1_config1_matches_oracle(gpu):
    """BASELINE config 1 through the fused path against the CPU oracle."""
    import bench

    scene = bench.config1()
    p, cam, target = scene["params"], scene["camera"], scene["target"]
    cam2 = dict(w2c=cam["w2c"], K=cam["K"], width=cam["width"], height=cam["height"])
    _, loss_c, grads_c, _, _ = helpers.forward_backward(orender.render, p, cam2, target, "cpu")
    b = _raw_leaves(p, gpu)
    loss_b, disp, _, _ = render_l1(cam["w2c"].to(gpu), cam["K"].to(gpu), cam["width"],
                                   cam["height"], b["means"], b["log_scales"], b["quats_raw"],
                                   b["opacity_logits"], b["sh_dc"], b["sh_rest"], target.to(gpu))
    loss_b.backward()
    assert abs(float(loss_b) - float(loss_c)) <= 1e-5
    for k in helpers.PARAMS:
        if float(grads_c[k].norm()) == 0.0:
            assert float(b[k].grad.norm()) == 0.0, k
        else:
            assert helpers.rel_l2(b[k].grad, grads_c[k]) <= 1e-3, k


def test_render_l1_colours_beside_binning_equal_joint(gpu, monkeypatch):
    """The colours on a second stream beside binning (scenes of at least
    BESIDE_MIN_GAUSSIANS) or inside the preprocess launch: the same loss, and the
    gradients up to the float atomics' order, over repeated steps."""
    import cuda_rasterizer.fused as fused

    p, cam, target = helpers.scene_orbit(20_000, 256, 192, 300.0, seed=29)
    w2c, K, tgt = cam["w2c"].to(gpu), cam["K"].to(gpu), target.to(gpu)
    b = _raw_leaves(p, gpu)
    out = {}
    for mode, threshold in (("joint", 10**9), ("beside", 0), ("beside again", 0)):
        monkeypatch.setattr(fused, "BESIDE_MIN_GAUSSIANS", threshold)
        for t in b.values():
            t.grad = None
        loss, _, _, _ = render_l1(w2c, K, 256, 192, b["means"], b["log_scales"],
                                  b["quats_raw"], b["opacity_logits"], b["sh_dc"], b["sh_rest"],
                                  tgt)
        loss.backward()
        out[mode] = (float(loss), {k: t.grad.clone() for k, t in b.items()})
    for mode in ("beside", "beside again"):
        assert out[mode][0] == out["joint"][0]
        for k in helpers.PARAMS:
            assert helpers.rel_l2(out[mode][1][k], out["joint"][1][k]) <= 1e-5, (mode, k)


def test_render_l1_repeated_calls_are_stable(gpu):
    """Two steps in a row on the same leaves give the same loss and gradients."""
    p, cam, target = helpers.scene_orbit(3_000, 96, 80, 140.0, seed=23)
    w2c, K, tgt = cam["w2c"].to(gpu), cam["K"].to(gpu), target.to(gpu)
    b = _raw_leaves(p, gpu)
    out = []
    for _ in range(2):
        for t in b.values():
            t.grad = None
        loss, _, _, _ = render_l1(w2c, K, 96, 80, b["means"], b["log_scales"], b["quats_raw"],
                                  b["opacity_logits"], b["sh_dc"], b["sh_rest"], tgt)
        loss.backward()
        out.append((float(loss), {k: t.grad.clone() for k, t in b.items()}))
    assert out[0][0] == out[1][0]
    for k in helpers.PARAMS:
        assert helpers.rel_l2(out[1][1][k], out[0][1][k]) <= 1e-5, k


@pytest.mark.parametrize("lam", [0.0, 0.2])
def test_render_l1_backward_twice_with_retain_graph(gpu, lam):
    """Two backward passes over one render_l1 graph (retain_graph) accumulate twice
    the gradients of one pass, as autograd does for any graph; the first pass's
    gradients are left untouched by the second (its blend accumulators are the
    forward's zeroed buffer, the second pass's are fresh)."""
    p, cam, target = helpers.scene_orbit(4_000, 128, 96, 180.0, seed=26)
    w2c, K, tgt = cam["w2c"].to(gpu), cam["K"].to(gpu), target.to(gpu)
    b = _raw_leaves(p, gpu)
    loss, _, _, _ = render_l1(w2c, K, 128, 96, b["means"], b["log_scales"], b["quats_raw"],
                              b["opacity_logits"], b["sh_dc"], b["sh_rest"], tgt, ssim_lambda=lam)
    g1 = torch.autograd.grad(loss, list(b.values()), retain_graph=True)
    once = [t.clone() for t in g1]
    g2 = torch.autograd.grad(loss, list(b.values()), retain_graph=True)
    for k, a, c, d in zip(b, once, g1, g2):
        assert torch.equal(c, a), k  # the first result is not written into
        assert helpers.rel_l2(d, a) <= 1e-5, k
    loss.backward(retain_graph=True)
    loss.backward()
    for k, a in zip(b, once):
        assert float(a.norm()) > 0.0, k
        assert helpers.rel_l2(b[k].grad, 2.0 * a) <= 1e-5, k


@pytest.mark.parametrize("count", [9 * 8000, 10, 4 * 8000 + 2])
def test_display_l1_clears_buffer(gpu, count):
    """rasterize_display_l1(clear=...) zeroes the buffer (in the blend launch when
    float4-aligned with a multiple of 4 elements, else with a fill), leaving the
    image, display and loss as without it."""
    p, cam, target = helpers.scene_box(8_000, 200, 130, 220.0, seed=23, log_scale=(-3.5, 0.6))
    W, H = cam["width"], cam["height"]
    a = _raw_leaves(p, gpu)
    with torch.no_grad():
        pts, depths, _, conic, radii, mask, opac, colors = cr.preprocess_forward(
            a["means"], a["log_scales"], a["quats_raw"], a["opacity_logits"], a["sh_dc"],
            a["sh_rest"], cam["w2c"].to(gpu), cam["K"].to(gpu), 0.01, 100.0, 1 / 255, 0.5, 128.0,
            W, H)
        off, ids = cr.compute_tile_intersection(pts, radii, depths, mask, W, H, 16)
        ref = cr.rasterize_display_l1(off, ids, pts, conic, opac, colors, W, H, target.to(gpu))
        buf = torch.full((count + 1,), 7.0, device=gpu)
        view = buf[1:] if count % 4 else buf[:count]  # a misaligned view for the odd counts
        got = cr.rasterize_display_l1(off, ids, pts, conic, opac, colors, W, H, target.to(gpu),
                                      clear=view)
    assert float(view.abs().max()) == 0.0
    assert float(buf[count if count % 4 == 0 else 0]) == 7.0  # nothing past the buffer
    for x, y in zip(got, ref):
        assert torch.equal(x, y)


def _xcd_ranges(n_tiles):
    base, rem = divmod(n_tiles, 8)
    start = 0
    for x in range(8):
        size = base + (1 if x < rem else 0)
        yield start, size
        start += size


def _order_code(w):
    """Work class of the backward's order: 16 steps per octave, heaviest first."""
    if w == 0:
        return 511
    e = int(w).bit_length() - 1
    m = (w >> (e - 4)) & 15 if e >= 4 else (w << (4 - e)) & 15
    return 510 - min(e * 16 + m, 510)


# XCD ranges of 0-1 tiles (a 2x2 and a 1x1 grid), 14-15, 1020, 2000, 4050 and
# 4224 tiles (one to nine chunks of 512 in the counting sort)
@pytest.mark.parametrize("size", [(32, 32), (16, 16), (200, 130), (1920, 1080), (2560, 1600),
                                  (3840, 2160), (4096, 2112)])
def test_tile_schedule(gpu, size):
    """rasterize_display_l1(schedule=...) leaves the image, display and loss as
    without it, writes each tile's work and, per XCD range, the tiles by
    descending work class (_order_code; ties by tile); rasterize_l1_backward
    gives the same gradients with the schedule as without (up to the order of
    the float atomics)."""
    W, H = size
    p, cam, target = helpers.scene_box(8_000, W, H, 220.0 * W / 200, seed=25,
                                       log_scale=(-3.5, 0.6))
    a = _raw_leaves(p, gpu)
    tgt = target.to(gpu)
    with torch.no_grad():
        pts, depths, _, conic, radii, mask, opac, colors = cr.preprocess_forward(
            a["means"], a["log_scales"], a["quats_raw"], a["opacity_logits"], a["sh_dc"],
            a["sh_rest"], cam["w2c"].to(gpu), cam["K"].to(gpu), 0.01, 100.0, 1 / 255, 0.5, 128.0,
            W, H)
        off, ids = cr.compute_tile_intersection(pts, radii, depths, mask, W, H, 16)
        n_tiles = off.shape[0]
        ref = cr.rasterize_display_l1(off, ids, pts, conic, opac, colors, W, H, tgt)
        sched = cr.tile_schedule(n_tiles, gpu)
        got = cr.rasterize_display_l1(off, ids, pts, conic, opac, colors, W, H, tgt,
                                      schedule=sched)
        for x, y in zip(got, ref):
            assert torch.equal(x, y)
        cost = sched[:n_tiles].cpu().numpy().view("uint32").astype("int64")
        order = sched[n_tiles:2 * n_tiles].cpu().numpy()
        assert cost.max() > 0
        for start, length in _xcd_ranges(n_tiles):
            got_order = list(order[start:start + length])
            want = sorted(range(start, start + length),
                          key=lambda t: (_order_code(int(cost[t])), t))
            assert got_order == want
        g = torch.full((1,), 0.7, device=gpu)
        grads = [cr.rasterize_l1_backward(tgt, g, off, ids, pts, conic, opac, colors, W, H,
                                          ref[0], schedule=s) for s in (None, sched)]
        # the drop-in render path's display entries: same work counts and order
        thr = (16, 1e-4, 1e-4, 9.21)
        sched_d = cr.tile_schedule(n_tiles, gpu)
        img_d, disp_d = cr.rasterize_display(off, ids, pts, conic, opac, colors, W, H, *thr,
                                             schedule=sched_d)
        img_r, disp_r = cr.rasterize_display(off, ids, pts, conic, opac, colors, W, H, *thr)
        assert torch.equal(img_d, img_r) and torch.equal(disp_d, disp_r)
        assert _written_schedule(sched_d, n_tiles) == _written_schedule(sched, n_tiles)
        up = torch.randn((H, W, 3), generator=torch.Generator().manual_seed(5)).to(gpu)
        grads_d = [cr.rasterize_display_backward(up, off, ids, pts, conic, opac, colors, W, H,
                                                 *thr, rendered_image=img_r, schedule=s)
                   for s in (None, sched_d)]
    for x, y in zip(*grads):
        assert helpers.rel_l2(y, x) <= 1e-5
    for x, y in zip(*grads_d):
        assert helpers.rel_l2(y, x) <= 1e-5


@pytest.mark.parametrize("lam", [0.2, 1.0])
def test_render_l1_with_ssim_matches_drop_in_path(gpu, lam):
    """render_l1(ssim_lambda=lam) against the reference's loss written with PyTorch
    around the drop-in render() and fused_ssim (scripts/train.py:185-205):
    (1 - lam) * l1(img / 255, t) + lam * (1 - SSIM(img / 255, t), padding valid)."""
    from cuda_rasterizer import fused_ssim

    p, cam, target = helpers.scene_orbit(20_000, 320, 240, 440.0, seed=24)
    W, H = cam["width"], cam["height"]
    w2c, K, tgt = cam["w2c"].to(gpu), cam["K"].to(gpu), target.to(gpu)
    a = _raw_leaves(p, gpu)
    scales, quats, opac = helpers.activated(a)
    img, _, _ = render(w2c, K, W, H, a["means"], scales, quats, opac, a["sh_dc"], a["sh_rest"])
    norm = img / 255.0
    ssim = fused_ssim(norm.permute(2, 0, 1).unsqueeze(0), tgt.permute(2, 0, 1).unsqueeze(0),
                      padding="valid")
    loss_a = (1 - lam) * torch.nn.functional.l1_loss(norm, tgt) + lam * (1.0 - ssim)
    loss_a.backward()
    b = _raw_leaves(p, gpu)
    loss_b, disp, _, _ = render_l1(w2c, K, W, H, b["means"], b["log_scales"], b["quats_raw"],
                                   b["opacity_logits"], b["sh_dc"], b["sh_rest"], tgt,
                                   ssim_lambda=lam)
    loss_b.backward()
    assert loss_b.shape == ()
    assert abs(float(loss_b.detach()) - float(loss_a.detach())) <= 1e-5 * float(loss_a.detach())
    assert helpers.max_abs(disp, img.detach()) <= 1e-4 * 255
    for k in helpers.PARAMS:
        assert helpers.rel_l2(b[k].grad, a[k].grad) <= 1e-4, k


def test_render_l1_and_render_with_outgrown_capacities(gpu, monkeypatch):
    """The fused step and render() bin with capacity-sized lists and check K and M
    only after the blend is queued; when the lists outgrow the capacities they bin
    again with exact sizes.  Forced small capacities give the loss, display and
    gradients of roomy ones."""
    import cuda_rasterizer as cr
    from cuda_rasterizer.wrapper import render

    monkeypatch.setattr(cr, "_CAPACITY", {})
    p, cam, target = helpers.scene_orbit(20_000, 256, 192, 300.0, seed=31)
    w2c, K, tgt = cam["w2c"].to(gpu), cam["K"].to(gpu), target.to(gpu)
    out = {}
    for mode in ("first", "roomy", "small", "roomy again"):
        if mode == "small":
            cr._CAPACITY[(gpu.index, 256, 192, 16)] = (1000, 100)
        b = _raw_leaves(p, gpu)
        loss, display, _, _ = render_l1(w2c, K, 256, 192, b["means"], b["log_scales"],
                                        b["quats_raw"], b["opacity_logits"], b["sh_dc"],
                                        b["sh_rest"], tgt)
        loss.backward()
        sc, qq, op = helpers.activated(b)
        if mode == "small":
            cr._CAPACITY[(gpu.index, 256, 192, 16)] = (1000, 100)
        disp, _, _ = render(w2c, K, 256, 192, b["means"].detach(), sc.detach(), qq.detach(),
                            op.detach(), b["sh_dc"].detach(), b["sh_rest"].detach())
        out[mode] = (float(loss), display.clone(), disp.clone(),
                     {k: t.grad.clone() for k, t in b.items()})
    assert cr._CAPACITY[(gpu.index, 256, 192, 16)][0] > 1000  # grown again by exact binning
    for mode in ("roomy", "small", "roomy again"):
        assert out[mode][0] == out["first"][0], mode
        assert torch.equal(out[mode][1], out["first"][1]), mode
        assert torch.equal(out[mode][2], out["first"][2]), mode
        for k in helpers.PARAMS:
            assert helpers.rel_l2(out[mode][3][k], out["first"][3][k]) <= 1e-5, (mode, k)


@pytest.mark.parametrize("size,n", [((256, 192), 60_000), ((800, 608), 150_000)])
def test_backward_segments_from_checkpoints(gpu, size, n):
    """Long tile lists: the forward saves up to 3 checkpoints per tile (every 128
    entries with one wave per tile, every 256 with four), and the backward given
    the schedule walks those tiles in segments that start from them.  Gradients
    equal the unsegmented walk's (no schedule) up to float rounding (the running
    colour-gradient sum restarts from a dot product; atomics reorder), for the
    L1 seed (fused) and the display seed (drop-in render path)."""
    W, H = size
    p, cam, target = helpers.scene_orbit(n, W, H, 1.2 * W, seed=57)
    a = _raw_leaves(p, gpu)
    tgt = target.to(gpu)
    with torch.no_grad():
        pts, depths, _, conic, radii, mask, opac, colors = cr.preprocess_forward(
            a["means"], a["log_scales"], a["quats_raw"], a["opacity_logits"], a["sh_dc"],
            a["sh_rest"], cam["w2c"].to(gpu), cam["K"].to(gpu), 0.01, 100.0, 1 / 255, 0.5, 128.0,
            W, H)
        off, ids = cr.compute_tile_intersection(pts, radii, depths, mask, W, H, 16)
        n_tiles = off.shape[0]
        sched = cr.tile_schedule(n_tiles, gpu)
        image, display, loss = cr.rasterize_display_l1(off, ids, pts, conic, opac, colors, W, H,
                                                       tgt, schedule=sched)
        counts = sched[2 * n_tiles:3 * n_tiles].cpu()
        assert int(counts.max()) == 3 and int((counts > 0).sum()) >= n_tiles // 4
        g = torch.full((1,), 0.9, device=gpu)
        plain, seg = [cr.rasterize_l1_backward(tgt, g, off, ids, pts, conic, opac, colors, W, H,
                                               image, schedule=s) for s in (None, sched)]
        for x, y in zip(plain, seg):
            assert helpers.rel_l2(y, x) <= 1e-5
        thr = (16, 1e-4, 1e-4, 9.21)
        sched_d = cr.tile_schedule(n_tiles, gpu)
        img_d, _ = cr.rasterize_display(off, ids, pts, conic, opac, colors, W, H, *thr,
                                        schedule=sched_d)
        assert torch.equal(img_d, image)
        up = torch.randn((H, W, 3), generator=torch.Generator().manual_seed(6)).to(gpu)
        plain, seg = [cr.rasterize_display_backward(up, off, ids, pts, conic, opac, colors, W,
                                                    H, *thr, rendered_image=img_d, schedule=s)
                      for s in (None, sched_d)]
        for x, y in zip(plain, seg):
            assert helpers.rel_l2(y, x) <= 1e-5

