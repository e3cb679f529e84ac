"""GPU parity of the training-loop kernels (cuda_rasterizer.train) against the
CPU oracle (oracle/train.py).

FusedAdam: parameters and moments after several steps, relative error <= 1e-5
(device sqrt / division vs PyTorch CPU rounding).  Densifier.update: bit-level
agreement of the accumulated gradient norms up to float rounding (rel 1e-6)
and exact counts.  Densifier.refine / clone_top_and_prune: every rebuilt
parameter and moment equals the oracle's row map applied with PyTorch
indexing (bit-exact: pure copies), split offsets checked separately.
"""

from __future__ import annotations

import pytest
import torch

import helpers
from cuda_rasterizer.train import DEFAULT_LR, PARAM_ORDER, Densifier, FusedAdam
from oracle import train as otrain

pytestmark = pytest.mark.gpu

SHAPES = {"means": (3,), "log_scales": (3,), "quats_raw": (4,), "opacity_logits": (),
          "sh_dc": (3,), "sh_rest": (15, 3)}


def _params(n, gen, dev, logits=None, log_scales=None):
    p = {k: torch.randn((n,) + s, generator=gen) for k, s in SHAPES.items()}
    if logits is not None:
        p["opacity_logits"] = logits
    if log_scales is not None:
        p["log_scales"] = log_scales
    return {k: v.to(dev).requires_grad_(True) for k, v in p.items()}


def test_fused_adam_matches_oracle(gpu):
    g = torch.Generator().manual_seed(1)
    params = _params(5000, g, gpu)
    ref = {k: v.detach().cpu().clone() for k, v in params.items()}
    m = {k: torch.zeros_like(v) for k, v in ref.items()}
    v2 = {k: torch.zeros_like(v) for k, v in ref.items()}
    opt = FusedAdam(params, means_decay_steps=1000)
    lr = {k: DEFAULT_LR[k] for k in params}
    for t in range(1, 6):
        grads = {k: torch.randn(v.shape, generator=g) * 10.0 ** (-t) for k, v in ref.items()}
        for k, p in params.items():
            p.grad = grads[k].to(gpu)
        opt.step()
        for k in ref:
            ref[k], m[k], v2[k] = otrain.adam_step(ref[k], grads[k], m[k], v2[k], t, lr[k], 0.9,
                                                   0.999, 1e-15)
        lr["means"] *= 0.01 ** (1 / 1000)
    for k in PARAM_ORDER:
        assert helpers.rel_l2(params[k], ref[k]) <= 1e-6, k
        assert helpers.rel_l2(opt.exp_avg[k], m[k]) <= 1e-5, k
        assert helpers.rel_l2(opt.exp_avg_sq[k], v2[k]) <= 1e-5, k


def test_accumulate_grad2d_matches_oracle(gpu):
    g = torch.Generator().manual_seed(2)
    n = 10_000
    gp = torch.randn(n, 2, generator=g) * 1e-3
    radii = torch.rand(n, 2, generator=g) * 10.0
    radii[::7, 0] = 0.0
    radii[::11, 1] = 0.0
    d = Densifier(n, gpu)
    grads, count = torch.zeros(n), torch.zeros(n)
    for _ in range(3):
        d.update(gp.to(gpu), radii.to(gpu), 640, 480)
        grads, count = otrain.accumulate_grad2d(grads, count, gp, radii, 640, 480)
    assert helpers.rel_l2(d.grads, grads) <= 1e-6
    assert torch.equal(d.count.cpu(), count)


def _opt_with_state(params, gen, dev):
    opt = FusedAdam(params)
    for k in params:
        opt.exp_avg[k] = torch.randn(params[k].shape, generator=gen).to(dev)
        opt.exp_avg_sq[k] = torch.rand(params[k].shape, generator=gen).to(dev)
    return opt


def _check_rebuild(params, before, opt, st_before, src, fresh, skip_rows=None, skip_keys=()):
    rows = torch.arange(len(src))
    keep_rows = rows if skip_rows is None else rows[~skip_rows]
    for k in PARAM_ORDER:
        want = before[k][src]
        got = params[k].detach().cpu()
        assert got.shape == want.shape, k
        if k in skip_keys:
            assert torch.equal(got[keep_rows], want[keep_rows]), k
        else:
            assert torch.equal(got, want), k
        for store, name in ((opt.exp_avg, "m"), (opt.exp_avg_sq, "v")):
            w = st_before[name][k][src].clone()
            w[fresh] = 0.0
            assert torch.equal(store[k].cpu(), w), (k, name)
        assert params[k].requires_grad and params[k].is_leaf


def test_refine_matches_oracle_row_map(gpu):
    g = torch.Generator().manual_seed(3)
    n = 4000
    logits = torch.randn(n, generator=g) * 3.0            # some below logit(0.005)
    log_scales = torch.randn(n, 3, generator=g) * 0.8 - 4.5  # mix of small and large
    params = _params(n, g, gpu, logits=logits, log_scales=log_scales)
    opt = _opt_with_state(params, g, gpu)
    before = {k: v.detach().cpu().clone() for k, v in params.items()}
    st_before = {"m": {k: v.cpu().clone() for k, v in opt.exp_avg.items()},
                 "v": {k: v.cpu().clone() for k, v in opt.exp_avg_sq.items()}}
    d = Densifier(n, gpu)
    d.grads = (torch.rand(n, generator=g) * 4e-4).to(gpu)
    d.count = torch.ones(n).to(gpu)
    src, fresh, n_split, split_src = otrain.refine_rows(logits, log_scales, d.grads.cpu(),
                                                        d.count.cpu(), step=600)
    assert n_split > 0 and bool(fresh.any()) and len(src) != n
    n_pruned, n_cloned, n_split2 = d.refine(params, opt, step=600,
                                            generator=torch.Generator(device=gpu).manual_seed(0))
    assert n_split2 == n_split
    split_rows = torch.zeros(len(src), dtype=torch.bool)
    split_rows[len(src) - 2 * n_split:] = True
    _check_rebuild(params, before, opt, st_before, src, fresh, skip_rows=split_rows,
                   skip_keys=("means", "log_scales"))
    # split copies: log-scale = log(scale / 1.6), stored as such (src/strategy.py:193-194:
    # the same torch ops on the same device, so bit-equal); means offset by samples of
    # norm ~ scale
    got_ls = params["log_scales"].detach().cpu()[split_rows]
    s_dev = torch.exp(before["log_scales"].to(gpu))[split_src.to(gpu)]
    want_ls = torch.log(s_dev / 1.6).repeat(2, 1).cpu()
    assert torch.equal(got_ls, want_ls)
    assert torch.allclose(got_ls, torch.log(torch.exp(before["log_scales"][split_src]) / 1.6)
                          .repeat(2, 1), rtol=0, atol=1e-5)
    off = params["means"].detach().cpu()[split_rows] - before["means"][split_src].repeat(2, 1)
    scale = torch.exp(before["log_scales"][split_src]).max(dim=1).values.repeat(2)
    assert bool((off.norm(dim=1) <= 6.0 * scale * 3 ** 0.5).all())
    assert float(d.grads.abs().max()) == 0.0 and d.grads.shape[0] == len(src)


def test_clone_top_and_prune_matches_oracle(gpu):
    g = torch.Generator().manual_seed(4)
    n = 3000
    logits = torch.randn(n, generator=g) * 3.0
    params = _params(n, g, gpu, logits=logits)
    opt = _opt_with_state(params, g, gpu)
    before = {k: v.detach().cpu().clone() for k, v in params.items()}
    st_before = {"m": {k: v.cpu().clone() for k, v in opt.exp_avg.items()},
                 "v": {k: v.cpu().clone() for k, v in opt.exp_avg_sq.items()}}
    d = Densifier(n, gpu)
    d.grads = torch.randperm(n, generator=g).float().to(gpu)  # distinct: top-k is well defined
    src, fresh = otrain.clone_top_rows(logits, d.grads.cpu(), fraction=0.05)
    n_pruned, n_top = d.clone_top_and_prune(params, opt, fraction=0.05, jitter=0.0)
    assert n_top == int(fresh.sum()) and n_pruned == int((torch.sigmoid(logits) < 0.005).sum())
    _check_rebuild(params, before, opt, st_before, src, fresh)


def test_config5_training_loop_events(gpu):
    """BASELINE configuration 5 through the library loop (render_l1 + FusedAdam +
    Densifier, the bench's run_train "fused" path) for 1600 steps: 16
    clone / prune events, the last ones above 400k Gaussians.  At each event every rebuilt parameter and both Adam
    moments equal the oracle's row map (oracle.train.clone_top_rows on the
    pre-event opacity logits and accumulated gradient norms) applied to the
    pre-event tensors, bit for bit; the cloned means add the jitter drawn from
    the same generator state; the sizes follow N' = kept + round(0.05 N); the
    loss stays finite and falls."""
    import bench
    from cuda_rasterizer.fused import render_l1

    steps = 1600
    scene = bench.config5(steps=steps)
    w2c_all = scene["w2c_per_step"].to(gpu)
    targets = scene["targets"].to(gpu)
    cam = scene["camera"]
    K, W, H = cam["K"].to(gpu), cam["width"], cam["height"]
    leaves = {k: v.to(gpu).requires_grad_(True) for k, v in scene["params"].items()}
    opt = FusedAdam(leaves, means_decay_steps=steps)
    dens = Densifier(leaves["means"].shape[0], gpu)
    gen = torch.Generator(device=gpu).manual_seed(0)
    losses, sizes = [], [leaves["means"].shape[0]]
    for step in range(steps):
        loss, _, _, _ = render_l1(w2c_all[step], K, W, H, leaves["means"], leaves["log_scales"],
                                  leaves["quats_raw"], leaves["opacity_logits"], leaves["sh_dc"],
                                  leaves["sh_rest"], targets[step % targets.shape[0]],
                                  near_plane=cam["near"], densifier=dens)
        loss.backward()
        opt.step()
        opt.zero_grad()
        losses.append(float(loss.detach()))
        if (step + 1) % 100:
            continue
        n = leaves["means"].shape[0]
        before = {k: v.detach().clone() for k, v in leaves.items()}
        m_before = {k: v.clone() for k, v in opt.exp_avg.items()}
        v_before = {k: v.clone() for k, v in opt.exp_avg_sq.items()}
        assert float(dens.count.max()) > 0.0
        src, fresh = otrain.clone_top_rows(before["opacity_logits"].cpu(), dens.grads.cpu(),
                                           fraction=0.05)
        gen_state = gen.get_state()
        n_pruned, n_top = dens.clone_top_and_prune(leaves, opt, 0.05, 0.01, generator=gen)
        assert n_top == round(0.05 * n) == int(fresh.sum())
        assert leaves["means"].shape[0] == len(src) == n - n_pruned + n_top
        src_d, fresh_d = src.to(gpu), fresh.to(gpu)
        jitter = torch.randn((n_top, 3), device=gpu,
                             generator=torch.Generator(device=gpu).set_state(gen_state)) * 0.01
        for k in PARAM_ORDER[1:] + PARAM_ORDER[:1]:  # the row map first, then the jitter
            want = before[k][src_d]
            if k == "means":
                assert torch.equal(leaves[k].detach()[~fresh_d], want[~fresh_d]), k
                want[fresh_d] = want[fresh_d] + jitter
            assert torch.equal(leaves[k].detach(), want), k
            for store, st in ((opt.exp_avg, m_before), (opt.exp_avg_sq, v_before)):
                w = st[k][src_d]
                w[fresh_d] = 0.0
                assert torch.equal(store[k], w), k
            assert leaves[k].requires_grad and leaves[k].is_leaf
        assert float(dens.grads.abs().max()) == 0.0 and dens.count.shape[0] == len(src)
        sizes.append(len(src))
    assert len(sizes) == 17 and sizes[-1] > sizes[0]
    assert sizes[-2] >= 400_000  # the events from step 1500 on run above 400k Gaussians
    assert all(x == x and abs(x) < 1e30 for x in losses)
    assert sum(losses[-50:]) < sum(losses[:50])


def _refine_with_cap(gpu, n, cap_from_keep, seed, max_gaussians=None):
    """Densifier.refine where the growth budget binds, against the oracle's row
    map given the same randperm draw (the generator's first draw in refine)."""
    g = torch.Generator().manual_seed(seed)
    logits = torch.randn(n, generator=g) * 3.0
    log_scales = torch.randn(n, 3, generator=g) * 0.8 - 4.5
    params = _params(n, g, gpu, logits=logits, log_scales=log_scales)
    opt = _opt_with_state(params, g, gpu)
    before = {k: v.detach().cpu().clone() for k, v in params.items()}
    st_before = {"m": {k: v.cpu().clone() for k, v in opt.exp_avg.items()},
                 "v": {k: v.cpu().clone() for k, v in opt.exp_avg_sq.items()}}
    d = Densifier(n, gpu)
    d.grads = (torch.rand(n, generator=g) * 4e-4).to(gpu)
    d.count = torch.ones(n).to(gpu)
    n_keep = int((torch.sigmoid(logits) >= d.prune_opacity).sum())
    free = otrain.refine_rows(logits, log_scales, d.grads.cpu(), d.count.cpu(), step=600,
                              max_gaussians=10**12)
    n_cand = int(free[1].sum()) - 2 * free[2]
    cap = max_gaussians if max_gaussians is not None else n_keep + cap_from_keep
    d.max_gaussians = cap
    budget = cap - n_keep
    assert 0 < budget < n_cand  # the cap binds
    seed_dev = 1234 + seed
    perm = torch.randperm(n_cand, device=gpu,
                          generator=torch.Generator(device=gpu).manual_seed(seed_dev)).cpu()
    src, fresh, n_split, split_src = otrain.refine_rows(
        logits, log_scales, d.grads.cpu(), d.count.cpu(), step=600, max_gaussians=cap,
        budget_perm=perm)
    n_pruned, n_cloned, n_split2 = d.refine(
        params, opt, step=600, generator=torch.Generator(device=gpu).manual_seed(seed_dev))
    assert (n_pruned, n_cloned, n_split2) == (n - n_keep, budget, n_split)
    assert len(src) == cap + n_split
    split_rows = torch.zeros(len(src), dtype=torch.bool)
    split_rows[len(src) - 2 * n_split:] = True
    _check_rebuild(params, before, opt, st_before, src, fresh, skip_rows=split_rows,
                   skip_keys=("means", "log_scales"))
    got_ls = params["log_scales"].detach().cpu()[split_rows]
    s_dev = torch.exp(before["log_scales"].to(gpu))[split_src.to(gpu)]
    assert torch.equal(got_ls, torch.log(s_dev / 1.6).repeat(2, 1).cpu())


def test_refine_growth_budget_matches_oracle(gpu):
    """src/strategy.py:116-137: more clone candidates than max_gaussians leaves
    room for (the cap set on the instance to 100 above the rows kept): the
    library clones the candidates its generator's randperm picks, in row order,
    and splits uncapped -- bit for bit the oracle's row map given that draw."""
    _refine_with_cap(gpu, 6000, 100, seed=5)


def test_refine_growth_budget_at_the_default_cap(gpu):
    """The same at the reference's own cap, max_gaussians = 1,000,000: of
    1,003,000 Gaussians 38,694 fall to the prune, so the budget is 35,694 rows
    for 43,424 clone candidates (and 439,691 uncapped splits)."""
    _refine_with_cap(gpu, 1_003_000, None, seed=6, max_gaussians=1_000_000)


def test_refine_at_the_cap_grows_nothing(gpu):
    """With as many rows kept as max_gaussians, refine prunes only: no clone, no
    split (src/strategy.py:119-124), as the oracle."""
    g = torch.Generator().manual_seed(8)
    n = 3000
    logits = torch.randn(n, generator=g) * 3.0
    log_scales = torch.randn(n, 3, generator=g) * 0.8 - 4.5
    params = _params(n, g, gpu, logits=logits, log_scales=log_scales)
    opt = _opt_with_state(params, g, gpu)
    before = {k: v.detach().cpu().clone() for k, v in params.items()}
    st_before = {"m": {k: v.cpu().clone() for k, v in opt.exp_avg.items()},
                 "v": {k: v.cpu().clone() for k, v in opt.exp_avg_sq.items()}}
    d = Densifier(n, gpu)
    d.grads = (torch.rand(n, generator=g) * 4e-4).to(gpu)
    d.count = torch.ones(n).to(gpu)
    n_keep = int((torch.sigmoid(logits) >= d.prune_opacity).sum())
    d.max_gaussians = n_keep
    src, fresh, n_split, _ = otrain.refine_rows(logits, log_scales, d.grads.cpu(),
                                                d.count.cpu(), step=600, max_gaussians=n_keep)
    assert d.refine(params, opt, step=600) == (n - n_keep, 0, 0)
    assert n_split == 0 and not bool(fresh.any())
    _check_rebuild(params, before, opt, st_before, src, fresh)


def test_reset_opacities_matches_oracle(gpu):
    """src/strategy.py:231-253: logits clamped from above at logit(0.01) computed
    on the device, the opacities' Adam moments zeroed, every other tensor
    untouched; the device threshold is within one float32 ulp of the oracle's."""
    import math

    g = torch.Generator().manual_seed(9)
    n = 50_000
    logits = torch.randn(n, generator=g) * 4.0
    params = _params(n, g, gpu, logits=logits)
    opt = _opt_with_state(params, g, gpu)
    before = {k: v.detach().cpu().clone() for k, v in params.items()}
    m_before = {k: v.cpu().clone() for k, v in opt.exp_avg.items()}
    v_before = {k: v.cpu().clone() for k, v in opt.exp_avg_sq.items()}
    d = Densifier(n, gpu)
    d.reset_opacities(params, opt)
    thr_dev = torch.logit(torch.tensor(0.01, device=gpu)).cpu()
    want, m0, v0 = otrain.reset_opacities(logits, m_before["opacity_logits"],
                                          v_before["opacity_logits"], threshold=thr_dev)
    assert torch.equal(params["opacity_logits"].detach().cpu(), want)
    assert int((want == thr_dev).sum()) > n // 10  # the clamp is exercised
    thr_cpu = otrain.reset_opacities(torch.tensor([0.0]), torch.zeros(1), torch.zeros(1))[0]
    assert abs(float(thr_dev) - float(thr_cpu)) <= 2.0 ** (math.floor(math.log2(4.6)) - 23)
    assert torch.equal(opt.exp_avg["opacity_logits"].cpu(), m0)
    assert torch.equal(opt.exp_avg_sq["opacity_logits"].cpu(), v0)
    for k in PARAM_ORDER:
        if k == "opacity_logits":
            continue
        assert torch.equal(params[k].detach().cpu(), before[k]), k
        assert torch.equal(opt.exp_avg[k].cpu(), m_before[k]), k
        assert torch.equal(opt.exp_avg_sq[k].cpu(), v_before[k]), k
    assert params["opacity_logits"].requires_grad
