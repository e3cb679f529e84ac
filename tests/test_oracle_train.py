"""CPU checks of the training-loop oracle (oracle/train.py) against PyTorch's
Adam and hand-derived densification cases."""

from __future__ import annotations

import pytest
import torch

from oracle import train as otrain


def test_adam_oracle_matches_torch_optim_adam():
    g = torch.Generator().manual_seed(0)
    p0 = torch.randn(64, 3, generator=g)
    p = p0.clone().requires_grad_(True)
    opt = torch.optim.Adam([p], lr=5e-3, eps=1e-15, betas=(0.9, 0.999), foreach=False)
    q, m, v = p0.clone(), torch.zeros_like(p0), torch.zeros_like(p0)
    for t in range(1, 6):
        grad = torch.randn(64, 3, generator=g) * (10.0 ** -t)
        p.grad = grad.clone()
        opt.step()
        q, m, v = otrain.adam_step(q, grad, m, v, t, 5e-3, 0.9, 0.999, 1e-15)
        # equal up to last-bit rounding of PyTorch's fused lerp / addcmul / addcdiv kernels
        assert torch.allclose(q, p.detach(), rtol=1e-5, atol=1e-8), t
        assert torch.allclose(m, opt.state[p]["exp_avg"], rtol=1e-5, atol=1e-12)
        assert torch.allclose(v, opt.state[p]["exp_avg_sq"], rtol=1e-5, atol=1e-15)


def test_adam_oracle_planted_mistake_is_caught():
    """A dropped bias correction changes the first step by a factor ~1/(1-b1)."""
    p = torch.ones(4)
    g = torch.full((4,), 0.5)
    good, _, _ = otrain.adam_step(p, g, torch.zeros(4), torch.zeros(4), 1, 1e-2, 0.9, 0.999, 1e-15)
    # first Adam step moves each coordinate by lr * sign(g) (bias-corrected m/sqrt(v) = 1)
    assert torch.allclose(p - good, torch.full((4,), 1e-2), rtol=1e-5)


def test_accumulate_grad2d_hand_case():
    grads = torch.zeros(3)
    count = torch.zeros(3)
    gp = torch.tensor([[0.1, 0.2], [1.0, 1.0], [0.3, -0.4]])
    radii = torch.tensor([[2.0, 3.0], [0.0, 5.0], [1.0, 1.0]])
    grads, count = otrain.accumulate_grad2d(grads, count, gp, radii, width=20, height=10)
    # row 0: (0.1*10, 0.2*5) = (1, 1) -> sqrt(2); row 1 invisible; row 2: (3, -2) -> sqrt(13)
    assert torch.allclose(grads, torch.tensor([2.0 ** 0.5, 0.0, 13.0 ** 0.5]))
    assert torch.equal(count, torch.tensor([1.0, 0.0, 1.0]))


def test_refine_rows_hand_case():
    # 5 Gaussians: #1 transparent (pruned), #2 high grad and small (cloned),
    # #3 high grad and large (split), #0 and #4 low grad (kept)
    logits = torch.logit(torch.tensor([0.5, 0.001, 0.5, 0.5, 0.5]))
    log_scales = torch.log(torch.tensor([[0.005] * 3, [0.005] * 3, [0.005] * 3, [0.05] * 3,
                                         [0.005] * 3]))
    grads = torch.tensor([0.0, 1.0, 1.0, 1.0, 0.0])
    count = torch.ones(5)
    src, fresh, n_split, split_src = otrain.refine_rows(logits, log_scales, grads, count, step=600)
    # kept = [0, 2, 3, 4]; X = [0, 2, 3, 4, 2(clone)]; split X[2] (= 3): rest = [0, 2, 4, 2c]
    assert src.tolist() == [0, 2, 4, 2, 3, 3]
    assert fresh.tolist() == [False, False, False, True, True, True]
    assert n_split == 1 and split_src.tolist() == [3]


def test_clone_top_rows_hand_case():
    logits = torch.logit(torch.tensor([0.5, 0.001, 0.5, 0.5]))
    grads = torch.tensor([0.1, 5.0, 3.0, 0.2])
    src, fresh = otrain.clone_top_rows(logits, grads, fraction=0.5)
    assert src.tolist() == [0, 2, 3, 1, 2]  # kept 0,2,3 then the top-2 rows by gradient
    assert fresh.tolist() == [False, False, False, True, True]


def test_clone_top_rows_ties_by_index():
    """Equal gradient norms are taken largest first, then by ascending index (also
    across the selection boundary), as cuda_rasterizer.train.top_rows takes them."""
    from cuda_rasterizer.train import top_rows

    logits = torch.zeros(8)
    grads = torch.tensor([3.0, 1.0, 3.0, 2.0, 0.0, 2.0, 3.0, 0.0])
    src, fresh = otrain.clone_top_rows(logits, grads, fraction=0.5)
    assert src.tolist() == list(range(8)) + [0, 2, 6, 3]
    assert fresh.tolist() == [False] * 8 + [True] * 4
    assert top_rows(grads, 4).tolist() == [0, 2, 6, 3]
    big = torch.randint(0, 50, (5000,), generator=torch.Generator().manual_seed(1)).float()
    src, _ = otrain.clone_top_rows(torch.zeros(5000), big, fraction=0.05)
    assert src[5000:].tolist() == top_rows(big, 250).tolist()


def _cap_case():
    """7 Gaussians: #0 transparent (pruned), #1-#4 high grad and small (clone
    candidates), #5 high grad and large (split), #6 low grad."""
    logits = torch.logit(torch.tensor([0.001, 0.5, 0.5, 0.5, 0.5, 0.5, 0.5]))
    log_scales = torch.log(torch.tensor([[0.005] * 3] * 5 + [[0.05] * 3] + [[0.005] * 3]))
    grads = torch.tensor([1.0, 1.0, 1.0, 1.0, 1.0, 1.0, 0.0])
    return logits, log_scales, grads, torch.ones(7)


def test_refine_rows_growth_budget_hand_case():
    """src/strategy.py:116-137 with max_gaussians = 8: 6 rows survive the prune,
    so the budget is 2 (not 1: it counts the rows after pruning); of the 4
    candidates the permutation [3, 1, 0, 2] picks candidates 3 and 1, which are
    cloned in row order (rows 2 and 4); the split is not capped, so the result
    has max_gaussians + n_split rows."""
    logits, log_scales, grads, count = _cap_case()
    src, fresh, n_split, split_src = otrain.refine_rows(
        logits, log_scales, grads, count, step=600, max_gaussians=8,
        budget_perm=torch.tensor([3, 1, 0, 2]))
    # kept = [1..6]; X = [1, 2, 3, 4, 5, 6, 2c, 4c]; split X[4] (= 5)
    assert src.tolist() == [1, 2, 3, 4, 6, 2, 4, 5, 5]
    assert fresh.tolist() == [False] * 5 + [True] * 4
    assert n_split == 1 and split_src.tolist() == [5]
    # another permutation, another pair, still in row order
    src2, _, _, _ = otrain.refine_rows(logits, log_scales, grads, count, step=600,
                                       max_gaussians=8, budget_perm=torch.tensor([2, 0, 3, 1]))
    assert src2.tolist() == [1, 2, 3, 4, 6, 1, 3, 5, 5]
    # the budget binds: without the reference's draw the oracle refuses
    with pytest.raises(ValueError, match="budget binds"):
        otrain.refine_rows(logits, log_scales, grads, count, step=600, max_gaussians=8)


def test_refine_rows_at_the_cap_grows_nothing():
    """6 rows after the prune and max_gaussians = 6 (or fewer): no clone and no
    split either (src/strategy.py:119-124 returns before both)."""
    logits, log_scales, grads, count = _cap_case()
    for cap in (6, 5):
        src, fresh, n_split, split_src = otrain.refine_rows(logits, log_scales, grads, count,
                                                            step=600, max_gaussians=cap)
        assert src.tolist() == [1, 2, 3, 4, 5, 6]
        assert not bool(fresh.any()) and n_split == 0 and split_src.numel() == 0


def test_refine_rows_budget_properties():
    """Random scene where the cap binds: exactly `budget` clones, all of them
    candidates, the ones the permutation's first `budget` entries name; the
    split count equals the uncapped one; with a cap that does not bind the
    result equals the uncapped row map whatever permutation is passed."""
    g = torch.Generator().manual_seed(7)
    n = 5000
    logits = torch.randn(n, generator=g) * 3.0
    log_scales = torch.randn(n, 3, generator=g) * 0.8 - 4.5
    grads = torch.rand(n, generator=g) * 4e-4
    count = torch.ones(n)
    free = otrain.refine_rows(logits, log_scales, grads, count, step=600, max_gaussians=10**9)
    n_keep = int((torch.sigmoid(logits) >= 0.005).sum())
    n_cand = int(free[1].sum()) - 2 * free[2]
    assert n_cand > 200
    budget = 150
    perm = torch.randperm(n_cand, generator=g)
    src, fresh, n_split, split_src = otrain.refine_rows(
        logits, log_scales, grads, count, step=600, max_gaussians=n_keep + budget,
        budget_perm=perm)
    assert n_split == free[2] and torch.equal(split_src, free[3])
    assert len(src) == n_keep + budget + n_split
    # the clones are the fresh rows before the split copies
    clones = src[:len(src) - 2 * n_split][fresh[:len(src) - 2 * n_split]]
    free_clones = free[0][:len(free[0]) - 2 * free[2]][free[1][:len(free[0]) - 2 * free[2]]]
    assert torch.equal(clones, torch.sort(free_clones[perm[:budget]]).values)
    loose = otrain.refine_rows(logits, log_scales, grads, count, step=600,
                               max_gaussians=n_keep + n_cand, budget_perm=perm)
    assert torch.equal(loose[0], free[0]) and torch.equal(loose[1], free[1])


def test_reset_opacities_oracle():
    """src/strategy.py:231-253: logits above logit(0.01) = ln(1/99) become it,
    the rest are unchanged; both moments are zeroed.  The float32 threshold is
    within one ulp of the exact value."""
    import math

    thr_exact = math.log(0.01 / 0.99)
    logits = torch.tensor([-10.0, -4.6, -4.5, 0.0, 3.0, float("inf")])
    m = torch.randn(6)
    v = torch.rand(6)
    out, m2, v2 = otrain.reset_opacities(logits, m, v)
    thr = float(out[3])
    f32_ulp = 2.0 ** (math.floor(math.log2(abs(thr_exact))) - 23)
    assert abs(thr - thr_exact) <= f32_ulp
    assert out.tolist()[:2] == [-10.0, -4.599999904632568]  # below: unchanged
    assert all(x == thr for x in out.tolist()[2:])
    assert float(m2.abs().max()) == 0.0 and float(v2.abs().max()) == 0.0
