"""CPU checks of the training-loop oracle (oracle/train.py) against PyTorch's
Adam and hand-derived densification cases."""

from __future__ import annotations

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
