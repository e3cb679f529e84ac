"""CPU oracle for the training-loop pieces -- TEST INFRASTRUCTURE ONLY.

Restates, in PyTorch on the CPU:
  adam_step            torch.optim.Adam's update as configured by
                       scripts/train.py:17-44 (no weight decay, no amsgrad), in
                       PyTorch's operation order (lerp for the first moment)
  accumulate_grad2d    src/strategy.py:47-68 (_update_state)
  refine_rows          the row map of src/strategy.py:71-229 (prune, then
                       clone / split, with the max_gaussians growth budget of
                       :116-137), the split samples and the budget's random
                       permutation supplied by the caller
  reset_opacities      src/strategy.py:231-253
  clone_top_rows       the benchmark's configuration-5 rule: clone the top
                       fraction by accumulated gradient norm, prune opacity

Each returns plain tensors so that tests compare the library's kernels with it.
"""

from __future__ import annotations

import math

import numpy as np
import torch


def adam_step(p, g, m, v, t, lr, beta1, beta2, eps):
    """One Adam step in float32; returns new (p, m, v).  t is the 1-based step."""
    m = m + (1 - beta1) * (g - m)
    v = v * beta2 + (1 - beta2) * (g * g)
    step_size = lr / (1 - beta1 ** t)
    bc2_sqrt = math.sqrt(1 - beta2 ** t)
    denom = v.sqrt() / bc2_sqrt + eps
    return p - step_size * (m / denom), m, v


def accumulate_grad2d(grads, count, grad_points_image, radii, width, height):
    """src/strategy.py:47-68: returns updated (grads, count)."""
    g = grad_points_image.clone()
    g[:, 0] *= width / 2.0
    g[:, 1] *= height / 2.0
    sel = torch.where((radii > 0.0).all(dim=1))[0]
    grads = grads.clone()
    count = count.clone()
    grads.index_add_(0, sel, g[sel].norm(dim=1))
    count.index_add_(0, sel, torch.ones_like(sel, dtype=torch.float))
    return grads, count


def refine_rows(opacity_logits, log_scales, grads, count, step, prune_opacity=0.005,
                prune_scale=0.1, grow_grad=0.0002, split_scale=0.01, reset_every=3000,
                max_gaussians=1_000_000, budget_perm=None):
    """Row map of one refinement (src/strategy.py:71-229): returns (src_rows,
    fresh, n_split, split_src) where the final tensors are src[src_rows], fresh
    rows have zero optimizer state, and the last 2 * n_split rows are the two
    copies of split_src (which get the sampled offsets).

    Growth follows src/strategy.py:116-137.  With N kept rows (after pruning):
    N >= max_gaussians grows nothing (no clone, no split); otherwise at most
    budget = max_gaussians - N rows are cloned.  When more are eligible the
    reference draws `perm = torch.randperm(n_clone)[:budget]` and clones the
    eligible rows selection_all[perm] -- in ascending row order, since it
    rebuilds the selection with torch.where.  The caller passes that draw as
    `budget_perm` (a permutation of n_clone, e.g. drawn from the generator the
    library used); the split set is not capped."""
    opac = torch.sigmoid(opacity_logits)
    scales = torch.exp(log_scales)
    is_prune = opac < prune_opacity
    if step > reset_every:
        is_prune = is_prune | (scales.max(dim=1).values > prune_scale)
    keep = torch.where(~is_prune)[0]
    n_keep = len(keep)
    if n_keep >= max_gaussians:  # src/strategy.py:119-124: growth skipped entirely
        return keep, torch.zeros(n_keep, dtype=torch.bool), 0, keep[:0]
    avg = (grads / count.clamp(min=1.0))[keep]
    high = avg > grow_grad
    small = scales[keep].max(dim=1).values < split_scale
    clone_sel = torch.where(high & small)[0]
    budget = max_gaussians - n_keep
    if len(clone_sel) > budget:  # src/strategy.py:132-138
        if budget_perm is None or len(budget_perm) != len(clone_sel):
            raise ValueError(f"the growth budget binds ({len(clone_sel)} eligible, budget "
                             f"{budget}): pass the reference's torch.randperm({len(clone_sel)})")
        chosen = torch.zeros(len(keep), dtype=torch.bool)
        chosen[clone_sel[budget_perm.to(torch.int64)[:budget]]] = True
        clone_sel = torch.where(chosen)[0]
    x_src = torch.cat([keep, keep[clone_sel]])
    x_fresh = torch.cat([torch.zeros(len(keep), dtype=torch.bool),
                         torch.ones(len(clone_sel), dtype=torch.bool)])
    x_split = torch.cat([high & ~small, torch.zeros(len(clone_sel), dtype=torch.bool)])
    rest = torch.where(~x_split)[0]
    split_sel = torch.where(x_split)[0]
    src_rows = torch.cat([x_src[rest], x_src[split_sel], x_src[split_sel]])
    fresh = torch.cat([x_fresh[rest], torch.ones(2 * len(split_sel), dtype=torch.bool)])
    return src_rows, fresh, len(split_sel), x_src[split_sel]


def reset_opacities(opacity_logits, exp_avg, exp_avg_sq, prune_opacity=0.005, threshold=None):
    """src/strategy.py:231-253: the logits clamped to logit(2 * prune_opacity)
    from above (computed in float32, as the reference does on the parameters'
    device; `threshold` overrides it with a value computed elsewhere) and both
    Adam moments of the opacities zeroed.  Returns (logits, exp_avg, exp_avg_sq)."""
    if threshold is None:
        threshold = torch.logit(torch.tensor(prune_opacity * 2.0, dtype=torch.float32))
    return (torch.clamp(opacity_logits, max=threshold), torch.zeros_like(exp_avg),
            torch.zeros_like(exp_avg_sq))


def clone_top_rows(opacity_logits, grads, fraction=0.05, prune_opacity=0.005):
    """Configuration-5 rule: (src_rows, fresh) = kept rows, then the top
    round(fraction * N) rows by accumulated gradient norm, largest first and
    equal norms by ascending index."""
    n = opacity_logits.shape[0]
    keep = torch.where(~(torch.sigmoid(opacity_logits) < prune_opacity))[0]
    n_top = int(round(fraction * n))
    g = grads.detach().cpu().numpy()
    order = np.lexsort((np.arange(n), -g))  # by -norm, then by index
    top = torch.from_numpy(order[:n_top].astype(np.int64))
    src_rows = torch.cat([keep, top])
    fresh = torch.cat([torch.zeros(len(keep), dtype=torch.bool), torch.ones(n_top, dtype=torch.bool)])
    return src_rows, fresh
