"""Training-loop pieces on the library's kernels: a fused Adam over all
parameter groups and the densification strategy.

FusedAdam mirrors the reference's optimizer setup (scripts/train.py:17-44: one
torch.optim.Adam per parameter group, eps 1e-15, betas scaled by the batch
size, learning rates scaled by sqrt(batch size), exponential decay of the
means learning rate to 1% at max_steps, :97-101) with one kernel launch per
step for all groups (gs_adam_step).

Densifier keeps src/strategy.py's state (accumulated |dL/d means2D| in NDC
scale and visibility counts, :47-68, via gs_accumulate_grad2d) and rebuilds
every parameter and Adam-state tensor in one gs_gather_rows launch for
  - the reference rules (`refine`: prune by opacity (and scale after the first
    opacity reset), then clone small / split large Gaussians whose mean
    gradient exceeds grow_grad, :71-229), and
  - the stress-test rule of the benchmark's configuration 5
    (`clone_top_and_prune`: clone the top fraction by accumulated gradient
    norm with jittered positions, prune opacity < 0.005).
New Gaussians start with zero Adam moments, as in the reference.
"""

from __future__ import annotations

import ctypes
import math

import torch

from . import _lib
from ._lib import GsAdamTensor, GsGatherTensor

PARAM_ORDER = ("means", "log_scales", "quats_raw", "opacity_logits", "sh_dc", "sh_rest")

# scripts/train.py:17-44 (the reference's parameter names: means, scales,
# quaternions, opacities, sh_coeffs_dc, sh_coeffs_rest)
DEFAULT_LR = {"means": 1.6e-4, "log_scales": 5e-3, "quats_raw": 1e-3, "opacity_logits": 5e-2,
              "sh_dc": 2.5e-3, "sh_rest": 2.5e-3 / 20}


def _ptr(t):
    return t.data_ptr() if t is not None else None


def _stream(t):
    return torch.cuda.current_stream(t.device).cuda_stream


class FusedAdam:
    """Adam over a dict of leaf tensors, one kernel launch per step."""

    def __init__(self, params: dict, lr: dict | None = None, batch_size: int = 1,
                 eps: float = 1e-15, means_decay_steps: int | None = None):
        self.params = params
        base = dict(DEFAULT_LR if lr is None else lr)
        self.lr = {k: base[k] * math.sqrt(batch_size) for k in params}
        self.beta1 = 1 - batch_size * (1 - 0.9)
        self.beta2 = 1 - batch_size * (1 - 0.999)
        self.eps = eps
        self.step_count = {k: 0 for k in params}
        self.exp_avg = {k: torch.zeros_like(v) for k, v in params.items()}
        self.exp_avg_sq = {k: torch.zeros_like(v) for k, v in params.items()}
        # ExponentialLR(gamma = 0.01 ** (1 / max_steps)) on the means group
        self.means_gamma = 0.01 ** (1 / means_decay_steps) if means_decay_steps else 1.0

    def step(self):
        specs = []
        for k, p in self.params.items():
            if p.grad is None:
                continue
            self.step_count[k] += 1
            t = self.step_count[k]
            g = p.grad
            if not g.is_contiguous():
                g = g.contiguous()
            specs.append(GsAdamTensor(
                _ptr(p), _ptr(g), _ptr(self.exp_avg[k]), _ptr(self.exp_avg_sq[k]), p.numel(),
                self.lr[k] / (1 - self.beta1 ** t), math.sqrt(1 - self.beta2 ** t)))
        if specs:
            arr = (GsAdamTensor * len(specs))(*specs)
            dev = next(iter(self.params.values()))
            with torch.no_grad(), torch.cuda.device(dev.device):
                _lib.check(_lib.load().gs_adam_step(arr, len(specs), self.beta1, self.beta2,
                                                    self.eps, _stream(dev)), "adam_step")
        if "means" in self.lr:
            self.lr["means"] *= self.means_gamma

    def zero_grad(self):
        for p in self.params.values():
            p.grad = None


class Densifier:
    """src/strategy.py on the library's kernels (see the module docstring)."""

    refine_start_step = 500
    refine_stop_step = 15000
    refine_every_n_steps = 100
    reset_every_n_steps = 3000
    prune_opacity = 0.005
    prune_scale = 0.1
    grow_grad = 0.0002
    split_scale = 0.01
    max_gaussians = 1000000

    def __init__(self, n: int, device):
        self.grads = torch.zeros(n, device=device)
        self.count = torch.zeros(n, device=device)

    def update(self, grad_points_image: torch.Tensor, radii: torch.Tensor, width: int, height: int):
        """src/strategy.py:47-68 (gs_accumulate_grad2d)."""
        n = self.grads.shape[0]
        g = grad_points_image.detach().contiguous()
        r = radii.detach().contiguous()
        with torch.cuda.device(g.device):
            _lib.check(_lib.load().gs_accumulate_grad2d(_ptr(g), _ptr(r), n, int(width),
                                                        int(height), _ptr(self.grads),
                                                        _ptr(self.count), _stream(g)),
                       "accumulate_grad2d")

    # --------------------------------------------------------------- rebuild
    def _rebuild(self, params: dict, opt: FusedAdam | None, src_rows: torch.Tensor,
                 fresh: torch.Tensor, deltas: dict):
        """Replace every parameter (and Adam moment) by its rows src_rows (plus
        deltas[name]); rows with fresh set get zero moments."""
        n_out = int(src_rows.numel())
        dev = src_rows.device
        src_rows = src_rows.to(torch.int32).contiguous()
        fresh = fresh.to(torch.uint8).contiguous()
        specs, keep = [], []
        new_params = {}
        for k in PARAM_ORDER:
            if k not in params:
                continue
            p = params[k].detach()
            width = p[0].numel() if p.shape[0] else int(torch.tensor(p.shape[1:]).prod())
            dst = torch.empty((n_out,) + tuple(p.shape[1:]), dtype=p.dtype, device=dev)
            d = deltas.get(k)
            d = d.contiguous() if d is not None else None
            keep.append(d)
            specs.append(GsGatherTensor(_ptr(p), _ptr(dst), _ptr(d), width, 0))
            new_params[k] = dst
            if opt is not None:
                for store in (opt.exp_avg, opt.exp_avg_sq):
                    s_dst = torch.empty_like(dst)
                    specs.append(GsGatherTensor(_ptr(store[k]), _ptr(s_dst), None, width, 1))
                    keep.append((store, k, s_dst))
        arr = (GsGatherTensor * len(specs))(*specs)
        with torch.cuda.device(dev):
            _lib.check(_lib.load().gs_gather_rows(n_out, _ptr(src_rows), _ptr(fresh), arr,
                                                  len(specs), _stream(src_rows)), "gather_rows")
        for item in keep:
            if isinstance(item, tuple):
                store, k, s_dst = item
                store[k] = s_dst
        for k, dst in new_params.items():
            params[k] = dst.requires_grad_(True)
        if opt is not None:
            opt.params = params
        self.grads = torch.zeros(n_out, device=dev)
        self.count = torch.zeros(n_out, device=dev)

    # -------------------------------------------------------- reference rules
    @torch.no_grad()
    def refine(self, params: dict, opt: FusedAdam | None, step: int, generator=None):
        """Prune, then clone / split, as src/strategy.py:71-229; returns
        (n_pruned, n_cloned, n_split)."""
        dev = params["means"].device
        opac = torch.sigmoid(params["opacity_logits"])
        scales = torch.exp(params["log_scales"])
        is_prune = opac < self.prune_opacity
        if step > self.reset_every_n_steps:
            is_prune = is_prune | (scales.max(dim=1).values > self.prune_scale)
        keep = torch.where(~is_prune)[0]
        grads = (self.grads / self.count.clamp(min=1.0))[keep]
        scales_k = scales[keep]
        n_keep = int(keep.numel())
        is_grad_high = grads > self.grow_grad
        small = scales_k.max(dim=1).values < self.split_scale
        is_clone = is_grad_high & small
        is_split = is_grad_high & ~small
        n_clone = int(is_clone.sum())
        if n_keep >= self.max_gaussians:
            is_clone[:] = False
            is_split[:] = False
            n_clone = 0
        budget = self.max_gaussians - n_keep
        if n_clone > budget:
            sel = torch.where(is_clone)[0]
            perm = torch.randperm(n_clone, device=dev, generator=generator)[:budget]
            is_clone = torch.zeros_like(is_clone)
            is_clone[sel[perm]] = True
            n_clone = budget
        # X = [kept; kept[clone]]; final = [X[rest]; X[split]; X[split]]
        clone_sel = torch.where(is_clone)[0]
        x_src = torch.cat([keep, keep[clone_sel]])
        x_fresh = torch.cat([torch.zeros(n_keep, dtype=torch.bool, device=dev),
                             torch.ones(n_clone, dtype=torch.bool, device=dev)])
        x_split = torch.cat([is_split, torch.zeros(n_clone, dtype=torch.bool, device=dev)])
        rest = torch.where(~x_split)[0]
        split_sel = torch.where(x_split)[0]
        n_split = int(split_sel.numel())
        src_rows = torch.cat([x_src[rest], x_src[split_sel], x_src[split_sel]])
        fresh = torch.cat([x_fresh[rest], torch.ones(2 * n_split, dtype=torch.bool, device=dev)])
        deltas = {}
        if n_split:
            q = torch.nn.functional.normalize(params["quats_raw"][x_src[split_sel]], dim=1)
            R = _rotation(q)
            s_split = scales[x_src[split_sel]]
            probe = torch.randn((2, n_split, 3), device=dev, generator=generator)
            samples = (R.unsqueeze(0) @ (s_split.unsqueeze(0) * probe).unsqueeze(-1)).squeeze(-1)
            n_rest = int(rest.numel())
            dm = torch.zeros((n_rest + 2 * n_split, 3), device=dev)
            dm[n_rest:] = samples.reshape(2 * n_split, 3)
            deltas = {"means": dm}  # src/strategy.py:191-192: param[selection] + samples
        self._rebuild(params, opt, src_rows, fresh, deltas)
        if n_split:  # src/strategy.py:193-194 stores log(scale / 1.6) itself (not a delta)
            params["log_scales"].data[n_rest:] = torch.log(s_split / 1.6).repeat(2, 1)
        return int(is_prune.sum()), n_clone, n_split

    @torch.no_grad()
    def reset_opacities(self, params: dict, opt: FusedAdam | None):
        """src/strategy.py:231-253: clamp logits to logit(2 * prune_opacity), zero their moments."""
        thr = torch.logit(torch.tensor(self.prune_opacity * 2.0, device=params["means"].device))
        params["opacity_logits"].data.clamp_(max=float(thr))
        if opt is not None:
            opt.exp_avg["opacity_logits"].zero_()
            opt.exp_avg_sq["opacity_logits"].zero_()

    # ------------------------------------------------- configuration-5 rule
    @torch.no_grad()
    def clone_top_and_prune(self, params: dict, opt: FusedAdam | None, fraction: float = 0.05,
                            jitter: float = 0.01, generator=None):
        """Clone the top `fraction` by accumulated gradient norm (means + N(0, jitter);
        ties by index, see top_rows), prune sigmoid(opacity) < prune_opacity; returns
        (n_pruned, n_cloned)."""
        dev = params["means"].device
        n = params["means"].shape[0]
        opac = torch.sigmoid(params["opacity_logits"])
        is_prune = opac < self.prune_opacity
        keep = torch.where(~is_prune)[0]
        n_top = int(round(fraction * n))
        top = top_rows(self.grads, n_top)
        src_rows = torch.cat([keep, top])
        fresh = torch.cat([torch.zeros(keep.numel(), dtype=torch.bool, device=dev),
                           torch.ones(n_top, dtype=torch.bool, device=dev)])
        dm = torch.zeros((src_rows.numel(), 3), device=dev)
        dm[keep.numel():] = torch.randn((n_top, 3), device=dev, generator=generator) * jitter
        self._rebuild(params, opt, src_rows, fresh, {"means": dm})
        return int(is_prune.sum()), n_top


def top_rows(values: torch.Tensor, count: int) -> torch.Tensor:
    """Indices of the `count` largest values, largest first, equal values by
    ascending index (a stable descending sort, so the choice among ties does not
    depend on the device or the sort implementation)."""
    return torch.sort(values, descending=True, stable=True).indices[:count]


def _rotation(q: torch.Tensor) -> torch.Tensor:
    """Rotation matrices of xyzw unit quaternions (src/gaussian.py:64-79)."""
    x, y, z, w = q.unbind(dim=1)
    return torch.stack([
        1 - 2 * (y * y + z * z), 2 * (x * y - z * w), 2 * (x * z + y * w),
        2 * (x * y + z * w), 1 - 2 * (x * x + z * z), 2 * (y * z - x * w),
        2 * (x * z - y * w), 2 * (y * z + x * w), 1 - 2 * (x * x + y * y),
    ], dim=1).reshape(-1, 3, 3)
