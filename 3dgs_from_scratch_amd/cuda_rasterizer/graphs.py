"""Training steps captured into HIP graphs.

A step of a small scene is bound by the host: each of its ~30 library and
PyTorch launches costs a few microseconds of Python, ctypes and HIP runtime
time, more than the GPU spends on many of them.  CapturedStep records a step
(any callable that renders through `render_l1` or the drop-in `render()` and
calls backward, e.g. the body of scripts/train.py:133-227's loop without the
optimizer's host logic) into one HIP graph (torch.cuda.CUDAGraph) and replays it
with one launch.  ConcurrentSteps replays several such graphs -- the
independent views of one step -- on several streams at once, so that one
view's short launches and tail overlap another's blend.

What the capture fixes, and what each replay must therefore keep:
  * tensor addresses: the inputs the step reads (parameters, camera, target)
    are the same tensors on every replay -- update them in place (copy_), and
    read outputs (loss, .grad) from the tensors the capture produced;
  * list capacities: the tile lists are sized by the capacities of the capped
    sort, taken from the warm-up calls.  A replay whose lists would outgrow them
    writes no list entries (its image and gradients are then incomplete) and is
    reported by ok(); run the step eagerly once (it rebins with exact sizes and
    raises the capacities) and recapture();
  * the depth hint of the sort (any hint gives the same lists; a stale one only
    slows the sort).
No library launch in the step uses hipMemsetAsync (buffers are cleared by
kernels), and none waits on the host once the capacities are set.
"""

from __future__ import annotations

import torch

import cuda_rasterizer as _cr


class CapturedStep:
    """`fn()` captured into a HIP graph on the current device after `warmup`
    eager calls (on a side stream, as torch.cuda.graphs requires; they also set
    the capacities).  replay() relaunches it on the current stream; `output` is
    what the captured call returned (its tensors are rewritten by every replay).
    ok() synchronises and returns whether every capped sort of the last replay
    fit its capacities."""

    def __init__(self, fn, warmup: int = 2):
        if warmup < 1:
            raise ValueError("CapturedStep: at least one warm-up call sets the capacities")
        self._fn = fn
        self.graph = None
        self.output = None
        self.checks: list = []
        self.capture(warmup)

    def capture(self, warmup: int = 1) -> None:
        dev = torch.device("cuda", torch.cuda.current_device())
        main = torch.cuda.current_stream(dev)
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(main)
        with torch.cuda.stream(side):
            for _ in range(warmup):
                self._fn()
        main.wait_stream(side)
        torch.cuda.synchronize(dev)
        self.graph = None  # release the previous graph's pool before capturing again
        self.output = None
        graph = torch.cuda.CUDAGraph()
        with _cr.CapturedChecks() as sink:
            with torch.cuda.graph(graph):
                out = self._fn()
        self.graph, self.output, self.checks = graph, out, sink.checks

    recapture = capture

    def replay(self) -> None:
        self.graph.replay()

    def ok(self) -> bool:
        torch.cuda.current_stream().synchronize()
        return all(c.replayed_ok() for c in self.checks)


class ConcurrentSteps:
    """Independent parts of one step -- e.g. the cameras of a multi-view batch --
    each captured into its own HIP graph (CapturedStep) and replayed concurrently
    on `streams` HIP streams of default priority; a further graph sums their
    outputs on the caller's stream.

    Each callable in `fns` returns a tuple of tensors of the same shapes (e.g. a
    view's weighted loss followed by torch.autograd.grad of it with respect to the
    parameters).  The parts must not write shared tensors: compute gradients with
    torch.autograd.grad, not .backward() into shared .grad fields.  replay() queues
    everything on the current stream's timeline and returns the summed tuple
    (tensors rewritten by every replay); the sum adds the parts in `fns` order, so
    it equals the sequential accumulation up to float summation order.  ok()
    synchronises and checks every part's capped sorts, as CapturedStep.ok()."""

    def __init__(self, fns, streams: int = 4, warmup: int = 2):
        if not fns:
            raise ValueError("ConcurrentSteps: no parts")
        if streams < 1:
            raise ValueError("ConcurrentSteps: streams must be >= 1")
        self.parts = [CapturedStep(f, warmup=warmup) for f in fns]
        outs = [p.output for p in self.parts]
        if any(not isinstance(o, tuple) or len(o) != len(outs[0]) for o in outs):
            raise ValueError("ConcurrentSteps: every part must return a tuple of the same length")
        dev = torch.device("cuda", torch.cuda.current_device())
        self.streams = [torch.cuda.Stream(device=dev) for _ in range(streams)]

        def total():
            acc = [t.clone() for t in outs[0]]
            for o in outs[1:]:
                torch._foreach_add_(acc, list(o))
            return tuple(acc)

        self._sum = CapturedStep(total, warmup=1)
        self.output = self._sum.output

    def replay(self):
        main = torch.cuda.current_stream()
        for s in self.streams:
            s.wait_stream(main)
        for i, part in enumerate(self.parts):
            with torch.cuda.stream(self.streams[i % len(self.streams)]):
                part.replay()
        for s in self.streams:
            main.wait_stream(s)
        self._sum.replay()
        return self.output

    def ok(self) -> bool:
        torch.cuda.current_stream().synchronize()
        return all(all(c.replayed_ok() for c in p.checks) for p in self.parts)
