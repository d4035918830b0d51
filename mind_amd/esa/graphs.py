"""Fixed-shape forwards captured once into a HIP graph and replayed.

An ESA forward over one batch of small graphs issues about a hundred kernel
launches (projections, layer norms, the attention and its plan, MLPs,
gathers), most of them a few microseconds long, so the host's launch rate and
the gaps between dependent launches take a fifth of the step.  For a serving
loop whose batches have a fixed shape (the same token count, graph count and
padded set size) the whole forward is captured into one HIP graph
(``torch.cuda.CUDAGraph``) and each batch is one graph launch: the inputs are
copied into the graph's own input buffers, the graph is replayed, and the
outputs appear in the graph's output buffers.

Everything the library launches takes torch's current stream and allocates
its workspaces as torch tensors, so capture records the library's kernels
with the rest; none of the library's entry points issue memsets, copies or
host synchronisations on the forward path.  Requirements of the captured
function: tensor inputs only (host values such as the batch size and the
padded set size are part of the capture), no host synchronisation (capture
raises), and outputs that depend on the inputs only (a replay recomputes them
from the input buffers).
"""
from __future__ import annotations

from typing import Callable, Sequence

import torch

from .. import _lib


def _as_tuple(out):
    return out if isinstance(out, tuple) else (out,)


class GraphedForward:
    """``fn`` captured for inputs of the example inputs' shapes, dtypes and device.

    ``fn(*inputs)`` must return a tensor or a tuple of tensors.  The constructor
    runs ``fn`` ``warmup`` times on a side stream (lazy library initialisation
    stays out of the graph), then captures one call under ``torch.no_grad()``.
    Calling the object copies the given inputs into the captured input buffers
    (skipped for an input that is that buffer), replays the graph on the
    current stream and returns the captured outputs.  Those output tensors are
    the graph's own buffers: the next call overwrites them, so clone what must
    be kept.  Calls that overlap on one device race on the buffers.
    """

    def __init__(self, fn: Callable[..., torch.Tensor | tuple], *example_inputs: torch.Tensor, warmup: int = 2):
        if _lib.profiling():
            raise RuntimeError("GraphedForward: the per-kernel profiling hook is on; its event records cannot be "
                               "captured (profile_enable(False) first)")
        if not example_inputs or not all(isinstance(x, torch.Tensor) for x in example_inputs):
            raise TypeError("GraphedForward takes one or more tensor inputs")
        devices = {x.device for x in example_inputs}
        if len(devices) != 1 or next(iter(devices)).type != "cuda":
            raise ValueError(f"inputs must share one GPU device (got {sorted(str(d) for d in devices)})")
        self.device = next(iter(devices))
        self.inputs = tuple(x.detach().clone() for x in example_inputs)
        side = torch.cuda.Stream(self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(side), torch.no_grad():
            for _ in range(warmup):
                fn(*self.inputs)
        torch.cuda.current_stream(self.device).wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.no_grad(), torch.cuda.graph(self.graph):
            out = fn(*self.inputs)
        self._single = not isinstance(out, tuple)
        self.outputs = _as_tuple(out)
        if not all(isinstance(y, torch.Tensor) for y in self.outputs):
            raise TypeError("the captured function must return a tensor or a tuple of tensors")

    def _check(self, inputs: Sequence[torch.Tensor]) -> None:
        if len(inputs) != len(self.inputs):
            raise ValueError(f"captured with {len(self.inputs)} inputs, called with {len(inputs)}")
        for i, (x, s) in enumerate(zip(inputs, self.inputs)):
            if not isinstance(x, torch.Tensor):
                raise TypeError(f"input {i} is not a tensor")
            if x.shape != s.shape or x.dtype != s.dtype or x.device != s.device:
                raise ValueError(f"input {i} is {tuple(x.shape)} {x.dtype} on {x.device}; the graph was captured "
                                 f"for {tuple(s.shape)} {s.dtype} on {s.device}")

    def __call__(self, *inputs: torch.Tensor):
        self._check(inputs)
        for x, s in zip(inputs, self.inputs):
            if x is not s:
                s.copy_(x)
        self.graph.replay()
        return self.outputs[0] if self._single else self.outputs
