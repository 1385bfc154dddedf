"""``compiled(model, int8=True)`` — the prepare-then-run wrapper of borch-ts/src/compile.ts:570-578.

Prepare (once): ``model.eval()``, the model's own ``fuse()`` if it has one (the BN fold,
compile.ts:49-54 / nn.ts:6756), then with ``int8=True`` ``quantize_for_int8`` — the number
of layers that took the int8 path is kept as ``int8_layers`` (compile.ts:197-198) so a
timing is never quoted for an "int8" forward that was mostly f32.

Run: eager, or with ``graph=True`` a HIP graph captured on the first call for that
input shape and replayed afterwards (the reference's record/replay, device.ts:634-660):
the int8 forward is many small launches, and a replay issues them as one.

Tune (``tune=True``, the default, as the reference's, compile.ts:55-62): before a shape's
first run on a GPU, the int8 GEMM / conv kernel of every distinct layer problem is chosen
by measurement (``borch_amd.tune``); ``tuned`` keeps the decisions, one list per shape.
The choice changes time only: every candidate computes the same result.
"""
from __future__ import annotations

import torch

from .nn import quantize_for_int8
from .tune import tune as _tune


class Compiled:
    def __init__(self, model, int8: bool = False, graph: bool = False, fuse: bool = True, tune: bool = True):
        self.model = model
        self.int8 = int8
        self.graph = graph
        self.tune = tune
        self.tuned = []  # the tuner's decisions, one list per input shape (borch_amd.tune.tune)
        self._tuned_keys = set()
        self.int8_layers = 0
        model.eval()
        if fuse and callable(getattr(model, "fuse", None)):
            model.fuse()
        if int8:
            self.int8_layers = quantize_for_int8(model)
        self._graphs = {}

    @torch.no_grad()
    def __call__(self, x):
        key = (tuple(x.shape), x.dtype, x.device)
        if self.tune and x.device.type == "cuda" and key not in self._tuned_keys:
            self._tuned_keys.add(key)
            self.tuned.append(_tune(self.model, x))
        if not self.graph or x.device.type != "cuda":
            return self.model(x)
        entry = self._graphs.get(key)
        if entry is None:
            static_in = x.clone()
            s = torch.cuda.Stream(device=x.device)
            s.wait_stream(torch.cuda.current_stream(x.device))
            with torch.cuda.stream(s):
                for _ in range(2):  # warm up the allocator and any lazy init outside capture
                    self.model(static_in)
            torch.cuda.current_stream(x.device).wait_stream(s)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                static_out = self.model(static_in)
            entry = (g, static_in, static_out)
            self._graphs[key] = entry
        g, static_in, static_out = entry
        static_in.copy_(x)
        g.replay()
        return static_out


def compiled(model, int8: bool = False, graph: bool = False, fuse: bool = True, tune: bool = True) -> Compiled:
    """``torch.compiled(model, {int8, tune})`` of borch-ts (compile.ts:55-62, 570-578)."""
    return Compiled(model, int8=int8, graph=graph, fuse=fuse, tune=tune)
