"""``compiled(model, int8=True)`` — the prepare-then-run wrapper of borch-ts/src/compile.ts:570-578.

Prepare (once): ``model.eval()``, the model's own ``fuse()`` if it has one (the BN fold,
compile.ts:49-54 / nn.ts:6756), then with ``int8=True`` ``quantize_for_int8`` — the number
of layers that took the int8 path is kept as ``int8_layers`` (compile.ts:197-198) so a
timing is never quoted for an "int8" forward that was mostly f32.

Run: eager, or with ``graph=True`` a HIP graph captured on the first call for that
input shape and replayed afterwards (the reference's record/replay, device.ts:634-660):
the int8 forward is many small launches, and a replay issues them as one. As with any
captured graph, the returned tensor is the graph's own output buffer: the next call with
the same input shape overwrites it (clone it to keep it).

Split (``split=n``, graph mode): the batch runs as ``n`` chunks on parallel streams inside
the one graph, so one chunk's store- or latency-bound kernels overlap another's MFMA work
(each stream with its own split-K workspace). Refused where it would change the result:
a conv with a dynamic per-tensor input scale takes the maximum over the whole batch, so the
model needs calibrated scales (``calibrate_int8``) or per-row (Linear) quantization only.
Measured at n = 2: EfficientNet-B0 b64 calibrated 1.55 -> 1.41 ms, ViT-B/16 b32 3.09 ->
2.87 ms; ResNet-18 b16 (small launch-bound layers) is slower split.

Tune (``tune=True``, the default, as the reference's, compile.ts:55-62): before a shape's
first run on a GPU, the int8 GEMM / conv kernel of every distinct layer problem is chosen
by measurement (``borch_amd.tune``); ``tuned`` keeps the decisions, one list per shape.
The choice changes time only: every candidate computes the same result. Decisions persist
in a plan table on disk (``plan_cache``: a path, or by default ``tune.default_cache_path()``;
False keeps them in the process only), so a later process with the same device and library
times nothing (the reference's localStorage cache, device.ts:2689-2697, 2810-2831).
"""
from __future__ import annotations

import torch

from . import int8 as _i8
from .nn import Conv2d, _int8_layers, pairing, quantize_for_int8
from .tune import PlanCache
from .tune import tune as _tune


class Compiled:
    def __init__(self, model, int8: bool = False, graph: bool = False, fuse: bool = True, tune: bool = True,
                 split: int = 1, plan_cache=None):
        self.model = model
        self.plan_cache = None if plan_cache is False else PlanCache(plan_cache)
        self.int8 = int8
        self.graph = graph
        self.tune = tune
        self.split = int(split)
        if self.split < 1:
            raise ValueError(f"split must be >= 1, got {split}")
        self._streams = {}  # device -> [stream], made on its first split call (each with its own split-K workspace)
        self.tuned = []  # the tuner's decisions, one list per input shape (borch_amd.tune.tune)
        self._tuned_keys = set()
        self.int8_layers = 0
        model.eval()
        if fuse and callable(getattr(model, "fuse", None)):
            model.fuse()
        if int8:
            self.int8_layers = quantize_for_int8(model)
        self._graphs = {}

    def _split_ok(self, x) -> bool:
        if self.split == 1 or not self.graph or x.device.type != "cuda" or x.shape[0] < self.split:
            return False
        for _, m in _int8_layers(self.model):
            if isinstance(m, Conv2d) and m.int8 is not None and m.in_scale is None:
                raise ValueError("split needs a forward that is exact per batch chunk: the int8 conv "
                                 "layers need calibrated input scales (calibrate_int8); a dynamic "
                                 "per-tensor scale is the maximum over the whole batch")
        return True

    def _run(self, x):
        """The model on ``x``: whole, or as ``split`` chunks on parallel streams; two int8 convs
        of one input run as one launch (``pairing``)."""
        with pairing():
            return self._run_chunks(x)

    def _run_chunks(self, x):
        if not self._split_ok(x):
            return self.model(x)
        streams = self._streams.get(x.device)
        if streams is None:  # the warm-up runs come first, outside any capture
            streams = self._streams[x.device] = [torch.cuda.Stream(device=x.device) for _ in range(self.split)]
            for s in streams:  # each chunk stream's split-K workspace, made now (outside any capture)
                _i8.split_workspace(x.device, s)
        cur = torch.cuda.current_stream(x.device)
        outs = []
        for s, xc in zip(streams, x.chunk(self.split)):
            s.wait_stream(cur)
            with torch.cuda.stream(s):
                outs.append(self.model(xc))
        for s in streams:
            cur.wait_stream(s)
        return torch.cat(outs)

    @torch.no_grad()
    def __call__(self, x):
        key = (tuple(x.shape), x.dtype, x.device)
        if self.tune and x.device.type == "cuda" and key not in self._tuned_keys:
            self._tuned_keys.add(key)
            self.tuned.append(_tune(self.model, x.chunk(self.split)[0] if self._split_ok(x) else x,
                                    cache=self.plan_cache))
        if not self.graph or x.device.type != "cuda":
            return self._run(x)
        entry = self._graphs.get(key)
        if entry is None:
            static_in = x.clone()
            s = torch.cuda.Stream(device=x.device)
            s.wait_stream(torch.cuda.current_stream(x.device))
            with torch.cuda.stream(s):
                for _ in range(2):  # warm up the allocator and any lazy init outside capture
                    self._run(static_in)
            torch.cuda.current_stream(x.device).wait_stream(s)
            g = torch.cuda.CUDAGraph()
            # captured on the warm-up stream: the split-K workspace made for it is the one
            # the graph records
            with torch.cuda.graph(g, stream=s):
                static_out = self._run(static_in)
            entry = (g, static_in, static_out)
            self._graphs[key] = entry
        g, static_in, static_out = entry
        static_in.copy_(x)
        g.replay()
        return static_out


def compiled(model, int8: bool = False, graph: bool = False, fuse: bool = True, tune: bool = True,
             split: int = 1, plan_cache=None) -> Compiled:
    """``torch.compiled(model, {int8, tune})`` of borch-ts (compile.ts:55-62, 570-578); ``split``
    runs the batch as parallel chunks inside the graph; ``plan_cache`` is where tuning
    decisions persist (None: the default table, False: none)."""
    return Compiled(model, int8=int8, graph=graph, fuse=fuse, tune=tune, split=split, plan_cache=plan_cache)
