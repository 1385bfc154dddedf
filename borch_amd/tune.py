"""Kernel choice by measurement for the int8 GEMM / conv kernels.

The library picks the tiled kernel's configuration (tile, ring depth) and K split per
problem by rule. ``tune(model, x)`` records the int8 launches of one forward, times every
candidate of each distinct problem on the device (HIP graphs of back-to-back launches,
HIP events), and records the fastest as the problem's plan (``bq_plan_set``) when it beats
the rule's pick by more than ``min_gain``; otherwise the rule stays. All candidates compute
the same exact int32 sums and the same epilogue, so tuning changes time only, never a
result.

Mirrors the reference's ``Device.choose`` / ``runTuning`` (borch-ts/src/device.ts:2686-2700,
2834-2846: the rule's pick first, the fastest cached per key) and ``compiled``'s ``tune``
option (borch-ts/src/compile.ts:55-62), with one report per decision like its
``TuneReport`` (device.ts:532-536).

Decisions persist in a JSON table (``PlanCache``), as the reference keeps them per adapter
in memory and in ``localStorage`` (device.ts:2689-2697, 2810-2831): keyed by the device
(architecture and compute-unit count), the built library (a hash of ``libbq.so``: a rebuild
may change what is fastest) and the problem. A later ``tune`` (a later process) takes a
stored decision without timing anything; a stored plan the library no longer offers is
ignored and the problem is timed again.
"""
from __future__ import annotations

import ctypes
import hashlib
import inspect
import json
import os
import tempfile
from pathlib import Path

import torch

from . import int8 as _i8
from ._lib import check, lib

# the borch_amd.int8 wrappers that launch a layer's int8 kernel on an int8 input
LAYER_KERNELS = ("conv2d_i8_nhwc", "conv2d_i8_nhwc_q", "conv2d_i8_nhwc_dq", "conv2d_nchw_fq", "dwconv_i8_nhwc",
                 "gemm_i8")


def record_launches(model, x):
    """One eager forward of ``model`` with the wrappers in ``LAYER_KERNELS`` recording their
    bound arguments: ``[(layer name, wrapper name, wrapper, arguments)]`` in launch order."""
    from . import nn as bnn
    calls, current, saved, hooks, by_w = [], [""], {}, [], {}
    for name, m in model.named_modules():
        if isinstance(m, (bnn.Conv2d, bnn.Linear)):
            hooks.append(m.register_forward_pre_hook(lambda mod, inp, _n=name: current.__setitem__(0, _n)))
            if getattr(m, "int8", None) is not None:
                by_w[id(m.int8)] = name  # names a launch made without the module's own call
    for n in LAYER_KERNELS:
        f = saved[n] = getattr(_i8, n)

        def rec(*a, _f=f, _n=n, **k):
            bound = inspect.signature(_f).bind(*a, **k)
            bound.apply_defaults()
            r = _f(*a, **k)  # recorded once it ran: a call the kernel refused is not a launch
            w = bound.arguments.get("wq", bound.arguments.get("w8"))
            calls.append((by_w.get(id(w), current[0]), _n, _f, dict(bound.arguments)))
            return r
        setattr(_i8, n, rec)
    try:
        with torch.no_grad():
            model(x)
    finally:
        for n, f in saved.items():
            setattr(_i8, n, f)
        for h in hooks:
            h.remove()
    return calls


def problem_of(kind: str, a: dict):
    """The plan key of a recorded launch: (M, N, K) for a dense GEMM, (N, H, W, Cpad, O, KH,
    KW, stride, pad) for a conv; None where there is no tiled kernel to choose."""
    if kind == "gemm_i8":
        M, K = a["qa"].shape
        return (int(M), int(a["qw"].shape[0]), int(K)) if M > 64 else None
    if kind in ("conv2d_i8_nhwc", "conv2d_i8_nhwc_q"):
        n, h, w, c = a["qx"].shape
        wq = a["wq"]
        return (int(n), int(h), int(w), int(c), int(wq.O), int(wq.KH), int(wq.KW), int(a["stride"]), int(a["pad"]))
    return None


def _arr(problem):
    return (ctypes.c_int64 * len(problem))(*problem)


def candidates(problem) -> list[tuple[int, int]]:
    """(configuration id, K split) pairs the library offers for ``problem``; the rule's pick first."""
    n = lib().bq_plan_candidates(_arr(problem), len(problem), None, None, 0)
    if n < 0:
        check(n)
    if n == 0:
        return []
    cfgs, splits = (ctypes.c_int32 * n)(), (ctypes.c_int32 * n)()
    lib().bq_plan_candidates(_arr(problem), len(problem), cfgs, splits, n)
    return list(zip(cfgs, splits))


def set_plan(problem, cfg: int, split: int) -> None:
    """Records the plan for ``problem``; ``cfg == 0`` returns it to the rule."""
    check(lib().bq_plan_set(_arr(problem), len(problem), int(cfg), int(split)))


def clear_plans() -> None:
    check(lib().bq_plan_clear())


def _time_us(fn, a, stream, calls: int, rounds: int) -> float:
    """Microseconds per launch of ``fn(**a)``: a HIP graph of ``calls`` launches, the
    minimum over ``rounds`` timed replays."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn(**a)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):  # the warm-up stream: the splits timed are the splits that run
        for _ in range(calls):
            fn(**a)
    g.replay()
    best = float("inf")
    for _ in range(rounds):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        g.replay()
        e1.record(stream)
        e1.synchronize()
        best = min(best, e0.elapsed_time(e1) * 1e3 / calls)
    del g
    return best


def _label(c) -> str:
    return f"cfg{c[0]}/split{c[1]}"


PLAN_FORMAT = "borch_amd-plans/1"
_LIB_ID = None


def library_id() -> str:
    """The built library's identity: the first 16 hex digits of the SHA-256 of libbq.so."""
    global _LIB_ID
    if _LIB_ID is None:
        from ._lib import LIB_PATH
        _LIB_ID = hashlib.sha256(Path(LIB_PATH).read_bytes()).hexdigest()[:16]
    return _LIB_ID


def device_id(device) -> str:
    props = torch.cuda.get_device_properties(device)
    return f"{getattr(props, 'gcnArchName', props.name)}/{props.multi_processor_count}cu"


def default_cache_path() -> Path:
    """``$BORCH_AMD_PLAN_CACHE``, else ``~/.cache/borch_amd/plans.json``."""
    env = os.environ.get("BORCH_AMD_PLAN_CACHE")
    return Path(env) if env else Path.home() / ".cache" / "borch_amd" / "plans.json"


class PlanCache:
    """Tuning decisions on disk: ``{"format", "tables": {"<device>|<library>": {"<problem>":
    {"cfg", "split", "rule_us", "chosen_us"}}}}``. ``cfg == 0`` records that the rule's
    pick stays. Writes merge with what is on disk and replace the file atomically."""

    def __init__(self, path=None):
        self.path = Path(path) if path is not None else default_cache_path()

    def _read(self) -> dict:
        try:
            data = json.loads(self.path.read_text())
        except (OSError, ValueError):
            return {"format": PLAN_FORMAT, "tables": {}}
        if not isinstance(data, dict) or data.get("format") != PLAN_FORMAT or not isinstance(data.get("tables"), dict):
            return {"format": PLAN_FORMAT, "tables": {}}
        return data

    @staticmethod
    def _table_key(device) -> str:
        return f"{device_id(device)}|{library_id()}"

    def load(self, device) -> dict:
        """{problem tuple: entry} stored for this device and library."""
        table = self._read()["tables"].get(self._table_key(device), {})
        out = {}
        for k, v in table.items():
            try:
                out[tuple(int(t) for t in k.split(","))] = {"cfg": int(v["cfg"]), "split": int(v["split"]),
                                                            "rule_us": float(v["rule_us"]),
                                                            "chosen_us": float(v["chosen_us"])}
            except (KeyError, TypeError, ValueError):
                continue
        return out

    def store(self, device, entries: dict) -> bool:
        """Adds ``{problem: entry}`` to the table; False (and nothing written) if the file
        cannot be written."""
        if not entries:
            return True
        data = self._read()
        table = data["tables"].setdefault(self._table_key(device), {})
        for problem, e in entries.items():
            table[",".join(str(int(t)) for t in problem)] = e
        try:
            self.path.parent.mkdir(parents=True, exist_ok=True)
            fd, tmp = tempfile.mkstemp(dir=str(self.path.parent), prefix=".plans-", suffix=".json")
            with os.fdopen(fd, "w") as f:
                json.dump(data, f, indent=1, sort_keys=True)
            os.replace(tmp, self.path)
        except OSError:
            return False
        return True


def tune(model, x, min_gain: float = 0.03, calls: int = 8, rounds: int = 3, cache: PlanCache | None = None) -> list[dict]:
    """Times every candidate of each distinct int8 problem in one forward of ``model`` on
    ``x`` and keeps the fastest when it is more than ``min_gain`` faster than the rule's
    pick. With ``cache``, a decision stored for this device and library is taken as it
    stands (nothing timed) and new decisions are stored. Returns one report per decision:
    key, prior, prior_us, chosen, chosen_us, candidates, cached."""
    if x.device.type != "cuda":
        return []
    _i8.split_workspace(x.device)  # the splits timed here are the splits that run later
    stream = torch.cuda.current_stream(x.device)
    stored = cache.load(x.device) if cache is not None else {}
    new_entries = {}
    reports, seen = [], set()
    for layer, kind, fn, a in record_launches(model, x):
        problem = problem_of(kind, a)
        if problem is None or problem in seen:
            continue
        seen.add(problem)
        cands = candidates(problem)
        if len(cands) < 2:
            continue
        e = stored.get(problem)
        if e is not None and (e["cfg"] == 0 or (e["cfg"], e["split"]) in cands):
            chosen = (e["cfg"], e["split"]) if e["cfg"] else cands[0]
            set_plan(problem, *(chosen if e["cfg"] else (0, 0)))
            reports.append({"key": problem, "layer": layer, "prior": _label(cands[0]), "prior_us": e["rule_us"],
                            "chosen": _label(chosen), "chosen_us": e["chosen_us"], "candidates": len(cands),
                            "cached": True})
            continue
        set_plan(problem, 0, 0)
        times = []
        for c in cands:
            set_plan(problem, *c)
            times.append(_time_us(fn, a, stream, calls, rounds))
        best = min(range(len(cands)), key=times.__getitem__)
        if best != 0:  # confirm against the rule's pick, back to back
            set_plan(problem, *cands[0])
            times[0] = min(times[0], _time_us(fn, a, stream, calls, rounds))
            set_plan(problem, *cands[best])
            times[best] = min(times[best], _time_us(fn, a, stream, calls, rounds))
        chosen = best if times[best] < times[0] * (1.0 - min_gain) else 0
        if chosen:
            set_plan(problem, *cands[chosen])
        else:
            set_plan(problem, 0, 0)
        reports.append({"key": problem, "layer": layer, "prior": _label(cands[0]), "prior_us": round(times[0], 2),
                        "chosen": _label(cands[chosen]), "chosen_us": round(times[chosen], 2),
                        "candidates": len(cands), "cached": False})
        new_entries[problem] = {"cfg": int(cands[chosen][0]) if chosen else 0,
                                "split": int(cands[chosen][1]) if chosen else 0,
                                "rule_us": round(times[0], 2), "chosen_us": round(times[chosen], 2)}
    torch.cuda.synchronize(x.device)
    if cache is not None:
        cache.store(x.device, new_entries)
    return reports
