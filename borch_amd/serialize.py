"""On-disk format for int8-packed weights (the reference's hub manifest
``weights.quant: "int8-perchannel"``, docs/SCALE.md:541-544): quantize once, ship the
packing, and let a later prepare attach it without re-quantizing.

The file is safetensors:

* for every int8 layer ``name``: ``{name}.q`` (I8, the packed layout the kernels read)
  and ``{name}.scale`` (F32, one scale per output channel);
* metadata ``{"quant": "int8-perchannel", "format": "borch_amd-int8/1"}`` plus, per
  layer, ``{name}`` -> a JSON record of the kind (``linear`` / ``conv`` / ``dw``) and its
  geometry, checked against the model on load.

The reference itself re-quantizes from f32 at every ``quantizeForInt8``
(nn.ts:6770-6780); loading this file gives the same bytes as quantizing (the packing is
deterministic), which ``tests/`` check bit for bit.
"""
from __future__ import annotations

import json

import torch
from safetensors.torch import load_file, save_file

from . import int8 as _i8
from .nn import _int8_layers

FORMAT = "borch_amd-int8/1"


def _record(w8) -> dict:
    if isinstance(w8, _i8.Int8Weight):
        rec = {"kind": "linear", "in_features": w8.in_features, "out_features": w8.out_features,
               "weight_only": bool(w8.weight_only)}
        if w8.per_tensor:
            rec["per_tensor"] = True
        return rec
    if isinstance(w8, _i8.Int8ConvWeight):
        return {"kind": "conv", "O": w8.O, "C": w8.C, "cpad": w8.cpad, "KH": w8.KH, "KW": w8.KW}
    if isinstance(w8, _i8.Int8DwWeight):
        return {"kind": "dw", "C": w8.C, "cpad": w8.cpad, "KH": w8.KH, "KW": w8.KW}
    raise TypeError(f"not an int8 weight: {type(w8).__name__}")


def save_int8(model, path) -> int:
    """Writes every int8-packed layer of ``model``; returns how many were written."""
    tensors, meta = {}, {"quant": "int8-perchannel", "format": FORMAT}
    n = 0
    for name, mod in _int8_layers(model):
        if mod.int8 is None:
            continue
        tensors[f"{name}.q"] = mod.int8.q.detach().contiguous().cpu()
        tensors[f"{name}.scale"] = mod.int8.s.detach().contiguous().cpu()
        meta[name] = json.dumps(_record(mod.int8))
        n += 1
    save_file(tensors, str(path), metadata=meta)
    return n


def _expected(mod) -> dict:
    if isinstance(mod, _i8_nn_linear()):
        return {"kind": "linear", "in_features": mod.in_features, "out_features": mod.out_features}
    O, Cg, KH, KW = mod.weight.shape
    if mod.groups == 1:
        return {"kind": "conv", "O": O, "C": Cg, "cpad": _i8.round_up(Cg, 16), "KH": KH, "KW": KW}
    return {"kind": "dw", "C": O, "cpad": _i8.round_up(O, 4), "KH": KH, "KW": KW}


def _packed_shapes(rec: dict):
    """(q shape, scale shape) of the packing a geometry record describes: a Linear's
    ``[out, Kpad]`` (Kpad = in rounded up to 16, at least 16) and ``[out]``; a conv's
    ``[O, KH*KW*cpad]`` and ``[O]``; a depthwise conv's ``[KH*KW, cpad]`` and ``[cpad]``."""
    kind = rec["kind"]
    if kind == "linear":
        return (rec["out_features"], _i8.round_up(max(rec["in_features"], 16), 16)), (rec["out_features"],)
    if kind == "conv":
        return (rec["O"], rec["KH"] * rec["KW"] * rec["cpad"]), (rec["O"],)
    return (rec["KH"] * rec["KW"], rec["cpad"]), (rec["cpad"],)


def _i8_nn_linear():
    from .nn import Linear
    return Linear


def load_int8(model, path, device=None) -> int:
    """Attaches the packed weights in ``path`` to the matching layers of ``model`` (no
    quantization runs); returns how many layers were loaded. A layer whose geometry does
    not match the file raises ``ValueError``; a layer absent from the file is left as is."""
    from safetensors import safe_open
    with safe_open(str(path), framework="pt") as f:
        meta = f.metadata() or {}
    if meta.get("quant") != "int8-perchannel":
        raise ValueError(f"{path}: not an int8-perchannel file (quant={meta.get('quant')!r})")
    tensors = load_file(str(path))
    n = 0
    for name, mod in _int8_layers(model):
        if name not in meta:
            continue
        rec = json.loads(meta[name])
        want = _expected(mod)
        if rec.get("kind") == "linear":
            want["weight_only"] = bool(rec.get("weight_only", False))
            if rec.get("per_tensor"):
                want["per_tensor"] = True
        if rec != want:
            raise ValueError(f"{path}: layer {name!r} is {rec}, the model has {want}")
        dev = device if device is not None else mod.weight.device
        q = tensors[f"{name}.q"].to(dev)
        s = tensors[f"{name}.scale"].to(dev)
        if q.dtype != torch.int8 or s.dtype != torch.float32:
            raise ValueError(f"{path}: layer {name!r} has dtypes {q.dtype}/{s.dtype}")
        kind = rec["kind"]
        # The kernels take their sizes from the record, not from the tensors: a tensor of
        # any other shape would be read past its end.
        want_q, want_s = _packed_shapes(rec)
        if tuple(q.shape) != want_q or tuple(s.shape) != want_s:
            raise ValueError(f"{path}: layer {name!r} has q {tuple(q.shape)} / scale {tuple(s.shape)}, "
                             f"its geometry needs {want_q} / {want_s}")
        if kind == "linear":
            mod.int8 = _i8.Int8Weight(q, s, rec["in_features"], rec["out_features"], rec.get("weight_only", False),
                                      bool(rec.get("per_tensor", False)))
        elif kind == "conv":
            mod.int8 = _i8.Int8ConvWeight(q, s, rec["O"], rec["C"], rec["cpad"], rec["KH"], rec["KW"])
        else:
            mod.int8 = _i8.Int8DwWeight(q, s, rec["C"], rec["cpad"], rec["KH"], rec["KW"])
        n += 1
    return n
