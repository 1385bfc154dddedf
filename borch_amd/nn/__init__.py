"""``borch_amd.nn`` — the operator surface of the int8 path, shaped like the numpy core's.

``Linear`` and ``Conv2d`` keep the numpy core's constructor and forward signatures
(borch/_nn.py:397-415, 1156-1190) over PyTorch-ROCm parameters. Each can be quantized
once for the int8 path (``quantize_int8()``, the prepare of borch-ts/src/nn.ts:967-980);
after that its forward runs the HIP kernels (W8A8 GEMM / implicit-GEMM conv / depthwise)
and otherwise the float32 op. The model-level calls mirror borch-ts/src/nn.ts:6770-6829:

* ``quantize_for_int8(model) -> int`` — quantizes every layer the kernels take and
  returns the count; refuses by name on a device without the int8 kernels;
* ``clear_int8(model)`` — back to float32 (the f32 weights never left);
* ``int8_report(model)`` — which layers took the path and why the others did not.

Every other ``torch.nn`` name (``ReLU``, ``Sequential``, ``BatchNorm2d``, ...) is torch's
own, re-exported unchanged: only the int8 path is this package's.
"""
from __future__ import annotations

import math

import torch
import torch.nn as _tnn

from .. import int8 as _i8
from .._lib import Int8Unavailable, require_device
from . import functional  # noqa: F401
from . import intrinsic  # noqa: F401
from . import utils  # noqa: F401

Module = _tnn.Module
Parameter = _tnn.Parameter


def _pair(v):
    if isinstance(v, (tuple, list)):
        if len(v) != 2:
            raise ValueError(f"expected a pair, got {v!r}")
        return int(v[0]), int(v[1])
    return int(v), int(v)


class Linear(_tnn.Module):
    """``nn.Linear(in_features, out_features, bias=True)``; forward ``x @ W.T + b``
    (borch/_nn.py:397-415). Init U(−1/√in, 1/√in) for weight and bias, as the core's."""

    def __init__(self, in_features, out_features, bias=True, device=None, dtype=None):
        super().__init__()
        self.in_features = int(in_features)
        self.out_features = int(out_features)
        bound = 1.0 / math.sqrt(in_features) if in_features else 0.0
        self.weight = Parameter(torch.empty((out_features, in_features), device=device,
                                            dtype=dtype or torch.float32).uniform_(-bound, bound))
        self.bias = (Parameter(torch.empty((out_features,), device=device, dtype=dtype or torch.float32)
                               .uniform_(-bound, bound)) if bias else None)
        self.int8 = None  # Int8Weight once quantize_int8() has run
        self.act = _i8.ACT_NONE  # fused epilogue activation (LinearReLU sets RELU)

    def quantize_int8(self) -> bool:
        """Packs the weight once per output channel (quant.ts:23-53). Any shape is taken
        (K is zero-padded to a multiple of 16). Returns True."""
        require_device(self.weight.device)
        with torch.no_grad():
            self.int8 = _i8.pack_linear_weight(self.weight.detach())
        return True

    def forward(self, x):
        if self.int8 is not None:
            return _i8.linear(x, self.int8, self.bias, self.act)
        out = functional._f32_linear(x, self.weight, self.bias)
        return torch.relu(out) if self.act == _i8.ACT_RELU else out

    def extra_repr(self):
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"bias={self.bias is not None}" + (", int8" if self.int8 is not None else ""))


class Conv2d(_tnn.Module):
    """``nn.Conv2d(in, out, kernel_size, stride=1, padding=0, dilation=1, groups=1,
    bias=True, padding_mode='zeros')`` (borch/_nn.py:1156-1190)."""

    def __init__(self, in_channels, out_channels, kernel_size, stride=1, padding=0, dilation=1,
                 groups=1, bias=True, padding_mode="zeros", device=None, dtype=None):
        super().__init__()
        if padding_mode not in ("zeros", "reflect", "replicate", "circular"):
            raise ValueError("padding_mode has to be one of ('zeros', 'reflect', 'replicate', 'circular'), "
                             f"got {padding_mode!r}")
        if in_channels % groups or out_channels % groups:
            raise ValueError("in_channels and out_channels must be divisible by groups")
        self.in_channels, self.out_channels = int(in_channels), int(out_channels)
        self.kernel_size, self.stride, self.padding = kernel_size, stride, padding
        self.dilation, self.groups, self.padding_mode = dilation, int(groups), padding_mode
        kh, kw = _pair(kernel_size)
        fan_in = (in_channels // groups) * kh * kw
        bound = 1.0 / math.sqrt(fan_in) if fan_in else 0.0
        dt = dtype or torch.float32
        self.weight = Parameter(torch.empty((out_channels, in_channels // groups, kh, kw), device=device,
                                            dtype=dt).uniform_(-bound, bound))
        self.bias = Parameter(torch.empty((out_channels,), device=device, dtype=dt)
                              .uniform_(-bound, bound)) if bias else None
        self.int8 = None  # Int8ConvWeight / Int8DwWeight once quantize_int8() has run
        self.act = _i8.ACT_NONE

    def _geometry(self):
        """(stride, pad) when square and zero-padded, else None."""
        sh, sw = _pair(self.stride)
        if isinstance(self.padding, str):
            if self.padding == "valid":
                ph = pw = 0
            else:
                return None
        else:
            ph, pw = _pair(self.padding)
        if sh != sw or ph != pw or self.padding_mode != "zeros" or _pair(self.dilation) != (1, 1):
            return None
        return sh, ph

    def int8_refusal(self):
        """Why the int8 kernels do not take this layer (None if they do)."""
        if self._geometry() is None:
            return "stride/padding not square, dilation != 1 or non-zero padding mode"
        if self.groups == 1:
            return None
        if self.groups == self.in_channels == self.out_channels:
            return None
        return f"groups={self.groups} (only 1 or depthwise)"

    def quantize_int8(self) -> bool:
        """Packs the weight once per output channel (quant.ts:80-103's scale rule) where
        the kernels take the layer; returns False (the layer stays f32) otherwise, as
        borch-ts/src/nn.ts:967-980 does."""
        if self.int8_refusal() is not None:
            return False
        require_device(self.weight.device)
        with torch.no_grad():
            w = self.weight.detach()
            self.int8 = _i8.pack_conv_weight(w) if self.groups == 1 else _i8.pack_dw_weight(w)
        return True

    def forward(self, x, residual=None):
        if self.int8 is not None:
            stride, pad = self._geometry()
            if isinstance(self.int8, _i8.Int8DwWeight):
                out = _i8.depthwise_conv2d(x, self.int8, self.bias, stride, pad,
                                           self.act if residual is None else _i8.ACT_NONE)
                if residual is not None:
                    out = out + residual
                    if self.act == _i8.ACT_RELU:
                        out = torch.relu(out)
                return out
            return _i8.conv2d(x, self.int8, self.bias, stride, pad, self.act, residual)
        out = functional._f32_conv2d(x, self.weight, self.bias, self.stride, self.padding, self.dilation,
                                     self.groups, self.padding_mode)
        if residual is not None:
            out = out + residual
        if self.act == _i8.ACT_RELU:
            out = torch.relu(out)
        elif self.act == _i8.ACT_SILU:
            out = torch.nn.functional.silu(out)
        return out

    def extra_repr(self):
        s = (f"{self.in_channels}, {self.out_channels}, kernel_size={self.kernel_size}, "
             f"stride={self.stride}, padding={self.padding}")
        if self.groups != 1:
            s += f", groups={self.groups}"
        return s + (", int8" if self.int8 is not None else "")


def _int8_layers(model):
    """Every Linear / Conv2d of this package in ``model`` that is not marked
    ``int8_exempt`` (a layer the configuration keeps in f32, e.g. a classifier head)."""
    for name, mod in model.named_modules():
        if isinstance(mod, (Linear, Conv2d)) and not getattr(mod, "int8_exempt", False):
            yield name, mod


def quantize_for_int8(model, linear: bool = True, conv: bool = True) -> int:
    """Every Linear / Conv2d of ``model`` the int8 kernels take, quantized once; returns
    how many took it (borch-ts/src/nn.ts:6770-6780). Refused by name where the device has
    no int8 kernels (nn.ts:6771-6773): the path is an accuracy trade a caller asks for and
    must not silently become the f32 forward."""
    layers = list(_int8_layers(model))
    dev = next((m.weight.device for _, m in layers), None)
    if dev is not None:
        try:
            require_device(dev)
        except Int8Unavailable as e:
            raise Int8Unavailable(f"int8: this device has no int8 kernels ({e}) — "
                                  "the int8 forward is not available here") from None
    taken = 0
    for _, mod in layers:
        if isinstance(mod, Linear) and linear:
            taken += bool(mod.quantize_int8())
        elif isinstance(mod, Conv2d) and conv:
            taken += bool(mod.quantize_int8())
    return taken


def clear_int8(model) -> None:
    """Back to f32: every layer's int8 weight dropped (nn.ts:6827-6829)."""
    for _, mod in _int8_layers(model):
        mod.int8 = None


def int8_report(model):
    """``[(name, kind, took_int8, reason)]`` for every Linear / Conv2d."""
    rows = []
    for name, mod in _int8_layers(model):
        kind = type(mod).__name__
        why = None if isinstance(mod, Linear) else mod.int8_refusal()
        rows.append((name, kind, mod.int8 is not None, why))
    return rows


def __getattr__(name):
    return getattr(_tnn, name)
