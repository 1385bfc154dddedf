"""``borch_amd.nn.functional`` — ``linear`` and ``conv2d`` with the numpy core's signatures
(borch/_nn.py:4675-4677, borch/_ops.py:738-791), plus their int8 forms.

``linear(input, weight, bias=None)`` and ``conv2d(input, weight, bias=None, stride=1,
padding=0, dilation=1, groups=1)`` take a float32 weight (the f32 op, torch-ROCm) or a
packed int8 weight (``borch_amd.int8.Int8Weight`` / ``Int8ConvWeight`` /
``Int8DwWeight``), which routes to the HIP kernels. Every other name is torch's.
"""
from __future__ import annotations

import torch
import torch.nn.functional as _tF

from .. import int8 as _i8
from .. import streaming as _stream


def _f32_linear(x, w, b=None):
    if x.shape[-1] != w.shape[-1]:
        a = "x".join(str(n) for n in x.reshape(-1, x.shape[-1]).shape)
        raise RuntimeError(f"mat1 and mat2 shapes cannot be multiplied ({a} and {w.shape[1]}x{w.shape[0]})")
    return _tF.linear(x, w, b)


def _f32_conv2d(x, w, b=None, stride=1, padding=0, dilation=1, groups=1, padding_mode="zeros"):
    if x.dim() == 4 and x.shape[1] != w.shape[1] * groups:
        raise RuntimeError(f"channels do not match: input {x.shape[1]}, filter {w.shape[1] * groups}")
    if padding_mode != "zeros" and not isinstance(padding, str):
        ph, pw = (padding, padding) if isinstance(padding, int) else padding
        x = _tF.pad(x, (pw, pw, ph, ph), mode=padding_mode)
        padding = 0
    return _tF.conv2d(x, w, b, stride, padding, dilation, groups)


def linear(input, weight, bias=None):  # noqa: A002
    """``input @ weight.T + bias``; an ``Int8Weight`` runs the W8A8 kernels (or the W8A32
    one when packed weight-only), a windowed int8 weight (``streaming.in_window_int8``) the
    W8A32 kernel on its window slot."""
    if isinstance(weight, _i8.Int8Weight):
        return _i8.linear(input, weight, bias)
    if isinstance(weight, _stream.WindowedWeight):
        return _stream._linear(input, weight, bias)
    return _f32_linear(input, weight, bias)


def conv2d(input, weight, bias=None, stride=1, padding=0, dilation=1, groups=1):  # noqa: A002
    """The 2-D convolution; an ``Int8ConvWeight`` / ``Int8DwWeight`` runs the int8 kernels
    (square stride and zero padding, dilation 1)."""
    if isinstance(weight, (_i8.Int8ConvWeight, _i8.Int8DwWeight)):
        st = stride if isinstance(stride, int) else stride[0]
        pd = padding if isinstance(padding, int) else padding[0]
        if (not isinstance(stride, int) and len(set(stride)) != 1) or \
                (not isinstance(padding, int) and len(set(padding)) != 1) or dilation not in (1, (1, 1)):
            raise NotImplementedError("int8 conv2d takes square stride/padding and dilation 1")
        if isinstance(weight, _i8.Int8DwWeight):
            return _i8.depthwise_conv2d(input, weight, bias, st, pd)
        if groups != 1:
            raise NotImplementedError("int8 conv2d with groups != 1 takes a depthwise weight")
        return _i8.conv2d(input, weight, bias, st, pd)
    return _f32_conv2d(input, weight, bias, stride, padding, dilation, groups)


def __getattr__(name):
    return getattr(_tF, name)
