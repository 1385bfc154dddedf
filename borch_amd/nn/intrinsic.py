"""Fused modules in the place of ``torch.ao.nn.intrinsic`` (borch-ts/src/nn.ts:6698-6750).

Each wraps a (BN-folded) conv or linear and fuses the ReLU and/or the residual add into
its kernel's epilogue: ``y = ((f32(acc)·sA)·sW) + b (+ residual)``, then ReLU
(kernels.ts:4230-4244's ``ConvEpilogue`` order). On the f32 path the same arithmetic
runs as separate torch ops.
"""
from __future__ import annotations

import torch.nn as _tnn

from .. import int8 as _i8


class ConvReLU2d(_tnn.Module):
    """``relu(conv(x))`` in one kernel (nn.ts:6698-6711)."""

    def __init__(self, conv, relu=None):
        super().__init__()
        self.conv = conv
        self.conv.act = _i8.ACT_RELU
        self.training = False

    def forward(self, x):
        return self.conv(x)


class ConvAdd2d(_tnn.Module):
    """``conv(x1) + x2`` in one kernel (nn.ts:6717-6731)."""

    def __init__(self, conv):
        super().__init__()
        self.conv = conv
        self.conv.act = _i8.ACT_NONE
        self.training = False

    def forward(self, x, residual=None, channel_scale=None):
        if residual is None:
            raise TypeError("ConvAdd2d.forward takes (x1, x2)")
        return self.conv(x, residual, channel_scale)


class ConvAddReLU2d(_tnn.Module):
    """``relu(conv(x1) + x2)`` in one kernel (nn.ts:6736-6750)."""

    def __init__(self, conv):
        super().__init__()
        self.conv = conv
        self.conv.act = _i8.ACT_RELU
        self.training = False

    def forward(self, x, residual=None):
        if residual is None:
            raise TypeError("ConvAddReLU2d.forward takes (x1, x2)")
        return self.conv(x, residual)


class LinearReLU(_tnn.Module):
    """``relu(linear(x))`` in one kernel (torch.ao.nn.intrinsic.LinearReLU)."""

    def __init__(self, linear, relu=None):
        super().__init__()
        self.linear = linear
        self.linear.act = _i8.ACT_RELU
        self.training = False

    def forward(self, x):
        return self.linear(x)


class ConvSiLU2d(_tnn.Module):
    """``silu(conv(x))`` in one kernel: the SiLU is evaluated in f32 in the epilogue
    (EfficientNet's conv-BN-SiLU after the BN fold). Not a torch.ao name; the same shape
    as ``ConvReLU2d``."""

    def __init__(self, conv):
        super().__init__()
        self.conv = conv
        self.conv.act = _i8.ACT_SILU
        self.training = False

    def forward(self, x):
        return self.conv(x)


class LinearGELU(_tnn.Module):
    """``gelu(linear(x))`` in one kernel: the erf GELU evaluated in f32 in the epilogue (a
    transformer MLP's first projection). Not a torch.ao name; the shape of ``LinearReLU``."""

    def __init__(self, linear):
        super().__init__()
        self.linear = linear
        self.linear.act = _i8.ACT_GELU
        self.training = False

    def forward(self, x):
        return self.linear(x)


class LinearAdd(_tnn.Module):
    """``linear(x1) + x2`` in one kernel (a transformer's projection and skip connection):
    the Linear counterpart of ``ConvAdd2d`` (nn.ts:6717-6731)."""

    def __init__(self, linear):
        super().__init__()
        self.linear = linear
        self.linear.act = _i8.ACT_NONE
        self.training = False

    def forward(self, x, residual=None, pre_act=None):
        if residual is None:
            raise TypeError("LinearAdd.forward takes (x1, x2)")
        return self.linear(x, residual, pre_act=pre_act)
