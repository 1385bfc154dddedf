"""``nn.utils.fusion`` — the eval-mode batch-norm fold (borch/_nn.py:4916-4955).

``scale = γ / √(running_var + eps)``, ``W' = W·scale`` per output channel,
``b' = (b − mean)·scale + β``; a conv without bias folds with zeros, a norm without affine
weights with γ = 1, β = 0. Computed on the tensors' own device in float32.
"""
from __future__ import annotations

import copy

import torch


def fuse_conv_bn_weights(conv_w, conv_b, bn_rm, bn_rv, bn_eps, bn_w, bn_b, transpose=False):
    """Returns ``(Parameter W', Parameter b')`` (borch/_nn.py:4916-4937)."""
    w = conv_w.detach()
    rm, rv = bn_rm.detach(), bn_rv.detach()
    b = torch.zeros_like(rm) if conv_b is None else conv_b.detach()
    gamma = torch.ones_like(rm) if bn_w is None else bn_w.detach()
    beta = torch.zeros_like(rm) if bn_b is None else bn_b.detach()
    scale = (gamma / torch.sqrt(rv + bn_eps)).to(w.dtype)
    shape = [1, -1] + [1] * (w.dim() - 2) if transpose else [-1, 1] + [1] * (w.dim() - 2)
    fused_w = (w * scale.reshape(shape)).to(w.dtype)
    fused_b = ((b - rm) * scale + beta).to(b.dtype)
    return torch.nn.Parameter(fused_w), torch.nn.Parameter(fused_b)


def fuse_conv_bn_eval(conv, bn, transpose=False):
    """A new conv with ``bn`` folded in, for inference (borch/_nn.py:4940-4955)."""
    if conv.training or bn.training:
        raise AssertionError("Fusion only for eval!")
    if bn.running_mean is None or bn.running_var is None:
        raise AssertionError("bn.running_mean and bn.running_var must not be None")
    fused = copy.deepcopy(conv)
    fused.weight, fused.bias = fuse_conv_bn_weights(
        fused.weight, fused.bias, bn.running_mean, bn.running_var, bn.eps, bn.weight, bn.bias, transpose)
    # An int8 packing (and calibrated scales) describe the unfolded weights: the copy must
    # not keep running them. It is re-packed from the folded weights when the original was
    # packed, and its scales are dropped (they measured the unfolded layer's output).
    packed = getattr(fused, "int8", None) is not None
    for attr in ("int8", "in_scale", "out_scale", "in_scale_v", "out_scale_v", "_calib"):
        if hasattr(fused, attr):
            setattr(fused, attr, None)
    if packed:
        fused.quantize_int8()
    return fused
