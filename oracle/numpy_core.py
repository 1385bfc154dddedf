"""The reference numpy core's f32 forward, restated — TEST AND MEASUREMENT INFRASTRUCTURE ONLY.

Only ``tests/`` and ``bench.py``'s CPU-baseline leg import this module. It is the f32
arithmetic borch's numpy core runs for the two operators on the int8 path, on the host:

* ``linear``: ``x @ W.T + b`` through numpy's BLAS (borch/_nn.py:413-415, F.linear
  borch/_nn.py:4675-4677);
* ``conv2d``: zero padding (borch/_ops.py:661-668), ``_im2col`` as a strided sliding-window
  view transposed to ``(N, OH, OW, C, KH, KW)`` rows (borch/_ops.py:671-689), one GEMM
  against ``W.reshape(F, -1).T``, back to NCHW, then the bias (borch/_ops.py:738-791);
* the CIFAR ResNet-18 forward of configuration C3 (tests/browser/export_resnet18.py:27-60)
  composed of those, with the folded convs' biases, ReLU, the residual sum, the mean over
  H, W and the Linear head.
"""
from __future__ import annotations

import numpy as np


def linear(x, w, b=None):
    """``x @ W.T (+ b)`` in float32 (borch/_nn.py:413-415)."""
    y = np.asarray(x, np.float32) @ np.asarray(w, np.float32).T
    return y if b is None else y + np.asarray(b, np.float32)


def im2col(xd, KH, KW, stride):
    """(N, C, H, W) -> (N*OH*OW, C*KH*KW) rows, channel-major then filter row and column
    within a row (borch/_ops.py:671-689, dilation 1)."""
    N, C, H, W = xd.shape
    OH = (H - KH) // stride + 1
    OW = (W - KW) // stride + 1
    win = np.lib.stride_tricks.sliding_window_view(xd, (KH, KW), axis=(2, 3))
    win = win[:, :, ::stride, ::stride]  # (N, C, OH, OW, KH, KW)
    cols = win.transpose(0, 2, 3, 1, 4, 5)
    return np.ascontiguousarray(cols).reshape(N * OH * OW, C * KH * KW), OH, OW


def conv2d(x, w, b=None, stride=1, pad=0):
    """NCHW f32 convolution as im2col + one GEMM (borch/_ops.py:738-791, groups 1)."""
    x = np.asarray(x, np.float32)
    w = np.asarray(w, np.float32)
    if pad:
        x = np.pad(x, ((0, 0), (0, 0), (pad, pad), (pad, pad)))
    F, C, KH, KW = w.shape
    if x.shape[1] != C:
        raise RuntimeError(f"channels do not match: input {x.shape[1]}, filter {C}")
    cols, OH, OW = im2col(x, KH, KW, stride)
    out = (cols @ w.reshape(F, -1).T).reshape(x.shape[0], OH, OW, F).transpose(0, 3, 1, 2)
    return out if b is None else out + np.asarray(b, np.float32).reshape(1, -1, 1, 1)


def resnet18_forward(params, x):
    """The folded CIFAR ResNet-18 (configuration C3) in f32 through ``conv2d`` / ``linear``.
    ``params`` maps ``stem`` / ``body.i.c1|c2|down`` to ``(w [O,C,k,k], b, stride, pad)`` and
    ``fc`` to ``(w, b)``."""
    def conv(h, key):
        w, b, s, p = params[key]
        return conv2d(h, w, b, s, p)
    h = np.maximum(conv(np.asarray(x, np.float32), "stem"), 0)
    for i in range(8):
        out = np.maximum(conv(h, f"body.{i}.c1"), 0)
        side = conv(h, f"body.{i}.down") if f"body.{i}.down" in params else h
        h = np.maximum(conv(out, f"body.{i}.c2") + side, 0)
    w, b = params["fc"]
    return linear(h.mean(axis=(2, 3)), w, b)
