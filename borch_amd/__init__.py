"""borch_amd — borch's int8 (W8A8) inference path on AMD Instinct MI355X (gfx950).

``import borch_amd as torch``: ``torch.nn.Linear`` / ``torch.nn.Conv2d`` /
``torch.nn.functional.linear`` / ``conv2d`` keep the signatures of borch's numpy core
(borch/_nn.py:397-415, 1156-1190; borch/_ops.py:738-791) and, once quantized with
``torch.quantize_for_int8(model)`` (borch-ts/src/nn.ts:6770-6780), run hand-written HIP
int8 MFMA kernels through a ctypes C ABI (``include/bq.h``). Everything outside that path
(tensors, other layers, ``Sequential``, ...) is PyTorch-ROCm's own and is re-exported.
"""
from __future__ import annotations

import types as _types

import torch as _torch

from . import int8, nn, streaming  # noqa: F401
from .compiled import Compiled, compiled  # noqa: F401
from .nn import calibrate_int8, clear_int8, int8_report, quantize_for_int8  # noqa: F401
from .serialize import load_int8, save_int8  # noqa: F401
from .nn import intrinsic as _intrinsic

ao = _types.SimpleNamespace(nn=_types.SimpleNamespace(intrinsic=_intrinsic))

__version__ = "0.1.0"


def __getattr__(name):
    return getattr(_torch, name)
