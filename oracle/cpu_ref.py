"""ctypes wrapper of oracle/lib/libcpuref.so — the C restatement of borch_cpu's f32
kernels (oracle/cpu_ref.c). Test and measurement infrastructure only."""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

LIB = Path(__file__).resolve().parent / "lib" / "libcpuref.so"
_lib = None
_fp = ctypes.POINTER(ctypes.c_float)
_sz = ctypes.c_size_t


def lib():
    global _lib
    if _lib is None:
        if not LIB.exists():
            from . import build
            build.build()
        h = ctypes.CDLL(str(LIB))
        h.ref_gemm_threaded.argtypes = [ctypes.c_int, _sz, _sz, _sz, _fp, _fp, _fp, _fp, ctypes.c_uint]
        h.ref_gemm_bias_act.argtypes = [_sz, _sz, _sz, _fp, _fp, _fp, _fp, ctypes.c_uint]
        h.ref_im2col_rows.argtypes = [_sz] * 9 + [_fp, _fp]
        h.ref_dwconv_rows.argtypes = [_sz] * 9 + [_fp, _fp, _fp, _fp, ctypes.c_uint]
        h.ref_conv2d_threaded.argtypes = [ctypes.c_int] + [_sz] * 7 + [_fp, _fp, _sz, _fp, ctypes.c_uint, _fp, _fp, _sz]
        _lib = h
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(_fp)


def threads() -> int:
    return int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)


def gemm(a, b, bias=None, act=0, nthreads=None):
    """C = a[m,k] @ b[k,n] + bias, n % 16 == 0 (gemm_bias_act, lib.rs:508-584)."""
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    m, k = a.shape
    n = b.shape[1]
    assert n % 16 == 0
    c = np.empty((m, n), np.float32)
    bias = None if bias is None else np.ascontiguousarray(bias, np.float32)
    lib().ref_gemm_threaded(nthreads or threads(), m, n, k, _p(a), _p(b), _p(c), _p(bias), act)
    return c


def conv2d_nhwc(x, wcol, k, stride, pad, bias=None, act=0, nthreads=None, block=64):
    """NHWC f32 conv via im2col_rows + gemm_bias_act; ``wcol`` is [k*k*c, cout]."""
    x = np.ascontiguousarray(x, np.float32)
    n, h, w, c = x.shape
    cout = wcol.shape[1]
    ho = (h + 2 * pad - k) // stride + 1
    wo = (w + 2 * pad - k) // stride + 1
    out = np.empty((n, ho, wo, cout), np.float32)
    t = nthreads or threads()
    cols = np.empty(t * block * k * k * c, np.float32)
    bias = None if bias is None else np.ascontiguousarray(bias, np.float32)
    lib().ref_conv2d_threaded(t, n, h, w, c, k, stride, pad, _p(x), _p(np.ascontiguousarray(wcol, np.float32)),
                              cout, _p(bias), act, _p(out), _p(cols), block)
    return out


def im2col_rows(x_img, k, stride, pad, row0, rows):
    h, w, c = x_img.shape
    wo = (w + 2 * pad - k) // stride + 1
    out = np.empty((rows, k * k * c), np.float32)
    lib().ref_im2col_rows(h, w, c, k, stride, pad, wo, row0, rows, _p(np.ascontiguousarray(x_img, np.float32)),
                          _p(out))
    return out


def dwconv(x_img, wt, k, stride, pad, bias, act=0):
    """One image, NHWC, c % 16 == 0; ``wt`` is [k, k, c] (dwconv_rows, lib.rs:598-641)."""
    h, w, c = x_img.shape
    ho = (h + 2 * pad - k) // stride + 1
    wo = (w + 2 * pad - k) // stride + 1
    out = np.empty((ho, wo, c), np.float32)
    lib().ref_dwconv_rows(h, w, c, k, stride, pad, wo, 0, ho, _p(np.ascontiguousarray(x_img, np.float32)),
                          _p(np.ascontiguousarray(wt, np.float32)), _p(out),
                          _p(np.ascontiguousarray(bias, np.float32)), act)
    return out


def resnet18_forward(params, x_nchw, nthreads=None):
    """The folded CIFAR ResNet-18 in f32 through the C kernels (NHWC, channels padded to
    16 for the stem as the reference runner pads them, runner.ts). ``params`` maps
    ``stem``/``body.i.c1|c2|down`` to ``(w [O,C,k,k], b, stride, pad)`` and ``fc`` to ``(w, b)``."""
    def conv(h, key, act, res=None):
        w, b, s, p = params[key]
        O, C, k, _ = w.shape
        cpad = h.shape[-1]
        wt = np.zeros((k, k, cpad, O), np.float32)
        wt[:, :, :C, :] = w.transpose(2, 3, 1, 0)
        y = conv2d_nhwc(h, wt.reshape(k * k * cpad, O), k, s, p, b, 0 if res is not None else act, nthreads)
        if res is not None:
            y = y + res
            if act:
                y = np.maximum(y, 0)
        return y
    x = np.ascontiguousarray(np.asarray(x_nchw, np.float32).transpose(0, 2, 3, 1))
    xp = np.zeros(x.shape[:3] + (16,), np.float32)
    xp[..., :3] = x
    h = conv(xp, "stem", 1)
    for i in range(8):
        out = conv(h, f"body.{i}.c1", 1)
        side = conv(h, f"body.{i}.down", 0) if f"body.{i}.down" in params else h
        h = conv(out, f"body.{i}.c2", 1, side)
    feats = h.mean(axis=(1, 2))
    w, b = params["fc"]
    return feats @ w.T + b
