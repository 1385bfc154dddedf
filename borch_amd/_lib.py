"""ctypes binding of ``libbq.so`` (declared in ``include/bq.h``).

The library is loaded from ``borch_amd/lib/libbq.so`` (built in-tree by
``borch_amd.build``). torch is imported first so that the library's ``libamdhip64.so.7``
dependency binds to the HIP runtime torch already loaded: one runtime, one context, and
``Tensor.data_ptr()`` values are valid device pointers for the kernels.

There is no fallback: when the library is missing every int8 entry point raises.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch  # noqa: F401  (must precede the CDLL: shares torch's HIP runtime)

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libbq.so"

BQ_OK = 0
BQ_ERR_ARG = -1
BQ_ERR_DEVICE = -2
BQ_ERR_LAUNCH = -3
BQ_ERR_UNSUPPORTED = -4

ACT_NONE, ACT_RELU, ACT_SILU, ACT_GELU = 0, 1, 2, 3
SCALE_A_PER_TENSOR = 0x100  # OR-ed into bq_gemm_i8's act: one activation scale for the whole A
ROUND_EXACT, ROUND_REFERENCE, ROUND_REFERENCE_CONV = 0, 1, 2  # bq_quantize_weight_host's rules
CFG_GEMV, CFG_SKINNY = 32, 33  # the decode kernels' configuration ids in the plan API (M <= 8)
CFG_SMALLK = 18  # the small-K kernel's configuration id in the plan API (N <= 256, K <= 256)

_c_i64 = ctypes.c_int64
_c_p = ctypes.c_void_p
_c_int = ctypes.c_int
_c_size = ctypes.c_size_t



class ConvDesc(ctypes.Structure):
    """``bq_conv_desc`` (include/bq.h): one convolution of ``bq_conv2d_i8_nhwc_pair``."""
    _fields_ = [("w", _c_p), ("O", _c_i64), ("KH", _c_i64), ("KW", _c_i64), ("stride", _c_i64), ("pad", _c_i64),
                ("sW", _c_p), ("bias", _c_p), ("residual", _c_p), ("act", _c_int), ("out", _c_p),
                ("s_out", _c_p), ("q_out", _c_p), ("amax", _c_p)]


# name -> (restype, argtypes); mirrors include/bq.h one for one.
SIGNATURES = {
    "bq_version": (_c_int, []),
    "bq_last_error": (ctypes.c_char_p, []),
    "bq_device_ok": (_c_int, [_c_int]),
    "bq_quantize_rows": (_c_int, [_c_p, _c_i64, _c_i64, _c_p, _c_p, _c_p]),
    "bq_quantize_rows_act": (_c_int, [_c_p, _c_i64, _c_i64, _c_int, _c_p, _c_p, _c_p, _c_p]),
    "bq_layernorm_quantize_rows": (_c_int, [_c_p, _c_i64, _c_i64, _c_p, _c_p, ctypes.c_float, _c_p, _c_p, _c_p,
                                            _c_p]),
    "bq_quantize_weight_per_channel": (_c_int, [_c_p, _c_i64, _c_i64, _c_p, _c_p, _c_p]),
    "bq_quantize_weight_host": (_c_int, [_c_p, _c_i64, _c_i64, _c_i64, _c_int, _c_p, _c_p, _c_int]),
    "bq_quantize_tensor_ws_bytes": (_c_size, [_c_i64]),
    "bq_quantize_tensor": (_c_int, [_c_p, _c_i64, _c_p, _c_p, _c_p, _c_size, _c_p]),
    "bq_quantize_nhwc": (_c_int, [_c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_size, _c_p]),
    "bq_quantize_nhwc_scaled": (_c_int, [_c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p]),
    "bq_quantize_nchw": (_c_int, [_c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_size, _c_p]),
    "bq_quantize_nchw_scaled": (_c_int, [_c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p]),
    "bq_gemm_ws_bytes": (_c_size, []),
    "bq_gemm_i8": (_c_int, [_c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_p, _c_int, _c_p, _c_p, _c_p,
                            _c_size, _c_p]),
    "bq_linear_i8": (_c_int, [_c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_int, _c_p, _c_p, _c_p, _c_p,
                              _c_size, _c_p]),
    "bq_gemm_i8_phases": (_c_i64, [_c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_p]),
    "bq_gemm_i8_noalloc": (_c_int, [_c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_p, _c_int, _c_p, _c_p,
                                    _c_p]),
    "bq_conv2d_i8_nhwc_q": (_c_int, [_c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_i64, _c_i64, _c_i64,
                                     _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_p, _c_int, _c_p, _c_p, _c_p, _c_p,
                                     _c_p, _c_p, _c_size, _c_p]),
    "bq_conv2d_i8_nhwc_dq": (_c_int, [_c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_i64, _c_i64, _c_i64,
                                      _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_p, _c_int, _c_p, _c_p, _c_p, _c_i64,
                                      _c_p]),
    "bq_conv2d_i8_nchw_fq": (_c_int, [_c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_i64,
                                      _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_int, _c_p, _c_p, _c_p, _c_p, _c_p, _c_i64,
                                      _c_p, _c_p, _c_p, _c_size, _c_p]),
    "bq_conv2d_absmax_parts": (_c_i64, [_c_i64] * 9),
    "bq_conv2d_i8_nhwc_dq_ok": (_c_int, [_c_i64] * 9),
    "bq_plan_candidates": (_c_int, [_c_p, _c_int, _c_p, _c_p, _c_int]),
    "bq_plan_set": (_c_int, [_c_p, _c_int, ctypes.c_int32, ctypes.c_int32]),
    "bq_plan_clear": (_c_int, []),
    "bq_conv2d_i8_nhwc": (_c_int, [_c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_i64, _c_i64, _c_i64,
                                   _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_p, _c_int, _c_p, _c_p, _c_p, _c_p,
                                   _c_size, _c_p]),
    "bq_conv2d_i8_nhwc_pair": (_c_int, [_c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, ctypes.POINTER(ConvDesc),
                                        ctypes.POINTER(ConvDesc), _c_p, _c_size, _c_p]),
    "bq_quantize_nhwc_parts": (_c_int, [_c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_i64, _c_p, _c_p, _c_p]),
    "bq_quantize_nhwc_chscale": (_c_int, [_c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_p, _c_p,
                                          _c_i64, _c_p, _c_size, _c_p]),
    "bq_dwconv_i8_nhwc": (_c_int, [_c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_i64, _c_i64, _c_i64,
                                   _c_i64, _c_p, _c_p, _c_p, _c_int, _c_p, _c_p, _c_p]),
    "bq_gemv_w8a32": (_c_int, [_c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_int, _c_p, _c_p]),
    "bq_linear_w8a32": (_c_int, [_c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_int, _c_p, _c_p]),
    "bq_dequant_i8": (_c_int, [_c_p, _c_i64, _c_i64, _c_p, _c_p, _c_p]),
    "bq_attention_f32": (_c_int, [_c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_p]),
    "bq_avgpool_linear_f32": (_c_int, [_c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_i64, _c_p, _c_p]),
    "bq_se_gate_ws_bytes": (_c_size, [_c_i64, _c_i64, _c_i64]),
    "bq_se_gate_absmax_parts": (_c_i64, [_c_i64, _c_i64]),
    "bq_se_gate_nhwc": (_c_int, [_c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_i64, _c_p, _c_p, _c_p, _c_p, _c_p,
                                 _c_size, _c_p]),
}

_lock = threading.Lock()
_lib = None


class Int8Unavailable(RuntimeError):
    """The int8 path cannot run here (library missing, no gfx950 device)."""


def lib():
    """The loaded library (loaded once); raises ``Int8Unavailable`` if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise Int8Unavailable(
                    f"int8: {LIB_PATH} is not built — run `python -m borch_amd.build` "
                    "(the int8 path has no CPU fallback)")
            h = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(h, name)
                fn.restype = res
                fn.argtypes = args
            _lib = h
    return _lib


def last_error() -> str:
    return (lib().bq_last_error() or b"").decode(errors="replace")


def check(rc: int) -> None:
    """Raises on a non-zero return code, with the library's message."""
    if rc == BQ_OK:
        return
    msg = last_error()
    if rc == BQ_ERR_DEVICE:
        raise Int8Unavailable(msg)
    if rc == BQ_ERR_UNSUPPORTED:
        raise NotImplementedError(msg)
    if rc == BQ_ERR_ARG:
        raise ValueError(msg)
    raise RuntimeError(msg)


_device_ok: dict[int, bool] = {}


def require_device(device: torch.device) -> None:
    """Refuses by name anything but a gfx950 CUDA(HIP) device (nn.ts:6771-6773's rule)."""
    if device.type != "cuda":
        raise Int8Unavailable(
            f"int8: tensors on {device} — the int8 path runs on a gfx950 GPU only (no CPU fallback)")
    idx = device.index if device.index is not None else torch.cuda.current_device()
    ok = _device_ok.get(idx)
    if ok is None:
        ok = bool(lib().bq_device_ok(idx))
        _device_ok[idx] = ok
    if not ok:
        raise Int8Unavailable(last_error())
