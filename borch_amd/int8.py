"""Tensor-level int8 operations over the HIP library (``include/bq.h``).

Everything here takes and returns PyTorch-ROCm device tensors and enqueues on torch's
current stream. Weights are packed once (``pack_*``, the prepare step of
borch-ts/src/nn.ts:967-980 and quant.ts:23-103); activations are quantized per call
(per row for Linear, per tensor for conv, as borch-ts/src/tensor.ts:11909-11921 does for
its conv input). There is no CPU path: a tensor that is not on a gfx950 device raises.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _lib
from ._lib import ACT_GELU, ACT_NONE, ACT_RELU, ACT_SILU, CFG_GEMV, CFG_SKINNY, SCALE_A_PER_TENSOR, check, lib, \
    require_device

__all__ = [
    "ACT_NONE", "ACT_RELU", "ACT_SILU", "ACT_GELU", "Int8Weight", "Int8ConvWeight", "Int8DwWeight",
    "quantize_rows", "quantize_weight_per_channel", "quantize_tensor", "quantize_nhwc",
    "gemm_i8", "conv2d_i8_nhwc", "conv2d_i8_nhwc_q", "conv2d_pair_i8_nhwc", "PairConv", "dwconv_i8_nhwc",
    "pack_linear_weight", "pack_conv_weight", "attention_f32", "avgpool_linear",
    "quantize_nhwc_scaled", "quantize_nhwc_chscale", "se_gate_nhwc", "linear_w8a32", "dequant_weight",
    "pack_dw_weight", "linear", "linear_rows", "conv2d", "depthwise_conv2d", "round_up", "split_workspace",
]


def round_up(v: int, m: int) -> int:
    return (v + m - 1) // m * m


def _ptr(t):
    return None if t is None else t.data_ptr()


def _stream(t: torch.Tensor):
    return torch.cuda.current_stream(t.device).cuda_stream


# The split-K workspaces of bq_gemm_i8 / bq_conv2d_i8_nhwc(_q) (bq_gemm_ws_bytes): one
# zero-filled buffer per (device, stream), made outside any graph capture (on the stream
# it serves) and kept for the life of the process, since a captured HIP graph keeps using
# the pointer it recorded. The kernels leave its counters zero after every call; calls on
# one stream run in order, so they may share it, while launches on two streams at once
# each have their own tile counters and partials. (torch hands out streams from a fixed
# pool per device, so the table stays small.)
_SPLIT_WS: dict = {}


def split_workspace(device: torch.device, stream=None):
    """The split-K workspace of ``stream`` (default: the current stream) on ``device``, or
    None while a graph is being captured on a stream that has none yet (those calls then
    run unsplit: the same results). Capture on the stream the warm-up ran on to keep it."""
    idx = torch.device(device).index
    idx = torch.cuda.current_device() if idx is None else idx
    st = torch.cuda.current_stream(idx) if stream is None else stream
    key = (idx, st.cuda_stream)
    ws = _SPLIT_WS.get(key)
    if ws is None:
        if torch.cuda.is_current_stream_capturing():
            return None
        with torch.cuda.stream(st):
            ws = torch.zeros(int(lib().bq_gemm_ws_bytes()), dtype=torch.uint8, device=torch.device("cuda", idx))
        _SPLIT_WS[key] = ws
    return ws


def _ws_args(device):
    """(pointer, bytes) of the current stream's split-K workspace, or (None, 0) (unsplit)."""
    ws = split_workspace(device)
    return (None, 0) if ws is None else (ws.data_ptr(), ws.numel())


def _need(t: torch.Tensor, name: str, dtype: torch.dtype) -> None:
    if t.dtype != dtype:
        raise TypeError(f"{name}: expected {dtype}, got {t.dtype}")
    require_device(t.device)


def _vec(t, n: int, name: str):
    """``t`` as a contiguous float32 vector of exactly ``n`` values (None stays None): the
    kernels read n values from the pointer, so a shorter vector must never reach them."""
    if t is None:
        return None
    if t.numel() != n:
        raise ValueError(f"{name}: expected {n} values, got {t.numel()}")
    return t.detach().reshape(-1).float().contiguous()


def _f32c(x: torch.Tensor) -> torch.Tensor:
    if x.dtype != torch.float32:
        raise TypeError(f"int8 path takes float32 activations, got {x.dtype}")
    return x.contiguous()


# --------------------------------------------------------------------------- quantizers

def quantize_rows(x: torch.Tensor, act: int = ACT_NONE, want_y: bool = False):
    """Per-row int8 of f32 ``[M, K]`` → ``(q int8 [M, K], s f32 [M])`` (bq_quantize_rows); of
    ``act(x)`` without storing it when ``act`` is given (bq_quantize_rows_act), and with
    ``want_y`` also the f32 ``act(x)`` the kernel quantized: ``(q, s, y)``."""
    x = _f32c(x)
    require_device(x.device)
    if x.dim() != 2:
        raise ValueError("quantize_rows wants a 2-D tensor")
    M, K = x.shape
    q = torch.empty((M, K), dtype=torch.int8, device=x.device)
    s = torch.empty((M,), dtype=torch.float32, device=x.device)
    if act == ACT_NONE and not want_y:
        check(lib().bq_quantize_rows(x.data_ptr(), M, K, q.data_ptr(), s.data_ptr(), _stream(x)))
        return q, s
    y = torch.empty((M, K), dtype=torch.float32, device=x.device) if want_y else None
    check(lib().bq_quantize_rows_act(x.data_ptr(), M, K, int(act), q.data_ptr(), s.data_ptr(), _ptr(y), _stream(x)))
    if want_y:
        return q, s, (x if act == ACT_NONE else y)
    return q, s


def quantize_weight_per_channel(w: torch.Tensor):
    """Per-output-channel int8 of a Linear weight ``[N, K]`` (quant.ts:23-53)."""
    w = _f32c(w)
    require_device(w.device)
    N, K = w.shape
    q = torch.empty((N, K), dtype=torch.int8, device=w.device)
    s = torch.empty((N,), dtype=torch.float32, device=w.device)
    check(lib().bq_quantize_weight_per_channel(w.data_ptr(), N, K, q.data_ptr(), s.data_ptr(), _stream(w)))
    return q, s


def _ws(n: int, device) -> torch.Tensor:
    return torch.empty((max(int(lib().bq_quantize_tensor_ws_bytes(n)), 4),), dtype=torch.uint8, device=device)


def quantize_tensor(x: torch.Tensor):
    """Per-tensor int8 of any f32 tensor → ``(q int8 same shape, s f32 [1])``."""
    x = _f32c(x)
    require_device(x.device)
    q = torch.empty(x.shape, dtype=torch.int8, device=x.device)
    s = torch.empty((1,), dtype=torch.float32, device=x.device)
    ws = _ws(x.numel(), x.device)
    check(lib().bq_quantize_tensor(x.data_ptr(), x.numel(), q.data_ptr(), s.data_ptr(), ws.data_ptr(),
                                   ws.numel(), _stream(x)))
    return q, s


def quantize_nhwc(x: torch.Tensor, cpad: int | None = None):
    """Per-tensor int8 of an NCHW f32 activation into NHWC int8 with channels padded to
    ``cpad`` (zeros) → ``(q int8 [N, H, W, cpad], s f32 [1])``. A channels-last input is
    read in place, and so is a contiguous NCHW input quantized into padded channels (a
    network's input image: bq_quantize_nchw); other NCHW inputs are converted first. An unmodified output of
    ``conv2d_i8_nhwc`` carries its per-tile maxima, and then one pass suffices
    (bq_quantize_nhwc_parts); otherwise partial maxima are computed first (bq_quantize_nhwc)."""
    if x.dtype != torch.float32:
        raise TypeError(f"int8 path takes float32 activations, got {x.dtype}")
    require_device(x.device)
    N, C, H, W = x.shape
    cpad = C if cpad is None else int(cpad)
    q = torch.empty((N, H, W, cpad), dtype=torch.int8, device=x.device)
    s = torch.empty((1,), dtype=torch.float32, device=x.device)
    P = N * H * W
    if getattr(x, "_bq_absmax", None) is None and _nchw_padded(x, cpad):
        ws = _ws(P * C, x.device)
        check(lib().bq_quantize_nchw(x.data_ptr(), N, C, H * W, cpad, q.data_ptr(), s.data_ptr(), ws.data_ptr(),
                                     ws.numel(), _stream(x)))
        return q, s
    xl = x.contiguous(memory_format=torch.channels_last)
    parts = getattr(xl, "_bq_absmax", None)
    if parts is not None and parts[2] == xl._version:
        # A conv output read by two int8 convs (a residual block's first conv and its
        # downsampling shortcut) is quantized once. Only such outputs are cached: they are
        # new tensors in every forward, so a graph capture never finds a warm-up's bytes.
        done = getattr(xl, "_bq_q8", None)
        if done is not None and done[2] == xl._version and done[3] == cpad:
            return done[0], done[1]
        # the producing conv's per-tile max |y| (bq_conv2d_i8_nhwc): no max pass over x
        check(lib().bq_quantize_nhwc_parts(xl.data_ptr(), P, C, cpad, parts[0].data_ptr(), parts[1], q.data_ptr(),
                                           s.data_ptr(), _stream(x)))
        xl._bq_q8 = (q, s, xl._version, cpad)
        return q, s
    ws = _ws(P * C, x.device)
    check(lib().bq_quantize_nhwc(xl.data_ptr(), P, C, cpad, q.data_ptr(), s.data_ptr(), ws.data_ptr(),
                                 ws.numel(), _stream(x)))
    return q, s


def _nchw_padded(x: torch.Tensor, cpad: int) -> bool:
    """An NCHW-contiguous activation quantized into padded channels (the stem's input): the
    NCHW entry points read it as it is."""
    C = x.shape[1]
    return (cpad > C and cpad % 16 == 0 and x.is_contiguous()
            and not x.is_contiguous(memory_format=torch.channels_last))


def quantize_nhwc_chscale(x: torch.Tensor, cs: torch.Tensor, cpad: int | None = None, scale=None):
    """Per-tensor int8 of ``x * cs[:, :, None, None]`` (x NCHW f32, cs [N, C] f32: a
    squeeze-excite gate) into NHWC int8 ``[N, H, W, cpad]`` without storing the product
    (bq_quantize_nhwc_chscale): ``(q, s [1])``, the same bytes as quantizing the product.
    With ``scale`` (a calibrated [1] tensor) one pass and that scale; else, when ``cs`` is
    the gate ``se_gate_nhwc`` made from this same, unchanged ``x``, one pass with the maxima
    it wrote; else two passes."""
    if x.dtype != torch.float32 or cs.dtype != torch.float32:
        raise TypeError("int8 path takes float32 activations and gates")
    require_device(x.device)
    N, C, H, W = x.shape
    if tuple(cs.shape) != (N, C):
        raise RuntimeError(f"channel scale shape {tuple(cs.shape)} != {(N, C)}")
    cpad = C if cpad is None else int(cpad)
    xl = x.contiguous(memory_format=torch.channels_last)
    csc = cs.contiguous()
    q = torch.empty((N, H, W, cpad), dtype=torch.int8, device=x.device)
    if scale is not None:
        check(lib().bq_quantize_nhwc_chscale(xl.data_ptr(), N, H * W, C, cpad, csc.data_ptr(), q.data_ptr(), None,
                                             scale.data_ptr(), None, 0, None, 0, _stream(x)))
        return q, scale
    s = torch.empty((1,), dtype=torch.float32, device=x.device)
    made = getattr(cs, "_bq_product_absmax", None)
    if made is not None and made[2] is x and made[3] == x._version and made[4] == cs._version and csc is cs:
        check(lib().bq_quantize_nhwc_chscale(xl.data_ptr(), N, H * W, C, cpad, csc.data_ptr(), q.data_ptr(),
                                             s.data_ptr(), None, made[0].data_ptr(), made[1], None, 0, _stream(x)))
        return q, s
    ws = _ws(N * H * W * C, x.device)
    check(lib().bq_quantize_nhwc_chscale(xl.data_ptr(), N, H * W, C, cpad, csc.data_ptr(), q.data_ptr(),
                                         s.data_ptr(), None, None, 0, ws.data_ptr(), ws.numel(), _stream(x)))
    return q, s


def se_gate_nhwc(x: torch.Tensor, w1: torch.Tensor, b1, w2: torch.Tensor, b2, w2t: torch.Tensor | None = None):
    """Squeeze-excite gates ``sigmoid(w2 · silu(w1 · mean_hw(x) + b1) + b2)`` in f32 for an
    NCHW activation (channels-last memory is read in place): ``[N, C]`` (bq_se_gate_nhwc;
    borch's CPU runner "se" node, runner.ts:256-268). ``w1 [S, C]``, ``w2 [C, S]``; ``w2t``
    (optional) is ``w2`` already transposed to ``[S, C]`` contiguous, as the kernel reads it.
    The gate carries the partial maxima of ``|x * gate|`` the kernel also writes, for
    ``quantize_nhwc_chscale`` of the same ``x`` (its dynamic scale without a max pass)."""
    if x.dtype != torch.float32:
        raise TypeError(f"squeeze-excite takes float32 activations, got {x.dtype}")
    require_device(x.device)
    N, C, H, W = x.shape
    S = w1.shape[0]
    if tuple(w1.shape) != (S, C) or tuple(w2.shape) != (C, S):
        raise RuntimeError(f"squeeze-excite weights {tuple(w1.shape)} / {tuple(w2.shape)} do not fit C={C}")
    xl = x.contiguous(memory_format=torch.channels_last)
    w1c = w1.float().contiguous()
    w2c = w2.float().t().contiguous() if w2t is None else w2t
    b1c = None if b1 is None else b1.float().contiguous()
    b2c = None if b2 is None else b2.float().contiguous()
    gate = torch.empty((N, C), dtype=torch.float32, device=x.device)
    nb = int(lib().bq_se_gate_ws_bytes(N, H * W, C))
    ws = torch.empty((max(nb // 4, 4),), dtype=torch.float32, device=x.device)
    nparts = int(lib().bq_se_gate_absmax_parts(N, C))
    if nparts < 0:
        check(nparts)
    parts = torch.empty((max(nparts, 1),), dtype=torch.float32, device=x.device)
    check(lib().bq_se_gate_nhwc(xl.data_ptr(), N, H * W, C, w1c.data_ptr(), _ptr(b1c), S, w2c.data_ptr(), _ptr(b2c),
                                gate.data_ptr(), parts.data_ptr(), ws.data_ptr(), ws.numel() * 4, _stream(x)))
    if xl is x:  # the maxima describe x itself (a channels-last x is read in place)
        gate._bq_product_absmax = (parts, nparts, x, x._version, gate._version)
    return gate


def quantize_nhwc_scaled(x: torch.Tensor, scale: torch.Tensor, cpad: int | None = None):
    """Per-tensor int8 of an NCHW f32 activation with a given (calibrated) scale ``[1]``
    into NHWC int8 ``[N, H, W, cpad]``: one pass (bq_quantize_nhwc_scaled)."""
    if x.dtype != torch.float32:
        raise TypeError(f"int8 path takes float32 activations, got {x.dtype}")
    require_device(x.device)
    N, C, H, W = x.shape
    cpad = C if cpad is None else int(cpad)
    q = torch.empty((N, H, W, cpad), dtype=torch.int8, device=x.device)
    if _nchw_padded(x, cpad):  # a network's NCHW input: read in place, no permute
        check(lib().bq_quantize_nchw_scaled(x.data_ptr(), N, C, H * W, cpad, scale.data_ptr(), q.data_ptr(),
                                            _stream(x)))
        return q
    xl = x.contiguous(memory_format=torch.channels_last)
    check(lib().bq_quantize_nhwc_scaled(xl.data_ptr(), N * H * W, C, cpad, scale.data_ptr(), q.data_ptr(),
                                        _stream(x)))
    return q


# ------------------------------------------------------------------------ packed weights

@dataclass
class Int8Weight:
    """A Linear weight packed for ``bq_gemm_i8``: ``q int8 [N, Kpad]``, ``s f32 [N]``.
    ``weight_only`` selects W8A32 (f32 activations, ``bq_linear_w8a32``) instead of W8A8;
    ``per_tensor`` quantizes the W8A8 activations with one scale for the whole input (the
    reference's ``matmulInt8(scaled)``, kernels.ts:1818-1827) instead of one per row."""
    q: torch.Tensor
    s: torch.Tensor
    in_features: int
    out_features: int
    weight_only: bool = False
    per_tensor: bool = False  # W8A8 with one activation scale per call (the reference's matmulInt8)

    @property
    def kpad(self) -> int:
        return self.q.shape[1]


@dataclass
class Int8ConvWeight:
    """A conv weight packed for ``bq_conv2d_i8_nhwc``: ``q int8 [O, KH*KW*Cpad]``
    (tap-major then channel), ``s f32 [O]``."""
    q: torch.Tensor
    s: torch.Tensor
    O: int
    C: int
    cpad: int
    KH: int
    KW: int


@dataclass
class Int8DwWeight:
    """A depthwise weight packed for ``bq_dwconv_i8_nhwc``: ``q int8 [KH*KW, Cpad]``,
    ``s f32 [Cpad]``."""
    q: torch.Tensor
    s: torch.Tensor
    C: int
    cpad: int
    KH: int
    KW: int


def pack_linear_weight(w: torch.Tensor, weight_only: bool = False, per_tensor: bool = False) -> Int8Weight:
    """Quantize once (quant.ts:23-53); K padded to a multiple of 16 with zeros (exact)."""
    if weight_only and per_tensor:
        raise ValueError("per_tensor is an activation quantization: a weight-only Linear has none")
    N, K = w.shape
    kp = round_up(max(K, 16), 16)
    wp = w if kp == K else torch.nn.functional.pad(w, (0, kp - K))
    q, s = quantize_weight_per_channel(wp.float())
    return Int8Weight(q, s, K, N, weight_only, per_tensor)


def dequant_weight(w8: Int8Weight) -> torch.Tensor:
    """f32 ``[N, Kpad]`` = f32(q) * s[n] (bq_dequant_i8; dequantInt8, kernels.ts:1264-1274)."""
    require_device(w8.q.device)
    N, K = w8.q.shape
    out = torch.empty((N, K), dtype=torch.float32, device=w8.q.device)
    check(lib().bq_dequant_i8(w8.q.data_ptr(), N, K, w8.s.data_ptr(), out.data_ptr(), _stream(w8.q)))
    return out


def linear_w8a32(x: torch.Tensor, w8: Int8Weight, bias=None, act=ACT_NONE, residual=None) -> torch.Tensor:
    """Weight-only int8 Linear (W8A32, matmul(..., weightInt8), kernels.ts:2661-2753): f32
    activations against the int8 weight read inside the kernel (bq_linear_w8a32; no f32 copy
    of the weight is made), effective weight f32(q)·s, f32 accumulation; ``residual [..., N]``
    is added after the bias and before ``act``."""
    if x.shape[-1] != w8.in_features:
        raise RuntimeError(f"mat1 and mat2 shapes cannot be multiplied "
                           f"({'x'.join(str(n) for n in x.reshape(-1, x.shape[-1]).shape)} and "
                           f"{w8.in_features}x{w8.out_features})")
    require_device(x.device)
    lead = x.shape[:-1]
    x2 = _f32c(x.reshape(-1, x.shape[-1]))
    if w8.kpad != w8.in_features:
        x2 = torch.nn.functional.pad(x2, (0, w8.kpad - w8.in_features))
    M, K = x2.shape
    N = w8.out_features
    out = torch.empty((M, N), dtype=torch.float32, device=x.device)
    b = _vec(bias, N, "bias")
    r = None
    if residual is not None:
        if tuple(residual.shape[:-1]) != tuple(lead) or residual.shape[-1] != N:
            raise RuntimeError(f"residual shape {tuple(residual.shape)} != output {(*lead, N)}")
        r = residual.reshape(M, N).float().contiguous()
    check(lib().bq_linear_w8a32(x2.data_ptr(), w8.q.data_ptr(), M, N, K, w8.s.data_ptr(), _ptr(b), _ptr(r), act,
                                out.data_ptr(), _stream(x2)))
    return out.reshape(*lead, N)


def pack_conv_weight(w: torch.Tensor) -> Int8ConvWeight:
    """Quantize a conv weight ``[O, C, KH, KW]`` once (quant.ts:80-103's scale rule) into
    ``[O, KH, KW, Cpad]`` with Cpad a multiple of 16 (zero channels: exact)."""
    O, C, KH, KW = w.shape
    cpad = round_up(C, 16)
    t = w.float().permute(0, 2, 3, 1)
    if cpad != C:
        t = torch.nn.functional.pad(t, (0, cpad - C))
    q, s = quantize_weight_per_channel(t.reshape(O, KH * KW * cpad))
    return Int8ConvWeight(q, s, O, C, cpad, KH, KW)


def pack_dw_weight(w: torch.Tensor) -> Int8DwWeight:
    """Quantize a depthwise weight ``[C, 1, KH, KW]`` once, one scale per channel over its
    taps, into tap-major ``[KH*KW, Cpad]`` (Cpad a multiple of 4)."""
    C, one, KH, KW = w.shape
    if one != 1:
        raise ValueError("depthwise weight must be [C, 1, KH, KW]")
    cpad = round_up(C, 4)
    t = w.float().reshape(C, KH * KW)
    if cpad != C:
        t = torch.nn.functional.pad(t, (0, 0, 0, cpad - C))
    q, s = quantize_weight_per_channel(t)
    return Int8DwWeight(q.t().contiguous(), s, C, cpad, KH, KW)


# --------------------------------------------------------------------------- int8 ops

def gemm_i8(qa, qw, sa, sw, bias=None, act=ACT_NONE, want_acc=False, residual=None):
    """``out = ((f32(qa @ qw.T) * sa[m]) * sw[n]) + bias[n]`` (+ ``residual [M, N]``) then
    act (bq_gemm_i8). ``sa`` holds one scale per row of ``qa``, or one for the whole of it
    (a per-tensor quantization: ``sa.numel() == 1``). Returns ``out`` or ``(out, acc int32)``."""
    _need(qa, "A", torch.int8)
    _need(qw, "W", torch.int8)
    M, K = qa.shape
    N, K2 = qw.shape
    if K != K2:
        raise RuntimeError(f"mat1 and mat2 shapes cannot be multiplied ({M}x{K} and {K2}x{N})")
    qa, qw = qa.contiguous(), qw.contiguous()
    sa, sw = sa.contiguous().float(), sw.contiguous().float()
    if sa.numel() not in (M, 1) or sw.numel() != N:
        raise ValueError("scale sizes do not match the operands")
    if sa.numel() == 1:  # one activation scale (for M == 1 both readings are the same)
        act = act | SCALE_A_PER_TENSOR
    b = _vec(bias, N, "bias")
    r = None
    if residual is not None:
        if tuple(residual.shape) != (M, N):
            raise RuntimeError(f"residual shape {tuple(residual.shape)} != output {(M, N)}")
        r = residual.float().contiguous()
    out = torch.empty((M, N), dtype=torch.float32, device=qa.device)
    acc = torch.empty((M, N), dtype=torch.int32, device=qa.device) if want_acc else None
    check(lib().bq_gemm_i8(qa.data_ptr(), qw.data_ptr(), M, N, K, sa.data_ptr(), sw.data_ptr(), _ptr(b), _ptr(r),
                           act, out.data_ptr(), _ptr(acc), *_ws_args(qa.device), _stream(qa)))
    return (out, acc) if want_acc else out


def conv2d_i8_nhwc(qx, sa, wq: Int8ConvWeight, stride=1, pad=0, bias=None, residual=None, act=ACT_NONE,
                   want_acc=False):
    """Implicit-GEMM int8 conv on NHWC int8 ``qx [N, H, W, Cpad]`` (bq_conv2d_i8_nhwc).
    Returns f32 NCHW-shaped output in channels-last memory (NHWC bytes), optionally with
    the int32 accumulators ``[N*OH*OW, O]``. ``residual`` is NCHW-shaped (any layout)."""
    _need(qx, "x", torch.int8)
    N, H, W, C = qx.shape
    if C != wq.cpad:
        raise RuntimeError(f"channels do not match: input {C}, filter {wq.cpad}")
    OH = (H + 2 * pad - wq.KH) // stride + 1
    OW = (W + 2 * pad - wq.KW) // stride + 1
    if OH < 1 or OW < 1:
        raise RuntimeError("the filter is larger than the input.")
    out = torch.empty((N, wq.O, OH, OW), dtype=torch.float32, device=qx.device, memory_format=torch.channels_last)
    res = None
    if residual is not None:
        if tuple(residual.shape) != (N, wq.O, OH, OW):
            raise RuntimeError(f"residual shape {tuple(residual.shape)} != output {(N, wq.O, OH, OW)}")
        res = residual.float().contiguous(memory_format=torch.channels_last)
    acc = torch.empty((N * OH * OW, wq.O), dtype=torch.int32, device=qx.device) if want_acc else None
    b = _vec(bias, wq.O, "bias")
    parts, nparts = _absmax_parts(N, H, W, C, wq, stride, pad, qx.device)
    check(lib().bq_conv2d_i8_nhwc(qx.contiguous().data_ptr(), N, H, W, C, wq.q.data_ptr(), wq.O, wq.KH, wq.KW,
                                  stride, pad, sa.data_ptr(), wq.s.data_ptr(), _ptr(b), _ptr(res), act,
                                  out.data_ptr(), _ptr(acc), parts.data_ptr(), *_ws_args(qx.device), _stream(qx)))
    out._bq_absmax = (parts, nparts, out._version)
    return (out, acc) if want_acc else out


def conv2d_nchw_fq(x, wq: Int8ConvWeight, stride=1, pad=0, bias=None, residual=None, act=ACT_NONE, s_x=None,
                   s_out=None, f32_out=True, want_acc=False, want_scale=False):
    """``conv2d_i8_nhwc(*quantize_nhwc(x, 16))`` (with ``s_out``: ``conv2d_i8_nhwc_q``) of an
    NCHW-contiguous f32 input of at most 8 channels (a network's image), the quantization
    fused into the conv (bq_conv2d_i8_nchw_fq): one launch with a calibrated scale ``s_x``
    [1], two without (partial maxima first). The same bytes as the two-pass form. Returns
    ``out`` (NCHW-shaped channels-last, carrying its per-workgroup maxima; None with
    ``f32_out=False``), then the int8 twin with ``s_out``, the accumulators with
    ``want_acc``, the input's scale with ``want_scale``. Raises NotImplementedError (nothing
    launched) where the small-K kernel does not take the layer."""
    if x.dtype != torch.float32:
        raise TypeError(f"int8 path takes float32 activations, got {x.dtype}")
    require_device(x.device)
    if x.dim() != 4 or not x.is_contiguous():
        raise ValueError("conv2d_nchw_fq takes an NCHW-contiguous 4-D input")
    N, C, H, W = x.shape
    if wq.cpad != 16 or C != wq.C or C > 8:
        raise NotImplementedError(f"conv2d_nchw_fq: {C} input channels packed over {wq.cpad} (16 padded channels)")
    if x.data_ptr() % 16:  # a view into a larger image batch: the two-pass form takes it
        raise NotImplementedError("conv2d_nchw_fq: the image is not 16-byte aligned")
    if wq.KH * wq.KW * 16 > 256 or wq.O > 64 or wq.O % 4:  # the library's own limits, checked before allocating
        raise NotImplementedError(f"conv2d_nchw_fq: O={wq.O}, {wq.KH}x{wq.KW} filter (O <= 64, O % 4 == 0, "
                                  "KH*KW <= 16)")
    OH = (H + 2 * pad - wq.KH) // stride + 1
    OW = (W + 2 * pad - wq.KW) // stride + 1
    if OH < 1 or OW < 1:
        raise RuntimeError("the filter is larger than the input.")
    dev = x.device
    out = (torch.empty((N, wq.O, OH, OW), dtype=torch.float32, device=dev, memory_format=torch.channels_last)
           if f32_out else None)
    q = torch.empty((N, OH, OW, wq.O), dtype=torch.int8, device=dev) if s_out is not None else None
    res = None
    if residual is not None:
        if tuple(residual.shape) != (N, wq.O, OH, OW):
            raise RuntimeError(f"residual shape {tuple(residual.shape)} != output {(N, wq.O, OH, OW)}")
        res = residual.float().contiguous(memory_format=torch.channels_last)
    acc = torch.empty((N * OH * OW, wq.O), dtype=torch.int32, device=dev) if want_acc else None
    sx = torch.empty((1,), dtype=torch.float32, device=dev) if want_scale else None
    parts = torch.empty((4096,), dtype=torch.float32, device=dev) if f32_out else None
    nparts = ctypes.c_int64(0)
    ws = _ws(x.numel(), dev) if s_x is None else None
    b = _vec(bias, wq.O, "bias")
    check(lib().bq_conv2d_i8_nchw_fq(x.data_ptr(), N, C, H, W, _ptr(s_x), wq.q.data_ptr(), wq.O, wq.KH, wq.KW,
                                     stride, pad, wq.s.data_ptr(), _ptr(b), _ptr(res), act, _ptr(out), _ptr(acc),
                                     _ptr(s_out), _ptr(q), _ptr(parts), 4096, ctypes.byref(nparts), _ptr(sx),
                                     _ptr(ws), 0 if ws is None else ws.numel(), _stream(x)))
    if out is not None:
        out._bq_absmax = (parts, int(nparts.value), out._version)
    ret = (out,) + ((q,) if s_out is not None else ()) + ((acc,) if want_acc else ()) + ((sx,) if want_scale else ())
    return ret if len(ret) > 1 else out


def _absmax_parts(N, H, W, C, wq, stride, pad, device):
    """The buffer a conv's epilogue fills with its per-tile max |y| (bq_conv2d_absmax_parts)."""
    n = int(lib().bq_conv2d_absmax_parts(N, H, W, C, wq.O, wq.KH, wq.KW, stride, pad))
    if n < 0:
        check(n)
    return torch.empty((max(n, 1),), dtype=torch.float32, device=device), max(n, 1)


def conv2d_i8_nhwc_q(qx, sa, wq: Int8ConvWeight, s_out, stride=1, pad=0, bias=None, residual=None, act=ACT_NONE,
                     f32_out=True):
    """``conv2d_i8_nhwc`` that also returns the output's int8 twin ``[N, OH, OW, O]``
    quantized with the calibrated scale ``s_out [1]`` (bq_conv2d_i8_nhwc_q; O % 16 == 0).
    ``f32_out=False``: the twin alone is written and returned as ``(None, q)``."""
    _need(qx, "x", torch.int8)
    N, H, W, C = qx.shape
    if C != wq.cpad:
        raise RuntimeError(f"channels do not match: input {C}, filter {wq.cpad}")
    OH = (H + 2 * pad - wq.KH) // stride + 1
    OW = (W + 2 * pad - wq.KW) // stride + 1
    if OH < 1 or OW < 1:
        raise RuntimeError("the filter is larger than the input.")
    out = (torch.empty((N, wq.O, OH, OW), dtype=torch.float32, device=qx.device, memory_format=torch.channels_last)
           if f32_out else None)
    q = torch.empty((N, OH, OW, wq.O), dtype=torch.int8, device=qx.device)
    res = None
    if residual is not None:
        if tuple(residual.shape) != (N, wq.O, OH, OW):
            raise RuntimeError(f"residual shape {tuple(residual.shape)} != output {(N, wq.O, OH, OW)}")
        res = residual.float().contiguous(memory_format=torch.channels_last)
    b = _vec(bias, wq.O, "bias")
    # no per-tile maxima: a calibrated layer's consumer takes the twin or its own static scale
    check(lib().bq_conv2d_i8_nhwc_q(qx.contiguous().data_ptr(), N, H, W, C, wq.q.data_ptr(), wq.O, wq.KH, wq.KW,
                                    stride, pad, sa.data_ptr(), wq.s.data_ptr(), _ptr(b), _ptr(res), act,
                                    _ptr(out), None, s_out.data_ptr(), q.data_ptr(), None,
                                    *_ws_args(qx.device), _stream(qx)))
    return out, q


def conv2d_i8_nhwc_dq_ok(N: int, H: int, W: int, wq: Int8ConvWeight, stride=1, pad=0) -> bool:
    """Whether ``conv2d_i8_nhwc_dq`` takes this conv of an [N, H, W, wq.cpad] input under the
    plans in force (bq_conv2d_i8_nhwc_dq_ok; host only)."""
    if N < 1:
        return False
    r = int(lib().bq_conv2d_i8_nhwc_dq_ok(N, H, W, wq.cpad, wq.O, wq.KH, wq.KW, stride, pad))
    if r < 0:
        check(r)
    return r == 1


def conv2d_i8_nhwc_dq(qx, sa, wq: Int8ConvWeight, stride=1, pad=0, bias=None, residual=None, act=ACT_NONE):
    """``quantize_nhwc(conv2d_i8_nhwc(...), O)`` with the f32 output never stored:
    ``(q int8 [N, OH, OW, O], s [1])`` at the output's dynamic per-tensor scale, bit for bit
    (bq_conv2d_i8_nhwc_dq: the small-K kernel twice, its maxima, then its twin).
    NotImplementedError (nothing launched) where the small-K kernel does not run the layer's
    twin or O % 16 != 0: the caller takes the two-call form."""
    _need(qx, "x", torch.int8)
    N, H, W, C = qx.shape
    if C != wq.cpad:
        raise RuntimeError(f"channels do not match: input {C}, filter {wq.cpad}")
    OH = (H + 2 * pad - wq.KH) // stride + 1
    OW = (W + 2 * pad - wq.KW) // stride + 1
    if OH < 1 or OW < 1:
        raise RuntimeError("the filter is larger than the input.")
    if wq.O % 16:
        raise NotImplementedError(f"conv2d_i8_nhwc_dq: O={wq.O} is not a multiple of 16")
    res = None
    if residual is not None:
        if tuple(residual.shape) != (N, wq.O, OH, OW):
            raise RuntimeError(f"residual shape {tuple(residual.shape)} != output {(N, wq.O, OH, OW)}")
        res = residual.float().contiguous(memory_format=torch.channels_last)
    b = _vec(bias, wq.O, "bias")
    q = torch.empty((N, OH, OW, wq.O), dtype=torch.int8, device=qx.device)
    s = torch.empty((1,), dtype=torch.float32, device=qx.device)
    parts = torch.empty((4096,), dtype=torch.float32, device=qx.device)
    check(lib().bq_conv2d_i8_nhwc_dq(qx.contiguous().data_ptr(), N, H, W, C, wq.q.data_ptr(), wq.O, wq.KH, wq.KW,
                                     stride, pad, sa.data_ptr(), wq.s.data_ptr(), _ptr(b), _ptr(res), act,
                                     q.data_ptr(), s.data_ptr(), parts.data_ptr(), parts.numel(), _stream(qx)))
    return q, s


@dataclass
class PairConv:
    """One convolution of ``conv2d_pair_i8_nhwc``: its packed filter and epilogue. ``s_out`` (a
    calibrated output scale [1]) adds the int8 twin; ``amax``: the f32 output's per-tile
    maxima are written too (the first conv of a pair only)."""
    wq: Int8ConvWeight
    stride: int = 1
    pad: int = 0
    bias: torch.Tensor | None = None
    act: int = ACT_NONE
    s_out: torch.Tensor | None = None
    amax: bool = False


def conv2d_pair_i8_nhwc(qx, sa, first: PairConv, second: PairConv):
    """Two convs of one NHWC int8 input ``qx`` (scale ``sa``) in one launch
    (bq_conv2d_i8_nhwc_pair): a residual block's first conv and its shortcut. Returns
    ``[(out, q), (out, q)]``: each f32 output NCHW-shaped in channels-last memory and its int8
    twin (None without ``s_out``), bit-identical to ``conv2d_i8_nhwc`` / ``conv2d_i8_nhwc_q``;
    the first output carries its per-tile maxima when ``first.amax``."""
    _need(qx, "x", torch.int8)
    N, H, W, C = qx.shape
    descs, results, keep = [], [], []
    for i, c in enumerate((first, second)):
        if C != c.wq.cpad:
            raise RuntimeError(f"channels do not match: input {C}, filter {c.wq.cpad}")
        OH = (H + 2 * c.pad - c.wq.KH) // c.stride + 1
        OW = (W + 2 * c.pad - c.wq.KW) // c.stride + 1
        if OH < 1 or OW < 1:
            raise RuntimeError("the filter is larger than the input.")
        out = torch.empty((N, c.wq.O, OH, OW), dtype=torch.float32, device=qx.device,
                          memory_format=torch.channels_last)
        q = torch.empty((N, OH, OW, c.wq.O), dtype=torch.int8, device=qx.device) if c.s_out is not None else None
        parts = None
        if c.amax:
            if i:
                raise ValueError("only the first conv of a pair writes per-tile maxima")
            parts, nparts = _absmax_parts(N, H, W, C, c.wq, c.stride, c.pad, qx.device)
            out._bq_absmax = (parts, nparts, out._version)
        b = _vec(c.bias, c.wq.O, "bias")
        keep.append((b, c.s_out))
        descs.append(_lib.ConvDesc(c.wq.q.data_ptr(), c.wq.O, c.wq.KH, c.wq.KW, c.stride, c.pad, c.wq.s.data_ptr(),
                                   _ptr(b), None, c.act, out.data_ptr(), _ptr(c.s_out), _ptr(q), _ptr(parts)))
        results.append((out, q))
    check(lib().bq_conv2d_i8_nhwc_pair(qx.contiguous().data_ptr(), N, H, W, C, sa.data_ptr(), descs[0], descs[1],
                                       *_ws_args(qx.device), _stream(qx)))
    return results


def attention_f32(qkv: torch.Tensor, heads: int) -> torch.Tensor:
    """Softmax attention of every head in f32, from a qkv projection's output ``[B, T, 3 D]``
    (per token q, k, v side by side, each ``[heads, 64]``) to ``[B, T, D]``, the heads side by
    side (bq_attention_f32: ``softmax((q k^T) / 8) v``, head width 64, T <= 256; the int8
    layers on either side stay as they are: this is f32 beside the path)."""
    if qkv.dtype != torch.float32:
        raise TypeError(f"attention_f32 takes float32, got {qkv.dtype}")
    require_device(qkv.device)
    B, T, D3 = qkv.shape
    D = D3 // 3
    if D3 != 3 * D or D % heads:
        raise RuntimeError(f"qkv of width {D3} does not hold {heads} heads of q, k and v")
    x = qkv.contiguous()
    out = torch.empty((B, T, D), dtype=torch.float32, device=qkv.device)
    check(lib().bq_attention_f32(x.data_ptr(), B, T, heads, D // heads, out.data_ptr(), _stream(x)))
    return out


def avgpool_linear(x: torch.Tensor, weight: torch.Tensor, bias=None) -> torch.Tensor:
    """``linear(x.mean((2, 3)), weight, bias)`` in f32 for a channels-last ``x [N, C, H, W]`` and a
    small head (``O * C <= 65536``) in one launch (bq_avgpool_linear_f32) → ``[N, O]``."""
    if x.dtype != torch.float32:
        raise TypeError(f"avgpool_linear takes float32, got {x.dtype}")
    require_device(x.device)
    N, C, H, W = x.shape
    O = weight.shape[0]
    if weight.shape[1] != C:
        raise RuntimeError(f"mat1 and mat2 shapes cannot be multiplied ({N}x{C} and {weight.shape[1]}x{O})")
    xl = x.contiguous(memory_format=torch.channels_last)
    w = weight.detach().float().contiguous()
    b = _vec(bias, O, "bias")
    out = torch.empty((N, O), dtype=torch.float32, device=x.device)
    check(lib().bq_avgpool_linear_f32(xl.data_ptr(), N, H * W, C, w.data_ptr(), _ptr(b), O, out.data_ptr(),
                                      _stream(xl)))
    return out


def dwconv_i8_nhwc(qx, sa, wq: Int8DwWeight, stride=1, pad=0, bias=None, act=ACT_NONE, want_acc=False):
    """Depthwise int8 conv on NHWC int8 ``qx [N, H, W, Cpad]`` (bq_dwconv_i8_nhwc).
    Returns f32 ``[N, Cpad, OH, OW]`` in channels-last memory (and int32 NHWC acc)."""
    _need(qx, "x", torch.int8)
    N, H, W, C = qx.shape
    if C != wq.cpad:
        raise RuntimeError(f"channels do not match: input {C}, filter {wq.cpad}")
    OH = (H + 2 * pad - wq.KH) // stride + 1
    OW = (W + 2 * pad - wq.KW) // stride + 1
    if OH < 1 or OW < 1:
        raise RuntimeError("the filter is larger than the input.")
    out = torch.empty((N, C, OH, OW), dtype=torch.float32, device=qx.device, memory_format=torch.channels_last)
    acc = torch.empty((N, OH, OW, C), dtype=torch.int32, device=qx.device) if want_acc else None
    b = None
    if bias is not None:
        if bias.numel() not in (wq.C, C):
            raise ValueError(f"bias: expected {wq.C} values, got {bias.numel()}")
        b = bias.contiguous().float()
        if b.numel() != C:
            b = torch.nn.functional.pad(b, (0, C - b.numel()))
    check(lib().bq_dwconv_i8_nhwc(qx.contiguous().data_ptr(), N, H, W, C, wq.q.data_ptr(), wq.KH, wq.KW, stride,
                                  pad, sa.data_ptr(), wq.s.data_ptr(), _ptr(b), act, out.data_ptr(), _ptr(acc),
                                  _stream(qx)))
    return (out, acc) if want_acc else out


# ----------------------------------------------------------------- float-in, float-out

def linear(x: torch.Tensor, w8: Int8Weight, bias=None, act=ACT_NONE, residual=None,
           pre_act=ACT_NONE) -> torch.Tensor:
    """Dynamic-quant int8 Linear: per-row activations, per-channel weights, f32 out
    ``[..., N]`` (the numpy core's ``x @ W.T + b``, borch/_nn.py:413-415, in W8A8), with an
    optional ``residual [..., N]`` added in the epilogue before ``act``. ``pre_act`` applies
    an activation to ``x`` first, inside the input quantizer. A weight-only packing runs
    ``linear_w8a32`` instead."""
    if pre_act != ACT_NONE and (w8.weight_only or w8.per_tensor or w8.kpad != w8.in_features):
        x = _act_f32(x, pre_act)
        pre_act = ACT_NONE
    if w8.weight_only:
        return linear_w8a32(x, w8, bias, act, residual)
    if x.shape[-1] != w8.in_features:
        a = "x".join(str(n) for n in (x.reshape(-1, x.shape[-1]).shape if x.dim() else ()))
        raise RuntimeError(
            f"mat1 and mat2 shapes cannot be multiplied ({a} and {w8.in_features}x{w8.out_features})")
    lead = x.shape[:-1]
    x2 = x.reshape(-1, x.shape[-1])
    if w8.kpad != w8.in_features:
        x2 = torch.nn.functional.pad(x2, (0, w8.kpad - w8.in_features))
    r = None if residual is None else residual.reshape(-1, w8.out_features)
    if x2.shape[0] <= 4 and pre_act == ACT_NONE and not w8.per_tensor:
        return linear_rows(x2, w8, bias, act, r).reshape(*lead, w8.out_features)
    qa, sa = quantize_tensor(x2) if w8.per_tensor else quantize_rows(x2, pre_act)
    out = gemm_i8(qa, w8.q, sa, w8.s, bias, act, residual=r)
    return out.reshape(*lead, w8.out_features)


def linear_rows(x2: torch.Tensor, w8: Int8Weight, bias=None, act=ACT_NONE, residual=None, want_q: bool = False):
    """The dynamic-quant W8A8 Linear on f32 ``x2 [M, Kpad]`` in one call (bq_linear_i8: for
    M <= 4 one launch, the per-row quantization fused into the GEMV). Returns ``out [M, N]``,
    or ``(out, q int8 [M, Kpad], s [M])`` with ``want_q``."""
    x2 = _f32c(x2)
    require_device(x2.device)
    M, K = x2.shape
    N = w8.out_features
    if K != w8.kpad:
        raise RuntimeError(f"mat1 and mat2 shapes cannot be multiplied ({M}x{K} and {w8.kpad}x{N})")
    b = _vec(bias, N, "bias")
    r = None
    if residual is not None:
        if tuple(residual.shape) != (M, N):
            raise RuntimeError(f"residual shape {tuple(residual.shape)} != output {(M, N)}")
        r = residual.float().contiguous()
    out = torch.empty((M, N), dtype=torch.float32, device=x2.device)
    need_q = want_q or M > 4 or K > 8192
    q = torch.empty((M, K), dtype=torch.int8, device=x2.device) if need_q else None
    s = torch.empty((M,), dtype=torch.float32, device=x2.device) if need_q else None
    check(lib().bq_linear_i8(x2.data_ptr(), w8.q.data_ptr(), M, N, K, w8.s.data_ptr(), _ptr(b), _ptr(r), act,
                             out.data_ptr(), _ptr(q), _ptr(s), *_ws_args(x2.device), _stream(x2)))
    return (out, q, s) if want_q else out


def layernorm_quantize_rows(x: torch.Tensor, weight, bias, eps: float, want_y: bool = False):
    """LayerNorm over the last axis of ``x [M, K]`` then per-row int8 of the result, in one
    pass (bq_layernorm_quantize_rows): ``(q int8 [M, K], s [M])``, and the normalised f32
    rows too with ``want_y``. The reference's layerNormRows order (kernels.ts:2935-2986)."""
    _need(x, "x", torch.float32)
    if x.dim() != 2:
        raise ValueError("layernorm_quantize_rows takes [M, K]")
    x = x.contiguous()
    M, K = x.shape
    g = _vec(weight, K, "weight")
    b = _vec(bias, K, "bias")
    q = torch.empty((M, K), dtype=torch.int8, device=x.device)
    s = torch.empty((M,), dtype=torch.float32, device=x.device)
    y = torch.empty((M, K), dtype=torch.float32, device=x.device) if want_y else None
    check(lib().bq_layernorm_quantize_rows(x.data_ptr(), M, K, _ptr(g), _ptr(b), float(eps), q.data_ptr(),
                                           s.data_ptr(), _ptr(y), _stream(x)))
    return (q, s, y) if want_y else (q, s)


def fusable_layernorm(ln, x: torch.Tensor, w8: Int8Weight) -> bool:
    """Whether ``ln`` (a torch LayerNorm) can run inside the W8A8 Linear's input quantizer."""
    K = x.shape[-1] if x.dim() else 0
    return (isinstance(ln, torch.nn.LayerNorm) and tuple(ln.normalized_shape) == (K,) and x.is_cuda
            and x.dtype == torch.float32 and not w8.weight_only and not w8.per_tensor and K % 4 == 0 and K <= 4096
            and w8.kpad == K == w8.in_features)


def layernorm_linear(x: torch.Tensor, ln, w8: Int8Weight, bias=None, act=ACT_NONE, residual=None) -> torch.Tensor:
    """``linear(ln(x))`` in W8A8 with the LayerNorm in the input quantizer: the normalised
    activation is never stored (``fusable_layernorm`` must hold)."""
    lead = x.shape[:-1]
    q, s = layernorm_quantize_rows(x.reshape(-1, x.shape[-1]), ln.weight, ln.bias, ln.eps)
    r = None if residual is None else residual.reshape(-1, w8.out_features)
    out = gemm_i8(q, w8.q, s, w8.s, bias, act, residual=r)
    return out.reshape(*lead, w8.out_features)


def _act_f32(out: torch.Tensor, act: int) -> torch.Tensor:
    """The epilogue activations as torch f32 ops (the f32 paths and fallbacks)."""
    if act == ACT_RELU:
        return torch.relu(out)
    if act == ACT_SILU:
        return torch.nn.functional.silu(out)
    if act == ACT_GELU:
        return torch.nn.functional.gelu(out)
    return out


def conv2d(x: torch.Tensor, w8: Int8ConvWeight, bias=None, stride=1, padding=0, act=ACT_NONE,
           residual=None) -> torch.Tensor:
    """Dynamic-quant int8 conv (per-tensor activation scale, tensor.ts:11915-11920):
    quantize into NHWC, implicit GEMM, fused epilogue; NCHW-shaped channels-last out."""
    if x.dim() != 4:
        raise RuntimeError(f"conv2d expects a 4-D input, got {x.dim()}-D")
    if x.shape[1] != w8.C:
        raise RuntimeError(f"channels do not match: input {x.shape[1]}, filter {w8.C}")
    qx, sa = quantize_nhwc(x, w8.cpad)
    return conv2d_i8_nhwc(qx, sa, w8, stride, padding, bias, residual, act)


def depthwise_conv2d(x: torch.Tensor, w8: Int8DwWeight, bias=None, stride=1, padding=0,
                     act=ACT_NONE) -> torch.Tensor:
    """Dynamic-quant int8 depthwise conv; NCHW-shaped channels-last f32 out."""
    if x.dim() != 4 or x.shape[1] != w8.C:
        raise RuntimeError(f"channels do not match: input {x.shape[1]}, filter {w8.C}")
    qx, sa = quantize_nhwc(x, w8.cpad)
    out = dwconv_i8_nhwc(qx, sa, w8, stride, padding, bias, act)
    return out if w8.cpad == w8.C else out[:, : w8.C]
