"""CPU oracle for the int8 inference path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg may
import this module, and only as the checker. The product path (``borch_amd``) never
calls it: it runs the HIP library or raises.

Every function restates the reference's arithmetic in numpy and cites the file:line it
follows (paths are into playidea-lab/borch). Integer results are exact: int8 products are
accumulated in float64 BLAS, which is exact while |acc| < 2**53 (K·127² = 66,064,384 at
K = 4096), then cast to int32.

Rounding rule (one rule for weights and activations, fixed by the task contract):

* ``s = float32(max|v| / 127)`` — a correctly rounded float32 division;
* ``q = clip(rint(float64(v) / float64(s)), -127, 127)`` — the exact quotient of two
  float32 values rounded half-to-even, as the numpy core's ``_quantize_round`` does
  (borch/_ops.py:4559-4568, ``np.round`` of a float64 quotient);
* ``s == 0`` (an all-zero row or tensor) gives ``q = 0`` (borch-ts/src/quant.ts:36).

The reference's two weight packers are restated bit for bit below
(``quantize_weight_reference_linear``, ``quantize_conv_weight_reference``), and they relate
to this rule differently:

* the conv packer (borch-ts/src/quant.ts:88-96) divides by the *stored* float32 scale and
  rounds with JS ``Math.round`` (half toward +inf): it differs from this rule only on exact
  ties;
* the Linear packer (quant.ts:35-40) multiplies by ``1/scale`` with the *unrounded* float64
  scale ``peak/127``. Its quotient ``w·(127/peak)`` differs from ``w/f32(peak/127)`` by up to
  a few 1e-6, so near-ties (not only exact ties) can round to the other side: on C2's
  4096×4096 weight 12 bytes differ and none is an exact tie; on C1's 512×512 none differ.
  ``tests/test_oracle.py`` pins both counts and positions.

Pinning (what checks each function; see tests/test_oracle.py):

* quantize_*: the reference golden ``top::fake_quantize*`` values (tests/golden.json of
  the reference, copied as data into tests/golden/ref_fake_quantize.json), hand-built
  exact ties, brute-force scalar restatement, invariants (|q| ≤ 127, peak → ±127,
  |q·s − v| ≤ s/2).
* gemm_i8_i32: a brute-force int64 triple loop on tiny shapes with the LCG operands of
  tests/browser/kernel_bench.html:300-303, closed forms (all ±127 rows, identity).
* dequant: closed-form order ``fround(fround(fround(acc·sA)·sW)+b)``
  (kernel_bench.html:321) on hand values.
* conv2d_i8_nhwc / dwconv_i8_nhwc: direct 7-deep brute-force loops on tiny shapes
  (kernel_bench.html:406-413), and im2col equivalence (borch/_ops.py:671-691).
* fma_f32 / linear_w8a32_gemv: exact-rational brute force of the single rounding, a hand
  case where the fused product keeps a bit that a separate product rounds away, integer
  operands whose every sum is exact (the result is the integer dot product, so a dropped
  or misplaced term shows), and a hand case whose value depends on the lane tree's order
  (it differs from both the exact sum and a left-to-right sum).
"""
from __future__ import annotations

import numpy as np

I8_MAX = 127


# ----------------------------------------------------------------------------- scales

def scale_of(peak):
    """float32(peak / 127), correctly rounded (numpy float32 division is IEEE).

    borch-ts/src/quant.ts:35 (``scale = peak / I8_MAX``) and quant.ts:88 for the conv
    packer, whose stored scale is the float32 of the same quotient."""
    peak = np.asarray(peak, dtype=np.float32)
    return (peak / np.float32(I8_MAX)).astype(np.float32)


def round_quotient(v, s):
    """``rint(f64(v) / f64(s))`` (half to even), 0 where s == 0, as float64.

    The rounding core of borch/_ops.py:4566 (``np.round(x / scale)`` on float64) with the
    zero-scale rule of borch-ts/src/quant.ts:36. ``s`` broadcasts against ``v``."""
    v64 = np.asarray(v, dtype=np.float32).astype(np.float64)
    s64 = np.broadcast_to(np.asarray(s, dtype=np.float32), v64.shape).astype(np.float64)
    with np.errstate(divide="ignore", invalid="ignore"):
        return np.rint(np.where(s64 != 0, v64 / np.where(s64 != 0, s64, 1.0), 0.0))


def quantize_with_scale(v, s):
    """``clip(rint(f64(v)/f64(s)), ±127)`` with s == 0 → 0: ``round_quotient`` and the
    symmetric clamp of borch-ts/src/quant.ts:40."""
    return np.clip(round_quotient(v, s), -I8_MAX, I8_MAX).astype(np.int8)


# ------------------------------------------------------------------------ quantizers

def quantize_rows(x):
    """Per-row symmetric int8: ``s[m] = f32(max|x[m,:]|/127)``, ``q = round(x/s)``.

    Follows the per-channel packer borch-ts/src/quant.ts:23-53 (one scale per row of a
    row-major matrix) applied to activations, as the task's per-row dynamic quantization
    asks (the reference's activation quantizer is per tensor, kernels.ts:2057-2081).
    Returns ``(q int8 [M,K], s float32 [M])``."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    if x.ndim != 2:
        raise ValueError("quantize_rows wants a 2-D array")
    peak = np.abs(x).max(axis=1) if x.shape[1] else np.zeros(x.shape[0], np.float32)
    s = scale_of(peak)
    return quantize_with_scale(x, s[:, None]), s


def quantize_weight_per_channel(w):
    """Per-output-channel int8 of a Linear weight ``[N, K]`` (row-major, ``x @ W.T``).

    borch-ts/src/quant.ts:23-53: ``scale[o] = max|W[o,:]|/127``, zero row → scale 0 and
    zeros (:36), byte order = W's own row-major order (:42-51). Returns
    ``(q int8 [N,K], s float32 [N])``."""
    return quantize_rows(w)


def js_math_round(x):
    """JavaScript ``Math.round`` on float64: the nearest integer, a tie going toward +inf
    (ECMA-262 §21.3.2.28). ``x - floor(x)`` is exact for every double, so the comparison
    with 0.5 decides ties exactly (``floor(x + 0.5)`` would not: 0.49999999999999994 + 0.5
    rounds up to 1)."""
    x = np.asarray(x, dtype=np.float64)
    f = np.floor(x)
    return f + ((x - f) >= 0.5)


def quantize_weight_reference_linear(w):
    """borch-ts/src/quant.ts:23-41 as JavaScript evaluates it, bit for bit.

    Per row ``o`` of ``w [N, K]``: ``peak`` = the largest ``|w|`` (a float32 value, held as
    a double); ``scale = peak / 127`` in float64 (:35), stored as float32 in the returned
    scales (``Float32Array``, :36); a zero scale leaves the row zero (:37); otherwise
    ``inv = 1 / scale`` in float64 (:38) and ``q = clamp(Math.round(w · inv), ±127)`` with the
    product in float64 (:39-41). Returns ``(q int8 [N, K], s float32 [N])``."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    N = w.shape[0]
    w2 = w.reshape(N, -1)
    peak = (np.abs(w2).max(axis=1) if w2.shape[1] else np.zeros(N, np.float32)).astype(np.float64)
    scale = peak / 127.0
    with np.errstate(divide="ignore"):
        inv = np.where(scale != 0, 1.0 / np.where(scale != 0, scale, 1.0), 0.0)
    r = js_math_round(w2.astype(np.float64) * inv[:, None])
    r = np.clip(r, -I8_MAX, I8_MAX)
    r[scale == 0] = 0
    return r.astype(np.int8).reshape(w.shape), scale.astype(np.float32)


def quantize_conv_weight_reference(w):
    """borch-ts/src/quant.ts:80-96's arithmetic, bit for bit, on a weight ``[O, ...]`` with
    one scale per leading index (the layout change of :97-99 aside).

    ``scales[o] = f32(peak / 127)`` (the float64 quotient stored in a ``Float32Array``,
    :88, which equals the correctly rounded float32 quotient); each element
    ``q = clamp(Math.round(w / scales[o]), ±127)`` with the division in float64 by the
    stored float32 scale (:93-95); a zero scale gives 0 (:92). Returns
    ``(q int8 [O, ...], s float32 [O])`` in the input's own order."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    O = w.shape[0]
    w2 = w.reshape(O, -1)
    peak = np.abs(w2).max(axis=1) if w2.shape[1] else np.zeros(O, np.float32)
    s = (peak.astype(np.float64) / 127.0).astype(np.float32)
    s64 = s.astype(np.float64)
    with np.errstate(divide="ignore", invalid="ignore"):
        r = js_math_round(w2.astype(np.float64) / np.where(s64 != 0, s64, 1.0)[:, None])
    r = np.clip(r, -I8_MAX, I8_MAX)
    r[s == 0] = 0
    return r.astype(np.int8).reshape(w.shape), s


def pack_words(q):
    """Four signed bytes per little-endian u32, low byte first (quant.ts:42-51).

    A pure byte view: int8 ``q`` flattened, padded with zero bytes to a whole word."""
    b = np.ascontiguousarray(q, dtype=np.int8).reshape(-1).view(np.uint8)
    pad = (-b.size) % 4
    if pad:
        b = np.concatenate([b, np.zeros(pad, np.uint8)])
    return (b[0::4].astype(np.uint32) | (b[1::4].astype(np.uint32) << 8)
            | (b[2::4].astype(np.uint32) << 16) | (b[3::4].astype(np.uint32) << 24))


def quantize_conv_weight(w, cpad=None):
    """Per-output-channel int8 of a conv weight ``[O, C, KH, KW]``.

    Scale rule of borch-ts/src/quant.ts:80-92 (one scale per O over all C·KH·KW). Layout:
    ``[O][KH][KW][Cpad]`` — K-contiguous per output channel, tap-major then channel
    (the NHWC im2col order of borch-ts/wasm/src/lib.rs:283-286), channels zero-padded to
    ``cpad``. Zero padding changes neither the peak nor any product. Returns
    ``(q int8 [O, KH*KW*cpad], s float32 [O])``."""
    w = np.asarray(w, dtype=np.float32)
    O, C, KH, KW = w.shape
    cpad = C if cpad is None else cpad
    t = np.zeros((O, KH, KW, cpad), np.float32)
    t[..., :C] = w.transpose(0, 2, 3, 1)
    return quantize_rows(t.reshape(O, KH * KW * cpad))


def quantize_dw_weight(w):
    """Depthwise weight ``[C, 1, KH, KW]`` → int8 ``[KH*KW, C]`` (tap-major, channel
    contiguous) with one scale per channel over its taps (quant.ts:80-92's rule)."""
    w = np.asarray(w, dtype=np.float32)
    C, one, KH, KW = w.shape
    assert one == 1
    q, s = quantize_rows(w.reshape(C, KH * KW))
    return np.ascontiguousarray(q.T), s


def quantize_tensor(x):
    """Per-tensor symmetric int8: ``s = f32(max|x|/127)`` over the whole tensor.

    borch-ts/src/kernels.ts:2024-2044 (``absMaxAtomic``: Max[0] = max|x|) and
    kernels.ts:2057-2081 (``quantizeActivationInt8``), with the exact-quotient rounding
    of this module instead of the reference's ``x·(1/s)``. Returns ``(q, s float32 [1])``."""
    x = np.asarray(x, dtype=np.float32)
    peak = np.abs(x).max() if x.size else np.float32(0)
    s = scale_of(np.array([peak], np.float32))
    return quantize_with_scale(x, s[0]), s


def quantize_act_nhwc(x_nchw, cpad=None):
    """Per-tensor int8 of an NCHW activation, laid out NHWC with channels zero-padded.

    Per-tensor scale as the reference's conv input (tensor.ts:11915-11920); layout NHWC
    instead of the reference's NC/4HW4 (kernels.ts:2057-2081). Returns
    ``(q int8 [N,H,W,cpad], s float32 [1])``."""
    x = np.asarray(x_nchw, dtype=np.float32)
    N, C, H, W = x.shape
    cpad = C if cpad is None else cpad
    q, s = quantize_tensor(x)
    out = np.zeros((N, H, W, cpad), np.int8)
    out[..., :C] = q.transpose(0, 2, 3, 1)
    return out, s


# ------------------------------------------------------------------------- integer ops

def gemm_i8_i32(a, w):
    """``acc[m,n] = Σ_k a[m,k]·w[n,k]`` exactly, int8 × int8 → int32.

    The integer product of borch-ts/src/kernels.ts:1808-1852 (``matmulInt8``) in the
    Linear layout ``x @ W.T`` (borch/_nn.py:413-415). Exact via float64 BLAS (every
    partial sum is an integer below 2**53)."""
    a64 = np.asarray(a, dtype=np.int8).astype(np.float64)
    w64 = np.asarray(w, dtype=np.int8).astype(np.float64)
    return (a64 @ w64.T).astype(np.int32)


def dequant(acc, sA, sW, bias=None, relu=False, residual=None):
    """The W8A8 epilogue, float32 with one rounding per operation:
    ``y = ((f32(acc)·sA[m])·sW[n]) + b[n]``, then ``+ residual``, then ``max(y, 0)``.

    Order of borch-ts/src/kernels.ts:1818-1827 and the check at
    tests/browser/kernel_bench.html:321 (``fround(fround(fround(acc·s0)·s1)+b)``); residual
    and relu after bias as ``ConvEpilogue`` (kernels.ts:4230-4244). ``sA`` is a per-row
    vector ``[M]`` or a scalar (per tensor); ``acc`` is ``[M, N]``."""
    acc = np.asarray(acc, dtype=np.int32)
    y = acc.astype(np.float32)
    sA = np.asarray(sA, dtype=np.float32)
    sA = sA.reshape(-1, 1) if sA.size == acc.shape[0] and sA.size != 1 else sA.reshape(())
    y = (y * sA).astype(np.float32)
    y = (y * np.asarray(sW, dtype=np.float32).reshape(1, -1)).astype(np.float32)
    if bias is not None:
        y = (y + np.asarray(bias, dtype=np.float32).reshape(1, -1)).astype(np.float32)
    if residual is not None:
        y = (y + np.asarray(residual, dtype=np.float32).reshape(y.shape)).astype(np.float32)
    if relu:
        y = np.where(y > 0, y, np.float32(0)).astype(np.float32)
    return y


def silu(y):
    """f32 SiLU ``y·sigmoid(y)`` (closed form; float64 then rounded)."""
    y64 = np.asarray(y, dtype=np.float64)
    return (y64 / (1.0 + np.exp(-y64))).astype(np.float32)


def gelu(y):
    """f32 GELU, erf form ``y·Φ(y) = 0.5·y·(1 + erf(y/√2))`` (closed form; float64 then
    rounded): the activation of a transformer MLP (torch's default ``gelu``)."""
    from scipy.special import erf
    y64 = np.asarray(y, dtype=np.float64)
    return (0.5 * y64 * (1.0 + erf(y64 / np.sqrt(2.0)))).astype(np.float32)


def im2col_nhwc(xq, KH, KW, stride, pad):
    """``(N, H, W, C)`` → ``(N·OH·OW, KH·KW·C)``, zero outside, tap-major then channel.

    The column order of borch-ts/wasm/src/lib.rs:643-678 (``im2col_rows``); the window
    walk of borch/_ops.py:671-691 (``_im2col``) on an NHWC tensor."""
    N, H, W, C = xq.shape
    xp = np.zeros((N, H + 2 * pad, W + 2 * pad, C), xq.dtype)
    xp[:, pad:pad + H, pad:pad + W] = xq
    OH = (H + 2 * pad - KH) // stride + 1
    OW = (W + 2 * pad - KW) // stride + 1
    cols = np.empty((N, OH, OW, KH, KW, C), xq.dtype)
    for kh in range(KH):
        for kw in range(KW):
            cols[:, :, :, kh, kw] = xp[:, kh:kh + stride * (OH - 1) + 1:stride,
                                       kw:kw + stride * (OW - 1) + 1:stride]
    return cols.reshape(N * OH * OW, KH * KW * C), OH, OW


def conv2d_i8_nhwc(xq, wq, KH, KW, stride=1, pad=0):
    """Integer conv: NHWC int8 ``xq [N,H,W,C]`` with ``wq [O, KH·KW·C]`` → int32
    ``[N·OH·OW, O]``.

    The implicit GEMM of borch-ts/src/kernels.ts:2156-2302 (``convForwardInt8``) as an
    explicit one: im2col (above) and the exact int8 GEMM. Checked against
    tests/browser/kernel_bench.html:406-413's direct loops in the tests."""
    cols, OH, OW = im2col_nhwc(np.asarray(xq, np.int8), KH, KW, stride, pad)
    return gemm_i8_i32(cols, wq), OH, OW


def dwconv_i8_nhwc(xq, wq, KH, KW, stride=1, pad=0):
    """Depthwise integer conv: ``xq [N,H,W,C]`` int8, ``wq [KH·KW, C]`` int8 → int32
    ``[N, OH, OW, C]``.

    The per-channel tap sum of borch-ts/wasm/src/lib.rs:598-641 (``dwconv_rows``) and
    kernels.ts:5932-5968 (``depthwiseForward``) on integers."""
    xq = np.asarray(xq, np.int8)
    N, H, W, C = xq.shape
    xp = np.zeros((N, H + 2 * pad, W + 2 * pad, C), np.int32)
    xp[:, pad:pad + H, pad:pad + W] = xq
    OH = (H + 2 * pad - KH) // stride + 1
    OW = (W + 2 * pad - KW) // stride + 1
    acc = np.zeros((N, OH, OW, C), np.int32)
    w32 = np.asarray(wq, np.int8).astype(np.int32).reshape(KH, KW, C)
    for kh in range(KH):
        for kw in range(KW):
            acc += xp[:, kh:kh + stride * (OH - 1) + 1:stride,
                      kw:kw + stride * (OW - 1) + 1:stride] * w32[kh, kw]
    return acc


# ----------------------------------------------------------------- composite oracles

def linear_int8(x, w, b=None, relu=False):
    """The whole dynamic-quant int8 Linear: per-row x, per-channel W, exact int32, f32
    epilogue. Returns ``(y, acc, (qx, sx), (qw, sw))``."""
    qx, sx = quantize_rows(np.asarray(x, np.float32))
    qw, sw = quantize_weight_per_channel(np.asarray(w, np.float32))
    acc = gemm_i8_i32(qx, qw)
    return dequant(acc, sx, sw, b, relu), acc, (qx, sx), (qw, sw)


def conv2d_int8(x_nchw, w, b=None, stride=1, pad=0, relu=False, residual_nchw=None, cpad=None):
    """The whole int8 conv: per-tensor activation, per-channel weight, exact int32, f32
    epilogue, NCHW out. Returns ``(y_nchw, acc [N·OH·OW, O], sA, sW)``."""
    x_nchw = np.asarray(x_nchw, np.float32)
    O, C, KH, KW = np.asarray(w).shape
    cpad = C if cpad is None else cpad
    xq, sA = quantize_act_nhwc(x_nchw, cpad)
    wq, sW = quantize_conv_weight(w, cpad)
    acc, OH, OW = conv2d_i8_nhwc(xq, wq, KH, KW, stride, pad)
    N = x_nchw.shape[0]
    res = None
    if residual_nchw is not None:
        res = np.asarray(residual_nchw, np.float32).transpose(0, 2, 3, 1).reshape(-1, O)
    y = dequant(acc, sA[0], sW, b, relu, res)
    return y.reshape(N, OH, OW, O).transpose(0, 3, 1, 2), acc, sA, sW


# ---------------------------------------------------------------- f32 numpy-core ops

def linear_f32(x, w, b=None):
    """numpy core ``F.linear``: ``x @ W.T (+ b)`` in float32 (borch/_nn.py:4675-4677)."""
    y = np.asarray(x, np.float32) @ np.asarray(w, np.float32).T
    return y + np.asarray(b, np.float32) if b is not None else y


def conv2d_f32(x, w, b=None, stride=1, pad=0):
    """numpy core ``conv2d`` (groups 1): pad, im2col, one float32 GEMM
    (borch/_ops.py:671-691, 738-791)."""
    x = np.asarray(x, np.float32)
    w = np.asarray(w, np.float32)
    if pad:
        x = np.pad(x, ((0, 0), (0, 0), (pad, pad), (pad, pad)))
    N, C, H, W = x.shape
    F, C2, KH, KW = w.shape
    if C != C2:
        raise RuntimeError(f"channels do not match: input {C}, filter {C2}")
    win = np.lib.stride_tricks.sliding_window_view(x, (KH, KW), axis=(2, 3))
    win = win[:, :, ::stride, ::stride]
    OH, OW = win.shape[2], win.shape[3]
    cols = np.ascontiguousarray(win.transpose(0, 2, 3, 1, 4, 5)).reshape(N * OH * OW, C * KH * KW)
    out = (cols @ w.reshape(F, -1).T).reshape(N, OH, OW, F).transpose(0, 3, 1, 2)
    return out + b.reshape(1, -1, 1, 1) if b is not None else out


def fuse_conv_bn_weights(w, b, rm, rv, eps, gamma, beta):
    """BN fold of borch/_nn.py:4916-4937:
    ``scale = γ/√(var+eps)``, ``W' = W·scale``, ``b' = (b − mean)·scale + β``."""
    w = np.asarray(w, np.float32)
    rm = np.asarray(rm, np.float32)
    b = np.zeros_like(rm) if b is None else np.asarray(b, np.float32)
    gamma = np.ones_like(rm) if gamma is None else np.asarray(gamma, np.float32)
    beta = np.zeros_like(rm) if beta is None else np.asarray(beta, np.float32)
    scale = (gamma / np.sqrt(np.asarray(rv, np.float32) + eps)).astype(w.dtype)
    fw = (w * scale.reshape([-1] + [1] * (w.ndim - 1))).astype(w.dtype)
    fb = ((b - rm) * scale + beta).astype(b.dtype)
    return fw, fb


# ----------------------------------------------------------------- weight-only (W8A32)

def dequant_weight(q, s):
    """``f32(q) · s[n]`` with one float32 rounding: the effective weight of the reference's
    int8 window matmul (kernels.ts:2695-2708, ``f32(q) * scale[bcol]``) and of
    ``dequantInt8PerChannel`` (quant.ts:60-71). ``q [N, K]`` int8, ``s [N]``."""
    return (np.asarray(q, np.int8).astype(np.float32) * np.asarray(s, np.float32).reshape(-1, 1)).astype(np.float32)


def fma_f32(a, b, c):
    """Correctly rounded float32 ``a * b + c`` (one rounding), elementwise on float32
    arrays: the product is exact in float64 (24 + 24 bits); the float64 sum ``t`` and its
    exact error ``e`` (TwoSum) give ``a * b + c = t + e`` exactly, and rounding ``t`` to
    float32 is then the correct rounding unless ``t`` sits exactly halfway between two
    float32 values with ``e != 0`` (an f32 midpoint is a float64 value, so the float64
    rounding cannot cross one): there the result goes the way ``e`` points."""
    a64 = np.asarray(a, np.float32).astype(np.float64)
    b64 = np.asarray(b, np.float32).astype(np.float64)
    c64 = np.asarray(c, np.float32).astype(np.float64)
    p = a64 * b64
    t = p + c64
    bb = t - p
    e = (p - (t - bb)) + (c64 - bb)
    r = t.astype(np.float32)
    other = np.nextafter(r, np.where(t > r.astype(np.float64), np.float32(np.inf), np.float32(-np.inf)))
    mid = (r.astype(np.float64) + other.astype(np.float64)) * 0.5
    fix = (t != r.astype(np.float64)) & (t == mid) & (e != 0)
    up = np.maximum(r, other)
    down = np.minimum(r, other)
    return np.where(fix, np.where(e > 0, up, down), r).astype(np.float32)


def linear_w8a32_gemv(x, q, s, b=None, residual=None, relu=False):
    """The W8A32 decode GEMV's own float32 arithmetic (M <= 4), restated operation for
    operation: the effective weight ``f32(q) * s[n]`` (one rounding, kernels.ts:2695-2708),
    then for each output 64 lane sums, lane l accumulating ``acc = fma(x[k], w[k], acc)`` over
    k = 1024 c + 16 l + j (chunk c, then j = 0..15, in that order), then the lanes added as
    a pairwise tree in lane order ((l0 + l1) + (l2 + l3)) + ..., then ``+ b``, ``+ residual``
    and ReLU, one rounding each. This is the reference's own gate for its int8 window weight
    (tests/browser/window_probe.html:219-233: the int8 op equals the f32 op on the
    reconstructed weight, bit for bit), with the f32 op in the GPU kernel's order."""
    x = np.asarray(x, np.float32)
    w = dequant_weight(q, s)
    M, K = x.shape
    N = w.shape[0]
    kc = -(-K // 1024)
    acc = np.zeros((M, N, 64), np.float32)
    lanes = np.arange(64)
    for c in range(kc):
        for j in range(16):
            k = c * 1024 + 16 * lanes + j            # [64]
            valid = k < K
            kk = np.where(valid, k, 0)
            xv = x[:, kk][:, None, :]                # [M, 1, 64]
            wv = w[:, kk][None, :, :]                # [1, N, 64]
            acc = np.where(valid[None, None, :], fma_f32(xv, wv, acc), acc)
    while acc.shape[-1] > 1:
        acc = (acc[..., 0::2] + acc[..., 1::2]).astype(np.float32)
    y = acc[..., 0]
    if b is not None:
        y = (y + np.asarray(b, np.float32)).astype(np.float32)
    if residual is not None:
        y = (y + np.asarray(residual, np.float32)).astype(np.float32)
    if relu:
        y = np.where(y > 0, y, np.float32(0)).astype(np.float32)
    return y


def linear_w8a32(x, q, s, b=None):
    """W8A32 Linear in float64 on the f32 effective weights, plus the bound an f32
    accumulation of K products may differ by: ``(K + 2) · 2^-24 · Σ|x·w|`` per output
    (Higham's γ_K for recursive/tree summation with one rounding per product)."""
    w = dequant_weight(q, s).astype(np.float64)
    x64 = np.asarray(x, np.float32).astype(np.float64)
    y = x64 @ w.T
    if b is not None:
        y = y + np.asarray(b, np.float64)
    K = w.shape[1]
    bound = (K + 2) * 2.0 ** -24 * (np.abs(x64) @ np.abs(w).T) + 2.0 ** -24 * np.abs(y)
    return y, bound
