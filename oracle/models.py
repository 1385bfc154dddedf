"""Model-level oracle: the int8 layers of the configurations restated in numpy — TEST
INFRASTRUCTURE ONLY (imported by tests/ and the CPU-baseline leg of bench.py).

Each function takes the layer's float32 parameters as numpy arrays (read from the model
under test after the BN fold) and applies oracle.quant's arithmetic:

* ``conv_layer`` — per-tensor activation quantization into NHWC (tensor.ts:11915-11920),
  per-channel weights (quant.ts:80-103's scale rule), exact int32 implicit GEMM
  (kernels.ts:2156-2302 restated as im2col + GEMM), epilogue
  ``((acc·sA)·sW)+b (+residual)`` then the activation (kernels.ts:4230-4244);
* ``dwconv_layer`` — the same for a depthwise conv (lib.rs:598-641's tap sum, integers);
* ``linear_layer`` — per-row activations, per-channel weights (quant.ts:23-53);
* ``resnet18_features`` — the CIFAR ResNet-18 conv stack of export_resnet18.py:27-60
  chained layer by layer (pinned by the per-layer checks and the brute-force conv tests);
* ``se_gate``, ``attention_qkv``, ``avgpool_linear`` — the f32 pieces beside the path in
  float64 (the GPU tests also hold the attention to torch's own f32 attention, an
  independent implementation, and tests/test_oracle.py pins these two against torch).
"""
from __future__ import annotations

import numpy as np

from . import quant as Q

ACT_NONE, ACT_RELU, ACT_SILU, ACT_GELU = 0, 1, 2, 3


def _act(y, act):
    if act == ACT_RELU:
        return np.where(y > 0, y, np.float32(0)).astype(np.float32)
    if act == ACT_SILU:
        return Q.silu(y)
    if act == ACT_GELU:
        return Q.gelu(y)
    return y


def conv_layer(x_nchw, w, b, stride, pad, act=ACT_NONE, residual_nchw=None):
    """Returns ``(y_nchw, acc [N·OH·OW, O], sA, sW, qw)``."""
    x_nchw = np.asarray(x_nchw, np.float32)
    O_, C, KH, KW = w.shape
    cpad = (C + 15) // 16 * 16
    xq, sA = Q.quantize_act_nhwc(x_nchw, cpad)
    qw, sW = Q.quantize_conv_weight(w, cpad)
    acc, OH, OW = Q.conv2d_i8_nhwc(xq, qw, KH, KW, stride, pad)
    res = None
    if residual_nchw is not None:
        res = np.asarray(residual_nchw, np.float32).transpose(0, 2, 3, 1).reshape(-1, O_)
    y = Q.dequant(acc, sA[0], sW, b, False, res)
    y = _act(y, act)
    N = x_nchw.shape[0]
    return y.reshape(N, OH, OW, O_).transpose(0, 3, 1, 2), acc, sA, sW, qw


def dwconv_layer(x_nchw, w, b, stride, pad, act=ACT_NONE):
    """Depthwise; returns ``(y_nchw, acc [N, OH, OW, C], sA, sW, qw [KH·KW, C])``."""
    x_nchw = np.asarray(x_nchw, np.float32)
    C, _, KH, KW = w.shape
    cpad = (C + 3) // 4 * 4
    wp = np.zeros((cpad, 1, KH, KW), np.float32)
    wp[:C] = w
    xq, sA = Q.quantize_act_nhwc(x_nchw, cpad)
    qw, sW = Q.quantize_dw_weight(wp)
    acc = Q.dwconv_i8_nhwc(xq, qw, KH, KW, stride, pad)
    N, OH, OW, _ = acc.shape
    bp = np.zeros(cpad, np.float32)
    if b is not None:
        bp[:C] = b
    y = Q.dequant(acc.reshape(-1, cpad), sA[0], sW, bp)
    y = _act(y, act).reshape(N, OH, OW, cpad)[..., :C]
    return y.transpose(0, 3, 1, 2), acc[..., :C], sA, sW, qw


def linear_layer(x, w, b, act=ACT_NONE, residual=None):
    """Returns ``(y [..., N], acc [M, N], sA [M], sW, qw)``; ``residual [..., N]`` is added
    after the bias and before ``act`` (the fused ``LinearAdd`` epilogue)."""
    x = np.asarray(x, np.float32)
    lead = x.shape[:-1]
    K = x.shape[-1]
    kp = (max(K, 16) + 15) // 16 * 16
    x2 = np.zeros((int(np.prod(lead)) if lead else 1, kp), np.float32)
    x2[:, :K] = x.reshape(-1, K)
    wp = np.zeros((w.shape[0], kp), np.float32)
    wp[:, :K] = w
    qa, sA = Q.quantize_rows(x2)
    qw, sW = Q.quantize_weight_per_channel(wp)
    acc = Q.gemm_i8_i32(qa, qw)
    r = None if residual is None else np.asarray(residual, np.float32).reshape(-1, w.shape[0])
    y = _act(Q.dequant(acc, sA, sW, b, residual=r), act)
    return y.reshape(*lead, w.shape[0]), acc, sA, sW, qw


def resnet18_features(params, x):
    """The folded CIFAR ResNet-18 conv stack, int8 layer by layer. ``params`` maps
    ``stem``, ``body.{i}.c1|c2|down`` to ``(w, b, stride, pad)``. Returns the features
    before the mean pool, NCHW f32."""
    w, b, s, p = params["stem"]
    h = conv_layer(x, w, b, s, p, ACT_RELU)[0]
    for i in range(8):
        w1, b1, s1, p1 = params[f"body.{i}.c1"]
        out = conv_layer(h, w1, b1, s1, p1, ACT_RELU)[0]
        if f"body.{i}.down" in params:
            wd, bd, sd, pd = params[f"body.{i}.down"]
            side = conv_layer(h, wd, bd, sd, pd, ACT_NONE)[0]
        else:
            side = h
        w2, b2, s2, p2 = params[f"body.{i}.c2"]
        h = conv_layer(out, w2, b2, s2, p2, ACT_RELU, side)[0]
    return h


def conv_layer_static(x_nchw, w, b, stride, pad, act, residual_nchw, s_in, s_out):
    """A conv with calibrated scales (nn.ts:6790-6824): the input quantized with ``s_in``
    (clamped), the epilogue as ``conv_layer``, and the output's int8 twin
    ``clip(rint(y / s_out))`` (kernels.ts:2177-2190 with this build's rounding rule).
    Returns ``(y_nchw, twin NHWC int8, acc)``."""
    x_nchw = np.asarray(x_nchw, np.float32)
    O_, C, KH, KW = w.shape
    cpad = (C + 15) // 16 * 16
    xq = np.zeros(x_nchw.shape[:1] + x_nchw.shape[2:] + (cpad,), np.int8)
    xq[..., :C] = Q.quantize_with_scale(x_nchw, np.float32(s_in)).transpose(0, 2, 3, 1)
    qw, sW = Q.quantize_conv_weight(w, cpad)
    acc, OH, OW = Q.conv2d_i8_nhwc(xq, qw, KH, KW, stride, pad)
    res = None
    if residual_nchw is not None:
        res = np.asarray(residual_nchw, np.float32).transpose(0, 2, 3, 1).reshape(-1, O_)
    y = _act(Q.dequant(acc, np.float32(s_in), sW, b, False, res), act)
    twin = Q.quantize_with_scale(y, np.float32(s_out)).reshape(x_nchw.shape[0], OH, OW, O_)
    N = x_nchw.shape[0]
    return y.reshape(N, OH, OW, O_).transpose(0, 3, 1, 2), twin, acc


def resnet18_features_static(params, scales, x):
    """The calibrated ResNet-18 conv stack. ``scales[key] = (s_in, s_out)``. A layer whose
    input is another layer's output uses that producer's twin when the scales agree (which
    the calibration guarantees), i.e. exactly ``quantize_with_scale(y, s_in)``: the twin
    and a fresh static quantization are the same bytes, so the chain is computed from the
    f32 values."""
    def run(key, h, act, res=None):
        w, b, s, p = params[key]
        return conv_layer_static(h, w, b, s, p, act, res, *scales[key])[0]
    h = run("stem", x, ACT_RELU)
    for i in range(8):
        out = run(f"body.{i}.c1", h, ACT_RELU)
        side = run(f"body.{i}.down", h, ACT_NONE) if f"body.{i}.down" in params else h
        h = run(f"body.{i}.c2", out, ACT_RELU, side)
    return h


def se_gate(x_nchw, w1, b1, w2, b2):
    """Squeeze-excite gates [N, C] in float64, then rounded to f32: the mean over H, W, then
    ``silu(w1 · p + b1)`` and ``sigmoid(w2 · z + b2)`` (the CPU runner's "se" node,
    borch-ts/src/cpu/runner.ts:256-268: meanRows, gemmBiasAct swish and sigmoid)."""
    x = np.asarray(x_nchw, np.float64)
    p = x.mean(axis=(2, 3))
    z = p @ np.asarray(w1, np.float64).T + (0.0 if b1 is None else np.asarray(b1, np.float64))
    z = z / (1.0 + np.exp(-z))
    g = z @ np.asarray(w2, np.float64).T + (0.0 if b2 is None else np.asarray(b2, np.float64))
    return (1.0 / (1.0 + np.exp(-g))).astype(np.float32)


def attention_qkv(qkv, heads):
    """Softmax attention of every head in float64 from a packed qkv projection output
    [B, T, 3 * heads * dh] (per token q, k, v side by side, each [heads, dh]) to [B, T, heads *
    dh]: scores = (q @ k^T) / sqrt(dh), softmax exp(s - max) / sum, then @ v
    (borch/_nn.py:2143-2170 scaled_dot_product_attention; its softmax borch-ts/src/kernels.ts:
    2483-2532 softmaxRows)."""
    x = np.asarray(qkv, np.float64)
    B, T, D3 = x.shape
    dh = D3 // (3 * heads)
    q, k, v = (x.reshape(B, T, 3, heads, dh)[:, :, i].transpose(0, 2, 1, 3) for i in range(3))
    s = (q @ k.transpose(0, 1, 3, 2)) / np.sqrt(dh)
    p = np.exp(s - s.max(axis=-1, keepdims=True))
    p /= p.sum(axis=-1, keepdims=True)
    return (p @ v).transpose(0, 2, 1, 3).reshape(B, T, heads * dh)


def avgpool_linear(x_nchw, w, b=None):
    """The configuration's f32 head in float64: the mean over H, W, then the Linear
    (tests/browser/export_resnet18.py:56-59; borch/_nn.py:397-415). Returns (out [N, O], the
    scale sum |pooled| . |w| the f32 error bound is proportional to)."""
    pooled = np.asarray(x_nchw, np.float64).mean(axis=(2, 3))
    wd = np.asarray(w, np.float64)
    out = pooled @ wd.T + (0.0 if b is None else np.asarray(b, np.float64))
    return out, np.abs(pooled) @ np.abs(wd).T
