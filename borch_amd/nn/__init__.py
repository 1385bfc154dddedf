"""``borch_amd.nn`` — the operator surface of the int8 path, shaped like the numpy core's.

``Linear`` and ``Conv2d`` keep the numpy core's constructor and forward signatures
(borch/_nn.py:397-415, 1156-1190) over PyTorch-ROCm parameters. Each can be quantized
once for the int8 path (``quantize_int8()``, the prepare of borch-ts/src/nn.ts:967-980);
after that its forward runs the HIP kernels (W8A8 GEMM / implicit-GEMM conv / depthwise)
and otherwise the float32 op. The model-level calls mirror borch-ts/src/nn.ts:6770-6829:

* ``quantize_for_int8(model) -> int`` — quantizes every layer the kernels take and
  returns the count; refuses by name on a device without the int8 kernels;
* ``calibrate_int8(model, batches) -> int`` — static scales and the int8 output twin;
* ``clear_int8(model)`` — back to float32 (the f32 weights never left);
* ``int8_report(model)`` — which layers took the path and why the others did not.

Every other ``torch.nn`` name (``ReLU``, ``Sequential``, ``BatchNorm2d``, ...) is torch's
own, re-exported unchanged: only the int8 path is this package's.
"""
from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn as _tnn

from .. import int8 as _i8
from .._lib import Int8Unavailable, require_device
from . import functional  # noqa: F401
from . import intrinsic  # noqa: F401
from . import utils  # noqa: F401

Module = _tnn.Module
Parameter = _tnn.Parameter

# Set by calibrate_int8: int8 convs run their f32 path and record max|input| / max|output|
# (the reference's setInt8Calibrating, tensor.ts:11896-11901).
_CALIBRATING = False
_PAIRING = False  # set by `pairing` (compiled forwards): see pair_forward


def _scale_value(peak: float) -> float:
    """float32(peak / 127), correctly rounded: the same value the device computes."""
    return float(np.float32(peak) / np.float32(127.0))


def _pair(v):
    if isinstance(v, (tuple, list)):
        if len(v) != 2:
            raise ValueError(f"expected a pair, got {v!r}")
        return int(v[0]), int(v[1])
    return int(v), int(v)


class Linear(_tnn.Module):
    """``nn.Linear(in_features, out_features, bias=True)``; forward ``x @ W.T + b``
    (borch/_nn.py:397-415). Init U(−1/√in, 1/√in) for weight and bias, as the core's."""

    def __init__(self, in_features, out_features, bias=True, device=None, dtype=None):
        super().__init__()
        self.in_features = int(in_features)
        self.out_features = int(out_features)
        bound = 1.0 / math.sqrt(in_features) if in_features else 0.0
        self.weight = Parameter(torch.empty((out_features, in_features), device=device,
                                            dtype=dtype or torch.float32).uniform_(-bound, bound))
        self.bias = (Parameter(torch.empty((out_features,), device=device, dtype=dtype or torch.float32)
                               .uniform_(-bound, bound)) if bias else None)
        self.int8 = None  # Int8Weight once quantize_int8() has run
        self.act = _i8.ACT_NONE  # fused epilogue activation (LinearReLU sets RELU)

    def quantize_int8(self, weight_only: bool = False, per_tensor: bool = False) -> bool:
        """Packs the weight once per output channel (quant.ts:23-53). Any shape is taken
        (K is zero-padded to a multiple of 16). ``weight_only`` keeps activations f32
        (W8A32, the reference's int8 window weight, tensor.ts:1681-1705); ``per_tensor``
        quantizes the activations with one scale for the whole input, as the reference's
        ``matmulInt8(scaled)`` takes them (kernels.ts:1818-1827), instead of one per row.
        Returns True."""
        require_device(self.weight.device)
        with torch.no_grad():
            self.int8 = _i8.pack_linear_weight(self.weight.detach(), weight_only, per_tensor)
        return True

    def forward(self, x, residual=None, pre_norm=None, pre_act=None):
        """``x @ W.T + b``; the fused modules (``LinearReLU``, ``LinearGELU``, ``LinearAdd``)
        add ``residual`` and apply the activation in the same epilogue. ``pre_norm`` (a
        LayerNorm) or ``pre_act`` (an activation id, e.g. GELU) is applied to ``x`` first; on
        the W8A8 path it runs inside the input quantizer, so the normalised or activated
        input is never stored."""
        if pre_norm is not None:
            if self.int8 is not None and _i8.fusable_layernorm(pre_norm, x, self.int8):
                return _i8.layernorm_linear(x, pre_norm, self.int8, self.bias, self.act, residual)
            x = pre_norm(x)
        if pre_act is not None and pre_act != _i8.ACT_NONE:
            if self.int8 is not None:
                return _i8.linear(x, self.int8, self.bias, self.act, residual, pre_act=pre_act)
            x = _i8._act_f32(x, pre_act)
        if self.int8 is not None:
            return _i8.linear(x, self.int8, self.bias, self.act, residual)
        out = functional._f32_linear(x, self.weight, self.bias)
        if residual is not None:
            out = out + residual
        return _i8._act_f32(out, self.act)

    def extra_repr(self):
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"bias={self.bias is not None}" + (", int8" if self.int8 is not None else ""))


class Conv2d(_tnn.Module):
    """``nn.Conv2d(in, out, kernel_size, stride=1, padding=0, dilation=1, groups=1,
    bias=True, padding_mode='zeros')`` (borch/_nn.py:1156-1190)."""

    def __init__(self, in_channels, out_channels, kernel_size, stride=1, padding=0, dilation=1,
                 groups=1, bias=True, padding_mode="zeros", device=None, dtype=None):
        super().__init__()
        if padding_mode not in ("zeros", "reflect", "replicate", "circular"):
            raise ValueError("padding_mode has to be one of ('zeros', 'reflect', 'replicate', 'circular'), "
                             f"got {padding_mode!r}")
        if in_channels % groups or out_channels % groups:
            raise ValueError("in_channels and out_channels must be divisible by groups")
        self.in_channels, self.out_channels = int(in_channels), int(out_channels)
        self.kernel_size, self.stride, self.padding = kernel_size, stride, padding
        self.dilation, self.groups, self.padding_mode = dilation, int(groups), padding_mode
        kh, kw = _pair(kernel_size)
        fan_in = (in_channels // groups) * kh * kw
        bound = 1.0 / math.sqrt(fan_in) if fan_in else 0.0
        dt = dtype or torch.float32
        self.weight = Parameter(torch.empty((out_channels, in_channels // groups, kh, kw), device=device,
                                            dtype=dt).uniform_(-bound, bound))
        self.bias = Parameter(torch.empty((out_channels,), device=device, dtype=dt)
                              .uniform_(-bound, bound)) if bias else None
        self.int8 = None  # Int8ConvWeight / Int8DwWeight once quantize_int8() has run
        self.act = _i8.ACT_NONE
        # calibrated static scales (calibrate_int8): device [1] tensors and their values
        self.in_scale = self.out_scale = None
        self.in_scale_v = self.out_scale_v = None
        self._calib = None

    def _geometry(self):
        """(stride, pad) when square and zero-padded, else None."""
        sh, sw = _pair(self.stride)
        if isinstance(self.padding, str):
            if self.padding == "valid":
                ph = pw = 0
            else:
                return None
        else:
            ph, pw = _pair(self.padding)
        if sh != sw or ph != pw or self.padding_mode != "zeros" or _pair(self.dilation) != (1, 1):
            return None
        return sh, ph

    def int8_refusal(self):
        """Why the int8 kernels do not take this layer (None if they do)."""
        if self._geometry() is None:
            return "stride/padding not square, dilation != 1 or non-zero padding mode"
        if self.groups == 1:
            return None
        if self.groups == self.in_channels == self.out_channels:
            return None
        return f"groups={self.groups} (only 1 or depthwise)"

    def reference_rule_refusal(self):
        """Why the reference's int8 conv would not take this layer (None if it would): the
        shape rules of its ``convInt8Fits`` (borch-ts/src/kernels.ts:2096-2103) — 2-D,
        groups 1, dilation 1, stride 1, kernel at most 3, input channels in 32s, output
        channels in 16s. Its band and workgroup-storage limits (WebGPU tiling constraints
        with no counterpart on this device) are not applied."""
        refusal = self.int8_refusal()
        if refusal is not None:
            return refusal
        stride, _ = self._geometry()
        kh, kw = _pair(self.kernel_size)
        if self.groups != 1:
            return f"groups={self.groups}"
        if stride != 1:
            return f"stride {stride}"
        if kh > 3 or kw > 3:
            return f"kernel {kh}x{kw} > 3"
        if self.in_channels % 32:
            return f"in_channels={self.in_channels} not a multiple of 32"
        if self.out_channels % 16:
            return f"out_channels={self.out_channels} not a multiple of 16"
        return None

    def quantize_int8(self, rule: str = "all") -> bool:
        """Packs the weight once per output channel (quant.ts:80-103's scale rule) where
        the kernels take the layer; returns False (the layer stays f32) otherwise, as
        borch-ts/src/nn.ts:967-980 does. ``rule="reference"`` takes only the layers the
        reference's conv kernel takes (``reference_rule_refusal``), for comparison."""
        if rule not in ("all", "reference"):
            raise ValueError(f"rule must be 'all' or 'reference', not {rule!r}")
        refusal = self.reference_rule_refusal() if rule == "reference" else self.int8_refusal()
        self.int8_why = refusal  # why the last quantize_int8 left this layer f32 (int8_report)
        if refusal is not None:
            return False
        require_device(self.weight.device)
        with torch.no_grad():
            w = self.weight.detach()
            self.int8 = _i8.pack_conv_weight(w) if self.groups == 1 else _i8.pack_dw_weight(w)
        if self.groups == 1:
            _i8.split_workspace(self.weight.device)  # made now, before any graph capture
        return True

    def _int8_input(self, x, channel_scale=None):
        """(q NHWC int8, scale [1]) for the int8 kernels, cheapest first, as
        tensor.ts:11909-11921: the producer's int8 twin when its scale is this layer's
        calibrated input scale and ``x`` is unchanged since; else one pass with the static
        scale; else the dynamic per-tensor quantization. With ``channel_scale`` [N, C] the
        layer's input is ``x * channel_scale`` (a squeeze-excite gate), quantized without
        storing the product."""
        cpad = self.int8.cpad
        if channel_scale is not None:
            return _i8.quantize_nhwc_chscale(x, channel_scale, cpad, self.in_scale)
        if self.in_scale is not None:
            twin = getattr(x, "_int8_twin", None)
            if (twin is not None and twin[2] == self.in_scale_v and twin[3] == x._version
                    and twin[0].shape[-1] == cpad):
                return twin[0], twin[1]
            return _i8.quantize_nhwc_scaled(x, self.in_scale, cpad), self.in_scale
        return _i8.quantize_nhwc(x, cpad)

    def _fused_input_forward(self, x, residual, twin_only=False):
        """A network's NCHW f32 image into a conv over 16 padded channels (the stem) with its
        quantization fused into the conv (conv2d_nchw_fq): ``forward`` / ``twin_forward``'s
        result, or None where that path does not take the layer (the caller quantizes first)."""
        wq = self.int8
        if not (isinstance(wq, _i8.Int8ConvWeight) and wq.cpad == 16 and _i8._nchw_padded(x, 16)
                and x.dtype == torch.float32 and getattr(x, "_bq_absmax", None) is None):
            return None
        stride, pad = self._geometry()
        twin = self.out_scale is not None and wq.O % 16 == 0
        try:
            r = _i8.conv2d_nchw_fq(x, wq, stride, pad, self.bias, residual, self.act, s_x=self.in_scale,
                                   s_out=self.out_scale if twin else None, f32_out=not twin_only)
        except NotImplementedError:
            return None
        if twin_only:
            return r[1], self.out_scale
        if twin:
            out, q = r
            out._int8_twin = (q, self.out_scale, self.out_scale_v, out._version)
            return out
        return r

    def _f32_forward(self, x, residual):
        out = functional._f32_conv2d(x, self.weight, self.bias, self.stride, self.padding, self.dilation,
                                     self.groups, self.padding_mode)
        if residual is not None:
            out = out + residual
        return _i8._act_f32(out, self.act)

    def forward(self, x, residual=None, channel_scale=None):
        """``conv(x) (+ residual)`` then the activation. ``channel_scale`` [N, C] (optional)
        multiplies the input per image and channel first (a squeeze-excite gate); the int8
        path folds it into the input's quantization."""
        if channel_scale is not None and (self.int8 is None or _CALIBRATING):
            x = x * channel_scale[:, :, None, None]
            channel_scale = None
        if self.int8 is not None and _CALIBRATING:
            out = self._f32_forward(x, residual)
            cin, cout = x.detach().abs().amax(), out.detach().abs().amax()
            self._calib = [cin, cout] if self._calib is None else [torch.maximum(self._calib[0], cin),
                                                                   torch.maximum(self._calib[1], cout)]
            return out
        if self.int8 is not None:
            if x.dim() != 4 or x.shape[1] != self.in_channels:
                raise RuntimeError(f"channels do not match: input {x.shape[1] if x.dim() > 1 else x.shape}, "
                                   f"filter {self.in_channels}")
            if channel_scale is None:
                out = self._fused_input_forward(x, residual)
                if out is not None:
                    return out
            qx, sa = self._int8_input(x, channel_scale)
            return self.forward_int8(qx, sa, residual)
        out = functional._f32_conv2d(x, self.weight, self.bias, self.stride, self.padding, self.dilation,
                                     self.groups, self.padding_mode)
        if residual is not None:
            out = out + residual
        return _i8._act_f32(out, self.act)

    def twin_only(self) -> bool:
        """Whether ``twin_forward`` applies: int8, calibrated output scale, O % 16 == 0."""
        return (self.int8 is not None and not _CALIBRATING and self.out_scale is not None
                and isinstance(self.int8, _i8.Int8ConvWeight) and self.int8.O % 16 == 0)

    def takes_twin_of(self, producer) -> bool:
        """Whether this layer reads ``producer``'s int8 twin as its input as it stands
        (int8, its calibrated input scale is the producer's output scale, same channels)."""
        return (self.int8 is not None and not _CALIBRATING and self.in_scale is not None
                and producer.out_scale is not None and self.in_scale_v == producer.out_scale_v
                and self.int8.cpad == producer.out_channels)

    def twin_forward(self, x, residual=None):
        """``self(x, residual)`` as its int8 twin alone, ``(q [N, OH, OW, O], out_scale)``, the
        f32 output never written: for a consumer that reads only the twin (``forward_int8``
        of a layer that ``takes_twin_of`` this one). Requires ``twin_only()``."""
        if not self.twin_only():
            raise RuntimeError("twin_forward needs an int8 layer with a calibrated output scale and O % 16 == 0")
        if x.dim() != 4 or x.shape[1] != self.in_channels:
            raise RuntimeError(f"channels do not match: input {x.shape[1] if x.dim() > 1 else x.shape}, "
                               f"filter {self.in_channels}")
        r = self._fused_input_forward(x, residual, twin_only=True)
        if r is not None:
            return r
        qx, sa = self._int8_input(x)
        stride, pad = self._geometry()
        _, q = _i8.conv2d_i8_nhwc_q(qx, sa, self.int8, self.out_scale, stride, pad, self.bias, residual, self.act,
                                    f32_out=False)
        return q, self.out_scale

    def dynamic_twin_of(self, consumer, x) -> bool:
        """Whether ``dynamic_twin_forward(x)`` feeds ``consumer`` through the dynamic twin: both
        int8 layers with dynamic per-tensor scales (not calibrated), this one a packed conv
        whose output channels are the consumer's padded input channels, and the kernel takes
        it at ``x``'s shape (conv2d_i8_nhwc_dq_ok). Where it does not, the caller runs the
        two layers as their own module calls."""
        if not (self.int8 is not None and not _CALIBRATING and isinstance(self.int8, _i8.Int8ConvWeight)
                and self.out_scale is None and self.int8.O % 16 == 0 and consumer.int8 is not None
                and consumer.in_scale is None and consumer.int8.cpad == self.int8.O
                and x.dim() == 4 and x.shape[1] == self.in_channels and x.is_cuda):
            return False
        g = self._geometry()
        return g is not None and _i8.conv2d_i8_nhwc_dq_ok(x.shape[0], x.shape[2], x.shape[3], self.int8, *g)

    def dynamic_twin_forward(self, x, residual=None):
        """For a consumer that reads only the int8 of this layer's output (``dynamic_twin_of``):
        ``(q [N, OH, OW, O], s [1])``, the output quantized at its dynamic per-tensor scale with
        the f32 output never stored (conv2d_i8_nhwc_dq), the bytes the consumer's own
        quantization of ``self(x, residual)`` gives. Where that kernel does not take the layer
        after all: ``self(x, residual)`` itself, for the consumer to quantize."""
        if x.dim() != 4 or x.shape[1] != self.in_channels:
            raise RuntimeError(f"channels do not match: input {x.shape[1] if x.dim() > 1 else x.shape}, "
                               f"filter {self.in_channels}")
        qx, sa = self._int8_input(x)
        stride, pad = self._geometry()
        try:
            return _i8.conv2d_i8_nhwc_dq(qx, sa, self.int8, stride, pad, self.bias, residual, self.act)
        except NotImplementedError:
            return self.forward_int8(qx, sa, residual)

    def forward_int8(self, qx, sa, residual=None):
        """The int8 layer on an already quantized NHWC input ``qx [N, H, W, cpad]`` with its
        per-tensor scale ``sa [1]``: the conv (or depthwise) kernel and its epilogue."""
        stride, pad = self._geometry()
        if isinstance(self.int8, _i8.Int8DwWeight):
            out = _i8.dwconv_i8_nhwc(qx, sa, self.int8, stride, pad, self.bias,
                                     self.act if residual is None else _i8.ACT_NONE)
            if self.int8.cpad != self.int8.C:
                out = out[:, : self.int8.C]
            if residual is not None:
                out = out + residual
                if self.act == _i8.ACT_RELU:
                    out = torch.relu(out)
            return out
        if self.out_scale is not None and self.int8.O % 16 == 0:
            out, q = _i8.conv2d_i8_nhwc_q(qx, sa, self.int8, self.out_scale, stride, pad, self.bias, residual,
                                          self.act)
            out._int8_twin = (q, self.out_scale, self.out_scale_v, out._version)
            return out
        return _i8.conv2d_i8_nhwc(qx, sa, self.int8, stride, pad, self.bias, residual, self.act)

    def extra_repr(self):
        s = (f"{self.in_channels}, {self.out_channels}, kernel_size={self.kernel_size}, "
             f"stride={self.stride}, padding={self.padding}")
        if self.groups != 1:
            s += f", groups={self.groups}"
        return s + (", int8" if self.int8 is not None else "")


class pairing:
    """Within this context ``pair_forward`` runs two int8 convs of one input in one launch
    (``compiled`` runs its model inside it). Outside it, each conv runs through its own module
    call, so forward hooks see every layer (the per-layer checks and the tuner use them)."""

    def __enter__(self):
        global _PAIRING
        self._prev, _PAIRING = _PAIRING, True
        return self

    def __exit__(self, *exc):
        global _PAIRING
        _PAIRING = self._prev
        return False


def pair_forward(first_mod, second_mod, x):
    """``(first_mod(x), second_mod(x))`` with no residual: a residual block's first conv and
    its downsampling shortcut, which read the same input (each a ``Conv2d`` or a fused module
    wrapping one, such as ``ConvReLU2d``). Inside ``pairing``, when both are int8 convs (not
    depthwise, neither a 1x1 stride-1 unpadded conv) on the same input scale, the input is
    quantized once and both run in one launch (``conv2d_pair_i8_nhwc``), with the results the
    two calls give. The first output keeps what its own call leaves for its consumer (the int8
    twin, or the per-tile maxima); the shortcut's f32 output is written alone, and a consumer
    quantizing it gets the bytes its twin would have held. Otherwise the two modules are
    called, so hooks on them (and on the convs they wrap) see both layers."""
    first = getattr(first_mod, "conv", first_mod)
    second = getattr(second_mod, "conv", second_mod)
    ok = (_PAIRING and not _CALIBRATING and x.dim() == 4 and isinstance(first, Conv2d) and isinstance(second, Conv2d)
          and isinstance(first.int8, _i8.Int8ConvWeight) and isinstance(second.int8, _i8.Int8ConvWeight)
          and x.shape[1] == first.in_channels == second.in_channels and first.int8.cpad == second.int8.cpad
          and first.in_scale_v == second.in_scale_v
          and not _dense_1x1(first) and not _dense_1x1(second))
    if not ok:
        return first_mod(x), second_mod(x)
    qx, sa = first._int8_input(x)
    s1, p1 = first._geometry()
    s2, p2 = second._geometry()
    twin = first.out_scale is not None and first.int8.O % 16 == 0
    (h, q), (side, _) = _i8.conv2d_pair_i8_nhwc(
        qx, sa,
        _i8.PairConv(first.int8, s1, p1, first.bias, first.act, first.out_scale if twin else None, amax=not twin),
        _i8.PairConv(second.int8, s2, p2, second.bias, second.act))
    if twin:
        h._int8_twin = (q, first.out_scale, first.out_scale_v, h._version)
    return h, side


def _dense_1x1(m: Conv2d) -> bool:
    """A 1x1 stride-1 unpadded conv (the dense GEMM loader, which a pair does not take)."""
    return m.int8.KH == 1 and m.int8.KW == 1 and m._geometry() == (1, 0)


def _int8_layers(model):
    """Every Linear / Conv2d of this package in ``model`` that is not marked
    ``int8_exempt`` (a layer the configuration keeps in f32, e.g. a classifier head)."""
    for name, mod in model.named_modules():
        if isinstance(mod, (Linear, Conv2d)) and not getattr(mod, "int8_exempt", False):
            yield name, mod


def quantize_for_int8(model, linear: bool = True, conv: bool = True, weight_only: bool = False,
                      rule: str = "all", per_tensor: bool = False) -> int:
    """Every Linear / Conv2d of ``model`` the int8 kernels take, quantized once; returns
    how many took it (borch-ts/src/nn.ts:6770-6780). Refused by name where the device has
    no int8 kernels (nn.ts:6771-6773): the path is an accuracy trade a caller asks for and
    must not silently become the f32 forward. ``rule="reference"`` restricts convs to the
    shapes the reference's int8 conv takes (13 of CIFAR ResNet-18's 20), for comparison
    with its published numbers; the default takes every conv this library can.
    ``per_tensor`` gives W8A8 Linears one activation scale per call (the reference's
    matmulInt8) instead of one per row."""
    if rule not in ("all", "reference"):
        raise ValueError(f"rule must be 'all' or 'reference', not {rule!r}")
    layers = list(_int8_layers(model))
    dev = next((m.weight.device for _, m in layers), None)
    if dev is not None:
        try:
            require_device(dev)
        except Int8Unavailable as e:
            raise Int8Unavailable(f"int8: this device has no int8 kernels ({e}) — "
                                  "the int8 forward is not available here") from None
    taken = 0
    for _, mod in layers:
        if isinstance(mod, Linear) and linear:
            taken += bool(mod.quantize_int8(weight_only, per_tensor))
        elif isinstance(mod, Conv2d) and conv:
            taken += bool(mod.quantize_int8(rule))
    return taken


def calibrate_int8(model, batches) -> int:
    """Static scales (borch-ts/src/nn.ts:6790-6824): every int8 conv runs f32 over the
    calibration ``batches`` while ``max|input|`` and ``max|output|`` accumulate on the
    device (no readback until the end); each layer then keeps both as scales. Its input is
    then quantized in one pass with the first, and its output is packed at its own store
    with the second (the int8 twin the next conv takes with no pass at all). Returns how
    many layers were calibrated. After ``quantize_for_int8``; ``clear_int8`` undoes both."""
    global _CALIBRATING
    layers = [m for _, m in _int8_layers(model) if isinstance(m, Conv2d) and m.int8 is not None]
    for m in layers:
        m._calib = None
    _CALIBRATING = True
    try:
        with torch.no_grad():
            for xb in batches:
                model(xb)
    finally:
        _CALIBRATING = False
    for m in layers:
        if m._calib is None:  # never reached by the calibration inputs
            continue
        in_max, out_max = (float(t) for t in m._calib)
        dev = m.weight.device
        m.in_scale_v, m.out_scale_v = _scale_value(in_max), _scale_value(out_max)
        m.in_scale = torch.tensor([m.in_scale_v], dtype=torch.float32, device=dev)
        m.out_scale = torch.tensor([m.out_scale_v], dtype=torch.float32, device=dev)
        m._calib = None
    return len(layers)


def clear_int8(model) -> None:
    """Back to f32: every layer's int8 weight and calibrated scales dropped (nn.ts:6827-6829)."""
    for _, mod in _int8_layers(model):
        mod.int8 = None
        if isinstance(mod, Conv2d):
            mod.in_scale = mod.out_scale = None
            mod.in_scale_v = mod.out_scale_v = None


def int8_report(model):
    """``[(name, kind, took_int8, reason)]`` for every Linear / Conv2d."""
    rows = []
    for name, mod in _int8_layers(model):
        kind = type(mod).__name__
        why = None if isinstance(mod, Linear) else (getattr(mod, "int8_why", None) or mod.int8_refusal())
        rows.append((name, kind, mod.int8 is not None, why))
    return rows


def __getattr__(name):
    return getattr(_tnn, name)
