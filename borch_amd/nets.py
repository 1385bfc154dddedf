"""The model workloads of the task configurations, built on ``borch_amd.nn``.

* ``ResNet18`` — the CIFAR variant of tests/browser/export_resnet18.py:27-60 in the
  reference (3x3 stem, no max-pool, 8 BasicBlocks with the reference's attribute names,
  mean pool, 10-way Linear). ``fuse()`` folds every BN (borch/_nn.py:4916-4955) and wraps
  the convs into the fused modules the reference's ``fuse()`` builds (borch-ts
  test/bench.ts:63-75, nn.ts:6698-6750): stem and conv1 -> ConvReLU2d, conv2 ->
  ConvAddReLU2d with the shortcut as residual, the 1x1 downsample a plain conv.
* ``EfficientNetB0`` — the published B0 (Tan & Le 2019; torchvision's layout): MBConv
  blocks with int8 1x1 expand/project convs and int8 depthwise 3x3/5x5; squeeze-excite and
  the classifier stay f32 (SE uses torch's own layers); SiLU runs in f32 in the epilogue.
  The reference holds no B0 definition (it comes from an npm package not vendored), so
  this one follows the paper.
* ``ViTEncoder`` — ViT-B/16's encoder (Dosovitskiy et al. 2021; torchvision's pre-norm
  layout, LayerNorm eps 1e-6): QKV / proj / MLP Linears are int8 dynamic-quant;
  LayerNorm, softmax attention and GELU stay f32. ``fuse()`` puts the two skip additions
  into the proj / fc2 epilogues.

Weights are random, from a seeded ``torch.Generator`` on the host: Kaiming-normal
(fan_out, ReLU gain) convs, BN running statistics as export_resnet18.py:84-91 (mean
N(0, 0.1²), var U(0.5, 1.5), gamma N(1, 0.1²), beta N(0, 0.1²)).
"""
from __future__ import annotations

import math

import torch
import torch.nn as tnn

from . import int8 as I8
from ._lib import Int8Unavailable, require_device
from . import nn
from .nn import intrinsic as I
from .nn.utils.fusion import fuse_conv_bn_eval


def _hip_f32_ok(t: torch.Tensor, *params) -> bool:
    """Whether the f32 side kernels (attention, the pooled head) take ``t``: float32 on a
    gfx950 device with the library built, and nothing for autograd to record (the raw-pointer
    kernels keep no graph, so a forward that needs gradients stays on torch's ops)."""
    if not (t.is_cuda and t.dtype == torch.float32):
        return False
    if torch.is_grad_enabled() and (t.requires_grad or any(p is not None and p.requires_grad for p in params)):
        return False
    try:
        require_device(t.device)
    except Int8Unavailable:
        return False
    return True


def _bn_stats(bn: tnn.BatchNorm2d, g: torch.Generator) -> None:
    with torch.no_grad():
        c = bn.num_features
        bn.running_mean.copy_(torch.randn(c, generator=g) * 0.1)
        bn.running_var.copy_(torch.rand(c, generator=g) + 0.5)
        bn.weight.copy_(1.0 + torch.randn(c, generator=g) * 0.1)
        bn.bias.copy_(torch.randn(c, generator=g) * 0.1)


def _kaiming(conv, g: torch.Generator) -> None:
    with torch.no_grad():
        o, ci, kh, kw = conv.weight.shape
        conv.weight.copy_(torch.randn(conv.weight.shape, generator=g) * math.sqrt(2.0 / (o * kh * kw)))
        if conv.bias is not None:
            conv.bias.zero_()


def init_weights(model: tnn.Module, seed: int = 0) -> tnn.Module:
    """Seeded random weights for every conv, BN and Linear (host generator)."""
    g = torch.Generator().manual_seed(seed)
    for m in model.modules():
        if isinstance(m, (nn.Conv2d, tnn.Conv2d)):
            _kaiming(m, g)
        elif isinstance(m, tnn.BatchNorm2d):
            _bn_stats(m, g)
        elif isinstance(m, (nn.Linear, tnn.Linear)):
            with torch.no_grad():
                bound = 1.0 / math.sqrt(m.in_features)
                m.weight.copy_((torch.rand(m.weight.shape, generator=g) * 2 - 1) * bound)
                if m.bias is not None:
                    m.bias.copy_((torch.rand(m.bias.shape, generator=g) * 2 - 1) * bound)
        elif isinstance(m, tnn.LayerNorm):
            with torch.no_grad():
                m.weight.copy_(1.0 + torch.randn(m.weight.shape, generator=g) * 0.1)
                m.bias.copy_(torch.randn(m.bias.shape, generator=g) * 0.1)
    return model


# ------------------------------------------------------------------------ ResNet-18

class Block(tnn.Module):
    """BasicBlock with the reference's attribute names (export_resnet18.py:27-43)."""

    def __init__(self, cin, cout, stride):
        super().__init__()
        self.conv1 = nn.Conv2d(cin, cout, 3, stride, 1, bias=False)
        self.bn1 = tnn.BatchNorm2d(cout)
        self.conv2 = nn.Conv2d(cout, cout, 3, 1, 1, bias=False)
        self.bn2 = tnn.BatchNorm2d(cout)
        shrinks = stride != 1 or cin != cout
        self.downConv = nn.Conv2d(cin, cout, 1, stride, 0, bias=False) if shrinks else None
        self.downBn = tnn.BatchNorm2d(cout) if shrinks else None
        self.c1 = self.c2 = self.down = None

    def forward(self, x):
        if self.c1 is not None:
            if self.down is None:
                return self.c2(self.c1(x), x)
            h, side = nn.pair_forward(self.c1, self.down, x)  # one launch for both when int8
            return self.c2(h, side)
        out = torch.relu(self.bn1(self.conv1(x)))
        out = self.bn2(self.conv2(out))
        side = self.downBn(self.downConv(x)) if self.downConv is not None else x
        return torch.relu(out + side)

    def fuse(self):
        if self.c1 is not None:  # already folded: the unfolded layers are gone
            return self
        self.c1 = I.ConvReLU2d(fuse_conv_bn_eval(self.conv1, self.bn1))
        self.c2 = I.ConvAddReLU2d(fuse_conv_bn_eval(self.conv2, self.bn2))
        self.down = fuse_conv_bn_eval(self.downConv, self.downBn) if self.downConv is not None else None
        self.conv1 = self.bn1 = self.conv2 = self.bn2 = self.downConv = self.downBn = None
        return self


class ResNet18(tnn.Module):
    """CIFAR ResNet-18 (export_resnet18.py:46-60)."""

    def __init__(self, classes=10):
        super().__init__()
        self.stem = nn.Conv2d(3, 64, 3, 1, 1, bias=False)
        self.bn = tnn.BatchNorm2d(64)
        self.body = tnn.Sequential(
            Block(64, 64, 1), Block(64, 64, 1), Block(64, 128, 2), Block(128, 128, 1),
            Block(128, 256, 2), Block(256, 256, 1), Block(256, 512, 2), Block(512, 512, 1))
        self.fc = nn.Linear(512, classes)
        self.fc.int8_exempt = True  # the f32 head of the configuration
        self.stem_f = None

    def features(self, x):
        if self.stem_f is not None:
            h = self.stem_f(x)
        else:
            h = torch.relu(self.bn(self.stem(x)))
        return self.body(h)

    def forward(self, x):
        h = self.features(x)
        fc = self.fc
        if (getattr(fc, "int8", None) is None and fc.weight.shape[0] * fc.weight.shape[1] <= 65536
                and _hip_f32_ok(h, fc.weight, fc.bias)):
            return I8.avgpool_linear(h, fc.weight, fc.bias)  # the f32 head in one launch
        return fc(h.mean(dim=(2, 3)))

    def fuse(self):
        self.eval()
        if self.stem_f is not None:  # already folded
            return self
        self.stem_f = I.ConvReLU2d(fuse_conv_bn_eval(self.stem, self.bn))
        self.stem = self.bn = None
        for b in self.body:
            b.fuse()
        return self


# ------------------------------------------------------------------ EfficientNet-B0

# (expand ratio, kernel, stride, in, out, repeats) — Tan & Le 2019, Table 1.
B0_STAGES = [(1, 3, 1, 32, 16, 1), (6, 3, 2, 16, 24, 2), (6, 5, 2, 24, 40, 2), (6, 3, 2, 40, 80, 3),
             (6, 5, 1, 80, 112, 3), (6, 5, 2, 112, 192, 4), (6, 3, 1, 192, 320, 1)]


class MBConv(tnn.Module):
    def __init__(self, cin, cout, k, stride, expand):
        super().__init__()
        mid = cin * expand
        self.has_expand = expand != 1
        self.expand = nn.Conv2d(cin, mid, 1, bias=False) if self.has_expand else None
        self.bn0 = tnn.BatchNorm2d(mid) if self.has_expand else None
        self.dw = nn.Conv2d(mid, mid, k, stride, k // 2, groups=mid, bias=False)
        self.bn1 = tnn.BatchNorm2d(mid)
        sq = max(1, cin // 4)
        self.se_reduce = tnn.Conv2d(mid, sq, 1)  # squeeze-excite stays f32 (torch's layer)
        self.se_expand = tnn.Conv2d(sq, mid, 1)
        self.project = nn.Conv2d(mid, cout, 1, bias=False)
        self.bn2 = tnn.BatchNorm2d(cout)
        self.residual = stride == 1 and cin == cout
        self.fused = False

    def _se_gate(self, h):
        """Squeeze-excite gates [N, C] in f32. With the block on the int8 path: one fused
        kernel pair (bq_se_gate_nhwc: mean, the two 1x1 layers with SiLU and sigmoid). In
        f32: torch ops, the 1x1 convs on the pooled 1x1 map as the equal matrix products."""
        conv = getattr(self.dw, "conv", self.dw)
        if getattr(conv, "int8", None) is not None:
            w2 = self.se_expand.weight
            if getattr(self, "_se_w2t", None) is None or self._se_w2t[1] != w2._version:
                self._se_w2t = (w2.detach().flatten(1).t().contiguous(), w2._version)  # made once, before capture
            return I8.se_gate_nhwc(h, self.se_reduce.weight.flatten(1), self.se_reduce.bias,
                                   w2.flatten(1), self.se_expand.bias, self._se_w2t[0])
        s = h.mean(dim=(2, 3))
        s = torch.nn.functional.silu(torch.nn.functional.linear(s, self.se_reduce.weight.flatten(1),
                                                               self.se_reduce.bias))
        return torch.sigmoid(torch.nn.functional.linear(s, self.se_expand.weight.flatten(1), self.se_expand.bias))

    def _se(self, h):
        return h * self._se_gate(h)[:, :, None, None]

    # With calibrated scales the depthwise conv reads the expand conv's int8 twin, so the
    # expand conv writes that twin alone (no f32 output: 866 MB a B0 b64 forward).
    twin_path = True

    def forward(self, x):
        if self.fused:
            # the gate multiplies the projection's input inside its int8 quantization
            # (f32: a plain product): the gated tensor is never stored
            ex = self.expand.conv if self.expand is not None else None
            dw = self.dw.conv
            if self.twin_path and ex is not None and ex.twin_only() and dw.takes_twin_of(ex):
                h = dw.forward_int8(*ex.twin_forward(x))
            elif self.twin_path and ex is not None and ex.dynamic_twin_of(dw, x):
                # dynamic scales: the expand conv's output quantized for the depthwise conv
                # without its f32 output (where the kernel takes the layer)
                r = ex.dynamic_twin_forward(x)
                h = dw.forward_int8(*r) if isinstance(r, tuple) else self.dw(r)
            else:
                h = self.expand(x) if self.expand is not None else x
                h = self.dw(h)
            g = self._se_gate(h)
            return self.project(h, x, channel_scale=g) if self.residual else self.project(h, channel_scale=g)
        h = torch.nn.functional.silu(self.bn0(self.expand(x))) if self.has_expand else x
        h = torch.nn.functional.silu(self.bn1(self.dw(h)))
        h = self.bn2(self.project(self._se(h)))
        return h + x if self.residual else h

    def fuse(self):
        if self.fused:  # already folded: the BNs are gone
            return self
        if self.has_expand:
            self.expand = I.ConvSiLU2d(fuse_conv_bn_eval(self.expand, self.bn0))
        self.dw = I.ConvSiLU2d(fuse_conv_bn_eval(self.dw, self.bn1))
        p = fuse_conv_bn_eval(self.project, self.bn2)
        self.project = I.ConvAdd2d(p) if self.residual else p
        self.bn0 = self.bn1 = self.bn2 = None
        self.fused = True
        return self


class EfficientNetB0(tnn.Module):
    def __init__(self, classes=1000):
        super().__init__()
        self.stem = nn.Conv2d(3, 32, 3, 2, 1, bias=False)
        self.bn = tnn.BatchNorm2d(32)
        blocks = []
        for e, k, s, cin, cout, n in B0_STAGES:
            for i in range(n):
                blocks.append(MBConv(cin if i == 0 else cout, cout, k, s if i == 0 else 1, e))
        self.blocks = tnn.Sequential(*blocks)
        self.head = nn.Conv2d(320, 1280, 1, bias=False)
        self.bn_head = tnn.BatchNorm2d(1280)
        self.fc = nn.Linear(1280, classes)
        self.fc.int8_exempt = True
        self.fused = False

    def forward(self, x):
        if self.fused:
            h = self.head(self.blocks(self.stem(x)))
        else:
            h = torch.nn.functional.silu(self.bn(self.stem(x)))
            h = torch.nn.functional.silu(self.bn_head(self.head(self.blocks(h))))
        return self.fc(h.mean(dim=(2, 3)))

    def fuse(self):
        self.eval()
        if self.fused:  # already folded
            return self
        self.stem = I.ConvSiLU2d(fuse_conv_bn_eval(self.stem, self.bn))
        self.head = I.ConvSiLU2d(fuse_conv_bn_eval(self.head, self.bn_head))
        self.bn = self.bn_head = None
        for b in self.blocks:
            b.fuse()
        self.fused = True
        return self


# ---------------------------------------------------------------- ViT-B/16 encoder

class EncoderLayer(tnn.Module):
    def __init__(self, d=768, heads=12, mlp=3072):
        super().__init__()
        self.heads = heads
        self.ln1 = tnn.LayerNorm(d, eps=1e-6)
        self.qkv = nn.Linear(d, 3 * d)
        self.proj = nn.Linear(d, d)
        self.ln2 = tnn.LayerNorm(d, eps=1e-6)
        self.fc1 = nn.Linear(d, mlp)
        self.fc2 = nn.Linear(mlp, d)
        self.proj_f = self.fc2_f = None

    def heads_out(self, h):
        """Multi-head softmax attention in f32 up to (not including) the output projection."""
        return self.attend(self.qkv(h))

    def attend(self, qkv):
        """The attention core on the qkv projection's output [B, T, 3 D], f32. On a gfx950
        device with heads of 64 and at most 256 tokens: ``I8.attention_f32`` (one HIP kernel,
        f32 MFMAs; q, k, v read in place and the heads written side by side). Otherwise torch's
        fused scaled-dot-product attention on strided views of the projection output."""
        B, T, D3 = qkv.shape
        D = D3 // 3
        H, dh = self.heads, D // self.heads
        if dh == 64 and T <= 256 and _hip_f32_ok(qkv):
            return I8.attention_f32(qkv, H)
        qkv = qkv.reshape(B, T, 3, H, dh).permute(2, 0, 3, 1, 4)
        o = torch.nn.functional.scaled_dot_product_attention(qkv[0], qkv[1], qkv[2])
        return o.transpose(1, 2).reshape(B, T, D)

    def attention(self, h):
        return self.proj(self.heads_out(h))

    def forward(self, x):
        if self.proj_f is not None:
            # fused: the skip additions ride in the projections' epilogues; on the W8A8 path
            # each LayerNorm runs inside the next Linear's input quantizer
            x = self.proj_f(self.attend(self.qkv(x, pre_norm=self.ln1)), x)
            return self.fc2_f(self.fc1(x, pre_norm=self.ln2), x, pre_act=I8.ACT_GELU)
        x = x + self.attention(self.ln1(x))
        return x + self.fc2(torch.nn.functional.gelu(self.fc1(self.ln2(x))))

    def fuse(self):
        """proj and fc2 -> LinearAdd (x + W·o in the epilogue): the same f32 arithmetic as
        forward's separate add (addition commutes exactly); ln1 / ln2 run in the qkv / fc1
        input quantizers (``Linear(x, pre_norm=ln)``) and the GELU in fc2's
        (``pre_act``): fc1 writes its f32 output once and fc2 reads it once. (The GELU in
        fc1's epilogue instead cost the GEMM what the separate pass cost: measured.)"""
        if self.proj_f is None:
            self.proj_f = I.LinearAdd(self.proj)
            self.fc2_f = I.LinearAdd(self.fc2)
        return self


class ViTEncoder(tnn.Module):
    """ViT-B/16 encoder on already patch-embedded tokens [B, 197, 768]."""

    def __init__(self, layers=12, d=768, heads=12, mlp=3072):
        super().__init__()
        self.layers = tnn.Sequential(*[EncoderLayer(d, heads, mlp) for _ in range(layers)])
        self.ln = tnn.LayerNorm(d, eps=1e-6)

    def forward(self, x):
        return self.ln(self.layers(x))

    def fuse(self):
        self.eval()
        for layer in self.layers:
            layer.fuse()
        return self


def build(name: str, seed: int = 0, device="cuda"):
    """A seeded model of configuration C3 / C4 / C5, folded for inference (not yet int8)."""
    if name == "resnet18":
        m = init_weights(ResNet18(), seed)
    elif name == "efficientnet_b0":
        m = init_weights(EfficientNetB0(), seed)
    elif name == "vit_b16":
        m = init_weights(ViTEncoder(), seed)
    else:
        raise ValueError(f"unknown model {name!r}")
    m = m.to(device).eval()
    if hasattr(m, "fuse"):
        m.fuse()
    return m
