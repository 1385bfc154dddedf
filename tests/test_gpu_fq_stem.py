"""GPU parity of the stem conv with its input quantization fused (bq_conv2d_i8_nchw_fq).

The fused call reads a network's f32 NCHW image of at most 8 channels, quantizes it per
tensor (a calibrated scale, or the dynamic scale from partial maxima computed first) and
convolves it over 16 padded channels in the small-K kernel. It must give, bit for bit,
what the two-pass form gives (``quantize_nhwc`` / ``quantize_nhwc_scaled`` into 16
channels, then ``conv2d_i8_nhwc`` / ``conv2d_i8_nhwc_q``): the f32 output, the int32
accumulators, the scale, the output's largest partial maximum and the int8 twin (with and
without the f32 output); on the small cases the accumulators and the scale are also held
to the CPU oracle.
"""
import sys

import numpy as np
import pytest
import torch

from borch_amd import int8 as I
from oracle import quant as O

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def n(x):
    return x.detach().cpu().numpy()


# (N, C, H, W, O, k, stride, pad): EfficientNet-B0 b64's stem and CIFAR ResNet-18 b16's first,
# then one, four and eight input channels (the 4- and 8-channel kernels), ragged images,
# 1x1 / 2x2 / 4x4 filters, strides above the filter, O % 16 != 0
CASES = [(64, 3, 224, 224, 32, 3, 2, 1), (16, 3, 32, 32, 64, 3, 1, 1), (2, 3, 40, 37, 32, 3, 2, 1),
         (3, 1, 17, 13, 20, 3, 1, 1), (2, 8, 15, 15, 64, 2, 2, 0), (1, 5, 23, 19, 48, 4, 1, 2),
         (2, 4, 12, 12, 8, 2, 3, 1), (2, 7, 11, 11, 4, 4, 4, 0), (4, 3, 9, 9, 12, 1, 2, 0)]


@pytest.mark.parametrize("Nimg,C,H,W,O_,k,stride,pad", CASES)
@pytest.mark.parametrize("static", [False, True])
def test_equals_the_two_pass_form(dev, Nimg, C, H, W, O_, k, stride, pad, static):
    say(f"fused stem N={Nimg} C={C} H={H} W={W} O={O_} k={k} s={stride} p={pad} static={static}")
    rng = np.random.default_rng(Nimg + C + H + W + O_ + k + stride + pad)
    xf = (rng.normal(size=(Nimg, C, H, W)) * 1.7).astype(np.float32)
    x = t(xf, dev)
    wq = I.pack_conv_weight(t((rng.normal(size=(O_, C, k, k)) * 0.1).astype(np.float32), dev))
    assert wq.cpad == 16
    b = t(rng.normal(size=O_).astype(np.float32), dev)
    OH, OW = (H + 2 * pad - k) // stride + 1, (W + 2 * pad - k) // stride + 1
    r = t(rng.normal(size=(Nimg, O_, OH, OW)).astype(np.float32), dev).contiguous(memory_format=torch.channels_last)
    s_in = t(np.array([0.021], np.float32), dev) if static else None
    s_out = t(np.array([0.05], np.float32), dev)
    if static:
        qx, sa = I.quantize_nhwc_scaled(x, s_in, 16), s_in
    else:
        qx, sa = I.quantize_nhwc(x, 16)
    want_s = 0.021 if static else O.scale_of(np.array([np.abs(xf).max()], np.float32))[0]
    assert n(sa)[0] == np.float32(want_s)
    for bias, res, act in ((b, r, I.ACT_SILU), (None, None, I.ACT_NONE), (b, None, I.ACT_RELU)):
        y_r, acc_r = I.conv2d_i8_nhwc(qx, sa, wq, stride, pad, bias, res, act, want_acc=True)
        y, acc, sx = I.conv2d_nchw_fq(x, wq, stride, pad, bias, res, act, s_x=s_in, want_acc=True, want_scale=True)
        assert torch.equal(sx, sa)
        assert torch.equal(acc, acc_r)
        assert torch.equal(y, y_r), f"max |diff| {float((y - y_r).abs().max())}"
        parts, nparts, _ = y._bq_absmax
        assert 1 <= nparts <= 4096 and torch.equal(parts[:nparts].max(), y.abs().max())
        if O_ % 16 == 0:
            y2_r, q_r = I.conv2d_i8_nhwc_q(qx, sa, wq, s_out, stride, pad, bias, res, act)
            y2, q = I.conv2d_nchw_fq(x, wq, stride, pad, bias, res, act, s_x=s_in, s_out=s_out)
            none, q_alone = I.conv2d_nchw_fq(x, wq, stride, pad, bias, res, act, s_x=s_in, s_out=s_out,
                                             f32_out=False)
            assert none is None
            assert torch.equal(y2, y2_r) and torch.equal(q, q_r) and torch.equal(q_alone, q_r)
    if Nimg * OH * OW <= 4096:  # the accumulators against the oracle's quantize and conv
        qo = np.zeros((Nimg, H, W, 16), np.int8)
        qo[..., :C] = O.quantize_with_scale(xf, np.float32(want_s)).transpose(0, 2, 3, 1)
        acc_o, _, _ = O.conv2d_i8_nhwc(qo, n(wq.q), k, k, stride, pad)
        assert np.array_equal(n(acc), acc_o)


def test_refuses_what_the_small_k_kernel_does_not_take(dev):
    """A 7x7 stem (K = 49 * 16 > 256), O > 64 and more than 8 input channels:
    NotImplementedError, nothing launched, so the layer falls back to the two-pass form;
    the C entry refuses the same (BQ_ERR_UNSUPPORTED) past the wrapper's checks."""
    rng = np.random.default_rng(3)
    for C, O_, k in ((3, 64, 7), (3, 80, 3), (12, 32, 3)):
        x = t(rng.normal(size=(2, C, 32, 32)).astype(np.float32), dev)
        wq = I.pack_conv_weight(t(rng.normal(size=(O_, C, k, k)).astype(np.float32), dev))
        with pytest.raises(NotImplementedError):
            I.conv2d_nchw_fq(x, wq, 2, k // 2)
        out = torch.empty((2 * 16 * 16 * O_,), dtype=torch.float32, device=dev)
        s_x = t(np.array([0.02], np.float32), dev)
        rc = I.lib().bq_conv2d_i8_nchw_fq(x.data_ptr(), 2, C, 32, 32, s_x.data_ptr(), wq.q.data_ptr(), O_, k, k, 2,
                                          k // 2, wq.s.data_ptr(), None, None, I.ACT_NONE, out.data_ptr(), None,
                                          None, None, None, 0, None, None, None, 0, I._stream(x))
        assert rc == I._lib.BQ_ERR_UNSUPPORTED


def test_a_network_stem_takes_the_fused_path(dev):
    """nn.Conv2d routes a contiguous NCHW f32 image into a 16-padded int8 conv through the
    fused call, static and dynamic, and gives the two-pass result."""
    import borch_amd as bt
    torch.manual_seed(0)
    conv = bt.nn.Conv2d(3, 32, 3, stride=2, padding=1).to(dev)
    x = torch.randn(4, 3, 64, 64, device=dev)
    assert conv.quantize_int8()
    calls = []
    real = I.conv2d_nchw_fq

    def spy(*a, **kw):
        calls.append(kw.get("s_x") is not None)
        return real(*a, **kw)

    I.conv2d_nchw_fq = spy
    try:
        with torch.no_grad():
            y = conv(x)
            qx, sa = I.quantize_nhwc(x, 16)
            assert torch.equal(y, I.conv2d_i8_nhwc(qx, sa, conv.int8, 2, 1, conv.bias, None, conv.act))
            assert bt.calibrate_int8(conv, [x]) == 1
            y_s = conv(x)
            qx_s = I.quantize_nhwc_scaled(x, conv.in_scale, 16)
            _, q_r = I.conv2d_i8_nhwc_q(qx_s, conv.in_scale, conv.int8, conv.out_scale, 2, 1, conv.bias, None,
                                        conv.act)
            assert torch.equal(y_s._int8_twin[0], q_r)
            q_alone, s = conv.twin_forward(x)
            assert torch.equal(q_alone, q_r) and s is conv.out_scale
    finally:
        I.conv2d_nchw_fq = real
    assert calls == [False, True, True]


def test_a_misaligned_image_and_an_empty_batch(dev):
    """An image 4 bytes off 16-byte alignment (a view into a larger buffer) is not taken by the
    fused call (NotImplementedError) and the layer gives the two-pass result; an empty batch
    is a no-op."""
    import borch_amd as bt
    torch.manual_seed(1)
    conv = bt.nn.Conv2d(3, 32, 3, stride=2, padding=1).to(dev)
    assert conv.quantize_int8()
    buf = torch.randn(4 * 3 * 40 * 40 + 1, device=dev)
    x = buf[1:].view(4, 3, 40, 40)
    assert x.data_ptr() % 16 == 4 and x.is_contiguous()
    with pytest.raises(NotImplementedError):
        I.conv2d_nchw_fq(x, conv.int8, 2, 1)
    with torch.no_grad():
        y = conv(x)
        qx, sa = I.quantize_nhwc(x, 16)
        assert torch.equal(y, I.conv2d_i8_nhwc(qx, sa, conv.int8, 2, 1, conv.bias, None, conv.act))
        s_x = t(np.array([0.02], np.float32), dev)
        y0 = I.conv2d_nchw_fq(torch.empty((0, 3, 40, 40), device=dev), conv.int8, 2, 1, s_x=s_x)
        assert tuple(y0.shape) == (0, 32, 20, 20)
