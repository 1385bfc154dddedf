"""GPU parity of the dynamic int8 twin (bq_conv2d_i8_nhwc_dq).

The call quantizes a conv's output per tensor at its dynamic scale without storing the f32
output: the small-K kernel runs twice, first storing only its workgroups' maxima, then the
twin at float32(max / 127) of them. It must give, bit for bit, what the two-call form gives
(``conv2d_i8_nhwc`` with its per-workgroup maxima, then ``quantize_nhwc`` into O channels):
the bytes and the scale, on the layers the small-K kernel takes by its rule (EfficientNet-B0
b64's 112^2 and 56^2 expansions) and, with a plan forcing it, on implicit-GEMM convs, with a
residual and each activation; the scale is also held to the oracle's scale of the device's
f32 output, and the bytes to the oracle's quantization of it.
"""
import sys

import numpy as np
import pytest
import torch

from borch_amd import int8 as I
from borch_amd import tune as T
from oracle import quant as O

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def n(x):
    return x.detach().cpu().numpy()


@pytest.fixture
def no_plans():
    T.clear_plans()
    yield
    T.clear_plans()


def _layer(dev, rng, Nimg, H, C, O_, k):
    qx = t(rng.integers(-127, 128, size=(Nimg, H, H, C), dtype=np.int8), dev)
    sa = t(np.array([0.013], np.float32), dev)
    wq = I.pack_conv_weight(t((rng.normal(size=(O_, C, k, k)) * 0.2).astype(np.float32), dev))
    b = t((rng.normal(size=O_) * 0.5).astype(np.float32), dev)
    return qx, sa, wq, b


def _two_call(qx, sa, wq, stride, pad, bias, res, act):
    y = I.conv2d_i8_nhwc(qx, sa, wq, stride, pad, bias, res, act)
    q, s = I.quantize_nhwc(y, wq.O)
    return y, q, s


def _check(y, q, s, q_r, s_r, name):
    assert torch.equal(s, s_r), f"{name}: scale {float(s)} != {float(s_r)}"
    assert torch.equal(q, q_r), f"{name}: {int((q != q_r).sum())} bytes differ"
    # the oracle's scale and quantization of the device's own f32 output
    yn = n(y).transpose(0, 2, 3, 1)
    want_s = O.scale_of(np.array([np.abs(yn).max()], np.float32))[0]
    assert n(s)[0] == want_s
    sel = slice(0, min(2, yn.shape[0]))
    assert np.array_equal(n(q[sel]), O.quantize_with_scale(yn[sel], want_s))


# (N, H, C, O, act): EfficientNet-B0 b64's blocks.1 expansion (802816 x 96 x 16) and blocks.2/3
# expansions (200704 x 144 x 32), then a 65536-row edge with 160 columns
RULE_CASES = [(64, 112, 16, 96, I.ACT_SILU), (64, 56, 32, 144, I.ACT_SILU), (16, 64, 16, 160, I.ACT_RELU)]


@pytest.mark.parametrize("Nimg,H,C,O_,act", RULE_CASES)
def test_rule_layers_equal_the_two_call_form(dev, no_plans, Nimg, H, C, O_, act):
    say(f"dynamic twin N={Nimg} H={H} C={C} O={O_} act={act}")
    rng = np.random.default_rng(Nimg + H + C + O_)
    qx, sa, wq, b = _layer(dev, rng, Nimg, H, C, O_, 1)
    y, q_r, s_r = _two_call(qx, sa, wq, 1, 0, b, None, act)
    q, s = I.conv2d_i8_nhwc_dq(qx, sa, wq, 1, 0, b, None, act)
    _check(y, q, s, q_r, s_r, "rule")
    # a second call on the same buffers' successors: the maxima are a fresh pass each time
    q2, s2 = I.conv2d_i8_nhwc_dq(qx, sa, wq, 1, 0, b, None, act)
    assert torch.equal(q2, q) and torch.equal(s2, s)


def test_residual_and_each_activation(dev, no_plans):
    rng = np.random.default_rng(5)
    qx, sa, wq, b = _layer(dev, rng, 8, 128, 32, 96, 1)
    r = t(rng.normal(size=(8, 96, 128, 128)).astype(np.float32), dev).contiguous(memory_format=torch.channels_last)
    for res in (None, r):
        for act in (I.ACT_NONE, I.ACT_RELU, I.ACT_SILU, I.ACT_GELU):
            say(f"dynamic twin 131072 x 96 x 32 residual={res is not None} act={act}")
            y, q_r, s_r = _two_call(qx, sa, wq, 1, 0, b, res, act)
            q, s = I.conv2d_i8_nhwc_dq(qx, sa, wq, 1, 0, b, res, act)
            _check(y, q, s, q_r, s_r, f"act {act}")


@pytest.mark.parametrize("Nimg,H,C,O_,k,stride,pad", [(16, 32, 16, 32, 3, 1, 1), (4, 33, 16, 48, 3, 2, 1),
                                                      (2, 20, 32, 64, 2, 2, 0)])
def test_implicit_gemm_convs_under_a_plan(dev, no_plans, Nimg, H, C, O_, k, stride, pad):
    """Below the rule's row count the call is refused (NotImplementedError, nothing launched);
    with a plan forcing the small-K kernel it runs the implicit-GEMM form, equal to two calls."""
    say(f"dynamic twin conv N={Nimg} H={H} C={C} O={O_} k={k} s={stride} p={pad}")
    rng = np.random.default_rng(H + O_ + k)
    qx, sa, wq, b = _layer(dev, rng, Nimg, H, C, O_, k)
    with pytest.raises(NotImplementedError):
        I.conv2d_i8_nhwc_dq(qx, sa, wq, stride, pad, b, None, I.ACT_SILU)
    T.set_plan((Nimg, H, H, C, O_, k, k, stride, pad), I._lib.CFG_SMALLK, 1)
    y, q_r, s_r = _two_call(qx, sa, wq, stride, pad, b, None, I.ACT_SILU)
    q, s = I.conv2d_i8_nhwc_dq(qx, sa, wq, stride, pad, b, None, I.ACT_SILU)
    _check(y, q, s, q_r, s_r, "conv")
    # the accumulators behind it against the oracle's integer conv
    _, acc = I.conv2d_i8_nhwc(qx, sa, wq, stride, pad, b, None, I.ACT_SILU, want_acc=True)
    acc_o, _, _ = O.conv2d_i8_nhwc(n(qx), n(wq.q), k, k, stride, pad)
    assert np.array_equal(n(acc), acc_o)


def test_refusals(dev, no_plans):
    rng = np.random.default_rng(9)
    qx, sa, wq, b = _layer(dev, rng, 64, 112, 16, 24, 1)  # O % 16 != 0
    with pytest.raises(NotImplementedError):
        I.conv2d_i8_nhwc_dq(qx, sa, wq)
    qx, sa, wq, b = _layer(dev, rng, 2, 16, 64, 64, 3)  # K = 576: the tiled kernel's
    with pytest.raises(NotImplementedError):
        I.conv2d_i8_nhwc_dq(qx, sa, wq, 1, 1)
    qx, sa, wq, b = _layer(dev, rng, 0, 112, 16, 96, 1)  # an empty batch
    q, s = I.conv2d_i8_nhwc_dq(qx, sa, wq)
    assert tuple(q.shape) == (0, 112, 112, 96)


def test_a_dynamic_block_takes_it(dev):
    """EfficientNet-B0's first expanding block with dynamic scales: the expand conv feeds the
    depthwise conv through the dynamic twin, and the block's output equals the two-call
    form's (the block run with the dynamic twin path off)."""
    from borch_amd import nets
    import borch_amd as bt
    torch.manual_seed(0)
    blk = nets.MBConv(16, 24, 3, 2, 6).to(dev).eval()
    blk.fuse()
    assert bt.quantize_for_int8(blk) == 3
    x = torch.randn(64, 16, 112, 112, device=dev).contiguous(memory_format=torch.channels_last)
    calls = []
    real = I.conv2d_i8_nhwc_dq

    def spy(*a, **kw):
        calls.append(1)
        return real(*a, **kw)

    I.conv2d_i8_nhwc_dq = spy
    try:
        with torch.no_grad():
            y = blk(x)
            ex, dw = blk.expand.conv, blk.dw.conv
            assert ex.dynamic_twin_of(dw, x) and not ex.dynamic_twin_of(dw, x[:2])  # 25088 rows: two calls
            h = dw(ex(x))  # the two-call form of the same two layers
            q, s = ex.dynamic_twin_forward(x)
            q_r, s_r = I.quantize_nhwc(ex(x), dw.int8.cpad)
            assert torch.equal(q, q_r) and torch.equal(s, s_r)
            assert torch.equal(dw.forward_int8(q, s), h)
    finally:
        I.conv2d_i8_nhwc_dq = real
    assert len(calls) == 2
    assert torch.isfinite(y).all()


def test_graph_replays_of_a_dynamic_forward(dev, no_plans):
    """EfficientNet-B0 b16 at 224^2 with dynamic scales (its 112^2 expansion, 200704 rows, takes
    the dynamic twin): HIP graph replays equal the eager forward, with eager work between
    them, and the eager forward with the dynamic twin off (the two-call form) gives the same
    logits."""
    import borch_amd as bt
    from borch_amd import nets, workloads as WL
    say("EfficientNet-B0 b16 dynamic: graph replays, eager, two-call form")
    model = nets.build("efficientnet_b0", seed=2, device=dev)
    c = bt.compiled(model, int8=True, graph=True)
    x = torch.from_numpy(WL.c4_input(16, 3)).to(dev)
    calls = []
    real = I.conv2d_i8_nhwc_dq

    def spy(*a, **kw):
        calls.append(1)
        return real(*a, **kw)

    I.conv2d_i8_nhwc_dq = spy
    try:
        with torch.no_grad():
            eager = model(x).clone()
            assert calls, "the dynamic twin was not taken"
            for i in range(3):
                got = c(x)
                assert torch.equal(got, eager), f"replay {i}"
                model(torch.randn_like(x))  # eager work in between
                torch.cuda.synchronize()
            for b in model.blocks:
                b.twin_path = False
            try:
                assert torch.equal(model(x), eager), "the two-call form differs"
            finally:
                for b in model.blocks:
                    del b.twin_path
    finally:
        I.conv2d_i8_nhwc_dq = real
