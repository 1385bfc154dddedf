"""GPU parity of the small-K dense kernel (smallk_i8_kernel, plan id BQ_CFG_SMALLK).

At the shapes the rule gives it (a narrow output over many rows) it is held to the CPU
oracle bit for bit. Everywhere it may run (N <= 256, N % 4 == 0, K <= 256), forced through
the plan API, it must give what the tiled kernel gives on every epilogue: per-row and
per-tensor activation scales, bias or none, the residual, ReLU / SiLU / GELU, the int32
accumulators, the int8 twin, the maxima and outputs that are not 16-byte aligned.
"""
import sys

import numpy as np
import pytest
import torch

from borch_amd import _lib as L
from borch_amd import int8 as I
from oracle import quant as O

pytestmark = pytest.mark.gpu

SMALLK = L.CFG_SMALLK


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def n(x):
    return x.detach().cpu().numpy()


@pytest.fixture
def no_plans():
    from borch_amd import tune as T
    T.clear_plans()
    yield T
    T.clear_plans()


def operands(M, N, K, seed, dev):
    rng = np.random.default_rng(seed)
    qa = rng.integers(-127, 128, size=(M, K)).astype(np.int8)
    qw = rng.integers(-127, 128, size=(N, K)).astype(np.int8)
    sa = rng.uniform(1e-4, 1e-3, M).astype(np.float32)
    sw = rng.uniform(1e-4, 1e-3, N).astype(np.float32)
    b = rng.normal(size=N).astype(np.float32)
    res = rng.normal(size=(M, N)).astype(np.float32)
    return qa, qw, sa, sw, b, res


@pytest.mark.parametrize("M,N,K,act", [(131072 + 37, 16, 32, I.ACT_NONE), (200704, 24, 96, I.ACT_RELU),
                                       (140001, 32, 144, I.ACT_NONE), (131079, 96, 16, I.ACT_RELU),
                                       (200704, 144, 32, I.ACT_NONE), (100352, 144, 32, I.ACT_RELU),
                                       (100352, 24, 96, I.ACT_NONE), (65536, 32, 16, I.ACT_NONE)])
def test_rule_shapes_match_the_oracle(dev, no_plans, M, N, K, act):
    """The rule's own pick at a narrow output over many rows, against the oracle: int32
    accumulators and the f32 epilogue bit for bit (ragged last step included)."""
    T = no_plans
    say(f"small-K rule M={M} N={N} K={K} act={act}")
    assert T.candidates((M, N, K))[0] == (SMALLK, 1)
    qa, qw, sa, sw, b, res = operands(M, N, K, M + N + K, dev)
    y, acc = I.gemm_i8(t(qa, dev), t(qw, dev), t(sa, dev), t(sw, dev), t(b, dev), act=act, want_acc=True,
                       residual=t(res, dev))
    acc_o = O.gemm_i8_i32(qa, qw)
    assert np.array_equal(n(acc), acc_o)
    want = O.dequant(acc_o, sa, sw, b, relu=act == I.ACT_RELU, residual=res)
    assert np.array_equal(n(y), want), f"max |diff| {np.abs(n(y) - want).max()}"


SHAPES = [(1000, 40, 96), (4097, 4, 16), (777, 64, 256), (130, 12, 48), (65, 36, 144), (50176, 40, 240),
          (70, 8, 208), (3001, 96, 16), (1000, 160, 64), (999, 112, 128), (300, 80, 192), (2000, 240, 48),
          (777, 256, 64)]


@pytest.mark.parametrize("M,N,K", SHAPES)
@pytest.mark.parametrize("act", [I.ACT_NONE, I.ACT_RELU, I.ACT_SILU, I.ACT_GELU])
def test_equals_the_tiled_kernel(dev, no_plans, M, N, K, act):
    """Forced through the plan API against the tiled 128 x 32 / 64 x 64 tiles: the f32 output
    and int32 accumulators bit for bit, with and without bias and residual (per-row scales)."""
    T = no_plans
    say(f"small-K vs tiled M={M} N={N} K={K} act={act}")
    qa, qw, sa, sw, b, res = (t(v, dev) for v in operands(M, N, K, M * 7 + N + K + act, dev))
    assert (SMALLK, 1) in T.candidates((M, N, K))
    for bias, r in ((b, res), (None, None), (b, None)):
        got = []
        for cfg in (SMALLK, 12, 7):
            T.set_plan((M, N, K), cfg, 1)
            got.append(I.gemm_i8(qa, qw, sa, sw, bias, act=act, want_acc=True, residual=r))
        for y, acc in got[1:]:
            assert torch.equal(acc, got[0][1])
            assert torch.equal(y, got[0][0]), f"max |diff| {float((y - got[0][0]).abs().max())}"


@pytest.mark.parametrize("Nimg,H,C,O_", [(64, 112, 32, 16), (64, 56, 96, 24), (3, 15, 48, 64), (7, 9, 256, 48),
                                         (5, 11, 16, 20), (64, 112, 16, 96), (64, 56, 32, 144), (64, 28, 48, 240)])
def test_conv_twin_and_maxima(dev, no_plans, Nimg, H, C, O_):
    """A 1x1 conv (per-tensor scale) under the small-K plan and a tiled plan: the f32 output,
    the accumulators, the largest of the per-workgroup maxima (which the next quantizer
    reads) and, where O % 16 == 0, the int8 twin of a calibrated scale (alone and beside the
    f32 output)."""
    T = no_plans
    say(f"small-K 1x1 conv N={Nimg} H={H} C={C} O={O_}")
    rng = np.random.default_rng(Nimg + H + C + O_)
    qx = t(rng.integers(-127, 128, size=(Nimg, H, H, C)).astype(np.int8), dev)
    sa = t(np.array([0.013], np.float32), dev)
    w8 = I.pack_conv_weight(t((rng.normal(size=(O_, C, 1, 1)) * 0.1).astype(np.float32), dev))
    b = t(rng.normal(size=O_).astype(np.float32), dev)
    r = t(rng.normal(size=(Nimg, O_, H, H)).astype(np.float32), dev).contiguous(memory_format=torch.channels_last)
    s_out = t(np.array([0.04], np.float32), dev)
    problem = (Nimg, H, H, C, O_, 1, 1, 1, 0)
    outs = []
    for cfg in (SMALLK, 12):
        T.set_plan(problem, cfg, 1)
        y, acc = I.conv2d_i8_nhwc(qx, sa, w8, 1, 0, b, r, I.ACT_RELU, want_acc=True)
        parts, nparts, _ = y._bq_absmax
        got = [y, acc, parts[:nparts].max()]
        if O_ % 16 == 0:
            y2, q = I.conv2d_i8_nhwc_q(qx, sa, w8, s_out, 1, 0, b, r, I.ACT_RELU)
            _, q_alone = I.conv2d_i8_nhwc_q(qx, sa, w8, s_out, 1, 0, b, r, I.ACT_RELU, f32_out=False)
            got += [y2, q, q_alone]
        outs.append(got)
    for a_, b_ in zip(outs[0], outs[1]):
        assert torch.equal(a_, b_)
    assert torch.equal(outs[0][2], outs[0][0].abs().max())
    if O_ % 16 == 0:
        assert torch.equal(outs[0][3], outs[0][0]) and torch.equal(outs[0][4], outs[0][5])


# (N, H, W, C, O, k, stride, pad): EfficientNet-B0 b64's stem (the rule's pick), then
# strides, paddings, ragged images and K steps, 2x2 and 4x4 filters (K <= 256), wider outputs
CONV_CASES = [(64, 224, 224, 16, 32, 3, 2, 1), (2, 40, 40, 16, 32, 3, 2, 1), (3, 17, 13, 16, 20, 3, 1, 1),
              (2, 15, 15, 32, 64, 2, 2, 0), (1, 23, 19, 16, 48, 4, 1, 2), (2, 12, 12, 16, 8, 2, 3, 1),
              (4, 9, 9, 96, 12, 1, 2, 0), (2, 11, 11, 16, 4, 4, 4, 0), (2, 13, 13, 16, 160, 2, 1, 0),
              (3, 10, 10, 32, 96, 1, 1, 0), (2, 9, 9, 48, 240, 1, 1, 0), (2, 12, 12, 16, 256, 2, 2, 0)]


@pytest.mark.parametrize("Nimg,H,W,C,O_,k,stride,pad", CONV_CASES)
def test_implicit_gemm_conv(dev, no_plans, Nimg, H, W, C, O_, k, stride, pad):
    """Implicit-GEMM convs under the small-K plan against the tiled kernel (f32 output,
    accumulators, maxima, residual and SiLU), and the small ones against the oracle."""
    T = no_plans
    say(f"small-K conv N={Nimg} H={H} W={W} C={C} O={O_} k={k} s={stride} p={pad}")
    rng = np.random.default_rng(Nimg + H + W + C + O_ + k)
    x = rng.integers(-127, 128, size=(Nimg, H, W, C)).astype(np.int8)
    qx = t(x, dev)
    sa = t(np.array([0.011], np.float32), dev)
    wf = (rng.normal(size=(O_, C, k, k)) * 0.1).astype(np.float32)
    w8 = I.pack_conv_weight(t(wf, dev))
    b = t(rng.normal(size=O_).astype(np.float32), dev)
    OH, OW = (H + 2 * pad - k) // stride + 1, (W + 2 * pad - k) // stride + 1
    r = t(rng.normal(size=(Nimg, O_, OH, OW)).astype(np.float32), dev).contiguous(memory_format=torch.channels_last)
    problem = (Nimg, H, W, C, O_, k, k, stride, pad)
    if Nimg * OH * OW >= 131072 and O_ <= 32:
        assert T.candidates(problem)[0] == (SMALLK, 1)
    outs = []
    for cfg in (SMALLK, 12):
        T.set_plan(problem, cfg, 1)
        y, acc = I.conv2d_i8_nhwc(qx, sa, w8, stride, pad, b, r, I.ACT_SILU, want_acc=True)
        parts, nparts, _ = y._bq_absmax
        outs.append((y, acc, parts[:nparts].max()))
    for a_, b_ in zip(outs[0], outs[1]):
        assert torch.equal(a_, b_)
    if Nimg * OH * OW <= 4096:
        acc_o, _, _ = O.conv2d_i8_nhwc(x, n(w8.q), k, k, stride, pad)
        assert np.array_equal(n(outs[0][1]), acc_o)


def test_unaligned_outputs(dev, no_plans):
    """Output, accumulator and residual pointers 4 bytes off 16-byte alignment (the C ABI
    takes any float pointer): the small-K kernel's four-byte stores give the tiled kernel's
    general-path results."""
    T = no_plans
    M, N, K = 3000, 20, 64
    say(f"small-K unaligned M={M} N={N} K={K}")
    qa, qw, sa, sw, b, res = (t(v, dev) for v in operands(M, N, K, 5, dev))
    res_u = torch.empty(M * N + 1, dtype=torch.float32, device=dev)
    res_u[1:] = res.reshape(-1)
    results = []
    for cfg in (SMALLK, 12):
        T.set_plan((M, N, K), cfg, 1)
        out = torch.full((M * N + 1,), 7.0, dtype=torch.float32, device=dev)
        acc = torch.full((M * N + 1,), 7, dtype=torch.int32, device=dev)
        I.check(L.lib().bq_gemm_i8(qa.data_ptr(), qw.data_ptr(), M, N, K, sa.data_ptr(), sw.data_ptr(), b.data_ptr(),
                                   res_u.data_ptr() + 4, I.ACT_SILU, out.data_ptr() + 4, acc.data_ptr() + 4,
                                   *I._ws_args(dev), I._stream(qa)))
        torch.cuda.synchronize()
        assert float(out[0]) == 7.0 and int(acc[0]) == 7  # nothing written before the outputs
        results.append((out, acc))
    assert torch.equal(results[0][0], results[1][0])
    assert torch.equal(results[0][1], results[1][1])
    y_al = I.gemm_i8(qa, qw, sa, sw, b, act=I.ACT_SILU, residual=res)
    assert torch.equal(results[0][0][1:].reshape(M, N), y_al)


def test_plan_set_refuses_what_it_does_not_take(dev, no_plans):
    T = no_plans
    with pytest.raises(ValueError):
        T.set_plan((1000, 260, 64), SMALLK, 1)  # N > 256
    with pytest.raises(ValueError):
        T.set_plan((1000, 80, 256), SMALLK, 1)  # 5 column blocks x 4 K steps of weight registers
    with pytest.raises(ValueError):
        T.set_plan((1000, 18, 64), SMALLK, 1)   # N % 4
    with pytest.raises(ValueError):
        T.set_plan((1000, 32, 272), SMALLK, 1)  # K > 256
    with pytest.raises(ValueError):
        T.set_plan((2, 32, 32, 32, 32, 3, 3, 1, 1), SMALLK, 1)  # a conv of K = 288
    with pytest.raises(ValueError):
        T.set_plan((1000, 32, 64), SMALLK, 2)   # split
    T.set_plan((2, 32, 32, 16, 32, 1, 1, 1, 0), SMALLK, 1)  # a 1x1 stride-1 unpadded conv
    T.set_plan((2, 32, 32, 16, 32, 3, 3, 2, 1), SMALLK, 1)  # an implicit-GEMM conv of K = 144


@pytest.mark.parametrize("Nimg,H,C,O_", [(64, 112, 16, 96), (3, 15, 48, 64)])
def test_twin_rows_and_unaligned_twin(dev, no_plans, Nimg, H, C, O_):
    """The int8 twin alone (the rule takes the small-K kernel for it from 65,536 rows): its
    rows staged through LDS and stored whole equal the tiled kernel's twin, and a twin
    pointer 4 bytes off 16-byte alignment (per-lane four-byte stores, the C ABI takes it)
    gives the same bytes."""
    T = no_plans
    say(f"small-K twin rows N={Nimg} H={H} C={C} O={O_}")
    rng = np.random.default_rng(Nimg + H + C + O_)
    qx = t(rng.integers(-127, 128, size=(Nimg, H, H, C)).astype(np.int8), dev)
    sa = t(np.array([0.013], np.float32), dev)
    w8 = I.pack_conv_weight(t((rng.normal(size=(O_, C, 1, 1)) * 0.1).astype(np.float32), dev))
    b = t(rng.normal(size=O_).astype(np.float32), dev)
    s_out = t(np.array([0.04], np.float32), dev)
    problem = (Nimg, H, H, C, O_, 1, 1, 1, 0)
    twins = []
    for cfg in (SMALLK, 12):
        T.set_plan(problem, cfg, 1)
        _, q = I.conv2d_i8_nhwc_q(qx, sa, w8, s_out, 1, 0, b, None, I.ACT_SILU, f32_out=False)
        twins.append(q)
    assert torch.equal(twins[0], twins[1])
    T.set_plan(problem, SMALLK, 1)
    M = Nimg * H * H
    qbuf = torch.full((M * O_ + 16,), 7, dtype=torch.int8, device=dev)
    I.check(L.lib().bq_conv2d_i8_nhwc_q(qx.data_ptr(), Nimg, H, H, C, w8.q.data_ptr(), O_, 1, 1, 1, 0,
                                        sa.data_ptr(), w8.s.data_ptr(), b.data_ptr(), None, I.ACT_SILU, None, None,
                                        s_out.data_ptr(), qbuf.data_ptr() + 4, None, *I._ws_args(dev), I._stream(qx)))
    torch.cuda.synchronize()
    assert torch.equal(qbuf[4:4 + M * O_].reshape(twins[0].shape), twins[0])
    assert int(qbuf[:4].eq(7).sum()) == 4 and int(qbuf[4 + M * O_:].eq(7).sum()) == 12
