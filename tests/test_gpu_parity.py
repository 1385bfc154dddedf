"""GPU parity: the HIP kernels through the C ABI against the CPU oracle on seeded inputs.

Integer results (int8 packings, int32 accumulators) must be bit-exact. f32 outputs are
held to the task's tolerance (1e-5 relative / 1e-6 absolute) and, since the epilogue does
one float32 rounding per operation in the oracle's order, are also checked bit-exact.
"""
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

ROOT = Path(__file__).resolve().parent.parent

from borch_amd import int8 as I
from borch_amd import workloads as WL
from oracle import quant as O

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-5, 1e-6


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def n(x):
    return x.detach().cpu().numpy()


def assert_f32(got, want):
    np.testing.assert_allclose(got, want, rtol=RTOL, atol=ATOL)
    assert np.array_equal(got, want), f"max |diff| {np.abs(got - want).max()}"


# ------------------------------------------------------------------------ quantizers

@pytest.mark.parametrize("M,K", [(1, 16), (16, 512), (7, 1000), (3, 4096), (6304 // 16, 768), (5, 10000),
                                 (4, 13), (2, 8192), (1, 3072), (9, 2052), (5, 1284), (6, 4100), (1029, 772), (1024, 256), (2048, 1024),
                                 (1500, 100), (5, 2048), (130, 6144)])
def test_quantize_rows(dev, M, K):
    say(f"quantize_rows M={M} K={K}")
    rng = np.random.default_rng(M * 131 + K)
    x = rng.normal(size=(M, K)).astype(np.float32) * np.float32(rng.uniform(0.1, 10))
    if M > 2:
        x[1] = 0.0
    q, s = I.quantize_rows(t(x, dev))
    qo, so = O.quantize_rows(x)
    assert np.array_equal(n(s), so)
    assert np.array_equal(n(q), qo)


def test_quantize_rows_exact_ties(dev):
    say("quantize_rows ties")
    # peak 127 -> s = 1 exactly; k + 0.5 ties and their neighbours
    ks = np.arange(-126, 126, dtype=np.float32)
    row = np.concatenate([[127.0], ks + 0.5, np.nextafter(ks + 0.5, np.float32(200)),
                          np.nextafter(ks + 0.5, np.float32(-200))]).astype(np.float32)
    row = np.pad(row, (0, (-row.size) % 4))
    x = np.stack([row, row * np.float32(0.5), -row]).astype(np.float32)
    q, s = I.quantize_rows(t(x, dev))
    qo, so = O.quantize_rows(x)
    assert np.array_equal(n(s), so)
    assert np.array_equal(n(q), qo)


@pytest.mark.parametrize("shape,cpad,cl", [((2, 3, 8, 8), 16, False), ((2, 64, 16, 16), 64, True),
                                          ((3, 24, 5, 7), 32, True), ((1, 5, 3, 3), 8, False),
                                          ((4, 3, 33, 31), 16, False), ((2, 40, 9, 9), 48, True),
                                          ((1, 17, 4, 4), 32, True)])
def test_quantize_nhwc(dev, shape, cpad, cl):
    say(f"quantize_nhwc {shape} cpad={cpad} channels_last={cl}")
    rng = np.random.default_rng(sum(shape))
    x = rng.normal(size=shape).astype(np.float32)
    xt = t(x, dev)
    if cl:
        xt = xt.contiguous(memory_format=torch.channels_last)
    q, s = I.quantize_nhwc(xt, cpad)
    qo, so = O.quantize_act_nhwc(x, cpad)
    assert np.array_equal(n(s), so)
    assert np.array_equal(n(q), qo)


def test_quantize_nhwc_padded_many_pixels(dev):
    """A channels-last input of 24 channels into 32 over more pixels than one grid covers
    (2.17 M, each thread takes several): the same bytes as the channel-scaled quantizer with a
    gate of ones (fl(x * 1) = x; another kernel), with the dynamic and a static scale, and the
    oracle's on the first and last images."""
    rng = np.random.default_rng(77)
    x = (rng.normal(size=(64, 24, 184, 184)) * 3).astype(np.float32)
    xt = t(x, dev).contiguous(memory_format=torch.channels_last)
    ones = torch.ones((64, 24), device=dev)
    q, s = I.quantize_nhwc(xt, 32)
    q_ch, s_ch = I.quantize_nhwc_chscale(xt, ones, 32)
    assert torch.equal(s, s_ch) and torch.equal(q, q_ch)
    sc = t(np.array([0.01], np.float32), dev)
    q2 = I.quantize_nhwc_scaled(xt, sc, 32)
    q2_ch, _ = I.quantize_nhwc_chscale(xt, ones, 32, sc)
    assert torch.equal(q2, q2_ch)
    for i in (0, 63):
        want = np.zeros((184, 184, 32), np.int8)
        want[..., :24] = O.quantize_with_scale(x[i], n(s)[0]).transpose(1, 2, 0)
        assert np.array_equal(n(q[i]), want)


@pytest.mark.parametrize("N,C,H,cpad", [(4, 96, 14, 96), (3, 36, 9, 48), (64, 1152, 7, 1152), (2, 8, 5, 16)])
def test_quantize_chscale(dev, N, C, H, cpad):
    """The squeeze-excite-gated quantizer equals quantizing the stored product x * gate
    (bytes and scale), dynamic and with a calibrated scale; padding channels are zero."""
    say(f"quantize_nhwc_chscale N={N} C={C} H={H} cpad={cpad}")
    rng = np.random.default_rng(N + C + H)
    x = t(rng.normal(size=(N, C, H, H)).astype(np.float32), dev).contiguous(memory_format=torch.channels_last)
    g = t(rng.uniform(0, 1, size=(N, C)).astype(np.float32), dev)
    prod = x * g[:, :, None, None]
    q1, s1 = I.quantize_nhwc_chscale(x, g, cpad)
    q2, s2 = I.quantize_nhwc(prod.clone(memory_format=torch.channels_last), cpad)
    assert torch.equal(s1, s2) and torch.equal(q1, q2)
    qo, so = O.quantize_act_nhwc(n(prod), cpad)
    assert np.array_equal(n(q1), qo) and np.array_equal(n(s1), so)
    sc = torch.tensor([float(s2) * 0.5], dtype=torch.float32, device=dev)  # saturates the top half
    q3, _ = I.quantize_nhwc_chscale(x, g, cpad, sc)
    q4 = I.quantize_nhwc_scaled(prod, sc, cpad)
    assert torch.equal(q3, q4)


@pytest.mark.parametrize("N,C,H,S", [(64, 32, 112, 8), (8, 144, 56, 6), (4, 1152, 7, 48), (2, 36, 9, 9), (3, 1200, 5, 50)])
def test_se_gate(dev, N, C, H, S):
    """The fused squeeze-excite gates (mean, two small layers, SiLU, sigmoid in f32) against
    the float64 closed form within 1e-5 rel / 1e-6 abs, and bit-identical on a second run."""
    say(f"se_gate N={N} C={C} H={H} S={S}")
    from oracle import models as OM
    rng = np.random.default_rng(N + C + H + S)
    x = rng.normal(size=(N, C, H, H)).astype(np.float32)
    w1 = (rng.normal(size=(S, C)) / np.sqrt(C)).astype(np.float32)
    b1 = rng.normal(size=S).astype(np.float32)
    w2 = (rng.normal(size=(C, S)) / np.sqrt(S)).astype(np.float32)
    b2 = rng.normal(size=C).astype(np.float32)
    xt = t(x, dev).contiguous(memory_format=torch.channels_last)
    g = I.se_gate_nhwc(xt, t(w1, dev), t(b1, dev), t(w2, dev), t(b2, dev))
    np.testing.assert_allclose(n(g), OM.se_gate(x, w1, b1, w2, b2), rtol=RTOL, atol=ATOL)
    assert torch.equal(g, I.se_gate_nhwc(xt, t(w1, dev), t(b1, dev), t(w2, dev), t(b2, dev)))


@pytest.mark.parametrize("N,C,H,S,cpad", [(64, 32, 112, 8, 32), (8, 144, 56, 6, 144), (4, 1152, 7, 48, 1152),
                                         (3, 1200, 5, 50, 1216), (2, 36, 9, 9, 48)])
def test_se_gate_maxima_give_the_product_scale(dev, N, C, H, S, cpad):
    """The partial maxima the squeeze-excite writes (max over pixels of |x| times the gate,
    per channel) give quantize_nhwc_chscale the same scale and bytes in one pass as its two
    passes over x * gate and as quantizing the stored product; an x changed in place after
    the gate falls back to the two passes."""
    say(f"se_gate maxima N={N} C={C} H={H} S={S}")
    rng = np.random.default_rng(N * C + H + S)
    xt = t(rng.normal(size=(N, C, H, H)).astype(np.float32), dev).contiguous(memory_format=torch.channels_last)
    w1 = t((rng.normal(size=(S, C)) / np.sqrt(C)).astype(np.float32), dev)
    w2 = t((rng.normal(size=(C, S)) / np.sqrt(S)).astype(np.float32), dev)
    b1, b2 = t(rng.normal(size=S).astype(np.float32), dev), t(rng.normal(size=C).astype(np.float32), dev)
    g = I.se_gate_nhwc(xt, w1, b1, w2, b2)
    assert getattr(g, "_bq_product_absmax", None) is not None
    q1, s1 = I.quantize_nhwc_chscale(xt, g, cpad)  # one pass, the gate's maxima
    q2, s2 = I.quantize_nhwc_chscale(xt, g.clone(), cpad)  # two passes
    prod = (xt * g[:, :, None, None]).contiguous(memory_format=torch.channels_last)
    q3, s3 = I.quantize_nhwc(prod, cpad)
    assert torch.equal(s1, s2) and torch.equal(s1, s3)
    assert torch.equal(q1, q2) and torch.equal(q1, q3)
    xt.mul_(2.0)  # in place: the maxima no longer describe x
    q4, s4 = I.quantize_nhwc_chscale(xt, g, cpad)
    assert torch.equal(s4, s1 * 2) and torch.equal(q4, q1)


@pytest.mark.parametrize("M,K,affine", [(6304 // 8, 768, True), (5, 768, False), (1, 100, True), (9, 772, True),
                                        (1030, 1024, True), (3, 3072, True), (2, 4096, False), (7, 16, True)])
def test_layernorm_quantize_rows(dev, M, K, affine):
    """Fused LayerNorm + per-row quantize: the normalised rows (y output) within 1e-5 rel /
    1e-6 abs of float64 torch.layer_norm (a library routine), and the int8 rows and scales
    bit-exact against the oracle's quantize_rows of those same f32 rows."""
    say(f"layernorm_quantize_rows M={M} K={K} affine={affine}")
    rng = np.random.default_rng(M * 3 + K)
    x = (rng.normal(size=(M, K)) * rng.uniform(0.5, 3.0, size=(M, 1)) + rng.uniform(-2, 2, size=(M, 1))).astype(np.float32)
    g = rng.uniform(0.5, 1.5, K).astype(np.float32) if affine else None
    b = rng.normal(size=K).astype(np.float32) * np.float32(0.1) if affine else None
    q, s, y = I.layernorm_quantize_rows(t(x, dev), None if g is None else t(g, dev), None if b is None else t(b, dev),
                                        1e-6, want_y=True)
    T = lambda a: None if a is None else torch.from_numpy(a).double()
    want = torch.nn.functional.layer_norm(T(x), (K,), T(g), T(b), 1e-6).numpy()
    np.testing.assert_allclose(n(y), want, rtol=RTOL, atol=ATOL)
    qo, so = O.quantize_rows(n(y))
    assert np.array_equal(n(s), so) and np.array_equal(n(q), qo)
    q2, s2 = I.layernorm_quantize_rows(t(x, dev), None if g is None else t(g, dev), None if b is None else t(b, dev),
                                       1e-6)
    assert torch.equal(q2, q) and torch.equal(s2, s)


@pytest.mark.parametrize("M,K,act", [(6304 // 8, 3072, 3), (1030, 768, 3), (5, 100, 3), (3, 4096, 3), (2, 8192, 3),
                                     (7, 13, 3), (1030, 768, 2), (9, 520, 1)])
def test_quantize_rows_act(dev, M, K, act):
    """Per-row quantization of act(x) without storing it: the activated rows (y output)
    within 1e-5 rel / 1e-6 abs of the oracle's activation (GELU from a Chebyshev erfc, so
    not bit-equal to torch's erf-form GELU; the count of differing bits is printed), and
    the int8 rows and scales bit-exact against the oracle's quantize_rows of those same rows."""
    say(f"quantize_rows_act M={M} K={K} act={act}")
    rng = np.random.default_rng(M + K + act)
    x = (rng.normal(size=(M, K)) * 2).astype(np.float32)
    q, s, y = I.quantize_rows(t(x, dev), act, want_y=True)
    ref = {1: np.maximum(x, 0), 2: O.silu(x), 3: O.gelu(x)}[act]
    np.testing.assert_allclose(n(y), ref, rtol=RTOL, atol=ATOL)
    qo, so = O.quantize_rows(n(y))
    assert np.array_equal(n(s), so) and np.array_equal(n(q), qo)
    q2, s2 = I.quantize_rows(t(x, dev), act)
    assert torch.equal(q2, q) and torch.equal(s2, s)
    if act == 3:  # torch's device GELU, for reference
        yt = torch.nn.functional.gelu(t(x, dev))
        say(f"  GELU bits differing from torch's: {int((yt != y).sum())} of {M * K}")


def test_layernorm_quantize_rows_rejects(dev):
    """Rows longer than 4096 or not a multiple of 4 are refused by name (the Linear then
    runs the LayerNorm and the quantizer separately); nothing is launched."""
    with pytest.raises(NotImplementedError, match="K=4100"):
        I.layernorm_quantize_rows(torch.zeros(2, 4100, device=dev), None, None, 1e-6)
    with pytest.raises(NotImplementedError, match="K=6"):
        I.layernorm_quantize_rows(torch.zeros(2, 6, device=dev), None, None, 1e-6)


def test_quantize_tensor(dev):
    say("quantize_tensor")
    rng = np.random.default_rng(11)
    for size in (1, 7, 1000, 1 << 20, (1 << 20) + 3):
        x = rng.normal(size=size).astype(np.float32)
        q, s = I.quantize_tensor(t(x, dev))
        qo, so = O.quantize_tensor(x)
        assert np.array_equal(n(s), so) and np.array_equal(n(q), qo), size


# ------------------------------------------------------------------------------ GEMM

def test_c1_linear(dev):
    """C1: the 16x512x512 int8 Linear, every stage against the oracle."""
    say("C1 linear 16x512x512")
    x, w, b = WL.c1_linear(0)
    y_o, acc_o, (qx_o, sx_o), (qw_o, sw_o) = O.linear_int8(x, w, b)
    qw, sw = I.quantize_weight_per_channel(t(w, dev))
    assert np.array_equal(n(qw), qw_o) and np.array_equal(n(sw), sw_o)
    qx, sx = I.quantize_rows(t(x, dev))
    assert np.array_equal(n(qx), qx_o) and np.array_equal(n(sx), sx_o)
    y, acc = I.gemm_i8(qx, qw, sx, sw, t(b, dev), want_acc=True)
    assert np.array_equal(n(acc), acc_o)
    assert_f32(n(y), y_o)


@pytest.mark.parametrize("M", [1, 16, 256])
def test_c2_gemm_full(dev, M):
    say(f"C2 gemm M={M} K=N=4096 (full oracle)")
    a, w, b = WL.c2_gemm(M, 0)
    qa_o, sa_o = O.quantize_rows(a)
    qw_o, sw_o = O.quantize_weight_per_channel(w)
    acc_o = O.gemm_i8_i32(qa_o, qw_o)
    y_o = O.dequant(acc_o, sa_o, sw_o, b)
    qa, sa = I.quantize_rows(t(a, dev))
    qw, sw = I.quantize_weight_per_channel(t(w, dev))
    assert np.array_equal(n(qa), qa_o) and np.array_equal(n(qw), qw_o)
    y, acc = I.gemm_i8(qa, qw, sa, sw, t(b, dev), want_acc=True)
    assert np.array_equal(n(acc), acc_o)
    assert_f32(n(y), y_o)


def test_c2_gemm_4096(dev):
    """C2 M=4096: exact on 256 sampled rows, and column/row checksums of every entry."""
    say("C2 gemm M=4096 K=N=4096 (sampled rows + checksums)")
    a, w, b = WL.c2_gemm(4096, 0)
    qa, sa = I.quantize_rows(t(a, dev))
    qw, sw = I.quantize_weight_per_channel(t(w, dev))
    y, acc = I.gemm_i8(qa, qw, sa, sw, t(b, dev), want_acc=True)
    qa_n, qw_n, acc_n, y_n = n(qa), n(qw), n(acc), n(y)
    rows = np.random.default_rng(0).choice(4096, 256, replace=False)
    qa_o, sa_o = O.quantize_rows(a[rows])
    assert np.array_equal(qa_n[rows], qa_o)
    qw_o, sw_o = O.quantize_weight_per_channel(w)
    assert np.array_equal(qw_n, qw_o)
    acc_o = O.gemm_i8_i32(qa_o, qw_o)
    assert np.array_equal(acc_n[rows], acc_o)
    assert_f32(y_n[rows], O.dequant(acc_o, sa_o, sw_o, b))
    # checksums over all rows/cols (exact in int64)
    A64, W64 = qa_n.astype(np.int64), qw_n.astype(np.int64)
    assert np.array_equal(acc_n.astype(np.int64).sum(0), A64.sum(0) @ W64.T)
    assert np.array_equal(acc_n.astype(np.int64).sum(1), A64 @ W64.sum(0))
    # the f32 epilogue of every entry from the device's own accumulators
    assert_f32(y_n, O.dequant(acc_n, n(sa), n(sw), b))


@pytest.mark.parametrize("M,N,K", [(17, 33, 16), (65, 100, 48), (100, 1, 272), (300, 130, 4096 + 16),
                                   (64, 64, 128), (129, 257, 1152), (6304, 768, 768), (2, 4100, 64),
                                   (1, 33, 8208), (3, 257, 2048), (4, 100, 1040), (1, 4096, 8192),
                                   (2, 17, 16), (4, 4096, 4096), (5, 300, 3072), (33, 70, 4096),
                                   (3900, 3300, 32)])  # the 256x256 16x16x64 tile by rule, ragged on both edges
@pytest.mark.parametrize("act", [0, 1])
def test_gemm_shapes(dev, M, N, K, act):
    say(f"gemm shape M={M} N={N} K={K} act={act}")
    rng = np.random.default_rng(M + N + K)
    qa = rng.integers(-127, 128, size=(M, K)).astype(np.int8)
    qw = rng.integers(-127, 128, size=(N, K)).astype(np.int8)
    sa = rng.uniform(1e-3, 1e-2, M).astype(np.float32)
    sw = rng.uniform(1e-3, 1e-2, N).astype(np.float32)
    b = rng.normal(size=N).astype(np.float32)
    y, acc = I.gemm_i8(t(qa, dev), t(qw, dev), t(sa, dev), t(sw, dev), t(b, dev), act=act, want_acc=True)
    acc_o = O.gemm_i8_i32(qa, qw)
    assert np.array_equal(n(acc), acc_o)
    assert_f32(n(y), O.dequant(acc_o, sa, sw, b, relu=bool(act)))


@pytest.mark.parametrize("M,N,K", [(6304 // 8, 3072, 768), (3, 200, 64), (40, 96, 256), (300, 130, 512)])
def test_gemm_gelu_and_residual_epilogue(dev, M, N, K):
    """The transformer epilogues: fc1's GELU (erf form, f32) and proj/fc2's skip addition
    (residual after the bias, before the activation), on the tiled, skinny and GEMV paths.
    Accumulators bit-exact; GELU within 1e-5 rel / 1e-6 abs of the closed form and of torch's
    own f32 gelu; the residual epilogue bit-exact."""
    say(f"gemm GELU / residual epilogue M={M} N={N} K={K}")
    rng = np.random.default_rng(M * 3 + N + K)
    qa = rng.integers(-127, 128, size=(M, K)).astype(np.int8)
    qw = rng.integers(-127, 128, size=(N, K)).astype(np.int8)
    sa = rng.uniform(1e-4, 1e-3, M).astype(np.float32)
    sw = rng.uniform(1e-4, 1e-3, N).astype(np.float32)
    b = rng.normal(size=N).astype(np.float32)
    res = rng.normal(size=(M, N)).astype(np.float32)
    acc_o = O.gemm_i8_i32(qa, qw)
    y, acc = I.gemm_i8(t(qa, dev), t(qw, dev), t(sa, dev), t(sw, dev), t(b, dev), act=I.ACT_GELU, want_acc=True)
    assert np.array_equal(n(acc), acc_o)
    pre = O.dequant(acc_o, sa, sw, b)
    np.testing.assert_allclose(n(y), O.gelu(pre), rtol=RTOL, atol=ATOL)
    np.testing.assert_allclose(n(y), n(torch.nn.functional.gelu(t(pre, dev))), rtol=RTOL, atol=ATOL)
    y2 = I.gemm_i8(t(qa, dev), t(qw, dev), t(sa, dev), t(sw, dev), t(b, dev), residual=t(res, dev))
    assert_f32(n(y2), O.dequant(acc_o, sa, sw, b, residual=res))
    y3 = I.gemm_i8(t(qa, dev), t(qw, dev), t(sa, dev), t(sw, dev), t(b, dev), act=I.ACT_RELU, residual=t(res, dev))
    assert_f32(n(y3), O.dequant(acc_o, sa, sw, b, relu=True, residual=res))


def test_gemm_no_bias_extremes(dev):
    say("gemm extremes (all +-127, K=4096)")
    K = 4096
    qa = np.full((80, K), 127, np.int8)
    qa[1::2] = -127
    qw = np.full((48, K), -127, np.int8)
    sa = np.ones(80, np.float32)
    sw = np.ones(48, np.float32)
    y, acc = I.gemm_i8(t(qa, dev), t(qw, dev), t(sa, dev), t(sw, dev), None, want_acc=True)
    assert np.array_equal(n(acc), O.gemm_i8_i32(qa, qw))


# ------------------------------------------------------------------------------ conv

CONV_CASES = [
    # N, C, H, O, k, stride, pad
    (2, 3, 32, 64, 3, 1, 1),     # ResNet stem (C padded to 16)
    (2, 64, 32, 64, 3, 1, 1),
    (2, 64, 32, 128, 3, 2, 1),
    (2, 64, 32, 128, 1, 2, 0),   # downsample 1x1 stride 2
    (2, 128, 16, 128, 3, 1, 1),
    (2, 256, 8, 512, 3, 2, 1),
    (2, 512, 4, 512, 3, 1, 1),
    (1, 16, 9, 24, 5, 2, 2),
    (2, 40, 7, 48, 1, 1, 0),     # 1x1 stride 1 (dense path), C padded to 48
    (16, 64, 32, 64, 3, 1, 1),   # C3 full batch
    (8, 3, 56, 32, 3, 2, 1),     # EfficientNet stem shape (N=32 outputs: the tall 256x64 tile)
    (4, 24, 28, 40, 1, 1, 0),    # 1x1 with C padded 24 -> 32, N=40
]


@pytest.mark.parametrize("N,C,H,O_,k,stride,pad", CONV_CASES)
def test_conv2d(dev, N, C, H, O_, k, stride, pad):
    say(f"conv N={N} C={C} H={H} O={O_} k={k} s={stride} p={pad}")
    rng = np.random.default_rng(N * C + H + O_ + k)
    x = rng.normal(size=(N, C, H, H)).astype(np.float32)
    w = (rng.normal(size=(O_, C, k, k)) * np.sqrt(2.0 / (C * k * k))).astype(np.float32)
    b = rng.normal(size=O_).astype(np.float32) * np.float32(0.1)
    OH = (H + 2 * pad - k) // stride + 1
    res = rng.normal(size=(N, O_, OH, OH)).astype(np.float32)
    cpad = I.round_up(C, 16)
    w8 = I.pack_conv_weight(t(w, dev))
    qw_o, sw_o = O.quantize_conv_weight(w, cpad)
    assert np.array_equal(n(w8.q), qw_o) and np.array_equal(n(w8.s), sw_o)
    for relu, residual in ((False, None), (True, res)):
        y_o, acc_o, sa_o, _ = O.conv2d_int8(x, w, b, stride, pad, relu, residual, cpad)
        qx, sa = I.quantize_nhwc(t(x, dev), cpad)
        assert np.array_equal(n(sa), sa_o)
        y, acc = I.conv2d_i8_nhwc(qx, sa, w8, stride, pad, t(b, dev), None if residual is None else t(residual, dev),
                                  I.ACT_RELU if relu else I.ACT_NONE, want_acc=True)
        assert np.array_equal(n(acc), acc_o)
        assert_f32(n(y), y_o)


# ---------------------------------------------------------------------------- split-K

def _gemm_c(qa, qw, sa, sw, b, out, acc, ws):
    from borch_amd import _lib
    M, K = qa.shape
    N = qw.shape[0]
    wp, wn = (None, 0) if ws is None else (ws.data_ptr(), ws.numel())
    _lib.check(_lib.lib().bq_gemm_i8(qa.data_ptr(), qw.data_ptr(), M, N, K, sa.data_ptr(), sw.data_ptr(),
                                     b.data_ptr(), None, 0, out.data_ptr(), acc.data_ptr(), wp, wn,
                                     torch.cuda.current_stream().cuda_stream))


@pytest.mark.parametrize("M,N,K", [(256, 512, 4608), (100, 200, 4112), (1024, 256, 4096), (65, 64, 8192),
                                   (130, 700, 5008), (1024, 256, 2304)])
def test_split_k_matches_unsplit(dev, M, N, K):
    """Grids of few 64x64 tiles over long K split along K (one launch, exact int32 partials,
    the last workgroup of a tile reduces; 4 to 16 splits here, ragged tiles included):
    bit-identical to the unsplit kernel (no workspace) and to the oracle, on repeated calls
    and on graph replays (the tile counters reset themselves). The last shape stays unsplit
    (too few stages): the same check holds trivially."""
    say(f"split-K M={M} N={N} K={K}")
    rng = np.random.default_rng(M * 7 + N + K)
    qa = t(rng.integers(-127, 128, size=(M, K)).astype(np.int8), dev)
    qw = t(rng.integers(-127, 128, size=(N, K)).astype(np.int8), dev)
    sa = t(rng.uniform(1e-3, 1e-2, M).astype(np.float32), dev)
    sw = t(rng.uniform(1e-3, 1e-2, N).astype(np.float32), dev)
    b = t(rng.normal(size=N).astype(np.float32), dev)
    ws = I.split_workspace(dev)
    outs = [(torch.empty(M, N, device=dev), torch.empty(M, N, dtype=torch.int32, device=dev)) for _ in range(4)]
    _gemm_c(qa, qw, sa, sw, b, *outs[0], None)
    for o in outs[1:3]:
        _gemm_c(qa, qw, sa, sw, b, *o, ws)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _gemm_c(qa, qw, sa, sw, b, *outs[3], ws)
    for _ in range(3):
        outs[3][0].zero_()
        outs[3][1].zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(outs[3][1], outs[0][1]) and torch.equal(outs[3][0], outs[0][0])
    torch.cuda.synchronize()
    for o in outs[1:]:
        assert torch.equal(o[1], outs[0][1])
        assert torch.equal(o[0], outs[0][0])
    assert np.array_equal(n(outs[0][1]), O.gemm_i8_i32(n(qa), n(qw)))
    assert int(ws[:4096].count_nonzero()) == 0  # every tile counter back at zero


def test_split_k_conv_twin_residual(dev):
    """A CIFAR ResNet stage-4 conv at batch 16 (256 pixels, K = 4608: 32 tiles split 8 ways)
    with residual, ReLU and the int8 output twin: bit-exact against the oracle."""
    say("split-K conv stage 4 with residual + twin")
    rng = np.random.default_rng(44)
    N, C, H, O_ = 16, 512, 4, 512
    x = np.maximum(rng.normal(size=(N, C, H, H)), 0).astype(np.float32)
    w = (rng.normal(size=(O_, C, 3, 3)) * np.sqrt(2.0 / (C * 9))).astype(np.float32)
    b = (rng.normal(size=O_) * 0.1).astype(np.float32)
    res = rng.normal(size=(N, O_, H, H)).astype(np.float32)
    w8 = I.pack_conv_weight(t(w, dev))
    y_o, acc_o, sa_o, _ = O.conv2d_int8(x, w, b, 1, 1, True, res, C)
    qx, sa = I.quantize_nhwc(t(x, dev), C)
    s_out_v = float(np.float32(np.abs(y_o).max()) / np.float32(127.0))
    s_out = torch.tensor([s_out_v], dtype=torch.float32, device=dev)
    y, q = I.conv2d_i8_nhwc_q(qx, sa, w8, s_out, 1, 1, t(b, dev), t(res, dev), I.ACT_RELU)
    assert_f32(n(y), y_o)
    q_o = O.quantize_with_scale(y_o.transpose(0, 2, 3, 1), np.float32(s_out_v))
    assert np.array_equal(n(q), q_o)


@pytest.mark.parametrize("N,C,H,O_,k,stride,pad,res", [(16, 64, 32, 64, 3, 1, 1, False), (16, 256, 8, 256, 3, 1, 1, True),
                                                     (16, 512, 4, 512, 3, 1, 1, True), (3, 40, 9, 50, 1, 1, 0, False),
                                                     (2, 16, 13, 24, 3, 2, 1, True),
                                                     (64, 32, 112, 96, 1, 1, 0, False)])
def test_conv_absmax_parts_feed_the_next_quantizer(dev, N, C, H, O_, k, stride, pad, res):
    """A conv's epilogue writes max |y| per output tile; the next layer's per-tensor
    quantizer takes its scale from those (no max pass) and gives the same int8 bytes and
    scale as the two-pass quantizer on the same tensor (split-K and ragged tiles included)."""
    say(f"absmax parts N={N} C={C} H={H} O={O_} k={k} s={stride} res={res}")
    rng = np.random.default_rng(N + C + H + O_)
    x = rng.normal(size=(N, C, H, H)).astype(np.float32)
    w = (rng.normal(size=(O_, C, k, k)) * np.sqrt(2.0 / (C * k * k))).astype(np.float32)
    OH = (H + 2 * pad - k) // stride + 1
    r = t(rng.normal(size=(N, O_, OH, OH)).astype(np.float32), dev) if res else None
    w8 = I.pack_conv_weight(t(w, dev))
    qx, sa = I.quantize_nhwc(t(x, dev), I.round_up(C, 16))
    from borch_amd import tune as T
    problem = (N, H, H, w8.cpad, O_, k, k, stride, pad)
    many = N * OH * OH >= 800000  # EfficientNet-B0's 112^2 expand at b64 on 128 x 128 tiles
    if many:  # the rule gives it the small-K kernel (2048 maxima); a tiled plan gives > 4096
        T.set_plan(problem, 5, 1)
    try:
        y = I.conv2d_i8_nhwc(qx, sa, w8, stride, pad, None, r, I.ACT_RELU if res else I.ACT_NONE)
    finally:
        T.set_plan(problem, 0, 0)
    parts, nparts, _ = y._bq_absmax
    assert float(parts[:nparts].max()) == float(y.abs().max())
    if many:  # the maxima are folded into the scale first
        assert nparts > 4096, nparts
    cpad = I.round_up(O_, 16)
    q1, s1 = I.quantize_nhwc(y, cpad)            # from the epilogue's partial maxima
    q1b, s1b = I.quantize_nhwc(y, cpad)          # a second consumer: the same bytes, not quantized again
    assert q1b is q1 and s1b is s1
    y2 = y.clone(memory_format=torch.channels_last)  # a copy carries no maxima
    assert getattr(y2, "_bq_absmax", None) is None
    q2, s2 = I.quantize_nhwc(y2, cpad)           # two passes
    assert torch.equal(s1, s2) and torch.equal(q1, q2)
    y.add_(0.0)                                  # modified in place: the maxima no longer apply
    q3, s3 = I.quantize_nhwc(y, cpad)
    assert torch.equal(s3, s2) and torch.equal(q3, q2)


def test_conv_maxima_count_of_a_deep_k_conv_over_many_rows(dev):
    """A 3x3 conv over 64 channels at 112^2 b64 (802816 rows, K = 576) under the rule: the
    small-K kernel does not take K > 256, so the tiled kernel runs it and writes one maximum
    per 64x64 tile, 12544 of them, and the buffer the wrapper sizes from
    bq_conv2d_absmax_parts holds exactly that many (a count made without K gave the small-K
    kernel's 4096, a buffer the launch would have overrun)."""
    from borch_amd import tune as T
    T.clear_plans()
    rng = np.random.default_rng(31)
    qx = t(rng.integers(-127, 128, size=(64, 112, 112, 64), dtype=np.int8), dev)
    sa = t(np.array([0.01], np.float32), dev)
    w8 = I.pack_conv_weight(t((rng.normal(size=(64, 64, 3, 3)) * 0.05).astype(np.float32), dev))
    y = I.conv2d_i8_nhwc(qx, sa, w8, 1, 1)
    parts, nparts, _ = y._bq_absmax
    assert nparts == 12544 and parts.numel() == 12544
    assert float(parts.max()) == float(y.abs().max())


# 3x3 / 5x5 at stride 1 / 2 take the register-blocked kernel (8 or 4 channels a thread;
# output widths that are not a multiple of its pixel block); 7x7 and the rest the generic one.
DW_CASES = [(2, 32, 16, 3, 1, 1), (2, 96, 15, 3, 2, 1), (2, 144, 14, 5, 1, 2), (2, 240, 13, 5, 2, 2),
            (1, 6, 7, 3, 1, 1), (4, 1152, 7, 5, 1, 2), (2, 12, 9, 3, 2, 1), (1, 20, 11, 5, 1, 2),
            (3, 40, 10, 3, 1, 0), (1, 16, 10, 7, 1, 3), (1, 24, 9, 5, 2, 1),
            # output rows of 14, 28 and 21 pixels: the 7-pixels-a-thread form, each filter and stride
            (2, 48, 28, 3, 2, 1), (2, 64, 28, 5, 2, 2), (1, 32, 56, 5, 2, 2), (2, 24, 28, 3, 1, 1),
            (1, 16, 21, 3, 1, 1), (2, 40, 5, 5, 1, 2),
            # 3x3 / 1 onto rows wider than 28: 7 pixels a thread where 7 divides the width (56,
            # 35), else 4, both with the row-by-row loads
            (1, 24, 56, 3, 1, 1), (1, 8, 35, 3, 1, 1), (1, 20, 33, 3, 1, 1)]


@pytest.mark.parametrize("N,C,H,k,stride,pad", DW_CASES)
def test_dwconv(dev, N, C, H, k, stride, pad):
    say(f"dwconv N={N} C={C} H={H} k={k} s={stride} p={pad}")
    rng = np.random.default_rng(N + C + H + k)
    x = rng.normal(size=(N, C, H, H)).astype(np.float32)
    w = rng.normal(size=(C, 1, k, k)).astype(np.float32)
    b = rng.normal(size=C).astype(np.float32)
    cpad = I.round_up(C, 4)
    w8 = I.pack_dw_weight(t(w, dev))
    qw_o, sw_o = O.quantize_dw_weight(np.pad(w, ((0, cpad - C), (0, 0), (0, 0), (0, 0))))
    assert np.array_equal(n(w8.q), qw_o) and np.array_equal(n(w8.s), sw_o)
    qx_o, sa_o = O.quantize_act_nhwc(x, cpad)
    acc_o = O.dwconv_i8_nhwc(qx_o, qw_o, k, k, stride, pad)
    bp = np.pad(b, (0, cpad - C))
    for act in (I.ACT_NONE, I.ACT_RELU, I.ACT_SILU):
        qx, sa = I.quantize_nhwc(t(x, dev), cpad)
        y, acc = I.dwconv_i8_nhwc(qx, sa, w8, stride, pad, t(b, dev), act, want_acc=True)
        assert np.array_equal(n(acc), acc_o)
        y_o = O.dequant(acc_o.reshape(-1, cpad), sa_o[0], sw_o, bp, relu=(act == I.ACT_RELU))
        if act == I.ACT_SILU:
            y_o = O.silu(y_o)
            np.testing.assert_allclose(n(y).transpose(0, 2, 3, 1).reshape(-1, cpad), y_o, rtol=RTOL, atol=ATOL)
        else:
            assert_f32(n(y).transpose(0, 2, 3, 1).reshape(-1, cpad), y_o)


# ------------------------------------------------------------------- weight-only W8A32

@pytest.mark.parametrize("M,N,K", [(1, 4096, 4096), (2, 17, 16), (5, 300, 1040), (8, 64, 8192), (1, 33, 2048),
                                   (64, 96, 768), (3, 4100, 4096), (4, 256, 4096), (5, 64, 3072),
                                   (8, 512, 4096), (7, 130, 2064),
                                   # the per-wave kernel's 128 KB LDS staging (M * K in (16384, 32768])
                                   (3, 130, 8192), (4, 257, 6144),
                                   # the f32-MFMA GEMV up to 16 rows
                                   (16, 4096, 4096), (12, 70, 1040),
                                   # the tiled bf16-MFMA kernel: 32 x 64 tiles (M <= 256), ragged
                                   # edges, a K tail inside a 128-deep stage, K > 8192 at small M
                                   (17, 300, 1040), (256, 4096, 4096), (100, 33, 2064), (5, 130, 8208),
                                   # 64 x 64 tiles (M > 256, fewer than 256 128 x 128 tiles)
                                   (300, 200, 2064), (1000, 520, 784),
                                   # 128 x 128 tiles, and ViT-B/16's MLP shapes at b32
                                   (1100, 4100, 1024), (6304, 3072, 768), (6304, 768, 3072)])
def test_w8a32_linear(dev, M, N, K):
    say(f"w8a32 M={M} N={N} K={K}")
    rng = np.random.default_rng(M * 7 + N + K)
    x = rng.normal(size=(M, K)).astype(np.float32)
    w = rng.normal(size=(N, K)).astype(np.float32) * np.float32(0.05)
    b = rng.normal(size=N).astype(np.float32)
    w8 = I.pack_linear_weight(t(w, dev), weight_only=True)
    qw_o, sw_o = O.quantize_weight_per_channel(w)
    assert np.array_equal(n(w8.q), qw_o) and np.array_equal(n(w8.s), sw_o)
    assert np.array_equal(n(I.dequant_weight(w8)), O.dequant_weight(qw_o, sw_o))
    y = n(I.linear_w8a32(t(x, dev), w8, t(b, dev)))
    y_o, bound = O.linear_w8a32(x, qw_o, sw_o, b)
    _check_w8a32(y, y_o, bound, x, qw_o, sw_o)


def _check_w8a32(y, y_o, bound, x, qw_o, sw_o):
    """Every output within the f32-accumulation bound of the float64 result on the same
    effective weights; the achieved error is printed relative to sum |x * w| (the scale
    the bound is proportional to) and to |y| where |y| is not tiny."""
    N = y_o.shape[-1]
    err = np.abs(y.astype(np.float64) - y_o)
    assert np.all(err <= bound + 1e-30), f"max err {err.max()} vs bound {bound[err.argmax() // N, err.argmax() % N]}"
    mag = np.abs(x.astype(np.float64)) @ np.abs(O.dequant_weight(qw_o, sw_o).astype(np.float64)).T
    big = np.abs(y_o) > 1e-3 * np.abs(y_o).max()
    say(f"  max err / sum|x*w| = {(err / np.maximum(mag, 1e-30)).max():.3g}, "
        f"max rel err (|y| > 1e-3 max) = {(err[big] / np.abs(y_o[big])).max():.3g}, "
        f"max err / bound = {(err / bound).max():.3g}")


@pytest.mark.parametrize("M", [1, 2, 3, 4])
@pytest.mark.parametrize("N,K", [(64, 16), (130, 1040), (96, 2048), (257, 4096), (33, 8192)])
def test_w8a32_decode_gemv_bit_exact(dev, M, N, K):
    """The decode GEMV (M <= 4) against the restatement of its own f32 arithmetic
    (oracle.linear_w8a32_gemv: f32(q) * s, per-lane FMA chains, the lane tree), bit for bit:
    the reference's gate for its int8 window weight (the int8 op equals the f32 op on the
    reconstructed weight, tests/browser/window_probe.html:219-233). With bias, then with a
    residual and ReLU."""
    say(f"w8a32 decode bit-exact M={M} N={N} K={K}")
    rng = np.random.default_rng(M * 31 + N + K)
    x = rng.normal(size=(M, K)).astype(np.float32)
    w = rng.normal(size=(N, K)).astype(np.float32) * np.float32(0.05)
    b = rng.normal(size=N).astype(np.float32)
    r = rng.normal(size=(M, N)).astype(np.float32)
    w8 = I.pack_linear_weight(t(w, dev), weight_only=True)
    qw, sw = n(w8.q), n(w8.s)
    y = n(I.linear_w8a32(t(x, dev), w8, t(b, dev)))
    assert np.array_equal(y, O.linear_w8a32_gemv(x, qw, sw, b))
    y2 = n(I.linear_w8a32(t(x, dev), w8, t(b, dev), I.ACT_RELU, residual=t(r, dev)))
    assert np.array_equal(y2, O.linear_w8a32_gemv(x, qw, sw, b, r, relu=True))


def test_w8a32_decode_gemv_hand_cases(dev):
    """The restatement's hand cases on the device: the fused product that keeps the 2^-24
    bit, and the lane tree's order (1 where the exact sum is 1 + 2^-23; 1 + 2^-23 where a
    left-to-right sum gives 1)."""
    K = 1024
    s = np.float32(1 + 2.0 ** -12)
    x = np.zeros((1, K), np.float32)
    x[0, 0], x[0, 1] = -1, s
    q = np.zeros((1, K), np.int8)
    q[0, :2] = 1
    w8 = I.Int8Weight(t(q, dev), t(np.array([s], np.float32), dev), K, 1, True)
    y = n(I.linear_w8a32(t(x, dev), w8))
    assert y[0, 0] == np.float32(2.0 ** -12 + 2.0 ** -24)
    x = np.zeros((1, K), np.float32)
    x[0, 0], x[0, 16], x[0, 32], x[0, 48] = 1, 2.0 ** -24, 2.0 ** -24, 2.0 ** -24
    q = np.zeros((2, K), np.int8)
    q[0, [0, 16, 32]] = 1
    q[1, [0, 32, 48]] = 1
    w8 = I.Int8Weight(t(q, dev), t(np.ones(2, np.float32), dev), K, 2, True)
    y = n(I.linear_w8a32(t(x, dev), w8))
    assert y[0, 0] == np.float32(1.0) and y[0, 1] == np.float32(1 + 2.0 ** -23)


@pytest.mark.parametrize("M", [3, 10, 100, 700])
def test_w8a32_residual(dev, M):
    """The residual is added after the bias and before the activation (the W8A8 epilogue's
    order), in every W8A32 kernel: the result equals the plain output plus the residual,
    then ReLU, one f32 rounding each."""
    say(f"w8a32 residual M={M}")
    rng = np.random.default_rng(60 + M)
    N, K = 136, 1040
    x = rng.normal(size=(M, K)).astype(np.float32)
    w = rng.normal(size=(N, K)).astype(np.float32) * np.float32(0.05)
    b = rng.normal(size=N).astype(np.float32)
    r = rng.normal(size=(M, N)).astype(np.float32)
    w8 = I.pack_linear_weight(t(w, dev), weight_only=True)
    plain = n(I.linear_w8a32(t(x, dev), w8, t(b, dev)))
    got = n(I.linear_w8a32(t(x, dev), w8, t(b, dev), I.ACT_RELU, residual=t(r, dev)))
    want = (plain + r).astype(np.float32)
    assert np.array_equal(got, np.where(want > 0, want, np.float32(0)))


@pytest.mark.parametrize("act", [I.ACT_RELU, I.ACT_GELU, I.ACT_SILU])
@pytest.mark.parametrize("M", [1, 3, 6, 40])
def test_w8a32_activation(dev, M, act):
    """The W8A32 epilogue's activation after the bias: ReLU exactly on the kernel's own f32
    sum, SiLU / GELU within 1e-5 rel / 1e-6 abs of the closed form of that sum."""
    say(f"w8a32 act={act} M={M}")
    rng = np.random.default_rng(40 + M + act)
    N, K = 200, 1024
    x = rng.normal(size=(M, K)).astype(np.float32)
    w = rng.normal(size=(N, K)).astype(np.float32) * np.float32(0.05)
    b = rng.normal(size=N).astype(np.float32)
    w8 = I.pack_linear_weight(t(w, dev), weight_only=True)
    plain = n(I.linear_w8a32(t(x, dev), w8, t(b, dev)))
    got = n(I.linear_w8a32(t(x, dev), w8, t(b, dev), act))
    if act == I.ACT_RELU:
        assert np.array_equal(got, np.where(plain > 0, plain, np.float32(0)))
    else:
        want = O.silu(plain) if act == I.ACT_SILU else O.gelu(plain)
        np.testing.assert_allclose(got, want, rtol=RTOL, atol=ATOL)


def test_w8a32_module(dev):
    say("w8a32 via quantize_for_int8(weight_only=True)")
    import borch_amd as bt
    torch.manual_seed(0)
    lin = bt.nn.Linear(768, 3072).to(dev)
    assert bt.quantize_for_int8(lin, weight_only=True) == 1
    for rows in (1, 64):
        x = torch.randn(rows, 768, device=dev)
        y = n(lin(x))
        y_o, bound = O.linear_w8a32(n(x), n(lin.int8.q), n(lin.int8.s), n(lin.bias))
        assert np.all(np.abs(y - y_o) <= bound)
    # the skip connection of a transformer layer (LinearAdd) rides in the W8A32 epilogue
    from borch_amd.nn.intrinsic import LinearAdd
    fused = LinearAdd(lin)
    x = torch.randn(2, 33, 768, device=dev)
    r = torch.randn(2, 33, 3072, device=dev)
    y = n(fused(x, r))
    y_o, bound = O.linear_w8a32(n(x).reshape(-1, 768), n(lin.int8.q), n(lin.int8.s), n(lin.bias))
    y_o = y_o.reshape(2, 33, 3072) + n(r).astype(np.float64)
    assert np.all(np.abs(y - y_o) <= bound.reshape(2, 33, 3072) + 2.0 ** -24 * np.abs(y_o))


def _false_ties(count=512, seed=21):
    """(v, s) pairs whose correctly rounded f32 quotient is exactly k + 0.5 while the exact
    quotient is not a tie (plus true ties), found by search and checked with rationals."""
    from fractions import Fraction
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < count:
        s = np.float32(rng.uniform(0.01, 1.0))
        k = int(rng.integers(-126, 126))
        v0 = np.float32((k + 0.5) * float(s))
        for d in (-2, -1, 0, 1, 2):
            v = v0
            for _ in range(abs(d)):
                v = np.nextafter(v, np.float32(np.inf if d > 0 else -np.inf))
            if np.float32(v) / s == np.float32(k + 0.5):
                exact = Fraction(float(v)) / Fraction(float(s))
                out.append((v, s, exact == Fraction(2 * k + 1, 2)))
    return out


def test_quantize_false_ties(dev):
    """Rows built from such pairs: each row's scale is forced to s by a peak element 127·s."""
    say("quantize false ties (f32 quotient exactly k+0.5, exact quotient not)")
    pairs = _false_ties()
    rows = []
    for v, s, _ in pairs[:256]:
        peak = np.float32(127) * s
        if np.float32(peak) / np.float32(127) != s:
            continue
        rows.append(np.array([peak, v, -v, 0.0], np.float32))
    x = np.stack(rows)
    assert len(rows) > 50
    q, s = I.quantize_rows(t(x, dev))
    qo, so = O.quantize_rows(x)
    assert np.array_equal(n(s), so)
    assert np.array_equal(n(q), qo)
    n_false = sum(1 for _, _, tie in pairs if not tie)
    say(f"  {len(rows)} rows, {n_false} of {len(pairs)} pairs are false ties")


@pytest.mark.gpu
def test_probe_stream_read_folds_every_byte(dev):
    """The read-floor probe bench.py times reads every 16-byte chunk once: its per-workgroup
    XOR fold equals the host's fold of the same bytes, for each load depth."""
    import ctypes
    lib = ctypes.CDLL(str(ROOT / "bench_probe" / "libbqprobe.so"))
    lib.bqp_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    g = torch.Generator().manual_seed(5)
    n16 = 3 * 2048 + 37  # a ragged last workgroup for every depth
    words = torch.randint(-2**31, 2**31 - 1, (n16 * 4,), dtype=torch.int64, generator=g).to(torch.int32)
    src = words.to(dev)
    st = torch.cuda.current_stream().cuda_stream
    for ch in (1, 2, 4, 8):
        per = 256 * ch
        nblk = (n16 + per - 1) // per
        sink = torch.zeros(nblk, dtype=torch.int32, device=dev)
        assert lib.bqp_stream_read(src.data_ptr(), n16 * 16, ch, sink.data_ptr(), st) == 0
        w = words.view(n16, 4).numpy()
        chunk_x = np.bitwise_xor.reduce(w, axis=1)
        pad = np.zeros(nblk * per, dtype=np.int32)
        pad[:n16] = chunk_x
        want = np.bitwise_xor.reduce(pad.reshape(nblk, per), axis=1)
        np.testing.assert_array_equal(sink.cpu().numpy(), want)


# ------------------------------------------------------------ kernel choice by measurement

@pytest.fixture
def no_plans():
    from borch_amd import tune as T
    T.clear_plans()
    yield T
    T.clear_plans()


@pytest.mark.parametrize("M,N,K,res,act", [(6304, 768, 768, True, 0), (300, 200, 4112, False, 1),
                                           (1000, 40, 96, False, 2), (257, 2304, 768, True, 3)])
def test_every_gemm_plan_gives_the_same_result(dev, no_plans, M, N, K, res, act):
    """Every (configuration, K split) the library offers for a dense GEMM gives the rule's
    output and int32 accumulators bit for bit (bias, residual and activation included)."""
    T = no_plans
    say(f"plans gemm M={M} N={N} K={K}")
    rng = np.random.default_rng(M + N + K)
    qa = t(rng.integers(-127, 128, size=(M, K)).astype(np.int8), dev)
    qw = t(rng.integers(-127, 128, size=(N, K)).astype(np.int8), dev)
    sa = t(rng.uniform(1e-4, 1e-3, M).astype(np.float32), dev)
    sw = t(rng.uniform(1e-4, 1e-3, N).astype(np.float32), dev)
    b = t(rng.normal(size=N).astype(np.float32), dev)
    r = t(rng.normal(size=(M, N)).astype(np.float32), dev) if res else None
    I.split_workspace(dev)
    want, want_acc = I.gemm_i8(qa, qw, sa, sw, b, act, want_acc=True, residual=r)
    cands = T.candidates((M, N, K))
    assert len(cands) >= 8
    for cfg, split in cands:
        T.set_plan((M, N, K), cfg, split)
        got, acc = I.gemm_i8(qa, qw, sa, sw, b, act, want_acc=True, residual=r)
        assert torch.equal(acc, want_acc), (cfg, split)
        assert torch.equal(got, want), (cfg, split)


@pytest.mark.parametrize("N,C,H,O_,k,stride,pad,res", [(16, 64, 32, 64, 3, 1, 1, True), (16, 512, 4, 512, 3, 1, 1, True),
                                                     (4, 32, 28, 240, 1, 1, 0, False), (2, 48, 15, 96, 5, 2, 2, False)])
def test_every_conv_plan_gives_the_same_result(dev, no_plans, N, C, H, O_, k, stride, pad, res):
    """Every candidate for a conv gives the rule's f32 output, int32 accumulators, int8 twin
    and per-tensor maximum bit for bit (its per-tile maxima follow the plan's tile count)."""
    T = no_plans
    say(f"plans conv N={N} C={C} H={H} O={O_} k={k} s={stride}")
    rng = np.random.default_rng(N * C + H + O_)
    x = rng.normal(size=(N, C, H, H)).astype(np.float32)
    w = (rng.normal(size=(O_, C, k, k)) * np.sqrt(2.0 / (C * k * k))).astype(np.float32)
    b = t((rng.normal(size=O_) * 0.1).astype(np.float32), dev)
    OH = (H + 2 * pad - k) // stride + 1
    r = t(rng.normal(size=(N, O_, OH, OH)).astype(np.float32), dev) if res else None
    w8 = I.pack_conv_weight(t(w, dev))
    qx, sa = I.quantize_nhwc(t(x, dev), w8.cpad)
    s_out = torch.tensor([0.05], dtype=torch.float32, device=dev)
    I.split_workspace(dev)
    want, want_acc = I.conv2d_i8_nhwc(qx, sa, w8, stride, pad, b, r, I.ACT_RELU, want_acc=True)
    want_max = want._bq_absmax[0][: want._bq_absmax[1]].max()
    _, want_q = I.conv2d_i8_nhwc_q(qx, sa, w8, s_out, stride, pad, b, r, I.ACT_RELU)
    problem = (N, H, H, w8.cpad, O_, k, k, stride, pad)
    cands = T.candidates(problem)
    assert len(cands) >= 8
    for cfg, split in cands:
        T.set_plan(problem, cfg, split)
        got, acc = I.conv2d_i8_nhwc(qx, sa, w8, stride, pad, b, r, I.ACT_RELU, want_acc=True)
        assert torch.equal(acc, want_acc), (cfg, split)
        assert torch.equal(got, want), (cfg, split)
        parts, nparts, _ = got._bq_absmax
        assert torch.equal(parts[:nparts].max(), want_max), (cfg, split)
        _, q = I.conv2d_i8_nhwc_q(qx, sa, w8, s_out, stride, pad, b, r, I.ACT_RELU)
        assert torch.equal(q, want_q), (cfg, split)


def test_phase_stamps_are_ordered_and_output_unchanged(dev):
    """bq_gemm_i8_phases: the output is bq_gemm_i8's bit for bit, one stamp record per
    workgroup, entry <= end of main loop <= last store, an XCC id below 8."""
    from borch_amd import _lib as L
    M, N, K = 1024, 768, 1040
    rng = np.random.default_rng(17)
    qa = t(rng.integers(-127, 128, size=(M, K)).astype(np.int8), dev)
    qw = t(rng.integers(-127, 128, size=(N, K)).astype(np.int8), dev)
    sa = t(rng.uniform(1e-4, 1e-3, M).astype(np.float32), dev)
    sw = t(rng.uniform(1e-4, 1e-3, N).astype(np.float32), dev)
    b = t(rng.normal(size=N).astype(np.float32), dev)
    out = torch.empty((M, N), dtype=torch.float32, device=dev)
    st = torch.zeros(4 * 4096, dtype=torch.int64, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    assert L.lib().bq_gemm_i8_phases(qa.data_ptr(), qw.data_ptr(), M, N, K, sa.data_ptr(), sw.data_ptr(),
                                     b.data_ptr(), out.data_ptr(), st.data_ptr(), 4, stream) == L.BQ_ERR_ARG
    nwg = L.lib().bq_gemm_i8_phases(qa.data_ptr(), qw.data_ptr(), M, N, K, sa.data_ptr(), sw.data_ptr(),
                                    b.data_ptr(), out.data_ptr(), st.data_ptr(), st.numel(), stream)
    assert nwg > 0
    assert torch.equal(out, I.gemm_i8(qa, qw, sa, sw, b))
    v = st[: 4 * nwg].view(nwg, 4).cpu().numpy()
    assert np.all(v[:, 0] > 0) and np.all(v[:, 0] <= v[:, 1]) and np.all(v[:, 1] <= v[:, 2])
    assert np.all(((v[:, 3] >> 6) & 15) < 8)
    assert not st[4 * nwg:].any()


@pytest.mark.parametrize("M", [1, 3, 4, 5, 6, 7, 8])
@pytest.mark.parametrize("N,K", [(4096, 4096), (300, 1040), (70, 8192)])
def test_decode_kernels_give_the_same_result(dev, no_plans, M, N, K):
    """Both decode kernels (the v_dot4 wave-reduction GEMV and the weight-streaming MFMA
    kernel), each forced through the plan API, give the oracle's int32 sums and f32 outputs
    bit for bit; the GEMV is offered only where it takes K."""
    T = no_plans
    say(f"decode kernels M={M} N={N} K={K}")
    rng = np.random.default_rng(M * 11 + N + K)
    qa_o = rng.integers(-127, 128, size=(M, K)).astype(np.int8)
    qw_o = rng.integers(-127, 128, size=(N, K)).astype(np.int8)
    sa_o = rng.uniform(1e-4, 1e-3, M).astype(np.float32)
    sw_o = rng.uniform(1e-4, 1e-3, N).astype(np.float32)
    b_o = rng.normal(size=N).astype(np.float32)
    acc_o = O.gemm_i8_i32(qa_o, qw_o)
    y_o = O.dequant(acc_o, sa_o, sw_o, b_o, relu=True)
    cands = T.candidates((M, N, K))
    want = {I.CFG_GEMV, I.CFG_SKINNY} if K <= (8192 if M <= 4 else 4096) else {I.CFG_SKINNY}
    assert {c for c, _ in cands} == want and all(sp == 1 for _, sp in cands)
    assert cands[0][0] == (I.CFG_GEMV if I.CFG_GEMV in want else I.CFG_SKINNY)  # the rule: the GEMV where it fits
    for cfg, sp in cands:
        T.set_plan((M, N, K), cfg, sp)
        y, acc = I.gemm_i8(t(qa_o, dev), t(qw_o, dev), t(sa_o, dev), t(sw_o, dev), t(b_o, dev), I.ACT_RELU,
                           want_acc=True)
        assert np.array_equal(n(acc), acc_o), cfg
        assert_f32(n(y), y_o)


@pytest.mark.parametrize("M,N,K", [(6304, 768, 768), (1000, 520, 784), (300, 200, 4112), (257, 2304, 768),
                                   (4096, 4096, 512)])
def test_regression_fast_path_stores_equal_general_path(dev, no_plans, M, N, K):
    """Regression test for the 16-byte buffer-store hazard: on every tile configuration the
    epilogue's fast path (no int32 output: buffer stores with the whole row offset in the
    VGPR, written through) equals the general path (int32 output requested) bit for bit,
    with bias and residual, dense and conv. With part of the row offset in the SGPR offset
    those stores once wrote wrong values to about 1% of the rows, so a toolchain that
    folds a uniform offset back into the SGPR fails here."""
    T = no_plans
    say(f"fast path vs general path M={M} N={N} K={K}")
    rng = np.random.default_rng(M * 3 + N + K)
    qa = t(rng.integers(-127, 128, size=(M, K)).astype(np.int8), dev)
    qw = t(rng.integers(-127, 128, size=(N, K)).astype(np.int8), dev)
    sa = t(rng.uniform(1e-4, 1e-3, M).astype(np.float32), dev)
    sw = t(rng.uniform(1e-4, 1e-3, N).astype(np.float32), dev)
    b = t(rng.normal(size=N).astype(np.float32), dev)
    r = t(rng.normal(size=(M, N)).astype(np.float32), dev)
    I.split_workspace(dev)
    cands = T.candidates((M, N, K))
    for cfg, split in cands:
        T.set_plan((M, N, K), cfg, split)
        fast = I.gemm_i8(qa, qw, sa, sw, b, I.ACT_RELU, residual=r)
        general, _ = I.gemm_i8(qa, qw, sa, sw, b, I.ACT_RELU, want_acc=True, residual=r)
        assert torch.equal(fast, general), (cfg, split, int((fast != general).any(1).sum()))
    # and a conv: the implicit-GEMM loader's configurations, a ragged last row tile
    T.clear_plans()
    Nn, C, H, O_ = 3, 64, 19, 128
    x = rng.normal(size=(Nn, C, H, H)).astype(np.float32)
    w8 = I.pack_conv_weight(t((rng.normal(size=(O_, C, 3, 3)) * 0.05).astype(np.float32), dev))
    qx, sx = I.quantize_nhwc(t(x, dev), w8.cpad)
    rr = t(rng.normal(size=(Nn, O_, H, H)).astype(np.float32), dev)
    problem = (Nn, H, H, w8.cpad, O_, 3, 3, 1, 1)
    for cfg, split in T.candidates(problem):
        T.set_plan(problem, cfg, split)
        fast = I.conv2d_i8_nhwc(qx, sx, w8, 1, 1, b[:O_].contiguous(), rr, I.ACT_RELU)
        general, _ = I.conv2d_i8_nhwc(qx, sx, w8, 1, 1, b[:O_].contiguous(), rr, I.ACT_RELU, want_acc=True)
        assert torch.equal(fast, general), (cfg, split)


@pytest.mark.parametrize("N,C,H,O_,stride", [(16, 64, 32, 128, 2), (16, 128, 16, 256, 2), (16, 256, 8, 512, 2),
                                             (3, 32, 9, 48, 2), (2, 16, 7, 16, 1)])
@pytest.mark.parametrize("twin", [False, True])
def test_conv_pair_matches_two_calls(dev, no_plans, N, C, H, O_, stride, twin):
    """A residual block's first conv (3x3) and its shortcut (1x1) in one launch
    (bq_conv2d_i8_nhwc_pair) give each conv's own call bit for bit: f32 outputs, the first's
    int8 twin (calibrated) or per-tile maxima (dynamic), under every plan of the first conv
    (paired kernels, the split first conv, and the configurations that run two launches).
    The last case's shortcut is a 1x1 stride-1 conv (the dense loader): two launches."""
    T = no_plans
    say(f"pair N={N} C={C} H={H} O={O_} s={stride} twin={twin}")
    rng = np.random.default_rng(N * C + H + O_ + stride)
    x = rng.normal(size=(N, C, H, H)).astype(np.float32)
    w1 = (rng.normal(size=(O_, C, 3, 3)) * np.sqrt(2.0 / (C * 9))).astype(np.float32)
    w2 = (rng.normal(size=(O_, C, 1, 1)) * np.sqrt(2.0 / C)).astype(np.float32)
    b1 = t((rng.normal(size=O_) * 0.1).astype(np.float32), dev)
    b2 = t((rng.normal(size=O_) * 0.1).astype(np.float32), dev)
    p1, p2 = I.pack_conv_weight(t(w1, dev)), I.pack_conv_weight(t(w2, dev))
    qx, sa = I.quantize_nhwc(t(x, dev), p1.cpad)
    s_out = torch.tensor([0.05], dtype=torch.float32, device=dev) if twin else None
    I.split_workspace(dev)
    problem = (N, H, H, p1.cpad, O_, 3, 3, stride, 1)
    for cfg, split in T.candidates(problem):
        T.set_plan(problem, cfg, split)
        if twin:
            want1, want_q = I.conv2d_i8_nhwc_q(qx, sa, p1, s_out, stride, 1, b1, None, I.ACT_RELU)
        else:
            want1, want_q = I.conv2d_i8_nhwc(qx, sa, p1, stride, 1, b1, None, I.ACT_RELU), None
        want2 = I.conv2d_i8_nhwc(qx, sa, p2, stride, 0, b2)
        (got1, q), (got2, q2) = I.conv2d_pair_i8_nhwc(
            qx, sa, I.PairConv(p1, stride, 1, b1, I.ACT_RELU, s_out, amax=not twin), I.PairConv(p2, stride, 0, b2))
        assert q2 is None
        assert torch.equal(got1, want1), (cfg, split)
        assert torch.equal(got2, want2), (cfg, split)
        if twin:
            assert torch.equal(q, want_q), (cfg, split)
        else:
            parts, nparts, _ = got1._bq_absmax
            wparts, wn, _ = want1._bq_absmax
            assert nparts == wn and torch.equal(parts[:nparts], wparts[:wn]), (cfg, split)


def test_conv_pair_rejects(dev):
    """Only the first conv of a pair writes per-tile maxima; a twin needs O % 16 == 0."""
    rng = np.random.default_rng(5)
    p1 = I.pack_conv_weight(t(rng.normal(size=(24, 16, 3, 3)).astype(np.float32), dev))
    p2 = I.pack_conv_weight(t(rng.normal(size=(24, 16, 1, 1)).astype(np.float32), dev))
    qx, sa = I.quantize_nhwc(t(rng.normal(size=(2, 16, 8, 8)).astype(np.float32), dev), 16)
    with pytest.raises(ValueError, match="first conv"):
        I.conv2d_pair_i8_nhwc(qx, sa, I.PairConv(p1, 2, 1), I.PairConv(p2, 2, 0, amax=True))
    s_out = torch.tensor([0.05], dtype=torch.float32, device=dev)
    with pytest.raises(ValueError, match="O % 16"):
        I.conv2d_pair_i8_nhwc(qx, sa, I.PairConv(p1, 2, 1, s_out=s_out), I.PairConv(p2, 2, 0))


# ------------------------------------------------- f32 attention beside the path (ViT)

@pytest.mark.parametrize("B,T,H,scale", [(2, 197, 12, 1.0), (1, 1, 1, 1.0), (3, 16, 2, 1.0), (2, 17, 3, 1.0),
                                         (1, 64, 4, 1.0), (1, 100, 2, 1.0), (2, 128, 1, 1.0), (1, 129, 2, 1.0),
                                         (1, 256, 2, 1.0), (2, 197, 2, 6.0)])
def test_attention_f32(dev, B, T, H, scale):
    """bq_attention_f32 against the float64 restatement of scaled_dot_product_attention
    (borch/_nn.py:2143-2170: scores = (q @ k^T) / sqrt(64), softmax exp(s - max) / sum,
    then @ v), on q, k, v read from a packed [B, T, 3, H, 64] projection output: within the
    f32 bound (1e-5 relative / 2e-6 absolute of the output's scale), across ragged T (the
    masked key padding, the partial query blocks) and with scores of +-50 (scale 6)."""
    say(f"attention B={B} T={T} H={H} scale={scale}")
    rng = np.random.default_rng(B * 1000 + T * 10 + H)
    qkv = (rng.normal(size=(B, T, 3, H, 64)) * scale).astype(np.float32)
    from oracle import models as OM
    got = n(I.attention_f32(t(qkv.reshape(B, T, 3 * H * 64), dev), H))
    want = OM.attention_qkv(qkv.reshape(B, T, 3 * H * 64), H)
    err = np.abs(got - want).max()
    say(f"  max |err| {err:.3g} (output scale {np.abs(want).max():.3g})")
    assert err <= 1e-5 * np.abs(want).max() + 2e-6
    # torch's own f32 attention on the same operands: within the same bound of float64, so
    # the two f32 results agree to twice it
    qt, kt, vt = (t(np.ascontiguousarray(qkv[:, :, i].transpose(0, 2, 1, 3)), dev) for i in range(3))
    ref = n(torch.nn.functional.scaled_dot_product_attention(qt, kt, vt).transpose(1, 2).reshape(B, T, H * 64))
    say(f"  torch f32: max |err| {np.abs(ref - want).max():.3g}")
    assert np.abs(got - ref).max() <= 2e-5 * np.abs(want).max() + 4e-6


@pytest.mark.parametrize("N,C,H,O_,bias", [(16, 512, 4, 10, True), (3, 64, 7, 100, False), (1, 16384, 1, 4, True),
                                          (5, 1000, 3, 65, True)])
def test_avgpool_linear(dev, N, C, H, O_, bias):
    """bq_avgpool_linear_f32 (the CIFAR ResNet-18 head: mean over H, W, then the f32 Linear)
    against float64, within the f32 bound of its two sums (1e-5 of sum |pooled * w| + 1e-6)."""
    say(f"avgpool+linear N={N} C={C} H={H} O={O_}")
    rng = np.random.default_rng(N + C + O_)
    x = rng.normal(size=(N, C, H, H)).astype(np.float32)
    w = (rng.normal(size=(O_, C)) / np.sqrt(C)).astype(np.float32)
    b = rng.normal(size=O_).astype(np.float32) if bias else None
    xt = t(x, dev).contiguous(memory_format=torch.channels_last)
    from oracle import models as OM
    got = n(I.avgpool_linear(xt, t(w, dev), None if b is None else t(b, dev)))
    want, scale = OM.avgpool_linear(x, w, b)
    assert np.all(np.abs(got - want) <= 1e-5 * scale + 1e-6)


# ------------------------------------------------- per-tensor activation scale (matmulInt8)

@pytest.mark.parametrize("M,N,K", [(1, 96, 512), (3, 300, 1040), (16, 512, 512), (40, 200, 768), (256, 512, 4608),
                                   (1000, 520, 784), (4096, 1024, 512)])
def test_gemm_per_tensor_activation_scale(dev, M, N, K):
    """bq_gemm_i8 with act | BQ_SCALE_A_PER_TENSOR: one activation scale sA[0] for every row,
    the reference's matmulInt8(scaled) arithmetic fround(fround(fround(acc*s0)*s[n])+b[n])
    (kernels.ts:1818-1827; kernel_bench.html:321), after a per-tensor quantize
    (bq_quantize_tensor). int32 and f32 bit-exact against the oracle, in every kernel family
    (GEMV, skinny, tiled, split-K), and through nn.Linear(per_tensor)."""
    say(f"per-tensor activation scale M={M} N={N} K={K}")
    rng = np.random.default_rng(M + 3 * N + K)
    x = rng.normal(size=(M, K)).astype(np.float32)
    w = (rng.normal(size=(N, K)) / np.sqrt(K)).astype(np.float32)
    b = (0.1 * rng.normal(size=N)).astype(np.float32)
    qa, sa = I.quantize_tensor(t(x, dev))
    qa_o, sa_o = O.quantize_tensor(x)
    assert np.array_equal(n(qa), qa_o) and n(sa)[0] == sa_o[0]
    qw, sw = I.quantize_weight_per_channel(t(w, dev))
    out, acc = I.gemm_i8(qa, qw, sa, sw, t(b, dev), want_acc=True)
    acc_o = O.gemm_i8_i32(qa_o, n(qw))
    assert np.array_equal(n(acc), acc_o)
    assert_f32(n(out), O.dequant(acc_o, sa_o[0], n(sw), b))
    import borch_amd as bt
    lin = bt.nn.Linear(K, N).to(dev)
    with torch.no_grad():
        lin.weight.copy_(t(w, dev))
        lin.bias.copy_(t(b, dev))
    assert bt.quantize_for_int8(lin, per_tensor=True) == 1 and lin.int8.per_tensor
    assert_f32(n(lin(t(x, dev))), O.dequant(acc_o, sa_o[0], n(sw), b))


@pytest.mark.parametrize("size", [1024, 2048])
def test_mmi8_lcg_procedure(dev, size):
    """The reference's exactness gate mmi8 (kernel_bench.html:294-337) at its published
    shapes: LCG int8 operands in [-8, 8), the raw int32 result held to the exact integer
    reference on EVERY entry, then the dequantising store (per-tensor activation scale,
    per-channel weight scales and bias, all in [0.5, 1.5) / N(0, 1)) bit for bit."""
    say(f"mmi8 {size}^3 on the LCG operands")
    from borch_amd import workloads as WL
    A, W = WL.mmi8_operands(size, size, size)
    rng = np.random.default_rng(size)
    s0 = np.float32(0.5 + rng.random())
    sw = (0.5 + rng.random(size)).astype(np.float32)
    b = rng.normal(size=size).astype(np.float32)
    out, acc = I.gemm_i8(t(A, dev), t(W, dev), torch.tensor([s0], device=dev), t(sw, dev), t(b, dev), want_acc=True)
    ref = O.gemm_i8_i32(A, W)
    wrong = int((n(acc) != ref).sum())
    assert wrong == 0, f"{wrong} of {size * size} entries differ from the int32 reference"
    assert_f32(n(out), O.dequant(ref, s0, sw, b))


# ------------------------------------- the dynamic-quant Linear in one call (bq_linear_i8)

@pytest.mark.parametrize("M,N,K", [(1, 4096, 4096), (2, 300, 1040), (3, 129, 8192), (4, 64, 16), (1, 33, 2064),
                                   (4, 4100, 4096), (5, 256, 1024), (17, 96, 784), (300, 520, 4608)])
@pytest.mark.parametrize("extras", [False, True])
def test_linear_rows_fused_quantize(dev, M, N, K, extras):
    """bq_linear_i8: for M <= 4 the per-row quantization runs inside the GEMV. Its quantized
    rows and scales equal the oracle's (bytes and bits), its int32 / f32 result equals
    bq_quantize_rows + bq_gemm_i8 bit for bit and the oracle's epilogue, with a residual and
    an activation too; larger M quantizes into the caller's buffers, then the GEMM."""
    say(f"bq_linear_i8 M={M} N={N} K={K} extras={extras}")
    rng = np.random.default_rng(M * 11 + N + K)
    x = rng.normal(size=(M, K)).astype(np.float32)
    x[0, : min(K, 8)] = [2.5, -2.5, 0.0, 1e-30, -7.25, 3.0, 0.5, -0.5][: min(K, 8)]
    w = (rng.normal(size=(N, K)) / np.sqrt(K)).astype(np.float32)
    b = (0.1 * rng.normal(size=N)).astype(np.float32)
    r = rng.normal(size=(M, N)).astype(np.float32) if extras else None
    act = I.ACT_RELU if extras else I.ACT_NONE
    w8 = I.pack_linear_weight(t(w, dev))
    out, q, s = I.linear_rows(t(x, dev), w8, t(b, dev), act, None if r is None else t(r, dev), want_q=True)
    q_o, s_o = O.quantize_rows(x)
    assert np.array_equal(n(q), q_o) and np.array_equal(n(s), s_o)
    qa, sa = I.quantize_rows(t(x, dev))
    want = I.gemm_i8(qa, w8.q, sa, w8.s, t(b, dev), act, residual=None if r is None else t(r, dev))
    assert torch.equal(out, want)
    y_o = O.dequant(O.gemm_i8_i32(q_o, n(w8.q)), s_o, n(w8.s), b, act == I.ACT_RELU, r)
    assert_f32(n(out), y_o)
    if M <= 4:  # without the optional quantized-row outputs: the same result
        assert torch.equal(I.linear_rows(t(x, dev), w8, t(b, dev), act, None if r is None else t(r, dev)), out)


@pytest.mark.parametrize("shape,cpad", [((2, 3, 17, 19), 16), ((1, 5, 8, 8), 16), ((3, 20, 5, 7), 32), ((4, 3, 32, 32), 16)])
def test_quantize_nchw_input(dev, shape, cpad):
    """An NCHW input quantized into padded NHWC channels straight from its planes
    (bq_quantize_nchw / bq_quantize_nchw_scaled): the same bytes and scale as the
    channels-last path on the permuted tensor, and as the oracle."""
    say(f"quantize NCHW input {shape} -> cpad {cpad}")
    rng = np.random.default_rng(sum(shape) + cpad)
    x = rng.normal(size=shape).astype(np.float32) * 3
    xt = t(x, dev)
    assert xt.is_contiguous() and not xt.is_contiguous(memory_format=torch.channels_last)
    q1, s1 = I.quantize_nhwc(xt, cpad)
    q2, s2 = I.quantize_nhwc(xt.contiguous(memory_format=torch.channels_last), cpad)
    assert n(s1).tobytes() == n(s2).tobytes()
    np.testing.assert_array_equal(n(q1), n(q2))
    q_o, s_o = O.quantize_act_nhwc(x, cpad)
    np.testing.assert_array_equal(n(q1), q_o)
    assert np.float32(n(s1)[0]) == np.float32(s_o)
    # calibrated: a given scale, one pass
    sc = torch.tensor([0.0173], device=dev)
    np.testing.assert_array_equal(n(I.quantize_nhwc_scaled(xt, sc, cpad)),
                                  n(I.quantize_nhwc_scaled(xt.contiguous(memory_format=torch.channels_last), sc, cpad)))
