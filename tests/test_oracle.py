"""Pins the CPU oracle (oracle/quant.py) against the reference's golden values, exact
rational arithmetic, brute force on tiny inputs and closed forms — never against a
retyped copy of its own formula."""
import json
import struct
from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest

from oracle import quant as O

GOLD = json.loads((Path(__file__).parent / "golden" / "ref_fake_quantize.json").read_text())["cases"]


def f32(v):
    return struct.unpack("f", struct.pack("f", v))[0]


# -------------------------------------------------------------- reference goldens

def _fake_quant(x, scale, zp, qmin, qmax):
    """round → +zp → clamp → dequant, built on the oracle's rounding core."""
    r = O.round_quotient(np.asarray(x, np.float32), np.asarray(scale, np.float32))
    q = np.clip(r + zp, qmin, qmax)
    return ((q - zp) * np.asarray(scale, np.float64)).astype(np.float32)


@pytest.mark.parametrize("key", ["top::fake_quantize(per_tensor)", "top::fake_quantize(zp=2)"])
def test_reference_golden_per_tensor(key):
    c = GOLD[key]
    i = c["input"]
    got = _fake_quant(i["x"], i["scale"], i["zero_point"], i["qmin"], i["qmax"])
    assert got.tolist() == c["expected"]["values"]


def test_reference_golden_per_channel():
    c = GOLD["top::fake_quantize(per_channel)"]
    i = c["input"]
    x = np.asarray(i["x"], np.float32)
    s = np.asarray(i["scale"], np.float32).reshape(-1, 1)
    z = np.asarray(i["zero_point"], np.float64).reshape(-1, 1)
    got = _fake_quant(x, s, z, i["qmin"], i["qmax"])
    assert got.reshape(-1).tolist() == c["expected"]["values"]


def test_reference_golden_grad_mask():
    """The straight-through mask (1 inside the range) agrees with the oracle's rounding."""
    c = GOLD["top::grad::fake_quantize"]
    i = c["input"]
    r = O.round_quotient(np.asarray(i["x"], np.float32), np.float32(i["scale"])) + i["zero_point"]
    mask = ((r >= i["qmin"]) & (r <= i["qmax"])).astype(np.float32)
    assert mask.tolist() == c["expected"]["values"]


# ------------------------------------------------------------- exact rational checks

def _exact_round(v, s):
    """Round-half-even of the exact rational v/s (Fraction.__round__ is half-even)."""
    if s == 0:
        return 0
    return max(-127, min(127, round(Fraction(v) / Fraction(s))))


def test_round_quotient_matches_exact_rationals():
    rng = np.random.default_rng(1)
    v = rng.normal(size=4000).astype(np.float32) * np.float32(3)
    s = rng.uniform(1e-3, 0.2, size=4000).astype(np.float32)
    got = O.quantize_with_scale(v, s)
    want = [_exact_round(float(a), float(b)) for a, b in zip(v, s)]
    assert got.tolist() == want


def test_exact_ties_round_half_even():
    # s = 1/2, 1/4, 1 are exact; k + 0.5 ties must go to the even neighbour.
    for s in (0.5, 0.25, 1.0, 2.0**-7):
        ks = np.arange(-126, 126)
        v = ((ks + 0.5) * s).astype(np.float32)
        assert np.all((v.astype(np.float64) / s) == ks + 0.5)  # true ties
        got = O.quantize_with_scale(v, np.float32(s)).astype(int)
        want = [_exact_round(float(a), s) for a in v]
        assert got.tolist() == want
        assert np.all(got % 2 == 0)


def test_near_ties_are_not_ties():
    """One ulp either side of an exact tie rounds away from the tie's even choice."""
    s = np.float32(0.5)
    tie = np.float32(1.25)  # 2.5 * s
    lo, hi = np.nextafter(tie, np.float32(0)), np.nextafter(tie, np.float32(10))
    assert O.quantize_with_scale(np.array([lo, tie, hi], np.float32), s).tolist() == [2, 2, 3]


def test_scale_is_correctly_rounded_f32():
    rng = np.random.default_rng(2)
    peaks = np.abs(rng.normal(size=2000)).astype(np.float32) * np.float32(10)
    s = O.scale_of(peaks)
    for p, sc in zip(peaks, s):
        exact = Fraction(float(p)) / 127
        err = abs(Fraction(float(sc)) - exact)
        ulp = Fraction(float(np.spacing(sc)))
        assert err <= ulp / 2


def test_quantize_rows_invariants():
    rng = np.random.default_rng(3)
    x = rng.normal(size=(64, 300)).astype(np.float32)
    x[5] = 0.0  # a zero row → s = 0, q = 0 (quant.ts:36)
    q, s = O.quantize_rows(x)
    assert s[5] == 0 and not q[5].any()
    assert np.abs(q.astype(int)).max() <= 127
    for m in range(64):
        if m == 5:
            continue
        j = np.argmax(np.abs(x[m]))
        assert abs(int(q[m, j])) == 127
        err = np.abs(q[m].astype(np.float64) * s[m] - x[m].astype(np.float64))
        assert np.all(err <= s[m] / 2 * (1 + 1e-6))


def test_quantize_rows_hand_row():
    x = np.array([[127.0, 2.5, 3.5, -0.5, -1.5, 0.49999997, -127.0, 126.5]], np.float32)
    q, s = O.quantize_rows(x)
    assert s.tolist() == [1.0]
    assert q.tolist() == [[127, 2, 4, 0, -2, 0, -127, 126]]


def test_pack_words_low_byte_first():
    q = np.array([1, -1, 2, -128, 5], np.int8)
    w = O.pack_words(q)
    assert w.tolist() == [0x80_02_FF_01, 0x00_00_00_05]


def test_quantize_tensor_and_nhwc_layout():
    rng = np.random.default_rng(4)
    x = rng.normal(size=(2, 3, 4, 5)).astype(np.float32)
    q, s = O.quantize_act_nhwc(x, cpad=16)
    assert q.shape == (2, 4, 5, 16) and not q[..., 3:].any()
    qt, st = O.quantize_tensor(x)
    assert s == st
    assert np.array_equal(q[..., :3], qt.transpose(0, 2, 3, 1))
    assert np.array_equal(qt, O.quantize_with_scale(x, np.float32(np.abs(x).max() / np.float32(127))))


# -------------------------------------------------------------------- integer GEMM

def _lcg_int8(n, seed):
    """kernel_bench.html:300-301: st = st·1664525 + 1013904223 (u32), int8 = (st>>>28) − 8."""
    out = np.empty(n, np.int8)
    st = seed
    for i in range(n):
        st = (st * 1664525 + 1013904223) & 0xFFFFFFFF
        out[i] = (st >> 28) - 8
    return out


def _brute_gemm(a, w):
    M, K = a.shape
    N = w.shape[0]
    out = np.zeros((M, N), np.int64)
    for m in range(M):
        for n in range(N):
            s = 0
            for k in range(K):
                s += int(a[m, k]) * int(w[n, k])
            out[m, n] = s
    return out


@pytest.mark.parametrize("M,K,N", [(32, 32, 32), (5, 48, 7), (1, 64, 3)])
def test_gemm_matches_brute_force_lcg(M, K, N):
    a = _lcg_int8(M * K, 7).reshape(M, K)
    w = _lcg_int8(K * N, 11).reshape(N, K)
    assert np.array_equal(O.gemm_i8_i32(a, w), _brute_gemm(a, w))


def test_gemm_closed_forms():
    K = 4096
    a = np.full((2, K), 127, np.int8)
    a[1] = -127
    w = np.full((3, K), -127, np.int8)
    acc = O.gemm_i8_i32(a, w)
    assert acc[0].tolist() == [-K * 16129] * 3 and acc[1].tolist() == [K * 16129] * 3
    eye = np.eye(16, dtype=np.int8)
    x = np.arange(-8, 8, dtype=np.int8).reshape(1, 16).repeat(4, 0)
    assert np.array_equal(O.gemm_i8_i32(x, eye), x.astype(np.int32))


# ----------------------------------------------------------------------- epilogue

def test_dequant_order_and_rounding():
    rng = np.random.default_rng(5)
    acc = rng.integers(-2**26, 2**26, size=(7, 9)).astype(np.int32)
    sA = rng.uniform(0.001, 0.1, 7).astype(np.float32)
    sW = rng.uniform(0.001, 0.1, 9).astype(np.float32)
    b = rng.normal(size=9).astype(np.float32)
    res = rng.normal(size=(7, 9)).astype(np.float32)
    y = O.dequant(acc, sA, sW, b, relu=True, residual=res)
    for m in range(7):
        for n in range(9):
            v = f32(f32(f32(float(acc[m, n])) * float(sA[m])) * float(sW[n]))
            v = f32(f32(v + float(b[n])) + float(res[m, n]))
            v = v if v > 0 else 0.0
            assert y[m, n] == np.float32(v)
    # hand value: 1000 * 0.5 * 0.25 + 1 = 126
    assert O.dequant(np.array([[1000]]), np.float32(0.5), np.array([0.25], np.float32),
                     np.array([1.0], np.float32))[0, 0] == 126.0


# ---------------------------------------------------------------------------- conv

def _brute_conv(xq, wq, KH, KW, stride, pad):
    """Direct loops as kernel_bench.html:406-413, NHWC x, [O][KH][KW][C] w."""
    N, H, W, C = xq.shape
    O_ = wq.shape[0]
    w4 = wq.reshape(O_, KH, KW, C).astype(np.int64)
    OH = (H + 2 * pad - KH) // stride + 1
    OW = (W + 2 * pad - KW) // stride + 1
    out = np.zeros((N, OH, OW, O_), np.int64)
    for n in range(N):
        for oy in range(OH):
            for ox in range(OW):
                for kh in range(KH):
                    iy = oy * stride - pad + kh
                    if iy < 0 or iy >= H:
                        continue
                    for kw in range(KW):
                        ix = ox * stride - pad + kw
                        if ix < 0 or ix >= W:
                            continue
                        out[n, oy, ox] += w4[:, kh, kw, :] @ xq[n, iy, ix].astype(np.int64)
    return out.reshape(-1, O_)


@pytest.mark.parametrize("KH,stride,pad", [(3, 1, 1), (3, 2, 1), (1, 2, 0), (5, 1, 2), (1, 1, 0)])
def test_conv_matches_brute_force(KH, stride, pad):
    rng = np.random.default_rng(6)
    xq = rng.integers(-127, 128, size=(2, 7, 6, 5)).astype(np.int8)
    wq = rng.integers(-127, 128, size=(4, KH * KH * 5)).astype(np.int8)
    acc, OH, OW = O.conv2d_i8_nhwc(xq, wq, KH, KH, stride, pad)
    assert np.array_equal(acc, _brute_conv(xq, wq, KH, KH, stride, pad))


@pytest.mark.parametrize("KH,stride,pad", [(3, 1, 1), (3, 2, 1), (5, 1, 2), (5, 2, 2)])
def test_dwconv_matches_brute_force(KH, stride, pad):
    rng = np.random.default_rng(7)
    N, H, W, C = 2, 9, 8, 6
    xq = rng.integers(-127, 128, size=(N, H, W, C)).astype(np.int8)
    wq = rng.integers(-127, 128, size=(KH * KH, C)).astype(np.int8)
    got = O.dwconv_i8_nhwc(xq, wq, KH, KH, stride, pad)
    # brute force: each channel is a single-channel conv
    for c in range(C):
        one = _brute_conv(xq[..., c:c + 1], wq[:, c].reshape(1, -1), KH, KH, stride, pad)
        assert np.array_equal(got[..., c].reshape(-1), one[:, 0])


def test_conv_f32_matches_torch():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(8)
    x = rng.normal(size=(2, 3, 9, 9)).astype(np.float32)
    w = rng.normal(size=(4, 3, 3, 3)).astype(np.float32)
    b = rng.normal(size=4).astype(np.float32)
    for stride, pad in ((1, 1), (2, 1), (2, 0)):
        got = O.conv2d_f32(x, w, b, stride, pad)
        want = torch.nn.functional.conv2d(torch.from_numpy(x), torch.from_numpy(w), torch.from_numpy(b),
                                          stride, pad).numpy()
        np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)


def test_conv_weight_layout_matches_f32_conv():
    """The [O][KH][KW][C] packing with im2col reproduces the f32 conv on exact values."""
    rng = np.random.default_rng(9)
    x = rng.integers(-3, 4, size=(1, 5, 6, 6)).astype(np.float32)
    w = rng.integers(-3, 4, size=(3, 5, 3, 3)).astype(np.float32)
    xq = x.transpose(0, 2, 3, 1).astype(np.int8)
    wq = w.transpose(0, 2, 3, 1).reshape(3, -1).astype(np.int8)
    acc, OH, OW = O.conv2d_i8_nhwc(xq, wq, 3, 3, 1, 1)
    ref = O.conv2d_f32(x, w, None, 1, 1)
    assert np.array_equal(acc.reshape(1, OH, OW, 3).transpose(0, 3, 1, 2), ref.astype(np.int32))


def test_bn_fold_equals_conv_then_bn():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(10)
    w = rng.normal(size=(4, 3, 3, 3)).astype(np.float32)
    rm, rv = rng.normal(size=4).astype(np.float32) * 0.1, rng.uniform(0.5, 1.5, 4).astype(np.float32)
    g, be = (1 + 0.1 * rng.normal(size=4)).astype(np.float32), (0.1 * rng.normal(size=4)).astype(np.float32)
    x = rng.normal(size=(2, 3, 8, 8)).astype(np.float32)
    fw, fb = O.fuse_conv_bn_weights(w, None, rm, rv, 1e-5, g, be)
    y = torch.nn.functional.conv2d(torch.from_numpy(x), torch.from_numpy(w), None, 1, 1)
    y = torch.nn.functional.batch_norm(y, torch.from_numpy(rm), torch.from_numpy(rv), torch.from_numpy(g),
                                       torch.from_numpy(be), False, 0.0, 1e-5)
    np.testing.assert_allclose(O.conv2d_f32(x, fw, fb, 1, 1), y.numpy(), rtol=1e-4, atol=1e-5)


def test_linear_int8_close_to_f32():
    """The quantized Linear stays near the f32 one (accuracy sanity, not parity)."""
    from borch_amd import workloads as WL
    x, w, b = WL.c1_linear(0)
    y, acc, _, _ = O.linear_int8(x, w, b)
    ref = O.linear_f32(x, w, b)
    assert np.abs(y - ref).max() < 0.05 * np.abs(ref).max()


def test_dequant_weight_is_one_f32_rounding():
    """f32(q)·s rounded once (quant.ts:60-71 stores the double product into a Float32Array)."""
    rng = np.random.default_rng(12)
    q = rng.integers(-127, 128, size=(7, 33)).astype(np.int8)
    s = rng.uniform(1e-4, 1e-1, 7).astype(np.float32)
    w = O.dequant_weight(q, s)
    for n in range(7):
        for k in range(33):
            assert w[n, k] == np.float32(float(q[n, k]) * float(s[n]))


def test_linear_w8a32_bound_holds_for_f32_accumulation():
    """The bound admits a plain sequential f32 FMA accumulation (the kernel's kind)."""
    rng = np.random.default_rng(13)
    x = rng.normal(size=(3, 256)).astype(np.float32)
    q = rng.integers(-127, 128, size=(5, 256)).astype(np.int8)
    s = rng.uniform(1e-3, 1e-2, 5).astype(np.float32)
    y, bound = O.linear_w8a32(x, q, s)
    w = O.dequant_weight(q, s)
    for m in range(3):
        for n in range(5):
            acc = np.float32(0)
            for k in range(256):
                acc = np.float32(acc + np.float32(x[m, k] * w[n, k]))
            assert abs(float(acc) - y[m, n]) <= bound[m, n]


def test_gelu_closed_form():
    """oracle.gelu against the definition with math.erf element by element, the exact
    identity gelu(x) - gelu(-x) = x (Φ(x) + Φ(-x) = 1), gelu(0) = 0, the large-|x| limits,
    and torch's own CPU gelu (a library routine) at float32 precision."""
    import math

    import torch
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.normal(size=2000) * 3, [0.0, 1e-8, -1e-8, 8.0, -8.0, 30.0, -30.0]]).astype(np.float32)
    g = O.gelu(x)
    ref = np.array([0.5 * float(v) * (1.0 + math.erf(float(v) / math.sqrt(2.0))) for v in x], np.float64)
    np.testing.assert_allclose(g, ref.astype(np.float32), rtol=0, atol=0)
    x64 = x.astype(np.float64)
    odd = O.gelu(x).astype(np.float64) - O.gelu(-x).astype(np.float64)
    np.testing.assert_allclose(odd, x64, rtol=2e-7, atol=1e-12)
    assert O.gelu(np.float32(0.0)) == 0.0
    assert O.gelu(np.float32(30.0)) == np.float32(30.0) and O.gelu(np.float32(-30.0)) == 0.0
    tg = torch.nn.functional.gelu(torch.from_numpy(x)).numpy()
    np.testing.assert_allclose(g, tg, rtol=1e-5, atol=1e-6)  # torch rounds in f32: 1 + erf cancels


def test_silu_closed_form():
    """oracle.silu against the definition with math.exp element by element, the identity
    silu(x) - silu(-x) = x (σ(x) + σ(-x) = 1), silu(0) = 0, and torch's CPU silu."""
    import math

    import torch
    rng = np.random.default_rng(4)
    x = np.concatenate([rng.normal(size=2000) * 4, [0.0, 1e-8, -1e-8, 20.0, -20.0, 80.0, -80.0]]).astype(np.float32)
    g = O.silu(x)
    ref = np.array([float(v) / (1.0 + math.exp(-float(v))) for v in x], np.float64)
    np.testing.assert_array_equal(g, ref.astype(np.float32))
    odd = O.silu(x).astype(np.float64) - O.silu(-x).astype(np.float64)
    np.testing.assert_allclose(odd, x.astype(np.float64), rtol=2e-7, atol=1e-30)
    assert O.silu(np.float32(0.0)) == 0.0
    np.testing.assert_allclose(g, torch.nn.functional.silu(torch.from_numpy(x)).numpy(), rtol=1e-5, atol=1e-6)


def _on_grid(rng, shape, step):
    """Values q * step with q in [-127, 127] and some |q| = 127 per row (quantization by the
    rule is then exact: the scale is step, the bytes are q)."""
    q = rng.integers(-127, 128, size=shape).astype(np.float64)
    q.reshape(shape[0], -1)[:, 0] = 127.0
    return (q * step).astype(np.float32)


def test_composed_layers_on_exact_grids():
    """The oracle's composed int8 layers (oracle/models.py conv_layer / dwconv_layer /
    linear_layer, oracle/quant.py conv2d_int8) on inputs whose quantization loses nothing
    (activations on a per-tensor grid, weights on per-channel grids, a power-of-two step so
    every product is exact): then y = conv(x, w) + b (+ residual) exactly in float64, which
    torch's float64 conv2d / linear (library routines) give independently, to a few f32 ulps."""
    import torch
    from oracle import models as OM
    F = torch.nn.functional
    rng = np.random.default_rng(5)
    step_x = 2.0 ** -6
    for (N, C, H, O_, k, stride, pad) in [(2, 3, 9, 8, 3, 1, 1), (1, 20, 8, 12, 3, 2, 1), (2, 16, 7, 16, 1, 1, 0),
                                          (1, 5, 11, 6, 5, 2, 2)]:
        x = _on_grid(rng, (N, C, H, H), step_x)
        x.reshape(-1)[0] = np.float32(127 * step_x)  # the tensor's peak is exactly 127 steps
        x = np.clip(x, -127 * step_x, 127 * step_x).astype(np.float32)
        w = np.stack([_on_grid(rng, (1, C, k, k), 2.0 ** -int(rng.integers(3, 9)))[0] for _ in range(O_)])
        b = (rng.integers(-64, 64, size=O_) * 2.0 ** -8).astype(np.float32)
        OH = (H + 2 * pad - k) // stride + 1
        res = (rng.integers(-64, 64, size=(N, O_, OH, OH)) * 2.0 ** -8).astype(np.float32)
        want = F.conv2d(torch.from_numpy(x).double(), torch.from_numpy(w).double(), torch.from_numpy(b).double(),
                        stride, pad).numpy()
        y, acc, sA, sW, qw = OM.conv_layer(x, w, b, stride, pad, OM.ACT_RELU, res)
        np.testing.assert_allclose(y, np.maximum(want + res, 0), rtol=1e-6, atol=1e-7)
        y2, _, _, _ = O.conv2d_int8(x, w, b, stride, pad, True, res, (C + 15) // 16 * 16)
        np.testing.assert_array_equal(y2, y)
        wd = np.stack([_on_grid(rng, (1, 1, k, k), 2.0 ** -5)[0] for _ in range(C)])
        yd, _, _, _, _ = OM.dwconv_layer(x, wd, b[:1].repeat(C), stride, pad)
        wantd = F.conv2d(torch.from_numpy(x).double(), torch.from_numpy(wd).double(),
                         torch.from_numpy(b[:1].repeat(C)).double(), stride, pad, groups=C).numpy()
        np.testing.assert_allclose(yd, wantd, rtol=1e-6, atol=1e-7)
    # Linear, per-row activations: each row on its own grid; residual and GELU after the bias
    xl = np.stack([_on_grid(rng, (1, 40), 2.0 ** -int(rng.integers(2, 8)))[0] for _ in range(6)])
    wl = np.stack([_on_grid(rng, (1, 40), 2.0 ** -int(rng.integers(4, 9)))[0] for _ in range(10)])
    bl = (rng.integers(-64, 64, size=10) * 2.0 ** -8).astype(np.float32)
    rl = (rng.integers(-64, 64, size=(6, 10)) * 2.0 ** -8).astype(np.float32)
    want = F.linear(torch.from_numpy(xl).double(), torch.from_numpy(wl).double(), torch.from_numpy(bl).double())
    y, _, _, _, _ = OM.linear_layer(xl, wl, bl, OM.ACT_GELU, rl)
    np.testing.assert_allclose(y, O.gelu((want.numpy() + rl).astype(np.float32)), rtol=1e-6, atol=1e-7)


def test_se_gate_against_torch_float64():
    """oracle.models.se_gate equals torch's float64 mean / linear / silu / sigmoid (library
    routines) composed as the CPU runner's squeeze-excite node."""
    import torch
    from oracle import models as OM
    rng = np.random.default_rng(6)
    x = rng.normal(size=(3, 24, 5, 7)).astype(np.float32)
    w1, b1 = rng.normal(size=(6, 24)).astype(np.float32), rng.normal(size=6).astype(np.float32)
    w2, b2 = rng.normal(size=(24, 6)).astype(np.float32), rng.normal(size=24).astype(np.float32)
    T = lambda a: torch.from_numpy(a).double()
    p = T(x).mean(dim=(2, 3))
    z = torch.nn.functional.silu(torch.nn.functional.linear(p, T(w1), T(b1)))
    want = torch.sigmoid(torch.nn.functional.linear(z, T(w2), T(b2))).float().numpy()
    np.testing.assert_allclose(OM.se_gate(x, w1, b1, w2, b2), want, rtol=1e-7, atol=1e-9)


@pytest.mark.parametrize("n,seed", [(1, 7), (4095, 11), (4096, 7), (10001, 11), (3 * 4096 + 5, 3)])
def test_vectorised_lcg_is_the_reference_generator(n, seed):
    """workloads.lcg_int8 (jump-ahead blocks) draws exactly kernel_bench.html:300-301's
    sequence, restated step by step in _lcg_int8."""
    from borch_amd import workloads as WL
    assert np.array_equal(WL.lcg_int8(n, seed), _lcg_int8(n, seed))


def test_mmi8_operands_layout():
    """A @ W.T of the Linear layout equals the reference's A @ B on its own operands."""
    from borch_amd import workloads as WL
    A, W = WL.mmi8_operands(32, 48, 16)
    assert np.array_equal(A.reshape(-1), _lcg_int8(32 * 48, 7))
    B = _lcg_int8(48 * 16, 11).reshape(48, 16)
    assert np.array_equal(W, B.T)
    ref = A.astype(np.int64) @ B.astype(np.int64)
    assert np.array_equal(O.gemm_i8_i32(A, W), ref.astype(np.int32))


def test_attention_oracle_against_torch_and_closed_forms():
    """oracle.models.attention_qkv against torch's scaled_dot_product_attention in float64 on
    the CPU (an independent implementation), and two closed forms: identical keys give every
    query the mean of v; one dominant key per query selects that key's value row."""
    import torch

    from oracle import models as OM
    rng = np.random.default_rng(3)
    B, T, H, dh = 2, 9, 3, 64
    qkv = rng.normal(size=(B, T, 3, H, dh))
    got = OM.attention_qkv(qkv.reshape(B, T, -1), H)
    x = torch.from_numpy(qkv).permute(2, 0, 3, 1, 4)
    ref = torch.nn.functional.scaled_dot_product_attention(x[0], x[1], x[2]).transpose(1, 2).reshape(B, T, -1)
    np.testing.assert_allclose(got, ref.numpy(), rtol=1e-12, atol=1e-12)
    same = qkv.copy()
    same[:, :, 1] = same[:, :1, 1]  # every key equal to token 0's
    np.testing.assert_allclose(OM.attention_qkv(same.reshape(B, T, -1), H).reshape(B, T, H, dh),
                               np.broadcast_to(same[:, :, 2].mean(axis=1, keepdims=True), (B, T, H, dh)), atol=1e-12)
    sel = np.zeros((1, 4, 3, 1, dh))
    sel[0, :, 0, 0, :] = np.eye(4, dh) * 400.0  # query t matches key t only (scores 0 or 400^2 / 8)
    sel[0, :, 1, 0, :] = np.eye(4, dh) * 400.0
    sel[0, :, 2, 0, :] = rng.normal(size=(4, dh))
    np.testing.assert_allclose(OM.attention_qkv(sel.reshape(1, 4, -1), 1).reshape(4, dh), sel[0, :, 2, 0], atol=1e-9)


def test_avgpool_linear_oracle_against_torch():
    """oracle.models.avgpool_linear against torch's mean over H, W and linear in float64."""
    import torch

    from oracle import models as OM
    rng = np.random.default_rng(4)
    x, w, b = rng.normal(size=(3, 8, 4, 4)), rng.normal(size=(5, 8)), rng.normal(size=5)
    got, scale = OM.avgpool_linear(x, w, b)
    ref = torch.nn.functional.linear(torch.from_numpy(x).mean(dim=(2, 3)), torch.from_numpy(w), torch.from_numpy(b))
    np.testing.assert_allclose(got, ref.numpy(), rtol=1e-12, atol=1e-12)
    assert np.all(scale >= np.abs(got - b) - 1e-12)


# ------------------------------------------- the reference's two weight packers, restated

def _js_round_scalar(x: float) -> float:
    """ECMA-262 Math.round from its definition: the integer nearest x, a tie toward +inf
    (decided in exact rationals, so independent of the oracle's floor-based form)."""
    fx = Fraction(x)
    lo = fx.numerator // fx.denominator  # floor
    return float(lo + 1) if fx - lo >= Fraction(1, 2) else float(lo)


def _ref_linear_row(row):
    """quant.ts:31-41 element by element in Python floats (IEEE doubles, as JavaScript)."""
    peak = 0.0
    for v in row:
        if abs(v) > peak:
            peak = abs(v)
    scale = peak / 127
    if scale == 0:
        return [0] * len(row), f32(scale)
    inv = 1 / scale
    return [int(max(-127.0, min(127.0, _js_round_scalar(v * inv)))) for v in row], f32(scale)


def _ref_conv_row(row):
    """quant.ts:86-96 element by element: the f32-stored scale, then Math.round(w / scale)."""
    peak = 0.0
    for v in row:
        if abs(v) > peak:
            peak = abs(v)
    scale = f32(peak / 127)
    if scale == 0:
        return [0] * len(row), scale
    return [int(max(-127.0, min(127.0, _js_round_scalar(v / scale)))) for v in row], scale


def test_js_math_round_known_answers():
    xs = [2.5, -2.5, 0.5, -0.5, 1.5, -1.5, 0.49999999999999994, -0.49999999999999994, 126.5, -126.5,
          1.4999999999999998, 3.0, -3.0]
    want = [3, -2, 1, 0, 2, -1, 0, 0, 127, -126, 1, 3, -3]
    assert O.js_math_round(np.array(xs)).tolist() == want
    assert [_js_round_scalar(x) for x in xs] == want


def _planted_rows(rng):
    rows = [rng.normal(size=64).astype(np.float32) * np.float32(0.05) for _ in range(6)]
    # exact ties of the stored f32 scale: peak 127 * 2^-6 gives s = 2^-6 exactly
    s = 2.0 ** -6
    tie = np.array([127 * s] + [(k + 0.5) * s for k in range(-126, 126, 7)], np.float32)
    rows.append(tie)
    rows.append(-tie)
    rows.append(np.zeros(40, np.float32))
    return rows


def test_reference_linear_packer_restates_quant_ts_35_41():
    rng = np.random.default_rng(11)
    for row in _planted_rows(rng):
        q, s = O.quantize_weight_reference_linear(row[None, :])
        q_s, s_s = _ref_linear_row([float(v) for v in row])
        assert q[0].tolist() == q_s and f32(float(s[0])) == s_s


def test_reference_conv_packer_restates_quant_ts_86_96():
    rng = np.random.default_rng(12)
    for row in _planted_rows(rng):
        q, s = O.quantize_conv_weight_reference(row[None, :])
        q_s, s_s = _ref_conv_row([float(v) for v in row])
        assert q[0].tolist() == q_s and float(s[0]) == s_s
    # the conv packer's scale is the build rule's (the f64 quotient stored in f32 equals
    # the correctly rounded f32 quotient)
    w = rng.normal(size=(300, 50)).astype(np.float32)
    assert np.array_equal(O.quantize_conv_weight_reference(w)[1], O.quantize_weight_per_channel(w)[1])


def _diff_positions(w):
    q0, s0 = O.quantize_weight_per_channel(w)
    q1, s1 = O.quantize_weight_reference_linear(w)
    q2, s2 = O.quantize_conv_weight_reference(w)
    assert np.array_equal(s0, s1) and np.array_equal(s0, s2)
    lin = [tuple(int(i) for i in p) for p in np.argwhere(q0 != q1)]
    conv = [tuple(int(i) for i in p) for p in np.argwhere(q0 != q2)]

    def tie(p):
        return (Fraction(float(w[p])) / Fraction(float(s0[p[0]]))).denominator == 2
    # the conv packer differs from the build rule exactly on ties of the exact quotient
    assert all(tie(p) for p in conv)
    return lin, [tie(p) for p in lin], conv, q0, q1


# C2's 4096 x 4096 weight (seed 0): the 12 bytes where quant.ts:35-41 and the build rule
# disagree, with the build's and the reference's byte. None is an exact tie: each exact
# quotient is within 1.1e-6 of k + 1/2, and the reference's double scale puts w·(1/scale)
# on the other side.
C2_LINEAR_DIFFS = [((147, 1391), -21, -22), ((490, 674), 21, 22), ((725, 1224), 57, 56), ((742, 1293), 47, 46),
                   ((805, 3780), 11, 10), ((1842, 3269), 55, 54), ((2067, 2755), 29, 28), ((2319, 1316), -16, -17),
                   ((2495, 3654), 45, 46), ((2515, 693), -15, -14), ((3207, 3640), -24, -23),
                   ((3682, 3921), -14, -15)]


def test_reference_linear_packer_against_build_rule_c1_c2():
    from borch_amd import workloads as WL
    _, w1, _ = WL.c1_linear(0)
    lin, ties, conv, _, _ = _diff_positions(w1)
    assert lin == [] and conv == []
    _, w2, _ = WL.c2_gemm(1, 0)
    lin, ties, conv, q0, q1 = _diff_positions(w2)
    assert conv == []
    assert [(p, int(q0[p]), int(q1[p])) for p in lin] == C2_LINEAR_DIFFS
    assert not any(ties)
    for p, _, _ in C2_LINEAR_DIFFS:  # near-ties: the exact quotient is within 1.1e-6 of k + 1/2
        qq = Fraction(float(w2[p])) / Fraction(float(O.scale_of(np.abs(w2[p[0]]).max())))
        frac = qq - (qq.numerator // qq.denominator)  # qq - floor(qq), in [0, 1)
        assert 0 < abs(frac - Fraction(1, 2)) < Fraction(11, 10**7)
    # the rows holding them, element by element in Python floats (JavaScript's arithmetic)
    for r in sorted({p[0] for p, _, _ in C2_LINEAR_DIFFS}):
        assert q1[r].tolist() == _ref_linear_row([float(v) for v in w2[r]])[0]


C5_DIFF_DIGEST = "83d7fa44705a776e"  # sha256 of the repr of the 150 (layer, name, n, k) positions


def test_reference_linear_packer_against_build_rule_c5():
    """C5's 48 Linear weights (ViT-B/16, seed 0): 150 bytes differ, one of them on an exact
    tie of the build rule's quotient; the conv packer's rule differs on exact ties only."""
    import hashlib
    from borch_amd import nets
    model = nets.build("vit_b16", seed=0, device="cpu")
    allpos, nties, per_kind = [], 0, {}
    for li, layer in enumerate(model.layers):
        for name in ("qkv", "proj", "fc1", "fc2"):
            w = getattr(layer, name).weight.detach().numpy()
            lin, ties, _, _, _ = _diff_positions(w)
            nties += sum(ties)
            per_kind[name] = per_kind.get(name, 0) + len(lin)
            allpos += [(li, name, *p) for p in lin]
    assert len(allpos) == 150 and nties == 1
    assert per_kind == {"qkv": 40, "proj": 15, "fc1": 45, "fc2": 50}
    digest = hashlib.sha256(repr(allpos).encode()).hexdigest()[:16]
    assert digest == C5_DIFF_DIGEST


# ------------------------------------------------- W8A32 decode GEMV, operation for operation

def _round_f32_exact(v):
    """Correct float32 rounding (half to even) of an exact rational, by scaling to a 24-bit
    integer significand; normal range only."""
    from fractions import Fraction
    if v == 0:
        return np.float32(0.0)
    sign = -1 if v < 0 else 1
    a = abs(v)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    m = round(a / Fraction(2) ** (e - 23))  # round() of a Fraction: half to even
    return np.float32(sign * float(m * Fraction(2) ** (e - 23)))


def test_fma_f32_is_one_correct_rounding():
    from fractions import Fraction
    rng = np.random.default_rng(5)
    a = rng.normal(size=3000).astype(np.float32)
    b = rng.normal(size=3000).astype(np.float32)
    c = np.concatenate([rng.normal(size=1000), -(a[1000:2000].astype(np.float64) * b[1000:2000]),
                        rng.normal(size=1000) * 1e-9]).astype(np.float32)
    got = O.fma_f32(a, b, c)
    for i in range(len(a)):
        want = _round_f32_exact(Fraction(float(a[i])) * Fraction(float(b[i])) + Fraction(float(c[i])))
        assert got[i] == want, (i, a[i], b[i], c[i], got[i], want)
    # the float64 sum lands exactly on a float32 midpoint: (1 + 2^-12)^2 = 1 + 2^-11 + 2^-24, and
    # a 2^-80 addend decides the side (a rounding of the float64 sum alone would tie to even)
    s = np.float32(1 + 2.0 ** -12)
    assert O.fma_f32(s, s, np.float32(2.0 ** -80)) == np.float32(1 + 2.0 ** -11 + 2.0 ** -23)
    assert O.fma_f32(s, s, np.float32(-(2.0 ** -80))) == np.float32(1 + 2.0 ** -11)


def test_w8a32_gemv_restatement_fused_products():
    """acc = fma(x, w, acc): with w = 1 + 2^-12 the product s^2 needs 25 bits; fused with
    the previous -s it is exact (2^-12 + 2^-24), where a separately rounded product gives
    2^-12."""
    s = np.float32(1 + 2.0 ** -12)
    q = np.zeros((1, 16), np.int8)
    q[0, :2] = 1
    x = np.zeros((1, 16), np.float32)
    x[0, 0], x[0, 1] = -1, s
    y = O.linear_w8a32_gemv(x, q, np.array([s], np.float32))
    assert y[0, 0] == np.float32(2.0 ** -12 + 2.0 ** -24)
    assert np.float32(np.float32(s * s) - s) == np.float32(2.0 ** -12)  # the unfused value differs


def test_w8a32_gemv_restatement_covers_every_term():
    """Small integer operands: every product and partial sum is exact, so the result is the
    integer dot product (any dropped, repeated or misplaced term shows), over ragged chunks
    (K = 2064: the third chunk's first lane only) and a bias, residual and ReLU."""
    rng = np.random.default_rng(9)
    M, N, K = 3, 37, 2064
    x = rng.integers(-4, 5, size=(M, K)).astype(np.float32)
    q = rng.integers(-127, 128, size=(N, K)).astype(np.int8)
    b = rng.integers(-50, 50, size=N).astype(np.float32)
    r = rng.integers(-50, 50, size=(M, N)).astype(np.float32)
    want = x.astype(np.int64) @ q.astype(np.int64).T + b.astype(np.int64) + r.astype(np.int64)
    y = O.linear_w8a32_gemv(x, q, np.ones(N, np.float32), b, r, relu=True)
    assert np.array_equal(y, np.maximum(want, 0).astype(np.float32))


def test_w8a32_gemv_restatement_lane_tree_order():
    """Lane sums of 1 and 2^-24 at chosen lanes: with lanes 0, 1, 2 the tree gives 1 (the
    exact sum is 1 + 2^-23); with lanes 0, 2, 3 it gives 1 + 2^-23 (a left-to-right sum
    gives 1)."""
    K = 1024
    x = np.zeros((1, K), np.float32)
    x[0, 0], x[0, 16], x[0, 32], x[0, 48] = 1, 2.0 ** -24, 2.0 ** -24, 2.0 ** -24
    q = np.zeros((2, K), np.int8)
    q[0, [0, 16, 32]] = 1  # lanes 0, 1, 2
    q[1, [0, 32, 48]] = 1  # lanes 0, 2, 3
    y = O.linear_w8a32_gemv(x, q, np.ones(2, np.float32))
    assert y[0, 0] == np.float32(1.0) and y[0, 1] == np.float32(1 + 2.0 ** -23)
