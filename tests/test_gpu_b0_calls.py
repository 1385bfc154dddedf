"""GPU parity of EfficientNet-B0 (config C4) at its full batch of 64, call by call.

Every int8 kernel call the real forward makes is checked against the oracle as it
happens, on sampled images (the per-tensor dynamic scale is a maximum over the whole
batch, so it is checked on the whole tensor; everything per image on the sample):

* quantizers (``quantize_nhwc``, ``quantize_nhwc_scaled``, ``quantize_nhwc_chscale``):
  the scale equals ``scale_of(max|v|)`` of the full tensor (v the input, or the
  squeeze-excite product ``fl(x * g)``) or the calibrated scale, and the bytes equal
  ``quantize_with_scale`` of the sampled images, bit for bit;
* convs (``conv2d_i8_nhwc``, ``conv2d_i8_nhwc_q`` with or without its f32 output, the
  stem's ``conv2d_nchw_fq`` with its input quantization fused) and depthwise convs: the packed weight equals the oracle packing of the layer's folded f32
  weight, the int32 accumulators (re-read through the C ABI) equal the oracle's exact
  integer conv of the int8 input actually passed, the f32 output equals the oracle
  epilogue (bit for bit, SiLU layers within 1e-5 rel / 1e-6 abs: the device's exp and
  numpy's differ in the last bit), and an int8 twin equals ``quantize_with_scale`` of the
  device's own f32 output with the calibrated scale. A twin-only call (no f32 output) is
  re-run with its f32 output and must give the same twin. The fused stem's scale equals
  ``scale_of(max|x|)`` or the calibrated one, and its accumulators the oracle's conv of
  ``quantize_with_scale`` of the sampled images;
* the dynamic twin (``conv2d_i8_nhwc_dq``, an expansion that feeds its depthwise conv with no
  f32 output): the same conv's f32 output is checked as above, and the twin and its scale
  must equal ``quantize_nhwc`` of it, bit for bit.

With calibrated scales this covers the bench's static path: the static network input, the
expand convs that write their twin alone, the depthwise convs that read those twins with a
static scale, and the channel-scaled quantize of each projection input.
"""
import sys

import numpy as np
import pytest
import torch

import borch_amd as bt
from borch_amd import int8 as I
from borch_amd import nets, workloads as WL
from borch_amd.nn import _int8_layers
from oracle import models as OM
from oracle import quant as Q

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-5, 1e-6
IMAGES = [0, 37, 63]


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def n(x):
    return x.detach().cpu().numpy()


class Recorder:
    """Wraps the int8 module's kernel calls; checks each one as it returns."""

    def __init__(self, model, images):
        self.images = images
        self.by_w = {}
        for name, m in _int8_layers(model):
            if m.int8 is not None:
                self.by_w[id(m.int8)] = (name, m)
        self.counts = {}
        self.real = {}

    def _count(self, kind):
        self.counts[kind] = self.counts.get(kind, 0) + 1

    def __enter__(self):
        for fn in ("quantize_nhwc", "quantize_nhwc_scaled", "quantize_nhwc_chscale", "conv2d_i8_nhwc",
                   "conv2d_i8_nhwc_q", "conv2d_i8_nhwc_dq", "conv2d_nchw_fq", "dwconv_i8_nhwc"):
            self.real[fn] = getattr(I, fn)
            setattr(I, fn, getattr(self, fn))
        return self

    def __exit__(self, *exc):
        for fn, f in self.real.items():
            setattr(I, fn, f)

    # ----------------------------------------------------------------- quantizers
    def _check_q(self, v_full, q, s, cpad, name):
        """q [N, H, W, cpad] of v_full (NCHW f32, on the device) with scale s (float)."""
        sel = v_full[self.images]
        C = v_full.shape[1]
        want = np.zeros(q[self.images].shape, np.int8)
        want[..., :C] = Q.quantize_with_scale(n(sel), np.float32(s)).transpose(0, 2, 3, 1)
        assert np.array_equal(n(q[self.images]), want), f"{name}: quantized bytes differ"

    def _peak_scale(self, v_full):
        # max|v| is exact in any order, so torch's device reduction gives numpy's value
        return Q.scale_of(np.array([float(v_full.abs().amax())], np.float32))[0]

    def quantize_nhwc(self, x, cpad=None):
        q, s = self.real["quantize_nhwc"](x, cpad)
        self._count("quantize_nhwc")
        want_s = self._peak_scale(x)
        assert n(s)[0] == want_s, "dynamic per-tensor scale differs"
        self._check_q(x, q, want_s, cpad, "quantize_nhwc")
        return q, s

    def quantize_nhwc_scaled(self, x, scale, cpad=None):
        q = self.real["quantize_nhwc_scaled"](x, scale, cpad)
        self._count("quantize_nhwc_scaled")
        self._check_q(x, q, n(scale)[0], cpad, "quantize_nhwc_scaled")
        return q

    def quantize_nhwc_chscale(self, x, cs, cpad=None, scale=None):
        q, s = self.real["quantize_nhwc_chscale"](x, cs, cpad, scale)
        self._count("quantize_nhwc_chscale" + ("_static" if scale is not None else ""))
        prod = x * cs[:, :, None, None]  # one f32 rounding per element, as the kernel's product
        if scale is None:
            want_s = self._peak_scale(prod)
            assert n(s)[0] == want_s, "channel-scaled dynamic scale differs"
        else:
            want_s = n(scale)[0]
            assert s is scale
        self._check_q(prod, q, want_s, cpad, "quantize_nhwc_chscale")
        return q, s

    # ----------------------------------------------------------------------- convs
    def _layer(self, wq):
        name, mod = self.by_w[id(wq)]
        return name, mod

    def _oracle_conv(self, qx, sa, wq, stride, pad, bias, residual, act, qsel=None):
        """The oracle conv of the sampled images of ``qx`` (or of ``qsel``, their int8 NHWC
        bytes given on the host) with scale ``sa``."""
        name, mod = self._layer(wq)
        w = n(mod.weight)
        qw_o, sw_o = Q.quantize_conv_weight(w, wq.cpad)
        assert np.array_equal(n(wq.q), qw_o) and np.array_equal(n(wq.s), sw_o), f"{name}: packing differs"
        if qsel is None:
            qsel = n(qx[self.images])
        acc_o, OH, OW = Q.conv2d_i8_nhwc(qsel, qw_o, wq.KH, wq.KW, stride, pad)
        res = None
        if residual is not None:
            res = n(residual[self.images].float()).transpose(0, 2, 3, 1).reshape(-1, wq.O)
        y = OM._act(Q.dequant(acc_o, n(sa)[0], sw_o, None if bias is None else n(bias), False, res), act)
        y = y.reshape(len(self.images), OH, OW, wq.O)
        return name, acc_o, y

    def _check_out(self, name, out, y_o, act):
        got = n(out[self.images]).transpose(0, 2, 3, 1)
        np.testing.assert_allclose(got, y_o, rtol=RTOL, atol=ATOL, err_msg=name)
        if act not in (I.ACT_SILU, I.ACT_GELU):
            assert np.array_equal(got, y_o), f"{name}: f32 output not bit-exact"

    def _acc(self, qx, sa, wq, stride, pad, bias, residual, act):
        _, acc = self.real["conv2d_i8_nhwc"](qx, sa, wq, stride, pad, bias, residual, act, want_acc=True)
        N = qx.shape[0]
        return n(acc.reshape(N, -1, wq.O)[self.images]).reshape(-1, wq.O)

    def conv2d_i8_nhwc(self, qx, sa, wq, stride=1, pad=0, bias=None, residual=None, act=I.ACT_NONE,
                       want_acc=False):
        r = self.real["conv2d_i8_nhwc"](qx, sa, wq, stride, pad, bias, residual, act, want_acc)
        self._count("conv2d_i8_nhwc")
        out = r[0] if want_acc else r
        name, acc_o, y_o = self._oracle_conv(qx, sa, wq, stride, pad, bias, residual, act)
        assert np.array_equal(self._acc(qx, sa, wq, stride, pad, bias, residual, act), acc_o), \
            f"{name}: int32 accumulators differ"
        self._check_out(name, out, y_o, act)
        return r

    def conv2d_i8_nhwc_q(self, qx, sa, wq, s_out, stride=1, pad=0, bias=None, residual=None, act=I.ACT_NONE,
                         f32_out=True):
        out, q = self.real["conv2d_i8_nhwc_q"](qx, sa, wq, s_out, stride, pad, bias, residual, act, f32_out)
        self._count("conv2d_i8_nhwc_q" + ("" if f32_out else "_twin_only"))
        name, acc_o, y_o = self._oracle_conv(qx, sa, wq, stride, pad, bias, residual, act)
        assert np.array_equal(self._acc(qx, sa, wq, stride, pad, bias, residual, act), acc_o), \
            f"{name}: int32 accumulators differ"
        full = out
        if not f32_out:  # the twin alone: the same call with its f32 output gives the same twin
            full, q2 = self.real["conv2d_i8_nhwc_q"](qx, sa, wq, s_out, stride, pad, bias, residual, act, True)
            assert torch.equal(q, q2), f"{name}: twin-only bytes differ from the f32 call's twin"
        self._check_out(name, full, y_o, act)
        y_dev = n(full[self.images]).transpose(0, 2, 3, 1)
        assert np.array_equal(n(q[self.images]), Q.quantize_with_scale(y_dev, n(s_out)[0])), f"{name}: twin differs"
        return out, q

    def conv2d_i8_nhwc_dq(self, qx, sa, wq, stride=1, pad=0, bias=None, residual=None, act=I.ACT_NONE):
        q, s = self.real["conv2d_i8_nhwc_dq"](qx, sa, wq, stride, pad, bias, residual, act)
        self._count("conv2d_i8_nhwc_dq")
        # the two-call form: the f32 output (held to the oracle as a conv2d_i8_nhwc call is)
        # quantized at its own dynamic scale gives the same bytes and scale
        out = self.real["conv2d_i8_nhwc"](qx, sa, wq, stride, pad, bias, residual, act)
        name, acc_o, y_o = self._oracle_conv(qx, sa, wq, stride, pad, bias, residual, act)
        assert np.array_equal(self._acc(qx, sa, wq, stride, pad, bias, residual, act), acc_o), \
            f"{name}: int32 accumulators differ"
        self._check_out(name, out, y_o, act)
        want_s = self._peak_scale(out)
        assert n(s)[0] == want_s, f"{name}: dynamic twin scale differs"
        q_r, s_r = self.real["quantize_nhwc"](out, wq.O)
        assert torch.equal(q, q_r) and torch.equal(s, s_r), f"{name}: dynamic twin differs from the two calls"
        self._check_q(out, q, want_s, wq.O, name)
        return q, s

    def conv2d_nchw_fq(self, x, wq, stride=1, pad=0, bias=None, residual=None, act=I.ACT_NONE, s_x=None,
                       s_out=None, f32_out=True, want_acc=False, want_scale=False):
        r = self.real["conv2d_nchw_fq"](x, wq, stride, pad, bias, residual, act, s_x, s_out, f32_out, want_acc,
                                        want_scale)
        self._count("conv2d_nchw_fq" + ("_static" if s_x is not None else "") + ("_twin" if s_out is not None else ""))
        # the same call with every output: its scale, accumulators and f32 output
        full = self.real["conv2d_nchw_fq"](x, wq, stride, pad, bias, residual, act, s_x, s_out, True, True, True)
        out, acc, sx = full[0], full[-2], full[-1]
        want_s = n(s_x)[0] if s_x is not None else self._peak_scale(x)
        assert n(sx)[0] == want_s, "fused stem: input scale differs"
        C, H, W = x.shape[1], x.shape[2], x.shape[3]
        qsel = np.zeros((len(self.images), H, W, wq.cpad), np.int8)
        qsel[..., :C] = Q.quantize_with_scale(n(x[self.images]), np.float32(want_s)).transpose(0, 2, 3, 1)
        name, acc_o, y_o = self._oracle_conv(None, sx, wq, stride, pad, bias, residual, act, qsel=qsel)
        got_acc = n(acc.reshape(x.shape[0], -1, wq.O)[self.images]).reshape(-1, wq.O)
        assert np.array_equal(got_acc, acc_o), f"{name}: int32 accumulators differ"
        self._check_out(name, out, y_o, act)
        rr = r if isinstance(r, tuple) else (r,)
        if f32_out:
            assert torch.equal(rr[0], out), f"{name}: f32 output differs between calls"
        if s_out is not None:
            assert torch.equal(rr[1], full[1]), f"{name}: twin differs between calls"
            y_dev = n(out[self.images]).transpose(0, 2, 3, 1)
            assert np.array_equal(n(rr[1][self.images]), Q.quantize_with_scale(y_dev, n(s_out)[0])), \
                f"{name}: twin differs"
        return r

    def dwconv_i8_nhwc(self, qx, sa, wq, stride=1, pad=0, bias=None, act=I.ACT_NONE, want_acc=False):
        r = self.real["dwconv_i8_nhwc"](qx, sa, wq, stride, pad, bias, act, want_acc)
        self._count("dwconv_i8_nhwc")
        out = r[0] if want_acc else r
        name, mod = self._layer(wq)
        C = wq.C
        wp = np.zeros((wq.cpad, 1, wq.KH, wq.KW), np.float32)
        wp[:C] = n(mod.weight)
        qw_o, sw_o = Q.quantize_dw_weight(wp)
        assert np.array_equal(n(wq.q), qw_o) and np.array_equal(n(wq.s), sw_o), f"{name}: packing differs"
        acc_o = Q.dwconv_i8_nhwc(n(qx[self.images]), qw_o, wq.KH, wq.KW, stride, pad)
        _, acc = self.real["dwconv_i8_nhwc"](qx, sa, wq, stride, pad, bias, act, want_acc=True)
        assert np.array_equal(n(acc[self.images]), acc_o), f"{name}: int32 accumulators differ"
        bp = np.zeros(wq.cpad, np.float32)
        if bias is not None:
            bp[: bias.numel()] = n(bias)
        y_o = OM._act(Q.dequant(acc_o.reshape(-1, wq.cpad), n(sa)[0], sw_o, bp), act).reshape(acc_o.shape)
        self._check_out(name, out, y_o, act)
        return r


def _b64(dev, seed=0):
    model = nets.build("efficientnet_b0", seed=seed, device=dev)
    assert bt.quantize_for_int8(model) == 49
    return model


def test_c4_b64_dynamic_calls(dev):
    say(f"C4 EfficientNet-B0 b64 at 224, dynamic scales: every int8 call, images {IMAGES}")
    model = _b64(dev)
    x = torch.from_numpy(WL.c4_input(64, 0)).to(dev)
    with Recorder(model, IMAGES) as rec, torch.no_grad():
        y = model(x)
    say(f"  calls checked: {rec.counts}")
    assert rec.counts["conv2d_nchw_fq"] == 1  # the stem, its input quantization fused
    # the 112^2 and 56^2 expansions feed their depthwise convs through the dynamic twin
    assert rec.counts["conv2d_i8_nhwc_dq"] == 3
    assert rec.counts["conv2d_i8_nhwc"] == 29 and rec.counts["dwconv_i8_nhwc"] == 16
    assert rec.counts["quantize_nhwc_chscale"] == 16
    assert torch.isfinite(y).all()


def test_c4_b64_calibrated_calls(dev):
    say(f"C4 EfficientNet-B0 b64 at 224, calibrated: every int8 call, images {IMAGES}")
    model = _b64(dev)
    calib = [torch.from_numpy(WL.c4_input(64, s)).to(dev) for s in (11,)]
    assert bt.calibrate_int8(model, calib) == 49
    x = torch.from_numpy(WL.c4_input(64, 0)).to(dev)
    with Recorder(model, IMAGES) as rec, torch.no_grad():
        y = model(x)
    say(f"  calls checked: {rec.counts}")
    assert rec.counts.get("conv2d_i8_nhwc_q_twin_only") == 15  # every expand conv: its twin alone
    assert rec.counts["dwconv_i8_nhwc"] == 16
    assert rec.counts.get("quantize_nhwc_chscale_static") == 16  # each projection input, gate folded in
    # the stem quantizes the network input itself and writes a twin; 12 projections (O % 16
    # == 0) and the head write a twin; the 4 projections with O = 24 or 40 cannot, so those
    # 4 outputs take a static pass
    assert rec.counts.get("conv2d_nchw_fq_static_twin") == 1
    assert rec.counts.get("conv2d_i8_nhwc_q") == 13 and rec.counts.get("conv2d_i8_nhwc") == 4
    assert rec.counts.get("quantize_nhwc_scaled", 0) == 4
    assert "quantize_nhwc" not in rec.counts
    assert torch.isfinite(y).all()
