"""The C restatement of borch_cpu's f32 kernels (oracle/cpu_ref.c), checked against
float64 numpy, the oracle's im2col and torch's f32 model (the CPU baseline must compute
the same thing the GPU path does, or its timing means nothing)."""
import numpy as np
import pytest

from oracle import cpu_ref as R
from oracle import quant as O


def test_gemm_bias_act_matches_f64():
    rng = np.random.default_rng(0)
    for m, k, n, act in ((37, 96, 48, 1), (4, 16, 16, 0), (1, 300, 64, 0), (9, 1024, 32, 1)):
        a = rng.normal(size=(m, k)).astype(np.float32)
        b = rng.normal(size=(k, n)).astype(np.float32)
        bias = rng.normal(size=n).astype(np.float32)
        ref = a.astype(np.float64) @ b + bias
        if act:
            ref = np.maximum(ref, 0)
        for t in (1, 3):
            np.testing.assert_allclose(R.gemm(a, b, bias, act, nthreads=t), ref, rtol=1e-4, atol=1e-4)


def test_im2col_rows_matches_oracle_exactly():
    rng = np.random.default_rng(1)
    x = rng.normal(size=(1, 7, 6, 8)).astype(np.float32)
    for k, s, p in ((3, 1, 1), (3, 2, 1), (5, 1, 2), (1, 2, 0)):
        cols, OH, OW = O.im2col_nhwc(x, k, k, s, p)
        got = R.im2col_rows(x[0], k, s, p, 0, OH * OW)
        assert np.array_equal(got, cols)
        part = R.im2col_rows(x[0], k, s, p, 3, 5)
        assert np.array_equal(part, cols[3:8])


def test_dwconv_rows_matches_direct_sum():
    rng = np.random.default_rng(2)
    h, w, c = 9, 8, 32
    x = rng.normal(size=(h, w, c)).astype(np.float32)
    for k, s, p in ((3, 1, 1), (3, 2, 1), (5, 1, 2), (5, 2, 2)):
        wt = rng.normal(size=(k, k, c)).astype(np.float32)
        bias = rng.normal(size=c).astype(np.float32)
        got = R.dwconv(x, wt, k, s, p, bias, 1)
        xp = np.zeros((h + 2 * p, w + 2 * p, c))
        xp[p:p + h, p:p + w] = x
        ho, wo = got.shape[:2]
        ref = np.zeros((ho, wo, c)) + bias
        for ky in range(k):
            for kx in range(k):
                ref += xp[ky:ky + s * (ho - 1) + 1:s, kx:kx + s * (wo - 1) + 1:s] * wt[ky, kx]
        np.testing.assert_allclose(got, np.maximum(ref, 0), rtol=1e-4, atol=1e-4)


def test_conv2d_nhwc_matches_f32_conv():
    rng = np.random.default_rng(3)
    x = rng.normal(size=(3, 16, 10, 10)).astype(np.float32)
    wgt = rng.normal(size=(32, 16, 3, 3)).astype(np.float32)
    b = rng.normal(size=32).astype(np.float32)
    for s, p in ((1, 1), (2, 1)):
        ref = O.conv2d_f32(x, wgt, b, s, p)
        wcol = wgt.transpose(2, 3, 1, 0).reshape(9 * 16, 32)
        got = R.conv2d_nhwc(x.transpose(0, 2, 3, 1), wcol, 3, s, p, b, 0, nthreads=2, block=7)
        np.testing.assert_allclose(got.transpose(0, 3, 1, 2), ref, rtol=1e-4, atol=1e-4)


def test_resnet18_forward_matches_torch_f32():
    torch = pytest.importorskip("torch")
    from borch_amd import nets, workloads as WL
    model = nets.build("resnet18", seed=3, device="cpu")
    x = WL.c3_input(2, 3)
    with torch.no_grad():
        ref = model(torch.from_numpy(x)).numpy()

    def cp(conv):
        s, p = conv._geometry()
        return (conv.weight.detach().numpy(), conv.bias.detach().numpy(), s, p)
    params = {"stem": cp(model.stem_f.conv), "fc": (model.fc.weight.detach().numpy(), model.fc.bias.detach().numpy())}
    for i, blk in enumerate(model.body):
        params[f"body.{i}.c1"] = cp(blk.c1.conv)
        params[f"body.{i}.c2"] = cp(blk.c2.conv)
        if blk.down is not None:
            params[f"body.{i}.down"] = cp(blk.down)
    got = R.resnet18_forward(params, x, nthreads=4)
    np.testing.assert_allclose(got, ref, rtol=1e-3, atol=1e-3)


# --------------------------------------------- the numpy core's f32 forward (oracle/numpy_core.py)

def test_numpy_core_im2col_brute_force():
    """borch/_ops.py:671-689's row layout: row (n, oh, ow), column (c, kh, kw)."""
    from oracle import numpy_core as NC
    rng = np.random.default_rng(4)
    x = rng.normal(size=(2, 3, 7, 6)).astype(np.float32)
    for k, s in ((3, 1), (3, 2), (1, 2), (2, 3)):
        cols, OH, OW = NC.im2col(x, k, k, s)
        want = np.zeros((2 * OH * OW, 3 * k * k), np.float32)
        for n_ in range(2):
            for oh in range(OH):
                for ow in range(OW):
                    r = (n_ * OH + oh) * OW + ow
                    for c in range(3):
                        for i in range(k):
                            for j in range(k):
                                want[r, (c * k + i) * k + j] = x[n_, c, oh * s + i, ow * s + j]
        assert np.array_equal(cols, want)


def test_numpy_core_conv_and_linear_match_torch():
    torch = pytest.importorskip("torch")
    from oracle import numpy_core as NC
    rng = np.random.default_rng(5)
    for (C, O, k, s, p) in ((3, 8, 3, 1, 1), (16, 32, 3, 2, 1), (16, 8, 1, 2, 0), (4, 4, 5, 1, 2)):
        x = rng.normal(size=(2, C, 9, 9)).astype(np.float32)
        w = rng.normal(size=(O, C, k, k)).astype(np.float32)
        b = rng.normal(size=O).astype(np.float32)
        ref = torch.nn.functional.conv2d(torch.from_numpy(x), torch.from_numpy(w), torch.from_numpy(b), s, p).numpy()
        np.testing.assert_allclose(NC.conv2d(x, w, b, s, p), ref, rtol=1e-4, atol=1e-4)
    with pytest.raises(RuntimeError, match="channels do not match: input 3, filter 4"):
        NC.conv2d(np.zeros((1, 3, 5, 5), np.float32), np.zeros((2, 4, 3, 3), np.float32))
    x = rng.normal(size=(5, 33)).astype(np.float32)
    w = rng.normal(size=(7, 33)).astype(np.float32)
    b = rng.normal(size=7).astype(np.float32)
    np.testing.assert_allclose(NC.linear(x, w, b), x.astype(np.float64) @ w.T.astype(np.float64) + b, rtol=1e-5,
                               atol=1e-5)


def test_numpy_core_resnet18_matches_torch_f32():
    torch = pytest.importorskip("torch")
    from borch_amd import nets, workloads as WL
    from oracle import numpy_core as NC
    model = nets.build("resnet18", seed=3, device="cpu")
    x = WL.c3_input(2, 3)
    with torch.no_grad():
        ref = model(torch.from_numpy(x)).numpy()

    def cp(conv):
        s, p = conv._geometry()
        return (conv.weight.detach().numpy(), conv.bias.detach().numpy(), s, p)
    params = {"stem": cp(model.stem_f.conv), "fc": (model.fc.weight.detach().numpy(), model.fc.bias.detach().numpy())}
    for i, blk in enumerate(model.body):
        params[f"body.{i}.c1"] = cp(blk.c1.conv)
        params[f"body.{i}.c2"] = cp(blk.c2.conv)
        if blk.down is not None:
            params[f"body.{i}.down"] = cp(blk.down)
    np.testing.assert_allclose(NC.resnet18_forward(params, x), ref, rtol=1e-3, atol=1e-3)
