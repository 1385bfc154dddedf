"""The product's BN fold (``borch_amd.nn.utils.fusion``, borch/_nn.py:4916-4955) and the
surface's torch error texts, on the CPU.

The fold is held three ways: bit for bit to the oracle's restatement (the same f32
operations in the same order), to torch's own ``torch.nn.utils.fusion`` (a different
operation order: rsqrt, so within a few ulps), and to the unfolded eval conv followed by
its BatchNorm (the mathematics it must equal). A whole model is checked too: the folded
ResNet-18 and EfficientNet-B0 give the unfolded models' f32 logits.
"""
import numpy as np
import pytest
import torch

import borch_amd as bt
from borch_amd import int8 as I
from borch_amd import nets
from borch_amd.nn.utils.fusion import fuse_conv_bn_eval, fuse_conv_bn_weights
from oracle import quant as O


def _bn(c, rng, affine=True):
    bn = torch.nn.BatchNorm2d(c, affine=affine).eval()
    with torch.no_grad():
        bn.running_mean.copy_(torch.from_numpy(rng.normal(size=c).astype(np.float32) * 0.3))
        bn.running_var.copy_(torch.from_numpy(rng.uniform(0.2, 2.0, c).astype(np.float32)))
        if affine:
            bn.weight.copy_(torch.from_numpy((1 + 0.3 * rng.normal(size=c)).astype(np.float32)))
            bn.bias.copy_(torch.from_numpy((0.2 * rng.normal(size=c)).astype(np.float32)))
    return bn


CASES = [  # (cin, cout, k, stride, pad, groups, conv bias, bn affine)
    (3, 16, 3, 1, 1, 1, False, True),
    (8, 24, 1, 1, 0, 1, True, True),
    (16, 32, 3, 2, 1, 1, True, False),
    (24, 24, 5, 1, 2, 24, False, True),  # depthwise
    (12, 20, 3, 1, 0, 1, False, False),
]


@pytest.mark.parametrize("case", CASES)
def test_fold_matches_oracle_torch_and_unfolded(case):
    cin, cout, k, s, p, g, has_b, affine = case
    rng = np.random.default_rng(cin * 100 + cout)
    conv = bt.nn.Conv2d(cin, cout, k, s, p, groups=g, bias=has_b).eval()
    bn = _bn(cout, rng, affine)
    fused = fuse_conv_bn_eval(conv, bn)
    fw, fb = fused.weight.detach().numpy(), fused.bias.detach().numpy()
    # the oracle restatement: bit for bit
    ow, ob = O.fuse_conv_bn_weights(conv.weight.detach().numpy(), None if conv.bias is None else
                                    conv.bias.detach().numpy(), bn.running_mean.numpy(), bn.running_var.numpy(),
                                    bn.eps, None if bn.weight is None else bn.weight.detach().numpy(),
                                    None if bn.bias is None else bn.bias.detach().numpy())
    assert np.array_equal(fw, ow) and np.array_equal(fb, ob)
    # torch's own fold (rsqrt, another operation order): within a few ulps
    tconv = torch.nn.Conv2d(cin, cout, k, s, p, groups=g, bias=has_b).eval()
    with torch.no_grad():
        tconv.weight.copy_(conv.weight)
        if has_b:
            tconv.bias.copy_(conv.bias)
    tf = torch.nn.utils.fusion.fuse_conv_bn_eval(tconv, bn)
    np.testing.assert_allclose(fw, tf.weight.detach().numpy(), rtol=2e-6, atol=1e-7)
    np.testing.assert_allclose(fb, tf.bias.detach().numpy(), rtol=2e-6, atol=1e-6)
    # the unfolded eval conv -> BN it replaces, in f32
    x = torch.from_numpy(rng.normal(size=(2, cin, 11, 11)).astype(np.float32))
    with torch.no_grad():
        ref = bn(conv(x)).numpy()
        got = fused(x).numpy()
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5 * np.abs(ref).max())
    # the original layers are untouched
    assert fused is not conv and fused.weight is not conv.weight


def test_fold_weights_keep_torch_signature():
    rng = np.random.default_rng(1)
    w = torch.from_numpy(rng.normal(size=(6, 4, 3, 3)).astype(np.float32))
    bn = _bn(6, rng)
    fw, fb = fuse_conv_bn_weights(w, None, bn.running_mean, bn.running_var, bn.eps, bn.weight, bn.bias)
    assert isinstance(fw, torch.nn.Parameter) and isinstance(fb, torch.nn.Parameter)
    assert fw.shape == w.shape and fb.shape == (6,) and fw.dtype == fb.dtype == torch.float32
    # transpose=True scales the second axis (a transposed conv's output channels)
    wt = torch.from_numpy(rng.normal(size=(4, 6, 3, 3)).astype(np.float32))
    ft, _ = fuse_conv_bn_weights(wt, None, bn.running_mean, bn.running_var, bn.eps, bn.weight, bn.bias, True)
    scale = bn.weight.detach() / torch.sqrt(bn.running_var + bn.eps)
    assert torch.equal(ft.detach(), wt * scale.reshape(1, -1, 1, 1))


def test_fold_refusals_have_torch_texts():
    conv, bn = bt.nn.Conv2d(4, 4, 3), torch.nn.BatchNorm2d(4)
    with pytest.raises(AssertionError, match="^Fusion only for eval!$"):
        fuse_conv_bn_eval(conv.eval(), bn.train())
    bn2 = torch.nn.BatchNorm2d(4, track_running_stats=False).eval()
    with pytest.raises(AssertionError, match="running_mean and bn.running_var must not be None"):
        fuse_conv_bn_eval(conv.eval(), bn2)


def test_fold_drops_stale_calibrated_scales():
    """A conv calibrated before the fold keeps nothing that describes the unfolded layer."""
    conv = bt.nn.Conv2d(4, 8, 3, padding=1).eval()
    conv.in_scale, conv.in_scale_v = torch.tensor([0.5]), 0.5
    conv.out_scale, conv.out_scale_v = torch.tensor([0.25]), 0.25
    fused = fuse_conv_bn_eval(conv, _bn(8, np.random.default_rng(2)))
    assert fused.int8 is None and fused.in_scale is None and fused.out_scale is None
    assert fused.in_scale_v is None and fused.out_scale_v is None
    assert conv.in_scale_v == 0.5  # the original keeps its own


@pytest.mark.parametrize("name,shape", [("resnet18", (2, 3, 32, 32)), ("efficientnet_b0", (1, 3, 64, 64))])
def test_folded_model_matches_unfolded_f32(name, shape):
    """The folded network's f32 logits equal the unfolded eval network's (conv, BN, ...)."""
    ctor = {"resnet18": nets.ResNet18, "efficientnet_b0": nets.EfficientNetB0}[name]
    model = nets.init_weights(ctor(), seed=4).eval()
    x = torch.from_numpy(np.random.default_rng(4).uniform(0, 1, shape).astype(np.float32))
    with torch.no_grad():
        ref = model(x).numpy()
        model.fuse()
        got = model(x).numpy()
        again = model.fuse()(x).numpy()  # a second fuse() is a no-op
    np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-4 * np.abs(ref).max())
    assert np.array_equal(again, got)


def test_compiled_fuses_a_built_model_once():
    """compiled(fuse=True) on a model nets.build() already folded: fuse() runs again and
    must leave it as it is."""
    model = nets.build("resnet18", seed=0, device="cpu")
    x = torch.from_numpy(np.random.default_rng(5).uniform(0, 1, (1, 3, 32, 32)).astype(np.float32))
    with torch.no_grad():
        ref = model(x)
    c = bt.compiled(model, int8=False, fuse=True, tune=False)
    with torch.no_grad():
        assert torch.equal(c(x), ref)
    vit = nets.build("vit_b16", seed=0, device="cpu")
    first = vit.layers[0].proj_f
    vit.fuse()
    assert vit.layers[0].proj_f is first


# ------------------------------------------------------------ torch error texts (surface)

def test_linear_shape_error_text():
    """borch/_tensor.py:924-931: "mat1 and mat2 shapes cannot be multiplied (AxB and CxD)"."""
    lin = bt.nn.Linear(4, 3)
    with pytest.raises(RuntimeError, match=r"^mat1 and mat2 shapes cannot be multiplied \(2x5 and 4x3\)$"):
        lin(torch.zeros(2, 5))
    with pytest.raises(RuntimeError, match=r"^mat1 and mat2 shapes cannot be multiplied \(6x5 and 4x3\)$"):
        bt.nn.functional.linear(torch.zeros(2, 3, 5), lin.weight)
    # an int8-packed Linear checks the same before any device work
    w8 = I.Int8Weight(torch.zeros((3, 16), dtype=torch.int8), torch.ones(3), 4, 3)
    with pytest.raises(RuntimeError, match=r"^mat1 and mat2 shapes cannot be multiplied \(2x5 and 4x3\)$"):
        I.linear(torch.zeros(2, 5), w8)
    w8.weight_only = True
    with pytest.raises(RuntimeError, match=r"^mat1 and mat2 shapes cannot be multiplied \(2x5 and 4x3\)$"):
        I.linear(torch.zeros(2, 5), w8)


def test_conv_channel_error_text():
    """borch/_ops.py:762: "channels do not match: input C, filter C'"."""
    conv = bt.nn.Conv2d(3, 8, 3)
    with pytest.raises(RuntimeError, match=r"^channels do not match: input 4, filter 3$"):
        conv(torch.zeros(1, 4, 8, 8))
    with pytest.raises(RuntimeError, match=r"^channels do not match: input 4, filter 3$"):
        bt.nn.functional.conv2d(torch.zeros(1, 4, 8, 8), conv.weight)
    w8 = I.Int8ConvWeight(torch.zeros((8, 9 * 16), dtype=torch.int8), torch.ones(8), 8, 3, 16, 3, 3)
    with pytest.raises(RuntimeError, match=r"^channels do not match: input 4, filter 3$"):
        I.conv2d(torch.zeros(1, 4, 8, 8), w8)
    dw8 = I.Int8DwWeight(torch.zeros((9, 8), dtype=torch.int8), torch.ones(8), 8, 8, 3, 3)
    with pytest.raises(RuntimeError, match=r"^channels do not match: input 4, filter 8$"):
        I.depthwise_conv2d(torch.zeros(1, 4, 8, 8), dw8)
