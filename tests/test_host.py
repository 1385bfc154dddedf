"""Host-side logic of the int8 surface (no GPU): which layers the int8 kernels take, under
this library's rule and under the reference's (borch-ts/src/kernels.ts:2096-2103)."""
import pytest
import torch

import borch_amd as bt
from borch_amd import nets
from borch_amd.nn import Conv2d, _int8_layers


def _convs(model):
    return [m for _, m in _int8_layers(model) if isinstance(m, Conv2d)]


def test_resnet18_layer_rules():
    model = nets.build("resnet18", seed=0, device="cpu")
    convs = _convs(model)
    assert len(convs) == 20
    assert sum(c.int8_refusal() is None for c in convs) == 20
    # The reference's convInt8Fits takes 13 of the 20: not the stem (C = 3), the three
    # stride-2 3x3 convs or the three stride-2 1x1 downsamples.
    refused = [c.reference_rule_refusal() for c in convs]
    assert sum(r is None for r in refused) == 13
    assert sorted(r for r in refused if r is not None) == ["in_channels=3 not a multiple of 32"] + ["stride 2"] * 6


def test_efficientnet_depthwise_not_in_reference_rule():
    model = nets.build("efficientnet_b0", seed=0, device="cpu")
    convs = _convs(model)
    dw = [c for c in convs if c.groups != 1]
    assert dw and all(c.int8_refusal() is None for c in dw)
    assert all(c.reference_rule_refusal() == f"groups={c.groups}" for c in dw)


def test_reference_rule_refusals_by_name():
    assert Conv2d(3, 64, 3, padding=1).reference_rule_refusal() == "in_channels=3 not a multiple of 32"
    assert Conv2d(64, 128, 3, stride=2, padding=1).reference_rule_refusal() == "stride 2"
    assert Conv2d(64, 64, 5, padding=2).reference_rule_refusal() == "kernel 5x5 > 3"
    assert Conv2d(64, 40, 1).reference_rule_refusal() == "out_channels=40 not a multiple of 16"
    assert Conv2d(64, 64, 3, padding=1, groups=64).reference_rule_refusal() == "groups=64"
    assert Conv2d(64, 64, 3, padding=1, dilation=2).reference_rule_refusal().startswith("stride/padding")
    assert Conv2d(64, 64, 3, padding=1).reference_rule_refusal() is None


def test_rule_argument_checked():
    with pytest.raises(ValueError, match="rule must be"):
        bt.quantize_for_int8(torch.nn.Sequential(), rule="fast")
    with pytest.raises(ValueError, match="rule must be"):
        Conv2d(64, 64, 3, padding=1).quantize_int8("fast")


def test_bench_layer_work_matches_the_implicit_gemm_shapes():
    """bench.layer_work's GEMM view of a conv: M = N·OH·OW, N = O, K = KH·KW·Cpad, with
    ops 2·M·N·K. The ResNet-18 b16 shapes are the ones tabulated for the reference's
    implicit-GEMM conv (kernels.ts:2084-2302): (16384, 64, 576), stride-2 (4096, 128, 576),
    1×1 downsample (4096, 128, 64). Depthwise and dense GEMM shapes likewise."""
    import types
    import bench
    import torch

    def conv(n, h, c, o, k, s, p, kind="conv2d_i8_nhwc", residual=None):
        wq = types.SimpleNamespace(KH=k, KW=k, O=o)
        a = {"qx": torch.empty((n, h, h, c), dtype=torch.int8), "wq": wq, "stride": s, "pad": p,
             "residual": residual}
        return bench.layer_work(kind, a)

    assert conv(16, 32, 64, 64, 3, 1, 1)[0] == (16384, 64, 576)
    assert conv(16, 32, 64, 128, 3, 2, 1)[0] == (4096, 128, 576)
    assert conv(16, 32, 64, 128, 1, 2, 0)[0] == (4096, 128, 64)
    shape, ops, byts = conv(16, 4, 512, 512, 3, 1, 1)
    assert shape == (256, 512, 4608) and ops == 2 * 256 * 512 * 4608
    assert byts == 16 * 4 * 4 * 512 + 512 * 4608 + 4 * 256 * 512
    # the int8 twin adds a byte per output, a residual four
    r = torch.empty(1)
    assert conv(16, 4, 512, 512, 3, 1, 1, "conv2d_i8_nhwc_q", r)[2] == byts + 4 * 256 * 512 + 256 * 512
    # the twin alone: no f32 output
    wq = types.SimpleNamespace(KH=3, KW=3, O=512)
    a = {"qx": torch.empty((16, 4, 4, 512), dtype=torch.int8), "wq": wq, "stride": 1, "pad": 1, "residual": None,
         "f32_out": False}
    assert bench.layer_work("conv2d_i8_nhwc_q", a)[2] == byts - 4 * 256 * 512 + 256 * 512
    # depthwise 3x3 stride 2 on 112² x 96 at b64: 2·9 ops per output
    shape, ops, byts = conv(64, 112, 96, 96, 3, 2, 1, "dwconv_i8_nhwc")
    assert shape == (64 * 56 * 56, 96, 9) and ops == 2 * 9 * 64 * 56 * 56 * 96
    assert byts == 64 * 112 * 112 * 96 + 4 * 64 * 56 * 56 * 96 + 9 * 96
    a = {"qa": torch.empty((6304, 768), dtype=torch.int8), "qw": torch.empty((2304, 768), dtype=torch.int8),
         "residual": None}
    assert bench.layer_work("gemm_i8", a)[:2] == ((6304, 2304, 768), 2 * 6304 * 2304 * 768)


def test_vectors_reaching_the_kernels_have_their_full_length():
    """Bias / scale vectors are passed to the kernels as bare pointers: a short one is
    refused on the host instead of being read past its end."""
    import pytest
    import torch
    from borch_amd import int8 as I
    assert I._vec(None, 4, "bias") is None
    v = I._vec(torch.arange(4, dtype=torch.float64), 4, "bias")
    assert v.dtype == torch.float32 and v.is_contiguous() and v.tolist() == [0.0, 1.0, 2.0, 3.0]
    with pytest.raises(ValueError, match="expected 5 values, got 4"):
        I._vec(torch.zeros(4), 5, "bias")


def test_plan_cache_file(tmp_path, monkeypatch):
    """The plan table on disk: decisions stored per (device, library) and problem, merged on
    write, unreadable or foreign files read as empty, another library's table ignored."""
    from borch_amd import tune as T
    monkeypatch.setattr(T, "device_id", lambda device: "gfx950/256cu")
    c = T.PlanCache(tmp_path / "sub" / "plans.json")
    assert c.load("cuda:0") == {}
    assert c.store("cuda:0", {(256, 512, 4608): {"cfg": 9, "split": 8, "rule_us": 10.5, "chosen_us": 9.1}})
    assert c.store("cuda:0", {(16, 32, 32, 64, 64, 3, 3, 1, 1): {"cfg": 0, "split": 0, "rule_us": 7.0,
                                                                  "chosen_us": 7.0}})
    got = c.load("cuda:0")
    assert got[(256, 512, 4608)]["cfg"] == 9 and got[(16, 32, 32, 64, 64, 3, 3, 1, 1)]["cfg"] == 0
    monkeypatch.setattr(T, "_LIB_ID", "another-build")
    assert c.load("cuda:0") == {}
    (tmp_path / "bad.json").write_text("{not json")
    assert T.PlanCache(tmp_path / "bad.json").load("cuda:0") == {}
    monkeypatch.setenv("BORCH_AMD_PLAN_CACHE", str(tmp_path / "x.json"))
    assert T.default_cache_path() == tmp_path / "x.json"
