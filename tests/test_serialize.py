"""The int8-perchannel on-disk format: packed weights round-trip bit for bit, geometry is
checked, and a loaded model runs the same forward as a freshly quantized one."""
import numpy as np
import pytest
import torch

import borch_amd as bt
from borch_amd import int8 as I
from oracle import quant as O


def _small(seed=0):
    torch.manual_seed(seed)
    m = torch.nn.Sequential(bt.nn.Conv2d(3, 24, 3, 1, 1), torch.nn.ReLU(),
                            bt.nn.Conv2d(24, 24, 3, 2, 1, groups=24),
                            torch.nn.Flatten(), bt.nn.Linear(24 * 4 * 4, 10))
    return m.eval()


def _pack_on_cpu(m):
    """Attach oracle packings as CPU tensors (no GPU needed to exercise the format)."""
    c, dw, lin = m[0], m[2], m[4]
    q, s = O.quantize_conv_weight(c.weight.detach().numpy(), 16)
    c.int8 = I.Int8ConvWeight(torch.from_numpy(q), torch.from_numpy(s), 24, 3, 16, 3, 3)
    q, s = O.quantize_dw_weight(dw.weight.detach().numpy())
    dw.int8 = I.Int8DwWeight(torch.from_numpy(q), torch.from_numpy(s), 24, 24, 3, 3)
    q, s = O.quantize_weight_per_channel(lin.weight.detach().numpy())
    lin.int8 = I.Int8Weight(torch.from_numpy(q), torch.from_numpy(s), 384, 10)


def test_round_trip_cpu(tmp_path):
    m = _small()
    _pack_on_cpu(m)
    f = tmp_path / "m.safetensors"
    assert bt.save_int8(m, f) == 3
    m2 = _small()
    assert bt.load_int8(m2, f, device="cpu") == 3
    for a, b in ((m[0], m2[0]), (m[2], m2[2]), (m[4], m2[4])):
        assert type(a.int8) is type(b.int8)
        assert torch.equal(a.int8.q, b.int8.q) and torch.equal(a.int8.s, b.int8.s)
        assert a.int8.q.dtype == torch.int8


def test_geometry_mismatch_raises(tmp_path):
    m = _small()
    _pack_on_cpu(m)
    f = tmp_path / "m.safetensors"
    bt.save_int8(m, f)
    other = torch.nn.Sequential(bt.nn.Conv2d(3, 24, 5, 1, 2), torch.nn.ReLU(),
                                bt.nn.Conv2d(24, 24, 3, 2, 1, groups=24),
                                torch.nn.Flatten(), bt.nn.Linear(24 * 4 * 4, 10))
    with pytest.raises(ValueError, match="layer '0'"):
        bt.load_int8(other, f, device="cpu")


def test_not_int8_file_raises(tmp_path):
    from safetensors.torch import save_file
    f = tmp_path / "plain.safetensors"
    save_file({"w": torch.zeros(2)}, str(f))
    with pytest.raises(ValueError, match="int8-perchannel"):
        bt.load_int8(_small(), f, device="cpu")


@pytest.mark.gpu
def test_loaded_model_matches_quantized_gpu(dev, tmp_path):
    from borch_amd import nets, workloads as WL
    model = nets.build("resnet18", seed=0, device=dev)
    assert bt.quantize_for_int8(model) == 20
    f = tmp_path / "r18.safetensors"
    assert bt.save_int8(model, f) == 20
    fresh = nets.build("resnet18", seed=0, device=dev)
    assert bt.load_int8(fresh, f) == 20
    for (n1, a), (n2, b) in zip(bt.nn._int8_layers(model), bt.nn._int8_layers(fresh)):
        assert n1 == n2 and torch.equal(a.int8.q, b.int8.q) and torch.equal(a.int8.s, b.int8.s)
    x = torch.from_numpy(WL.c3_input(4, 5)).to(dev)
    with torch.no_grad():
        assert torch.equal(model(x), fresh(x))


@pytest.mark.parametrize("layer,bad_q,bad_s", [
    ("0", (2, 16), (1,)),      # conv: O=24, KH*KW*cpad=144 expected
    ("0", (24, 144), (23,)),
    ("2", (9, 20), (24,)),     # depthwise: [9, 24] / [24] expected
    ("4", (10, 368), (10,)),   # linear: [10, 384] / [10] expected (a shorter q.shape[1] changes Kpad)
])
def test_truncated_tensor_raises(tmp_path, layer, bad_q, bad_s):
    """The kernels size their reads from the geometry record: a packed tensor of any other
    shape is refused on load instead of being read past its end."""
    from safetensors.torch import load_file, save_file
    from safetensors import safe_open
    m = _small()
    _pack_on_cpu(m)
    f = tmp_path / "m.safetensors"
    bt.save_int8(m, f)
    with safe_open(str(f), framework="pt") as h:
        meta = h.metadata()
    t = load_file(str(f))
    t[f"{layer}.q"] = torch.zeros(bad_q, dtype=torch.int8)
    t[f"{layer}.scale"] = torch.ones(bad_s, dtype=torch.float32)
    g = tmp_path / "bad.safetensors"
    save_file(t, str(g), metadata=meta)
    with pytest.raises(ValueError, match=f"layer '{layer}' has q"):
        bt.load_int8(_small(), g, device="cpu")
