"""Host-side logic of the weight window (no GPU): the slot bookkeeping of
borch-ts/src/device.ts:3015-3165, the host int8 packer in its three rounding rules against
the oracle, and the refusals of a windowed weight."""
import types

import numpy as np
import pytest
import torch

from borch_amd import streaming as S
from oracle import quant as O


def test_regions_place_align_and_reuse():
    r = S.Regions(4096, 256)
    a = r.reserve(20)
    b = r.reserve(20)
    assert (a[0], b[0]) == (0, 256)  # window_probe.html:26-34: offsets 0 and align
    assert r.used == 512 and r.live == 512
    assert r.gen_of(0) == a[1] and r.gen_of(256) == b[1] and r.gen_of(512) == -1
    r.release(0, "evt-a")
    assert r.gen_of(0) != a[1]  # a stale use of the slot is detectable
    assert r.live == 256 and r.used == 512
    c = r.reserve(100)
    assert c[0] == 0 and c[2] == "evt-a"  # the freed region, with its eviction token
    assert r.used == 512  # reuse does not grow the cursor


def test_regions_first_fit_takes_region_whole():
    r = S.Regions(1 << 20, 256)
    big = r.reserve(1000)  # 1024 bytes
    small = r.reserve(10)
    r.release(big[0])
    got = r.reserve(10)
    assert got[0] == big[0]
    assert r.reserved[big[0]] == 1024  # taken whole: its full size returns on the next eviction
    r.release(got[0])
    r.release(small[0])
    assert r.live == 0


def test_regions_full_raises_reference_text():
    r = S.Regions(1024, 256)
    for _ in range(4):
        r.reserve(256)
    with pytest.raises(S.WindowFull, match=r"window is full: 1024 \+ 256 > 1024 bytes, and no freed region fits"):
        r.reserve(1)


def test_regions_stream_many_through_three():
    """24 equal blocks through room for three (window_probe.html:160-183): the cursor stays
    at three blocks."""
    need = 16 * 16 * 4
    cap = 3 * need
    r = S.Regions(cap, 256)
    live = []
    for i in range(24):
        live.append(r.reserve(need)[0])
        if len(live) == 2:  # the scheduler keeps block k and k+1
            r.release(live.pop(0))
    assert r.used <= cap


@pytest.mark.parametrize("rounding,oracle_fn", [
    ("exact", O.quantize_weight_per_channel),
    ("reference", O.quantize_weight_reference_linear),
    ("reference_conv", O.quantize_conv_weight_reference),
])
def test_host_packer_matches_oracle(rounding, oracle_fn):
    rng = np.random.default_rng(5)
    for N, K in [(512, 512), (64, 27), (33, 100), (7, 16), (3, 0 + 16)]:
        w = (rng.normal(size=(N, K)) / np.sqrt(K)).astype(np.float32)
        w[1] = 0.0  # a zero row: scale 0, bytes 0 (quant.ts:36)
        hw = S.pack_int8_host(w, rounding=rounding)
        q0, s0 = oracle_fn(w)
        kp = hw.q.shape[1]
        assert kp % 16 == 0 and kp >= K
        assert np.array_equal(hw.q.numpy()[:, :K], q0)
        assert not hw.q.numpy()[:, K:].any()
        assert np.array_equal(hw.s.numpy().view(np.uint32), s0.view(np.uint32))
    # exact ties and the two roundings (half to even / half toward +inf)
    w = np.array([[127.0, 2.5, -2.5, 1.5, -1.5, 0.5, -0.5, 3.5] + [0.0] * 8], np.float32)
    assert np.array_equal(S.pack_int8_host(w, rounding=rounding).q.numpy()[:, :16], oracle_fn(w)[0])


def test_host_packer_at_c2_reproduces_the_reference_bytes():
    """The 12 bytes of C2's weight where borch-ts's packer differs from the exact rule come
    out of the host packer in either rule as the oracle says; threads do not change bytes."""
    from borch_amd import workloads as WL
    _, w, _ = WL.c2_gemm(1, 0)
    ex = S.pack_int8_host(w, rounding="exact", threads=1).q.numpy()
    ref = S.pack_int8_host(w, rounding="reference").q.numpy()
    assert np.array_equal(ex, O.quantize_weight_per_channel(w)[0])
    assert np.array_equal(ref, O.quantize_weight_reference_linear(w)[0])
    assert int((ex != ref).sum()) == 12
    assert np.array_equal(S.pack_int8_host(w, rounding="exact", threads=3).q.numpy(), ex)


def test_host_packer_shapes_and_refusals():
    w = np.arange(2 * 3 * 3 * 3, dtype=np.float32).reshape(2, 3, 3, 3) - 20
    hw = S.pack_int8_host(w)  # a conv-shaped weight: per output channel over C*KH*KW
    assert hw.shape == (2, 3, 3, 3) and hw.q.shape == (2, 32) and hw.in_features == 27
    assert np.array_equal(hw.q.numpy()[:, :27], O.quantize_weight_per_channel(w.reshape(2, 27))[0])
    with pytest.raises(ValueError, match="rounding"):
        S.pack_int8_host(w, rounding="half-up")
    with pytest.raises(ValueError, match="does not have the shape"):
        S.pack_int8_host(w, shape=(5, 5))


def _fake_weight(kind="f32"):
    """A windowed weight over host-side bookkeeping only (no device buffer)."""
    regions = S.Regions(1 << 16)
    off, gen, _ = regions.reserve(64)
    win = types.SimpleNamespace(_open=True, regions=regions, device=torch.device("cpu"))
    win.evict = lambda slot: regions.release(slot.offset)
    slot = S.Slot(win, off, 64, gen, None)
    return S.WindowedWeight(slot, (4, 4), kind)


def test_windowed_weight_refuses_generic_ops():
    ww = _fake_weight()
    t = torch.ones(4, 4)
    for op in (lambda: torch.add(ww, t), lambda: t + ww, lambda: torch.relu(ww), lambda: t.add(ww)):
        with pytest.raises(RuntimeError, match="weight operand only"):
            op()


def test_windowed_weight_use_after_evict_raises():
    ww = _fake_weight("int8")
    ww.evict()
    x = torch.ones(2, 4)
    with pytest.raises(RuntimeError, match="was evicted — its slot holds another weight now"):
        torch.nn.functional.linear(x, ww)
    with pytest.raises(RuntimeError, match="evicted"):
        x @ ww
    from borch_amd.nn import functional as F
    with pytest.raises(RuntimeError, match="evicted"):
        F.linear(x, ww)
    assert "evicted" in repr(ww)
