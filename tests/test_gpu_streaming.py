"""GPU: frozen weights streamed through a device window — the checks of the reference's
window probe (tests/browser/window_probe.html:26-270) restated for this surface, through the
C ABI (bq_quantize_weight_host, bq_linear_w8a32, bq_dequant_i8).

The reference's own inputs are its xorshift32 ``seed(n, s)`` values (window_probe.html:67).
Its int8 gate holds the windowed int8 Linear to the f32 op on the host-reconstructed weight
bit for bit; that holds there because both run the same matmul kernel in the same order.
Here the windowed weight runs the W8A32 kernel, so the gates are: bit-identical to the
same kernel on the resident packing; within the f32-accumulation bound of the float64
result on the reconstructed weight; and bit-identical to torch's f32 Linear on the
reconstructed weight on inputs where every sum is exact in f32 (any summation order).
"""
import sys

import numpy as np
import pytest
import torch

from borch_amd import int8 as I
from borch_amd import streaming as S
from borch_amd.nn import functional as F
from oracle import quant as O

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def seed(n: int, s: int) -> np.ndarray:
    """window_probe.html:67: xorshift32 (13, 17, 5) from ``s``, each value x / 2^32 - 0.5."""
    out = np.empty(n, np.float32)
    x = s & 0xFFFFFFFF
    for i in range(n):
        x ^= (x << 13) & 0xFFFFFFFF
        x ^= x >> 17
        x ^= (x << 5) & 0xFFFFFFFF
        out[i] = np.float32(x / 4294967296.0 - 0.5)
    return out


def n(x):
    return x.detach().cpu().numpy()


def test_window_slots_fill_and_read_back(dev):
    say("window: two slots of one buffer")
    win = S.window(1 << 20, dev)
    a = np.array([1, 2, 3, 4, 5], np.float32)
    b = np.array([10, 11, 12, 13, 14], np.float32)
    sa, sb = win.place(a), win.place(b)
    assert (sa.offset, sb.offset) == (0, S.ALIGN) and sb.offset % S.ALIGN == 0
    torch.cuda.current_stream().wait_event(sb.ready)
    torch.cuda.current_stream().wait_event(sa.ready)
    assert np.array_equal(n(sa.view(torch.float32, (5,))), a)
    assert np.array_equal(n(sb.view(torch.float32, (5,))), b)
    win2 = S.window(1 << 20, dev)
    sc = win2.place(np.array([7, 8, 9, 10, 11], np.float32))
    torch.cuda.current_stream().wait_event(sc.ready)
    assert n(sc.view(torch.float32, (5,))).tolist() == [7, 8, 9, 10, 11]
    assert win.used == 2 * S.ALIGN
    win.free()
    win2.free()


def _values(shape, s):
    """The probe's seed() values for small arrays; seeded normals past 2^16 values (the
    xorshift loop runs in Python)."""
    count = int(np.prod(shape))
    if count <= 1 << 16:
        return seed(count, s).reshape(shape)
    return (np.random.default_rng(s).normal(size=shape) / np.sqrt(shape[-1])).astype(np.float32)


def _int8_window_case(dev, M, K, N, xs, ws, rounding="exact"):
    w = _values((N, K), ws) if isinstance(ws, int) else ws
    x = _values((M, K), xs) if isinstance(xs, int) else xs
    win = S.window(4 * N * K + (1 << 16), dev)
    weight, evict = S.in_window_int8(win, w, (N, K), rounding=rounding)
    i8_live = win.live
    xt = torch.from_numpy(x).to(dev)
    got = n(F.linear(xt, weight))
    # the slot holds the host packer's bytes: the device packer's for the exact rule
    q_slot = n(weight.int8_weight().q)[:, :K]
    q_want, s_want = (O.quantize_weight_per_channel(w) if rounding == "exact"
                      else O.quantize_weight_reference_linear(w))
    assert np.array_equal(q_slot, q_want) and np.array_equal(n(weight.scales), s_want)
    # the same kernel on the resident packing: bit for bit
    if rounding == "exact":
        w8 = I.pack_linear_weight(torch.from_numpy(w).to(dev), weight_only=True)
        assert np.array_equal(n(w8.q)[:, :K], q_slot)
        assert np.array_equal(got, n(I.linear_w8a32(xt, w8)))
    y_o, bound = O.linear_w8a32(x, q_want, s_want)
    err = np.abs(got.astype(np.float64) - y_o)
    assert np.all(err <= bound + 1e-30)
    if M <= 4:  # the decode GEMV: bit for bit the f32 op on the reconstructed weight, in its order
        assert np.array_equal(got, O.linear_w8a32_gemv(x, q_want, s_want))
    # a quarter of an f32 slot
    gw = S.window(4 * N * K + (1 << 16), dev)
    S.in_window(gw, w, (N, K))
    f32_live = gw.live
    evict()
    gw.free()
    win.free()
    return i8_live, f32_live


@pytest.mark.parametrize("M,K,N,xs,ws", [(8, 16, 16, 92, 91),   # window_probe.html:219-233
                                          (16, 512, 512, 3, 4),  # C1's shape
                                          (1, 4096, 4096, 5, 6), (5, 1040, 300, 7, 8), (40, 768, 130, 9, 10)])
def test_int8_window_linear(dev, M, K, N, xs, ws):
    say(f"int8 window linear M={M} K={K} N={N}")
    i8_live, f32_live = _int8_window_case(dev, M, K, N, xs, ws)
    # a quarter of the f32 slot; each slot rounds up to the alignment, so a weight whose
    # bytes are not a multiple of it may take up to one alignment unit more
    assert i8_live <= f32_live // 4 + (0 if (N * K) % S.ALIGN == 0 else S.ALIGN)


def test_int8_window_reference_rounding(dev):
    """rounding="reference": the slot holds borch-ts's own Linear bytes (quant.ts:35-41),
    which differ from the exact rule on C2's weight in 12 places."""
    from borch_amd import workloads as WL
    say("int8 window, the reference's rounding, C2 weight")
    x, w, _ = WL.c2_gemm(1, 0)
    _int8_window_case(dev, 1, 4096, 4096, x, w, rounding="reference")


def test_int8_window_exact_grid_equals_f32_linear(dev):
    """On values where every product and partial sum is exact in f32 (w = k 2^-6 with each
    row's peak 127 2^-6, so s = 2^-6 and f32(q) s = w; x = j 2^-8 with |j| < 256, K = 256),
    the windowed int8 Linear equals torch's f32 Linear on the host-reconstructed weight
    (dequantInt8PerChannel, quant.ts:60-71) and the float64 result, bit for bit."""
    say("int8 window linear on an exact grid")
    rng = np.random.default_rng(3)
    M, K, N = 8, 256, 96
    k = rng.integers(-127, 128, size=(N, K))
    k[:, 0] = np.where(rng.random(N) < 0.5, -127, 127)
    w = (k * 2.0 ** -6).astype(np.float32)
    x = (rng.integers(-255, 256, size=(M, K)) * 2.0 ** -8).astype(np.float32)
    b = (rng.integers(-1000, 1000, size=N) * 2.0 ** -14).astype(np.float32)
    rec = O.dequant_weight(*O.quantize_weight_reference_linear(w))
    assert np.array_equal(rec, w)
    win = S.window(1 << 20, dev)
    weight, _ = S.in_window_int8(win, w, (N, K))
    xt, bt = torch.from_numpy(x).to(dev), torch.from_numpy(b).to(dev)
    got = n(F.linear(xt, weight, bt))
    want = (x.astype(np.float64) @ rec.astype(np.float64).T + b).astype(np.float32)
    assert np.array_equal(got, want)
    assert np.array_equal(got, n(torch.nn.functional.linear(xt, torch.from_numpy(rec).to(dev), bt)))
    win.free()


def test_int8_window_conv_and_matmul_unpack(dev):
    """A conv or a matmul reads an int8 window weight through the f32 unpack (the
    reference's conv funnel, window_probe.html:106-125): equal, bit for bit, to the same
    torch op on the host-reconstructed weight; the larger slot is a quarter of f32."""
    say("int8 window conv2d / matmul")
    for (N, C, H, Oc, kh, s) in [(1, 3, 8, 4, 3, 21), (1, 16, 16, 16, 3, 33)]:
        xd = seed(N * C * H * H, s).reshape(N, C, H, H)
        wd = seed(Oc * C * kh * kh, s + 5).reshape(Oc, C, kh, kh)
        rec = O.dequant_weight(*O.quantize_weight_per_channel(wd.reshape(Oc, -1))).reshape(wd.shape)
        xt = torch.from_numpy(xd).to(dev)
        ref = n(torch.nn.functional.conv2d(xt, torch.from_numpy(rec).to(dev), None, 1, 1))
        cw = S.window(1 << 20, dev)
        weight, _ = S.in_window_int8(cw, wd, wd.shape)
        got = n(torch.nn.functional.conv2d(xt, weight, None, 1, 1))
        assert np.array_equal(got, ref)
        assert np.array_equal(n(F.conv2d(xt, weight, None, 1, 1)), ref)
        if C == 16:
            gw = S.window(1 << 20, dev)
            S.in_window(gw, wd, wd.shape)
            assert cw.live <= gw.live // 4
            gw.free()
        cw.free()
    # matmul layout [K, N]: one scale per row of the stored array (shape[0]), unpacked
    Kd, Nn = 16, 16
    wd = seed(Kd * Nn, 71).reshape(Kd, Nn)
    rec = O.dequant_weight(*O.quantize_weight_per_channel(wd))
    x = torch.from_numpy(seed(8 * Kd, 72).reshape(8, Kd)).to(dev)
    mw = S.window(1 << 20, dev)
    weight, _ = S.in_window_int8(mw, wd, (Kd, Nn))
    assert np.array_equal(n(x @ weight), n(x @ torch.from_numpy(rec).to(dev)))
    assert np.array_equal(n(torch.matmul(x, weight)), n(x @ torch.from_numpy(rec).to(dev)))
    mw.free()


def test_window_evict_is_loud_and_generic_ops_refused(dev):
    say("window: eviction and refusals")
    ew = S.window(1 << 20, dev)
    wd = seed(16 * 16, 41).reshape(16, 16)
    x = torch.from_numpy(seed(16 * 16, 42).reshape(16, 16)).to(dev)
    weight, evict = S.in_window(ew, wd, (16, 16))
    assert np.array_equal(n(x @ weight), n(x @ torch.from_numpy(wd).to(dev)))
    evict()
    with pytest.raises(RuntimeError, match="evicted"):
        x @ weight
    w8, evict8 = S.in_window_int8(ew, wd, (16, 16))
    F.linear(x, w8)
    evict8()
    with pytest.raises(RuntimeError, match="evicted"):
        F.linear(x, w8)
    w4, _ = S.in_window(ew, np.array([1, 2, 3, 4], np.float32), (2, 2))
    with pytest.raises(RuntimeError, match="weight operand only"):
        w4 + torch.ones(2, 2, device=dev)
    with pytest.raises(RuntimeError, match="weight operand only"):
        torch.ones(2, 2, device=dev).add(w4)
    ew.free()
    with pytest.raises(RuntimeError, match="freed"):
        torch.ones(3, 2, device=dev) @ w4


def test_window_streams_24_blocks_through_3(dev):
    """window_probe.html:160-183: 24 blocks placed, used and evicted one at a time through
    room for three; every result equals the resident weight's, and the buffer stays there."""
    say("window: 24 blocks through a 3-block window")
    M, Kd, Nn, B = 8, 16, 16, 24
    need = -(-Kd * Nn * 4 // S.ALIGN) * S.ALIGN
    sw = S.window(3 * need, dev)
    x = torch.from_numpy(seed(M * Kd, 1).reshape(M, Kd)).to(dev)
    for i in range(B):
        wd = seed(Kd * Nn, 100 + i).reshape(Kd, Nn)
        weight, evict = S.in_window(sw, wd, (Kd, Nn))
        assert np.array_equal(n(x @ weight), n(x @ torch.from_numpy(wd).to(dev)))
        evict()
    assert sw.used <= 3 * need
    sw.free()


@pytest.mark.parametrize("mode", ["f32", "f16", "int8"])
@pytest.mark.parametrize("prefetch", [True, False])
def test_stream_sequential_10_blocks_through_3(dev, mode, prefetch):
    """window_probe.html:247-270: ten Linear+ReLU blocks streamed through a window sized for
    three equal the resident network bit for bit, and the window never grows past three."""
    say(f"stream_sequential {mode} prefetch={prefetch}")
    D, NB = 16, 10
    Ws = [seed(D * D, 200 + i).reshape(D, D) for i in range(NB)]
    x0 = torch.from_numpy(seed(4 * D, 199).reshape(4, D)).to(dev)
    if mode == "int8":
        per = -(-D * D // S.ALIGN) * S.ALIGN
        res = [I.pack_linear_weight(torch.from_numpy(w).to(dev), weight_only=True) for w in Ws]
        hr = x0
        for w8 in res:
            hr = torch.relu(I.linear_w8a32(hr, w8))

        def run(h, ws):
            return torch.relu(F.linear(h, ws[0]))
    else:
        per = -(-D * D * (4 if mode == "f32" else 2) // S.ALIGN) * S.ALIGN
        hr = x0
        for w in Ws:
            wt = torch.from_numpy(w).to(dev)
            hr = (hr @ (wt.half().float() if mode == "f16" else wt)).relu()

        def run(h, ws):
            return (h @ ws[0]).relu()
    nw = S.window(3 * per, dev)
    blocks = [S.StreamBlock([w], [(D, D)], run) for w in Ws]
    hs = S.stream_sequential(nw, x0, blocks, int8=mode == "int8", f16=mode == "f16", prefetch=prefetch)
    assert np.array_equal(n(hs), n(hr))
    assert nw.used <= 3 * per
    nw.free()


@pytest.mark.parametrize("M,D,NB,slots", [(1, 4096, 8, 3), (16, 4096, 6, 3), (4, 1024, 12, 2), (64, 2048, 6, 2)])
def test_stream_sequential_int8_at_size(dev, M, D, NB, slots):
    """Full-size blocks (4096 x 4096 is C2's weight) with the copies of block k+1 running
    under block k: the streamed forward equals the resident W8A32 chain bit for bit. With
    room for two blocks every placement reuses the region evicted one block before, so each
    copy is ordered after the kernels that last read that region."""
    say(f"stream_sequential int8 M={M} D={D} blocks={NB} window={slots} blocks")
    rng = np.random.default_rng(M + D + NB)
    Ws = [(rng.normal(size=(D, D)) / np.sqrt(D)).astype(np.float32) for _ in range(NB)]
    bs = [(rng.normal(size=D) * 0.1).astype(np.float32) for _ in range(NB)]
    x0 = torch.from_numpy(rng.normal(size=(M, D)).astype(np.float32)).to(dev)
    packed = [S.pack_int8_host(w) for w in Ws]
    bias = [torch.from_numpy(b).to(dev) for b in bs]
    hr = x0
    for w, b in zip(Ws, bias):
        hr = torch.relu(I.linear_w8a32(hr, I.pack_linear_weight(torch.from_numpy(w).to(dev), weight_only=True), b))

    def make(b):
        return lambda h, ws: torch.relu(F.linear(h, ws[0], b))
    blocks = [S.StreamBlock([p], [(D, D)], make(b)) for p, b in zip(packed, bias)]
    nw = S.window(slots * D * D, dev)
    for prefetch in (True, False):
        hs = S.stream_sequential(nw, x0, blocks, int8=True, prefetch=prefetch)
        assert np.array_equal(n(hs), n(hr)), f"prefetch={prefetch}"
    # f32 host weights quantized at placement give the same bytes, so the same result
    blocks32 = [S.StreamBlock([w], [(D, D)], make(b)) for w, b in zip(Ws, bias)]
    assert np.array_equal(n(S.stream_sequential(nw, x0, blocks32, int8=True)), n(hr))
    assert nw.used <= slots * D * D
    nw.free()
