"""GPU parity of the model configurations C3–C5, layer by layer, through the module surface.

Every int8 layer's input is captured during the real forward; the oracle recomputes that
layer from the captured input and the layer's folded f32 parameters. Per layer: int8
weight packing and int32 accumulators bit-exact (accumulators re-read through the C ABI
with the layer's input), f32 output bit-exact (SiLU and GELU layers: within 1e-5 rel /
1e-6 abs, since the device's expf / erff and numpy's differ in the last bit). ResNet-18's whole conv
stack is additionally chained in the oracle from the network input and matches bit for
bit; logits after the f32 pool + head are held to 1e-5 (rel and abs).
"""
import sys

import numpy as np
import pytest
import torch

import borch_amd as bt
from borch_amd import int8 as I
from borch_amd import nets, workloads as WL
from oracle import models as OM

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-5, 1e-6


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def n(x):
    return x.detach().float().cpu().numpy()


def int8_modules(model):
    return [(name, m) for name, m in model.named_modules()
            if isinstance(m, (bt.nn.Linear, bt.nn.Conv2d)) and m.int8 is not None]


def capture(model, rows=None):
    """Hooks recording (name, module, x, residual, y) for every int8 layer. ``rows(name)``
    may return row indices to keep (Linear inputs flattened to [M, K])."""
    recs, hooks = [], []
    for name, m in int8_modules(model):
        def hook(mod, args, kwargs, out, name=name):
            x = args[0].detach()
            res = args[1].detach() if len(args) > 1 and args[1] is not None else None
            pre = kwargs.get("pre_norm")
            if pre is not None:  # the layer's input is the fused LayerNorm's f32 rows (the kernel's own)
                if I.fusable_layernorm(pre, x, mod.int8):
                    y_ln = I.layernorm_quantize_rows(x.reshape(-1, x.shape[-1]), pre.weight, pre.bias, pre.eps,
                                                     want_y=True)[2]
                    x = y_ln.reshape(x.shape)
                else:
                    x = pre(x)
            pre_act = kwargs.get("pre_act")
            if pre_act:  # the layer's input is act(x) as its input quantizer evaluates it
                x2 = x.reshape(-1, x.shape[-1]).contiguous()
                x = I.quantize_rows(x2, pre_act, want_y=True)[2].reshape(x.shape)
            gate = args[2] if len(args) > 2 else kwargs.get("channel_scale")
            if gate is not None:  # the layer's input is x * gate (the kernel forms the same f32 products)
                x = x * gate.detach()[:, :, None, None]
            if isinstance(mod, bt.nn.Linear):
                x2, y2 = x.reshape(-1, x.shape[-1]), out.detach().reshape(-1, out.shape[-1])
                r2 = None if res is None else res.reshape(-1, res.shape[-1])
                sel = rows(name, x2.shape[0]) if rows else None
                if sel is not None:
                    x2, y2 = x2[sel], y2[sel]
                    r2 = None if r2 is None else r2[sel]
                recs.append((name, mod, n(x2), None if r2 is None else n(r2), n(y2)))
            else:
                recs.append((name, mod, n(x), None if res is None else n(res), n(out)))
        hooks.append(m.register_forward_hook(hook, with_kwargs=True))
    return recs, hooks


def check_layer(name, mod, x, res, y):
    dev = mod.weight.device
    w = n(mod.weight)
    b = None if mod.bias is None else n(mod.bias)
    if isinstance(mod, bt.nn.Linear):
        y_o, acc_o, sa_o, sw_o, qw_o = OM.linear_layer(x, w, b, mod.act, res)
        assert np.array_equal(n(mod.int8.q), qw_o), name
        xt = torch.from_numpy(x).to(dev)
        if mod.int8.kpad != mod.int8.in_features:
            xt = torch.nn.functional.pad(xt, (0, mod.int8.kpad - mod.int8.in_features))
        qa, sa = I.quantize_rows(xt)
        r = None if res is None else torch.from_numpy(res).to(dev)
        _, acc = I.gemm_i8(qa, mod.int8.q, sa, mod.int8.s, mod.bias, mod.act, want_acc=True, residual=r)
    elif isinstance(mod.int8, I.Int8DwWeight):
        stride, pad = mod._geometry()
        y_o, acc_o, sa_o, sw_o, qw_o = OM.dwconv_layer(x, w, b, stride, pad, mod.act)
        assert np.array_equal(n(mod.int8.q), qw_o), name
        qx, sa = I.quantize_nhwc(torch.from_numpy(x).to(dev), mod.int8.cpad)
        _, acc = I.dwconv_i8_nhwc(qx, sa, mod.int8, stride, pad, mod.bias, mod.act, want_acc=True)
        acc = acc[..., : mod.int8.C]
    else:
        stride, pad = mod._geometry()
        y_o, acc_o, sa_o, sw_o, qw_o = OM.conv_layer(x, w, b, stride, pad, mod.act, res)
        assert np.array_equal(n(mod.int8.q), qw_o), name
        qx, sa = I.quantize_nhwc(torch.from_numpy(x).to(dev), mod.int8.cpad)
        r = None if res is None else torch.from_numpy(res).to(dev)
        _, acc = I.conv2d_i8_nhwc(qx, sa, mod.int8, stride, pad, mod.bias, r, mod.act, want_acc=True)
    assert np.array_equal(n(acc).astype(np.int32), acc_o), f"{name}: int32 accumulators differ"
    np.testing.assert_allclose(y, y_o, rtol=RTOL, atol=ATOL, err_msg=name)
    if mod.act not in (I.ACT_SILU, I.ACT_GELU):  # device expf / erff vs numpy: last bits
        assert np.array_equal(y, y_o), f"{name}: f32 output not bit-exact"


def _conv_params(conv):
    s, p = conv._geometry()
    return (n(conv.weight), None if conv.bias is None else n(conv.bias), s, p)


# --------------------------------------------------------------------------- C3

def test_c3_resnet18(dev):
    say("C3 ResNet-18 CIFAR b16")
    model = nets.build("resnet18", seed=0, device=dev)
    x = WL.c3_input(16, 0)
    xt = torch.from_numpy(x).to(dev)
    with torch.no_grad():
        f32_logits = n(model(xt))
    assert bt.quantize_for_int8(model) == 20  # every conv; the fc head stays f32
    recs, hooks = capture(model)
    with torch.no_grad():
        feats = model.features(xt)
        logits = model(xt)
    for h in hooks:
        h.remove()
    assert len(recs) == 40  # 20 layers, two forwards
    for rec in recs[:20]:
        check_layer(*rec)
    # the whole conv stack, chained in the oracle from the network input
    params = {"stem": _conv_params(model.stem_f.conv)}
    for i, blk in enumerate(model.body):
        params[f"body.{i}.c1"] = _conv_params(blk.c1.conv)
        params[f"body.{i}.c2"] = _conv_params(blk.c2.conv)
        if blk.down is not None:
            params[f"body.{i}.down"] = _conv_params(blk.down)
    feats_o = OM.resnet18_features(params, x)
    assert np.array_equal(n(feats), feats_o), "conv stack not bit-exact"
    logits_o = feats_o.mean(axis=(2, 3)) @ n(model.fc.weight).T + n(model.fc.bias)
    np.testing.assert_allclose(n(logits), logits_o, rtol=1e-5, atol=1e-5)
    gap = np.abs(n(logits) - f32_logits).max() / np.abs(f32_logits).max()
    say(f"  int8 vs f32 logits: max |diff| / max |logit| = {gap:.3g}")
    assert gap < 0.05


def test_c3_resnet18_reference_rule(dev):
    say("C3 ResNet-18 b16 under the reference's conv rule (13 of 20 convs int8)")
    model = nets.build("resnet18", seed=0, device=dev)
    xt = torch.from_numpy(WL.c3_input(16, 0)).to(dev)
    with torch.no_grad():
        f32_logits = n(model(xt))
    assert bt.quantize_for_int8(model, rule="reference") == 13
    convs = [m for m in model.modules() if isinstance(m, bt.nn.Conv2d)]
    f32_convs = [m for m in convs if m.int8 is None]
    assert len(f32_convs) == 7 and all(m.reference_rule_refusal() is not None for m in f32_convs)
    recs, hooks = capture(model)
    with torch.no_grad():
        logits = n(model(xt))
    for h in hooks:
        h.remove()
    assert len(recs) == 13
    for rec in recs:
        check_layer(*rec)
    gap = np.abs(logits - f32_logits).max() / np.abs(f32_logits).max()
    say(f"  int8 (reference rule) vs f32 logits: max |diff| / max |logit| = {gap:.3g}")
    assert gap < 0.05


# --------------------------------------------------------------------------- C4

def test_c4_efficientnet_b0_layers(dev):
    say("C4 EfficientNet-B0 per-layer parity (batch 2 at 224)")
    model = nets.build("efficientnet_b0", seed=0, device=dev)
    assert bt.quantize_for_int8(model) == 49  # 1x1 + depthwise + stem + head; SE and fc f32
    x = torch.from_numpy(WL.c4_input(2, 0)).to(dev)
    recs, hooks = capture(model)
    with torch.no_grad():
        model(x)
    for h in hooks:
        h.remove()
    assert len(recs) == 49
    for rec in recs:
        check_layer(*rec)


def test_c4_efficientnet_b0_batch64(dev):
    say("C4 EfficientNet-B0 b64 forward")
    model = nets.build("efficientnet_b0", seed=0, device=dev)
    x = torch.from_numpy(WL.c4_input(64, 0)).to(dev)
    with torch.no_grad():
        ref = n(model(x))
        assert bt.quantize_for_int8(model) == 49
        y = n(model(x))
    assert y.shape == (64, 1000) and np.isfinite(y).all()
    gap = np.abs(y - ref).max() / np.abs(ref).max()
    say(f"  int8 vs f32 logits: max |diff| / max |logit| = {gap:.3g}")
    assert gap < 0.1


# --------------------------------------------------------------------------- C5

def test_c5_vit_b16(dev):
    say("C5 ViT-B/16 encoder b32 (layer 0 full, every other Linear on 256 sampled rows)")
    model = nets.build("vit_b16", seed=0, device=dev)
    x = torch.from_numpy(WL.c5_input(32, 197, 768, 0)).to(dev)
    with torch.no_grad():
        ref = n(model(x))
    assert bt.quantize_for_int8(model) == 48
    sample = np.random.default_rng(0).choice(32 * 197, 256, replace=False)

    def rows(name, m):
        return None if name.startswith("layers.0.") else sample

    recs, hooks = capture(model, rows)
    with torch.no_grad():
        y = n(model(x))
    for h in hooks:
        h.remove()
    assert len(recs) == 48
    for rec in recs:
        check_layer(*rec)
    gap = np.abs(y - ref).max() / np.abs(ref).max()
    say(f"  int8 vs f32 encoder output: max |diff| / max |out| = {gap:.3g}")
    assert np.isfinite(y).all() and gap < 0.1


def test_graph_replay_matches_eager(dev):
    """The compiled (HIP graph) int8 forward equals the eager int8 forward bit for bit, on
    every replay, with eager work and synchronizations between replays (the compiled ResNet
    runs each block's first conv and its shortcut as one launch, the eager one as two)."""
    say("graph replay vs eager (ResNet-18 b4, EfficientNet-B0 b2)")
    for name, x in (("resnet18", WL.c3_input(4, 1)), ("efficientnet_b0", WL.c4_input(2, 1))):
        model = nets.build(name, seed=1, device=dev)
        c = bt.compiled(model, int8=True, graph=True, fuse=False)
        xt = torch.from_numpy(x).to(dev)
        with torch.no_grad():
            eager = n(model(xt))
            for i in range(4):
                got = n(c(xt))
                assert np.array_equal(got, eager), f"{name} replay {i}"
                model(torch.randn_like(xt))  # eager work in between
                torch.cuda.synchronize()
            other = torch.from_numpy(WL.c3_input(4, 2) if name == "resnet18" else WL.c4_input(2, 2)).to(dev)
            assert np.array_equal(n(c(other)), n(model(other))), f"{name} new input"


def test_c3_resnet18_static_calibrated(dev):
    """Static scales + int8 twins (calibrate_int8): the calibrated conv stack equals the
    oracle chain bit for bit; each producer's twin equals the oracle quantization of its
    f32 output; the consumer really takes the twin (no quantize pass runs)."""
    say("C3 ResNet-18 b16, calibrated static scales + int8 twins")
    model = nets.build("resnet18", seed=0, device=dev)
    x = WL.c3_input(16, 0)
    xt = torch.from_numpy(x).to(dev)
    with torch.no_grad():
        f32_logits = n(model(xt))
    assert bt.quantize_for_int8(model) == 20
    calib = [torch.from_numpy(WL.c3_input(16, s)).to(dev) for s in (11, 12)]
    assert bt.calibrate_int8(model, calib) == 20
    twins = {}
    hooks = []
    for name, m in int8_modules(model):
        def hook(mod, args, out, name=name):
            twins[name] = (n(out), None if getattr(out, "_int8_twin", None) is None else n(out._int8_twin[0]),
                           mod.out_scale_v)
        hooks.append(m.register_forward_hook(hook))
    calls = {"n": 0, "stem": 0}
    orig, orig_fq = I.quantize_nhwc_scaled, I.conv2d_nchw_fq

    def counting(*a, **k):
        calls["n"] += 1
        return orig(*a, **k)

    def stem(*a, **k):
        assert k.get("s_x") is not None
        calls["stem"] += 1
        return orig_fq(*a, **k)
    I.quantize_nhwc_scaled, I.conv2d_nchw_fq = counting, stem
    try:
        with torch.no_grad():
            feats = model.features(xt)
    finally:
        I.quantize_nhwc_scaled, I.conv2d_nchw_fq = orig, orig_fq
        for h in hooks:
            h.remove()
    # the stem (3x3 over the 3-channel image) quantizes the network input inside its own
    # conv with the calibrated scale; every other input is its producer's twin
    assert calls["stem"] == 1 and calls["n"] == 0, f"{calls} static quantize passes / fused stems"
    for name, (y, twin, s_out) in twins.items():
        assert twin is not None, name
        assert np.array_equal(twin, O_quant().quantize_with_scale(y.transpose(0, 2, 3, 1), np.float32(s_out))), name
    params, scales = {}, {}

    def put(key, conv):
        params[key] = _conv_params(conv)
        scales[key] = (conv.in_scale_v, conv.out_scale_v)
    put("stem", model.stem_f.conv)
    for i, blk in enumerate(model.body):
        put(f"body.{i}.c1", blk.c1.conv)
        put(f"body.{i}.c2", blk.c2.conv)
        if blk.down is not None:
            put(f"body.{i}.down", blk.down)
    feats_o = OM.resnet18_features_static(params, scales, x)
    assert np.array_equal(n(feats), feats_o), "calibrated conv stack not bit-exact"
    with torch.no_grad():
        logits = n(model(xt))
    gap = np.abs(logits - f32_logits).max() / np.abs(f32_logits).max()
    say(f"  static int8 vs f32 logits: max |diff| / max |logit| = {gap:.3g}")
    assert gap < 0.05
    # compiled: each block's first conv and its shortcut in one launch, the same logits
    pairs = {"n": 0}
    orig_pair = I.conv2d_pair_i8_nhwc

    def counting_pair(*a, **k):
        pairs["n"] += 1
        return orig_pair(*a, **k)
    I.conv2d_pair_i8_nhwc = counting_pair
    try:
        c = bt.compiled(model, int8=False, graph=True, fuse=False, plan_cache=False)
        with torch.no_grad():
            for _ in range(3):
                assert np.array_equal(n(c(xt)), logits), "paired graph != eager"
    finally:
        I.conv2d_pair_i8_nhwc = orig_pair
    assert pairs["n"] >= 3, pairs
    bt.clear_int8(model)
    assert model.stem_f.conv.in_scale is None


def O_quant():
    from oracle import quant
    return quant


def test_tuned_compiled_matches_untuned(dev):
    """compiled(tune=True) chooses each int8 conv's kernel by measurement before its first
    capture; the tuned forward equals the untuned one bit for bit, and every decision kept
    a candidate no slower than the rule's pick."""
    from borch_amd import tune as T
    say("tuned vs untuned compiled (ResNet-18 b4, ViT encoder b2)")
    T.clear_plans()
    try:
        for name, x in (("resnet18", WL.c3_input(4, 3)), ("vit_b16", WL.c5_input(2, 197, 768, 3))):
            model = nets.build(name, seed=3, device=dev)
            xt = torch.from_numpy(x).to(dev)
            c0 = bt.compiled(model, int8=True, graph=True, fuse=False, tune=False)
            ref = n(c0(xt))
            c1 = bt.compiled(model, int8=True, graph=True, fuse=False, tune=True)
            got = n(c1(xt))
            assert np.array_equal(got, ref), name
            assert len(c1.tuned) == 1 and len(c1.tuned[0]) > 0, name
            for rep in c1.tuned[0]:
                assert rep["chosen"] == rep["prior"] or rep["chosen_us"] < rep["prior_us"], rep
            assert np.array_equal(n(c1(xt)), ref), name  # a replay, with the plans in force
    finally:
        T.clear_plans()


def test_c4_efficientnet_b0_static_twin_only(dev):
    """EfficientNet-B0 with calibrated scales: each MBConv's expand conv writes its int8
    twin alone (no f32 output) and the depthwise conv reads it. The forward equals the one
    that writes and passes the f32 expand output (whose depthwise conv took the same twin),
    bit for bit, eagerly and as a HIP-graph replay."""
    say("C4 EfficientNet-B0 b2 at 128^2, calibrated: twin-only expand outputs")
    model = nets.build("efficientnet_b0", seed=5, device=dev)
    bt.compiled(model, int8=True, graph=False, fuse=False, tune=False)
    calib = [torch.from_numpy(WL.c4_input(2, s, side=128)).to(dev) for s in (21, 22)]
    bt.calibrate_int8(model, calib)
    x = torch.from_numpy(WL.c4_input(2, 23, side=128)).to(dev)
    twin_only = {"n": 0}
    real = I.conv2d_i8_nhwc_q

    def counting(*a, **k):
        twin_only["n"] += k.get("f32_out", True) is False
        return real(*a, **k)
    I.conv2d_i8_nhwc_q = counting
    try:
        with torch.no_grad():
            y_twin = n(model(x))
    finally:
        I.conv2d_i8_nhwc_q = real
    assert twin_only["n"] == 15, twin_only  # every MBConv with an expand conv (blocks 1-15)
    nets.MBConv.twin_path = False
    try:
        with torch.no_grad():
            y_f32 = n(model(x))
    finally:
        nets.MBConv.twin_path = True
    assert np.array_equal(y_twin, y_f32)
    c = bt.compiled(model, int8=False, graph=True, fuse=False, tune=False)
    for _ in range(2):
        assert np.array_equal(n(c(x)), y_twin)


def test_c4_static_graph_at_full_resolution(dev):
    """EfficientNet-B0 b16 at 224^2 with calibrated scales, where the stem quantizes the
    image inside its conv, the 112^2 expand conv (200,704 rows) writes its int8 twin alone
    through the small-K kernel's LDS-staged rows and the 56^2 ones (50,176 rows) through the
    tiled kernel: the HIP-graph replays equal the eager forward bit for bit, with eager
    work between replays."""
    say("C4 EfficientNet-B0 b16 at 224^2, calibrated: graph replays vs eager")
    model = nets.build("efficientnet_b0", seed=3, device=dev)
    bt.compiled(model, int8=True, graph=False, fuse=False, tune=False)
    bt.calibrate_int8(model, [torch.from_numpy(WL.c4_input(16, 31)).to(dev)])
    x = torch.from_numpy(WL.c4_input(16, 32)).to(dev)
    with torch.no_grad():
        eager = n(model(x))
        c = bt.compiled(model, int8=False, graph=True, fuse=False, tune=False)
        for i in range(3):
            assert np.array_equal(n(c(x)), eager), f"replay {i}"
            model(torch.randn_like(x))
            torch.cuda.synchronize()
    assert np.isfinite(eager).all()


def test_split_batch_graph_matches_whole(dev):
    """compiled(split=2): the batch runs as two chunks on parallel streams inside the graph
    (each with its own split-K workspace). Where every quantization is per row or uses a
    calibrated scale the result equals the whole-batch graph bit for bit, on every replay;
    a model whose convs take dynamic per-tensor scales (a maximum over the whole batch) is
    refused."""
    say("split batch graphs (ViT encoder b4, calibrated EfficientNet-B0 b4 at 96^2)")
    vit = nets.build("vit_b16", seed=7, device=dev)
    x = torch.from_numpy(WL.c5_input(4, 197, 768, 7)).to(dev)
    whole = n(bt.compiled(vit, int8=True, graph=True, fuse=False, tune=False)(x))
    c = bt.compiled(vit, int8=False, graph=True, fuse=False, tune=False, split=2)
    for _ in range(3):
        assert np.array_equal(n(c(x)), whole)
    b0 = nets.build("efficientnet_b0", seed=7, device=dev)
    bt.compiled(b0, int8=True, graph=False, fuse=False, tune=False)
    xb = torch.from_numpy(WL.c4_input(4, 8, side=96)).to(dev)
    with pytest.raises(ValueError, match="calibrated"):
        bt.compiled(b0, int8=False, graph=True, fuse=False, tune=False, split=2)(xb)
    bt.calibrate_int8(b0, [torch.from_numpy(WL.c4_input(4, s, side=96)).to(dev) for s in (9, 10)])
    whole = n(bt.compiled(b0, int8=False, graph=True, fuse=False, tune=False)(xb))
    c = bt.compiled(b0, int8=False, graph=True, fuse=False, tune=True, split=2)
    for _ in range(3):
        assert np.array_equal(n(c(xb)), whole)


def test_split_workspace_per_stream(dev):
    """Split-K GEMMs and convs issued on two streams at once each use their own split-K
    workspace (tile counters and partials): both give the serial results, bit for bit."""
    say("split-K on two concurrent streams")
    rng = np.random.default_rng(5)
    M, N, K = 256, 512, 4608  # 32 tiles of 64 x 64 over 36 stages: split 8 ways
    ops = []
    for _ in range(2):
        qa = torch.from_numpy(rng.integers(-127, 128, size=(M, K)).astype(np.int8)).to(dev)
        qw = torch.from_numpy(rng.integers(-127, 128, size=(N, K)).astype(np.int8)).to(dev)
        sa = torch.from_numpy(rng.uniform(1e-3, 1e-2, M).astype(np.float32)).to(dev)
        sw = torch.from_numpy(rng.uniform(1e-3, 1e-2, N).astype(np.float32)).to(dev)
        ops.append((qa, qw, sa, sw))
    want = [I.gemm_i8(*o) for o in ops]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(device=dev), torch.cuda.Stream(device=dev)]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream(dev))
    ws = [I.split_workspace(dev, s) for s in streams]
    assert ws[0].data_ptr() != ws[1].data_ptr()
    got = [[], []]
    for _ in range(16):
        for i, s in enumerate(streams):
            with torch.cuda.stream(s):
                got[i].append(I.gemm_i8(*ops[i]))
    torch.cuda.synchronize()
    for i in range(2):
        for g in got[i]:
            assert torch.equal(g, want[i]), f"stream {i}"
    for w in ws:
        assert int(w[:4096].count_nonzero()) == 0


def test_plan_cache_persists_decisions(dev, tmp_path):
    """tune(cache=...) stores every decision (device, library hash, problem); a second tune
    with the table, in this process after the plans are cleared and in a fresh process,
    times nothing and sets the same plans; the forward under the loaded plans equals the
    tuned one bit for bit."""
    import subprocess
    from borch_amd import tune as T
    say("persisted tuning plans (ResNet-18 b4)")
    T.clear_plans()
    path = tmp_path / "plans.json"
    cache = T.PlanCache(path)
    try:
        model = nets.build("resnet18", seed=3, device=dev)
        bt.quantize_for_int8(model)
        x = torch.from_numpy(WL.c3_input(4, 3)).to(dev)
        first = T.tune(model, x, cache=cache)
        assert first and not any(r["cached"] for r in first)
        assert path.exists() and len(cache.load(dev)) == len(first)
        with torch.no_grad():
            y1 = model(x).clone()
        T.clear_plans()
        timed = {"n": 0}
        real = T._time_us

        def counting(*a, **k):
            timed["n"] += 1
            return real(*a, **k)
        T._time_us = counting
        try:
            second = T.tune(model, x, cache=cache)
        finally:
            T._time_us = real
        assert timed["n"] == 0 and all(r["cached"] for r in second)
        assert [(r["key"], r["chosen"]) for r in second] == [(r["key"], r["chosen"]) for r in first]
        with torch.no_grad():
            assert torch.equal(model(x), y1)
        # a fresh process with the same table times nothing either
        code = ("import sys, torch; sys.path.insert(0, '.');"
                "import borch_amd as bt; from borch_amd import nets, workloads as WL, tune as T;"
                "m = nets.build('resnet18', seed=3, device='cuda'); bt.quantize_for_int8(m);"
                "x = torch.from_numpy(WL.c3_input(4, 3)).cuda();"
                f"r = T.tune(m, x, cache=T.PlanCache({str(path)!r}));"
                "print('CACHED', sum(q['cached'] for q in r), len(r))")
        import os
        root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
        out = subprocess.run([sys.executable, "-c", code], cwd=root, capture_output=True, text=True, timeout=240)
        assert out.returncode == 0, out.stderr[-2000:]
        line = [ln for ln in out.stdout.splitlines() if ln.startswith("CACHED")][-1].split()
        assert line[1] == line[2] == str(len(first)), line
    finally:
        T.clear_plans()
