"""bq_gemm_i8_noalloc — bq_gemm_i8 with its split-K workspace in the library's own static
device memory, for callers that cannot allocate — against bq_gemm_i8 with a caller
workspace, through the C ABI: outputs and int32 accumulators bit for bit, and the
accumulators against the oracle's exact integer GEMM. Two split-K calls in a row (the
second smaller, so it reuses the scratch the first left behind), then a GEMV-sized one
that needs no scratch, then the first shape again. Every K split the library offers for a
split-K shape is forced in turn (bq_plan_set), so the static scratch is what the split
workgroups exchange their partials through; and the calls replayed from a captured HIP
graph give the same bits on every replay."""
import sys

import numpy as np
import pytest
import torch

from borch_amd import _lib as L
from borch_amd import int8 as I
from oracle import quant as O

pytestmark = pytest.mark.gpu


def _fn():
    return L.lib().bq_gemm_i8_noalloc


def _case(dev, M, N, K, act, seed):
    rng = np.random.default_rng(seed)
    a = rng.normal(size=(M, K)).astype(np.float32)
    w = (rng.normal(size=(N, K)) / np.sqrt(K)).astype(np.float32)
    b = (0.1 * rng.normal(size=N)).astype(np.float32)
    r = rng.normal(size=(M, N)).astype(np.float32)
    qa, sa = I.quantize_rows(torch.from_numpy(a).to(dev))
    qw, sw = I.quantize_weight_per_channel(torch.from_numpy(w).to(dev))
    return qa, sa, qw, sw, torch.from_numpy(b).to(dev), torch.from_numpy(r).to(dev)


@pytest.mark.parametrize("M,N,K,act", [(256, 512, 4608, I.ACT_RELU), (128, 256, 4096, I.ACT_NONE),
                                       (3, 300, 1024, I.ACT_NONE), (256, 512, 4608, I.ACT_NONE)])
def test_noalloc_matches_workspace_entry(dev, M, N, K, act):
    print(f"bq_gemm_i8_noalloc M={M} N={N} K={K} act={act}", flush=True)
    sys.stdout.flush()
    qa, sa, qw, sw, b, r = _case(dev, M, N, K, act, seed=M + N + K)
    stream = torch.cuda.current_stream(dev).cuda_stream
    out0 = torch.empty((M, N), dtype=torch.float32, device=dev)
    acc0 = torch.empty((M, N), dtype=torch.int32, device=dev)
    ws = I.split_workspace(dev)
    L.check(L.lib().bq_gemm_i8(qa.data_ptr(), qw.data_ptr(), M, N, K, sa.data_ptr(), sw.data_ptr(), b.data_ptr(),
                               r.data_ptr(), act, out0.data_ptr(), acc0.data_ptr(), ws.data_ptr(), ws.numel(),
                               stream))
    out1 = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
    acc1 = torch.full((M, N), -1, dtype=torch.int32, device=dev)
    L.check(_fn()(qa.data_ptr(), qw.data_ptr(), M, N, K, sa.data_ptr(), sw.data_ptr(), b.data_ptr(), r.data_ptr(),
                  act, out1.data_ptr(), acc1.data_ptr(), stream))
    torch.cuda.synchronize()
    assert torch.equal(acc1, acc0), "int32 accumulators differ from bq_gemm_i8's"
    assert torch.equal(out1, out0), "f32 outputs differ from bq_gemm_i8's"
    assert np.array_equal(acc1.cpu().numpy(), O.gemm_i8_i32(qa.cpu().numpy(), qw.cpu().numpy()))
    # and without an accumulator output, the bias or the residual
    out2 = torch.empty((M, N), dtype=torch.float32, device=dev)
    L.check(_fn()(qa.data_ptr(), qw.data_ptr(), M, N, K, sa.data_ptr(), sw.data_ptr(), None, None, act,
                  out2.data_ptr(), None, stream))
    out3 = torch.empty((M, N), dtype=torch.float32, device=dev)
    L.check(L.lib().bq_gemm_i8(qa.data_ptr(), qw.data_ptr(), M, N, K, sa.data_ptr(), sw.data_ptr(), None, None,
                               act, out3.data_ptr(), None, ws.data_ptr(), ws.numel(), stream))
    torch.cuda.synchronize()
    assert torch.equal(out2, out3)


@pytest.fixture
def no_plans():
    from borch_amd import tune as T
    T.clear_plans()
    yield T
    T.clear_plans()


def _both(dev, qa, qw, sa, sw, b, r, M, N, K, act, stream):
    out0 = torch.empty((M, N), dtype=torch.float32, device=dev)
    acc0 = torch.empty((M, N), dtype=torch.int32, device=dev)
    ws = I.split_workspace(dev)
    L.check(L.lib().bq_gemm_i8(qa.data_ptr(), qw.data_ptr(), M, N, K, sa.data_ptr(), sw.data_ptr(), b.data_ptr(),
                               r.data_ptr(), act, out0.data_ptr(), acc0.data_ptr(), ws.data_ptr(), ws.numel(),
                               stream))
    out1 = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
    acc1 = torch.full((M, N), -1, dtype=torch.int32, device=dev)
    L.check(_fn()(qa.data_ptr(), qw.data_ptr(), M, N, K, sa.data_ptr(), sw.data_ptr(), b.data_ptr(), r.data_ptr(),
                  act, out1.data_ptr(), acc1.data_ptr(), stream))
    return out0, acc0, out1, acc1


@pytest.mark.parametrize("M,N,K", [(256, 512, 4608), (128, 256, 8192)])
def test_noalloc_forced_splits(dev, no_plans, M, N, K):
    """Each (configuration, K split) candidate with a split, forced through the plan API:
    bq_gemm_i8_noalloc then splits K through its static scratch, bit for bit as bq_gemm_i8
    with a caller workspace and the oracle."""
    T = no_plans
    qa, sa, qw, sw, b, r = _case(dev, M, N, K, I.ACT_RELU, seed=M + K)
    stream = torch.cuda.current_stream(dev).cuda_stream
    want = O.gemm_i8_i32(qa.cpu().numpy(), qw.cpu().numpy())
    splits = [(cfg, sp) for cfg, sp in T.candidates((M, N, K)) if sp > 1]
    assert splits, "the shape offers no K split"
    for cfg, sp in splits:
        print(f"bq_gemm_i8_noalloc M={M} N={N} K={K} cfg={cfg} split={sp}", flush=True)
        T.set_plan((M, N, K), cfg, sp)
        out0, acc0, out1, acc1 = _both(dev, qa, qw, sa, sw, b, r, M, N, K, I.ACT_RELU, stream)
        torch.cuda.synchronize()
        assert torch.equal(acc1, acc0) and torch.equal(out1, out0), (cfg, sp)
        assert np.array_equal(acc1.cpu().numpy(), want), (cfg, sp)


def test_noalloc_in_a_captured_graph(dev, no_plans):
    """Warmed up outside the capture (the scratch address looked up), then captured: the
    graph's replays, with eager work between them, equal bq_gemm_i8's output every time."""
    T = no_plans
    M, N, K = 256, 512, 4608
    qa, sa, qw, sw, b, r = _case(dev, M, N, K, I.ACT_NONE, seed=7)
    cands = [(cfg, sp) for cfg, sp in T.candidates((M, N, K)) if sp > 1]
    T.set_plan((M, N, K), *cands[0])
    side = torch.cuda.Stream(device=dev)
    out0, _, _, _ = _both(dev, qa, qw, sa, sw, b, r, M, N, K, I.ACT_NONE, torch.cuda.current_stream(dev).cuda_stream)
    outg = torch.empty((M, N), dtype=torch.float32, device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        L.check(_fn()(qa.data_ptr(), qw.data_ptr(), M, N, K, sa.data_ptr(), sw.data_ptr(), b.data_ptr(),
                      r.data_ptr(), I.ACT_NONE, outg.data_ptr(), None, side.cuda_stream))
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        L.check(_fn()(qa.data_ptr(), qw.data_ptr(), M, N, K, sa.data_ptr(), sw.data_ptr(), b.data_ptr(),
                      r.data_ptr(), I.ACT_NONE, outg.data_ptr(), None, side.cuda_stream))
    for i in range(4):
        print(f"noalloc graph replay {i}", flush=True)
        outg.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(outg, out0), f"replay {i}"
        _both(dev, qa, qw, sa, sw, b, r, 64, N, K, I.ACT_NONE, torch.cuda.current_stream(dev).cuda_stream)
        torch.cuda.synchronize()
    del g


def test_noalloc_refuses_what_bq_gemm_i8_refuses(dev):
    f = _fn()
    assert f(None, None, 4, 4, 20, None, None, None, None, 0, None, None, None) == L.BQ_ERR_UNSUPPORTED
    assert "bq_gemm_i8_noalloc" in L.last_error() and "multiple of 16" in L.last_error()
    assert f(None, None, 4, 4, 16, None, None, None, None, 0, None, None, None) == L.BQ_ERR_ARG
