"""Benchmark of the int8 (W8A8) inference path on one MI355X.

``python bench.py [--gpus 1] [--steps K] [--warmup W]`` prints ONE JSON line.

Headline (``value``): the 4096³ dynamic-quant GEMM of config C2 — a step is one pass of
the hot path over one batch: per-row quantization of A (f32 [4096,4096] → int8) plus the
int8 MFMA GEMM with the fused dequant+bias epilogue (f32 out), inputs resident in HBM.
``value`` = 2·M·N·K / step time, in TOPS (int8 ops).

``roofline`` is the dominant kernel (the GEMM) timed alone with HIP events on the stream
it runs on: achieved = 2·M·N·K ops ÷ average kernel duration vs. the dense int8 peak.
Beside it: the GEMV (M = 1, 16) and M = 256 rows of the same sweep, cache-cold (the
weight rotates over > 256 MB of copies so the 256 MB Infinity Cache cannot hold it), and
the CPU baseline (the oracle's int8 arithmetic on the host cores, a bounded sample).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_INT8_TOPS = 5000.0  # MI355X dense int8 MFMA, 5.0 POP/s
PEAK_HBM_GBS = 8000.0    # MI355X HBM3E, 8 TB/s
METRIC = "int8 GEMM TOPS (% MFMA peak) at 4096³; ResNet-18 int8 b16 fwd ms; GEMV GB/s"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def time_events(fn, reps, stream):
    """Average ms per call of ``fn`` over ``reps`` back-to-back calls, HIP events on ``stream``."""
    import torch
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for i in range(reps):
        fn(i)
    end.record(stream)
    end.synchronize()
    return start.elapsed_time(end) / reps


def capture(fn, calls):
    """A HIP graph of ``calls`` back-to-back ``fn(i)`` launches (no host launch cost on
    replay: the sub-10 us kernels would otherwise be timed at the Python call rate)."""
    import torch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(calls):
            fn(i)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):  # the warm-up stream: its split-K workspace is recorded
        for i in range(calls):
            fn(i)
    return g


def time_graph(g, calls, replays, stream):
    """Average ms per launch over ``replays`` replays of a graph of ``calls`` launches."""
    g.replay()
    stream.synchronize()
    return time_events(lambda i: g.replay(), replays, stream) / calls


def layer_work(kind, a):
    """(GEMM view (M, N, K), int8 ops, algorithmic bytes) of one recorded launch. Convs are
    implicit GEMMs: M = N·OH·OW pixels, N = output channels, K = KH·KW·Cpad; bytes = the
    int8 input and weight read once, the f32 output (and int8 twin, residual) once. Depthwise:
    2·KH·KW ops per output, bytes = int8 input + f32 output + taps."""
    if kind == "gemm_i8":
        M, K = a["qa"].shape
        N = a["qw"].shape[0]
        byts = M * K + N * K + 4 * M + 8 * N + 4 * M * N * (2 if a["residual"] is not None else 1)
        return (M, N, K), 2 * M * N * K, byts
    if kind == "conv2d_nchw_fq":  # the stem on the f32 NCHW image, its quantization fused
        n, c, h, w = a["x"].shape
        wq, s, p = a["wq"], a["stride"], a["pad"]
        m = n * ((h + 2 * p - wq.KH) // s + 1) * ((w + 2 * p - wq.KW) // s + 1)
        k = wq.KH * wq.KW * wq.cpad
        out_b = (4 * m * wq.O * bool(a.get("f32_out", True)) + 4 * m * wq.O * (a.get("residual") is not None)
                 + m * wq.O * (a.get("s_out") is not None))
        return (m, wq.O, k), 2 * m * wq.O * k, 4 * n * c * h * w + wq.O * k + out_b
    n, h, w, c = a["qx"].shape
    wq, s, p = a["wq"], a["stride"], a["pad"]
    oh, ow = (h + 2 * p - wq.KH) // s + 1, (w + 2 * p - wq.KW) // s + 1
    m = n * oh * ow
    if kind == "dwconv_i8_nhwc":
        return (m, c, wq.KH * wq.KW), 2 * m * c * wq.KH * wq.KW, n * h * w * c + 4 * m * c + wq.KH * wq.KW * c
    k = wq.KH * wq.KW * c
    # the f32 output unless the launch writes the twin alone (conv2d_i8_nhwc_dq: always; its
    # two passes over the input count once, as the algorithm's bytes)
    f32_out = kind == "conv2d_i8_nhwc" or (kind == "conv2d_i8_nhwc_q" and a.get("f32_out", True))
    out_b = (4 * m * wq.O * f32_out + 4 * m * wq.O * (a.get("residual") is not None)
             + (m * wq.O if kind.endswith(("_q", "_dq")) else 0))
    return (m, wq.O, k), 2 * m * wq.O * k, n * h * w * c + wq.O * k + out_b


def layer_table(model, x, stream, calls=10, replays=5):
    """Each int8 layer of one forward timed alone: its recorded launch replayed ``calls``
    times in a HIP graph (operands warm in cache, as in the forward, where the producer
    has just written them), HIP events around ``replays`` replays. One row per layer."""
    import torch
    rows = []
    from borch_amd.tune import record_launches
    for name, kind, f, a in record_launches(model, x):
        g = capture(lambda i: f(**a), calls)
        ms = time_graph(g, calls, replays, stream)
        del g
        (M, N, K), ops, byts = layer_work(kind, a)
        rows.append({"layer": name, "kernel": kind, "M": M, "N": N, "K": K, "us": round(ms * 1e3, 2),
                     "ops": ops, "bytes": byts, "TOPS": round(ops / (ms * 1e-3) / 1e12, 1),
                     "mfma_frac": round(ops / (ms * 1e-3) / 1e12 / PEAK_INT8_TOPS, 4),
                     "GBps": round(byts / (ms * 1e-3) / 1e9, 1)})
    torch.cuda.synchronize()
    return rows


def layer_summary(rows):
    """Totals of a layer table: the MFMA layers (convs, GEMMs) and the depthwise ones."""
    out = {}
    mm = [r for r in rows if r["kernel"] != "dwconv_i8_nhwc"]
    dw = [r for r in rows if r["kernel"] == "dwconv_i8_nhwc"]
    if mm:
        ops, us = sum(r["ops"] for r in mm), sum(r["us"] for r in mm)
        out["mfma_layers"] = {"count": len(mm), "ops": ops, "us": round(us, 1),
                              "TOPS": round(ops / (us * 1e-6) / 1e12, 1),
                              "mfma_frac": round(ops / (us * 1e-6) / 1e12 / PEAK_INT8_TOPS, 4)}
    if dw:
        byts, us = sum(r["bytes"] for r in dw), sum(r["us"] for r in dw)
        out["depthwise_layers"] = {"count": len(dw), "bytes": byts, "us": round(us, 1),
                                   "GBps": round(byts / (us * 1e-6) / 1e9, 1),
                                   "hbm_frac": round(byts / (us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4)}
    return out


def probes(dev, stream, qa, qw, wcopies):
    """The day's ceilings on this GPU (bench_probe/libbqprobe.so, bench_probe/bq_probe.h), measured in the same
    run as the kernels they bound:
    * the int8 MFMA rate with no memory traffic, on fragments of the 4096^3 GEMM's own
      quantized operands (the MFMA clock falls with the power the operand bits draw), in the
      GEMM tile's per-wave shape and occupancy (8 waves a CU); best of 3; in the 16x16x64 form
      the 256x256 tile runs (the ceiling) and in the 32x32x32 form beside it;
    * the plain streaming read of the GEMV's cache-cold 16 MiB weight copies: best of four
      load depths per lane; the floor of any kernel that reads those bytes once."""
    import ctypes
    import torch
    lib = ctypes.CDLL(str(ROOT / "bench_probe" / "libbqprobe.so"))
    lib.bqp_mfma_rate.restype = ctypes.c_int
    lib.bqp_mfma_rate.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int,
                                  ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    lib.bqp_stream_read.restype = ctypes.c_int
    lib.bqp_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    lib.bqp_last_error.restype = ctypes.c_char_p

    def ok(rc):
        if rc != 0:
            raise RuntimeError(lib.bqp_last_error().decode())

    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    sink = torch.empty(cus * 512, dtype=torch.int32, device=dev)
    iters = 400
    st = stream.cuda_stream
    rate, took = {}, {}
    for form in (32, 16):
        ok(lib.bqp_mfma_rate(qa.data_ptr(), qa.numel(), qw.data_ptr(), qw.numel(), form, cus, 8, sink.data_ptr(), st))
        took[form] = min(time_events(lambda i: ok(lib.bqp_mfma_rate(qa.data_ptr(), qa.numel(), qw.data_ptr(), qw.numel(),
                                                                    form, cus, iters, sink.data_ptr(), st)), 1, stream)
                         for _ in range(3))
        rate[form] = cus * 8 * iters * 2097152 / (took[form] * 1e-3) / 1e12
    nbytes = wcopies[0].numel()
    rsink = torch.empty(nbytes // 4096 + 1, dtype=torch.int32, device=dev)
    read_us = {}
    for ch in (1, 2, 4, 8):
        g = capture(lambda i: ok(lib.bqp_stream_read(wcopies[i].data_ptr(), nbytes, ch, rsink.data_ptr(),
                                                     torch.cuda.current_stream().cuda_stream)), len(wcopies))
        read_us[ch] = time_graph(g, len(wcopies), 8, stream) * 1e3
        del g
    ch = min(read_us, key=read_us.get)
    return {"mfma_int8_TOPS_no_memory": round(rate[16], 1), "mfma_32x32x32_TOPS_no_memory": round(rate[32], 1),
            "mfma_probe": f"{cus} CUs x 8 waves on the 4096^3 operands' bytes: {iters * 64} v_mfma_i32_16x16x64_i8 "
                          f"a wave (the GEMM's form) {took[16]:.3f} ms, {iters * 32} v_mfma_i32_32x32x32_i8 a wave "
                          f"{took[32]:.3f} ms",
            "read_16MiB_cold_us": round(read_us[ch], 3), "read_GBps": round(nbytes / (read_us[ch] * 1e-6) / 1e9, 1),
            "read_probe": f"plain streaming read of {nbytes} B over {len(wcopies)} rotated copies, "
                          f"{ch} x 16 B loads a lane (best of 1/2/4/8)"}


def _fit_line(xs, ys):
    """Least-squares t = t0 + x / bw over (bytes, us) points: (t0 us, bw GB/s)."""
    A = np.vstack([np.ones(len(xs)), np.asarray(xs, np.float64)]).T
    (t0, slope), *_ = np.linalg.lstsq(A, np.asarray(ys, np.float64), rcond=None)
    return float(t0), float(1.0 / slope / 1e3)  # bytes / us -> GB/s: 1e-3


def gemv_sweep(dev, stream):
    """The M = 1 int8 GEMV (bq_gemm_i8, gemv_i8_kernel) and a plain streaming read of the
    same bytes (bqp_stream_read, the best of 1/2/4/8 loads a lane) over weights of 16 to
    256 MiB (K = 4096, N = 4096 ... 65536), each timed over rotated copies that together
    exceed the 256 MB Infinity Cache (cache-cold). A line t = t0 + bytes / BW fitted to each
    separates the fixed cost of a launch (ramp-up, drain) from the steady streaming rate."""
    import ctypes
    import torch
    from borch_amd import int8 as I
    lib = ctypes.CDLL(str(ROOT / "bench_probe" / "libbqprobe.so"))
    lib.bqp_stream_read.restype = ctypes.c_int
    lib.bqp_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    K = 4096
    rows = []
    rng = np.random.default_rng(1)
    x = torch.from_numpy(rng.normal(size=(1, K)).astype(np.float32)).to(dev)
    qa, sa = I.quantize_rows(x)
    for N in (4096, 8192, 16384, 32768, 65536):
        nbytes = N * K
        copies = max(3, -(-(768 << 20) // nbytes))
        base = torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev)
        ws = [base.clone() for _ in range(copies)]
        del base
        sw = torch.rand(N, device=dev) * 1e-3
        b = torch.zeros(N, device=dev)
        g = capture(lambda i: I.gemm_i8(qa, ws[i], sa, sw, b), copies)
        t_g = time_graph(g, copies, 6, stream) * 1e3
        del g
        rsink = torch.empty(nbytes // 4096 + 1, dtype=torch.int32, device=dev)
        t_r = float("inf")
        for ch in (1, 2, 4, 8):
            g = capture(lambda i: lib.bqp_stream_read(ws[i].data_ptr(), nbytes, ch, rsink.data_ptr(),
                                                      torch.cuda.current_stream().cuda_stream), copies)
            t_r = min(t_r, time_graph(g, copies, 6, stream) * 1e3)
            del g
        gbytes = WL_gemm_bytes(1, N, K)
        rows.append({"N": N, "weight_MiB": nbytes >> 20, "gemv_us": round(t_g, 3), "read_us": round(t_r, 3),
                     "gemv_GBps": round(gbytes / (t_g * 1e-6) / 1e9, 1),
                     "read_GBps": round(nbytes / (t_r * 1e-6) / 1e9, 1)})
        log(f"GEMV sweep: {rows[-1]}")
        del ws, rsink
        torch.cuda.empty_cache()
    g0, gbw = _fit_line([WL_gemm_bytes(1, r["N"], K) for r in rows], [r["gemv_us"] for r in rows])
    r0, rbw = _fit_line([r["N"] * K for r in rows], [r["read_us"] for r in rows])
    return {"rows": rows,
            "gemv_fit": {"t0_us": round(g0, 3), "steady_GBps": round(gbw, 1),
                         "steady_hbm_frac": round(gbw / PEAK_HBM_GBS, 4)},
            "read_fit": {"t0_us": round(r0, 3), "steady_GBps": round(rbw, 1),
                         "steady_hbm_frac": round(rbw / PEAK_HBM_GBS, 4)},
            "method": "t = t0 + bytes / BW, least squares over 16-256 MiB weights (K = 4096), cache-cold rotations"}


def decode_rows(dev, stream, copies=24):
    """The two decode kernels at M = 1..8 on C2's 4096 x 4096 weight (cache-cold: 24 rotated
    copies), each forced through the plan API: the v_dot4 wave-reduction GEMV (gemv_i8_kernel)
    and the weight-streaming MFMA kernel (skinny_i8_kernel). The rule's pick is reported."""
    import torch
    from borch_amd import int8 as I
    from borch_amd import tune as T
    rows = {}
    rng = np.random.default_rng(3)
    qw = torch.randint(-127, 128, (4096, 4096), dtype=torch.int8, device=dev)
    qws = [qw.clone() for _ in range(copies)]
    sw = torch.rand(4096, device=dev) * 1e-3
    b = torch.zeros(4096, device=dev)
    for M in range(1, 9):
        qa = torch.from_numpy(rng.integers(-127, 128, size=(M, 4096)).astype(np.int8)).to(dev)
        sa = torch.rand(M, device=dev) * 1e-3
        row = {}
        for cfg, name in ((I.CFG_GEMV, "gemv_us"), (I.CFG_SKINNY, "skinny_us")):
            T.set_plan((M, 4096, 4096), cfg, 1)
            g = capture(lambda i: I.gemm_i8(qa, qws[i], sa, sw, b), copies)
            row[name] = round(time_graph(g, copies, 8, stream) * 1e3, 3)
            del g
        T.set_plan((M, 4096, 4096), 0, 1)
        row["rule"] = "gemv" if T.candidates((M, 4096, 4096))[0][0] == I.CFG_GEMV else "skinny"
        rows[f"M{M}"] = row
        log(f"decode M={M}: {row}")
    del qws
    torch.cuda.empty_cache()
    return rows


def gemm_phases(dev, stream, M=4096, N=4096, K=4096, launches=6):
    """Where one launch of the tiled GEMM spends its time: ``bq_gemm_i8_phases`` stamps each
    workgroup's entry, the end of its main loop and the completion of its last store with the
    steady wall clock (hipDeviceAttributeWallClockRate), and its XCC. Per launch, relative to
    the first workgroup's entry: each XCC's first entry (the staggered start), the main loop
    (prologue + K loop) and the epilogue (the f32 stores) per workgroup, and the span from the
    first entry to the last store. Printed as one JSON line."""
    import ctypes
    import torch
    from borch_amd import _lib as L
    from borch_amd import int8 as I
    from borch_amd import workloads as WL
    hip = ctypes.CDLL("libamdhip64.so.7")
    rate = ctypes.c_int(0)
    hip.hipDeviceGetAttribute(ctypes.byref(rate), 10017, dev.index or 0)  # hipDeviceAttributeWallClockRate, kHz
    khz = rate.value or 100000
    a, w, b = WL.c2_gemm(M, 0, K, N)
    qa, sa = I.quantize_rows(torch.from_numpy(a).to(dev))
    qw, sw = I.quantize_weight_per_channel(torch.from_numpy(w).to(dev))
    B = torch.from_numpy(b).to(dev)
    out = torch.empty((M, N), dtype=torch.float32, device=dev)
    cap = 4 * 4096
    nwg = [0]

    def launch(buf):
        n = L.lib().bq_gemm_i8_phases(qa.data_ptr(), qw.data_ptr(), M, N, K, sa.data_ptr(), sw.data_ptr(),
                                      B.data_ptr(), out.data_ptr(), buf.data_ptr(), cap,
                                      torch.cuda.current_stream().cuda_stream)
        if n < 0:
            L.check(int(n))
        nwg[0] = int(n)
    # eager launches back to back (the first two warm up), then the same from a HIP graph
    st_e = [torch.zeros(cap, dtype=torch.int64, device=dev) for _ in range(launches)]
    for i in range(launches + 2):
        launch(st_e[max(0, i - 2)])
    torch.cuda.synchronize()
    ref = I.gemm_i8(qa, qw, sa, sw, B)
    same = bool(torch.equal(out, ref))
    st_g = [torch.zeros(cap, dtype=torch.int64, device=dev) for _ in range(launches)]
    g = capture(lambda i: launch(st_g[i]), launches)
    g.replay()
    torch.cuda.synchronize()
    del g
    n = nwg[0]
    us = 1e3 / khz

    def summary(t):
        v = t[: 4 * n].view(n, 4).cpu().numpy().astype(np.int64)
        t0 = v[:, 0].min()
        entry, loop, end = (v[:, 0] - t0) * us, (v[:, 1] - v[:, 0]) * us, (v[:, 2] - v[:, 1]) * us
        xcc = (v[:, 3] >> 6) & 15
        per = {}
        for x in sorted(set(xcc.tolist())):
            m = xcc == x
            per[int(x)] = {"first_entry_us": round(float(entry[m].min()), 2), "last_entry_us": round(float(entry[m].max()), 2),
                           "main_loop_us_median": round(float(np.median(loop[m])), 2),
                           "epilogue_us_median": round(float(np.median(end[m])), 2),
                           "last_store_us": round(float((entry[m] + loop[m] + end[m]).max()), 2)}
        return {"span_us": round(float((entry + loop + end).max()), 2), "start_us": int(t0),
                "main_loop_us": [round(float(q), 2) for q in np.percentile(loop, [0, 50, 100])],
                "epilogue_us": [round(float(q), 2) for q in np.percentile(end, [0, 50, 100])],
                "xcc": per}
    eager = [summary(t) for t in st_e]
    graph = [summary(t) for t in st_g]
    gaps = [round((graph[i + 1]["start_us"] - graph[i]["start_us"]) * us, 2) for i in range(len(graph) - 1)]
    for r in eager + graph:
        del r["start_us"]
    g = capture(lambda i: I.gemm_i8(qa, qw, sa, sw, B), 10)
    t_graph = time_graph(g, 10, 5, stream) * 1e3
    print(json.dumps({"phases": f"{M}x{N}x{K}", "workgroups": n, "wall_clock_kHz": khz,
                      "output_equals_bq_gemm_i8": same, "graph_us_per_launch_bq_gemm_i8": round(t_graph, 2),
                      "graph_entry_to_entry_us": gaps, "graph_launches": graph, "eager_launches": eager}), flush=True)


def WL_gemm_bytes(M, N, K):
    from borch_amd import workloads as WL
    return WL.gemm_bytes(M, N, K)


def stream_rows(dev, stream, D=4096, NB=12, slots=3):
    """stream_sequential(int8=True) (borch_amd.streaming; stream.ts:36-68): NB blocks of a
    D x D Linear + ReLU (16 MiB of int8 each at D = 4096, C2's weight), packed once on the
    host into pinned memory, streamed through a window of ``slots`` blocks with block k+1's
    copy on the window's copy stream under block k's kernel; M = 1 and 16 rows. Beside it:
    the same pass with no prefetch (copy, then compute), the plain pinned host-to-device
    copy of one block's bytes (the link's rate on the day), the W8A32 kernel alone on a
    resident block, and the host packing of one block."""
    import torch
    from borch_amd import int8 as I
    from borch_amd import streaming as S
    from borch_amd.nn import functional as F
    rng = np.random.default_rng(9)
    Ws = [(rng.normal(size=(D, D)) / np.sqrt(D)).astype(np.float32) for _ in range(NB)]
    t0 = time.perf_counter()
    packed = [S.pack_int8_host(w) for w in Ws]
    pack_ms = (time.perf_counter() - t0) * 1e3 / NB
    bias = [torch.from_numpy((rng.normal(size=D) * 0.1).astype(np.float32)).to(dev) for _ in range(NB)]

    def make(b):
        return lambda h, ws: torch.relu(F.linear(h, ws[0], b))
    blocks = [S.StreamBlock([p], [(D, D)], make(b)) for p, b in zip(packed, bias)]
    win = S.window(slots * D * D, dev)
    out = {"blocks": NB, "block_MiB": D * D >> 20, "window_blocks": slots, "host_pack_ms_per_block": round(pack_ms, 2)}
    # the link: one block's pinned bytes to the device on a side stream
    dst = torch.empty(D * D, dtype=torch.uint8, device=dev)
    side = torch.cuda.Stream(device=dev)
    src = packed[0].q.reshape(-1).view(torch.uint8)
    with torch.cuda.stream(side):
        dst.copy_(src, non_blocking=True)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(side)
        for _ in range(8):
            dst.copy_(src, non_blocking=True)
        e1.record(side)
    torch.cuda.synchronize()
    copy_ms = e0.elapsed_time(e1) / 8
    out["h2d_copy_GBps"] = round(D * D / (copy_ms * 1e-3) / 1e9, 2)
    for M in (1, 16):
        x0 = torch.from_numpy(rng.normal(size=(M, D)).astype(np.float32)).to(dev)
        w8 = I.Int8Weight(torch.empty((D, D), dtype=torch.int8, device=dev).copy_(packed[0].q), packed[0].s.to(dev),
                          D, D, True)
        g = capture(lambda i: I.linear_w8a32(x0, w8, bias[0]), 10)
        gemv_us = time_graph(g, 10, 6, stream) * 1e3
        del g
        res = {}
        for prefetch in (True, False):
            S.stream_sequential(win, x0, blocks, int8=True, prefetch=prefetch)
            best = float("inf")
            for _ in range(3):
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                S.stream_sequential(win, x0, blocks, int8=True, prefetch=prefetch)
                torch.cuda.synchronize()
                best = min(best, time.perf_counter() - t0)
            res[prefetch] = best * 1e3
        out[f"M{M}"] = {"pass_ms": round(res[True], 3), "pass_ms_no_prefetch": round(res[False], 3),
                        "ms_per_block": round(res[True] / NB, 4),
                        "h2d_GBps": round(NB * D * D / (res[True] * 1e-3) / 1e9, 2),
                        "frac_of_copy_rate": round(NB * D * D / (res[True] * 1e-3) / 1e9 / out["h2d_copy_GBps"], 4),
                        "w8a32_kernel_us_resident": round(gemv_us, 3)}
        log(f"stream_sequential int8 M={M}: {out[f'M{M}']}")
    out["window_used_MiB"] = round(win.used / 2**20, 2)
    out["method"] = ("host wall clock around one stream_sequential call between synchronizations, best of 3; "
                     "h2d_GBps = the blocks' int8 bytes / that time")
    win.free()
    return out


# EfficientNet-B0 b64 depthwise layers (channels, input size, kernel, stride) timed alone
B0_DW = [(96, 112, 3, 2), (144, 56, 3, 1), (144, 56, 5, 2), (240, 28, 5, 1), (672, 14, 5, 1), (1152, 7, 5, 1)]


def hbm_kernels(dev):
    """The bandwidth-bound kernels alone, for counter runs (FETCH_SIZE / WRITE_SIZE and the
    kernel trace): one JSON line of what ran, with the algorithmic bytes of each."""
    import torch
    from borch_amd import int8 as I
    from borch_amd import workloads as WL
    g = torch.Generator().manual_seed(0)
    ran = {}
    a1, w1, b1 = WL.c2_gemm(16, 0)
    qw, sw = I.quantize_weight_per_channel(torch.from_numpy(w1).to(dev))
    qws = [qw.clone() for _ in range(24)]
    B = torch.from_numpy(b1).to(dev)
    for m in (1, 16):
        qa, sa = I.quantize_rows(torch.from_numpy(a1[:m]).to(dev))
        for q in qws:
            I.gemm_i8(qa, q, sa, sw, B)
        ran[f"gemm M={m} (24 rotated weights)"] = WL.gemm_bytes(m)
    a256 = WL.c2_gemm(256, 0)[0]
    qa, sa = I.quantize_rows(torch.from_numpy(a256).to(dev))
    for q in qws:
        I.gemm_i8(qa, q, sa, sw, B)
    ran["gemm M=256 (24 rotated weights)"] = WL.gemm_bytes(256)
    w8v = [I.Int8Weight(q, sw, 4096, 4096, True) for q in qws]
    x1 = torch.from_numpy(a1[:1]).to(dev)
    for w8 in w8v:
        I.linear_w8a32(x1, w8, B)
    ran["w8a32 M=1 (24 rotated weights)"] = 4096 * 4096 + 4 * 4096 * 3 + 4 * 4096
    for w8 in w8v:
        I.linear_rows(x1, I.Int8Weight(w8.q, sw, 4096, 4096), B)
    ran["linear_rows M=1, quantize fused (24 rotated weights)"] = WL.gemm_bytes(1) + 4 * 4096
    A = torch.from_numpy(WL.c2_gemm(4096, 0)[0]).to(dev)
    for _ in range(5):
        I.quantize_rows(A)
    ran["quantize_rows 4096x4096 (5x)"] = 5 * 4096 * 4096 + 4 * 4096
    del A
    for C, H, k, st in B0_DW:
        x = torch.randn(64, C, H, H, generator=g).to(dev).contiguous(memory_format=torch.channels_last)
        w8 = I.pack_dw_weight(torch.randn(C, 1, k, k, generator=g).to(dev))
        qx, sa = I.quantize_nhwc(x, w8.cpad)
        for _ in range(3):
            I.dwconv_i8_nhwc(qx, sa, w8, st, k // 2, None, I.ACT_SILU)
        OH = (H + 2 * (k // 2) - k) // st + 1
        ran[f"dwconv C={C} H={H} k={k} s={st} (3x)"] = 64 * H * H * w8.cpad + 64 * OH * OH * w8.cpad * 4 + k * k * w8.cpad
        del x, qx
    x = torch.randn(64, 144, 56, 56, generator=g).to(dev).contiguous(memory_format=torch.channels_last)
    for _ in range(3):
        I.quantize_nhwc(x, 144)
    ran["quantize_nhwc 64x144x56x56 two-pass (3x)"] = 64 * 144 * 56 * 56 * 9
    del x
    # the small-K kernel (the rule's pick): EfficientNet-B0 b64's blocks.0.project (1x1, 32 -> 16
    # channels at 112^2) and its stem (3x3 / 2, 16 padded channels -> 32 at 224^2), f32 out
    sa1 = torch.tensor([0.02], device=dev)
    for (H, C, O_, k, st, pad) in ((112, 32, 16, 1, 1, 0), (224, 16, 32, 3, 2, 1)):
        qx = torch.randint(-127, 128, (64, H, H, C), generator=g, dtype=torch.int8).to(dev)
        w8 = I.pack_conv_weight(torch.randn(O_, C, k, k, generator=g).to(dev))
        OH = (H + 2 * pad - k) // st + 1
        for _ in range(3):
            I.conv2d_i8_nhwc(qx, sa1, w8, st, pad, None, None, I.ACT_NONE)
        ran[f"conv {k}x{k}/{st} {C}->{O_} at {H}^2 b64 (3x)"] = 64 * H * H * C + 64 * OH * OH * O_ * 4 + O_ * k * k * C
        del qx
    # EfficientNet-B0 b64's blocks.1.expand with a calibrated scale: 1x1, 16 -> 96 channels at
    # 112^2, SiLU, its int8 twin alone (the small-K kernel's LDS-staged rows)
    qx = torch.randint(-127, 128, (64, 112, 112, 16), generator=g, dtype=torch.int8).to(dev)
    w8 = I.pack_conv_weight(torch.randn(96, 16, 1, 1, generator=g).to(dev))
    s_tw = torch.tensor([0.05], device=dev)
    for _ in range(3):
        I.conv2d_i8_nhwc_q(qx, sa1, w8, s_tw, 1, 0, None, None, I.ACT_SILU, f32_out=False)
    ran["conv 1x1/1 16->96 at 112^2 b64, SiLU, int8 twin alone (3x)"] = 64 * 112 * 112 * (16 + 96) + 96 * 16
    del qx
    # the same stem on the f32 NCHW image with its quantization fused (bq_conv2d_i8_nchw_fq,
    # calibrated scale): the image read once as f32, no int8 copy of it written or read
    xf = torch.rand(64, 3, 224, 224, generator=g).to(dev)
    w8 = I.pack_conv_weight(torch.randn(32, 3, 3, 3, generator=g).to(dev))
    for _ in range(3):
        I.conv2d_nchw_fq(xf, w8, 2, 1, s_x=sa1)
    ran["conv 3x3/2 3->32 at 224^2 b64, f32 NCHW input quantized in the conv (3x)"] = (
        64 * 3 * 224 * 224 * 4 + 64 * 112 * 112 * 32 * 4 + 32 * 9 * 16)
    del xf
    src = torch.randn(16 << 20, device=dev)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"hbm_kernels": ran, "copy_launches": 5, "copy_bytes": 64 << 20}))


def _resnet18_params():
    """The folded C3 ResNet-18's f32 parameters by name, for the CPU legs."""
    from borch_amd import nets
    model = nets.build("resnet18", seed=0, device="cpu")

    def cp(conv):
        s, p = conv._geometry()
        return (conv.weight.detach().numpy(), conv.bias.detach().numpy(), s, p)
    params = {"stem": cp(model.stem_f.conv), "fc": (model.fc.weight.detach().numpy(), model.fc.bias.detach().numpy())}
    for i, blk in enumerate(model.body):
        params[f"body.{i}.c1"] = cp(blk.c1.conv)
        params[f"body.{i}.c2"] = cp(blk.c2.conv)
        if blk.down is not None:
            params[f"body.{i}.down"] = cp(blk.down)
    return params


def cpu_baseline(M_sample=512):
    """The reference's CPU paths on the host cores, on a bounded sample of the same workload.

    ``value``: borch_cpu's f32 ``gemm_bias_act`` (4x16 register-blocked, row-sliced over
    threads; restated in C from borch-ts/wasm/src/lib.rs:508-584 in oracle/cpu_ref.c) on
    M_sample rows of the 4096^3 Linear, min of 3 — "kind": "port" (the Rust/wasm original
    cannot be built or run here). Beside it: the numpy core's own f32 arithmetic on the same
    sample (``x @ W.T + b`` through numpy's BLAS, borch/_nn.py:413-415, with the BLAS library
    and its thread count from threadpoolctl) and its im2col + GEMM ResNet-18 b16 forward
    (borch/_ops.py:671-791; oracle/numpy_core.py); the numpy int8 oracle on 256 rows; one
    ResNet-18 CIFAR b16 f32 forward through the C kernels (im2col_rows + gemm_bias_act per
    conv, as the reference CPU runner does)."""
    from oracle import cpu_ref as R
    from oracle import numpy_core as NC
    from oracle import quant as O
    from borch_amd import workloads as WL
    nthreads = R.threads()
    a, w, b = WL.c2_gemm(M_sample, 0)
    wt = np.ascontiguousarray(w.T)
    R.gemm(a[:16], wt, b, 0, nthreads)
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        R.gemm(a, wt, b, 0, nthreads)
        times.append(time.perf_counter() - t0)
    t = min(times)
    out = {"value": round(2 * M_sample * 4096 * 4096 / t / 1e12, 5), "unit": "TOPS", "cores": int(nthreads),
           "kind": "port",
           "sample": f"borch_cpu gemm_bias_act (f32, C restatement of lib.rs:508-584, {nthreads} threads) on "
                     f"{M_sample}x4096x4096 rows of the 4096^3 workload, min of 3: {t * 1e3:.1f} ms",
           "host_cpu_count": os.cpu_count()}
    # the numpy core: x @ W.T + b through numpy's BLAS, on the same rows
    try:
        from threadpoolctl import threadpool_info
        blas = [{"api": i.get("internal_api"), "threads": i.get("num_threads"), "version": i.get("version")}
                for i in threadpool_info() if i.get("user_api") == "blas"]
    except Exception as e:  # pragma: no cover - reported, not fatal
        blas = f"threadpoolctl failed: {e}"
    NC.linear(a[:16], w, b)
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        NC.linear(a, w, b)
        times.append(time.perf_counter() - t0)
    tn = min(times)
    out["numpy_core"] = {"linear_TOPS": round(2 * M_sample * 4096 * 4096 / tn / 1e12, 5),
                         "linear_ms": round(tn * 1e3, 2), "blas": blas,
                         "sample": f"x @ W.T + b (borch/_nn.py:413-415) in f32 numpy on {M_sample}x4096x4096, min of 3"}
    # int8 oracle (numpy: per-row quantize + float64-BLAS exact GEMM + f32 epilogue)
    a2, w2, b2 = WL.c2_gemm(256, 0)
    qw, sw = O.quantize_weight_per_channel(w2)
    t0 = time.perf_counter()
    qa, sa = O.quantize_rows(a2)
    O.dequant(O.gemm_i8_i32(qa, qw), sa, sw, b2)
    out["int8_oracle_TOPS"] = round(2 * 256 * 4096 * 4096 / (time.perf_counter() - t0) / 1e12, 5)
    # ResNet-18 CIFAR b16 f32: through the C kernels, and through the numpy core's im2col conv
    try:
        params = _resnet18_params()
        x = WL.c3_input(16, 0)
        R.resnet18_forward(params, x[:2], nthreads)
        t0 = time.perf_counter()
        R.resnet18_forward(params, x, nthreads)
        out["resnet18_b16_f32_ms"] = round((time.perf_counter() - t0) * 1e3, 2)
        NC.resnet18_forward(params, x[:2])
        t0 = time.perf_counter()
        NC.resnet18_forward(params, x)
        out["numpy_core"]["resnet18_b16_f32_ms"] = round((time.perf_counter() - t0) * 1e3, 2)
    except Exception as e:  # pragma: no cover - reported, not fatal
        out["resnet18_b16_f32_ms"] = f"failed: {e}"
    return out


def bench_models(dev, stream, steps, layers_out=None):
    """Forward ms of the model configurations: int8 (HIP-graph replay of the compiled
    model, and eager) beside the same folded model in f32 (torch-ROCm ops), and each int8
    layer timed alone (``layer_table``; the rows go into ``layers_out`` when given)."""
    import torch
    import borch_amd as bt
    from borch_amd import nets, workloads as WL
    out = {}
    cases = [("resnet18_b16", "resnet18", lambda s: WL.c3_input(16, s)),
             ("efficientnet_b0_b64", "efficientnet_b0", lambda s: WL.c4_input(64, s)),
             ("vit_b16_b32", "vit_b16", lambda s: WL.c5_input(32, 197, 768, s))]
    for key, name, make_seeded in cases:
        model = nets.build(name, seed=0, device=dev)
        x = torch.from_numpy(make_seeded(0)).to(dev)
        with torch.no_grad():
            f32_ms = time_events(lambda i: model(x), 3, stream)
            f32_ms = time_events(lambda i: model(x), steps, stream)
            ref = model(x)
        # ViT's quantization is per row, so its batch may run as two parallel chunks (exact)
        split = 2 if name == "vit_b16" else 1
        c = bt.compiled(model, int8=True, graph=True, fuse=False, split=split)
        with torch.no_grad():
            y = c(x)
            eager_ms = time_events(lambda i: model(x), steps, stream)
            g_ms = time_events(lambda i: c(x), steps, stream)
        gap = float((y - ref).abs().max() / ref.abs().max())
        out[key] = {"int8_graph_ms": round(g_ms, 4), "int8_eager_ms": round(eager_ms, 4),
                    "f32_ms": round(f32_ms, 4), "int8_layers": c.int8_layers,
                    "max_abs_diff_vs_f32_rel": round(gap, 5), "graph_split": split}
        dec = c.tuned[0] if c.tuned else []
        out[key]["tuned"] = {"problems": len(dec), "changed": sum(d["chosen"] != d["prior"] for d in dec),
                             "rule_us": round(sum(d["prior_us"] for d in dec), 1),
                             "tuned_us": round(sum(d["chosen_us"] for d in dec), 1)}
        if layers_out is not None:
            layers_out[key + "_tuning"] = dec
        from borch_amd.tune import tune as _tune
        _tune(model, x)  # the whole batch's problems too (a split graph tuned its chunks')
        rows = layer_table(model, x, stream)
        out[key]["layers_alone"] = layer_summary(rows)
        if name == "resnet18":  # per-layer MFMA fraction: [layer, M, N, K, us, fraction of 5.0 POP/s]
            out[key]["per_layer"] = [[r["layer"], r["M"], r["N"], r["K"], r["us"], r["mfma_frac"]] for r in rows]
        if layers_out is not None:
            layers_out[key] = rows
        if name in ("resnet18", "efficientnet_b0"):
            # calibrated static scales + int8 twins (calibrate_int8): no max pass, and no
            # quantize pass where the producer writes the next layer's int8 input
            calib = [torch.from_numpy(make_seeded(s)).to(dev) for s in (11, 12)]
            bt.calibrate_int8(model, calib)
            # calibrated scales make every chunk exact: EfficientNet's batch runs as two
            # parallel chunks (ResNet-18's small launch-bound layers are slower split)
            split_s = 2 if name == "efficientnet_b0" else 1
            c2 = bt.compiled(model, int8=False, graph=True, fuse=False, split=split_s)
            with torch.no_grad():
                ys = c2(x)
                s_ms = time_events(lambda i: c2(x), steps, stream)
            out[key]["int8_static_graph_ms"] = round(s_ms, 4)
            out[key]["static_graph_split"] = split_s
            out[key]["static_max_abs_diff_vs_f32_rel"] = round(float((ys - ref).abs().max() / ref.abs().max()), 5)
            del c2, ys, calib
        if name == "resnet18":
            # the reference's own conv rule (convInt8Fits): 13 of the 20 convs int8, the rest f32
            bt.clear_int8(model)
            n_ref = bt.quantize_for_int8(model, rule="reference")
            c3 = bt.compiled(model, int8=False, graph=True, fuse=False)
            with torch.no_grad():
                c3(x)
                r_ms = time_events(lambda i: c3(x), steps, stream)
            out[key]["int8_reference_rule_graph_ms"] = round(r_ms, 4)
            out[key]["int8_layers_reference_rule"] = n_ref
            del c3
        log(f"{key}: {out[key]}")
        del model, c, x, y, ref
        torch.cuda.empty_cache()
    return out


# The reference's published matmulInt8 points (docs/INT8.md:176, 222-225; RTX 5080, WebGPU):
# context for the rows below, not a target (different hardware).
MMI8_PUBLISHED = {1024: {"ms": 0.038, "TOPS": 56.6}, 2048: {"ms": 0.273, "TOPS": 62.9}}


def mmi8_rows(dev, stream):
    """The reference's int8 GEMM gate ``mmi8`` (tests/browser/kernel_bench.html:294-337) at its
    published shapes 1024^3 and 2048^3: its LCG operands in [-8, 8), the int32 result checked
    on every entry before anything is timed (against an exact float64 product on the device:
    every partial sum is an integer below 2^53), then the dequantising store timed with a
    per-tensor activation scale, per-channel weight scales and a bias (matmulInt8(scaled))."""
    import torch
    from borch_amd import int8 as I
    from borch_amd import workloads as WL
    rows = {}
    for size in (1024, 2048):
        A, W = WL.mmi8_operands(size, size, size)
        At, Wt = torch.from_numpy(A).to(dev), torch.from_numpy(W).to(dev)
        g = torch.Generator().manual_seed(size)
        s0 = (0.5 + torch.rand(1, generator=g)).to(dev)
        sw = (0.5 + torch.rand(size, generator=g)).to(dev)
        bv = torch.randn(size, generator=g).to(dev)
        out, acc = I.gemm_i8(At, Wt, s0, sw, bv, want_acc=True)
        exact = (At.double() @ Wt.double().t()).to(torch.int32)
        wrong = int((acc != exact).sum())
        gk = capture(lambda i: I.gemm_i8(At, Wt, s0, sw, bv), 10)
        t = time_graph(gk, 10, 8, stream)
        del gk
        ops = 2 * size ** 3
        rows[f"{size}^3"] = {"kernel_us": round(t * 1e3, 3), "TOPS": round(ops / (t * 1e-3) / 1e12, 1),
                             "mfma_frac": round(ops / (t * 1e-3) / 1e12 / PEAK_INT8_TOPS, 4),
                             "i32_wrong_entries": wrong, "entries": size * size,
                             "reference_published_rtx5080": MMI8_PUBLISHED[size]}
        log(f"mmi8 {size}^3: {rows[f'{size}^3']}")
        del At, Wt, out, acc, exact
    return rows


def w8a32_rows(dev, stream):
    """Weight-only W8A32 Linear (bq_linear_w8a32: the int8 weight read inside the kernel)
    beside the unpack-then-f32-GEMM path it replaces (bq_dequant_i8 writes the f32 weight,
    torch-ROCm's f32 GEMM reads it): M = 16 and 256 on the 4096 x 4096 weight (24 rotated
    copies, cache-cold), M = 6304 on ViT-B/16 b32's MLP shapes. Also the f32 GEMM alone on a
    weight unpacked beforehand (what a resident f32 weight would cost)."""
    import torch
    from borch_amd import int8 as I
    from borch_amd import workloads as WL
    rows = {}
    for M, N, K, copies in ((16, 4096, 4096, 24), (256, 4096, 4096, 24), (6304, 3072, 768, 4), (6304, 768, 3072, 4)):
        rng = np.random.default_rng(M + N + K)
        X = torch.from_numpy(rng.normal(size=(M, K)).astype(np.float32)).to(dev)
        Wt = torch.from_numpy((rng.normal(size=(N, K)) / np.sqrt(K)).astype(np.float32)).to(dev)
        Bv = torch.from_numpy((0.1 * rng.normal(size=N)).astype(np.float32)).to(dev)
        w8 = I.pack_linear_weight(Wt, weight_only=True)
        del Wt
        ws = [I.Int8Weight(w8.q.clone(), w8.s, K, N, True) for _ in range(copies)]
        g = capture(lambda i: I.linear_w8a32(X, ws[i], Bv), copies)
        t_ours = time_graph(g, copies, 6, stream)
        del g
        g = capture(lambda i: torch.nn.functional.linear(X, I.dequant_weight(ws[i]), Bv), copies)
        t_old = time_graph(g, copies, 6, stream)
        del g
        wf = [I.dequant_weight(w) for w in ws[:4]]
        g = capture(lambda i: torch.nn.functional.linear(X, wf[i % 4], Bv), copies)
        t_f32 = time_graph(g, copies, 6, stream)
        del g, wf, ws
        flops = 2 * M * N * K
        rows[f"M{M}_N{N}_K{K}"] = {"us": round(t_ours * 1e3, 2), "dequant_then_f32_gemm_us": round(t_old * 1e3, 2),
                                   "f32_gemm_on_unpacked_weight_us": round(t_f32 * 1e3, 2),
                                   "TFLOPs": round(flops / (t_ours * 1e-3) / 1e12, 1),
                                   "weight_GBps": round(N * K / (t_ours * 1e-3) / 1e9, 1)}
        log(f"W8A32 M={M} N={N} K={K}: {rows[f'M{M}_N{N}_K{K}']}")
        torch.cuda.empty_cache()
    return rows


VIT_GEMMS = [("qkv", 6304, 2304, 768, False), ("proj", 6304, 768, 768, True), ("fc1", 6304, 3072, 768, False),
             ("fc2", 6304, 768, 3072, True), ("4096^3", 4096, 4096, 4096, False)]


def gemm_shapes(dev):
    """The MFMA GEMMs of the configurations alone, for counter runs and kernel traces: ViT-B/16
    b32's four Linears at the full batch (the kernel the shape rule picks) and the 4096^3 GEMM,
    five launches each, then five 64 MiB device copies (the FETCH / WRITE calibration)."""
    import torch
    from borch_amd import int8 as I
    g = torch.Generator().manual_seed(0)
    ran = {}
    for name, M, N, K, res in VIT_GEMMS:
        qa = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8).to(dev)
        qw = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8).to(dev)
        sa = (torch.rand(M, generator=g) * 1e-3).to(dev)
        sw = (torch.rand(N, generator=g) * 1e-3).to(dev)
        b = torch.randn(N, generator=g).to(dev)
        r = torch.randn(M, N, generator=g).to(dev) if res else None
        for _ in range(5):
            I.gemm_i8(qa, qw, sa, sw, b, residual=r)
        byts = M * K + N * K + 4 * M + 8 * N + 4 * M * N * (2 if res else 1)
        ran[name] = {"M": M, "N": N, "K": K, "ops": 2 * M * N * K, "bytes": byts, "residual": res}
        del qa, qw, r
    src = torch.randn(16 << 20, device=dev)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"gemm_shapes": ran, "copy_launches": 5, "copy_bytes": 64 << 20}))


def model_trace(dev, stream, name, steps):
    """One configuration's int8 forward for a kernel trace: the compiled HIP graph replayed
    ``steps`` times with dynamic scales (and, for the conv nets, ``steps`` times with calibrated
    scales), each replay timed with HIP events. The trace's per-kernel durations against these
    replay times split each forward into time inside kernels and the gaps between them."""
    import torch
    import borch_amd as bt
    from borch_amd import nets, workloads as WL
    make = {"resnet18": lambda s: WL.c3_input(16, s), "efficientnet_b0": lambda s: WL.c4_input(64, s),
            "vit_b16": lambda s: WL.c5_input(32, 197, 768, s)}[name]
    model = nets.build(name, seed=0, device=dev)
    x = torch.from_numpy(make(0)).to(dev)
    out = {"model": name, "steps": steps}
    c = bt.compiled(model, int8=True, graph=True, fuse=False, plan_cache=False)
    with torch.no_grad():
        c(x)
        torch.cuda.synchronize()
        out["dynamic_replay_ms"] = [round(time_events(lambda i: c(x), 1, stream), 4) for _ in range(steps)]
    if name != "vit_b16":
        bt.calibrate_int8(model, [torch.from_numpy(make(s)).to(dev) for s in (11, 12)])
        c2 = bt.compiled(model, int8=False, graph=True, fuse=False, plan_cache=False)
        with torch.no_grad():
            c2(x)
            torch.cuda.synchronize()
            out["static_replay_ms"] = [round(time_events(lambda i: c2(x), 1, stream), 4) for _ in range(steps)]
    print(json.dumps(out), flush=True)


def print_layer_tables(models, tables):
    """Markdown: per model, the forward times and one row per int8 layer timed alone."""
    for key, rows in tables.items():
        if key.endswith("_tuning"):
            continue
        m = models[key]
        print(f"## {key}\n")
        print(f"int8 forward (HIP graph, dynamic scales): {m['int8_graph_ms']} ms; "
              f"static scales: {m.get('int8_static_graph_ms', '-')} ms; f32 (torch-ROCm): {m['f32_ms']} ms; "
              f"layers alone: {json.dumps(m['layers_alone'])}\n")
        print("| layer | kernel | M | N | K | ops | bytes | us alone | TOPS | of 5.0 POP/s | GB/s |")
        print("|---|---|---|---|---|---|---|---|---|---|---|")
        for r in rows:
            print(f"| {r['layer']} | {r['kernel']} | {r['M']} | {r['N']} | {r['K']} | {r['ops']} | {r['bytes']} | "
                  f"{r['us']} | {r['TOPS']} | {r['mfma_frac']} | {r['GBps']} |")
        print()
        dec = tables.get(key + "_tuning", [])
        if dec:
            print(f"Kernel choice by measurement (compiled(tune=True)): {json.dumps(m['tuned'])}\n")
            print("| first layer of the problem | problem | candidates | rule's pick | us | chosen | us |")
            print("|---|---|---|---|---|---|---|")
            for d in dec:
                print(f"| {d['layer']} | {d['key']} | {d['candidates']} | {d['prior']} | {d['prior_us']} | "
                      f"{d['chosen']} | {d['chosen_us']} |")
            print()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--kernels-only", action="store_true",
                    help="for counter runs: 5 launches of the 4096^3 GEMM and 5 of a 64 MiB device copy "
                         "(the copy calibrates FETCH_SIZE / WRITE_SIZE), nothing else")
    ap.add_argument("--hbm-kernels", action="store_true",
                    help="for counter runs: the bandwidth-bound kernels alone (GEMV M=1 and skinny M=16 over 24 "
                         "rotated weights, the 4096x4096 per-row quantize, EfficientNet-B0 b64 depthwise layers, a "
                         "per-tensor quantize) and 5 launches of a 64 MiB device copy; prints their shapes and bytes")
    ap.add_argument("--gemm-shapes", action="store_true",
                    help="for counter runs: 5 launches each of ViT-B/16 b32's four Linear GEMMs (qkv, proj with its "
                         "residual, fc1, fc2 with its residual; per-row scales, bias, f32 out), the 4096^3 GEMM, and a "
                         "64 MiB device copy; prints their shapes and algorithmic bytes and ops")
    ap.add_argument("--model-trace", choices=["resnet18", "efficientnet_b0", "vit_b16"],
                    help="for kernel traces: the model's int8 forward as a HIP graph, replayed --steps times with "
                         "dynamic scales, then (ResNet-18, EfficientNet-B0) --steps times calibrated; prints the "
                         "replay times")
    ap.add_argument("--phases", action="store_true",
                    help="per-workgroup phase stamps of the 4096^3 GEMM (bq_gemm_i8_phases), one JSON line")
    ap.add_argument("--layers", action="store_true",
                    help="the model configurations only, then every int8 layer's table as markdown "
                         "(GEMM shape, ops, bytes, us alone, TOPS, MFMA fraction, GB/s)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(json.dumps({"error": "this build runs on one GPU only: the int8 path is measured on 1 MI355X "
                                   "(the multi-GPU sharding is a design note, not a benchmark)"}))
        sys.exit(2)

    import torch
    from borch_amd import int8 as I
    from borch_amd import workloads as WL

    dev = torch.device("cuda:0")
    from borch_amd._lib import require_device
    require_device(dev)
    stream = torch.cuda.current_stream(dev)
    M = N = K = 4096

    if args.hbm_kernels:
        hbm_kernels(dev)
        return

    if args.gemm_shapes:
        gemm_shapes(dev)
        return

    if args.model_trace:
        model_trace(dev, stream, args.model_trace, args.steps)
        return

    if args.phases:
        gemm_phases(dev, stream)
        return
    if args.layers:
        tables = {}
        models = bench_models(dev, stream, steps=max(args.steps // 2, 10), layers_out=tables)
        print_layer_tables(models, tables)
        return

    if args.kernels_only:
        from borch_amd import workloads as WL2
        a, w, b = WL2.c2_gemm(M, 0)
        qa, sa = I.quantize_rows(torch.from_numpy(a).to(dev))
        qw, sw = I.quantize_weight_per_channel(torch.from_numpy(w).to(dev))
        B = torch.from_numpy(b).to(dev)
        src = torch.randn(16 << 20, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(5):
            I.gemm_i8(qa, qw, sa, sw, B)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"kernels_only": True, "gemm_launches": 5, "copy_launches": 5, "copy_bytes": 64 << 20}))
        return

    # ---- headline: 4096³ dynamic-quant GEMM (quantize + GEMM)
    a, w, b = WL.c2_gemm(M, 0)
    A = torch.from_numpy(a).to(dev)
    W = torch.from_numpy(w).to(dev)
    B = torch.from_numpy(b).to(dev)
    qw, sw = I.quantize_weight_per_channel(W)
    del W
    qa, sa = I.quantize_rows(A)
    out = I.gemm_i8(qa, qw, sa, sw, B)

    def step(_i):
        q, s = I.quantize_rows(A)
        I.gemm_i8(q, qw, s, sw, B)

    # One step = quantize + GEMM. The K timed steps are captured as one HIP graph and replayed
    # once (every kernel of every step runs; a graph launch per step would add its own
    # submission gap to each step). The W warm-up steps run first, as a graph of their own.
    # The same steps replayed as one single-step graph each are reported beside it.
    if args.warmup:
        capture(step, args.warmup).replay()
    g_steps = capture(step, args.steps)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ms_events = time_events(lambda i: g_steps.replay(), 1, stream) / args.steps
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / args.steps
    del g_steps
    g_step = capture(step, 1)
    g_step.replay()
    torch.cuda.synchronize()
    ms_one_graph_per_step = time_events(lambda i: g_step.replay(), args.steps, stream)
    del g_step
    ops = WL.gemm_ops(M)
    value = ops / (ms_events * 1e-3) / 1e12

    # kernels alone (graphs of 10 launches each)
    g_gemm = capture(lambda i: I.gemm_i8(qa, qw, sa, sw, B), 10)
    gemm_ms = time_graph(g_gemm, 10, max(args.steps // 5, 4), stream)
    g_q = capture(lambda i: I.quantize_rows(A), 10)
    quant_ms = time_graph(g_q, 10, max(args.steps // 5, 4), stream)
    del g_gemm, g_q
    gemm_tops = ops / (gemm_ms * 1e-3) / 1e12
    quant_bytes = 5 * M * K + 4 * M
    # The main loop alone, by difference: the same kernel (the rule picks the same tile and
    # no split at either K) at K = 8192, its operands the K = 4096 ones repeated along K (the
    # same values, so the same MFMA power draw), less the K = 4096 time. Launch, the XCDs'
    # staggered start, prologue and epilogue cancel; what remains is 32 more 128-byte stages
    # per tile. Timed interleaved, the minimum of each.
    qa2, qw2 = torch.cat([qa, qa], 1), torch.cat([qw, qw], 1)
    g_2k = capture(lambda i: I.gemm_i8(qa2, qw2, sa, sw, B), 10)
    g_1k = capture(lambda i: I.gemm_i8(qa, qw, sa, sw, B), 10)
    t1k = t2k = float("inf")
    for _ in range(4):
        t1k = min(t1k, time_graph(g_1k, 10, 3, stream))
        t2k = min(t2k, time_graph(g_2k, 10, 3, stream))
    del g_2k, g_1k, qa2, qw2
    main_loop_tops = ops / ((t2k - t1k) * 1e-3) / 1e12
    del A, out

    # ---- sweep rows (cache-cold weight rotation for the HBM-bound ones)
    sweep = {}
    for m in (1, 16, 256):
        a_m, w_m, b_m = WL.c2_gemm(m, 0)
        Am = torch.from_numpy(a_m).to(dev)
        qw_m, sw_m = I.quantize_weight_per_channel(torch.from_numpy(w_m).to(dev))
        Bm = torch.from_numpy(b_m).to(dev)
        copies = 24  # 24 x 16 MiB = 384 MiB > 256 MiB Infinity Cache
        qws = [qw_m.clone() for _ in range(copies)]
        qa_m, sa_m = I.quantize_rows(Am)
        g_k = capture(lambda i: I.gemm_i8(qa_m, qws[i], sa_m, sw_m, Bm), copies)
        t_k = time_graph(g_k, copies, 8, stream)
        g_e = capture(lambda i: (lambda q_s: I.gemm_i8(q_s[0], qws[i], q_s[1], sw_m, Bm))(I.quantize_rows(Am)), copies)
        t_e2e = time_graph(g_e, copies, 8, stream)
        del g_k, g_e
        t_fused = None
        if m <= 4:  # f32 in, f32 out in one launch: the per-row quantize fused into the GEMV (bq_linear_i8)
            w8s_m = [I.Int8Weight(q, sw_m, K, N) for q in qws]
            g_f = capture(lambda i: I.linear_rows(Am, w8s_m[i], Bm), copies)
            t_fused = time_graph(g_f, copies, 8, stream)
            del g_f, w8s_m
        if m == 1:
            ceilings = probes(dev, stream, qa, qw, qws)
            log(f"ceilings: {ceilings}")
        byts = WL.gemm_bytes(m)
        sweep[f"M{m}"] = {"kernel_us": round(t_k * 1e3, 3), "GBps": round(byts / (t_k * 1e-3) / 1e9, 1),
                          "hbm_frac": round(byts / (t_k * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                          "TOPS": round(WL.gemm_ops(m) / (t_k * 1e-3) / 1e12, 2),
                          "e2e_us_with_quantize": round(t_e2e * 1e3, 3), "bytes": byts,
                          **({"fused_quantize_e2e_us": round(t_fused * 1e3, 3),
                              "fused_GBps": round((byts + 4 * m * K) / (t_fused * 1e-3) / 1e9, 1)}
                             if t_fused is not None else {}),
                          "read_floor_us": ceilings["read_16MiB_cold_us"],
                          "frac_of_read_floor": round(ceilings["read_16MiB_cold_us"] / (t_k * 1e3), 4)}
        del qws, Am
        log(f"M={m}: {sweep[f'M{m}']}")
    # weight-only W8A32 decode GEMV (M = 1): f32 x against the int8 weight, cache-cold
    a_1, w_1, b_1 = WL.c2_gemm(1, 0)
    w8s = [I.pack_linear_weight(torch.from_numpy(w_1).to(dev), weight_only=True) for _ in range(1)]
    qws = [w8s[0].q.clone() for _ in range(24)]
    X1 = torch.from_numpy(a_1).to(dev)
    B1 = torch.from_numpy(b_1).to(dev)
    w8v = [I.Int8Weight(q, w8s[0].s, 4096, 4096, True) for q in qws]
    g_w = capture(lambda i: I.linear_w8a32(X1, w8v[i], B1), 24)
    t_w = time_graph(g_w, 24, 8, stream)
    wbytes = 4096 * 4096 + 4 * 4096 * 3 + 4 * 4096
    sweep["W8A32_M1"] = {"kernel_us": round(t_w * 1e3, 3), "GBps": round(wbytes / (t_w * 1e-3) / 1e9, 1),
                         "hbm_frac": round(wbytes / (t_w * 1e-3) / 1e9 / PEAK_HBM_GBS, 4), "bytes": wbytes}
    log(f"W8A32 M=1: {sweep['W8A32_M1']}")
    del g_w, qws, w8v, w8s
    sweep["W8A32"] = w8a32_rows(dev, stream)
    sweep["stream_int8"] = stream_rows(dev, stream)
    sweep["gemv_size_sweep"] = gemv_sweep(dev, stream)
    sweep["decode_kernels"] = decode_rows(dev, stream)
    # C1: the Linear 16x512x512 through nn.Linear (per-row quantize + GEMM), latency
    from borch_amd import nn as bnn
    x_c1, w_c1, b_c1 = WL.c1_linear(0)
    lin = bnn.Linear(512, 512, device=dev)
    with torch.no_grad():
        lin.weight.copy_(torch.from_numpy(w_c1))
        lin.bias.copy_(torch.from_numpy(b_c1))
    lin.quantize_int8()
    X_c1 = torch.from_numpy(x_c1).to(dev)
    g_l = capture(lambda i: lin(X_c1), 10)
    t_l = time_graph(g_l, 10, 8, stream)
    qa_c1, sa_c1 = I.quantize_rows(X_c1)
    g_l2 = capture(lambda i: I.gemm_i8(qa_c1, lin.int8.q, sa_c1, lin.int8.s, lin.bias), 10)
    t_l2 = time_graph(g_l2, 10, 8, stream)
    del g_l, g_l2
    sweep["C1_linear_16x512x512"] = {"e2e_us_with_quantize": round(t_l * 1e3, 3), "kernel_us": round(t_l2 * 1e3, 3),
                                     "ops": 2 * 16 * 512 * 512,
                                     "bytes": 16 * 512 + 512 * 512 + 4 * 16 + 8 * 512 + 4 * 16 * 512}
    log(f"C1: {sweep['C1_linear_16x512x512']}")
    sweep["mmi8"] = mmi8_rows(dev, stream)
    sweep["M4096"] = {"kernel_us": round(gemm_ms * 1e3, 3), "TOPS": round(gemm_tops, 1),
                      "mfma_frac": round(gemm_tops / PEAK_INT8_TOPS, 4),
                      "quantize_us": round(quant_ms * 1e3, 3),
                      "quantize_GBps": round(quant_bytes / (quant_ms * 1e-3) / 1e9, 1)}

    models = bench_models(dev, stream, steps=max(args.steps // 2, 10))

    traffic = None
    tf = ROOT / "profiles" / "gemm_4096_traffic.json"
    if tf.exists():
        try:
            traffic = json.loads(tf.read_text()).get("hbm_bytes_per_launch")
        except Exception:
            traffic = None

    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_events, 5),
        "wall_ms_per_step": round(wall, 5),
        "step_timing": "the K steps captured as one HIP graph, replayed once between HIP events",
        "ms_per_step_one_graph_per_step": round(ms_one_graph_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded numpy default_rng(0): A ~ N(0,1), W ~ N(0,1/4096), b ~ N(0,0.01))",
        "config": {"workload": "C2 dynamic-quant GEMM M=N=K=4096: per-row int8 quantize of A + int8 MFMA GEMM "
                               "+ fused dequant/bias epilogue, f32 out", "M": M, "N": N, "K": K},
        "roofline": {"bound": "mfma", "achieved": round(gemm_tops, 2), "peak": PEAK_INT8_TOPS, "unit": "TOPS",
                     "frac": round(gemm_tops / PEAK_INT8_TOPS, 4), "traffic": traffic,
                     "traffic_source": ("not measured in this run: HBM bytes per launch from the committed "
                                        "rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE runs of this kernel "
                                        "(profiles/gemm_4096_traffic.json)") if traffic is not None else None,
                     "kernel": "gemm_i8_kernel 256x256 (bq_gemm_i8)", "kernel_ms": round(gemm_ms, 5),
                     "timing": "HIP events around HIP-graph replays on the launch stream",
                     "measured_ceiling_TOPS": ceilings["mfma_int8_TOPS_no_memory"],
                     "frac_of_measured_ceiling": round(gemm_tops / ceilings["mfma_int8_TOPS_no_memory"], 4),
                     "main_loop": {"TOPS": round(main_loop_tops, 1),
                                   "frac_of_measured_ceiling": round(main_loop_tops / ceilings["mfma_int8_TOPS_no_memory"], 4),
                                   "us_K4096": round(t1k * 1e3, 3), "us_K8192": round(t2k * 1e3, 3),
                                   "method": "2*4096^3 ops / (t(K=8192) - t(K=4096)), the same kernel and "
                                             "operands repeated along K: the 32 extra 128-byte stages alone"}},
        "ceilings": ceilings,
        "sweep": sweep,
        "models": models,
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
