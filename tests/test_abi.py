"""The C ABI library loads (no GPU needed) and exports exactly what include/bq.h declares;
host-side argument checks run without touching a device."""
import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "bq.h"


def declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(bq_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_path():
    names = declared()
    for n in ("bq_quantize_rows", "bq_quantize_weight_per_channel", "bq_quantize_tensor", "bq_quantize_nhwc",
              "bq_gemm_i8", "bq_conv2d_i8_nhwc", "bq_dwconv_i8_nhwc", "bq_device_ok", "bq_last_error"):
        assert n in names


def test_library_exports_every_declared_symbol():
    from borch_amd import _lib
    lib = _lib.lib()
    for name in declared():
        assert hasattr(lib, name), name
    assert sorted(_lib.SIGNATURES) == declared()


def test_version_and_error_without_gpu():
    from borch_amd import _lib
    lib = _lib.lib()
    assert lib.bq_version() >= 1
    import torch
    if not torch.cuda.is_available():
        assert lib.bq_device_ok(0) == 0
        assert "device" in _lib.last_error()


def test_argument_checks_run_on_host():
    """Bad sizes are refused before any launch (no device memory is touched)."""
    from borch_amd import _lib
    lib = _lib.lib()
    assert lib.bq_gemm_i8(None, None, 4, 4, 20, None, None, None, None, 0, None, None, None, 0, None) == _lib.BQ_ERR_UNSUPPORTED
    assert "multiple of 16" in _lib.last_error()
    assert lib.bq_gemm_i8(None, None, -1, 4, 16, None, None, None, None, 0, None, None, None, 0, None) == _lib.BQ_ERR_ARG
    assert lib.bq_gemm_i8(None, None, 4, 4, 16, None, None, None, None, 0, None, None, None, 0, None) == _lib.BQ_ERR_ARG
    assert lib.bq_conv2d_i8_nhwc(None, 1, 4, 4, 8, None, 8, 3, 3, 1, 1, None, None, None, None, 0, None, None,
                                 None, None, 0, None) == _lib.BQ_ERR_UNSUPPORTED
    assert lib.bq_conv2d_i8_nhwc(None, 1, 2, 2, 16, None, 8, 5, 5, 1, 0, None, None, None, None, 0, None, None,
                                 None, None, 0, None) == _lib.BQ_ERR_ARG
    assert "larger than the input" in _lib.last_error()
    assert lib.bq_dwconv_i8_nhwc(None, 1, 4, 4, 6, None, 3, 3, 1, 1, None, None, None, 0, None, None,
                                 None) == _lib.BQ_ERR_UNSUPPORTED
    assert lib.bq_quantize_nhwc(None, 4, 3, 2, None, None, None, 0, None) == _lib.BQ_ERR_ARG
    # the weight-only Linear: K % 16, sizes, and the decode-only entry's M and K limits
    assert lib.bq_linear_w8a32(None, None, 4, 4, 20, None, None, None, 0, None, None) == _lib.BQ_ERR_UNSUPPORTED
    assert lib.bq_linear_w8a32(None, None, -1, 4, 16, None, None, None, 0, None, None) == _lib.BQ_ERR_ARG
    assert lib.bq_linear_w8a32(None, None, 40, 4, 16, None, None, None, 0, None, None) == _lib.BQ_ERR_ARG  # null
    assert lib.bq_gemv_w8a32(None, None, 17, 4, 16, None, None, 0, None, None) == _lib.BQ_ERR_UNSUPPORTED
    assert lib.bq_gemv_w8a32(None, None, 2, 4, 8208, None, None, 0, None, None) == _lib.BQ_ERR_UNSUPPORTED
    # past K = 133152 an int32 sum of int8 products could wrap: refused, not computed
    assert lib.bq_gemm_i8(None, None, 4, 4, 133168, None, None, None, None, 0, None, None, None, 0, None) == _lib.BQ_ERR_UNSUPPORTED
    assert "overflow" in _lib.last_error()
    assert lib.bq_conv2d_i8_nhwc(None, 1, 9, 9, 16656, None, 8, 3, 3, 1, 1, None, None, None, None, 0, None, None,
                                 None, None, 0, None) == _lib.BQ_ERR_UNSUPPORTED
    assert "overflow" in _lib.last_error()
    # the paired convs: descriptors required, per-tile maxima from the first conv only, and
    # each conv's own geometry checks
    d = _lib.ConvDesc(None, 32, 3, 3, 2, 1, None, None, None, 0, None, None, None, None)
    d_amax = _lib.ConvDesc(None, 32, 1, 1, 2, 0, None, None, None, 0, None, None, None, 16)
    assert lib.bq_conv2d_i8_nhwc_pair(None, 1, 8, 8, 16, None, None, d, None, 0, None) == _lib.BQ_ERR_ARG
    assert lib.bq_conv2d_i8_nhwc_pair(None, 1, 8, 8, 16, None, d, d_amax, None, 0, None) == _lib.BQ_ERR_UNSUPPORTED
    assert "first conv" not in _lib.last_error() and "absmax" in _lib.last_error()
    # the phase-stamped GEMM: stamps required, the tiled kernel only
    assert lib.bq_gemm_i8_phases(None, None, 256, 256, 256, None, None, None, None, None, 0, None) == _lib.BQ_ERR_ARG
    assert lib.bq_gemm_i8_phases(None, None, 16, 256, 256, None, None, None, None, 1, 64, None) == _lib.BQ_ERR_ARG
    big = _lib.ConvDesc(None, 32, 9, 9, 1, 0, None, None, None, 0, None, None, None, None)
    assert lib.bq_conv2d_i8_nhwc_pair(None, 1, 8, 8, 16, None, big, d, None, 0, None) == _lib.BQ_ERR_ARG
    assert "larger than the input" in _lib.last_error()
    # the stem on an f32 NCHW image: at most 8 input channels, the small-K kernel's limits, and
    # an empty batch is a no-op (x may then be NULL)
    nparts = ctypes.c_int64(-1)
    assert lib.bq_conv2d_i8_nchw_fq(None, 2, 12, 32, 32, None, None, 32, 3, 3, 2, 1, None, None, None, 0, None,
                                    None, None, None, None, 0, None, None, None, 0, None) == _lib.BQ_ERR_UNSUPPORTED
    assert lib.bq_conv2d_i8_nchw_fq(None, 2, 3, 32, 32, None, None, 32, 3, 3, 2, 1, None, None, None, 0, None,
                                    None, None, None, None, 0, None, None, None, 0, None) == _lib.BQ_ERR_ARG
    assert lib.bq_conv2d_i8_nchw_fq(None, 0, 3, 32, 32, None, None, 32, 3, 3, 2, 1, None, None, None, 0, None,
                                    None, None, None, None, 0, ctypes.byref(nparts), None, None, 0, None) == 0
    assert nparts.value == 0
    # the dynamic twin: its three outputs, O % 16, the small-K kernel's layers only, room for
    # its maxima; an empty batch is a no-op (host checks only: the pointers are never read)
    fake = ctypes.c_void_p(1 << 20)
    def dq(n, h, c, o, k, q=fake, cap=4096):
        return lib.bq_conv2d_i8_nhwc_dq(fake, n, h, h, c, fake, o, k, k, 1, k // 2, fake, fake, None, None, 0,
                                        q, fake, fake, cap, None)
    assert dq(64, 112, 16, 96, 1, q=None) == _lib.BQ_ERR_ARG
    assert dq(64, 112, 16, 24, 1) == _lib.BQ_ERR_UNSUPPORTED
    assert dq(16, 32, 64, 64, 3) == _lib.BQ_ERR_UNSUPPORTED  # K = 576: the tiled kernel's
    assert dq(64, 112, 16, 96, 1, cap=100) == _lib.BQ_ERR_ARG  # 4096 workgroups' maxima
    assert dq(0, 112, 16, 96, 1) == 0
    assert lib.bq_conv2d_i8_nhwc_dq(None, 0, 112, 112, 16, None, 96, 1, 1, 1, 0, None, None, None, None, 0, None,
                                    None, None, 0, None) == 0
    # which convs the dynamic twin takes (the rule's small-K twin: from 65536 rows, up to 160
    # columns, K <= 256; O % 16), decided on the host
    assert lib.bq_conv2d_i8_nhwc_dq_ok(64, 112, 112, 16, 96, 1, 1, 1, 0) == 1
    assert lib.bq_conv2d_i8_nhwc_dq_ok(64, 56, 56, 32, 144, 1, 1, 1, 0) == 1
    assert lib.bq_conv2d_i8_nhwc_dq_ok(2, 112, 112, 16, 96, 1, 1, 1, 0) == 0
    assert lib.bq_conv2d_i8_nhwc_dq_ok(64, 112, 112, 16, 24, 1, 1, 1, 0) == 0
    assert lib.bq_conv2d_i8_nhwc_dq_ok(64, 56, 56, 64, 64, 3, 3, 1, 1) == 0
    assert lib.bq_conv2d_i8_nhwc_dq_ok(0, 112, 112, 16, 96, 1, 1, 1, 0) == _lib.BQ_ERR_ARG
    # a plan that gives the layer a tiled configuration takes it away from the dynamic twin;
    # removing the plan gives it back (plans are host state: no device touched)
    prob = (ctypes.c_int64 * 9)(64, 112, 112, 16, 96, 1, 1, 1, 0)
    assert lib.bq_plan_set(prob, 9, 4, 1) == 0
    try:
        assert lib.bq_conv2d_i8_nhwc_dq_ok(64, 112, 112, 16, 96, 1, 1, 1, 0) == 0
    finally:
        assert lib.bq_plan_set(prob, 9, 0, 0) == 0
    assert lib.bq_conv2d_i8_nhwc_dq_ok(64, 112, 112, 16, 96, 1, 1, 1, 0) == 1
    # the per-tile maxima count is the launch's: a 3x3 conv over 64 channels (K = 576, the
    # tiled kernel's 64x64 tiles) at 112^2 b64 writes 12544 maxima, not the small-K kernel's
    # 4096 that a count blind to K would give (the buffer sized by it would be overrun)
    assert lib.bq_conv2d_absmax_parts(64, 112, 112, 64, 64, 3, 3, 1, 1) == 12544
    assert lib.bq_conv2d_absmax_parts(64, 112, 112, 16, 96, 1, 1, 1, 0) == 4096  # the small-K kernel's
    # f32 attention: head width 64 and at most 256 tokens
    assert lib.bq_attention_f32(None, 1, 10, 2, 32, None, None) == _lib.BQ_ERR_UNSUPPORTED
    assert lib.bq_attention_f32(None, 1, 257, 2, 64, None, None) == _lib.BQ_ERR_UNSUPPORTED
    assert lib.bq_attention_f32(None, 1, 10, 2, 64, None, None) == _lib.BQ_ERR_ARG
    # the f32 head: small heads only
    assert lib.bq_avgpool_linear_f32(None, 2, 16, 1000, None, None, 1000, None, None) == _lib.BQ_ERR_UNSUPPORTED
    assert lib.bq_avgpool_linear_f32(None, 2, 16, 512, None, None, 10, None, None) == _lib.BQ_ERR_ARG
    # zero-size work is a no-op success
    assert lib.bq_gemm_i8(None, None, 0, 4, 16, None, None, None, None, 0, None, None, None, 0, None) == 0


def test_cpu_tensors_are_refused_by_name():
    import torch
    from borch_amd import int8
    from borch_amd._lib import Int8Unavailable
    with pytest.raises(Int8Unavailable, match="gfx950"):
        int8.quantize_rows(torch.zeros(2, 16))


def test_quantize_for_int8_refuses_without_device():
    import torch
    import borch_amd as bt
    from borch_amd._lib import Int8Unavailable
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    m = bt.nn.Sequential(bt.nn.Linear(16, 8), bt.nn.ReLU())
    with pytest.raises(Int8Unavailable, match="int8"):
        bt.quantize_for_int8(m)


PROBE_HEADER = ROOT / "bench_probe" / "bq_probe.h"


def probe_lib():
    lib = ctypes.CDLL(str(ROOT / "bench_probe" / "libbqprobe.so"))
    lib.bqp_last_error.restype = ctypes.c_char_p
    return lib


def test_probe_library_exports_its_header():
    """bench.py's measurement probes (libbqprobe): every declared symbol is exported, and bad
    arguments are refused on the host."""
    text = re.sub(r"/\*.*?\*/", "", PROBE_HEADER.read_text(), flags=re.S)
    names = sorted(set(re.findall(r"\b(bqp_[a-z0-9_]+)\s*\(", text)))
    assert names == ["bqp_last_error", "bqp_mfma_rate", "bqp_stream_read"]
    lib = probe_lib()
    for n in names:
        assert hasattr(lib, n), n
    i64, p = ctypes.c_int64, ctypes.c_void_p
    lib.bqp_mfma_rate.argtypes = [p, i64, p, i64, ctypes.c_int, ctypes.c_int, ctypes.c_int, p, p]
    lib.bqp_stream_read.argtypes = [p, i64, ctypes.c_int, p, p]
    assert lib.bqp_mfma_rate(None, 4096, None, 4096, 16, 1, 1, None, None) == -1
    assert b"null" in lib.bqp_last_error()
    assert lib.bqp_mfma_rate(16, 4000, 16, 4096, 16, 1, 1, 16, None) == -1
    assert lib.bqp_mfma_rate(16, 4096, 16, 4096, 8, 1, 1, 16, None) == -1
    assert b"form" in lib.bqp_last_error()
    assert lib.bqp_stream_read(16, 24, 1, 16, None) == -1
    assert lib.bqp_stream_read(16, 32, 3, 16, None) == -1
    assert b"chunks" in lib.bqp_last_error()


def test_ctypes_signatures_match_the_header():
    """Every entry point's ctypes argument list has as many parameters as its declaration
    in include/bq.h (a stale or mismatched binding shifts every argument after the change)."""
    from borch_amd import _lib
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    decls = dict((m.group(1), m.group(2)) for m in re.finditer(r"\b(bq_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", text))
    assert sorted(decls) == sorted(_lib.SIGNATURES)
    for name, params in decls.items():
        params = params.strip()
        n = 0 if params in ("", "void") else params.count(",") + 1
        assert n == len(_lib.SIGNATURES[name][1]), (name, n, len(_lib.SIGNATURES[name][1]))


def _candidates(lib, problem):
    arr = (ctypes.c_int64 * len(problem))(*problem)
    n = lib.bq_plan_candidates(arr, len(problem), None, None, 0)
    if n <= 0:
        return n
    cfgs, splits = (ctypes.c_int32 * n)(), (ctypes.c_int32 * n)()
    assert lib.bq_plan_candidates(arr, len(problem), cfgs, splits, n) == n
    return list(zip(cfgs, splits))


@pytest.mark.parametrize("problem", [(4096, 4096, 4096), (6304, 768, 3072), (256, 512, 4608), (65, 64, 8192),
                                     (16, 32, 32, 64, 64, 3, 3, 1, 1), (16, 4, 4, 512, 512, 3, 3, 1, 1),
                                     (64, 112, 112, 32, 96, 1, 1, 1, 0), (2, 13, 13, 16, 24, 3, 3, 2, 1)])
def test_plan_candidates(problem):
    """The kernel-choice candidates (host code, no GPU): the rules' pick first, no pair twice,
    configuration ids of the tiled kernel (3 and 9 are never offered, 16 only for a dense
    GEMM) and the small-K kernel (only where N <= 256, N % 4 == 0, K <= 256 and its weight
    fragments fit, unsplit), K
    splits only on tiles of at most 4096 outputs, and never more splits than K stages."""
    from borch_amd import _lib
    lib = _lib.lib()
    cands = _candidates(lib, problem)
    assert isinstance(cands, list) and len(cands) >= 2
    assert len(set(cands)) == len(cands)
    small = {7, 9, 10, 12}  # tiles of 64 x 64 and 128 x 32 outputs
    N, K = (problem[1], problem[2]) if len(problem) == 3 else (problem[4], problem[3] * problem[5] * problem[6])
    smallk_ok = N <= 256 and N % 4 == 0 and K <= 256 and ((N + 15) // 16) * ((K + 63) // 64) <= 16
    assert ((_lib.CFG_SMALLK, 1) in cands) == smallk_ok
    for cfg, split in cands:
        if cfg == _lib.CFG_SMALLK:
            assert split == 1
            continue
        assert 1 <= cfg <= 17 and split >= 1
        assert cfg not in (3, 9) or (cfg, split) == cands[0]
        # 16 only where the dense loader runs: a GEMM or a 1x1 stride-1 unpadded conv
        assert cfg != 16 or len(problem) == 3 or (problem[5:7] == (1, 1) and problem[7:] == (1, 0))
        if split > 1:
            assert cfg in small
    K = problem[2] if len(problem) == 3 else problem[3] * problem[5] * problem[6]
    assert all(split <= (K + 127) // 128 for _, split in cands)


def test_plan_rejects_bad_problems_and_small_gemms():
    from borch_amd import _lib
    lib = _lib.lib()
    assert _candidates(lib, (64, 4096, 4096)) == 0  # the GEMV / skinny kernels: nothing to choose
    assert _candidates(lib, (100, 100, 100)) < 0  # K % 16
    assert _candidates(lib, (1, 2, 3, 4)) < 0  # neither 3 nor 9 dimensions
    assert _candidates(lib, (1, 4, 4, 16, 8, 5, 5, 1, 0)) < 0  # the filter is larger than the input
    arr = (ctypes.c_int64 * 3)(4096, 4096, 4096)
    assert lib.bq_plan_set(arr, 3, 3, 1) < 0 and lib.bq_plan_set(arr, 3, 18, 1) < 0
    assert lib.bq_plan_set(arr, 3, 1, 0) < 0
    conv = (ctypes.c_int64 * 9)(16, 32, 32, 64, 64, 3, 3, 1, 1)
    assert lib.bq_plan_set(conv, 9, 16, 1) < 0  # the 320 x 256 tile is dense only
    small = (ctypes.c_int64 * 3)(16, 512, 512)
    assert lib.bq_plan_set(small, 3, 1, 1) < 0


def test_plan_sets_the_conv_tile_count():
    """A plan changes the tiled kernel's configuration, so the per-tile maxima a conv writes
    (bq_conv2d_absmax_parts) follow it; removing the plan restores the rule."""
    from borch_amd import _lib
    lib = _lib.lib()
    geom = (16, 32, 32, 64, 128, 3, 3, 1, 1)  # M = 16384 pixels, 128 output channels
    arr = (ctypes.c_int64 * 9)(*geom)
    try:
        rule = lib.bq_conv2d_absmax_parts(*geom)
        assert rule > 0
        assert lib.bq_plan_set(arr, 9, 1, 1) == 0  # 256 x 256 tiles
        assert lib.bq_conv2d_absmax_parts(*geom) == (16384 // 256) * 1
        assert lib.bq_plan_set(arr, 9, 12, 1) == 0  # 128 x 32 tiles
        assert lib.bq_conv2d_absmax_parts(*geom) == (16384 // 128) * 4
        assert _candidates(lib, geom)[0][0] == _candidates(lib, geom)[0][0]  # the rule's pick stays first
        assert lib.bq_plan_set(arr, 9, 0, 0) == 0
        assert lib.bq_conv2d_absmax_parts(*geom) == rule
        assert lib.bq_plan_set(arr, 9, 1, 1) == 0
        assert lib.bq_plan_clear() == 0
        assert lib.bq_conv2d_absmax_parts(*geom) == rule
    finally:
        lib.bq_plan_clear()


def test_rule_picks_the_16x16x64_tile_for_large_dense_gemms():
    """The rule's first pick (host code, no GPU): the 256x256 tile on 16x16x64 MFMAs
    (configuration 15) for a large dense GEMM, ragged or not; the same tile size stays on
    32x32x32 (configuration 1) for an implicit-GEMM conv."""
    from borch_amd import _lib
    lib = _lib.lib()
    assert _candidates(lib, (4096, 4096, 4096))[0] == (15, 1)
    assert _candidates(lib, (3900, 3300, 32))[0] == (15, 1)
    assert _candidates(lib, (64, 32, 32, 64, 256, 3, 3, 1, 1))[0] == (1, 1)
    assert _candidates(lib, (64, 32, 32, 64, 256, 1, 1, 1, 0))[0] == (15, 1)  # a 1x1 conv is the dense GEMM
