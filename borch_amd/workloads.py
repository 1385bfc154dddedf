"""Seeded synthetic inputs of the five task configurations (C1–C5).

Generator ``numpy.random.default_rng(seed)``, draws in float64 in the order listed, then
cast to float32, generated on the host. ``N(mu, v)`` reads its second argument as a
*variance* (std = sqrt(v)): ``W ~ N(0, 1/K)`` is the Kaiming-normal scale.
"""
from __future__ import annotations

import numpy as np

# CIFAR-10 per-channel normalisation for C3 (torchvision's commonly used constants).
CIFAR_MEAN = np.array([0.4914, 0.4822, 0.4465], np.float32)
CIFAR_STD = np.array([0.2470, 0.2435, 0.2616], np.float32)

GEMM_K = 4096
GEMM_N = 4096
GEMM_MS = (1, 16, 256, 4096)


def _normal(rng, shape, var):
    return rng.normal(0.0, np.sqrt(var), size=shape).astype(np.float32)


def c1_linear(seed: int = 0):
    """C1: x [16,512] ~ N(0,1); W [512,512] ~ N(0,1/512); b [512] ~ N(0,0.01)."""
    rng = np.random.default_rng(seed)
    x = _normal(rng, (16, 512), 1.0)
    w = _normal(rng, (512, 512), 1.0 / 512)
    b = _normal(rng, (512,), 0.01)
    return x, w, b


def c2_gemm(M: int, seed: int = 0, K: int = GEMM_K, N: int = GEMM_N):
    """C2: A [M,K] ~ N(0,1); W [N,K] ~ N(0,1/K); bias [N] ~ N(0,0.01)."""
    rng = np.random.default_rng(seed)
    a = _normal(rng, (M, K), 1.0)
    w = _normal(rng, (N, K), 1.0 / K)
    b = _normal(rng, (N,), 0.01)
    return a, w, b


def c3_input(batch: int = 16, seed: int = 0):
    """C3: x [B,3,32,32] ~ U(0,1), then per-channel (x − mean)/std."""
    rng = np.random.default_rng(seed)
    x = rng.uniform(0.0, 1.0, size=(batch, 3, 32, 32)).astype(np.float32)
    return ((x - CIFAR_MEAN.reshape(1, 3, 1, 1)) / CIFAR_STD.reshape(1, 3, 1, 1)).astype(np.float32)


def c4_input(batch: int = 64, seed: int = 0, side: int = 224):
    """C4: x [B,3,224,224] ~ U(0,1)."""
    rng = np.random.default_rng(seed)
    return rng.uniform(0.0, 1.0, size=(batch, 3, side, side)).astype(np.float32)


def c5_input(batch: int = 32, tokens: int = 197, dim: int = 768, seed: int = 0):
    """C5: token embeddings [B,197,768] ~ N(0,1) (the patch-embedded input)."""
    rng = np.random.default_rng(seed)
    return _normal(rng, (batch, tokens, dim), 1.0)


def lcg_int8(n: int, seed: int) -> np.ndarray:
    """The int8 operands of the reference's exactness gate ``mmi8``
    (tests/browser/kernel_bench.html:300-301): ``st = st * 1664525 + 1013904223`` (mod 2^32)
    from ``st = seed``, each value ``(st >> 28) - 8``, in [-8, 7]. Vectorised by jumping
    ahead: within a block of B steps, ``st_{j} = a^j st_0 + c (a^{j-1} + ... + 1)``."""
    a, c, B = 1664525, 1013904223, 4096
    mask = np.uint64(0xFFFFFFFF)
    aj = np.empty(B, np.uint64)
    cj = np.empty(B, np.uint64)
    x, y = 1, 0
    for j in range(B):  # aj[j] = a^(j+1), cj[j] = c (a^j + ... + 1), mod 2^32
        x = (x * a) & 0xFFFFFFFF
        y = (y * a + c) & 0xFFFFFFFF
        aj[j], cj[j] = x, y
    out = np.empty(n, np.int8)
    st = np.uint64(seed & 0xFFFFFFFF)
    for i in range(0, n, B):
        blk = (aj * st + cj) & mask
        k = min(B, n - i)
        out[i:i + k] = ((blk[:k] >> np.uint64(28)).astype(np.int16) - 8).astype(np.int8)
        st = blk[B - 1]
    return out


def mmi8_operands(M: int, K: int, N: int):
    """``mmi8``'s shape ``M x K x N``: A int8 [M, K] = lcg(seed 7), B int8 [K, N] = lcg(seed 11),
    as that procedure draws them (kernel_bench.html:301), returned in the Linear layout this
    library takes: A [M, K] and W = B^T [N, K] (so A @ W.T is the reference's A @ B)."""
    A = lcg_int8(M * K, 7).reshape(M, K)
    B = lcg_int8(K * N, 11).reshape(K, N)
    return A, np.ascontiguousarray(B.T)


def gemm_bytes(M: int, N: int = GEMM_N, K: int = GEMM_K) -> int:
    """Algorithmic HBM bytes of one W8A8 GEMM launch: A int8 + W int8 + sA + sW + bias +
    f32 out."""
    return M * K + N * K + 4 * M + 4 * N + 4 * N + 4 * M * N


def gemm_ops(M: int, N: int = GEMM_N, K: int = GEMM_K) -> int:
    return 2 * M * N * K
