// Quantizers: per-row (activations, Linear weights) and per-tensor (conv activations).
//
// Per-row: one 256-thread block a row (many rows of up to 1024 floats: one wave a row),
// the row held in registers between the max and the quantize, so x is read from HBM once
// (read 4 B + write 1 B per element: HBM-bound).
// Per-tensor: partial maxima (one per block) into a workspace, then every block of the
// quantize kernel reduces the partials itself — no atomics, no zeroing, deterministic.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "bq_common.h"

namespace bq {

static thread_local char g_err[512];

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(BQ_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return BQ_OK;
}

constexpr int QR_THREADS = 256;

template <int T>
__device__ __forceinline__ float block_max(float v, float* red) {
  v = wave_max(v);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float m = red[0];
#pragma unroll
  for (int i = 1; i < T / 64; ++i) m = fmaxf(m, red[i]);
  return m;
}

// NV float4 per thread kept in registers (K <= NV * 4 * T); NV == 0: any K, two reads.
// ACT: the activation applied to x first (BQ_ACT_*; compile-time in the vector kernels,
// run time in the scalar one, NV == 0). T threads a row.
template <int NV, int ACT, int T = QR_THREADS>
__global__ __launch_bounds__(T) void quantize_rows_kernel(const float* __restrict__ x,
                                                                  int K, int8_t* __restrict__ q,
                                                                  float* __restrict__ s, int act,
                                                                  float* __restrict__ y_out) {
  __shared__ float red[T / 64];
  const size_t row = blockIdx.x;
  const float* xr = x + row * (size_t)K;
  int8_t* qr = q + row * (size_t)K;
  const int t = threadIdx.x;
  if constexpr (NV > 0) {
    float4 v[NV];
    float m = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int k = (t + i * T) * 4;
      if (k < K) {
        v[i] = activate4_inline(*reinterpret_cast<const float4*>(xr + k), ACT);
        if (ACT != BQ_ACT_NONE && y_out) *reinterpret_cast<float4*>(y_out + row * (size_t)K + k) = v[i];
        m = fmaxf(m, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
      } else {
        v[i] = make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
    const float sc = scale_of(block_max<T>(m, red));
    if (t == 0) s[row] = sc;
    const Quantizer qz(sc);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int k = (t + i * T) * 4;
      if (k < K)
        *reinterpret_cast<uint32_t*>(qr + k) = qz.pack(v[i]);
    }
  } else {
    float m = 0.f;
    for (int k = t; k < K; k += T) {
      const float a = activate(xr[k], act);
      if (act != BQ_ACT_NONE && y_out) y_out[row * (size_t)K + k] = a;
      m = fmaxf(m, fabsf(a));
    }
    const float sc = scale_of(block_max<T>(m, red));
    if (t == 0) s[row] = sc;
    const Quantizer qz(sc);
    for (int k = t; k < K; k += T) qr[k] = (int8_t)qz(activate(xr[k], act));
  }
}

// One wave per row, QW_WAVES rows per block, for rows of up to NV * 256 floats (NV <= 4): every lane
// loads its NV float4 (coalesced: lane l reads bytes [16 l, 16 l + 16) of each 1 KB run)
// before any arithmetic, so a wave has NV KB in flight; the max is a wave reduction (no
// LDS, no barrier). The same max, scale and rounding as the block-per-row kernel.
constexpr int QW_WAVES = 4;

template <int NV, int ACT>
__global__ __launch_bounds__(QW_WAVES * 64) void quantize_rows_wave_kernel(const float* __restrict__ x, int M,
                                                                          int K, int8_t* __restrict__ q,
                                                                          float* __restrict__ s,
                                                                          float* __restrict__ y_out) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * QW_WAVES + (threadIdx.x >> 6);
  if (row >= M) return;
  const float* xr = x + (size_t)row * K;
  int8_t* qr = q + (size_t)row * K;
  float4 v[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int k = (lane + i * 64) * 4;
    v[i] = k < K ? *reinterpret_cast<const float4*>(xr + k) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  float m = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    if (ACT != BQ_ACT_NONE && (lane + i * 64) * 4 < K) {
      v[i] = activate4_inline(v[i], ACT);
      if (y_out) *reinterpret_cast<float4*>(y_out + (size_t)row * K + (lane + i * 64) * 4) = v[i];
    }
    m = fmaxf(m, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
  }
  const float sc = scale_of(wave_max(m));  // the whole wave is here: rows are per wave
  if (lane == 0) s[row] = sc;
  const Quantizer qz(sc);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int k = (lane + i * 64) * 4;
    if (k < K) *reinterpret_cast<uint32_t*>(qr + k) = qz.pack(v[i]);
  }
}

// LayerNorm over each row, then the per-row quantization of the result, in one pass: the
// normalised row is never stored (unless y is given). The reference's layerNormRows
// (borch-ts/src/kernels.ts:2935-2986): mean = sum / K, var = sum((x - mean)^2) / K (biased,
// centred in a second pass over the row), rstd = 1 / sqrt(var + eps), y = ((x - mean) *
// rstd) * gamma + beta, one f32 rounding per operation; here the row stays in registers
// (one wave a row, four rows a block) and both sums are fixed-order wave reductions. Then
// max |y|, the scale rule and the quantizer of quantize_rows_kernel.
template <int NV>
__global__ __launch_bounds__(QW_WAVES * 64) void ln_quantize_rows_kernel(const float* __restrict__ x, int M, int K,
                                                                        const float* __restrict__ gamma,
                                                                        const float* __restrict__ beta, float eps,
                                                                        int8_t* __restrict__ q, float* __restrict__ s,
                                                                        float* __restrict__ y_out) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * QW_WAVES + (threadIdx.x >> 6);
  if (row >= M) return;  // whole waves
  const float* xr = x + (size_t)row * K;
  float4 v[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int k = (lane + i * 64) * 4;
    v[i] = k < K ? *reinterpret_cast<const float4*>(xr + k) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i)
    sum = __fadd_rn(__fadd_rn(sum, __fadd_rn(v[i].x, v[i].y)), __fadd_rn(v[i].z, v[i].w));
  const float mean = __fdiv_rn(wave_sum_fixed(sum), (float)K);
  float sq = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    if ((lane + i * 64) * 4 < K) {  // the padding lanes hold zeros, not centred values
      const float a = __fsub_rn(v[i].x, mean), b = __fsub_rn(v[i].y, mean);
      const float c = __fsub_rn(v[i].z, mean), d = __fsub_rn(v[i].w, mean);
      sq = __fadd_rn(sq, __fadd_rn(__fadd_rn(__fmul_rn(a, a), __fmul_rn(b, b)),
                                   __fadd_rn(__fmul_rn(c, c), __fmul_rn(d, d))));
    }
  }
  const float var = __fdiv_rn(wave_sum_fixed(sq), (float)K);
  const float rstd = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(var, eps)));
  float m = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int k = (lane + i * 64) * 4;
    if (k < K) {
      const float4 g = gamma ? *reinterpret_cast<const float4*>(gamma + k) : make_float4(1.f, 1.f, 1.f, 1.f);
      const float4 b = beta ? *reinterpret_cast<const float4*>(beta + k) : make_float4(0.f, 0.f, 0.f, 0.f);
      v[i].x = __fadd_rn(__fmul_rn(__fmul_rn(__fsub_rn(v[i].x, mean), rstd), g.x), b.x);
      v[i].y = __fadd_rn(__fmul_rn(__fmul_rn(__fsub_rn(v[i].y, mean), rstd), g.y), b.y);
      v[i].z = __fadd_rn(__fmul_rn(__fmul_rn(__fsub_rn(v[i].z, mean), rstd), g.z), b.z);
      v[i].w = __fadd_rn(__fmul_rn(__fmul_rn(__fsub_rn(v[i].w, mean), rstd), g.w), b.w);
      m = fmaxf(m, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
      if (y_out) *reinterpret_cast<float4*>(y_out + (size_t)row * K + k) = v[i];
    }
  }
  const float sc = scale_of(wave_max(m));
  if (lane == 0) s[row] = sc;
  const Quantizer qz(sc);
  int8_t* qr = q + (size_t)row * K;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int k = (lane + i * 64) * 4;
    if (k < K) *reinterpret_cast<uint32_t*>(qr + k) = qz.pack(v[i]);
  }
}

constexpr int QT_THREADS = 256;
constexpr int QT_MAX_PARTS = 1024;

// Partial maxima: block b covers elements [b*chunk, (b+1)*chunk).
__global__ __launch_bounds__(QT_THREADS) void absmax_parts_kernel(const float* __restrict__ x, int64_t n,
                                                                  int64_t chunk, float* __restrict__ parts) {
  __shared__ float red[QT_THREADS / 64];
  const int64_t lo = (int64_t)blockIdx.x * chunk;
  const int64_t hi = max(lo, min(lo + chunk, n));
  float m = 0.f;
  if (((uintptr_t)x & 15) == 0 && (lo & 3) == 0) {
    const int64_t hi4 = lo + ((hi - lo) & ~(int64_t)3);
    for (int64_t i = lo + threadIdx.x * 4; i < hi4; i += QT_THREADS * 4) {
      const float4 v = *reinterpret_cast<const float4*>(x + i);
      m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
    for (int64_t i = hi4 + threadIdx.x; i < hi; i += QT_THREADS) m = fmaxf(m, fabsf(x[i]));
  } else {
    for (int64_t i = lo + threadIdx.x; i < hi; i += QT_THREADS) m = fmaxf(m, fabsf(x[i]));
  }
  m = wave_max(m);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    float r = red[0];
    for (int i = 1; i < QT_THREADS / 64; ++i) r = fmaxf(r, red[i]);
    parts[blockIdx.x] = r;
  }
}

// One block: s[0] = the scale of max(parts). Run before a quantize pass when the maxima are
// very many (a conv's per-tile maxima: 12,544 for one EfficientNet-B0 layer at b64), so that
// the pass's blocks read one scale instead of each reducing every maximum again. Its own
// launch costs about 4.6 us, so below 4096 maxima every block reducing them is cheaper
// (EfficientNet-B0 b64 dynamic: 1.92 ms folding from 64 maxima, 1.89 ms from 4096).
__global__ __launch_bounds__(1024) void scale_from_parts_kernel(const float* __restrict__ parts, int nparts,
                                                               float* __restrict__ s) {
  __shared__ float red[1024 / 64];
  float m = 0.f;
  for (int i = threadIdx.x; i < nparts; i += 1024) m = fmaxf(m, parts[i]);
  m = wave_max(m);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    float peak = red[0];
    for (int i = 1; i < 1024 / 64; ++i) peak = fmaxf(peak, red[i]);
    s[0] = scale_of(peak);
  }
}

// Quantize with the scale from the partial maxima. Output element e of [P, Cpad]:
// channel c = e % Cpad reads x[p*C + c] when c < C, else 0. Four output bytes a thread.
__global__ __launch_bounds__(QT_THREADS) void quantize_tensor_kernel(const float* __restrict__ x, int64_t P,
                                                                     int C, int Cpad,
                                                                     const float* __restrict__ parts,
                                                                     int nparts, int8_t* __restrict__ q,
                                                                     float* __restrict__ s,
                                                                     const float* __restrict__ s_given) {
  __shared__ float red[QT_THREADS / 64];
  const int64_t total = P * (int64_t)Cpad;
  const int64_t words = (total + 3) / 4;
  const bool flat = (C == Cpad) && ((uintptr_t)x & 15) == 0 && ((uintptr_t)q & 3) == 0 && (total & 3) == 0;
  const int64_t stride = (int64_t)gridDim.x * QT_THREADS;
  int64_t wi = (int64_t)blockIdx.x * QT_THREADS + threadIdx.x;
  // This thread's first words are loaded before the scale is known: their round trip
  // overlaps the partial maxima's (the scale does not depend on them).
  float4 pv[4];
  const bool pre4 = flat && wi + 3 * stride < words;
  const bool pre1 = flat && !pre4 && wi < words;
  if (pre4) {
#pragma unroll
    for (int u = 0; u < 4; ++u) pv[u] = *reinterpret_cast<const float4*>(x + (wi + u * stride) * 4);
  } else if (pre1) {
    pv[0] = *reinterpret_cast<const float4*>(x + wi * 4);
  }
  float m = 0.f;
  for (int i = threadIdx.x; i < nparts; i += QT_THREADS) m = fmaxf(m, parts[i]);
  m = wave_max(m);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  float peak = red[0];
  for (int i = 1; i < QT_THREADS / 64; ++i) peak = fmaxf(peak, red[i]);
  const float sc = s_given ? s_given[0] : scale_of(peak);
  if (!s_given && blockIdx.x == 0 && threadIdx.x == 0) s[0] = sc;
  const Quantizer qz(sc);
  if (pre4) {
#pragma unroll
    for (int u = 0; u < 4; ++u) *reinterpret_cast<uint32_t*>(q + (wi + u * stride) * 4) = qz.pack(pv[u]);
    wi += 4 * stride;
  } else if (pre1) {
    *reinterpret_cast<uint32_t*>(q + wi * 4) = qz.pack(pv[0]);
    wi += stride;
  }
  if (flat) {
    // four float4 loads a thread in flight before any is quantized (one at a time left
    // the pass latency-bound)
    for (; wi + 3 * stride < words; wi += 4 * stride) {
      float4 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) v[u] = *reinterpret_cast<const float4*>(x + (wi + u * stride) * 4);
#pragma unroll
      for (int u = 0; u < 4; ++u) *reinterpret_cast<uint32_t*>(q + (wi + u * stride) * 4) = qz.pack(v[u]);
    }
  }
  for (; wi < words; wi += stride) {
    const int64_t e0 = wi * 4;
    if (flat) {
      const float4 v = *reinterpret_cast<const float4*>(x + e0);
      *reinterpret_cast<uint32_t*>(q + e0) = qz.pack(v);
    } else {
      for (int j = 0; j < 4; ++j) {
        const int64_t e = e0 + j;
        if (e >= total) break;
        const int64_t p = e / Cpad;
        const int c = (int)(e - p * Cpad);
        q[e] = c < C ? (int8_t)qz(x[p * C + c]) : (int8_t)0;
      }
    }
  }
}

// Padded-channel variant (C < Cpad, Cpad % 16 == 0): one thread per 16-byte chunk of a
// pixel's Cpad output bytes; it reads that chunk's (up to 16) input channels and stores one
// 16-byte word (a channels-last input of C % 4 == 0 takes one thread a pixel instead). The input is channels-last (HW == 0: a pixel's channels contiguous) or
// NCHW (HW = H*W: channel c of pixel n*HW + hw at (n*C + c)*HW + hw, so consecutive threads
// read consecutive pixels of each plane) — an NCHW network input needs no permute first.
__global__ __launch_bounds__(QT_THREADS) void quantize_pad16_kernel(const float* __restrict__ x, int64_t P,
                                                                    int C, int Cpad,
                                                                    const float* __restrict__ parts, int nparts,
                                                                    int8_t* __restrict__ q, float* __restrict__ s,
                                                                    const float* __restrict__ s_given, int HW) {
  __shared__ float red[QT_THREADS / 64];
  float m = 0.f;
  for (int i = threadIdx.x; i < nparts; i += QT_THREADS) m = fmaxf(m, parts[i]);
  m = wave_max(m);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  float peak = red[0];
  for (int i = 1; i < QT_THREADS / 64; ++i) peak = fmaxf(peak, red[i]);
  const float sc = s_given ? s_given[0] : scale_of(peak);
  if (!s_given && blockIdx.x == 0 && threadIdx.x == 0) s[0] = sc;
  const Quantizer qz(sc);
  if (HW == 0 && (C & 3) == 0 && ((uintptr_t)x & 15) == 0) {
    // Channels-last with C % 4 == 0 (a conv output of 24 or 40 channels into 32 or 48): one
    // thread a pixel, its channels as 16-byte loads (consecutive threads on consecutive
    // pixels' contiguous rows), four values a pack, its Cpad bytes as 16-byte stores; no
    // 64-bit division or 4-byte load an element
    for (int64_t p = (int64_t)blockIdx.x * QT_THREADS + threadIdx.x; p < P; p += (int64_t)gridDim.x * QT_THREADS) {
      const float* xp = x + p * C;
      int8_t* qp = q + p * Cpad;
      for (int c0 = 0; c0 < Cpad; c0 += 16) {
        uint32_t wv[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int c = c0 + 4 * j;
          wv[j] = c < C ? qz.pack(*reinterpret_cast<const float4*>(xp + c)) : 0u;
        }
        *reinterpret_cast<uint4*>(qp + c0) = make_uint4(wv[0], wv[1], wv[2], wv[3]);
      }
    }
    return;
  }
  const int chunks = Cpad / 16;
  const int64_t total = P * chunks;
  for (int64_t i = (int64_t)blockIdx.x * QT_THREADS + threadIdx.x; i < total; i += (int64_t)gridDim.x * QT_THREADS) {
    const int64_t p = i / chunks;
    const int c0 = (int)(i - p * chunks) * 16;
    const float* xp;  // channel 0 of pixel p
    int64_t cs;       // elements between channels
    if (HW) {
      const int64_t n = p / HW;
      xp = x + (n * C * HW + (p - n * HW));
      cs = HW;
    } else {
      xp = x + p * C;
      cs = 1;
    }
    uint32_t wv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      int b[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int c = c0 + j * 4 + t;
        b[t] = c < C ? qz(xp[c * cs]) : 0;
      }
      wv[j] = pack4(b[0], b[1], b[2], b[3]);
    }
    *reinterpret_cast<uint4*>(q + i * 16) = make_uint4(wv[0], wv[1], wv[2], wv[3]);
  }
}

// Per-(image, channel) pre-scaled per-tensor quantization (a squeeze-excite product feeding
// a conv): the value quantized is v = fl(x[p, c] * cs[p / HW, c]), one f32 multiply, never
// stored. x [P, C] channels-last with C % 4 == 0; cs [N, C]; P * Cpad < 2^31 (32-bit
// indices). Thread: one 4-channel group of one pixel; the (pixel, group) walk advances by a
// fixed stride, so no per-element division; the image index is a multiply-high division.
struct ChWalk {
  int pix, g;            // current pixel and 4-channel group
  int step_pix, step_g;  // the grid stride in (pixels, groups)
  int groups;
  __device__ ChWalk(int groups_, int start, int stride) : groups(groups_) {
    pix = start / groups;
    g = start - pix * groups;
    step_pix = stride / groups;
    step_g = stride - step_pix * groups;
  }
  __device__ void next() {
    pix += step_pix;
    g += step_g;
    if (g >= groups) {
      g -= groups;
      ++pix;
    }
  }
};

__device__ __forceinline__ float4 chscaled(const float* __restrict__ x, const float* __restrict__ cs, int pix, int g,
                                           int C, uint32_t hw_mul, int hw_shift) {
  const float4 v = *reinterpret_cast<const float4*>(x + (size_t)pix * C + g * 4);
  const int n = fdiv(pix, hw_mul, hw_shift);
  const float4 k = *reinterpret_cast<const float4*>(cs + (size_t)n * C + g * 4);
  return make_float4(__fmul_rn(v.x, k.x), __fmul_rn(v.y, k.y), __fmul_rn(v.z, k.z), __fmul_rn(v.w, k.w));
}

__global__ __launch_bounds__(QT_THREADS) void absmax_chscale_kernel(const float* __restrict__ x,
                                                                    const float* __restrict__ cs, int P, int C,
                                                                    uint32_t hw_mul, int hw_shift,
                                                                    float* __restrict__ parts) {
  __shared__ float red[QT_THREADS / 64];
  const int stride = gridDim.x * QT_THREADS;
  float m = 0.f;
  for (ChWalk w(C / 4, blockIdx.x * QT_THREADS + threadIdx.x, stride); w.pix < P; w.next()) {
    const float4 v = chscaled(x, cs, w.pix, w.g, C, hw_mul, hw_shift);
    m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
  }
  m = wave_max(m);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    float r = red[0];
    for (int i = 1; i < QT_THREADS / 64; ++i) r = fmaxf(r, red[i]);
    parts[blockIdx.x] = r;
  }
}

// q [P, Cpad]: channels C..Cpad-1 zero (Cpad % 4 == 0). Thread: one 4-byte word.
__global__ __launch_bounds__(QT_THREADS) void quantize_chscale_kernel(const float* __restrict__ x,
                                                                      const float* __restrict__ cs, int P, int C,
                                                                      int Cpad, uint32_t hw_mul, int hw_shift,
                                                                      const float* __restrict__ parts, int nparts,
                                                                      int8_t* __restrict__ q, float* __restrict__ s,
                                                                      const float* __restrict__ s_given) {
  __shared__ float red[QT_THREADS / 64];
  float m = 0.f;
  for (int i = threadIdx.x; i < nparts; i += QT_THREADS) m = fmaxf(m, parts[i]);
  m = wave_max(m);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  float peak = red[0];
  for (int i = 1; i < QT_THREADS / 64; ++i) peak = fmaxf(peak, red[i]);
  const float sc = s_given ? s_given[0] : scale_of(peak);
  if (!s_given && blockIdx.x == 0 && threadIdx.x == 0) s[0] = sc;
  const int c4n = C / 4;
  const Quantizer qz(sc);
  for (ChWalk w(Cpad / 4, blockIdx.x * QT_THREADS + threadIdx.x, gridDim.x * QT_THREADS); w.pix < P; w.next()) {
    uint32_t word = 0;
    if (w.g < c4n) {
      const float4 v = chscaled(x, cs, w.pix, w.g, C, hw_mul, hw_shift);
      word = qz.pack(v);
    }
    *reinterpret_cast<uint32_t*>(q + (size_t)w.pix * Cpad + w.g * 4) = word;
  }
}

static int nparts_for(int64_t n) {
  int64_t p = (n + QT_THREADS * 16 - 1) / (QT_THREADS * 16);
  if (p < 1) p = 1;
  if (p > QT_MAX_PARTS) p = QT_MAX_PARTS;
  return (int)p;
}

int absmax_parts_ws(const char* what, const float* x, int64_t n, void* ws, size_t ws_bytes, hipStream_t st, int* np) {
  const int parts = nparts_for(n);
  if (!ws || ws_bytes < (size_t)parts * sizeof(float))
    return set_error(BQ_ERR_ARG, "%s: workspace %zu bytes, need %zu", what, ws_bytes, (size_t)parts * sizeof(float));
  const int64_t chunk = n == 0 ? 1 : (n + parts - 1) / parts;
  absmax_parts_kernel<<<parts, QT_THREADS, 0, st>>>(x, n, ((chunk + 3) / 4) * 4, static_cast<float*>(ws));
  *np = parts;
  return check_launch(what);
}

static int launch_rows(const float* x, int64_t M, int64_t K, int8_t* q, float* s, hipStream_t st,
                       const char* what, int act = BQ_ACT_NONE, float* y = nullptr) {
  if (M < 0 || K < 0) return set_error(BQ_ERR_ARG, "%s: negative size (%lld x %lld)", what, (long long)M, (long long)K);
  if (M == 0) return BQ_OK;
  if (!x || !q || !s) return set_error(BQ_ERR_ARG, "%s: null pointer", what);
  if (M > 0x7fffffff || K > 0x7fffffff) return set_error(BQ_ERR_ARG, "%s: size too large", what);
  if (act < BQ_ACT_NONE || act > BQ_ACT_GELU) return set_error(BQ_ERR_ARG, "%s: bad activation %d", what, act);
  const bool vec = (K % 4 == 0) && (((uintptr_t)x | (uintptr_t)q | (uintptr_t)y) & 15) == 0;
  // the vector kernels are built plain and with GELU (a transformer MLP's second input);
  // ReLU / SiLU inputs take the scalar kernel
  const bool vact = act == BQ_ACT_NONE || act == BQ_ACT_GELU;
  // Short rows in numbers: one wave a row (at 6304 x 768, 8.1 -> 7.0 us). Longer rows keep
  // a block a row: a single wave then does a whole row's quantize arithmetic alone (6304 x
  // 3072: 20.5 -> 22.2 us; one row of 4096: 3.4 -> 6.2 us as one wave).
  const int nw = vec && vact && K > 0 ? (int)((K + 255) / 256) : 0;  // float4 a lane
  if (nw > 0 && nw <= 4 && M >= 1024) {
    dim3 g((unsigned)((M + QW_WAVES - 1) / QW_WAVES)), b(QW_WAVES * 64);
    auto wave = [&](auto k0, auto kg) {
      (act == BQ_ACT_GELU ? kg : k0)<<<g, b, 0, st>>>(x, (int)M, (int)K, q, s, y);
    };
    switch (nw) {
      case 1: wave(quantize_rows_wave_kernel<1, 0>, quantize_rows_wave_kernel<1, BQ_ACT_GELU>); break;
      case 2: wave(quantize_rows_wave_kernel<2, 0>, quantize_rows_wave_kernel<2, BQ_ACT_GELU>); break;
      case 3: wave(quantize_rows_wave_kernel<3, 0>, quantize_rows_wave_kernel<3, BQ_ACT_GELU>); break;
      default: wave(quantize_rows_wave_kernel<4, 0>, quantize_rows_wave_kernel<4, BQ_ACT_GELU>); break;
    }
    return check_launch(what);
  }
  if (vec && vact && K % 2048 == 0 && K <= 8192) {
    // Rows of whole 2048-float multiples: 512 threads a row (no idle lane): 4096 x 4096
    // 17.5 -> 16.8 us, one row of 4096 3.1 -> 2.5 us. Others keep 256 threads (K = 3072
    // over 512 threads would leave a quarter of the lanes idle: 18.8 -> 21.3 us).
    dim3 grid((unsigned)M), block(512);
    auto blk = [&](auto k0, auto kg) {
      (act == BQ_ACT_GELU ? kg : k0)<<<grid, block, 0, st>>>(x, (int)K, q, s, act, y);
    };
    switch (K / 2048) {
      case 1: blk(quantize_rows_kernel<1, 0, 512>, quantize_rows_kernel<1, BQ_ACT_GELU, 512>); break;
      case 2: blk(quantize_rows_kernel<2, 0, 512>, quantize_rows_kernel<2, BQ_ACT_GELU, 512>); break;
      default: blk(quantize_rows_kernel<4, 0, 512>, quantize_rows_kernel<4, BQ_ACT_GELU, 512>); break;
    }
    return check_launch(what);
  }
  const int nv = vec && vact ? (int)((K + 1023) / 1024) : 0;
  dim3 grid((unsigned)M), block(QR_THREADS);
  auto blk = [&](auto k0, auto kg) {
    (act == BQ_ACT_GELU ? kg : k0)<<<grid, block, 0, st>>>(x, (int)K, q, s, act, y);
  };
  switch (nv) {
    case 1: blk(quantize_rows_kernel<1, 0>, quantize_rows_kernel<1, BQ_ACT_GELU>); break;
    case 2: blk(quantize_rows_kernel<2, 0>, quantize_rows_kernel<2, BQ_ACT_GELU>); break;
    case 3: blk(quantize_rows_kernel<3, 0>, quantize_rows_kernel<3, BQ_ACT_GELU>); break;
    case 4: blk(quantize_rows_kernel<4, 0>, quantize_rows_kernel<4, BQ_ACT_GELU>); break;
    case 5:
    case 6: blk(quantize_rows_kernel<6, 0>, quantize_rows_kernel<6, BQ_ACT_GELU>); break;
    case 7:
    case 8: blk(quantize_rows_kernel<8, 0>, quantize_rows_kernel<8, BQ_ACT_GELU>); break;
    default: quantize_rows_kernel<0, 0><<<grid, block, 0, st>>>(x, (int)K, q, s, act, y); break;
  }
  return check_launch(what);
}

}  // namespace bq

using namespace bq;

extern "C" {

int bq_version(void) { return (0 << 16) | 1; }

const char* bq_last_error(void) { return g_err; }

int bq_device_ok(int device) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n == 0) return (set_error(BQ_ERR_DEVICE, "int8: no HIP device"), 0);
  if (device < 0 || device >= n) return (set_error(BQ_ERR_DEVICE, "int8: no device %d (%d present)", device, n), 0);
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) != hipSuccess)
    return (set_error(BQ_ERR_DEVICE, "int8: cannot query device %d", device), 0);
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return (set_error(BQ_ERR_DEVICE,
                      "int8: device %d is %s; the int8 kernels are built for gfx950 (MI350/MI355X) only",
                      device, prop.gcnArchName),
            0);
  return 1;
}

int bq_quantize_rows(const float* x, int64_t M, int64_t K, int8_t* q, float* s, bq_stream_t stream) {
  return launch_rows(x, M, K, q, s, (hipStream_t)stream, "bq_quantize_rows");
}

int bq_quantize_rows_act(const float* x, int64_t M, int64_t K, int act, int8_t* q, float* s, float* y,
                         bq_stream_t stream) {
  return launch_rows(x, M, K, q, s, (hipStream_t)stream, "bq_quantize_rows_act", act, y);
}

int bq_quantize_weight_per_channel(const float* w, int64_t N, int64_t K, int8_t* q, float* s,
                                   bq_stream_t stream) {
  return launch_rows(w, N, K, q, s, (hipStream_t)stream, "bq_quantize_weight_per_channel");
}

size_t bq_quantize_tensor_ws_bytes(int64_t n) { return (size_t)nparts_for(n < 0 ? 0 : n) * sizeof(float); }

// Per-tensor quantization of x [P, C] into q [P, Cpad]. The scale is, in this order of
// precedence: s_given (calibrated); from given_parts (partial maxima a producer wrote, e.g.
// the conv epilogue's per-tile max |y|); else from partial maxima computed here into ws.
// HW > 0: x is NCHW with planes of HW pixels (the padded path only), else channels-last.
static int quantize_nhwc_impl(const char* what, const float* x, int64_t P, int64_t C, int64_t Cpad, int8_t* q,
                              float* s, const float* s_given, void* ws, size_t ws_bytes, hipStream_t st,
                              const float* given_parts = nullptr, int64_t given_np = 0, int64_t HW = 0) {
  if (P < 0 || C < 0 || Cpad < C) return set_error(BQ_ERR_ARG, "%s: bad sizes P=%lld C=%lld Cpad=%lld", what, (long long)P, (long long)C, (long long)Cpad);
  if (HW && (HW < 0 || HW > 0x7fffffff || P % HW || C == Cpad || Cpad % 16 || ((uintptr_t)q & 15)))
    return set_error(BQ_ERR_UNSUPPORTED, "%s: an NCHW input needs Cpad > C, Cpad %% 16 == 0 and a 16-byte aligned q", what);
  if (!x || !q || (!s && !s_given) || (!ws && !s_given && !given_parts))
    return set_error(BQ_ERR_ARG, "%s: null pointer", what);
  if (Cpad > 0x7fffffff) return set_error(BQ_ERR_ARG, "%s: too many channels", what);
  const int64_t n = P * C;
  int np = 0;
  const float* parts = nullptr;
  if (given_parts) {
    if (given_np < 1 || given_np > 0x7fffffff) return set_error(BQ_ERR_ARG, "%s: bad partial count %lld", what, (long long)given_np);
    parts = given_parts;
    np = (int)given_np;
  } else if (!s_given) {
    np = nparts_for(n);
    if (ws_bytes < (size_t)np * sizeof(float))
      return set_error(BQ_ERR_ARG, "%s: workspace %zu bytes, need %zu", what, ws_bytes, (size_t)np * sizeof(float));
    float* wparts = (float*)ws;
    parts = wparts;
    const int64_t chunk = n == 0 ? 1 : (n + np - 1) / np;
    absmax_parts_kernel<<<np, QT_THREADS, 0, st>>>(x, n, ((chunk + 3) / 4) * 4, wparts);
    if (int r = check_launch(what)) return r;
  }
  if (!s_given && np > 4096) {  // many maxima: fold them into s once, then quantize with it
    scale_from_parts_kernel<<<1, 1024, 0, st>>>(parts, np, s);
    if (int r = check_launch(what)) return r;
    s_given = s;
    parts = nullptr;
    np = 0;
  }
  if (C != Cpad && Cpad % 16 == 0 && ((uintptr_t)q & 15) == 0) {
    const int64_t chunks = P * (Cpad / 16);
    int64_t blocks = (chunks + QT_THREADS - 1) / QT_THREADS;
    if (blocks > 8192) blocks = 8192;
    if (blocks < 1) blocks = 1;
    quantize_pad16_kernel<<<(unsigned)blocks, QT_THREADS, 0, st>>>(x, P, (int)C, (int)Cpad, parts, np, q, s, s_given,
                                                                    (int)HW);
    return check_launch(what);
  }
  const int64_t words = (P * Cpad + 3) / 4;
  int64_t blocks = (words + QT_THREADS - 1) / QT_THREADS;
  if (blocks > 4096) blocks = 4096;
  if (blocks < 1) blocks = 1;
  quantize_tensor_kernel<<<(unsigned)blocks, QT_THREADS, 0, st>>>(x, P, (int)C, (int)Cpad, parts, np, q, s, s_given);
  return check_launch(what);
}

int bq_quantize_nhwc(const float* x, int64_t P, int64_t C, int64_t Cpad, int8_t* q, float* s, void* ws,
                     size_t ws_bytes, bq_stream_t stream) {
  return quantize_nhwc_impl("bq_quantize_nhwc", x, P, C, Cpad, q, s, nullptr, ws, ws_bytes, (hipStream_t)stream);
}

int bq_quantize_nhwc_parts(const float* x, int64_t P, int64_t C, int64_t Cpad, const float* absmax_parts,
                           int64_t nparts, int8_t* q, float* s, bq_stream_t stream) {
  if (!absmax_parts) return set_error(BQ_ERR_ARG, "bq_quantize_nhwc_parts: null partial maxima");
  return quantize_nhwc_impl("bq_quantize_nhwc_parts", x, P, C, Cpad, q, s, nullptr, nullptr, 0, (hipStream_t)stream,
                            absmax_parts, nparts);
}

int bq_quantize_nhwc_chscale(const float* x, int64_t N, int64_t HW, int64_t C, int64_t Cpad, const float* cs,
                             int8_t* q, float* s, const float* s_given, const float* absmax_parts, int64_t nparts,
                             void* ws, size_t ws_bytes, bq_stream_t stream) {
  const char* what = "bq_quantize_nhwc_chscale";
  if (N < 0 || HW < 1 || C < 1 || Cpad < C) return set_error(BQ_ERR_ARG, "%s: bad sizes", what);
  if (C % 4 || Cpad % 4) return set_error(BQ_ERR_UNSUPPORTED, "%s: C and Cpad must be multiples of 4", what);
  if (Cpad > 0x7fffffff) return set_error(BQ_ERR_ARG, "%s: too many channels", what);
  if (!x || !cs || !q || (!s && !s_given)) return set_error(BQ_ERR_ARG, "%s: null pointer", what);
  if (((uintptr_t)x | (uintptr_t)cs) & 15 || (uintptr_t)q & 3)
    return set_error(BQ_ERR_ARG, "%s: x and cs must be 16-byte aligned, q 4-byte aligned", what);
  const int64_t P = N * HW;
  if (P == 0) return BQ_OK;
  if (P * Cpad >= ((int64_t)1 << 31) || HW > 0x7fffffff)
    return set_error(BQ_ERR_ARG, "%s: size too large (P * Cpad must be < 2^31)", what);
  hipStream_t st = (hipStream_t)stream;
  const FastDiv dhw = fast_div((uint32_t)HW);
  int np = 0;
  const float* parts = nullptr;
  if (!s_given && absmax_parts) {  // the maxima of the product, from the gate's producer
    if (nparts < 1 || nparts > 0x7fffffff) return set_error(BQ_ERR_ARG, "%s: bad nparts %lld", what, (long long)nparts);
    parts = absmax_parts;
    np = (int)nparts;
  } else if (!s_given) {
    np = nparts_for(P * C);
    if (!ws || ws_bytes < (size_t)np * sizeof(float))
      return set_error(BQ_ERR_ARG, "%s: workspace %zu bytes, need %zu", what, ws_bytes, (size_t)np * sizeof(float));
    parts = (float*)ws;
    absmax_chscale_kernel<<<np, QT_THREADS, 0, st>>>(x, cs, (int)P, (int)C, dhw.mul, dhw.shift, (float*)ws);
    if (int r = check_launch(what)) return r;
  }
  if (!s_given && np > 4096) {  // many maxima: fold them into s once
    scale_from_parts_kernel<<<1, 1024, 0, st>>>(parts, np, s);
    if (int r = check_launch(what)) return r;
    s_given = s;
    parts = nullptr;
    np = 0;
  }
  int64_t blocks = (P * (Cpad / 4) + QT_THREADS - 1) / QT_THREADS;
  if (blocks > 8192) blocks = 8192;
  quantize_chscale_kernel<<<(unsigned)blocks, QT_THREADS, 0, st>>>(x, cs, (int)P, (int)C, (int)Cpad, dhw.mul,
                                                                   dhw.shift, parts, np, q, s, s_given);
  return check_launch(what);
}

int bq_quantize_nhwc_scaled(const float* x, int64_t P, int64_t C, int64_t Cpad, const float* s, int8_t* q,
                            bq_stream_t stream) {
  if (!s) return set_error(BQ_ERR_ARG, "bq_quantize_nhwc_scaled: null scale");
  return quantize_nhwc_impl("bq_quantize_nhwc_scaled", x, P, C, Cpad, q, nullptr, s, nullptr, 0, (hipStream_t)stream);
}

int bq_quantize_nchw(const float* x, int64_t N, int64_t C, int64_t HW, int64_t Cpad, int8_t* q, float* s, void* ws,
                     size_t ws_bytes, bq_stream_t stream) {
  if (N < 0 || HW < 1) return set_error(BQ_ERR_ARG, "bq_quantize_nchw: bad sizes");
  return quantize_nhwc_impl("bq_quantize_nchw", x, N * HW, C, Cpad, q, s, nullptr, ws, ws_bytes, (hipStream_t)stream,
                            nullptr, 0, HW);
}

int bq_quantize_nchw_scaled(const float* x, int64_t N, int64_t C, int64_t HW, int64_t Cpad, const float* s, int8_t* q,
                            bq_stream_t stream) {
  if (!s) return set_error(BQ_ERR_ARG, "bq_quantize_nchw_scaled: null scale");
  if (N < 0 || HW < 1) return set_error(BQ_ERR_ARG, "bq_quantize_nchw_scaled: bad sizes");
  return quantize_nhwc_impl("bq_quantize_nchw_scaled", x, N * HW, C, Cpad, q, nullptr, s, nullptr, 0,
                            (hipStream_t)stream, nullptr, 0, HW);
}

int bq_layernorm_quantize_rows(const float* x, int64_t M, int64_t K, const float* gamma, const float* beta, float eps,
                               int8_t* q, float* s, float* y, bq_stream_t stream) {
  const char* what = "bq_layernorm_quantize_rows";
  if (M < 0 || K < 1) return set_error(BQ_ERR_ARG, "%s: bad sizes (%lld x %lld)", what, (long long)M, (long long)K);
  if (M == 0) return BQ_OK;
  if (M > 0x7fffffff) return set_error(BQ_ERR_ARG, "%s: size too large", what);
  if (K % 4 || K > 4096)
    return set_error(BQ_ERR_UNSUPPORTED, "%s: K=%lld (a multiple of 4, at most 4096)", what, (long long)K);
  if (!x || !q || !s) return set_error(BQ_ERR_ARG, "%s: null pointer", what);
  if (((uintptr_t)x | (uintptr_t)gamma | (uintptr_t)beta | (uintptr_t)y) & 15 || (uintptr_t)q & 3)
    return set_error(BQ_ERR_ARG, "%s: x, gamma, beta, y must be 16-byte aligned, q 4-byte aligned", what);
  if (!(eps >= 0.f)) return set_error(BQ_ERR_ARG, "%s: eps must be >= 0", what);
  hipStream_t st = (hipStream_t)stream;
  dim3 g((unsigned)((M + QW_WAVES - 1) / QW_WAVES)), b(QW_WAVES * 64);
  const int nw = (int)((K + 255) / 256);
  auto go = [&](auto kern) { kern<<<g, b, 0, st>>>(x, (int)M, (int)K, gamma, beta, eps, q, s, y); };
  if (nw == 1) go(ln_quantize_rows_kernel<1>);
  else if (nw == 2) go(ln_quantize_rows_kernel<2>);
  else if (nw == 3) go(ln_quantize_rows_kernel<3>);
  else if (nw == 4) go(ln_quantize_rows_kernel<4>);
  else if (nw <= 6) go(ln_quantize_rows_kernel<6>);
  else if (nw <= 8) go(ln_quantize_rows_kernel<8>);
  else if (nw <= 12) go(ln_quantize_rows_kernel<12>);
  else go(ln_quantize_rows_kernel<16>);
  return check_launch(what);
}

int bq_quantize_tensor(const float* x, int64_t n, int8_t* q, float* s, void* ws, size_t ws_bytes,
                       bq_stream_t stream) {
  return bq_quantize_nhwc(x, n, 1, 1, q, s, ws, ws_bytes, stream);
}

}  // extern "C"
