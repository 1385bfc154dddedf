// Squeeze-excite gates in f32 for a channels-last activation (EfficientNet's MBConv):
//   pooled[n, c] = (sum over the HW pixels of x[n, p, c]) * (1 / HW)
//   z[n, j]      = silu(b1[j] + sum_c w1[j, c] * pooled[n, c])        (j < S, the squeeze width)
//   gate[n, c]   = sigmoid(b2[c] + sum_j w2t[j, c] * z[n, j])   (w2t: the expand weight transposed)
// the operation of borch's CPU runner "se" node (borch-ts/src/cpu/runner.ts:256-268:
// meanRows, gemmBiasAct(swish), gemmBiasAct(sigmoid); lib.rs:222-244 mean_rows). The gate
// multiplies the activation inside the next conv's quantizer (bq_quantize_nhwc_chscale)
// instead of the runner's scaleRows pass. Two kernels: partial sums (and maxima) over row
// chunks (the bandwidth pass), then one workgroup per image finishes the mean and runs the
// small MLP. Every sum has a fixed order: results do not depend on scheduling.
//
// The excite also gives the quantizer of the product its dynamic scale without a pass over
// x: the gate is positive and f32 rounding is monotonic, so over the pixels of (n, c)
// max |fl(x * g)| = fl(max |x| * g). The partial pass keeps max |x| per chunk and channel;
// the gate workgroup of each image writes the maximum of fl(max|x| * g) over its channels.
#include <algorithm>

#include "bq_common.h"

namespace bq {

constexpr int SE_THREADS = 256;     // the partial-sum pass
constexpr int GATE_THREADS = 1024;  // the per-image pass: 16 waves cover the squeeze outputs and channels

__device__ __forceinline__ float sigmoid_f(float v) {
  return __builtin_amdgcn_rcpf(__fadd_rn(1.0f, __builtin_amdgcn_exp2f(__fmul_rn(v, -1.4426950408889634f))));
}

// Block (n, chunk): rows [chunk * rows_per, ...) of image n; thread t sums channel group
// g = t % G (4 channels) over the rows r = t / G, t / G + TR, ... of the chunk (TR = 256 / G
// row lanes, G >= 1 groups a pass, more passes when C / 4 > 256), eight rows' loads issued
// before they are added in row order; the TR row-lane sums of a group are then added in
// lane order through LDS. partial[(n * chunks + chunk) * C + c]; with `pmax`, max |x| of the
// same rows at the same index.
__global__ __launch_bounds__(SE_THREADS) void se_partial_kernel(const float* __restrict__ x, int HW, int C,
                                                                int chunks, int rows_per,
                                                                float* __restrict__ partial,
                                                                float* __restrict__ pmax) {
  __shared__ float4 red[SE_THREADS];
  __shared__ float4 redm[SE_THREADS];
  const int n = blockIdx.x / chunks, chunk = blockIdx.x - n * chunks;
  const int r0 = chunk * rows_per, r1 = min(HW, r0 + rows_per);
  const int groups = C / 4;
  const int G = min(groups, SE_THREADS);
  const int TR = SE_THREADS / G;
  const int t = threadIdx.x;
  const int lane_r = t / G, g0 = t - lane_r * G;
  const float* xn = x + (size_t)n * HW * C;
  constexpr int U = 8;
  for (int gb = 0; gb < groups; gb += G) {
    const int g = gb + g0;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f), mx = acc;
    if (lane_r < TR && g < groups) {
      const float* xg = xn + g * 4;
      for (int r = r0 + lane_r; r < r1; r += U * TR) {
        float4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int rr = r + u * TR;
          v[u] = rr < r1 ? *reinterpret_cast<const float4*>(xg + (size_t)rr * C) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          acc.x = __fadd_rn(acc.x, v[u].x); acc.y = __fadd_rn(acc.y, v[u].y);
          acc.z = __fadd_rn(acc.z, v[u].z); acc.w = __fadd_rn(acc.w, v[u].w);
          mx.x = fmaxf(mx.x, fabsf(v[u].x)); mx.y = fmaxf(mx.y, fabsf(v[u].y));
          mx.z = fmaxf(mx.z, fabsf(v[u].z)); mx.w = fmaxf(mx.w, fabsf(v[u].w));
        }
      }
    }
    red[t] = acc;
    redm[t] = mx;
    __syncthreads();
    if (t < G && gb + t < groups) {
      float4 s = red[t], m = redm[t];
      for (int k = 1; k < TR; ++k) {
        const float4 v = red[k * G + t], w = redm[k * G + t];
        s.x = __fadd_rn(s.x, v.x); s.y = __fadd_rn(s.y, v.y);
        s.z = __fadd_rn(s.z, v.z); s.w = __fadd_rn(s.w, v.w);
        m.x = fmaxf(m.x, w.x); m.y = fmaxf(m.y, w.y); m.z = fmaxf(m.z, w.z); m.w = fmaxf(m.w, w.w);
      }
      const size_t o = ((size_t)n * chunks + chunk) * C + (gb + t) * 4;
      *reinterpret_cast<float4*>(partial + o) = s;
      if (pmax) *reinterpret_cast<float4*>(pmax + o) = m;
    }
    __syncthreads();
  }
}

// One block per image: pooled and max |x| per channel (in LDS), z = silu(W1 pooled + b1)
// (one wave per output j, its lanes over c, a wave tree), gate = sigmoid(W2 z + b2) (one
// thread per channel, reading the transposed expand weight w2t [S, C] so a wave's loads are
// contiguous). With `amax`: max over c of fl(max|x[n, :, c]| * gate[n, c]) into amax[n].
// (Splitting the squeeze and the excite into two wider kernels was slower on every B0
// layer: 9-18 us against 5.5-18 us, each small launch paying its own latency chain.)
__global__ __launch_bounds__(GATE_THREADS) void se_gate_kernel(const float* __restrict__ partial,
                                                             const float* __restrict__ pmax, int chunks, int HW,
                                                             int C, int S, const float* __restrict__ w1,
                                                             const float* __restrict__ b1,
                                                             const float* __restrict__ w2t,
                                                             const float* __restrict__ b2, float* __restrict__ gate,
                                                             float* __restrict__ amax) {
  extern __shared__ float sm[];  // pooled [C], z [S], xmax [C] (with amax)
  __shared__ float wmax[GATE_THREADS / 64];
  float* pooled = sm;
  float* z = sm + C;
  float* xmax = sm + C + S;
  const int n = blockIdx.x;
  const float inv = __fdiv_rn(1.0f, (float)HW);
  for (int c = threadIdx.x; c < C; c += GATE_THREADS) {
    float s = 0.f, m = 0.f;
    for (int k0 = 0; k0 < chunks; k0 += 8) {  // eight loads in flight, added in chunk order
      float v[8], w[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const size_t o = ((size_t)n * chunks + k0 + k) * C + c;
        v[k] = k0 + k < chunks ? partial[o] : 0.f;
        w[k] = (amax && k0 + k < chunks) ? pmax[o] : 0.f;
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        if (k0 + k < chunks) s = __fadd_rn(s, v[k]);
        m = fmaxf(m, w[k]);
      }
    }
    pooled[c] = __fmul_rn(s, inv);
    if (amax) xmax[c] = m;
  }
  __syncthreads();
  // z: each wave builds JW outputs at once, its lanes over c (c = lane, lane + 64, ... in
  // order for every output), all loads of a batch issued before its FMAs; then a fixed-order
  // DPP wave sum.
  constexpr int JW = 4, CU = 4;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int j0 = wave * JW; j0 < S; j0 += (GATE_THREADS / 64) * JW) {
    float acc[JW];
#pragma unroll
    for (int q = 0; q < JW; ++q) acc[q] = 0.f;
    for (int c0 = lane; c0 < C; c0 += 64 * CU) {
      float pv[CU], wv[JW][CU];
#pragma unroll
      for (int u = 0; u < CU; ++u) {
        const int c = c0 + 64 * u;
        pv[u] = c < C ? pooled[c] : 0.f;
#pragma unroll
        for (int q = 0; q < JW; ++q) wv[q][u] = (c < C && j0 + q < S) ? w1[(size_t)(j0 + q) * C + c] : 0.f;
      }
#pragma unroll
      for (int u = 0; u < CU; ++u)
#pragma unroll
        for (int q = 0; q < JW; ++q) acc[q] = __fmaf_rn(wv[q][u], pv[u], acc[q]);
    }
#pragma unroll
    for (int q = 0; q < JW; ++q) {
      const float v = wave_sum_fixed(acc[q]);  // the whole wave is here (the loop is per wave)
      if (lane == 0 && j0 + q < S) z[j0 + q] = silu(__fadd_rn(v, b1 ? b1[j0 + q] : 0.f));
    }
  }
  __syncthreads();
  // gate: each thread CW channels at once (c0, c0 + 1024, ...), j in order, JU loads of w2t
  // a channel issued before their FMAs.
  constexpr int CW = 4, JU = 8;
  float m = 0.f;
  for (int c0 = threadIdx.x; c0 < C; c0 += GATE_THREADS * CW) {
    float acc[CW];
#pragma unroll
    for (int u = 0; u < CW; ++u) {
      const int c = c0 + GATE_THREADS * u;
      acc[u] = (b2 && c < C) ? b2[c] : 0.f;
    }
    for (int j0 = 0; j0 < S; j0 += JU) {
      float wv[JU][CW], zv[JU];
#pragma unroll
      for (int v = 0; v < JU; ++v) {
        zv[v] = j0 + v < S ? z[j0 + v] : 0.f;
#pragma unroll
        for (int u = 0; u < CW; ++u) {
          const int c = c0 + GATE_THREADS * u;
          wv[v][u] = (j0 + v < S && c < C) ? w2t[(size_t)(j0 + v) * C + c] : 0.f;
        }
      }
#pragma unroll
      for (int v = 0; v < JU; ++v)
#pragma unroll
        for (int u = 0; u < CW; ++u) acc[u] = __fmaf_rn(wv[v][u], zv[v], acc[u]);
    }
#pragma unroll
    for (int u = 0; u < CW; ++u) {
      const int c = c0 + GATE_THREADS * u;
      if (c < C) {
        const float g = sigmoid_f(acc[u]);
        gate[(size_t)n * C + c] = g;
        if (amax) m = fmaxf(m, __fmul_rn(xmax[c], g));
      }
    }
  }
  if (amax) {  // uniform
    m = wave_max(m);
    if (lane == 0) wmax[wave] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
      float r = wmax[0];
#pragma unroll
      for (int w = 1; w < GATE_THREADS / 64; ++w) r = fmaxf(r, wmax[w]);
      amax[n] = r;
    }
  }
}

static int se_chunks(int64_t HW, int64_t C) {
  int64_t k = HW * C / 16384;
  k = std::min<int64_t>(k, std::min<int64_t>(HW, 64));
  return (int)std::max<int64_t>(k, 1);
}

// A classifier head in f32, beside the int8 path: the global average pool of a channels-last
// activation x [N, HW, C] and the Linear after it, out[n, o] = b[o] + sum_c pooled[n, c] *
// w[o, c] with pooled[n, c] = (sum over the HW pixels of x[n, p, c], in pixel order) / HW.
// One workgroup per image: the pooled vector in LDS, then a wave per output, its lanes over
// c in order and a fixed-order wave sum. For the small heads (O * C <= 65536: CIFAR
// ResNet-18's 512 -> 10) where the pool and the GEMM would be two launches of a few
// microseconds each.
constexpr int HEAD_THREADS = 256;

__global__ __launch_bounds__(HEAD_THREADS) void avgpool_linear_kernel(const float* __restrict__ x, int HW, int C,
                                                                      const float* __restrict__ w,
                                                                      const float* __restrict__ b, int O,
                                                                      float* __restrict__ out) {
  extern __shared__ float pooled[];
  const int n = blockIdx.x;
  const float* xn = x + (size_t)n * HW * C;
  // eight loads in flight before their adds / FMAs (in order): a loop of dependent round trips
  // would cost one each
  constexpr int U = 8;
  for (int c = threadIdx.x; c < C; c += HEAD_THREADS) {
    float s = 0.f;
    for (int p0 = 0; p0 < HW; p0 += U) {
      float v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) v[u] = p0 + u < HW ? xn[(size_t)(p0 + u) * C + c] : 0.f;
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (p0 + u < HW) s = __fadd_rn(s, v[u]);
    }
    pooled[c] = __fdiv_rn(s, (float)HW);
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int o = wave; o < O; o += HEAD_THREADS / 64) {
    const float* wo = w + (size_t)o * C;
    float acc = 0.f;
    for (int c0 = lane; c0 < C; c0 += 64 * U) {
      float v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) v[u] = c0 + 64 * u < C ? wo[c0 + 64 * u] : 0.f;
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (c0 + 64 * u < C) acc = __fmaf_rn(pooled[c0 + 64 * u], v[u], acc);
    }
    const float v = wave_sum_fixed(acc);  // the whole wave is here (the loop is per wave)
    if (lane == 0) out[(size_t)n * O + o] = b ? __fadd_rn(v, b[o]) : v;
  }
}

}  // namespace bq

using namespace bq;

extern "C" {

size_t bq_se_gate_ws_bytes(int64_t N, int64_t HW, int64_t C) {
  if (N < 0 || HW < 1 || C < 0) return 0;
  return 2 * (size_t)N * se_chunks(HW, C) * C * sizeof(float);  // partial sums, then partial maxima
}

int64_t bq_se_gate_absmax_parts(int64_t N, int64_t C) {
  if (N < 0 || C < 1) return set_error(BQ_ERR_ARG, "bq_se_gate_absmax_parts: bad sizes");
  return N;
}

int bq_se_gate_nhwc(const float* x, int64_t N, int64_t HW, int64_t C, const float* w1, const float* b1, int64_t S,
                    const float* w2t, const float* b2, float* gate, float* absmax_parts, void* ws, size_t ws_bytes,
                    bq_stream_t stream) {
  const char* what = "bq_se_gate_nhwc";
  if (N < 0 || HW < 1 || C < 4 || S < 1) return set_error(BQ_ERR_ARG, "%s: bad sizes", what);
  if (C % 4) return set_error(BQ_ERR_UNSUPPORTED, "%s: C=%lld is not a multiple of 4", what, (long long)C);
  if (N * HW * C >= ((int64_t)1 << 40) || HW > 0x7fffffff || C > 65536 || S > 65536)
    return set_error(BQ_ERR_ARG, "%s: size too large", what);
  if (N == 0) return BQ_OK;
  if (!x || !w1 || !w2t || !gate) return set_error(BQ_ERR_ARG, "%s: null pointer", what);
  if ((uintptr_t)x & 15) return set_error(BQ_ERR_ARG, "%s: x must be 16-byte aligned", what);
  const int chunks = se_chunks(HW, C);
  const size_t need = bq_se_gate_ws_bytes(N, HW, C);
  if (!ws || ws_bytes < need) return set_error(BQ_ERR_ARG, "%s: workspace %zu bytes, need %zu", what, ws_bytes, need);
  if ((uintptr_t)ws & 15) return set_error(BQ_ERR_ARG, "%s: workspace must be 16-byte aligned", what);
  if ((2 * C + S) * sizeof(float) > 64 * 1024) return set_error(BQ_ERR_UNSUPPORTED, "%s: 2 C + S too large", what);
  float* partial = (float*)ws;
  float* pmax = partial + (size_t)N * chunks * C;
  hipStream_t st = (hipStream_t)stream;
  const int rows_per = (int)((HW + chunks - 1) / chunks);
  se_partial_kernel<<<(unsigned)(N * chunks), SE_THREADS, 0, st>>>(x, (int)HW, (int)C, chunks, rows_per, partial,
                                                                   absmax_parts ? pmax : nullptr);
  if (int r = check_launch(what)) return r;
  const size_t lds = (size_t)(C + S + (absmax_parts ? C : 0)) * sizeof(float);
  se_gate_kernel<<<(unsigned)N, GATE_THREADS, lds, st>>>(partial, pmax, chunks, (int)HW, (int)C, (int)S, w1, b1, w2t,
                                                         b2, gate, absmax_parts);
  return check_launch(what);
}

int bq_avgpool_linear_f32(const float* x, int64_t N, int64_t HW, int64_t C, const float* w, const float* b,
                          int64_t O, float* out, bq_stream_t stream) {
  const char* what = "bq_avgpool_linear_f32";
  if (N < 0 || HW < 1 || C < 1 || O < 1) return set_error(BQ_ERR_ARG, "%s: bad sizes", what);
  if (O * C > 65536 || C > 16384) return set_error(BQ_ERR_UNSUPPORTED, "%s: O * C = %lld (at most 65536)", what,
                                                   (long long)(O * C));
  if (N * HW * C >= ((int64_t)1 << 31) || N > 0x7fffffff) return set_error(BQ_ERR_ARG, "%s: size too large", what);
  if (N == 0) return BQ_OK;
  if (!x || !w || !out) return set_error(BQ_ERR_ARG, "%s: null pointer", what);
  avgpool_linear_kernel<<<(unsigned)N, HEAD_THREADS, (size_t)C * sizeof(float), (hipStream_t)stream>>>(
      x, (int)HW, (int)C, w, b, (int)O, out);
  return check_launch(what);
}

}  // extern "C"
