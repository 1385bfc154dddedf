// Weight-only int8 (W8A32): f32 activations against an int8 weight with one f32 scale per
// output channel; the effective weight is f32(q) * scale (one rounding), the products are
// accumulated in f32 (FMA). The reference's `matmul(..., weightInt8)` (borch-ts/src/
// kernels.ts:2695-2708) for streamed/windowed weights, and its `dequantInt8` unpack pass
// (kernels.ts:1264-1274).
//
// gemv_w8a32_kernel (M <= 4, the decode shape; gemv_w8a32_mfma_kernel below for M = 5..8):
// HBM-bound on the int8 weight — a quarter of the f32 bytes. Each wave owns RPW weight rows; a row is read as contiguous 1 KB
// wave-loads (64 lanes x 16 bytes) and every load of the wave's rows is issued before any
// arithmetic; each lane multiplies its 16 weights against the matching 16 activations
// (L1/L2-resident, reused across the wave's rows) and the wave reduces the lane sums.
#include "bq_common.h"

namespace bq {

constexpr uint32_t W_OOB = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t w_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

constexpr int WA_WAVES = 8;
constexpr int WA_MMAX = 8;  // activation rows a launch takes (the decode shapes)
// From this many activation rows the MFMA kernel runs (4096 x 4096, us, per-wave / MFMA:
// M=2 7.9 / 11.4, M=4 10.5 / 11.7, M=5 13.0 / 11.7, M=6 14.4 / 11.9, M=8 17.3 / 12.8).
constexpr int WA_MFMA_MIN_M = 5;
constexpr int WA_MPW = WA_MFMA_MIN_M - 1;  // activation rows the per-wave kernel takes
constexpr int WA_XLDS = 16384;       // f32 activations staged through registers (64 KB of LDS)
constexpr int WA_XLDS_BIG = 32768;   // staged by a load loop after the weights (128 KB of LDS)

// XL: the activation rows (M rows of KC * 1024 floats, K padded to whole 1 KB weight chunks)
// are staged in LDS once per workgroup and every wave reads them from there (up to
// WA_XLDS floats, their loads issued before the weights' and held in registers, so that
// the wait for them is not a wait for the weights; up to WA_XLDS_BIG, by a loop after the
// weight loads: 8 rows of 4096 at 23.8 -> 19.1 us instead of every wave reading them from
// L2). The register staging: one row of 4096 at 7.6 -> 7.3 us, four at 12.3 -> 11.5 us.
// CO: the products chunk by chunk as each weight chunk lands (M = 1: one row of 4096 at
// 7.0 -> 6.5 us); else row by row once every chunk has landed (M = 2..4: 8.0 / 9.0 / 10.1
// us, 0.1-0.8 us less than chunk by chunk).
template <int KC, int RPW, bool XL, int XN = WA_XLDS, bool CO = false>
__global__ __launch_bounds__(WA_WAVES * 64) void gemv_w8a32_kernel(const float* __restrict__ x, const int8_t* W,
                                                                   int M, int N, int K, const float* __restrict__ sW,
                                                                   const float* __restrict__ bias, int act,
                                                                   float* __restrict__ out) {
  __shared__ __attribute__((aligned(16))) float xs[XL ? XN : 4];
  constexpr int T = WA_WAVES * 64;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int row0 = (blockIdx.x * WA_WAVES + wave) * RPW;
  const int nrows = max(0, min(RPW, N - row0));  // 0 past N: every weight load out of range
  const __amdgpu_buffer_rsrc_t rw = w_rsrc(W + (size_t)min(row0, N) * K, (uint32_t)(nrows * K));
  // the activations' loads first: the wait for them (before the LDS writes) then does not
  // wait for the weight loads issued after them
  constexpr bool XREG = XL && XN <= WA_XLDS;  // staged through registers
  constexpr int XR = XREG ? XN / 4 / T : 1;
  float4 xr[XR];
  const int k4 = K / 4;
  const int n4 = M * k4;
  if constexpr (XREG) {
#pragma unroll
    for (int r = 0; r < XR; ++r) {
      const int i = tid + r * T;
      xr[r] = i < n4 ? reinterpret_cast<const float4*>(x)[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  float sc[RPW];  // before the weights: the first products then wait for chunk 0 only
#pragma unroll
  for (int j = 0; j < RPW; ++j) sc[j] = j < nrows ? sW[row0 + j] : 0.f;
  v4i w[RPW][KC];
  // chunk-major, the order the products use them: chunk c waits for its own loads only
#pragma unroll
  for (int c = 0; c < KC; ++c)
#pragma unroll
    for (int j = 0; j < RPW; ++j) {
      const int k = c * 1024 + lane * 16;
      w[j][c] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rw, k < K ? (uint32_t)(j * K + k) : W_OOB, 0, 0));
    }
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (XL) {
    // Row m's float4 number c*256 + l*4 + t (the t-th of lane l's four in 1 KB chunk c) is
    // stored at float4 (m*KC + c)*256 + t*64 + l, so the four reads of a chunk each take
    // 64 consecutive float4s across the wave (no bank conflicts).
    if constexpr (XREG) {
#pragma unroll
      for (int rr = 0; rr < XR; ++rr) {
        const int i = tid + rr * T;
        if (i < n4) {
          const int m = i / k4;
          const int r = i - m * k4;
          const int dst = (m * KC + (r >> 8)) * 256 + (r & 3) * 64 + ((r >> 2) & 63);
          reinterpret_cast<float4*>(xs)[dst] = xr[rr];
        }
      }
    } else {
      for (int i = tid; i < n4; i += T) {
        const int m = i / k4;
        const int r = i - m * k4;
        const int dst = (m * KC + (r >> 8)) * 256 + (r & 3) * 64 + ((r >> 2) & 63);
        reinterpret_cast<float4*>(xs)[dst] = reinterpret_cast<const float4*>(x)[i];
      }
    }
    __syncthreads();
  }
  if constexpr (CO) {
    // Chunk by chunk, as the loads arrive: the chunk's effective weights f32(q) * scale, then
    // every row's FMAs against them (each output accumulates chunk by chunk, byte by byte).
    float acc[WA_MPW][RPW];
#pragma unroll
    for (int m = 0; m < WA_MPW; ++m)
#pragma unroll
      for (int j = 0; j < RPW; ++j) acc[m][j] = 0.f;
#pragma unroll
    for (int c = 0; c < KC; ++c) {
      const int k = c * 1024 + lane * 16;
      if (c * 1024 >= K) break;  // uniform
      float wf[RPW][16];
#pragma unroll
      for (int j = 0; j < RPW; ++j)
#pragma unroll
        for (int q = 0; q < 16; ++q)
          wf[j][q] = __fmul_rn((float)(int)(int8_t)((uint32_t)w[j][c][q >> 2] >> ((q & 3) * 8)), sc[j]);
#pragma unroll
      for (int m = 0; m < WA_MPW; ++m) {
        if (m >= M) break;  // uniform
        const float4* xp = XL ? reinterpret_cast<const float4*>(xs) + (m * KC + c) * 256 + lane
                              : reinterpret_cast<const float4*>(x + (size_t)m * K + k);
        float xv[16];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const float4 v = k < K ? xp[XL ? t * 64 : t] : make_float4(0.f, 0.f, 0.f, 0.f);
          xv[t * 4] = v.x; xv[t * 4 + 1] = v.y; xv[t * 4 + 2] = v.z; xv[t * 4 + 3] = v.w;
        }
#pragma unroll
        for (int j = 0; j < RPW; ++j)
#pragma unroll
          for (int q = 0; q < 16; ++q) acc[m][j] = __fmaf_rn(xv[q], wf[j][q], acc[m][j]);
      }
    }
#pragma unroll
    for (int m = 0; m < WA_MPW; ++m) {
      if (m >= M) break;
#pragma unroll
      for (int j = 0; j < RPW; ++j) {
        const float s = wave_sum_fixed(acc[m][j]);  // every lane is here
        const int n = row0 + j;
        if (lane == 0 && j < nrows) {
          float v = bias ? __fadd_rn(s, bias[n]) : s;
          v = activate(v, act);
          out[(size_t)m * N + n] = v;
        }
      }
    }
  } else {
    for (int m = 0; m < M; ++m) {
      float acc[RPW];
#pragma unroll
      for (int j = 0; j < RPW; ++j) acc[j] = 0.f;
#pragma unroll
      for (int c = 0; c < KC; ++c) {
        const int k = c * 1024 + lane * 16;
        if (k >= K) break;
        const float4* xp = XL ? reinterpret_cast<const float4*>(xs) + (m * KC + c) * 256 + lane
                              : reinterpret_cast<const float4*>(x + (size_t)m * K + k);
        float xv[16];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const float4 v = xp[XL ? t * 64 : t];
          xv[t * 4] = v.x; xv[t * 4 + 1] = v.y; xv[t * 4 + 2] = v.z; xv[t * 4 + 3] = v.w;
        }
#pragma unroll
        for (int j = 0; j < RPW; ++j)
#pragma unroll
          for (int q = 0; q < 16; ++q) {
            const int b = (int)(int8_t)((uint32_t)w[j][c][q >> 2] >> ((q & 3) * 8));
            acc[j] = __fmaf_rn(xv[q], __fmul_rn((float)b, sc[j]), acc[j]);
          }
      }
#pragma unroll
      for (int j = 0; j < RPW; ++j) {
        const float s = wave_sum_fixed(acc[j]);  // every lane is here
        const int n = row0 + j;
        if (lane == 0 && j < nrows) {
          float v = bias ? __fadd_rn(s, bias[n]) : s;
          v = activate(v, act);
          out[(size_t)m * N + n] = v;
        }
      }
    }
  }
}

// gemv_w8a32_mfma_kernel (2 <= M <= 8): the products on v_mfma_f32_16x16x4_f32. A
// workgroup owns 16 weight rows; its waves split K into 64-byte chunks (wave w takes
// chunks w, w + 8, ...). Lane l holds 16 bytes of weight row l % 16 at K offset
// 64 c + 16 (l / 16) and the 16 matching floats of activation row l % 16 (zero for rows
// >= M); MFMA j of a chunk multiplies byte j of every lane's piece, so the MFMA's K index
// l / 16 stands for K offset 64 c + 16 (l / 16) + j in both operands. The effective weight
// is f32(q) * scale (one rounding, as in the kernel above); the f32 sums take another
// order, within the same f32-accumulation bound. The per-wave kernel above reads every
// activation row in every wave and does M FMAs a weight on the VALU: at M = 8, 17.3 us for
// a 4096 x 4096 weight. Partial 16 x 16 blocks meet through LDS in wave order.
constexpr int WM_ROWS = 16;
template <int CPW>  // 64-byte chunks a wave: K <= CPW * 8 * 64
__global__ __launch_bounds__(WA_WAVES * 64) void gemv_w8a32_mfma_kernel(const float* __restrict__ x, const int8_t* W,
                                                                        int M, int N, int K,
                                                                        const float* __restrict__ sW,
                                                                        const float* __restrict__ bias, int act,
                                                                        float* __restrict__ out) {
  typedef float v4f __attribute__((ext_vector_type(4)));
  __shared__ float red[WA_WAVES][WM_ROWS][16];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int n0 = blockIdx.x * WM_ROWS;
  const int nrows = min(WM_ROWS, N - n0);
  const int r = lane & 15;        // weight row (A operand) and activation row (B operand) of this lane
  const int kq = (lane >> 4) * 16;  // this lane's 16-byte piece of a 64-byte chunk
  const __amdgpu_buffer_rsrc_t rw = w_rsrc(W + (size_t)n0 * K, (uint32_t)(nrows * K));  // rows past N read 0
  const bool xrow = r < M;
  // The activations in batches of up to 8 chunks (64 floats a lane in registers). The scale
  // and the first batch are issued before the weights, so that chunk c's MFMAs wait for
  // weight chunk c only (the counter drains in issue order), not for the whole stream.
  constexpr int XB = CPW < 8 ? CPW : 8;
  float4 xv[XB][4];
  auto load_x = [&](int b0) {
#pragma unroll
    for (int c = 0; c < XB; ++c) {
      const int k = (wave + WA_WAVES * (b0 + c)) * 64 + kq;
#pragma unroll
      for (int t = 0; t < 4; ++t)
        xv[c][t] = xrow && k < K ? *reinterpret_cast<const float4*>(x + (size_t)r * K + k + 4 * t)
                                 : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  const float sc = r < nrows ? sW[n0 + r] : 0.f;
  load_x(0);
  v4i w[CPW];
#pragma unroll
  for (int c = 0; c < CPW; ++c) {
    const int k = (wave + WA_WAVES * c) * 64 + kq;
    w[c] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rw, k < K ? (uint32_t)(r * K + k) : W_OOB, 0, 0));
  }
  __builtin_amdgcn_sched_barrier(0);  // every load above is issued before the first MFMA
  v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int b0 = 0; b0 < CPW; b0 += XB) {
    if ((wave + WA_WAVES * b0) * 64 >= K) break;  // uniform across the wave
    if (b0 > 0) load_x(b0);
#pragma unroll
    for (int c = 0; c < XB; ++c) {
      if ((wave + WA_WAVES * (b0 + c)) * 64 >= K) break;  // uniform across the wave
      const float xs[16] = {xv[c][0].x, xv[c][0].y, xv[c][0].z, xv[c][0].w, xv[c][1].x, xv[c][1].y,
                            xv[c][1].z, xv[c][1].w, xv[c][2].x, xv[c][2].y, xv[c][2].z, xv[c][2].w,
                            xv[c][3].x, xv[c][3].y, xv[c][3].z, xv[c][3].w};
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const float wf = __fmul_rn((float)(int)(int8_t)((uint32_t)w[b0 + c][j >> 2] >> ((j & 3) * 8)), sc);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(wf, xs[j], acc, 0, 0, 0);
      }
    }
  }
  // result register i of lane l: weight row 4 (l / 16) + i, activation row l % 16
#pragma unroll
  for (int i = 0; i < 4; ++i) red[wave][(lane >> 4) * 4 + i][lane & 15] = acc[i];
  __syncthreads();
  if (tid < WM_ROWS * 16) {
    const int row = tid >> 4;
    const int m = tid & 15;
    if (m < M && row < nrows) {
      float s = red[0][row][m];
#pragma unroll
      for (int wv = 1; wv < WA_WAVES; ++wv) s = __fadd_rn(s, red[wv][row][m]);
      const float v = bias ? __fadd_rn(s, bias[n0 + row]) : s;
      out[(size_t)m * N + n0 + row] = activate(v, act);
    }
  }
}

// w[n, k] = f32(q[n, k]) * s[n] (one rounding), four elements a thread.
__global__ __launch_bounds__(256) void dequant_i8_kernel(const int8_t* __restrict__ q, int64_t N, int64_t K,
                                                         const float* __restrict__ s, float* __restrict__ w) {
  const int64_t total = N * K;
  for (int64_t e = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4; e < total; e += (int64_t)gridDim.x * 256 * 4) {
    if (e + 3 < total && (K & 3) == 0) {
      const uint32_t v = *reinterpret_cast<const uint32_t*>(q + e);
      const float sc = s[e / K];
      *reinterpret_cast<float4*>(w + e) =
          make_float4(__fmul_rn((float)(int8_t)(v & 0xff), sc), __fmul_rn((float)(int8_t)((v >> 8) & 0xff), sc),
                      __fmul_rn((float)(int8_t)((v >> 16) & 0xff), sc), __fmul_rn((float)(int8_t)(v >> 24), sc));
    } else {
      for (int64_t i = e; i < e + 4 && i < total; ++i) w[i] = __fmul_rn((float)q[i], s[i / K]);
    }
  }
}

}  // namespace bq

using namespace bq;

extern "C" {

int bq_gemv_w8a32(const float* x, const int8_t* W, int64_t M, int64_t N, int64_t K, const float* sW,
                  const float* bias, int act, float* out, bq_stream_t stream) {
  const char* what = "bq_gemv_w8a32";
  if (M < 0 || N < 0 || K < 0) return set_error(BQ_ERR_ARG, "%s: negative size", what);
  if (M == 0 || N == 0) return BQ_OK;
  if (M > WA_MMAX) return set_error(BQ_ERR_UNSUPPORTED, "%s: M=%lld > %d (dequantize and use an f32 GEMM)", what, (long long)M, WA_MMAX);
  if (K % 16 || K > 8192) return set_error(BQ_ERR_UNSUPPORTED, "%s: K=%lld (needs K %% 16 == 0 and K <= 8192)", what, (long long)K);
  if (N > 0x7fffffff || (int64_t)N * K >= ((int64_t)1 << 31)) return set_error(BQ_ERR_ARG, "%s: size too large", what);
  if (!x || !W || !sW || !out) return set_error(BQ_ERR_ARG, "%s: null pointer", what);
  if (((uintptr_t)x & 15) || ((uintptr_t)W & 15)) return set_error(BQ_ERR_ARG, "%s: x and W must be 16-byte aligned", what);
  if (act < BQ_ACT_NONE || act > BQ_ACT_GELU) return set_error(BQ_ERR_ARG, "%s: bad activation %d", what, act);
  constexpr int RPW = 2;
  const unsigned grid = (unsigned)((N + WA_WAVES * RPW - 1) / (WA_WAVES * RPW));
  hipStream_t st = (hipStream_t)stream;
  const int m = (int)M, n = (int)N, k = (int)K;
  if (M >= WA_MFMA_MIN_M) {
    const unsigned g2 = (unsigned)((N + WM_ROWS - 1) / WM_ROWS);
    if (K <= 2048) gemv_w8a32_mfma_kernel<4><<<g2, WA_WAVES * 64, 0, st>>>(x, W, m, n, k, sW, bias, act, out);
    else if (K <= 4096) gemv_w8a32_mfma_kernel<8><<<g2, WA_WAVES * 64, 0, st>>>(x, W, m, n, k, sW, bias, act, out);
    else gemv_w8a32_mfma_kernel<16><<<g2, WA_WAVES * 64, 0, st>>>(x, W, m, n, k, sW, bias, act, out);
    return check_launch(what);
  }
  const int64_t kc = K <= 1024 ? 1 : K <= 2048 ? 2 : K <= 4096 ? 4 : 8;  // the kernel's KC
  if (M * kc * 1024 <= WA_XLDS) {
    if (K <= 1024) (M == 1 ? gemv_w8a32_kernel<1, RPW, true, WA_XLDS, true> : gemv_w8a32_kernel<1, RPW, true>)<<<grid, WA_WAVES * 64, 0, st>>>(x, W, m, n, k, sW, bias, act, out);
    else if (K <= 2048) (M == 1 ? gemv_w8a32_kernel<2, RPW, true, WA_XLDS, true> : gemv_w8a32_kernel<2, RPW, true>)<<<grid, WA_WAVES * 64, 0, st>>>(x, W, m, n, k, sW, bias, act, out);
    else if (K <= 4096) (M == 1 ? gemv_w8a32_kernel<4, RPW, true, WA_XLDS, true> : gemv_w8a32_kernel<4, RPW, true>)<<<grid, WA_WAVES * 64, 0, st>>>(x, W, m, n, k, sW, bias, act, out);
    else (M == 1 ? gemv_w8a32_kernel<8, RPW, true, WA_XLDS, true> : gemv_w8a32_kernel<8, RPW, true>)<<<grid, WA_WAVES * 64, 0, st>>>(x, W, m, n, k, sW, bias, act, out);
  } else if (M * kc * 1024 <= WA_XLDS_BIG) {
    constexpr int B = WA_XLDS_BIG;
    if (K <= 1024) gemv_w8a32_kernel<1, RPW, true, B><<<grid, WA_WAVES * 64, 0, st>>>(x, W, m, n, k, sW, bias, act, out);
    else if (K <= 2048) gemv_w8a32_kernel<2, RPW, true, B><<<grid, WA_WAVES * 64, 0, st>>>(x, W, m, n, k, sW, bias, act, out);
    else if (K <= 4096) gemv_w8a32_kernel<4, RPW, true, B><<<grid, WA_WAVES * 64, 0, st>>>(x, W, m, n, k, sW, bias, act, out);
    else gemv_w8a32_kernel<8, RPW, true, B><<<grid, WA_WAVES * 64, 0, st>>>(x, W, m, n, k, sW, bias, act, out);
  } else {
    if (K <= 1024) gemv_w8a32_kernel<1, RPW, false><<<grid, WA_WAVES * 64, 0, st>>>(x, W, m, n, k, sW, bias, act, out);
    else if (K <= 2048) gemv_w8a32_kernel<2, RPW, false><<<grid, WA_WAVES * 64, 0, st>>>(x, W, m, n, k, sW, bias, act, out);
    else if (K <= 4096) gemv_w8a32_kernel<4, RPW, false><<<grid, WA_WAVES * 64, 0, st>>>(x, W, m, n, k, sW, bias, act, out);
    else gemv_w8a32_kernel<8, RPW, false><<<grid, WA_WAVES * 64, 0, st>>>(x, W, m, n, k, sW, bias, act, out);
  }
  return check_launch(what);
}

int bq_dequant_i8(const int8_t* q, int64_t N, int64_t K, const float* s, float* w, bq_stream_t stream) {
  const char* what = "bq_dequant_i8";
  if (N < 0 || K < 0) return set_error(BQ_ERR_ARG, "%s: negative size", what);
  if (N == 0 || K == 0) return BQ_OK;
  if (!q || !s || !w) return set_error(BQ_ERR_ARG, "%s: null pointer", what);
  if (((uintptr_t)q & 3) || ((uintptr_t)w & 15)) return set_error(BQ_ERR_ARG, "%s: misaligned pointer", what);
  int64_t blocks = (N * K / 4 + 255) / 256;
  if (blocks > 16384) blocks = 16384;
  if (blocks < 1) blocks = 1;
  dequant_i8_kernel<<<(unsigned)blocks, 256, 0, (hipStream_t)stream>>>(q, N, K, s, w);
  return check_launch(what);
}

}  // extern "C"
