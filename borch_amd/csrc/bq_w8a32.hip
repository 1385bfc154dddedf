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
constexpr int WA_MMAX = 16;  // activation rows the GEMV kernels take (the MFMA one: 5..16)
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
                                                                   const float* __restrict__ bias,
                                                                   const float* __restrict__ res, int act,
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
      w[j][c] = load_nt16(rw, k < K ? (uint32_t)(j * K + k) : W_OOB);
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
          if (res) v = __fadd_rn(v, res[(size_t)m * N + n]);
          out[(size_t)m * N + n] = activate(v, act);
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
          if (res) v = __fadd_rn(v, res[(size_t)m * N + n]);
          out[(size_t)m * N + n] = activate(v, act);
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
typedef float v4f __attribute__((ext_vector_type(4)));
constexpr int WM_ROWS = 16;
template <int CPW>  // 64-byte chunks a wave: K <= CPW * 8 * 64
__global__ __launch_bounds__(WA_WAVES * 64) void gemv_w8a32_mfma_kernel(const float* __restrict__ x, const int8_t* W,
                                                                        int M, int N, int K,
                                                                        const float* __restrict__ sW,
                                                                        const float* __restrict__ bias,
                                                                        const float* __restrict__ res, int act,
                                                                        float* __restrict__ out) {
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
    w[c] = load_nt16(rw, k < K ? (uint32_t)(r * K + k) : W_OOB);
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
      float v = bias ? __fadd_rn(s, bias[n0 + row]) : s;
      if (res) v = __fadd_rn(v, res[(size_t)m * N + n0 + row]);
      out[(size_t)m * N + n0 + row] = activate(v, act);
    }
  }
}

// ------------------------------------------------------------ W8A32 for any M: tiled
//
// w8a32_gemm_kernel: out[m, n] = act(fl(fl(acc[m, n] * s[n]) + bias[n]) + res[m, n]) with
// acc[m, n] = sum_k x[m, k] * q[n, k] accumulated in f32. The bf16 MFMA runs 16 times the
// f32 MFMA rate on this chip, and every product fits it exactly:
//  * q (|q| <= 127: 7 bits) is exact in bf16 (8 significant bits);
//  * x is split into x = x1 + x2 + x3 with x1 the bf16 nearest x and x2 the bf16 nearest
//    x - x1. x - x1 is a multiple of ulp_f32(x) below 2^-8 |x| (at most 16 significant
//    bits), (x - x1) - x2 a multiple of it below 2^-16 |x| (at most 8), so x3 = (x - x1) - x2
//    is exact in bf16 and the split loses nothing (|x| >= 2^-100, so no piece is subnormal).
// Each x * q is then three exact products x_i * q (at most 15 significant bits), which three
// v_mfma_f32_16x16x32_bf16 add into one f32 accumulator: the accumulation is the only
// rounding before the per-channel scale, applied once to the sum. The reference's order
// (the effective weight f32(q) * s rounded per element, then f32 FMAs, kernels.ts:2695-2708)
// and this one are both within the f32-accumulation bound (K + 2) 2^-24 sum |x * w| of the
// exact result on the effective weights.
//
// Tiles: BM x BN outputs a workgroup of WM x WN waves, each wave (BM / WM) x (BN / WN) in
// 16 x 16 MFMA blocks. K goes in stages of 32 (one MFMA's K) through two LDS buffers: the
// next stage's global loads (x as float4, the weight as 16-byte pieces) are issued before
// the current stage's MFMAs and written to the other buffer after them, x as its three bf16
// planes and q as bf16, so the MFMAs read ready operands. LDS rows are 64 bytes (32 bf16)
// with the 16-byte chunk index XORed by bits 2..3 of the row: the 16 lanes that read one
// fragment (16 rows, one chunk) then cover all 64 banks once.

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef float v2f __attribute__((ext_vector_type(2)));

// Byte offset of 16-byte chunk c of LDS row r, rows of CPR chunks (BK bf16): the chunk index
// is XORed with the row bits that make the 16 rows of one fragment read cover all 64 banks.
template <int CPR>
__device__ __forceinline__ int w8_lds_off(int r, int c) {
  if constexpr (CPR == 4) return r * 64 + ((c ^ ((r >> 2) & 3)) << 4);
  else if constexpr (CPR == 8) return r * 128 + ((c ^ ((r >> 1) & 7)) << 4);
  else return r * 256 + ((c ^ (r & 15)) << 4);
}

// Two floats to two bf16 (round to nearest even, v_cvt_pk_bf16_f32), packed low first.
__device__ __forceinline__ uint32_t bf2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((v2f){a, b}, v2bf));
}

// The three bf16 planes of four floats: p1 = bf16(v), p2 = bf16(v - p1), p3 = v - p1 - p2.
__device__ __forceinline__ void split3(float4 v, uint2& p1, uint2& p2, uint2& p3) {
  const uint32_t a = bf2(v.x, v.y), b = bf2(v.z, v.w);
  const float r0 = __fsub_rn(v.x, __uint_as_float(a << 16)), r1 = __fsub_rn(v.y, __uint_as_float(a & 0xffff0000u));
  const float r2 = __fsub_rn(v.z, __uint_as_float(b << 16)), r3 = __fsub_rn(v.w, __uint_as_float(b & 0xffff0000u));
  const uint32_t c = bf2(r0, r1), d = bf2(r2, r3);
  const float t0 = __fsub_rn(r0, __uint_as_float(c << 16)), t1 = __fsub_rn(r1, __uint_as_float(c & 0xffff0000u));
  const float t2 = __fsub_rn(r2, __uint_as_float(d << 16)), t3 = __fsub_rn(r3, __uint_as_float(d & 0xffff0000u));
  p1 = make_uint2(a, b);
  p2 = make_uint2(c, d);
  p3 = make_uint2(bf2(t0, t1), bf2(t2, t3));
}

// Four signed bytes (low first) to four bf16, exactly: f32(q) has at most 7 significant
// bits, so its bf16 is its upper half.
__device__ __forceinline__ uint2 i8x4_bf16(uint32_t w) {
  const float f0 = (float)(int)(int8_t)(w & 0xff), f1 = (float)(int)(int8_t)((w >> 8) & 0xff);
  const float f2 = (float)(int)(int8_t)((w >> 16) & 0xff), f3 = (float)(int)(int8_t)(w >> 24);
  return make_uint2(__builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u),
                    __builtin_amdgcn_perm(__float_as_uint(f3), __float_as_uint(f2), 0x07060302u));
}

struct W8P {
  const float* x;    // [M, K]
  const int8_t* W;   // [N, K]
  int M, N, K;
  const float* sW;   // [N]
  const float* bias; // [N] or null
  const float* res;  // [M, N] or null
  int act;
  float* out;        // [M, N]
};

template <int BM, int BN, int WM, int WN, int BK>
__global__ __launch_bounds__(WM * WN * 64) void w8a32_gemm_kernel(W8P p) {
  static_assert(BK == 32 || BK == 64 || BK == 128, "K per stage");
  constexpr int CPR = BK / 8;  // 16-byte chunks of an LDS row (BK bf16)
  constexpr int T = WM * WN * 64;
  constexpr int WTM = BM / WM, WTN = BN / WN;  // wave tile
  constexpr int FM = WTM / 16, FN = WTN / 16;  // MFMA blocks a wave
  static_assert(FM >= 1 && FN >= 1 && WTM % 16 == 0 && WTN % 16 == 0, "wave tile of whole 16x16 blocks");
  constexpr int PLANE = BM * BK * 2;            // bytes of one bf16 plane of the x stage
  constexpr int STAGE = 3 * PLANE + BN * BK * 2;  // x planes, then the weight
  constexpr int NA = BM * (BK / 4);             // float4s of x a stage
  constexpr int NW = BN * (BK / 16);            // 16-byte weight pieces a stage
  constexpr int RA = (NA + T - 1) / T, RW = (NW + T - 1) / T;
  __shared__ __attribute__((aligned(16))) unsigned char lds[2 * STAGE];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int tiles_m = (p.M + BM - 1) / BM, tiles_n = (p.N + BN - 1) / BN;
  int bm, bn;
  tile_of(xcd_order(blockIdx.x, gridDim.x), tiles_m, tiles_n, bm, bn);
  const int m0 = bm * BM, n0 = bn * BN;
  const int K = p.K;
  const __amdgpu_buffer_rsrc_t rx = w_rsrc(p.x, (uint32_t)((size_t)p.M * K * 4));
  const __amdgpu_buffer_rsrc_t rw = w_rsrc(p.W, (uint32_t)((size_t)p.N * K));

  float4 xa[RA];
  v4i wq[RW];
  auto load = [&](int kt) {
    const int k0 = kt * BK;
#pragma unroll
    for (int r = 0; r < RA; ++r) {
      const int i = tid + r * T;
      const int row = i / (BK / 4), k = k0 + (i % (BK / 4)) * 4;
      const bool ok = (NA % T == 0 || i < NA) && m0 + row < p.M && k < K;
      xa[r] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
                                             rx, ok ? (uint32_t)(((m0 + row) * K + k) * 4) : W_OOB, 0, 0));
    }
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      const int i = tid + r * T;
      const int row = i / (BK / 16), k = k0 + (i % (BK / 16)) * 16;
      const bool ok = (NW % T == 0 || i < NW) && n0 + row < p.N && k < K;
      wq[r] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(
                                         rw, ok ? (uint32_t)((n0 + row) * K + k) : W_OOB, 0, 0));
    }
  };
  auto store = [&](int buf) {
    unsigned char* st = lds + buf * STAGE;
#pragma unroll
    for (int r = 0; r < RA; ++r) {
      const int i = tid + r * T;
      if (NA % T == 0 || i < NA) {
        const int row = i / (BK / 4), c4 = i % (BK / 4);  // floats 4 c4 .. 4 c4 + 3: chunk c4 / 2, half c4 % 2
        const int off = w8_lds_off<CPR>(row, c4 >> 1) + (c4 & 1) * 8;
        uint2 p1, p2, p3;
        split3(xa[r], p1, p2, p3);
        *reinterpret_cast<uint2*>(st + off) = p1;
        *reinterpret_cast<uint2*>(st + PLANE + off) = p2;
        *reinterpret_cast<uint2*>(st + 2 * PLANE + off) = p3;
      }
    }
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      const int i = tid + r * T;
      if (NW % T == 0 || i < NW) {
        const int row = i / (BK / 16), c0 = (i % (BK / 16)) * 2;  // 16 weights: chunks c0, c0 + 1
        const uint2 a = i8x4_bf16((uint32_t)wq[r][0]), b = i8x4_bf16((uint32_t)wq[r][1]);
        const uint2 c = i8x4_bf16((uint32_t)wq[r][2]), d = i8x4_bf16((uint32_t)wq[r][3]);
        *reinterpret_cast<uint4*>(st + 3 * PLANE + w8_lds_off<CPR>(row, c0)) = make_uint4(a.x, a.y, b.x, b.y);
        *reinterpret_cast<uint4*>(st + 3 * PLANE + w8_lds_off<CPR>(row, c0 + 1)) = make_uint4(c.x, c.y, d.x, d.y);
      }
    }
  };

  v4f acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = (v4f){0.f, 0.f, 0.f, 0.f};

  const int KT = (K + BK - 1) / BK;
  const int fr = lane & 15, fc = lane >> 4;  // a fragment lane's row in its block, and its 16-byte chunk
  load(0);
  store(0);
  for (int kt = 0; kt < KT; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < KT) load(kt + 1);
    __syncthreads();
    const unsigned char* st = lds + buf * STAGE;
#pragma unroll
    for (int ks = 0; ks < BK / 32; ++ks) {  // one MFMA K (32) at a time: chunks 4 ks .. 4 ks + 3
      const int ch = ks * 4 + fc;
      v8bf b[FN];
#pragma unroll
      for (int j = 0; j < FN; ++j)
        b[j] = *reinterpret_cast<const v8bf*>(st + 3 * PLANE + w8_lds_off<CPR>(wn * WTN + j * 16 + fr, ch));
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int off = w8_lds_off<CPR>(wm * WTM + i * 16 + fr, ch);
        const v8bf a1 = *reinterpret_cast<const v8bf*>(st + off);
        const v8bf a2 = *reinterpret_cast<const v8bf*>(st + PLANE + off);
        const v8bf a3 = *reinterpret_cast<const v8bf*>(st + 2 * PLANE + off);
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a3, b[j], acc[i][j], 0, 0, 0);
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2, b[j], acc[i][j], 0, 0, 0);
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b[j], acc[i][j], 0, 0, 0);
        }
      }
    }
    if (kt + 1 < KT) store(buf ^ 1);
  }

  // Epilogue: block (i, j) register r of lane l is row 4 (l / 16) + r, column l % 16.
  float sc[FN], bi[FN];
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int n = n0 + wn * WTN + j * 16 + fr;
    sc[j] = n < p.N ? p.sW[n] : 0.f;
    bi[j] = (p.bias && n < p.N) ? p.bias[n] : 0.f;
  }
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = m0 + wm * WTM + i * 16 + fc * 4 + r;
      if (m >= p.M) continue;
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int n = n0 + wn * WTN + j * 16 + fr;
        if (n >= p.N) continue;
        float v = __fmul_rn(acc[i][j][r], sc[j]);
        if (p.bias) v = __fadd_rn(v, bi[j]);
        if (p.res) v = __fadd_rn(v, p.res[(size_t)m * p.N + n]);
        p.out[(size_t)m * p.N + n] = activate(v, p.act);
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

// The GEMV kernels (M <= 16, K <= 8192): the per-wave kernel below WA_MFMA_MIN_M rows, the
// f32-MFMA one from there (its 16 MFMA columns hold up to 16 activation rows).
static void launch_gemv_w8a32(const float* x, const int8_t* W, int m, int n, int k, const float* sW,
                              const float* bias, const float* res, int act, float* out, hipStream_t st) {
  constexpr int RPW = 2;
  const unsigned grid = (unsigned)((n + WA_WAVES * RPW - 1) / (WA_WAVES * RPW));
  const int64_t M = m, K = k;
  if (m >= WA_MFMA_MIN_M) {
    const unsigned g2 = (unsigned)((n + WM_ROWS - 1) / WM_ROWS);
    if (K <= 2048) gemv_w8a32_mfma_kernel<4><<<g2, WA_WAVES * 64, 0, st>>>(x, W, m, n, k, sW, bias, res, act, out);
    else if (K <= 4096) gemv_w8a32_mfma_kernel<8><<<g2, WA_WAVES * 64, 0, st>>>(x, W, m, n, k, sW, bias, res, act, out);
    else gemv_w8a32_mfma_kernel<16><<<g2, WA_WAVES * 64, 0, st>>>(x, W, m, n, k, sW, bias, res, act, out);
    return;
  }
  const int64_t kc = K <= 1024 ? 1 : K <= 2048 ? 2 : K <= 4096 ? 4 : 8;  // the kernel's KC
  if (M * kc * 1024 <= WA_XLDS) {
    if (K <= 1024) (m == 1 ? gemv_w8a32_kernel<1, RPW, true, WA_XLDS, true> : gemv_w8a32_kernel<1, RPW, true>)<<<grid, WA_WAVES * 64, 0, st>>>(x, W, m, n, k, sW, bias, res, act, out);
    else if (K <= 2048) (m == 1 ? gemv_w8a32_kernel<2, RPW, true, WA_XLDS, true> : gemv_w8a32_kernel<2, RPW, true>)<<<grid, WA_WAVES * 64, 0, st>>>(x, W, m, n, k, sW, bias, res, act, out);
    else if (K <= 4096) (m == 1 ? gemv_w8a32_kernel<4, RPW, true, WA_XLDS, true> : gemv_w8a32_kernel<4, RPW, true>)<<<grid, WA_WAVES * 64, 0, st>>>(x, W, m, n, k, sW, bias, res, act, out);
    else (m == 1 ? gemv_w8a32_kernel<8, RPW, true, WA_XLDS, true> : gemv_w8a32_kernel<8, RPW, true>)<<<grid, WA_WAVES * 64, 0, st>>>(x, W, m, n, k, sW, bias, res, act, out);
  } else if (M * kc * 1024 <= WA_XLDS_BIG) {
    constexpr int B = WA_XLDS_BIG;
    if (K <= 1024) gemv_w8a32_kernel<1, RPW, true, B><<<grid, WA_WAVES * 64, 0, st>>>(x, W, m, n, k, sW, bias, res, act, out);
    else if (K <= 2048) gemv_w8a32_kernel<2, RPW, true, B><<<grid, WA_WAVES * 64, 0, st>>>(x, W, m, n, k, sW, bias, res, act, out);
    else if (K <= 4096) gemv_w8a32_kernel<4, RPW, true, B><<<grid, WA_WAVES * 64, 0, st>>>(x, W, m, n, k, sW, bias, res, act, out);
    else gemv_w8a32_kernel<8, RPW, true, B><<<grid, WA_WAVES * 64, 0, st>>>(x, W, m, n, k, sW, bias, res, act, out);
  } else {
    if (K <= 1024) gemv_w8a32_kernel<1, RPW, false><<<grid, WA_WAVES * 64, 0, st>>>(x, W, m, n, k, sW, bias, res, act, out);
    else if (K <= 2048) gemv_w8a32_kernel<2, RPW, false><<<grid, WA_WAVES * 64, 0, st>>>(x, W, m, n, k, sW, bias, res, act, out);
    else if (K <= 4096) gemv_w8a32_kernel<4, RPW, false><<<grid, WA_WAVES * 64, 0, st>>>(x, W, m, n, k, sW, bias, res, act, out);
    else gemv_w8a32_kernel<8, RPW, false><<<grid, WA_WAVES * 64, 0, st>>>(x, W, m, n, k, sW, bias, res, act, out);
  }
}

template <int BM, int BN, int WM, int WN, int BK>
static void launch_w8a32_tiled(const W8P& p, hipStream_t st) {
  const unsigned tiles = (unsigned)(((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN));
  w8a32_gemm_kernel<BM, BN, WM, WN, BK><<<tiles, WM * WN * 64, 0, st>>>(p);
}

static int w8a32_common(const char* what, const float* x, const int8_t* W, int64_t M, int64_t N, int64_t K,
                        const float* sW, const float* bias, const float* res, int act, float* out, int max_m,
                        bq_stream_t stream) {
  if (M < 0 || N < 0 || K < 0) return set_error(BQ_ERR_ARG, "%s: negative size", what);
  if (M == 0 || N == 0) return BQ_OK;
  if (M > max_m)
    return set_error(BQ_ERR_UNSUPPORTED, "%s: M=%lld > %d (bq_linear_w8a32 takes any M)", what, (long long)M, max_m);
  if (K % 16) return set_error(BQ_ERR_UNSUPPORTED, "%s: K=%lld is not a multiple of 16", what, (long long)K);
  if (M > 0x7fffffff || N > 0x7fffffff || M * K * 4 >= ((int64_t)1 << 31) || N * K >= ((int64_t)1 << 31) ||
      M * N >= ((int64_t)1 << 40))
    return set_error(BQ_ERR_ARG, "%s: size too large (x and W must each be < 2 GiB)", what);
  if (!x || !W || !sW || !out) return set_error(BQ_ERR_ARG, "%s: null pointer", what);
  if (((uintptr_t)x & 15) || ((uintptr_t)W & 15)) return set_error(BQ_ERR_ARG, "%s: x and W must be 16-byte aligned", what);
  if (act < BQ_ACT_NONE || act > BQ_ACT_GELU) return set_error(BQ_ERR_ARG, "%s: bad activation %d", what, act);
  hipStream_t st = (hipStream_t)stream;
  if (M <= WA_MMAX && K <= 8192) {
    launch_gemv_w8a32(x, W, (int)M, (int)N, (int)K, sW, bias, res, act, out, st);
    return check_launch(what);
  }
  W8P p{x, W, (int)M, (int)N, (int)K, sW, bias, res, act, out};
  // Measured (4096 x 4096 weight; M = 17 .. 256 and 1024, 4096, ViT-B's 6304-row shapes):
  // skinny 32 x 64 tiles with 128-deep K stages while M <= 256 (37-53 us, against 57-128
  // with 32-deep stages: fewer stage round trips), 128 x 128 tiles once they give a
  // workgroup per CU (4096^3: 384 us), 64 x 64 with 64-deep stages between.
  const int64_t t128 = ((M + 127) / 128) * ((N + 127) / 128);
  const int pick = M <= 256 ? 2 : t128 >= 256 ? 1 : 3;
  switch (pick) {
    case 1: launch_w8a32_tiled<128, 128, 2, 2, 32>(p, st); break;
    case 2: launch_w8a32_tiled<32, 64, 1, 4, 128>(p, st); break;
    default: launch_w8a32_tiled<64, 64, 2, 2, 64>(p, st); break;
  }
  return check_launch(what);
}

}  // namespace bq

using namespace bq;

extern "C" {

int bq_gemv_w8a32(const float* x, const int8_t* W, int64_t M, int64_t N, int64_t K, const float* sW,
                  const float* bias, int act, float* out, bq_stream_t stream) {
  if (K > 8192) return set_error(BQ_ERR_UNSUPPORTED, "bq_gemv_w8a32: K=%lld > 8192", (long long)K);
  return w8a32_common("bq_gemv_w8a32", x, W, M, N, K, sW, bias, nullptr, act, out, WA_MMAX, stream);
}

int bq_linear_w8a32(const float* x, const int8_t* W, int64_t M, int64_t N, int64_t K, const float* sW,
                    const float* bias, const float* residual, int act, float* out, bq_stream_t stream) {
  return w8a32_common("bq_linear_w8a32", x, W, M, N, K, sW, bias, residual, act, out, 0x7fffffff, stream);
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
