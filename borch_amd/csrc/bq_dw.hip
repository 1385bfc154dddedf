// Depthwise convolution on int8 NHWC activations (EfficientNet's MBConv depthwise layers):
// exact int32 tap sums on v_dot4 / byte multiplies (no MFMA: the f32 output write makes it
// bandwidth-bound), then the dequant epilogue the GEMM kernels share. The reference has no
// int8 depthwise; its f32 depthwiseForward (borch-ts/src/kernels.ts:5932-5975) and the CPU
// dwconv_rows (borch-ts/wasm/src/lib.rs:586-641) compute the same tap sum in f32.
#include "bq_common.h"

namespace bq {

// One thread: CPT (4 or 8) consecutive channels of one output pixel; consecutive threads
// take consecutive channel groups of the same pixel, so each tap load and the output
// store are contiguous across the wave. x NHWC int8, w [KH*KW, C] int8; no MFMA
// (bandwidth-bound: the f32 output write dominates).
template <int CPT>
__global__ __launch_bounds__(256) void dwconv_i8_kernel(const int8_t* __restrict__ x, int Nimg, int H, int Wd,
                                                        int C, const int8_t* __restrict__ w, int KH, int KW,
                                                        int stride, int pad, int OH, int OW,
                                                        const float* __restrict__ sA, const float* __restrict__ sW,
                                                        const float* __restrict__ bias, int act,
                                                        float* __restrict__ out, int32_t* __restrict__ acc) {
  typedef int vw __attribute__((ext_vector_type(CPT / 4)));
  const int CG = C / CPT;
  const int64_t total = (int64_t)Nimg * OH * OW * CG;
  const float sa = sA[0];
  for (int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; g < total; g += (int64_t)gridDim.x * blockDim.x) {
    const int cg = (int)(g % CG);
    const int64_t pix = g / CG;
    const int ow = (int)(pix % OW);
    const int64_t t = pix / OW;
    const int oh = (int)(t % OH);
    const int n = (int)(t / OH);
    const int c = cg * CPT;
    int a[CPT];
#pragma unroll
    for (int j = 0; j < CPT; ++j) a[j] = 0;
    for (int kh = 0; kh < KH; ++kh) {
      const int ih = oh * stride - pad + kh;
      if (ih < 0 || ih >= H) continue;
      const int8_t* xrow = x + (((size_t)n * H + ih) * Wd) * C + c;
      const int8_t* wrow = w + (size_t)(kh * KW) * C + c;
      for (int kw = 0; kw < KW; ++kw) {
        const int iw = ow * stride - pad + kw;
        if (iw < 0 || iw >= Wd) continue;
        const vw xv = *reinterpret_cast<const vw*>(xrow + (size_t)iw * C);
        const vw wv = *reinterpret_cast<const vw*>(wrow + (size_t)kw * C);
#pragma unroll
        for (int q = 0; q < CPT / 4; ++q) {
          const uint32_t xq = (uint32_t)xv[q], wq = (uint32_t)wv[q];
#pragma unroll
          for (int b = 0; b < 4; ++b)
            a[q * 4 + b] += (int)(int8_t)((xq >> (8 * b)) & 0xff) * (int)(int8_t)((wq >> (8 * b)) & 0xff);
        }
      }
    }
    const size_t idx = (size_t)pix * C + c;
#pragma unroll
    for (int q = 0; q < CPT / 4; ++q) {
      float o[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int cc = c + q * 4 + j;
        o[j] = dequant_one(a[q * 4 + j], sa, sW[cc], bias ? bias[cc] : 0.f, bias != nullptr, 0.f, false, act);
      }
      *reinterpret_cast<float4*>(out + idx + q * 4) = make_float4(o[0], o[1], o[2], o[3]);
      if (acc) *reinterpret_cast<int4*>(acc + idx + q * 4) = make_int4(a[q * 4], a[q * 4 + 1], a[q * 4 + 2], a[q * 4 + 3]);
    }
  }
}

// 4x4 byte transpose: t[ch] byte b = byte ch of word b (four NHWC column words of four
// channels into four per-channel words of four columns), eight v_perm_b32.
__device__ __forceinline__ void transpose4x4(uint32_t a, uint32_t b, uint32_t c, uint32_t d, uint32_t (&t)[4]) {
  const uint32_t ab_lo = __builtin_amdgcn_perm(b, a, 0x05010400u);  // a0 b0 a1 b1
  const uint32_t ab_hi = __builtin_amdgcn_perm(b, a, 0x07030602u);  // a2 b2 a3 b3
  const uint32_t cd_lo = __builtin_amdgcn_perm(d, c, 0x05010400u);  // c0 d0 c1 d1
  const uint32_t cd_hi = __builtin_amdgcn_perm(d, c, 0x07030602u);  // c2 d2 c3 d3
  t[0] = __builtin_amdgcn_perm(cd_lo, ab_lo, 0x05040100u);  // a0 b0 c0 d0
  t[1] = __builtin_amdgcn_perm(cd_lo, ab_lo, 0x07060302u);  // a1 b1 c1 d1
  t[2] = __builtin_amdgcn_perm(cd_hi, ab_hi, 0x05040100u);
  t[3] = __builtin_amdgcn_perm(cd_hi, ab_hi, 0x07060302u);
}

// Bytes sh .. sh + 3 of the eight-byte value hi:lo (sh in 0..3, known at compile time).
__device__ __forceinline__ uint32_t window4(uint32_t hi, uint32_t lo, int sh) {
  return sh == 0 ? lo : __builtin_amdgcn_alignbyte(hi, lo, (uint32_t)sh);
}

// Register-blocked depthwise conv for square KS x KS filters at stride S (the shapes of
// EfficientNet-style networks). One thread: OWB consecutive output pixels of one output row
// for CPT = 4 consecutive channels. Each input column the OWB outputs need is loaded once
// (stride 1: NCOL = OWB + KS - 1 columns instead of OWB * KS) and the columns are regrouped
// by byte permutes into per-channel words of four consecutive columns; an output's four
// taps of a filter row are then one byte-aligned window of those words and one v_dot4
// (four int8 products summed into the int32 accumulator, exact). About 90 VALU
// instructions a filter row for a 5x5 filter, against 132 with each byte sign-extended
// and multiplied on its own.
// All index arithmetic is 32-bit (the host checks the ranges). Same arithmetic as
// dwconv_i8_kernel: exact int32 tap sums, then the shared dequant epilogue.
template <int KS, int S, int CPT, int OWB, bool PRE>
__global__ __launch_bounds__(256) void dwconv_blk_kernel(const int8_t* __restrict__ x, int H, int Wd, int C,
                                                         const int8_t* __restrict__ w, int pad, int OH, int OW,
                                                         int rows, const float* __restrict__ sA,
                                                         const float* __restrict__ sW, const float* __restrict__ bias,
                                                         int act, float* __restrict__ out, int32_t* __restrict__ acc) {
  static_assert(CPT == 4 && (KS == 3 || KS == 5), "four channels a thread, 3- or 5-wide filters");
  constexpr int NCOL = (OWB - 1) * S + KS;
  const int CG = C / CPT;
  const int items = ((OW + OWB - 1) / OWB) * CG;
  const int total = rows * items;
  const float sa = sA[0];
  // the output, written through (the host keeps it under 4 GB)
  const __amdgpu_buffer_rsrc_t r_out = make_rsrc(out, (uint32_t)((size_t)rows * OW * C * 4));
  // Consecutive output rows share input rows (KS - S of them): the blocks of a run of rows
  // are regrouped onto one XCD so those rows come from its L2 rather than once per XCD.
  const int lb = xcd_order(blockIdx.x, gridDim.x);
  for (int g = lb * 256 + threadIdx.x; g < total; g += gridDim.x * 256) {
    const int row = g / items;  // n * OH + oh
    const int it = g - row * items;
    const int owb = it / CG;
    const int cg = it - owb * CG;
    const int n = row / OH;
    const int oh = row - n * OH;
    const int c = cg * CPT;
    const int ow0 = owb * OWB;
    const int iw0 = ow0 * S - pad;
    int a[OWB][CPT];
#pragma unroll
    for (int o = 0; o < OWB; ++o)
#pragma unroll
      for (int j = 0; j < CPT; ++j) a[o][j] = 0;
    if constexpr (PRE) {
      // PRE: every filter row's columns and taps are loaded before any is used (rows outside
      // the input read as zeros instead of being skipped), so the KS rows' loads are in
      // flight together rather than one row's round trip after another; more registers
      // (up to 193 VGPRs), which the 5x5 filters on larger maps pay for in occupancy.
      constexpr int NWT = (NCOL + 3) / 4;
      uint32_t colv[KS][NWT * 4], wtv[KS][KS];
  #pragma unroll
      for (int kh = 0; kh < KS; ++kh) {
        const int ih = oh * S - pad + kh;
        const bool rin = (unsigned)ih < (unsigned)H;
        const int8_t* xrow = x + ((size_t)(n * H + (rin ? ih : 0)) * Wd) * C + c;
  #pragma unroll
        for (int kw = 0; kw < KS; ++kw) wtv[kh][kw] = *reinterpret_cast<const uint32_t*>(w + (size_t)(kh * KS + kw) * C + c);
  #pragma unroll
        for (int jj = 0; jj < NWT * 4; ++jj) {
          const int iw = iw0 + jj;
          colv[kh][jj] = (rin && jj < NCOL && (unsigned)iw < (unsigned)Wd)
                             ? *reinterpret_cast<const uint32_t*>(xrow + (size_t)iw * C) : 0u;
        }
      }
  #pragma unroll
      for (int kh = 0; kh < KS; ++kh) {
        uint32_t wa[CPT], wb[CPT];
        transpose4x4(wtv[kh][0], wtv[kh][1], wtv[kh][2], KS > 3 ? wtv[kh][3 % KS] : 0u, wa);
        if constexpr (KS == 5) {
  #pragma unroll
          for (int ch = 0; ch < CPT; ++ch) wb[ch] = (wtv[kh][4 % KS] >> (8 * ch)) & 0xffu;
        }
        uint32_t xs[NWT + 1][CPT];
  #pragma unroll
        for (int t = 0; t < NWT; ++t) transpose4x4(colv[kh][4 * t], colv[kh][4 * t + 1], colv[kh][4 * t + 2], colv[kh][4 * t + 3], xs[t]);
  #pragma unroll
        for (int ch = 0; ch < CPT; ++ch) xs[NWT][ch] = 0u;
  #pragma unroll
        for (int o = 0; o < OWB; ++o) {
          const int p0 = o * S;
  #pragma unroll
          for (int ch = 0; ch < CPT; ++ch) {
            const uint32_t win = window4(xs[p0 / 4 + 1][ch], xs[p0 / 4][ch], p0 % 4);
            a[o][ch] = __builtin_amdgcn_sdot4((int)win, (int)wa[ch], a[o][ch], false);
            if constexpr (KS == 5) {
              const int p1 = p0 + 4;
              const uint32_t win2 = window4(xs[p1 / 4 + 1][ch], xs[p1 / 4][ch], p1 % 4);
              a[o][ch] = __builtin_amdgcn_sdot4((int)win2, (int)wb[ch], a[o][ch], false);
            }
          }
        }
      }
    } else {
  #pragma unroll 1
      for (int kh = 0; kh < KS; ++kh) {
        const int ih = oh * S - pad + kh;
        if ((unsigned)ih >= (unsigned)H) continue;
        const int8_t* xrow = x + ((size_t)(n * H + ih) * Wd) * C + c;
        // The filter row's taps per channel: wa[ch] = taps 0..3 of channel ch (tap 3 zero for a
        // 3-wide filter), wb[ch] = tap 4 in byte 0 (5-wide filters).
        uint32_t wt[4], wa[CPT], wb[CPT];
  #pragma unroll
        for (int kw = 0; kw < 4; ++kw)
          wt[kw] = kw < KS ? *reinterpret_cast<const uint32_t*>(w + (size_t)(kh * KS + kw) * C + c) : 0u;
        transpose4x4(wt[0], wt[1], wt[2], wt[3], wa);
        if constexpr (KS == 5) {
          const uint32_t w4 = *reinterpret_cast<const uint32_t*>(w + (size_t)(kh * KS + 4) * C + c);
  #pragma unroll
          for (int ch = 0; ch < CPT; ++ch) wb[ch] = (w4 >> (8 * ch)) & 0xffu;
        }
        // The NCOL input columns (zero outside the row), regrouped four at a time into
        // per-channel words: xs[t][ch] byte b = column 4 t + b of channel ch.
        constexpr int NWT = (NCOL + 3) / 4;
        uint32_t xs[NWT + 1][CPT];
  #pragma unroll
        for (int t = 0; t < NWT; ++t) {
          uint32_t col[4];
  #pragma unroll
          for (int b = 0; b < 4; ++b) {
            const int jj = 4 * t + b;
            const int iw = iw0 + jj;
            col[b] = (jj < NCOL && (unsigned)iw < (unsigned)Wd) ? *reinterpret_cast<const uint32_t*>(xrow + (size_t)iw * C)
                                                                : 0u;
          }
          transpose4x4(col[0], col[1], col[2], col[3], xs[t]);
        }
  #pragma unroll
        for (int ch = 0; ch < CPT; ++ch) xs[NWT][ch] = 0u;
        // Output o's taps start at column o S: four taps are one byte-aligned word of the
        // channel's column sequence, multiplied and summed by one v_dot4 (exact int32).
  #pragma unroll
        for (int o = 0; o < OWB; ++o) {
          const int p0 = o * S;
  #pragma unroll
          for (int ch = 0; ch < CPT; ++ch) {
            const uint32_t win = window4(xs[p0 / 4 + 1][ch], xs[p0 / 4][ch], p0 % 4);
            a[o][ch] = __builtin_amdgcn_sdot4((int)win, (int)wa[ch], a[o][ch], false);
            if constexpr (KS == 5) {
              const int p1 = p0 + 4;
              const uint32_t win2 = window4(xs[p1 / 4 + 1][ch], xs[p1 / 4][ch], p1 % 4);
              a[o][ch] = __builtin_amdgcn_sdot4((int)win2, (int)wb[ch], a[o][ch], false);
            }
          }
        }
      }
    }
    float swv[CPT], bv[CPT];
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
      swv[j] = sW[c + j];
      bv[j] = bias ? bias[c + j] : 0.f;
    }
#pragma unroll
    for (int o = 0; o < OWB; ++o) {
      if (ow0 + o >= OW) break;
      const size_t idx = ((size_t)row * OW + ow0 + o) * C + c;
#pragma unroll
      for (int q = 0; q < CPT / 4; ++q) {
        float v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          v[j] = dequant_one(a[o][q * 4 + j], sa, swv[q * 4 + j], bv[q * 4 + j], bias != nullptr, 0.f, false, act);
        store_wt16(r_out, (uint32_t)(idx + q * 4) * 4u, make_float4(v[0], v[1], v[2], v[3]));
        if (acc)
          *reinterpret_cast<int4*>(acc + idx + q * 4) =
              make_int4(a[o][q * 4], a[o][q * 4 + 1], a[o][q * 4 + 2], a[o][q * 4 + 3]);
      }
    }
  }
}

}  // namespace bq

using namespace bq;

extern "C" {

int bq_dwconv_i8_nhwc(const int8_t* x, int64_t N, int64_t H, int64_t W, int64_t C, const int8_t* w, int64_t KH,
                      int64_t KW, int64_t stride, int64_t pad, const float* sA, const float* sW, const float* bias,
                      int act, float* out, int32_t* acc, bq_stream_t stream) {
  const char* what = "bq_dwconv_i8_nhwc";
  if (N < 0 || H < 1 || W < 1 || C < 1 || KH < 1 || KW < 1 || stride < 1 || pad < 0)
    return set_error(BQ_ERR_ARG, "%s: bad geometry", what);
  if (C % 4) return set_error(BQ_ERR_UNSUPPORTED, "%s: C=%lld is not a multiple of 4", what, (long long)C);
  const int64_t OH = (H + 2 * pad - KH) / stride + 1;
  const int64_t OW = (W + 2 * pad - KW) / stride + 1;
  if (H + 2 * pad < KH || W + 2 * pad < KW || OH < 1 || OW < 1)
    return set_error(BQ_ERR_ARG, "%s: the filter is larger than the input.", what);
  if (N * H * W * C > ((int64_t)1 << 40) || H > 0x7fffffff || W > 0x7fffffff || C > 0x7fffffff)
    return set_error(BQ_ERR_ARG, "%s: size too large", what);
  if (N == 0) return BQ_OK;
  if (!x || !w || !sA || !sW || !out) return set_error(BQ_ERR_ARG, "%s: null pointer", what);
  if (((uintptr_t)x & 3) || ((uintptr_t)w & 3) || ((uintptr_t)out & 15) || ((uintptr_t)acc & 15))
    return set_error(BQ_ERR_ARG, "%s: misaligned pointer", what);
  if (act < BQ_ACT_NONE || act > BQ_ACT_GELU) return set_error(BQ_ERR_ARG, "%s: bad activation %d", what, act);
  const bool wide = (C % 8 == 0) && ((uintptr_t)x & 7) == 0 && ((uintptr_t)w & 7) == 0;
  hipStream_t st = (hipStream_t)stream;
  // Square 3x3 / 5x5 filters at stride 1 or 2: the register-blocked kernel (32-bit indices,
  // its output under 4 GB for the buffer stores).
  if (KH == KW && (KH == 3 || KH == 5) && (stride == 1 || stride == 2) && N * OH * OW * C < ((int64_t)1 << 30)) {
    // 4 channels and 4 output pixels a thread (measured on EfficientNet-B0's layers at b64:
    // 8 channels a thread was 0-20% slower, 1-2 pixels a thread up to 2x slower).
    const int rows = (int)(N * OH);
    const int cpt = 4;
    auto launch = [&](auto kern, int owb) {
      const int64_t items = (OW + owb - 1) / owb * (C / cpt);
      int64_t blocks = (rows * items + 255) / 256;
      if (blocks > 65536) blocks = 65536;
      blocks = (blocks + 7) / 8 * 8;  // a multiple of the 8 XCDs, for the kernel's regrouping
      kern<<<(unsigned)blocks, 256, 0, st>>>(x, (int)H, (int)W, (int)C, w, (int)pad, (int)OH, (int)OW, rows, sA, sW,
                                             bias, act, out, acc);
    };
    // Output rows of 7, 14 or 28 pixels: 7 pixels a thread (no idle slot, and each loaded
    // column serves more outputs), except a 5x5 stride-2 filter onto 7 pixels, whose 17-column
    // window costs more than the idle slot (B0 b64's 16 layers 282.8 -> 267.8 us).
    // Wider rows of a multiple of 7 take 7 pixels a thread too at 3x3 / 1 (B0 b64's 112^2
    // and 56^2 layers: 37.8 -> 33.8 and 52.0 -> 42.8 us, eager with rotated inputs).
    // All filter rows' loads issued first (PRE) for 3x3 filters and for output rows of at
    // most 7 pixels; the 5x5 filters on larger maps keep the row-by-row loop, whose fewer
    // registers they need for occupancy (B0 b64: 267.6 -> ~254 us over the 16 layers), and
    // so do 3x3 / 1 filters on rows wider than 28 (the two layers above: 37.1 and 49.6 us
    // with PRE). A two-row load pipeline between the two was slower than one or the other
    // on every B0 layer (5x5 on 28^2: 27.2 against 21.0 us).
    const bool seven = OW % 7 == 0 && (OW <= 28 || (KH == 3 && stride == 1)) && !(KH == 5 && stride == 2 && OW < 14);
    const bool pre = OW <= 7 || (KH == 3 && !(stride == 1 && OW > 28));
    switch ((int)KH * 10 + (int)stride + (seven ? 100 : 0) + (pre ? 1000 : 0)) {
      case 31: launch(dwconv_blk_kernel<3, 1, 4, 4, false>, 4); break;
      case 131: launch(dwconv_blk_kernel<3, 1, 4, 7, false>, 7); break;
      case 51: launch(dwconv_blk_kernel<5, 1, 4, 4, false>, 4); break;
      case 52: launch(dwconv_blk_kernel<5, 2, 4, 4, false>, 4); break;
      case 151: launch(dwconv_blk_kernel<5, 1, 4, 7, false>, 7); break;
      case 152: launch(dwconv_blk_kernel<5, 2, 4, 7, false>, 7); break;
      case 1031: launch(dwconv_blk_kernel<3, 1, 4, 4, true>, 4); break;
      case 1032: launch(dwconv_blk_kernel<3, 2, 4, 4, true>, 4); break;
      case 1051: launch(dwconv_blk_kernel<5, 1, 4, 4, true>, 4); break;
      case 1052: launch(dwconv_blk_kernel<5, 2, 4, 4, true>, 4); break;
      case 1131: launch(dwconv_blk_kernel<3, 1, 4, 7, true>, 7); break;
      case 1132: launch(dwconv_blk_kernel<3, 2, 4, 7, true>, 7); break;
      default: launch(dwconv_blk_kernel<5, 1, 4, 7, true>, 7); break;  // 1151
    }
    return check_launch(what);
  }
  const int64_t total = N * OH * OW * (C / (wide ? 8 : 4));
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  if (wide)
    dwconv_i8_kernel<8><<<(unsigned)blocks, 256, 0, st>>>(
        x, (int)N, (int)H, (int)W, (int)C, w, (int)KH, (int)KW, (int)stride, (int)pad, (int)OH, (int)OW, sA, sW,
        bias, act, out, acc);
  else
    dwconv_i8_kernel<4><<<(unsigned)blocks, 256, 0, st>>>(
        x, (int)N, (int)H, (int)W, (int)C, w, (int)KH, (int)KW, (int)stride, (int)pad, (int)OH, (int)OW, sA, sW,
        bias, act, out, acc);
  return check_launch(what);
}

}  // extern "C"
