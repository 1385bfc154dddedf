// Shared helpers of the int8 inference library (libbq): error state, vector types and
// the exact rounding rule every quantizer uses.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/bq.h"

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

namespace bq {

// Records the message for bq_last_error() and returns `code`.
int set_error(int code, const char* fmt, ...);

// Maps the launch status (hipGetLastError) onto the return codes.
int check_launch(const char* what);

// Partial maxima of |x| over n floats into ws (bq_quantize_tensor_ws_bytes(n) bytes): one
// launch; *np receives their count. Defined with the quantizers.
int absmax_parts_ws(const char* what, const float* x, int64_t n, void* ws, size_t ws_bytes, hipStream_t st, int* np);

// Division by a run-time invariant d >= 1 of any n < 2^31 as (umulhi(n, mul) + n) >> shift
// with shift = ceil(log2 d) and mul = floor(2^32 (2^shift - d) / d) + 1 (Granlund and
// Montgomery, "Division by invariant integers using multiplication", PLDI 1994, the
// round-up method; the sum cannot overflow 32 bits for n < 2^31). Three instructions
// instead of a full integer division in per-element or per-stage index arithmetic.
struct FastDiv {
  uint32_t mul;
  int shift;
};
static inline FastDiv fast_div(uint32_t d) {
  int l = 0;
  while ((1ull << l) < d) ++l;
  return FastDiv{(uint32_t)(((1ull << 32) * ((1ull << l) - d)) / d + 1), l};
}
__device__ __forceinline__ int fdiv(int n, uint32_t mul, int shift) {
  return (int)((__umulhi((uint32_t)n, mul) + (uint32_t)n) >> shift);
}

// Workgroup -> output tile. Workgroups are dispatched round-robin over the 8 XCDs (each
// with its own L2), so workgroup id is first regrouped by XCD (xcd_order: consecutive
// regrouped ids run on one XCD; the K splits of a tile are consecutive), then tiles are handed out
// in bands of 8 tile columns walking down M: the 32 workgroups of one XCD at a 4096^2
// problem cover a 4 x 8 block of tiles, and each K step's A and W slabs are fetched into
// that XCD's L2 once and then shared. Any grid size: with G = 8 q + r, XCD x runs q + 1
// workgroups if x < r, else q, and takes the regrouped ids from x q + min(x, r) on (a
// grid of 300 128 x 128 tiles fetched 3.4x its operands from HBM with ids left in
// dispatch order).
__device__ __forceinline__ int xcd_order(int id, int G) {
  constexpr int XCDS = 8;
  const int q = G / XCDS, r = G % XCDS, x = id % XCDS;
  return x * q + min(x, r) + id / XCDS;
}
__device__ __forceinline__ void tile_of(int id, int tiles_m, int tiles_n, int& bm, int& bn) {
  constexpr int GROUP = 8;
  const int per_group = GROUP * tiles_m;
  const int g = id / per_group;
  const int first_n = g * GROUP;
  const int gsize = min(tiles_n - first_n, GROUP);
  const int in = id - g * per_group;
  bm = in / gsize;
  bn = first_n + in % gsize;
}

// Wave64 max of a non-negative float; every lane of the wave must be active (each caller
// reaches it with the whole workgroup, before a barrier or a per-wave store). Within each
// row of 16 lanes by DPP (quad_perm [1,0,3,2], [2,3,0,1], row_half_mirror, row_mirror),
// then the four row maxima read out of lanes 0, 16, 32, 48: no LDS round trips.
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, false)));
  const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return fmaxf(fmaxf(a, b), fmaxf(c, d));
}

// Wave64 sum in a fixed order (deterministic), every lane active: the same DPP butterfly
// within rows of 16 (each lane of a row ends with the row's sum), then
// (row0 + row1) + (row2 + row3) from lanes 0, 16, 32, 48.
__device__ __forceinline__ float wave_sum_fixed(float v) {
  v = __fadd_rn(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false)));
  v = __fadd_rn(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, false)));
  v = __fadd_rn(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, false)));
  v = __fadd_rn(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, false)));
  const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return __fadd_rn(__fadd_rn(a, b), __fadd_rn(c, d));
}

// The scale rule: float32(peak / 127), correctly rounded (HIP's f32 division is the IEEE
// correctly rounded one; __fdiv_rn makes that explicit).
__device__ __forceinline__ float scale_of(float peak) { return __fdiv_rn(peak, 127.0f); }

// q = clip(rint(v / s), -127, 127) of the EXACT quotient, half to even; s == 0 gives 0.
// f = fl32(v / s) is the correctly rounded quotient. Rounding is monotonic and k + 0.5 is
// representable for |k| <= 127, so rint(f) equals rint(v / s) unless f lands exactly on
// k + 0.5 while v / s does not; then the sign of the exact remainder v - (k + 0.5)·s, which
// one fma rounds without changing its sign, picks k or k + 1. (|v / s| <= 127.00001 since
// s >= max|v| / 127 · (1 - 2^-24).)
__device__ __forceinline__ int quant_one(float v, float s) {
  if (s == 0.f) return 0;
  const float f = __fdiv_rn(v, s);
  float r = rintf(f);
  const float fl = floorf(f);
  if (f - fl == 0.5f) {
    const float d = __fmaf_rn(-f, s, v);
    if (d > 0.f) r = fl + 1.f;
    else if (d < 0.f) r = fl;
  }
  r = fminf(fmaxf(r, -127.f), 127.f);
  return (int)r;
}

__device__ __forceinline__ uint32_t pack4(int a, int b, int c, int d) {
  return (uint32_t)(a & 0xff) | ((uint32_t)(b & 0xff) << 8) | ((uint32_t)(c & 0xff) << 16) |
         ((uint32_t)(d & 0xff) << 24);
}

// The same rounding without a division per element. One quantizer per scale s holds
// r = 1/s (correctly rounded). f = fl(v * r) is within |v/s| * 1.2e-7 of the exact quotient
// t = v/s (two roundings of 2^-24 each), i.e. within 1.6e-5 for |t| <= 127.00002 (s is at
// least max|v| / 127 * (1 - 2^-24)). So rint(f) = rint(t) unless f lies within 4e-5 of a
// half-integer b; there the sign of the exact remainder v - b*s (one fma: its rounding
// keeps the sign and the zero) picks the side, and an exact tie goes to even. A
// non-finite f (a subnormal s whose reciprocal overflows, or a non-finite v) takes
// quant_one. Beyond the clamp (|t| > 127.5, possible with a calibrated scale) both
// roundings clamp to the same +-127.
struct Quantizer {
  float s, r;
  __device__ Quantizer() : s(0.f), r(0.f) {}  // the zero scale: every value to 0
  __device__ explicit Quantizer(float s_) : s(s_), r(s_ == 0.f ? 0.f : __fdiv_rn(1.0f, s_)) {}
  static __device__ __forceinline__ bool near_half(float f, float k) {
    return !(fabsf(__fsub_rn(f, k)) < 0.49996f);
  }
  // The rounding of v when f = v * r lies near a half-integer (or is not finite).
  __device__ float settle(float v, float f, float k) const {
    if (!__builtin_isfinite(f)) return (float)quant_one(v, s);
    const float b = __fadd_rn(k, __builtin_copysignf(0.5f, __fsub_rn(f, k)));  // the half-integer f is near
    const float d = __fmaf_rn(-b, s, v);
    const float lo = __fsub_rn(b, 0.5f);
    return d > 0.f ? __fadd_rn(b, 0.5f) : d < 0.f ? lo : ((((int)lo) & 1) ? __fadd_rn(lo, 1.0f) : lo);
  }
  static __device__ __forceinline__ int clamp127(float k) { return (int)fminf(fmaxf(k, -127.f), 127.f); }
  __device__ __forceinline__ int operator()(float v) const {
    if (s == 0.f) return 0;
    const float f = __fmul_rn(v, r);
    float k = rintf(f);
    if (near_half(f, k)) k = settle(v, f, k);
    return clamp127(k);
  }
  // Four values, packed low byte first: the same rounding with one branch for the four
  // (the near-half case is rare: about 8e-5 of uniformly spread quotients).
  __device__ __forceinline__ uint32_t pack(float4 v) const {
    if (s == 0.f) return 0u;
    const float f0 = __fmul_rn(v.x, r), f1 = __fmul_rn(v.y, r), f2 = __fmul_rn(v.z, r), f3 = __fmul_rn(v.w, r);
    float k0 = rintf(f0), k1 = rintf(f1), k2 = rintf(f2), k3 = rintf(f3);
    if ((int)near_half(f0, k0) | (int)near_half(f1, k1) | (int)near_half(f2, k2) | (int)near_half(f3, k3)) {
      if (near_half(f0, k0)) k0 = settle(v.x, f0, k0);
      if (near_half(f1, k1)) k1 = settle(v.y, f1, k1);
      if (near_half(f2, k2)) k2 = settle(v.z, f2, k2);
      if (near_half(f3, k3)) k3 = settle(v.w, f3, k3);
    }
    return pack4(clamp127(k0), clamp127(k1), clamp127(k2), clamp127(k3));
  }
};

// SiLU v * sigmoid(v) = v / (1 + e^-v) from the hardware exp2 and reciprocal (v_exp_f32,
// v_rcp_f32, about 1 ulp each): five instructions instead of a full-precision expf and an
// IEEE division (about 25), a few ulp from the exact value, within the 1e-5 relative /
// 1e-6 absolute tolerance SiLU outputs are held to. Very negative v: e^-v overflows to inf
// and the result is -0.0 (the exact value is below 1e-30 in magnitude).
__device__ __forceinline__ float silu(float v) {
  const float e = __builtin_amdgcn_exp2f(__fmul_rn(v, -1.4426950408889634f));
  return __fmul_rn(v, __builtin_amdgcn_rcpf(__fadd_rn(1.0f, e)));
}

// erfc(z) for z >= 0 by the Chebyshev fit of Numerical Recipes (Press et al., 2nd ed.,
// section 6.2, "erfcc"): erfc(z) = t exp(-z^2 + P(t)), t = 1 / (1 + z/2), P of degree 9;
// fractional error below 1.2e-7 everywhere, so the small erfc of a GELU's negative tail is
// as accurate as the rest. One reciprocal, nine FMAs and one exp2 (the hardware v_rcp_f32 /
// v_exp_f32): the erf of the math library took about 40 instructions an element.
__device__ __forceinline__ float erfc_nonneg(float z) {
  const float t = __builtin_amdgcn_rcpf(__fmaf_rn(0.5f, z, 1.0f));
  float p = __fmaf_rn(t, 0.17087277f, -0.82215223f);
  p = __fmaf_rn(t, p, 1.48851587f);
  p = __fmaf_rn(t, p, -1.13520398f);
  p = __fmaf_rn(t, p, 0.27886807f);
  p = __fmaf_rn(t, p, -0.18628806f);
  p = __fmaf_rn(t, p, 0.09678418f);
  p = __fmaf_rn(t, p, 0.37409196f);
  p = __fmaf_rn(t, p, 1.00002368f);
  p = __fmaf_rn(t, p, -1.26551223f);
  const float y = __fmaf_rn(-z, z, p);
  return __fmul_rn(t, __builtin_amdgcn_exp2f(__fmul_rn(y, 1.4426950408889634f)));
}

// GELU, erf form: v/2 (1 + erf(v / sqrt 2)) = v/2 erfc(-v / sqrt 2), with erfc(-u) = 2 - erfc(u)
// for u > 0. Within 3% of the 1e-5 relative / 1e-6 absolute tolerance GELU outputs are held
// to (checked on the CPU over [-12, 12] against math.erf; the tests hold it on the device).
// Out of line in the GEMM epilogue: inlined at every epilogue store it grew the GEMM kernels
// and slowed layers that never use it; only GELU layers pay for the call.
__device__ __forceinline__ float gelu_inline(float v) {
  const float c = erfc_nonneg(__fmul_rn(fabsf(v), 0.70710678118654752f));
  return __fmul_rn(__fmul_rn(v, 0.5f), v <= 0.f ? c : __fsub_rn(2.0f, c));
}

__device__ __attribute__((noinline)) float gelu(float v) { return gelu_inline(v); }

__device__ __attribute__((noinline)) float4 gelu4(float4 v) {
  return make_float4(gelu(v.x), gelu(v.y), gelu(v.z), gelu(v.w));
}

// act (uniform across the launch) applied to four values; BQ_ACT_NONE leaves them.
__device__ __forceinline__ float4 activate4_inline(float4 v, int act) {
  if (act == BQ_ACT_GELU) return make_float4(gelu_inline(v.x), gelu_inline(v.y), gelu_inline(v.z), gelu_inline(v.w));
  if (act == BQ_ACT_SILU) return make_float4(silu(v.x), silu(v.y), silu(v.z), silu(v.w));
  if (act == BQ_ACT_RELU)
    return make_float4(v.x > 0.f ? v.x : 0.f, v.y > 0.f ? v.y : 0.f, v.z > 0.f ? v.z : 0.f, v.w > 0.f ? v.w : 0.f);
  return v;
}

__device__ __forceinline__ float activate(float v, int act) {
  if (act == BQ_ACT_RELU) return v > 0.f ? v : 0.f;
  if (act == BQ_ACT_SILU) return silu(v);
  if (act == BQ_ACT_GELU) return gelu(v);
  return v;
}

// The f32 epilogue, one rounding per operation (no contraction into FMA):
// y = ((f32(acc) * sa) * sw) + b, then + residual, then the activation.
__device__ __forceinline__ float dequant_one(int acc, float sa, float sw, float b, bool has_b,
                                             float r, bool has_r, int act) {
  float v = __fmul_rn(__fmul_rn((float)acc, sa), sw);
  if (has_b) v = __fadd_rn(v, b);
  if (has_r) v = __fadd_rn(v, r);
  return activate(v, act);
}

// Raw (stride 0) buffer resource over `bytes` bytes from `base`: a load at or past `bytes`
// returns zeros and a store there is dropped.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// Stores at byte offset `off` of a buffer resource that write through the XCD's L2 to
// memory (cache policy sc1): a large output then leaves no dirty lines for the L2
// write-back at the kernel's end. The whole offset is in the VGPR (SGPR offset 0): with part
// of it in the SGPR offset, 16-byte stores wrote wrong values to a few rows when the next
// instruction reloaded their data registers.
constexpr int CPOL_WT = 16;  // sc1
// Loads of a stream read once (a decode kernel's weights): the non-temporal hint (nt). On
// the 4096 x 4096 GEMV (16 MiB, cache-cold) 5.00 -> 4.45 us, and its steady rate over 16 to
// 256 MiB 6.08 -> 6.74 TB/s.
constexpr int CPOL_NT = 2;
__device__ __forceinline__ v4i load_nt16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, CPOL_NT));
}
__device__ __forceinline__ void store_wt16(__amdgpu_buffer_rsrc_t r, uint32_t off, float4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4i, v), r, off, 0, CPOL_WT);
}
__device__ __forceinline__ void store_wt4(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t v) {
  __builtin_amdgcn_raw_buffer_store_b32(v, r, off, 0, CPOL_WT);
}

}  // namespace bq
