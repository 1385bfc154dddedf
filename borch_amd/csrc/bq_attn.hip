// Softmax attention in f32 for a transformer's heads of width 64 and sequences of at most
// 256 tokens (ViT-B/16's 197): out = softmax((q k^T) * (1 / sqrt(64))) v per (image, head),
// the computation of borch's scaled_dot_product_attention (borch/_nn.py:2143-2170; its
// softmax is softmaxRows, borch-ts/src/kernels.ts:2483-2532: exp(x - max) / sum). It reads
// q, k and v straight from the qkv projection's output [B, T, 3, H, 64] and writes the heads
// side by side, [B, T, H * 64], the layout the output projection reads (no permute or
// transpose pass on either side).
//
// One workgroup per (image, head, 128 queries): its 8 waves share the head's whole k and v
// in LDS (2 x 256 x 68 floats at most) and take 16 queries each. Every product runs on
// v_mfma_f32_16x16x4_f32 (f32 operands, f32 accumulation). The scores are computed
// transposed, S^T = k q^T, so that each lane holds one query's scores (keys
// 16 j + 4 (lane / 16) + i in register i of key block j): the softmax of a query is a
// reduction over the lane's own registers and its 3 partner lanes, and the exponentials are,
// register for register, the B operand of O^T = v^T E^T (O divided by the row sum last). In both
// products the contracted index is permuted alike in the two operands (lane group g takes
// head dims 16 g .. 16 g + 15 of q and k; keys 16 j + 4 g + i of P and v), which changes
// only the order of the f32 sums.
#include <math.h>

#include "bq_common.h"

namespace bq {

typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int ATT_DH = 64;     // head width
constexpr int ATT_PITCH = 68;  // floats an LDS row of k or v (conflict-free fragment reads)
constexpr int ATT_WAVES = 8;   // 16 queries each (two waves a SIMD beside the LDS-bound one workgroup a CU)

__device__ __forceinline__ float xor_max(float v, int m) { return fmaxf(v, __shfl_xor(v, m)); }
__device__ __forceinline__ float xor_add(float v, int m) { return __fadd_rn(v, __shfl_xor(v, m)); }

template <int KB>
__global__ __launch_bounds__(ATT_WAVES * 64) void attention_f32_kernel(const float* __restrict__ qkv, int T, int H,
                                                                       int qblocks, float* __restrict__ out) {
  constexpr int TK = KB * 16;  // keys held (T rounded up to 16)
  __shared__ __attribute__((aligned(16))) float ks[TK * ATT_PITCH];
  __shared__ __attribute__((aligned(16))) float vs[TK * ATT_PITCH];
  const int bh = blockIdx.x / qblocks, qb = blockIdx.x - bh * qblocks;
  const int b = bh / H, h = bh - b * H;
  const int D = H * ATT_DH;
  const size_t tok = (size_t)3 * D;  // floats from one token's q to the next's
  const float* base = qkv + (size_t)b * T * tok + (size_t)h * ATT_DH;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int n = lane & 15;  // this lane's query within the wave's 16
  const int g = lane >> 4;  // its group: head dims 16 g .. 16 g + 15 of q and k
  const int q0 = qb * (ATT_WAVES * 16) + wave * 16;
  const int q = q0 + n;

  // Every load of the workgroup issued before the first is waited for: this lane's q
  // (q[q][16 g .. 16 g + 15], zeros past T), then its share of the head's k and v (keys past
  // T as zeros: their scores are masked below), then k and v go to LDS. (A load-then-store
  // loop waited for each round trip in turn.)
  float4 q4[4];
#pragma unroll
  for (int e = 0; e < 4; ++e)
    q4[e] = q < T ? *reinterpret_cast<const float4*>(base + q * tok + 16 * g + 4 * e) : make_float4(0.f, 0.f, 0.f, 0.f);
  constexpr int THREADS = ATT_WAVES * 64;
  constexpr int PER = (TK * (ATT_DH / 4) + THREADS - 1) / THREADS;  // float4 of k (and of v) a thread
  float4 kr[PER], vr[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int idx = threadIdx.x + i * THREADS;
    const int key = idx >> 4, c4 = (idx & 15) * 4;
    kr[i] = vr[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (key < T) {
      kr[i] = *reinterpret_cast<const float4*>(base + key * tok + D + c4);
      vr[i] = *reinterpret_cast<const float4*>(base + key * tok + 2 * D + c4);
    }
  }
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int idx = threadIdx.x + i * THREADS;
    const int key = idx >> 4, c4 = (idx & 15) * 4;
    if (key < TK) {
      *reinterpret_cast<float4*>(&ks[key * ATT_PITCH + c4]) = kr[i];
      *reinterpret_cast<float4*>(&vs[key * ATT_PITCH + c4]) = vr[i];
    }
  }
  __syncthreads();
  if (q0 >= T) return;  // a wave past the last query (no barrier follows)
  float qv[16];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    qv[4 * e] = q4[e].x; qv[4 * e + 1] = q4[e].y; qv[4 * e + 2] = q4[e].z; qv[4 * e + 3] = q4[e].w;
  }

  // S^T = k q^T: key block j, lane (n, g), register i -> key 16 j + 4 g + i, query q
  v4f s[KB];
#pragma unroll
  for (int j = 0; j < KB; ++j) s[j] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float4 kf[KB];  // every key block's 4 head dims first: consecutive MFMAs use different accumulators
#pragma unroll
    for (int j = 0; j < KB; ++j) kf[j] = *reinterpret_cast<const float4*>(&ks[(16 * j + n) * ATT_PITCH + 16 * g + 4 * e]);
#pragma unroll
    for (int j = 0; j < KB; ++j) s[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[j].x, qv[4 * e], s[j], 0, 0, 0);
#pragma unroll
    for (int j = 0; j < KB; ++j) s[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[j].y, qv[4 * e + 1], s[j], 0, 0, 0);
#pragma unroll
    for (int j = 0; j < KB; ++j) s[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[j].z, qv[4 * e + 2], s[j], 0, 0, 0);
#pragma unroll
    for (int j = 0; j < KB; ++j) s[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[j].w, qv[4 * e + 3], s[j], 0, 0, 0);
  }

  // softmax over the keys of query q: scores * 1/sqrt(64) (exact), keys past T at -inf
  constexpr float factor = 0.125f;
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < KB; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int key = 16 * j + 4 * g + i;
      const float v = key < T ? __fmul_rn(s[j][i], factor) : -INFINITY;
      s[j][i] = v;
      m = fmaxf(m, v);
    }
  m = xor_max(xor_max(m, 16), 32);
  float sum = 0.f;
#pragma unroll
  for (int j = 0; j < KB; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float e = expf(__fsub_rn(s[j][i], m));  // exp(-inf) = 0 for the masked keys
      s[j][i] = e;
      sum = __fadd_rn(sum, e);
    }
  sum = xor_add(xor_add(sum, 16), 32);

  // O^T = v^T E^T with the unnormalised exponentials E, then O / sum (16 divisions a lane,
  // not one a score: the normalisation moves past the f32 sums, within their bound). Head-dim
  // block d, lane (n, g), register r -> dim 16 d + 4 g + r, query q; two accumulator sets
  // (even and odd key blocks) keep eight independent MFMA chains in flight.
  v4f o[2][4];
#pragma unroll
  for (int d = 0; d < 4; ++d) o[0][d] = o[1][d] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < KB; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float* vrow = &vs[(16 * j + 4 * g + i) * ATT_PITCH + n];
#pragma unroll
      for (int d = 0; d < 4; ++d)
        o[j & 1][d] = __builtin_amdgcn_mfma_f32_16x16x4f32(vrow[16 * d], s[j][i], o[j & 1][d], 0, 0, 0);
    }
  if (q < T) {
    float* orow = out + ((size_t)b * T + q) * D + (size_t)h * ATT_DH;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const v4f a = o[0][d] + o[1][d];
      *reinterpret_cast<float4*>(orow + 16 * d + 4 * g) =
          make_float4(__fdiv_rn(a[0], sum), __fdiv_rn(a[1], sum), __fdiv_rn(a[2], sum), __fdiv_rn(a[3], sum));
    }
  }
}

}  // namespace bq

using namespace bq;

int bq_attention_f32(const float* qkv, int64_t B, int64_t T, int64_t H, int64_t dh, float* out, bq_stream_t stream) {
  const char* what = "bq_attention_f32";
  if (B < 0 || T < 0 || H < 1) return set_error(BQ_ERR_ARG, "%s: bad sizes", what);
  if (dh != ATT_DH) return set_error(BQ_ERR_UNSUPPORTED, "%s: head width %lld (64 only)", what, (long long)dh);
  if (T > 256) return set_error(BQ_ERR_UNSUPPORTED, "%s: %lld tokens (at most 256)", what, (long long)T);
  if (B == 0 || T == 0) return BQ_OK;
  if (B * T * 3 * H * dh >= ((int64_t)1 << 31) || B * H > 0x7fffffff / 4)
    return set_error(BQ_ERR_ARG, "%s: size too large", what);
  if (!qkv || !out) return set_error(BQ_ERR_ARG, "%s: null pointer", what);
  if (((uintptr_t)qkv & 15) || ((uintptr_t)out & 15)) return set_error(BQ_ERR_ARG, "%s: misaligned pointer", what);
  const int qblocks = (int)((T + ATT_WAVES * 16 - 1) / (ATT_WAVES * 16));
  const unsigned grid = (unsigned)(B * H * qblocks);
  hipStream_t st = (hipStream_t)stream;
  const int kb = (int)((T + 15) / 16);
  if (kb <= 4) attention_f32_kernel<4><<<grid, ATT_WAVES * 64, 0, st>>>(qkv, (int)T, (int)H, qblocks, out);
  else if (kb <= 8) attention_f32_kernel<8><<<grid, ATT_WAVES * 64, 0, st>>>(qkv, (int)T, (int)H, qblocks, out);
  else if (kb <= 13) attention_f32_kernel<13><<<grid, ATT_WAVES * 64, 0, st>>>(qkv, (int)T, (int)H, qblocks, out);
  else attention_f32_kernel<16><<<grid, ATT_WAVES * 64, 0, st>>>(qkv, (int)T, (int)H, qblocks, out);
  return check_launch(what);
}
