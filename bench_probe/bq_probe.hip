// Measurement probes for bench.py (declared in bq_probe.h beside this file): the int8 MFMA rate the
// GPU sustains on given operand bytes, and the duration of a plain streaming read. They
// give the day's ceilings beside the nominal peaks; nothing in the int8 path calls them.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "../include/bq.h"
#include "bq_probe.h"

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

namespace {

thread_local char g_err[256] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

int launched(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(BQ_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  g_err[0] = 0;
  return BQ_OK;
}

constexpr int SETS = 4, TM = 4, TN = 2;

// Fragment loads are spread over the operands with a multiplicative hash of (lane, slot),
// so the waves hold as varied a sample of the bytes as the GEMM's LDS reads give them.
__device__ __forceinline__ v4i frag(const int8_t* p, uint32_t chunks, uint32_t key) {
  const uint32_t c = (key * 2654435761u) % chunks;
  return *reinterpret_cast<const v4i*>(p + (size_t)c * 16);
}

__global__ __launch_bounds__(512) void mfma_rate_kernel(const int8_t* A, uint32_t a_chunks, const int8_t* W,
                                                        uint32_t w_chunks, int iters, int32_t* sink) {
  const uint32_t g = blockIdx.x * 512u + threadIdx.x;
  v4i af[SETS][TM], bf[SETS][TN];
#pragma unroll
  for (int s = 0; s < SETS; ++s) {
#pragma unroll
    for (int i = 0; i < TM; ++i) af[s][i] = frag(A, a_chunks, g * 64u + s * TM + i);
#pragma unroll
    for (int j = 0; j < TN; ++j) bf[s][j] = frag(W, w_chunks, g * 64u + 32u + s * TN + j);
  }
  v16i c[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) c[i][j] = v16i{};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int s = 0; s < SETS; ++s)
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) c[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[s][i], bf[s][j], c[i][j], 0, 0, 0);
  }
  int r = 0;
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) r ^= c[i][j][e];
  sink[g] = r;
}

// The same with v_mfma_i32_16x16x64_i8 in the 256x256 tile's 16x16 form: 8 x 4 accumulators
// per wave, two fragment sets (the two 64-byte K slices of a stage).
constexpr int SETS16 = 2, TM16 = 8, TN16 = 4;
__global__ __launch_bounds__(512) void mfma_rate16_kernel(const int8_t* A, uint32_t a_chunks, const int8_t* W,
                                                          uint32_t w_chunks, int iters, int32_t* sink) {
  const uint32_t g = blockIdx.x * 512u + threadIdx.x;
  v4i af[SETS16][TM16], bf[SETS16][TN16];
#pragma unroll
  for (int s = 0; s < SETS16; ++s) {
#pragma unroll
    for (int i = 0; i < TM16; ++i) af[s][i] = frag(A, a_chunks, g * 64u + s * TM16 + i);
#pragma unroll
    for (int j = 0; j < TN16; ++j) bf[s][j] = frag(W, w_chunks, g * 64u + 32u + s * TN16 + j);
  }
  v4i c[TM16][TN16];
#pragma unroll
  for (int i = 0; i < TM16; ++i)
#pragma unroll
    for (int j = 0; j < TN16; ++j) c[i][j] = v4i{};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int s = 0; s < SETS16; ++s)
#pragma unroll
      for (int i = 0; i < TM16; ++i)
#pragma unroll
        for (int j = 0; j < TN16; ++j) c[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[s][i], bf[s][j], c[i][j], 0, 0, 0);
  }
  int r = 0;
#pragma unroll
  for (int i = 0; i < TM16; ++i)
#pragma unroll
    for (int j = 0; j < TN16; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) r ^= c[i][j][e];
  sink[g] = r;
}

template <int CH>
__global__ __launch_bounds__(256) void stream_read_kernel(const v4i* src, uint32_t n16, int32_t* sink) {
  const uint32_t base = blockIdx.x * (256u * CH) + threadIdx.x;
  v4i v[CH];
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const uint32_t k = base + i * 256u;
    v[i] = k < n16 ? __builtin_nontemporal_load(src + k) : v4i{};
  }
  int r = 0;
#pragma unroll
  for (int i = 0; i < CH; ++i) r ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) r ^= __shfl_xor(r, off, 64);
  __shared__ int red[4];
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = r;
  __syncthreads();
  if (threadIdx.x == 0) sink[blockIdx.x] = red[0] ^ red[1] ^ red[2] ^ red[3];
}

}  // namespace

extern "C" {

const char* bqp_last_error(void) { return g_err; }

int bqp_mfma_rate(const int8_t* A, int64_t a_bytes, const int8_t* W, int64_t w_bytes, int form, int blocks,
                  int iters, int32_t* sink, void* stream) {
  if (form != 32 && form != 16) return fail(BQ_ERR_ARG, "bqp_mfma_rate: form must be 32 or 16");
  if (!A || !W || !sink) return fail(BQ_ERR_ARG, "bqp_mfma_rate: null pointer");
  if (a_bytes < 4096 || w_bytes < 4096 || a_bytes % 16 || w_bytes % 16 || a_bytes / 16 > 0xffffffffll ||
      w_bytes / 16 > 0xffffffffll)
    return fail(BQ_ERR_ARG, "bqp_mfma_rate: operand sizes must be multiples of 16, >= 4096 and < 64 GiB");
  if (((uintptr_t)A & 15) || ((uintptr_t)W & 15)) return fail(BQ_ERR_ARG, "bqp_mfma_rate: unaligned operands");
  if (blocks < 1 || blocks > 65536 || iters < 1) return fail(BQ_ERR_ARG, "bqp_mfma_rate: bad blocks/iters");
  if (form == 16)
    mfma_rate16_kernel<<<blocks, 512, 0, (hipStream_t)stream>>>(A, (uint32_t)(a_bytes / 16), W,
                                                                (uint32_t)(w_bytes / 16), iters, sink);
  else
    mfma_rate_kernel<<<blocks, 512, 0, (hipStream_t)stream>>>(A, (uint32_t)(a_bytes / 16), W,
                                                              (uint32_t)(w_bytes / 16), iters, sink);
  return launched("bqp_mfma_rate");
}

int bqp_stream_read(const void* src, int64_t bytes, int chunks, int32_t* sink, void* stream) {
  if (!src || !sink) return fail(BQ_ERR_ARG, "bqp_stream_read: null pointer");
  if (bytes < 16 || bytes % 16 || bytes / 16 > 0x7fffffffll) return fail(BQ_ERR_ARG, "bqp_stream_read: bad size");
  if ((uintptr_t)src & 15) return fail(BQ_ERR_ARG, "bqp_stream_read: unaligned source");
  const uint32_t n16 = (uint32_t)(bytes / 16);
  hipStream_t st = (hipStream_t)stream;
  const v4i* s = (const v4i*)src;
  switch (chunks) {
    case 1: stream_read_kernel<1><<<(n16 + 255) / 256, 256, 0, st>>>(s, n16, sink); break;
    case 2: stream_read_kernel<2><<<(n16 + 511) / 512, 256, 0, st>>>(s, n16, sink); break;
    case 4: stream_read_kernel<4><<<(n16 + 1023) / 1024, 256, 0, st>>>(s, n16, sink); break;
    case 8: stream_read_kernel<8><<<(n16 + 2047) / 2048, 256, 0, st>>>(s, n16, sink); break;
    default: return fail(BQ_ERR_ARG, "bqp_stream_read: chunks must be 1, 2, 4 or 8");
  }
  return launched("bqp_stream_read");
}

}  // extern "C"
