// W8A8 GEMM and implicit-GEMM convolution on gfx950 int8 MFMA, with the dequant epilogue.
//
// One kernel template serves both: C[M, N] = A[M, K] · W[N, K]^T where W is the int8
// weight (K-contiguous rows) and A is either a dense int8 matrix (Linear) or the implicit
// im2col of an NHWC int8 activation (conv: M = N·OH·OW pixels, K = KH·KW·C, tap-major then
// channel). Both operands are K-contiguous, so each MFMA lane reads 16 contiguous bytes
// of one row of each — no transposes anywhere.
//
// Tiles: BM x BN output per workgroup, K walked in 128-byte stages (one 128 B cache line
// per row per stage) through a ring of NBUF LDS stage buffers, XOR-swizzled by 16-byte
// chunk, that direct-to-LDS buffer loads fill (no VGPR staging) while earlier stages
// compute. Each wave owns a (BM/WAVES_M) x (BN/WAVES_N) sub-tile of 32x32
// v_mfma_i32_32x32x32_i8 results. With random int8 operands the MFMA pipe is power-limited
// near 22 ns per 32x32x32 MFMA per SIMD (measured, about 3.0 POPS chip-wide), which the
// main loop of the 256x256 tile reaches to within about 15%.
//
// Skinny path (M <= 64): the weight is streamed once at HBM rate. A workgroup owns 16
// output channels; its waves split K; each lane loads 64 contiguous weight bytes per step
// and v_mfma_i32_16x16x64_i8 multiplies them against up to four 16-row activation tiles.
#include <stdlib.h>

#include <algorithm>
#include <array>
#include <map>
#include <mutex>
#include <type_traits>
#include <utility>

#include "bq_common.h"

namespace bq {

struct GemmP {
  const int8_t* A;  // dense [M, K]; conv: NHWC [Nimg, H, W, C]
  const int8_t* W;  // [N, K]
  int M, N, K;
  const float* sA;  // [M] per row, or [1] per tensor
  int sa_per_row;
  const float* sW;  // [N]
  const float* bias;
  const float* res;  // [M, N] or null
  int act;
  float* out;    // [M, N]
  int32_t* acc;  // [M, N] or null
  // conv geometry (CONV only)
  int H, Wd, C, OH, OW, KWd, stride, pad;
  // k / C and tap / KW of the implicit im2col as multiply-high and shift (FastDiv), and
  // m / (OH OW) and r / OW (the small-K kernel's per-row decomposition)
  uint32_t c_mul, kw_mul, plane_mul, ow_mul;
  int c_shift, kw_shift, plane_shift, ow_shift;
  int64_t Nimg_HWC;  // conv: bytes of the NHWC activation (the small-K f32 input: of Xf)
  int vec_ok;        // N % 4 == 0 and out/res/acc 16-byte aligned: float4 epilogue
  const float* s_out;  // static output scale [1] (nullable): the int8 twin of the output
  int8_t* q_out;       // [M, N] int8 = clip(rint(y / s_out)) (nullable)
  // Split-K (tiled kernel only): ksplit workgroups per output tile, each over a contiguous
  // run of K stages; each stores its int32 partial tile in `part` and bumps the tile's
  // counter in `cnt`; the last to arrive adds the partials and runs the epilogue, then
  // resets the counter to zero. ksplit == 1: no partials, no counters.
  int ksplit;
  int32_t* part;  // [tiles][ksplit][BM * BN] int32, in the accumulator register order
  int* cnt;       // [tiles], zero between launches
  // Tiled kernel only (nullable): max |y| over each output tile's final values (after bias,
  // residual and activation), one float per tile at bm * tiles_n + bn — the partial maxima
  // from which the next layer's per-tensor quantizer takes its scale without a max pass.
  float* amax;
  // Host-side selection only (the kernels ignore them): a tuned plan's configuration id
  // (0: the shape rule) and K split (0: the split rule).
  int plan_cfg, plan_split;
  // GEMV with the per-row quantize fused (gemv_i8_fq_kernel): f32 activations X [M, K] in
  // place of A / sA; the quantized rows and their scales are also written to qx [M, K] and
  // sx [M] (nullable) by workgroup 0.
  const float* X;
  int8_t* qx;
  float* sx;
  // The small-K conv on an f32 NCHW input [N, Cin, H, W] (Cin <= 8 < C = 16, the padded
  // channels of the packed weight read as zeros), its per-tensor quantization fused: Xf in
  // place of A; the scale sx_given[0] (calibrated) or float32(max / 127) of the partial
  // maxima xparts [nxparts]; sx_out (nullable) receives it.
  const float* Xf;
  int Cin;
  const float* sx_given;
  const float* xparts;
  int nxparts;
  float* sx_out;
  // The int8 twin at a dynamic per-tensor scale (small-K kernel only): with oparts set, the
  // twin's scale is float32(max / 127) of the partial maxima oparts [noparts] that a pass
  // before this one wrote for the same outputs (s_out unused), and workgroup 0 writes it to
  // sout_write [1] (nullable).
  const float* oparts;
  int noparts;
  float* sout_write;
  // Diagnostics (tiled kernel, nullable): four words a workgroup at 4 * (its regrouped id):
  // the steady wall clock (100 MHz) at entry, after the main loop and after its last store
  // completed, then its hardware id (__smid: XCC, SE, CU). bq_gemm_i8_phases sets it.
  uint64_t* stamps;
};

constexpr int BK = 128;  // bytes of K per LDS stage: one cache line per row
// Split-K is compiled into (and offered to) tiles of at most this many outputs only.
constexpr int SPLIT_MAX_TILE = 64 * 64;
// The largest K whose int32 sum of products is exact for any int8 operands in [-127, 127]:
// K * 127^2 <= 2^31 - 1.
constexpr int KMAX_EXACT = 133152;

// Buffer resources: raw (stride 0) descriptors whose range check returns zero for any
// 16-byte load at or past `bytes` — the tile edges (rows past M or N, the K tail, conv
// padding) become zeros without a branch. OOB is the offset that is always out of range.
constexpr uint32_t OOB = 0x80000000u;


__device__ __forceinline__ v4i buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}


// Byte offset of 16-byte chunk `c` (0..7) of LDS row `r`. The chunk index is XORed with
// bits 1..3 of the row: the 16 lanes that read one MFMA fragment (16 consecutive rows,
// one chunk) then cover all 64 four-byte banks exactly once (rows 2j and 2j+1 sit in the
// two 128-byte halves of the 256-byte bank line). Measured: zero LDS bank conflicts.
__device__ __forceinline__ int lds_off(int r, int c) { return r * BK + ((c ^ ((r >> 1) & 7)) << 4); }

// Scheduling hints: NMMA MFMAs, each followed by up to ceil(COUNT/NMMA) instructions of
// class MASK (0x008 MFMA, 0x020 VMEM read, 0x100 DS read, 0x200 DS write), so memory
// instructions issue between MFMAs instead of in one block.
template <int MASK, int N>
__device__ __forceinline__ void sched_group() {
  if constexpr (N > 0) __builtin_amdgcn_sched_group_barrier(MASK, N, 0);
}
template <int MASK, int COUNT, int NMMA, int... I>
__device__ __forceinline__ void interleave_impl(std::integer_sequence<int, I...>) {
  constexpr int per = (COUNT + NMMA - 1) / NMMA;
  ((sched_group<0x008, 1>(),
    sched_group<MASK, (COUNT - I * per >= per ? per : (COUNT - I * per > 0 ? COUNT - I * per : 0))>()),
   ...);
}
template <bool ON, int MASK, int COUNT, int NMMA>
__device__ __forceinline__ void interleave() {
  if constexpr (ON) interleave_impl<MASK, COUNT, NMMA>(std::make_integer_sequence<int, NMMA>{});
}
// The same with the COUNT instructions spread over the first SPREAD MFMAs only, the rest
// of the NMMA MFMAs after them: used for the LDS reads that precede a wait for them, so that
// they have returned by the time the wave reaches the wait.
template <int MASK, int COUNT, int NMMA, int SPREAD>
__device__ __forceinline__ void interleave_front() {
  interleave_impl<MASK, COUNT, SPREAD>(std::make_integer_sequence<int, SPREAD>{});
  sched_group<0x008, NMMA - SPREAD>();
}

// One 16-byte-per-lane load straight into LDS (no VGPR staging): lane l's 16 bytes land at
// LDS byte address m0v + 16 * l. Issued from inline assembly so that the compiler, which
// cannot tell these writes from the fragment reads of the other buffer, does not add a
// full vmcnt wait before every LDS read; the caller waits (vmcnt) before the barrier that
// publishes a stage. M0 is written here and used by nothing else in these kernels; the
// s_nop covers the M0-write -> LDS-DMA hazard.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t m0v) {
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(r), "s"(m0v)
               : "m0");
#pragma clang diagnostic pop
}
__device__ __forceinline__ void wait_dma_all() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// A barrier orders LDS stores, not loads still in flight: before a barrier after which a
// buffer this wave read is refilled, its reads must have returned.
__device__ __forceinline__ void wait_lds() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
template <int N>
__device__ __forceinline__ void wait_dma() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Main loop with direct-to-LDS loads into a ring of NBUF stage buffers. A stage's LDS image
// is written by wave-wide DMAs of 8 rows (1 KB) each: lane l covers row 8*band + l/8 and
// LDS chunk slot l%8, and fetches the global 16-byte chunk that the XOR swizzle maps to that
// slot, so each 16 bytes land where lds_off() places them for the fragment reads.
// Stage kt+NBUF is fetched into the buffer stage kt just left, right after the barrier that
// ends stage kt, and must land by the barrier that ends stage kt+NBUF-1: NBUF-1 stages of
// MFMAs cover its latency (small tiles, whose stages are short, take deep rings).
template <int BM, int BN, int WAVES_M, int WAVES_N, bool CONV, int NBUF, int FD, bool MF16, typename Acc>
__device__ __forceinline__ void mainloop_dma(const GemmP& p, int m0, int n0, int kt0, int KT, int8_t* lds,
                                             float* s_sa, float* s_sw, float* s_b, Acc& c) {
  constexpr int WAVES = WAVES_M * WAVES_N;
  constexpr int T = WAVES * 64;
  constexpr int WTM = BM / WAVES_M;
  constexpr int WTN = BN / WAVES_N;
  constexpr int TM = WTM / 32;
  constexpr int TN = WTN / 32;
  constexpr int BAND = 8 * WAVES;  // rows one DMA per wave covers
  constexpr int A_DMA = BM / BAND;
  constexpr int B_DMA = BN / BAND;
  static_assert(BM % BAND == 0 && BN % BAND == 0 && (WAVES % 2) == 0, "tile/waves");
  static_assert(BM <= T && BN <= T, "one scale per thread");
  constexpr int PER = A_DMA + B_DMA;  // DMAs a wave issues per stage
  static_assert(NBUF >= 2 && (NBUF - 1) * PER <= 63, "ring depth / vmcnt range");
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WAVES_N;
  const int wn = wave % WAVES_N;
  const int wv = __builtin_amdgcn_readfirstlane(wave);

  // Scales and bias: loaded now, written to LDS after the loop (their latency hides
  // behind the main loop instead of delaying its start).
  const int sm = m0 + tid, sn = n0 + tid;
  const float r_sa = (tid < BM && sm < p.M) ? p.sA[p.sa_per_row ? sm : 0] : 0.f;
  const float r_sw = (tid < BN && sn < p.N) ? p.sW[sn] : 0.f;
  const float r_b = (tid < BN && sn < p.N && p.bias) ? p.bias[sn] : 0.f;

  // This lane's row within each band and the global chunk it fetches. Every band starts at
  // a multiple of 16 rows (WAVES even), so the swizzle term is the same in every band.
  const int drow = wv * 8 + (lane >> 3);
  const int dch = (lane & 7) ^ ((drow >> 1) & 7);
  const uint32_t lds_base = (uint32_t)(uintptr_t)lds;

  const __amdgpu_buffer_rsrc_t rb = make_rsrc(p.W + (size_t)n0 * p.K, (uint32_t)(min(BN, p.N - n0) * p.K));
  __amdgpu_buffer_rsrc_t ra;
  uint32_t a_pix[A_DMA];
  int a_ih0[A_DMA], a_iw0[A_DMA];
  if constexpr (CONV) {
    ra = make_rsrc(p.A, (uint32_t)((size_t)p.Nimg_HWC));
    const int plane = p.OH * p.OW;
#pragma unroll
    for (int i = 0; i < A_DMA; ++i) {
      const int m = m0 + i * BAND + drow;
      const int n = m / plane;
      const int r = m - n * plane;
      const int oh = r / p.OW;
      const int ow = r - oh * p.OW;
      const bool ok = m < p.M;
      a_ih0[i] = ok ? oh * p.stride - p.pad : -(1 << 20);  // an invalid row never passes the bounds test
      a_iw0[i] = ow * p.stride - p.pad;
      a_pix[i] = (uint32_t)(n * p.H * p.Wd * p.C);
    }
  } else {
    ra = make_rsrc(p.A + (size_t)m0 * p.K, (uint32_t)(min(BM, p.M - m0) * p.K));
#pragma unroll
    for (int i = 0; i < A_DMA; ++i) {
      a_pix[i] = (uint32_t)((i * BAND + drow) * p.K);
      a_ih0[i] = a_iw0[i] = 0;
    }
  }
  uint32_t b_row[B_DMA];
#pragma unroll
  for (int i = 0; i < B_DMA; ++i) b_row[i] = (uint32_t)((i * BAND + drow) * p.K);

  // Stages kt0 .. kt0+KT-1 of K (a split-K slice, or all of K); past them every offset is
  // out of range and reads zeros.
  const int kend = min(p.K, (kt0 + KT) * BK);
  auto dma_stage = [&](int buf, int kt) {
    const int k0 = (kt0 + kt) * BK + dch * 16;
    const bool kin = k0 < kend;
    const uint32_t am0 = lds_base + (uint32_t)(buf * (BM + BN) * BK + wv * 1024);
    const uint32_t bm0 = am0 + BM * BK;
    if constexpr (CONV) {
      const int tap = fdiv(k0, p.c_mul, p.c_shift);
      const int c0 = k0 - tap * p.C;
      const int kh = fdiv(tap, p.kw_mul, p.kw_shift);
      const int kw = tap - kh * p.KWd;
#pragma unroll
      for (int i = 0; i < A_DMA; ++i) {
        const int ih = a_ih0[i] + kh, iw = a_iw0[i] + kw;
        const bool ok = kin && (unsigned)ih < (unsigned)p.H && (unsigned)iw < (unsigned)p.Wd;
        dma16(ra, ok ? a_pix[i] + (uint32_t)((ih * p.Wd + iw) * p.C + c0) : OOB, am0 + i * BAND * BK);
      }
    } else {
#pragma unroll
      for (int i = 0; i < A_DMA; ++i) dma16(ra, kin ? a_pix[i] + (uint32_t)k0 : OOB, am0 + i * BAND * BK);
    }
#pragma unroll
    for (int i = 0; i < B_DMA; ++i) dma16(rb, kin ? b_row[i] + (uint32_t)k0 : OOB, bm0 + i * BAND * BK);
  };
  const int fr = lane & 31;
  const int fh = lane >> 5;
  auto frags = [&](int buf, int ks, v4i (&af)[TM], v4i (&bf)[TN]) {
    const int8_t* as = lds + buf * (BM + BN) * BK;
    const int8_t* bs = as + BM * BK;
#pragma unroll
    for (int i = 0; i < TM; ++i) af[i] = *reinterpret_cast<const v4i*>(as + lds_off(wm * WTM + i * 32 + fr, ks * 2 + fh));
#pragma unroll
    for (int j = 0; j < TN; ++j) bf[j] = *reinterpret_cast<const v4i*>(bs + lds_off(wn * WTN + j * 32 + fr, ks * 2 + fh));
  };
  auto mma = [&](const auto (&a)[TM], const auto (&b)[TN]) {  // generic: instantiated by the 32x32 loops only
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) c[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[j], c[i][j], 0, 0, 0);
  };
  constexpr int NMMA = TM * TN, NRD = TM + TN;

  // Stage pipeline (ks = the four 32-byte K slices of a 128-byte stage):
  //   ks0..ks2: MFMAs of slice ks | LDS reads of slice ks+1
  //   wait for this wave's DMAs of stage kt+1 (the NBUF-2 later stages may stay in flight);
  //   barrier (stage kt+1 landed for every wave; every read of stage kt is done, so its
  //   buffer is free)
  //   DMAs of stage kt+NBUF into that buffer
  //   ks3: MFMAs of slice 3 | LDS reads of slice 0 of stage kt+1
  // Stages past K are fetched too: every offset is then out of range and the DMA writes zeros.
#pragma unroll
  for (int st = 0; st < NBUF; ++st) dma_stage(st, st);
  wait_dma<(NBUF - 1) * PER>();
  __syncthreads();
  if constexpr (MF16) {
    // v_mfma_i32_16x16x64_i8: the wave tile as (2 TM) x (2 TN) blocks of 16 x 16, a stage as
    // two 64-byte K slices. The same MACs and LDS bytes as the 32x32x32 form, in twice as
    // many half-size MFMAs, which sustain a higher rate at the power limit on random int8
    // operands (3.66 against 3.21 POP/s, the same operand bytes, no memory traffic).
    // Lane l reads row l % 16 of a 16-row block and 16-byte K chunk l / 16 of the slice; its
    // result register r is row 4 (l / 16) + r, column l % 16.
    constexpr int TM2 = 2 * TM, TN2 = 2 * TN;
    constexpr int NM16 = TM2 * TN2, NR16 = TM2 + TN2;
    const int gr = lane & 15, gc = lane >> 4;
    auto frags16 = [&](int buf, int ks, v4i (&af)[TM2], v4i (&bf)[TN2]) {
      const int8_t* as = lds + buf * (BM + BN) * BK;
      const int8_t* bs = as + BM * BK;
#pragma unroll
      for (int i = 0; i < TM2; ++i) af[i] = *reinterpret_cast<const v4i*>(as + lds_off(wm * WTM + i * 16 + gr, ks * 4 + gc));
#pragma unroll
      for (int j = 0; j < TN2; ++j) bf[j] = *reinterpret_cast<const v4i*>(bs + lds_off(wn * WTN + j * 16 + gr, ks * 4 + gc));
    };
    auto mma16 = [&](const v4i (&a)[TM2], const v4i (&b)[TN2]) {
#pragma unroll
      for (int i = 0; i < TM2; ++i)
#pragma unroll
        for (int j = 0; j < TN2; ++j) c[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i], b[j], c[i][j], 0, 0, 0);
    };
    v4i af[2][TM2], bf[2][TN2];
    frags16(0, 0, af[0], bf[0]);
    int cur = 0;
    for (int kt = 0; kt < KT; ++kt) {
      const int nxt = cur + 1 == NBUF ? 0 : cur + 1;
      frags16(cur, 1, af[1], bf[1]);
      mma16(af[0], bf[0]);
      interleave_front<0x100, NR16, NM16, (NM16 + 1) / 2>();
      __builtin_amdgcn_sched_barrier(0);
      wait_dma<(NBUF - 2) * PER>();
      wait_lds();  // this wave's reads of the buffer about to be refilled have returned
      __syncthreads();
      frags16(nxt, 0, af[0], bf[0]);  // past the last stage: data no one uses
      dma_stage(cur, kt + NBUF);
      mma16(af[1], bf[1]);
      interleave<true, 0x100, NR16, NM16>();
      __builtin_amdgcn_sched_barrier(0);
      cur = nxt;
    }
  } else if constexpr (FD == 2) {
    // Fragments two slices ahead (four register sets, one per slice); the barrier sits
    // after slice 1 so that slices 0 and 1 of stage kt+1 are read under slices 2 and 3.
    v4i af[4][TM], bf[4][TN];
    frags(0, 0, af[0], bf[0]);
    frags(0, 1, af[1], bf[1]);
    int cur = 0;
    for (int kt = 0; kt < KT; ++kt) {
      const int nxt = cur + 1 == NBUF ? 0 : cur + 1;
      frags(cur, 2, af[2], bf[2]);
      mma(af[0], bf[0]);
      interleave<true, 0x100, NRD, NMMA>();
      __builtin_amdgcn_sched_barrier(0);
      frags(cur, 3, af[3], bf[3]);
      mma(af[1], bf[1]);
      interleave_front<0x100, NRD, NMMA, (NMMA + 1) / 2>();
      __builtin_amdgcn_sched_barrier(0);
      wait_dma<(NBUF - 2) * PER>();
      wait_lds();  // this wave's reads of the buffer about to be refilled have returned
      __syncthreads();
      frags(nxt, 0, af[0], bf[0]);  // past the last stage: data no one uses
      dma_stage(cur, kt + NBUF);
      mma(af[2], bf[2]);
      interleave<true, 0x100, NRD, NMMA>();
      __builtin_amdgcn_sched_barrier(0);
      frags(nxt, 1, af[1], bf[1]);
      mma(af[3], bf[3]);
      interleave<true, 0x100, NRD, NMMA>();
      __builtin_amdgcn_sched_barrier(0);
      cur = nxt;
    }
  } else {
  v4i af[2][TM], bf[2][TN];
  frags(0, 0, af[0], bf[0]);
  int cur = 0;
  for (int kt = 0; kt < KT; ++kt) {
    const int nxt = cur + 1 == NBUF ? 0 : cur + 1;
    frags(cur, 1, af[1], bf[1]);
    mma(af[0], bf[0]);
    interleave<true, 0x100, NRD, NMMA>();
    __builtin_amdgcn_sched_barrier(0);
    frags(cur, 2, af[0], bf[0]);
    mma(af[1], bf[1]);
    interleave<true, 0x100, NRD, NMMA>();
    __builtin_amdgcn_sched_barrier(0);
    frags(cur, 3, af[1], bf[1]);
    mma(af[0], bf[0]);
    interleave_front<0x100, NRD, NMMA, (NMMA + 1) / 2>();
    __builtin_amdgcn_sched_barrier(0);
    wait_dma<(NBUF - 2) * PER>();
    wait_lds();  // this wave's reads of the buffer about to be refilled have returned
    __syncthreads();
    frags(nxt, 0, af[0], bf[0]);  // past the last stage: data no one uses
    dma_stage(cur, kt + NBUF);
    mma(af[1], bf[1]);
    interleave<true, 0x100, NRD, NMMA>();
    __builtin_amdgcn_sched_barrier(0);
    cur = nxt;
  }
  }
  wait_dma_all();  // the zero-filling DMAs past K land before the epilogue reuses the buffers
  if (tid < BM) s_sa[tid] = r_sa;
  if (tid < BN) {
    s_sw[tid] = r_sw;
    s_b[tid] = r_b;
  }
  __syncthreads();
}

// The tiled kernel's LDS: the ring of stage buffers (reused by the epilogue's patches), and
// the tile's scales and bias, staged once so the epilogue reads no global memory (on gfx9
// stores and loads share one counter, and a load between stores waits for them).
template <int BM, int BN, int WAVES, int NBUF>
struct TileLds {
  __attribute__((aligned(16))) int8_t ring[NBUF * (BM + BN) * BK];
  __attribute__((aligned(16))) float sa[BM];
  __attribute__((aligned(16))) float sw[BN];
  __attribute__((aligned(16))) float b[BN];
  int last;            // split-K: this workgroup is the last of its tile
  float wmax[WAVES];   // per-wave max |y| (p.amax)
};

// One workgroup of the tiled GEMM / implicit-GEMM conv: the workgroup of XCD-regrouped id
// L (xcd_order over the whole launch) among those that cover problem p (its tiles times its
// K split).
template <int BM, int BN, int WAVES_M, int WAVES_N, bool CONV, int NBUF, int FD, bool MF16>
__device__ __forceinline__ void gemm_tile(const GemmP& p, const int L,
                                          TileLds<BM, BN, WAVES_M * WAVES_N, NBUF>& sh) {
  constexpr int T = WAVES_M * WAVES_N * 64;
  constexpr int WTM = BM / WAVES_M;  // wave tile rows
  constexpr int WTN = BN / WAVES_N;
  constexpr int TM = WTM / 32;
  constexpr int TN = WTN / 32;
  static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile");
  int8_t* const lds = sh.ring;
  float* const s_sa = sh.sa;
  float* const s_sw = sh.sw;
  float* const s_b = sh.b;
  int& s_last = sh.last;
  float* const s_wmax = sh.wmax;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WAVES_N;
  const int wn = wave % WAVES_N;

  const int tiles_m = (p.M + BM - 1) / BM;
  const int tiles_n = (p.N + BN - 1) / BN;
  const int KT = (p.K + BK - 1) / BK;
  constexpr bool CAN_SPLIT = BM * BN <= SPLIT_MAX_TILE;
  const int S = CAN_SPLIT ? p.ksplit : 1;
  const int split = L % S;
  int bm, bn;
  tile_of(L / S, tiles_m, tiles_n, bm, bn);
  const int m0 = bm * BM;
  const int n0 = bn * BN;
  const int per = (KT + S - 1) / S;  // stages of each split (the host picks S with no empty split)
  const int kt0 = split * per;

  const uint64_t t_entry = p.stamps ? (uint64_t)wall_clock64() : 0;
  const Quantizer qz_out(p.q_out ? p.s_out[0] : 0.f);
  // the accumulators: TM x TN blocks of 32 x 32 (16 registers each), or with MF16
  // (2 TM) x (2 TN) blocks of 16 x 16 (4 registers each): the same registers either way
  std::conditional_t<MF16, v4i[2 * TM][2 * TN], v16i[TM][TN]> c;
  if constexpr (MF16) {
#pragma unroll
    for (int i = 0; i < 2 * TM; ++i)
#pragma unroll
      for (int j = 0; j < 2 * TN; ++j) c[i][j] = v4i{};
  } else {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) c[i][j] = v16i{};
  }
  mainloop_dma<BM, BN, WAVES_M, WAVES_N, CONV, NBUF, FD, MF16>(p, m0, n0, kt0, min(per, KT - kt0), lds, s_sa, s_sw,
                                                         s_b, c);
  const uint64_t t_loop = p.stamps ? (uint64_t)wall_clock64() : 0;
  if (CAN_SPLIT && S > 1) {
    // Exact split-K reduction in the same launch. Partials are int32, so the sum is exact
    // whatever the order. Each lane stores its accumulator registers as 8-byte chunks at
    // [tile][split][chunk][lane] (contiguous across the workgroup); the last workgroup of
    // the tile reads the other splits' chunks at its own lanes' offsets, so no re-layout is
    // needed. No workgroup ever waits for another: the counter only elects the one that
    // finishes the tile.
    // Coherence across XCDs (each has its own L2) without cache-wide write-back or
    // invalidation: partials are written and read with device-scope relaxed atomics
    // (write-through stores and L2-bypassing loads at agent scope); every store has
    // completed (vmcnt 0) before the workgroup's counter increment, and the last
    // workgroup's loads are issued after its increment returned S - 1.
    constexpr int NV = TM * TN * 8;  // 8-byte chunks per lane
    const int tile = bm * tiles_n + bn;
    uint64_t* const part = reinterpret_cast<uint64_t*>(p.part);
    uint64_t* mine = part + ((size_t)(tile * S + split) * NV) * T + tid;
    // chunk e of a lane: two consecutive accumulator registers, in the order of c
    auto chunk = [&](int e) -> uint64_t {
      int lo, hi;
      if constexpr (MF16) {
        lo = c[e / (4 * TN)][(e / 2) % (2 * TN)][2 * (e % 2)];
        hi = c[e / (4 * TN)][(e / 2) % (2 * TN)][2 * (e % 2) + 1];
      } else {
        lo = c[e / (8 * TN)][(e / 8) % TN][2 * (e % 8)];
        hi = c[e / (8 * TN)][(e / 8) % TN][2 * (e % 8) + 1];
      }
      return (uint64_t)(uint32_t)lo | ((uint64_t)(uint32_t)hi << 32);
    };
    auto add_chunk = [&](int e, uint64_t w) {
      if constexpr (MF16) {
        c[e / (4 * TN)][(e / 2) % (2 * TN)][2 * (e % 2)] += (int)(uint32_t)w;
        c[e / (4 * TN)][(e / 2) % (2 * TN)][2 * (e % 2) + 1] += (int)(uint32_t)(w >> 32);
      } else {
        c[e / (8 * TN)][(e / 8) % TN][2 * (e % 8)] += (int)(uint32_t)w;
        c[e / (8 * TN)][(e / 8) % TN][2 * (e % 8) + 1] += (int)(uint32_t)(w >> 32);
      }
    };
#pragma unroll
    for (int e = 0; e < NV; ++e)
      __hip_atomic_store(mine + (size_t)e * T, chunk(e), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    wait_dma_all();  // every partial store of this lane has completed
    __syncthreads();
    if (tid == 0)
      s_last = __hip_atomic_fetch_add(p.cnt + tile, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == S - 1;
    __syncthreads();
    if (!s_last) return;  // uniform across the workgroup
    // Four splits' chunks are loaded before any is added, so their round trips overlap.
    constexpr int BATCH = 4;
    for (int sp0 = 0; sp0 < S; sp0 += BATCH) {
      uint64_t v[BATCH][NV];
#pragma unroll
      for (int u = 0; u < BATCH; ++u) {
        const int sp = sp0 + u;
        const bool use = sp < S && sp != split;
        uint64_t* other = part + ((size_t)(tile * S + (use ? sp : split)) * NV) * T + tid;
#pragma unroll
        for (int e = 0; e < NV; ++e)
          v[u][e] = use ? __hip_atomic_load(other + (size_t)e * T, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0;
      }
#pragma unroll
      for (int u = 0; u < BATCH; ++u)
#pragma unroll
        for (int e = 0; e < NV; ++e) add_chunk(e, v[u][e]);
    }
    if (tid == 0) __hip_atomic_store(p.cnt + tile, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  // Epilogue, one 32-row slice of the wave tile at a time: the int32 results go through a
  // per-wave LDS patch (exact), come back as four consecutive columns of one row per lane,
  // and leave as 16-byte stores of whole 256-byte row segments. 32x32 result layout:
  // lane l, register r holds row 8*(r/4) + 4*(l/32) + r%4, column l%32.
  // Patch pitch (ints) for conflict-free ds_write_b32 of a whole wave (64 banks): the 32x32
  // layout writes two 32-column rows 4 apart (4 PITCH % 64 == 32 keeps them apart), the
  // 16x16 layout four 16-column rows 4 apart (4 PITCH % 64 == 16). The read-back takes one
  // 256-byte row per 16 lanes, conflict-free at any 16-byte-aligned pitch.
  constexpr int PITCH = WTN + (MF16 ? 4 : 8);
  static_assert(WAVES_M * WAVES_N * 32 * PITCH * 4 <= NBUF * (BM + BN) * BK, "epilogue patch");
  static_assert((PITCH * 4) % 16 == 0 && (4 * PITCH) % 64 == (MF16 ? 16 : 32), "patch pitch");
  int* patch = reinterpret_cast<int*>(lds) + wave * 32 * PITCH;
  constexpr int C4 = WTN / 4;                 // float4 columns per row
  constexpr int ROWS_PER_STORE = 64 / C4;     // rows one 64-lane store covers
  constexpr int NST = 32 / ROWS_PER_STORE;    // stores per slice
  const bool has_r = p.res != nullptr;
  float amax = 0.f;  // max |y| of the values this lane stores (fmaxf: a NaN is skipped)

  // Fast path: no int32 output, float4-aligned, and a tile's rows within 2 GB. Its stores
  // are buffer stores through resources that end at row M of the tile: a lane's offset
  // within the tile is one 32-bit VGPR, and rows past M fall out of range and are dropped by
  // the hardware (no per-row test, no 64-bit address arithmetic per store). About 5 VALU
  // instructions per output against 12 on the general path, whose per-row branches on every
  // optional output stay for the other cases. The stores write through to memory (sc1): the
  // output does not sit dirty in the XCD's L2 to be written back at the kernel's end, which
  // measured 4-16% faster per launch back to back (ViT qkv 23.2 -> 21.2 us, half-batch qkv
  // 16.0 -> 13.5). The int8 twin of a calibrated layer (no per-tile maxima) takes this path
  // on tiles of up to 128x128, beside the f32 output or alone: four packed bytes a lane and
  // row (ResNet-18 b16's 64x64 convs: 7.3 -> 6.4 us with both outputs, 6.7 -> 6.4 us with
  // the twin alone). The larger tiles keep the general path for the twin: inlined there, its
  // packing pushed their kernel arguments out of SGPRs.
  constexpr bool FASTQ = BM * BN <= 128 * 128;
  const bool has_out = p.out != nullptr;
  const bool fast = p.vec_ok && !p.acc && (p.q_out ? FASTQ && !p.amax : has_out) &&
                    (long long)BM * p.N * 4 < (1ll << 31);
  const int tile_rows = min(BM, p.M - m0);
  const uint32_t tile_bytes = fast ? (uint32_t)((long long)tile_rows * p.N * 4) : 0u;
  const __amdgpu_buffer_rsrc_t r_out = make_rsrc(has_out ? p.out + (size_t)m0 * p.N : p.out, has_out ? tile_bytes : 0u);
  const __amdgpu_buffer_rsrc_t r_res = make_rsrc(has_r ? p.res + (size_t)m0 * p.N : p.res, has_r ? tile_bytes : 0u);
  const __amdgpu_buffer_rsrc_t r_q = make_rsrc(p.q_out ? p.q_out + (size_t)m0 * p.N : p.q_out,
                                               fast && p.q_out ? (uint32_t)(tile_rows * p.N) : 0u);
  const uint32_t row_step = (uint32_t)(ROWS_PER_STORE * p.N) * 4u;  // bytes between a lane's rows
  // Rows rl, rl + ROWS_PER_STORE, ... of the tile (rl: this lane's first row of the slice).
  // (always inlined: a call would take the kernel argument block's address and move its
  // fields from SGPRs to VGPRs)
  // Q: the int8 twin through r_q (byte offsets a quarter of the f32 ones), and the f32 row
  // only when there is an f32 output.
  auto fast_rows = [&]<bool RES, bool AMAX, bool Q>(int rl, int col4, int ncol) __attribute__((always_inline)) {
    const float4 sw4 = *reinterpret_cast<const float4*>(&s_sw[ncol]);
    const float4 b4 = *reinterpret_cast<const float4*>(&s_b[ncol]);
    const uint32_t voffq = (uint32_t)rl * (uint32_t)p.N + (uint32_t)(n0 + ncol);
    const uint32_t voff = voffq * 4u;
    float4 rv[NST];
    if constexpr (RES) {  // every residual row first: a load after a store waits for it
#pragma unroll
      for (int k = 0; k < NST; ++k)
        rv[k] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r_res, voff + k * row_step, 0, 0));
    }
#pragma unroll
    for (int k = 0; k < NST; ++k) {
      const int row = k * ROWS_PER_STORE + lane / C4;  // within the slice
      const int4 a = *reinterpret_cast<const int4*>(&patch[row * PITCH + col4 * 4]);
      const float sa = s_sa[rl + k * ROWS_PER_STORE];
      float4 o;
      o.x = __fadd_rn(__fmul_rn(__fmul_rn((float)a.x, sa), sw4.x), b4.x);
      o.y = __fadd_rn(__fmul_rn(__fmul_rn((float)a.y, sa), sw4.y), b4.y);
      o.z = __fadd_rn(__fmul_rn(__fmul_rn((float)a.z, sa), sw4.z), b4.z);
      o.w = __fadd_rn(__fmul_rn(__fmul_rn((float)a.w, sa), sw4.w), b4.w);
      if constexpr (RES) {
        o.x = __fadd_rn(o.x, rv[k].x); o.y = __fadd_rn(o.y, rv[k].y);
        o.z = __fadd_rn(o.z, rv[k].z); o.w = __fadd_rn(o.w, rv[k].w);
      }
      if (p.act == BQ_ACT_RELU) {
        o.x = o.x > 0.f ? o.x : 0.f; o.y = o.y > 0.f ? o.y : 0.f;
        o.z = o.z > 0.f ? o.z : 0.f; o.w = o.w > 0.f ? o.w : 0.f;
      } else if (p.act == BQ_ACT_SILU) {
        o.x = silu(o.x); o.y = silu(o.y); o.z = silu(o.z); o.w = silu(o.w);
      } else if (p.act == BQ_ACT_GELU) {
        o = gelu4(o);
      }
      // The row step goes into the VGPR offset: with it in the SGPR offset these stores
      // wrote wrong values to about 1% of the rows (each store followed by an LDS read
      // into its data registers); with it in the VGPR offset, none.
      if (!Q || has_out) store_wt16(r_out, voff + k * row_step, o);
      if constexpr (Q) store_wt4(r_q, voffq + k * (row_step / 4u), qz_out.pack(o));
      if constexpr (AMAX) {  // rows past M are computed (and dropped) but must not count
        if (m0 + rl + k * ROWS_PER_STORE < p.M)
          amax = fmaxf(amax, fmaxf(fmaxf(fabsf(o.x), fabsf(o.y)), fmaxf(fabsf(o.z), fabsf(o.w))));
      }
    }
  };
  // One slice per compile-time i (a run-time i would index the accumulators dynamically
  // and send them to scratch memory).
  auto slice = [&](auto ic) {
    constexpr int i = decltype(ic)::value;
    if constexpr (MF16) {  // blocks 2i and 2i + 1 of 16 rows: lane l, register r is row 4 (l / 16) + r
#pragma unroll
      for (int sub = 0; sub < 2; ++sub)
#pragma unroll
        for (int j = 0; j < 2 * TN; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            patch[(sub * 16 + (lane >> 4) * 4 + r) * PITCH + j * 16 + (lane & 15)] = c[2 * i + sub][j][r];
    } else {
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          patch[((r >> 2) * 8 + (lane >> 5) * 4 + (r & 3)) * PITCH + j * 32 + (lane & 31)] = c[i][j][r];
    }
    // This wave's patch is written before any lane reads another lane's values. The wait is
    // an asm statement with a memory clobber: the compiler, which sees only one lane, would
    // otherwise move a read above a write that cannot alias within that lane (the builtin
    // waitcnt and wave barrier do not order memory for it).
    wait_lds();
    __builtin_amdgcn_wave_barrier();
    const int col4 = lane % C4;
    const int ncol = wn * WTN + col4 * 4;  // tile-local column of this lane's 4 values
    const int n = n0 + ncol;
    if (fast) {
      if (n < p.N) {
        const int rl = wm * WTM + i * 32 + lane / C4;
        if (FASTQ && p.q_out) {
          if constexpr (FASTQ) {
            if (has_r) fast_rows.template operator()<true, false, true>(rl, col4, ncol);
            else fast_rows.template operator()<false, false, true>(rl, col4, ncol);
          }
        } else if (has_r) {
          if (p.amax) fast_rows.template operator()<true, true, false>(rl, col4, ncol);
          else fast_rows.template operator()<true, false, false>(rl, col4, ncol);
        } else {
          if (p.amax) fast_rows.template operator()<false, true, false>(rl, col4, ncol);
          else fast_rows.template operator()<false, false, false>(rl, col4, ncol);
        }
      }
    } else if (p.vec_ok && n < p.N) {
      const float4 sw4 = *reinterpret_cast<const float4*>(&s_sw[ncol]);
      const float4 b4 = *reinterpret_cast<const float4*>(&s_b[ncol]);
      // Bias 0 when absent: y + 0.0f == y for every y this produces (no -0.0).
      auto store_row = [&](int rr, float4 rv, bool with_r) {
        const int row = rr + lane / C4;
        const int mloc = wm * WTM + i * 32 + row;
        const int m = m0 + mloc;
        if (m < p.M) {
          const int4 a = *reinterpret_cast<const int4*>(&patch[row * PITCH + col4 * 4]);
          const float sa = s_sa[mloc];
          const size_t idx = (size_t)m * p.N + n;
          float4 o;
          o.x = __fadd_rn(__fmul_rn(__fmul_rn((float)a.x, sa), sw4.x), b4.x);
          o.y = __fadd_rn(__fmul_rn(__fmul_rn((float)a.y, sa), sw4.y), b4.y);
          o.z = __fadd_rn(__fmul_rn(__fmul_rn((float)a.z, sa), sw4.z), b4.z);
          o.w = __fadd_rn(__fmul_rn(__fmul_rn((float)a.w, sa), sw4.w), b4.w);
          if (with_r) {
            o.x = __fadd_rn(o.x, rv.x); o.y = __fadd_rn(o.y, rv.y);
            o.z = __fadd_rn(o.z, rv.z); o.w = __fadd_rn(o.w, rv.w);
          }
          if (p.act == BQ_ACT_RELU) {
            o.x = o.x > 0.f ? o.x : 0.f; o.y = o.y > 0.f ? o.y : 0.f;
            o.z = o.z > 0.f ? o.z : 0.f; o.w = o.w > 0.f ? o.w : 0.f;
          } else if (p.act == BQ_ACT_SILU) {
            o.x = silu(o.x); o.y = silu(o.y); o.z = silu(o.z); o.w = silu(o.w);
          } else if (p.act == BQ_ACT_GELU) {
            o = gelu4(o);
          }
          if (p.out) *reinterpret_cast<float4*>(p.out + idx) = o;  // null: the twin alone
          if (p.acc) *reinterpret_cast<int4*>(p.acc + idx) = a;
          if (p.q_out)
            *reinterpret_cast<uint32_t*>(p.q_out + idx) =
                qz_out.pack(o);
          amax = fmaxf(amax, fmaxf(fmaxf(fabsf(o.x), fabsf(o.y)), fmaxf(fabsf(o.z), fabsf(o.w))));
        }
      };
      if (has_r) {
        // The slice's residual rows are all loaded before any of its stores: on gfx9 a
        // load issued after stores waits (vmcnt) for them too, so a load per row would
        // serialize the stores. Unrolled, so the values stay in registers; this path's
        // code runs only for residual layers.
        constexpr int NR = 32 / ROWS_PER_STORE;
        float4 rv[NR];
#pragma unroll
        for (int k = 0; k < NR; ++k) {
          const int m = m0 + wm * WTM + i * 32 + k * ROWS_PER_STORE + lane / C4;
          rv[k] = m < p.M ? *reinterpret_cast<const float4*>(p.res + (size_t)m * p.N + n)
                          : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int k = 0; k < NR; ++k) store_row(k * ROWS_PER_STORE, rv[k], true);
      } else {
        // Rolled on purpose: an unrolled copy per row and slice overflows the instruction
        // cache.
#pragma unroll 1
        for (int rr = 0; rr < 32; rr += ROWS_PER_STORE) store_row(rr, make_float4(0.f, 0.f, 0.f, 0.f), false);
      }
    } else if (!p.vec_ok) {
#pragma unroll 1
      for (int rr = 0; rr < 32; rr += ROWS_PER_STORE) {
        const int row = rr + lane / C4;
        const int mloc = wm * WTM + i * 32 + row;
        const int m = m0 + mloc;
#pragma unroll 1
        for (int q = 0; q < 4; ++q) {
          if (m < p.M && n + q < p.N) {
            const int a = patch[row * PITCH + col4 * 4 + q];
            const size_t idx = (size_t)m * p.N + n + q;
            const float rv = has_r ? p.res[idx] : 0.f;
            const float o = dequant_one(a, s_sa[mloc], s_sw[ncol + q], s_b[ncol + q], true, rv, has_r, p.act);
            if (p.out) p.out[idx] = o;
            if (p.acc) p.acc[idx] = a;
            if (p.q_out) p.q_out[idx] = (int8_t)qz_out(o);
            amax = fmaxf(amax, fabsf(o));
          }
        }
      }
    }
    wait_lds();  // this slice's patch reads are done before the next slice's writes
    __builtin_amdgcn_wave_barrier();
  };
  [&]<int... Is>(std::integer_sequence<int, Is...>) {
    (slice(std::integral_constant<int, Is>{}), ...);
  }(std::make_integer_sequence<int, TM>{});
  if (p.amax) {  // uniform: every wave of the workgroup takes it
    amax = wave_max(amax);
    if (lane == 0) s_wmax[wave] = amax;
    __syncthreads();
    if (tid == 0) {
      float m = s_wmax[0];
#pragma unroll
      for (int w = 1; w < WAVES_M * WAVES_N; ++w) m = fmaxf(m, s_wmax[w]);
      p.amax[bm * tiles_n + bn] = m;
    }
  }
  if (p.stamps) {  // uniform
    wait_dma_all();  // this lane's stores have completed
    __syncthreads();
    if (tid == 0) {
      uint64_t* st = p.stamps + 4 * (size_t)L;
      st[0] = t_entry;
      st[1] = t_loop;
      st[2] = (uint64_t)wall_clock64();
      st[3] = __smid();
    }
  }
}

template <int BM, int BN, int WAVES_M, int WAVES_N, bool CONV, int NBUF, int FD, bool MF16 = false>
__global__ __launch_bounds__(WAVES_M* WAVES_N * 64) void gemm_i8_kernel(const GemmP p) {
  __shared__ TileLds<BM, BN, WAVES_M * WAVES_N, NBUF> sh;
  gemm_tile<BM, BN, WAVES_M, WAVES_N, CONV, NBUF, FD, MF16>(p, xcd_order(blockIdx.x, gridDim.x), sh);
}

// Two problems of one tile configuration in one launch: workgroups [0, g0) run p0, the
// rest p1 (a residual block's first conv and its downsampling shortcut, which read the same
// input: two launches' fixed cost paid once, and the smaller grids share the chip). Only p0
// may split K.
template <int BM, int BN, int WAVES_M, int WAVES_N, bool CONV, int NBUF, int FD>
__global__ __launch_bounds__(WAVES_M* WAVES_N * 64) void gemm_i8_pair_kernel(const GemmP p0, const GemmP p1,
                                                                           int g0) {
  __shared__ TileLds<BM, BN, WAVES_M * WAVES_N, NBUF> sh;
  // regrouped once over the whole grid (the hardware puts workgroup i on XCD i % 8), so
  // both convs' consecutive ids stay on one XCD whatever g0 is
  const int L = xcd_order(blockIdx.x, gridDim.x);
  if (L < g0)
    gemm_tile<BM, BN, WAVES_M, WAVES_N, CONV, NBUF, FD, false>(p0, L, sh);
  else
    gemm_tile<BM, BN, WAVES_M, WAVES_N, CONV, NBUF, FD, false>(p1, L - g0, sh);
}

// ----------------------------------------------------------------------------- skinny

constexpr int SK_COLS = 16;  // output channels a workgroup

// Weight-streaming GEMM for M <= 64: W is read once, at HBM rate. A workgroup owns 16
// weight rows (output channels); its WAVES waves split K; the MFMA j of a 256-byte step
// takes bytes [64 j, 64 j + 64) of each row, 16 a lane, so one wave-load reads 64
// contiguous bytes of each of the 16 rows (16-byte pieces 64 bytes apart: 7.4 -> 6.9 us at
// M = 16, the same sums in another order of k), and every weight load of a wave's share
// (U steps) is issued before the first MFMA, so a whole 16-row slab is in flight at once.
// The activation rows (tiny, L2-resident) are loaded first, after the epilogue's scales,
// bias and residual, so that no memory round trip is left after the sums. v_mfma_i32_16x16x64_i8
// multiplies the weight bytes against up to four 16-row activation tiles; the waves'
// partial sums meet in LDS.
template <int MT, int WAVES, int U>
__global__ __launch_bounds__(WAVES * 64) void skinny_i8_kernel(const GemmP p) {
  __shared__ int red[WAVES][MT][64][4];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int n0 = blockIdx.x * SK_COLS;
  const int col = lane & 15;  // weight row within the 16 (the B operand's column)
  const int kg = lane >> 4;   // which 64-byte group of a 256-byte step
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(p.W + (size_t)n0 * p.K, (uint32_t)(min(SK_COLS, p.N - n0) * p.K));
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.A, (uint32_t)(p.M * p.K));

  // Thread e < 256 writes output (t * 16 + e / 16, n0 + e % 16) of each 16-row tile t: its
  // epilogue operands are fetched now, ahead of the operand stream.
  const int e = threadIdx.x;
  const int ml = (e >> 4) & 15, nl = e & 15;
  const int nn = n0 + nl;
  const bool writer = e < 256 && nn < p.N;
  float e_sw = 0.f, e_b = 0.f, e_sa[MT], e_r[MT];
  if (writer) {
    e_sw = p.sW[nn];
    e_b = p.bias ? p.bias[nn] : 0.f;
  }
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    const int m = t * 16 + ml;
    const bool mine = writer && m < p.M;
    e_sa[t] = mine ? (p.sa_per_row ? p.sA[m] : p.sA[0]) : 0.f;
    e_r[t] = mine && p.res ? p.res[(size_t)m * p.N + nn] : 0.f;
  }

  v4i c[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) c[t] = v4i{};

  const int steps = (p.K + 255) / 256;
  for (int s0 = wave * U; s0 < steps; s0 += WAVES * U) {
    v4i a[U][MT][4], w[U][4];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int k = (s0 + u) * 256 + j * 64 + kg * 16;
          a[u][t][j] = buf_load16(ra, k < p.K ? (uint32_t)((t * 16 + col) * p.K + k) : OOB);
        }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int k = (s0 + u) * 256 + j * 64 + kg * 16;
        w[u][j] = load_nt16(rw, k < p.K ? (uint32_t)(col * p.K + k) : OOB);
      }
    __builtin_amdgcn_sched_barrier(0);  // keep every load of the share ahead of the MFMAs
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int j = 0; j < 4; ++j) c[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[u][t][j], w[u][j], c[t], 0, 0, 0);
  }
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) red[wave][t][lane][r] = c[t][r];
  __syncthreads();
  // 16x16 result layout: lane l, register r holds row 4*(l/16) + r, column l%16.
  if (!writer) return;
  const int src_lane = (ml >> 2) * 16 + nl, src_r = ml & 3;
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    const int m = t * 16 + ml;
    if (m < p.M) {
      int acc = 0;
#pragma unroll
      for (int w = 0; w < WAVES; ++w) acc += red[w][t][src_lane][src_r];
      const size_t idx = (size_t)m * p.N + nn;
      p.out[idx] = dequant_one(acc, e_sa[t], e_sw, e_b, p.bias != nullptr, e_r[t], p.res != nullptr, p.act);
      if (p.acc) p.acc[idx] = acc;
    }
  }
}

// ----------------------------------------------------------------------------- small K

// GEMM for a narrow output (N <= 256, N % 4 == 0) and a short K (<= 256) over many rows: a
// 1x1 conv's projection or expansion over a large image (EfficientNet-B0 b64's
// blocks.1.expand, 802816 x 96 x 16), or with CONV an implicit-GEMM conv of that shape (its
// stem: 3x3 / 2 over 16 padded channels into 32, each lane's 16-byte chunk of a row at the
// tap its K offset names). The tiled kernel spends most of its time outside its MFMAs there
// (one K stage, a 128 x 128 tile for 96 columns). Here the weight fragments stay in
// registers for the whole launch, and each wave takes 16 rows a step: the weight is the
// MFMA's first operand and the activation rows its second (v_mfma_i32_16x16x64_i8; lane l
// holds row l % 16 and K chunk l / 16 of each), so lane l's four results of 16-column block
// j are columns 16 j + 4 (l / 16) .. + 3 of row l % 16, four consecutive outputs it stores
// as one 16-byte piece straight from the accumulators (the epilogue arithmetic of the
// tiled kernel's, in the same order). The next step's activation rows load before this
// step's MFMAs, its residual pieces before its stores. The column scales and bias sit in
// registers up to 8 column blocks and in LDS beyond (the registers they would take cost more
// occupancy than the reads: 50176 x 240 x 48 19.9 -> 13.0 us). Stores write through (sc1):
// 802816 x 96 75.7 against 96.1 us plain. The int8 twin goes through a per-wave LDS patch
// and leaves as whole rows (below); its scale is a calibrated one, or float32(max / 127) of
// the maxima an earlier launch over the same layer wrote with no output stored (the
// dynamic twin: two passes of the epilogue instead of an f32 output and a quantize pass
// over it). With CINM > 0 the input is the network's f32 NCHW image
// (at most CINM real channels a tap, the rest of the 16 zero): each lane loads its taps' raw
// floats a step ahead and quantizes them when the step runs (the scale calibrated, or taken
// from partial maxima at the start). Workgroups stride over the 64-row steps; each writes
// one max |y| (p.amax). Unaligned outputs take four-byte stores.
constexpr int SMALLK_ROWS = 64;  // rows a workgroup step: 4 waves x 16
template <int NB, int KS, bool CONV, int CINM = 0>
__global__ __launch_bounds__(256) void smallk_i8_kernel(const GemmP p) {
  constexpr bool F32IN = CINM > 0;  // an f32 NCHW input of at most CINM channels, quantized here
  static_assert(!F32IN || CONV, "an f32 input is a conv's");
  constexpr bool LDSS = NB > 8;  // column scales and bias in LDS
  __shared__ float s_wmax[4];
  __shared__ __attribute__((aligned(16))) float s_sw[LDSS ? NB * 16 : 4], s_b[LDSS ? NB * 16 : 4];
  // The int8 twin of a wave's 16 rows, packed here before it is stored as whole rows, in
  // the rows' own layout (row r at byte r * N): the 16-byte piece e of the run is LDS word 4 e
  __shared__ __attribute__((aligned(16))) uint32_t s_tw[4][16 * 4 * NB];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c16 = lane & 15, kq = lane >> 4;
  const int M = p.M, N = p.N, K = p.K;
  const int steps = (M + SMALLK_ROWS - 1) / SMALLK_ROWS;
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(p.W, (uint32_t)(N * K));
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.A, CONV ? (uint32_t)p.Nimg_HWC : (uint32_t)(M * K));
  v4i b[NB][KS];
  constexpr int NE = LDSS ? 1 : NB;
  float4 e_sw[NE], e_b[NE];  // the scales and bias of this lane's four columns of block j
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    const int n = j * 16 + c16;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int k = ks * 64 + kq * 16;
      b[j][ks] = buf_load16(rw, (n < N && k < K) ? (uint32_t)(n * K + k) : OOB);
    }
    if constexpr (!LDSS) {
      const int n0 = j * 16 + 4 * kq;
      e_sw[j] = n0 < N ? make_float4(p.sW[n0], p.sW[n0 + 1], p.sW[n0 + 2], p.sW[n0 + 3])
                       : make_float4(0.f, 0.f, 0.f, 0.f);
      // 0 without bias: y + 0.0f == y for every y this produces
      e_b[j] = (n0 < N && p.bias) ? make_float4(p.bias[n0], p.bias[n0 + 1], p.bias[n0 + 2], p.bias[n0 + 3])
                                  : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  if constexpr (LDSS) {
    if (tid < NB * 16) {
      s_sw[tid] = tid < N ? p.sW[tid] : 0.f;
      s_b[tid] = (tid < N && p.bias) ? p.bias[tid] : 0.f;
    }
    __syncthreads();
  }
  // CONV: this lane's K chunks as (filter row, filter column, channel offset); a chunk past K
  // gets a row offset no input row passes
  int t_kh[KS], t_kw[KS], t_c0[KS];
  if constexpr (CONV) {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int k = ks * 64 + kq * 16;
      const int tap = fdiv(k, p.c_mul, p.c_shift);
      t_c0[ks] = k - tap * p.C;
      t_kh[ks] = fdiv(tap, p.kw_mul, p.kw_shift);
      t_kw[ks] = tap - t_kh[ks] * p.KWd;
      if (k >= K) t_kh[ks] = -(1 << 20);
    }
  }
  float sa0;
  if constexpr (F32IN) {
    // the input's scale: calibrated, or from the partial maxima (every workgroup reduces
    // them; a maximum does not depend on the order)
    if (p.sx_given) {
      sa0 = p.sx_given[0];
    } else {
      float mx = 0.f;
      for (int i = tid; i < p.nxparts; i += 256) mx = fmaxf(mx, p.xparts[i]);
      mx = wave_max(mx);
      if (lane == 0) s_wmax[wave] = mx;
      __syncthreads();
      sa0 = scale_of(fmaxf(fmaxf(s_wmax[0], s_wmax[1]), fmaxf(s_wmax[2], s_wmax[3])));
      __syncthreads();  // s_wmax is reused for the output's maximum
    }
    if (p.sx_out && blockIdx.x == 0 && tid == 0) p.sx_out[0] = sa0;
  } else {
    sa0 = p.sa_per_row ? 0.f : p.sA[0];
  }
  const Quantizer qz_in(F32IN ? sa0 : 0.f);
  float so = 0.f;
  if (p.q_out) {
    if (p.oparts) {
      // the twin's dynamic scale from the maxima of a pass before this one, reduced by every
      // workgroup as the input's are above
      float mx = 0.f;
      for (int i = tid; i < p.noparts; i += 256) mx = fmaxf(mx, p.oparts[i]);
      mx = wave_max(mx);
      if (lane == 0) s_wmax[wave] = mx;
      __syncthreads();
      so = scale_of(fmaxf(fmaxf(s_wmax[0], s_wmax[1]), fmaxf(s_wmax[2], s_wmax[3])));
      __syncthreads();  // s_wmax is reused for the output's maximum
      if (p.sout_write && blockIdx.x == 0 && tid == 0) p.sout_write[0] = so;
    } else {
      so = p.s_out[0];
    }
  }
  const Quantizer qz_out(so);
  const bool has_r = p.res != nullptr, vec = p.vec_ok;
  // the twin as whole rows through LDS (O % 16 == 0 always holds for a twin; its base aligned)
  const bool tw_rows = p.q_out && vec && (N & 15) == 0 && ((uintptr_t)p.q_out & 15) == 0;
  const uint32_t out_bytes = (uint32_t)std::min<long long>((long long)M * N * 4, 0x7fffffff);
  const __amdgpu_buffer_rsrc_t r_out = make_rsrc(p.out, p.out ? out_bytes : 0u);
  const __amdgpu_buffer_rsrc_t r_acc = make_rsrc(p.acc, p.acc ? out_bytes : 0u);
  const __amdgpu_buffer_rsrc_t r_res = make_rsrc(p.res, has_r ? out_bytes : 0u);
  const __amdgpu_buffer_rsrc_t r_q = make_rsrc(p.q_out, p.q_out ? out_bytes / 4u : 0u);
  float amax = 0.f;
  // The next step's operand in flight: its int8 chunks, or with F32IN the raw f32 values of
  // this lane's taps (quantized when the step runs, so their loads overlap this step's work)
  constexpr int CM = F32IN ? CINM : 1;
  struct Pending {
    v4i q[KS];
    float x[KS][CM];
  };
  const __amdgpu_buffer_rsrc_t r_x =
      make_rsrc(p.Xf, F32IN ? (uint32_t)p.Nimg_HWC : 0u);
  auto fetch = [&](Pending& pd, int t) {
    const int row = t * SMALLK_ROWS + wave * 16 + c16;
    const bool live = t < steps && row < M;
    if constexpr (CONV) {
      const int n = fdiv(row, p.plane_mul, p.plane_shift);
      const int r = row - n * p.OH * p.OW;
      const int oh = fdiv(r, p.ow_mul, p.ow_shift);
      const int ih0 = oh * p.stride - p.pad, iw0 = (r - oh * p.OW) * p.stride - p.pad;
      if constexpr (F32IN) {
        // a chunk is one tap's 16 channels (C == 16): the Cin real ones from the NCHW planes,
        // the rest zeros (an out-of-range buffer load reads 0)
        const uint32_t plane = (uint32_t)(p.H * p.Wd);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const int ih = ih0 + t_kh[ks], iw = iw0 + t_kw[ks];
          const bool ok = live && (unsigned)ih < (unsigned)p.H && (unsigned)iw < (unsigned)p.Wd;
          const uint32_t o = ((uint32_t)n * (uint32_t)p.Cin * plane + (uint32_t)(ih * p.Wd + iw)) * 4u;
#pragma unroll
          for (int c = 0; c < CM; ++c)
            pd.x[ks][c] = __builtin_bit_cast(
                float, __builtin_amdgcn_raw_buffer_load_b32(r_x, ok && c < p.Cin ? o + (uint32_t)c * plane * 4u : OOB,
                                                            0, 0));
        }
      } else {
        const uint32_t img = (uint32_t)(n * p.H * p.Wd * p.C);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const int ih = ih0 + t_kh[ks], iw = iw0 + t_kw[ks];
          const bool ok = live && (unsigned)ih < (unsigned)p.H && (unsigned)iw < (unsigned)p.Wd;
          pd.q[ks] = buf_load16(ra, ok ? img + (uint32_t)((ih * p.Wd + iw) * p.C + t_c0[ks]) : OOB);
        }
      }
    } else {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int k = ks * 64 + kq * 16;
        pd.q[ks] = buf_load16(ra, (live && k < K) ? (uint32_t)(row * K + k) : OOB);
      }
    }
  };
  auto operand = [&](v4i (&a)[KS], const Pending& pd) {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if constexpr (F32IN) {
        uint32_t w4[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int c4 = 0; c4 < CM / 4; ++c4)
          w4[c4] = qz_in.pack(make_float4(pd.x[ks][4 * c4], pd.x[ks][4 * c4 + 1], pd.x[ks][4 * c4 + 2],
                                          pd.x[ks][4 * c4 + 3]));
        a[ks] = v4i{(int)w4[0], (int)w4[1], (int)w4[2], (int)w4[3]};
      } else {
        a[ks] = pd.q[ks];
      }
    }
  };
  Pending pd;
  int t = blockIdx.x;
  fetch(pd, t);
  for (; t < steps; t += gridDim.x) {
    v4i a[KS];
    operand(a, pd);
    fetch(pd, t + gridDim.x);
    const int m = t * SMALLK_ROWS + wave * 16 + c16;  // this lane's row
    const bool live = m < M;
    const float sa = p.sa_per_row ? (live ? p.sA[m] : 0.f) : sa0;
    // the row's residual pieces, all before any store (on gfx9 a load issued after stores
    // waits for them); past M or N the range check gives zeros
    float4 rv[NB] = {};
    if (has_r) {
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        const int n0 = j * 16 + 4 * kq;
        const uint32_t off = live && n0 < N ? (uint32_t)((size_t)m * N + n0) * 4u : OOB;
        if (vec) {
          rv[j] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r_res, off, 0, 0));
        } else {
          rv[j] = make_float4(__builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r_res, off, 0, 0)),
                              __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r_res, off + 4, 0, 0)),
                              __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r_res, off + 8, 0, 0)),
                              __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r_res, off + 12, 0, 0)));
        }
      }
    }
    // Column block j, j known at compile time (a loop the unroller left rolled at 12 or more
    // blocks put the weight fragments in scratch memory)
    auto block = [&](auto jc) __attribute__((always_inline)) {
      constexpr int j = decltype(jc)::value;
      v4i c = v4i{};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) c = __builtin_amdgcn_mfma_i32_16x16x64_i8(b[j][ks], a[ks], c, 0, 0, 0);
      const int n0 = j * 16 + 4 * kq;
      if (!live || n0 >= N) return;
      float4 sw4, b4;
      if constexpr (LDSS) {
        sw4 = *reinterpret_cast<const float4*>(s_sw + n0);
        b4 = *reinterpret_cast<const float4*>(s_b + n0);
      } else {
        sw4 = e_sw[LDSS ? 0 : j];
        b4 = e_b[LDSS ? 0 : j];
      }
      float4 o;
      o.x = __fadd_rn(__fmul_rn(__fmul_rn((float)c[0], sa), sw4.x), b4.x);
      o.y = __fadd_rn(__fmul_rn(__fmul_rn((float)c[1], sa), sw4.y), b4.y);
      o.z = __fadd_rn(__fmul_rn(__fmul_rn((float)c[2], sa), sw4.z), b4.z);
      o.w = __fadd_rn(__fmul_rn(__fmul_rn((float)c[3], sa), sw4.w), b4.w);
      if (has_r) {
        o.x = __fadd_rn(o.x, rv[j].x); o.y = __fadd_rn(o.y, rv[j].y);
        o.z = __fadd_rn(o.z, rv[j].z); o.w = __fadd_rn(o.w, rv[j].w);
      }
      if (p.act == BQ_ACT_RELU) {
        o.x = o.x > 0.f ? o.x : 0.f; o.y = o.y > 0.f ? o.y : 0.f;
        o.z = o.z > 0.f ? o.z : 0.f; o.w = o.w > 0.f ? o.w : 0.f;
      } else if (p.act == BQ_ACT_SILU) {
        o.x = silu(o.x); o.y = silu(o.y); o.z = silu(o.z); o.w = silu(o.w);
      } else if (p.act == BQ_ACT_GELU) {
        o = gelu4(o);
      }
      const uint32_t off = (uint32_t)((size_t)m * N + n0) * 4u;
      if (vec) {
        if (p.out) store_wt16(r_out, off, o);
        if (p.acc) __builtin_amdgcn_raw_buffer_store_b128(c, r_acc, off, 0, CPOL_WT);
        if (p.q_out) {
          if (tw_rows)
            s_tw[wave][c16 * (N >> 2) + j * 4 + kq] = qz_out.pack(o);
          else
            store_wt4(r_q, off / 4u, qz_out.pack(o));
        }
      } else {
        const float of[4] = {o.x, o.y, o.z, o.w};
        const uint32_t qw = p.q_out ? qz_out.pack(o) : 0u;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (p.out) __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, of[e]), r_out, off + 4 * e, 0, CPOL_WT);
          if (p.acc) __builtin_amdgcn_raw_buffer_store_b32((uint32_t)c[e], r_acc, off + 4 * e, 0, CPOL_WT);
          if (p.q_out) __builtin_amdgcn_raw_buffer_store_b8((uint8_t)(qw >> (8 * e)), r_q, off / 4u + e, 0, CPOL_WT);
        }
      }
      if (p.amax) amax = fmaxf(amax, fmaxf(fmaxf(fabsf(o.x), fabsf(o.y)), fmaxf(fabsf(o.z), fabsf(o.w))));
    };
    [&]<int... J>(std::integer_sequence<int, J...>) __attribute__((always_inline)) {
      (block(std::integral_constant<int, J>{}), ...);
    }(std::make_integer_sequence<int, NB>{});
    if (tw_rows) {
      // The wave's 16 twin rows are one contiguous run of 16 N bytes: 16-byte pieces of it
      // from LDS, consecutive lanes on consecutive pieces (four-byte pieces of 16 rows a
      // store measured 90 us for EfficientNet-B0's 802816 x 96 twin). The run's start is in
      // the resource base, so a lane's offset is its own piece and the SGPR offset stays 0
      // (the form the tiled kernel's LDS-fed stores need); rows past M fall out of range.
      wait_lds();
      __builtin_amdgcn_wave_barrier();
      const int m_first = t * SMALLK_ROWS + wave * 16;
      if (m_first < M) {
        const __amdgpu_buffer_rsrc_t r_tw =
            make_rsrc(p.q_out + (size_t)m_first * N, (uint32_t)(min(16, M - m_first) * N));
        for (int e = lane; e < N; e += 64) {  // 16 rows of N bytes: N pieces of 16
          const v4i v = *reinterpret_cast<const v4i*>(&s_tw[wave][4 * e]);
          __builtin_amdgcn_raw_buffer_store_b128(v, r_tw, (uint32_t)e * 16u, 0, CPOL_WT);
        }
      }
      wait_lds();  // every read of the patch is done before the next step writes it
      __builtin_amdgcn_wave_barrier();
    }
  }
  if (p.amax) {
    amax = wave_max(amax);
    if (lane == 0) s_wmax[wave] = amax;
    __syncthreads();
    if (tid == 0) p.amax[blockIdx.x] = fmaxf(fmaxf(s_wmax[0], s_wmax[1]), fmaxf(s_wmax[2], s_wmax[3]));
  }
}

// GEMV for M <= 8 (the HBM-bound decode shapes): no MFMA. A weight row is read as
// contiguous 1 KB wave-loads (64 lanes x 16 bytes); each lane dots its 16 weight bytes
// (v_dot4_i32_i8) against the same 16 bytes of every activation row, which sit in
// registers for the whole kernel (K <= KC * 1024); one wave reduction per (row, m).
// Each wave keeps RPW rows (RPW * KC loads) in flight.
constexpr int GV_WAVES = 8;

// Wave64 integer sum, every lane active: a DPP butterfly within rows of 16 (quad_perm
// [1,0,3,2], [2,3,0,1], row_half_mirror, row_mirror), then the four row sums read out of
// lanes 0, 16, 32, 48 (no LDS permutes; integer addition is exact in any order).
__device__ __forceinline__ int wave_sum(int v) {
  v += __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false);
  v += __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false);
  v += __builtin_amdgcn_mov_dpp(v, 0x141, 0xF, 0xF, false);
  v += __builtin_amdgcn_mov_dpp(v, 0x140, 0xF, 0xF, false);
  return __builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16) + __builtin_amdgcn_readlane(v, 32) +
         __builtin_amdgcn_readlane(v, 48);
}

template <int MR, int KC, int RPW, int WAVES = GV_WAVES>
__global__ __launch_bounds__(WAVES * 64) void gemv_i8_kernel(const GemmP p) {
  constexpr int T = WAVES * 64;
  constexpr int XCH = MR * KC * 64;          // 16-byte chunks of the (padded) activation rows
  constexpr int XPT = (XCH + T - 1) / T;     // chunks a thread loads
  // The activation rows, loaded once per workgroup (not once per wave) and shared from LDS:
  // row m's chunk c (1 KB, 64 lanes x 16 bytes) at (m * KC + c) * 1024.
  __shared__ __attribute__((aligned(16))) int8_t xs[MR * KC * 1024];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int row0 = (blockIdx.x * WAVES + wave) * RPW;
  const int nrows = max(0, min(RPW, p.N - row0));  // 0 for a wave past N: all its loads are out of range
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(p.W + (size_t)min(row0, p.N) * p.K, (uint32_t)(nrows * p.K));
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.A, (uint32_t)(p.M * p.K));
  v4i xr[XPT];
#pragma unroll
  for (int i = 0; i < XPT; ++i) {
    const int ch = tid + i * T;
    const int m = ch / (KC * 64);
    const int k = (ch - m * (KC * 64)) * 16;
    xr[i] = buf_load16(ra, (ch < XCH && m < p.M && k < p.K) ? (uint32_t)(m * p.K + k) : OOB);
  }
  // Lane j*MR + m stores output (m, row0 + j); its scales and bias are fetched now, ahead
  // of the weight stream, so the tail does not wait on another memory round trip.
  const int my_j = lane / MR, my_m = lane % MR;
  const int my_n = row0 + my_j;
  const bool writer = lane < RPW * MR && my_j < nrows && my_m < p.M;
  float e_sa = 0.f, e_sw = 0.f, e_b = 0.f;
  if (writer) {
    e_sa = p.sa_per_row ? p.sA[my_m] : p.sA[0];
    e_sw = p.sW[my_n];
    e_b = p.bias ? p.bias[my_n] : 0.f;
  }
  v4i w[RPW][KC];
#pragma unroll
  for (int j = 0; j < RPW; ++j)
#pragma unroll
    for (int c = 0; c < KC; ++c) {
      const int k = c * 1024 + lane * 16;
      w[j][c] = load_nt16(rw, k < p.K ? (uint32_t)(j * p.K + k) : OOB);
    }
  __builtin_amdgcn_sched_barrier(0);  // every load of the wave in flight before anything waits
#pragma unroll
  for (int i = 0; i < XPT; ++i) {
    const int ch = tid + i * T;
    if (ch < XCH) *reinterpret_cast<v4i*>(xs + ch * 16) = xr[i];
  }
  __syncthreads();
  v4i x[MR][KC];
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int c = 0; c < KC; ++c) x[m][c] = *reinterpret_cast<const v4i*>(xs + (m * KC + c) * 1024 + lane * 16);
  int acc[RPW][MR];
#pragma unroll
  for (int j = 0; j < RPW; ++j)
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      int a = 0;
#pragma unroll
      for (int c = 0; c < KC; ++c)
#pragma unroll
        for (int q = 0; q < 4; ++q) a = __builtin_amdgcn_sdot4(w[j][c][q], x[m][c][q], a, false);
      acc[j][m] = wave_sum(a);
    }
  int mine = 0;
#pragma unroll
  for (int j = 0; j < RPW; ++j)
#pragma unroll
    for (int m = 0; m < MR; ++m)
      if (lane == j * MR + m) mine = acc[j][m];
  if (writer) {
    const size_t idx = (size_t)my_m * p.N + my_n;
    const float rv = p.res ? p.res[idx] : 0.f;
    p.out[idx] = dequant_one(mine, e_sa, e_sw, e_b, p.bias != nullptr, rv, p.res != nullptr, p.act);
    if (p.acc) p.acc[idx] = mine;
  }
}

// The same GEMV on f32 activations, their per-row quantization fused (M <= 4): every
// workgroup loads the MR rows of X (L2-resident after the first), issues its weight
// stream, then takes each row's max|x| (wave DPP maxima, then across the waves through
// LDS), its scale float32(max / 127) and the exact-quotient rounding of every element
// (Quantizer: the rule bq_quantize_rows applies, so the same bytes and scales) into the
// LDS image the dot products read, while the weight loads are in flight. One launch
// instead of the quantize kernel and the GEMV (a 4096-float row: 2.5 us of launch and
// kernel). Workgroup 0 also writes the quantized rows and scales (qx, sx, nullable).
template <int MR, int KC, int RPW, int WAVES = GV_WAVES>
__global__ __launch_bounds__(WAVES * 64) void gemv_i8_fq_kernel(const GemmP p) {
  constexpr int T = WAVES * 64;
  constexpr int XF4 = MR * KC * 256;        // float4s of the (padded) activation rows
  constexpr int XPT = (XF4 + T - 1) / T;    // float4s a thread loads
  __shared__ __attribute__((aligned(16))) int8_t xs[MR * KC * 1024];
  __shared__ float red[WAVES][MR];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int row0 = (blockIdx.x * WAVES + wave) * RPW;
  const int nrows = max(0, min(RPW, p.N - row0));
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(p.W + (size_t)min(row0, p.N) * p.K, (uint32_t)(nrows * p.K));
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(p.X, (uint32_t)(p.M * p.K * 4));
  float4 xr[XPT];
#pragma unroll
  for (int i = 0; i < XPT; ++i) {
    const int f = tid + i * T;
    const int m = f / (KC * 256);
    const int k = (f - m * (KC * 256)) * 4;
    xr[i] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
                                           rx, (f < XF4 && m < p.M && k < p.K) ? (uint32_t)((m * p.K + k) * 4) : OOB, 0, 0));
  }
  const int my_j = lane / MR, my_m = lane % MR;
  const int my_n = row0 + my_j;
  const bool writer = lane < RPW * MR && my_j < nrows && my_m < p.M;
  float e_sw = 0.f, e_b = 0.f;
  if (writer) {
    e_sw = p.sW[my_n];
    e_b = p.bias ? p.bias[my_n] : 0.f;
  }
  v4i w[RPW][KC];
#pragma unroll
  for (int j = 0; j < RPW; ++j)
#pragma unroll
    for (int c = 0; c < KC; ++c) {
      const int k = c * 1024 + lane * 16;
      w[j][c] = load_nt16(rw, k < p.K ? (uint32_t)(j * p.K + k) : OOB);
    }
  __builtin_amdgcn_sched_barrier(0);  // every load in flight before anything waits
  // row maxima (the padding and rows past M read as zeros)
  float pm[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) pm[m] = 0.f;
#pragma unroll
  for (int i = 0; i < XPT; ++i) {
    const int m = (tid + i * T) / (KC * 256);
    const float4 v = xr[i];
    const float a = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
#pragma unroll
    for (int mm = 0; mm < MR; ++mm)
      if (mm == m) pm[mm] = fmaxf(pm[mm], a);
  }
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    const float v = wave_max(pm[m]);
    if (lane == 0) red[wave][m] = v;
  }
  __syncthreads();
  float sc[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    float v = red[0][m];
#pragma unroll
    for (int wv = 1; wv < WAVES; ++wv) v = fmaxf(v, red[wv][m]);
    sc[m] = scale_of(v);
  }
  // one reciprocal per row's scale, not per element group
  Quantizer qz[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) qz[m] = Quantizer(sc[m]);
#pragma unroll
  for (int i = 0; i < XPT; ++i) {
    const int f = tid + i * T;
    if (f < XF4) {
      const int m = f / (KC * 256);
      const int k = (f - m * (KC * 256)) * 4;
      Quantizer q0 = qz[0];
#pragma unroll
      for (int mm = 1; mm < MR; ++mm)
        if (mm == m) q0 = qz[mm];
      const uint32_t packed = q0.pack(xr[i]);
      *reinterpret_cast<uint32_t*>(xs + m * (KC * 1024) + k) = packed;
      if (blockIdx.x == 0 && p.qx && m < p.M && k < p.K) *reinterpret_cast<uint32_t*>(p.qx + (size_t)m * p.K + k) = packed;
    }
  }
  if (blockIdx.x == 0 && p.sx && tid < p.M && tid < MR) {
    float smm = sc[0];
#pragma unroll
    for (int mm = 1; mm < MR; ++mm)
      if (mm == tid) smm = sc[mm];
    p.sx[tid] = smm;
  }
  __syncthreads();
  float e_sa = sc[0];
#pragma unroll
  for (int mm = 1; mm < MR; ++mm)
    if (mm == my_m) e_sa = sc[mm];
  v4i x[MR][KC];
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int c = 0; c < KC; ++c) x[m][c] = *reinterpret_cast<const v4i*>(xs + (m * KC + c) * 1024 + lane * 16);
  int acc[RPW][MR];
#pragma unroll
  for (int j = 0; j < RPW; ++j)
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      int a = 0;
#pragma unroll
      for (int c = 0; c < KC; ++c)
#pragma unroll
        for (int q = 0; q < 4; ++q) a = __builtin_amdgcn_sdot4(w[j][c][q], x[m][c][q], a, false);
      acc[j][m] = wave_sum(a);
    }
  int mine = 0;
#pragma unroll
  for (int j = 0; j < RPW; ++j)
#pragma unroll
    for (int m = 0; m < MR; ++m)
      if (lane == j * MR + m) mine = acc[j][m];
  if (writer) {
    const size_t idx = (size_t)my_m * p.N + my_n;
    const float rv = p.res ? p.res[idx] : 0.f;
    p.out[idx] = dequant_one(mine, e_sa, e_sw, e_b, p.bias != nullptr, rv, p.res != nullptr, p.act);
    if (p.acc) p.acc[idx] = mine;
  }
}

template <int MR, int RPW, int WAVES>
static bool launch_gemv_fq_cfg(const GemmP& p, hipStream_t st) {
  const unsigned grid = (unsigned)((p.N + WAVES * RPW - 1) / (WAVES * RPW));
  if (p.K <= 1024) gemv_i8_fq_kernel<MR, 1, RPW, WAVES><<<grid, WAVES * 64, 0, st>>>(p);
  else if (p.K <= 2048) gemv_i8_fq_kernel<MR, 2, RPW, WAVES><<<grid, WAVES * 64, 0, st>>>(p);
  else if (p.K <= 4096) gemv_i8_fq_kernel<MR, 4, RPW, WAVES><<<grid, WAVES * 64, 0, st>>>(p);
  else if (p.K <= 8192) gemv_i8_fq_kernel<MR, 8, RPW, WAVES><<<grid, WAVES * 64, 0, st>>>(p);
  else return false;
  return true;
}

// Eight waves a workgroup (the f32 rows are loaded and quantized once per workgroup, so
// more weight rows a workgroup spend less of the L2 -> CU traffic on them): one weight row
// a wave for one activation row, two for two to four. Measured, 4096 x 4096, cache-cold,
// one launch against quantize + GEMV: M = 1 5.37 against 7.75 us, M = 2 6.6 against 8.0,
// M = 4 8.4 against 8.4 (four waves a workgroup: 6.1 / 8.3 / 10.1 us).
template <int MR>
static bool launch_gemv_fq(const GemmP& p, hipStream_t st) {
  if constexpr (MR == 1) return launch_gemv_fq_cfg<MR, 1, 8>(p, st);
  else return launch_gemv_fq_cfg<MR, 2, 8>(p, st);
}

template <int MR, int RPW, int WAVES>
static bool launch_gemv_cfg(const GemmP& p, hipStream_t st) {
  const unsigned grid = (unsigned)((p.N + WAVES * RPW - 1) / (WAVES * RPW));
  if (p.K <= 1024) gemv_i8_kernel<MR, 1, RPW, WAVES><<<grid, WAVES * 64, 0, st>>>(p);
  else if (p.K <= 2048) gemv_i8_kernel<MR, 2, RPW, WAVES><<<grid, WAVES * 64, 0, st>>>(p);
  else if (p.K <= 4096) gemv_i8_kernel<MR, 4, RPW, WAVES><<<grid, WAVES * 64, 0, st>>>(p);
  else if (p.K <= 8192) gemv_i8_kernel<MR, 8, RPW, WAVES><<<grid, WAVES * 64, 0, st>>>(p);
  else return false;
  return true;
}

// One weight row per wave (the most rows in flight per byte of activation); four waves a
// workgroup for one or two activation rows, eight for three or more (measured). From five
// rows the activations held in registers (MR * KC * 4 VGPRs) limit K to 4096.
template <int MR>
static bool launch_gemv(const GemmP& p, hipStream_t st) {
  if constexpr (MR > 4) {
    if (p.K > 4096) return false;
  }
  if constexpr (MR <= 2) return launch_gemv_cfg<MR, 1, 4>(p, st);
  else return launch_gemv_cfg<MR, 1, 8>(p, st);
}

// The wave-reduction GEMV for 1..8 activation rows; false where it does not apply.
static bool launch_gemv_rows(const GemmP& p, hipStream_t st) {
  switch (p.M) {
    case 1: return launch_gemv<1>(p, st);
    case 2: return launch_gemv<2>(p, st);
    case 3: return launch_gemv<3>(p, st);
    case 4: return launch_gemv<4>(p, st);
    case 5: return launch_gemv<5>(p, st);
    case 6: return launch_gemv<6>(p, st);
    case 7: return launch_gemv<7>(p, st);
    case 8: return launch_gemv<8>(p, st);
    default: return false;
  }
}

// ---------------------------------------------------------------------------- dispatch

// Split-K workspace: the tile counters first (SPLIT_CNT_BYTES), the int32 partial tiles
// after. Splitting is offered to tiles of at most SPLIT_MAX_TILE outputs, and only when the
// grid has fewer than SPLIT_MAX_TILES tiles; with S <= ceil(256 / tiles) the partials take
// at most (256 + SPLIT_MAX_TILES) tiles' worth, which bounds the workspace for every shape.
constexpr int SPLIT_MAX_TILES = 160;
constexpr size_t SPLIT_CNT_BYTES = 4096;
constexpr size_t SPLIT_WS_BYTES = SPLIT_CNT_BYTES + (size_t)(256 + SPLIT_MAX_TILES) * SPLIT_MAX_TILE * 4;

struct Ws {
  void* ptr;
  size_t bytes;
};

// K splits for a grid of `tiles` tiles of `KT` stages: enough workgroups to cover the
// chip's 256 CUs, each split at least 4 stages long, and no split left empty. The split
// costs a fixed 2-3 us (partials written through to the device-coherent level, the counter
// round trip, the last workgroup's reads); measured on 64x64 tiles it pays from 16 stages
// for a conv (whose loader makes a stage dearer) and from 32 for a dense GEMM.
static int pick_split(long long tiles, int KT, bool conv, int planned = 0) {
  int S;
  if (planned > 0) {
    S = planned;
  } else {
    if (tiles >= SPLIT_MAX_TILES || KT < (conv ? 16 : 32)) return 1;
    S = (int)std::min<long long>((256 + tiles - 1) / tiles, KT / 4);
  }
  S = std::max(1, std::min(S, KT));
  const int per = (KT + S - 1) / S;
  return (KT + per - 1) / per;
}

// The K split of p on BM x BN tiles (the plan's, else the rule's; 1 when the workspace cannot
// hold it), recorded in p with the workspace's counters and partials; returns the workgroups.
template <int BM, int BN, bool CONV>
static long long setup_split(GemmP& p, const Ws& ws) {
  const long long tiles = (long long)((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN);
  int S = BM * BN <= SPLIT_MAX_TILE ? pick_split(tiles, (p.K + BK - 1) / BK, CONV, p.plan_split) : 1;
  if (S > 1) {
    const size_t need = SPLIT_CNT_BYTES + (size_t)tiles * S * BM * BN * 4;
    if (!ws.ptr || ws.bytes < need || tiles * 4 > (long long)SPLIT_CNT_BYTES || tiles * S > 0x7fffffffll) {
      S = 1;
    } else {
      p.cnt = static_cast<int*>(ws.ptr);
      p.part = reinterpret_cast<int32_t*>(static_cast<char*>(ws.ptr) + SPLIT_CNT_BYTES);
    }
  }
  p.ksplit = S;
  return tiles * S;
}

template <int BM, int BN, int WAVES_M, int WAVES_N, bool CONV, int NBUF, int FD, bool MF16 = false>
static void launch_tiled(GemmP p, hipStream_t st, const Ws& ws) {
  const long long groups = setup_split<BM, BN, CONV>(p, ws);
  gemm_i8_kernel<BM, BN, WAVES_M, WAVES_N, CONV, NBUF, FD, MF16><<<(unsigned)groups, WAVES_M * WAVES_N * 64, 0, st>>>(p);
}

// p0 and p1 in one launch on p0's configuration; p1 runs unsplit. False (nothing launched)
// when the grid would not fit one launch.
template <int BM, int BN, int WAVES_M, int WAVES_N, bool CONV, int NBUF, int FD>
static bool launch_pair_tiled(GemmP p0, GemmP p1, hipStream_t st, const Ws& ws) {
  const long long g0 = setup_split<BM, BN, CONV>(p0, ws);
  p1.ksplit = 1;
  const long long g1 = (long long)((p1.M + BM - 1) / BM) * ((p1.N + BN - 1) / BN);
  if (g0 + g1 > 0x7fffffffll) return false;
  gemm_i8_pair_kernel<BM, BN, WAVES_M, WAVES_N, CONV, NBUF, FD>
      <<<(unsigned)(g0 + g1), WAVES_M * WAVES_N * 64, 0, st>>>(p0, p1, (int)g0);
  return true;
}

// Tiled-kernel configurations, by id: <BM, BN, waves M x N, ring depth, fragment distance>.
//   1 <256,256,2,4,2,1>  2 <256,256,2,4,2,2>  3 <256,256,2,2,2,2>  4 <128,128,2,2,4,2>
//   5 <128,128,2,2,2,2>  6 <256,128,2,2,3,1>  7 <64,64,2,2,4,2>    8 <256,64,4,1,3,1>
//   9 <64,64,2,2,8,1>   10 <64,64,2,2,2,2>   11 <128,64,4,1,2,1>  12 <128,32,4,1,2,1>
//  13 <256,64,4,1,2,1>  14 <128,64,4,1,3,1>
//  15 <256,256,2,4,2,1> on 16x16x64 MFMAs (the same form measured 4-13% slower than 5 and
//     6 on 128x128 and 256x128 tiles, so those stay on 32x32x32)
//  16 <320,256,2,4,2,1> dense only: 160x64 wave tiles (256 VGPRs; the 16x16 form would spill),
//     for grids that take two rounds of 256x256 tiles but one of 320x256
//  17 <128,256,2,4,2,2> 8 waves of 64x64, for grids of more than one round of 128x128 tiles
//     but one of 128x256 (ViT-B/16 b32's proj and fc2, N = 768: 6-8% faster than 128x128)
// Ids 3 and 9 never won a measurement: neither the rule nor a plan selects them, and their
// kernels are not built (the id numbering stays, for stored plans).
struct TileDims {
  int bm, bn;
};
constexpr int NCFG = 18;  // tiled ids 1 .. NCFG - 1
constexpr int CFG_SMALLK = BQ_CFG_SMALLK;  // smallk_i8_kernel (dense)
static_assert(CFG_SMALLK == NCFG, "the small-K kernel's id follows the tiled ids");
constexpr TileDims CFG_TILES[NCFG] = {{0, 0},    {256, 256}, {256, 256}, {256, 256}, {128, 128}, {128, 128},
                                      {256, 128}, {64, 64},   {256, 64},  {64, 64},   {64, 64},   {128, 64},
                                      {128, 32},  {256, 64},  {128, 64},  {256, 256}, {320, 256}, {128, 256}};

// The configuration the tiled kernel runs for M x N x K. Narrow outputs (N <= 64: 1x1 convs
// of mobile networks, the stem, early ResNet layers) take small-LDS tiles that fit several
// workgroups per CU (measured 2-2.5x over a 256x64 tile at K <= 240 and 5-15% at
// K = 2304-4096). Otherwise the largest tile that still fills the chip (>= 192 / 128
// workgroups; a dense 256x256 grid from 150) without wasting most of its columns; a dense
// grid that would need a second round of 256x256 tiles but fits one round of 320x256 takes
// those (ViT-B/16 b32's fc1, 6304x3072x768: 36.5 -> 26.9 us; at 156 tiles the 256x256 tile
// beat 128x128 by 15%, at 117 it lost by 20%); likewise a dense grid of more than one round
// of 128x128 tiles that fits one round of 128x256 (8 waves). Ring depth: deep rings keep several
// stages of a small tile's operands in flight; when there are more tiles than CUs, a small
// tile takes the 2-deep ring instead so that several workgroups share a CU. The 256x256
// tile's 64 KB stages leave room for two buffers only. Small tiles read their fragments two
// K slices ahead (short MFMA runs). The dense 256x256 tile runs on 16x16x64 MFMAs, which
// sustain a higher rate than 32x32x32 at the power limit (4096^3: 67-69 against 73-75 us);
// its convolution form keeps 32x32x32, which needs fewer fragment registers next to the
// implicit-GEMM addressing (the 16x16 form spills there).
// Whether the small-K kernel takes a problem (its shape only: an unaligned output takes
// its four-byte stores), and its grid.
static bool smallk_ok(const GemmP& p, bool conv) {
  const int NB = (p.N + 15) / 16, KS = (p.K + 63) / 64;
  return !p.stamps && p.M >= 1 && p.N >= 4 && p.N <= 256 && p.N % 4 == 0 && p.K <= 256 && NB * KS <= 16 &&
         (long long)p.M * p.N * 4 < (1ll << 31) && (conv || (long long)p.M * p.K < (1ll << 31));
}
static int smallk_grid(const GemmP& p) {  // by measurement on EfficientNet-B0 b64's shapes
  const long long steps = (p.M + SMALLK_ROWS - 1) / SMALLK_ROWS;
  return (int)std::min<long long>(steps, p.N >= 64 ? 4096 : steps >= 8192 ? 2048 : 1024);
}

static int choose_cfg(const GemmP& p, bool conv) {
  if (p.plan_cfg == CFG_SMALLK) {
    if (smallk_ok(p, conv)) return CFG_SMALLK;
  } else if (p.plan_cfg >= 1 && p.plan_cfg < NCFG) {
    return p.plan_cfg;
  }
  // A narrow output over many rows (a 1x1 projection or expansion, a stem conv): the small-K
  // kernel (EfficientNet-B0 b64 against the best tiled configuration, each layer alone with
  // fresh outputs: 802816 x 16 x 32 34.2 -> 10.7 us, 802816 x 96 x 16 88.2 -> 75.7 us,
  // 200704 x 144 x 32 37.9 -> 29.4 us, 200704 x 24 x 96 11.8 -> 8.5 us), and for a
  // calibrated layer's int8 twin alone, whose rows it stores whole (802816 x 96 x 16: 74.8
  // against 108 us). From 65,536 rows it also takes up to 160 columns for the twin alone, and
  // for an f32 output at most 32 or at least 128 columns (100352 x 144 x 32: twin 21.3 / f32
  // 23.4 against 35.7 / 29.7 us, 100352 x 24 x 96 f32 6.9 against 8.3 us; at 96 columns the
  // tiled kernel's f32 output stays faster below 131,072 rows: 100352 x 96 x 16 16.6 against
  // 17.3 us).
  const bool twin_only = p.q_out && !p.out;
  if (smallk_ok(p, conv) &&
      (p.M >= 131072 || (p.M >= 65536 && p.N <= 160 && (twin_only || p.N <= 32 || p.N >= 128))))
    return CFG_SMALLK;
  const long long t256 = (long long)((p.M + 255) / 256) * ((p.N + 255) / 256);
  const long long t128 = (long long)((p.M + 127) / 128) * ((p.N + 127) / 128);
  const long long t128x32 = (long long)((p.M + 127) / 128) * ((p.N + 31) / 32);
  const long long t64 = (long long)((p.M + 63) / 64) * ((p.N + 63) / 64);
  const long long t320 = (long long)((p.M + 319) / 320) * ((p.N + 255) / 256);
  if (p.N <= 32 && t128x32 >= 128) return 12;
  if (p.N <= 64 && t64 > 256) return 10;
  if (!conv && t256 > 256 && t320 <= 256 && p.N >= 192) return 16;
  if (t256 >= (conv ? 192 : 150) && p.N >= 192) return conv ? 1 : 15;
  const long long t128x256 = (long long)((p.M + 127) / 128) * ((p.N + 255) / 256);
  if (!conv && t128 > 256 && t128x256 <= 256 && p.N >= 512) return 17;
  if (t128 >= 128 && p.N >= 96) return t128 > 256 ? 5 : 4;
  return 7;
}

// Output tiles of the tiled kernel for this problem (the length of its absmax output).
static long long out_tiles(const GemmP& p, bool conv) {
  const int cfg = choose_cfg(p, conv);
  if (cfg == CFG_SMALLK) return smallk_grid(p);  // one maximum a workgroup
  const TileDims d = CFG_TILES[cfg];
  return (long long)((p.M + d.bm - 1) / d.bm) * ((p.N + d.bn - 1) / d.bn);
}

template <bool CONV>
static void launch_smallk(const GemmP& p, hipStream_t st) {
  const dim3 grid((unsigned)smallk_grid(p));
  const int NB = (p.N + 15) / 16, KS = (p.K + 63) / 64;
  switch ((NB - 1) * 4 + (KS - 1)) {  // NB * KS <= 16 (smallk_ok)
#define BQ_SMALLK(nb, ks) \
  case (nb - 1) * 4 + (ks - 1): smallk_i8_kernel<nb, ks, CONV><<<grid, 256, 0, st>>>(p); break;
    BQ_SMALLK(1, 1) BQ_SMALLK(1, 2) BQ_SMALLK(1, 3) BQ_SMALLK(1, 4)
    BQ_SMALLK(2, 1) BQ_SMALLK(2, 2) BQ_SMALLK(2, 3) BQ_SMALLK(2, 4)
    BQ_SMALLK(3, 1) BQ_SMALLK(3, 2) BQ_SMALLK(3, 3) BQ_SMALLK(3, 4)
    BQ_SMALLK(4, 1) BQ_SMALLK(4, 2) BQ_SMALLK(4, 3) BQ_SMALLK(4, 4)
    BQ_SMALLK(5, 1) BQ_SMALLK(5, 2) BQ_SMALLK(5, 3)
    BQ_SMALLK(6, 1) BQ_SMALLK(6, 2)
    BQ_SMALLK(7, 1) BQ_SMALLK(7, 2)
    BQ_SMALLK(8, 1) BQ_SMALLK(8, 2)
    BQ_SMALLK(9, 1) BQ_SMALLK(10, 1) BQ_SMALLK(11, 1) BQ_SMALLK(12, 1) BQ_SMALLK(13, 1) BQ_SMALLK(14, 1)
    BQ_SMALLK(15, 1) BQ_SMALLK(16, 1)
#undef BQ_SMALLK
  }
}

// The small-K conv on an f32 NCHW input: up to 4 column blocks, 4 or 8 input channels a tap.
template <int CINM>
static void launch_smallk_f32in(const GemmP& p, hipStream_t st) {
  const dim3 grid((unsigned)smallk_grid(p));
  const int NB = (p.N + 15) / 16, KS = (p.K + 63) / 64;
  switch ((NB - 1) * 4 + (KS - 1)) {
#define BQ_SMALLK(nb, ks) \
  case (nb - 1) * 4 + (ks - 1): smallk_i8_kernel<nb, ks, true, CINM><<<grid, 256, 0, st>>>(p); break;
    BQ_SMALLK(1, 1) BQ_SMALLK(1, 2) BQ_SMALLK(1, 3) BQ_SMALLK(1, 4)
    BQ_SMALLK(2, 1) BQ_SMALLK(2, 2) BQ_SMALLK(2, 3) BQ_SMALLK(2, 4)
    BQ_SMALLK(3, 1) BQ_SMALLK(3, 2) BQ_SMALLK(3, 3) BQ_SMALLK(3, 4)
    BQ_SMALLK(4, 1) BQ_SMALLK(4, 2) BQ_SMALLK(4, 3) BQ_SMALLK(4, 4)
#undef BQ_SMALLK
  }
}

template <bool CONV>
static void launch_gemm(const GemmP& p, hipStream_t st, const Ws& ws) {
  switch (choose_cfg(p, CONV)) {
    case 1: return launch_tiled<256, 256, 2, 4, CONV, 2, 1>(p, st, ws);
    case 2: return launch_tiled<256, 256, 2, 4, CONV, 2, 2>(p, st, ws);
    case 4: return launch_tiled<128, 128, 2, 2, CONV, 4, 2>(p, st, ws);
    case 5: return launch_tiled<128, 128, 2, 2, CONV, 2, 2>(p, st, ws);
    case 6: return launch_tiled<256, 128, 2, 2, CONV, 3, 1>(p, st, ws);
    case 8: return launch_tiled<256, 64, 4, 1, CONV, 3, 1>(p, st, ws);
    case 10: return launch_tiled<64, 64, 2, 2, CONV, 2, 2>(p, st, ws);
    case 11: return launch_tiled<128, 64, 4, 1, CONV, 2, 1>(p, st, ws);
    case 12: return launch_tiled<128, 32, 4, 1, CONV, 2, 1>(p, st, ws);
    case 13: return launch_tiled<256, 64, 4, 1, CONV, 2, 1>(p, st, ws);
    case 14: return launch_tiled<128, 64, 4, 1, CONV, 3, 1>(p, st, ws);
    case 15: return launch_tiled<256, 256, 2, 4, CONV, 2, 1, true>(p, st, ws);
    case 17: return launch_tiled<128, 256, 2, 4, CONV, 2, 2>(p, st, ws);
    case 16:  // dense only (the implicit-GEMM loader does not fit beside its 160 accumulators)
      if constexpr (!CONV) return launch_tiled<320, 256, 2, 4, CONV, 2, 1>(p, st, ws);
      [[fallthrough]];
    case CFG_SMALLK: return launch_smallk<CONV>(p, st);
    default: return launch_tiled<64, 64, 2, 2, CONV, 4, 2>(p, st, ws);
  }
}

// Two implicit-GEMM convs in one launch on the configuration the first would run (the
// small-tile configurations only: the deep K of a residual block's first conv is split, and
// its shortcut's grid fills the rest of the chip). False: not offered for that configuration.
static bool launch_conv_pair(const GemmP& p0, const GemmP& p1, hipStream_t st, const Ws& ws) {
  switch (choose_cfg(p0, true)) {
    case 7: return launch_pair_tiled<64, 64, 2, 2, true, 4, 2>(p0, p1, st, ws);
    case 10: return launch_pair_tiled<64, 64, 2, 2, true, 2, 2>(p0, p1, st, ws);
    case 11: return launch_pair_tiled<128, 64, 4, 1, true, 2, 1>(p0, p1, st, ws);
    case 12: return launch_pair_tiled<128, 32, 4, 1, true, 2, 1>(p0, p1, st, ws);
    case 14: return launch_pair_tiled<128, 64, 4, 1, true, 3, 1>(p0, p1, st, ws);
    default: return false;
  }
}

static bool aligned16(const void* q) { return ((uintptr_t)q & 15) == 0; }

// ---------------------------------------------------------------- kernel choice by measurement
//
// A plan fixes, for one problem, the tiled kernel's configuration and K split that the
// rules above would otherwise pick. Every configuration and split computes the same exact
// int32 sums and the same epilogue, so a plan changes time only, never a result. Problems
// are keyed by their full geometry: a dense GEMM (0, M, N, K) or a convolution (1, N, H, W,
// C, O, KH, KW, stride, pad). The host tuner times the candidates (bq_plan_candidates, the
// rules' pick first) and records the fastest (bq_plan_set).
using PlanKey = std::array<int64_t, 10>;
struct Plan {
  int cfg, split;
};
static std::mutex g_plan_mu;
static std::map<PlanKey, Plan> g_plans;

static PlanKey dense_key(int64_t M, int64_t N, int64_t K) { return PlanKey{0, M, N, K, 0, 0, 0, 0, 0, 0}; }
static PlanKey conv_key(int64_t N, int64_t H, int64_t W, int64_t C, int64_t O, int64_t KH, int64_t KW,
                        int64_t stride, int64_t pad) {
  return PlanKey{1, N, H, W, C, O, KH, KW, stride, pad};
}

static void apply_plan(GemmP& p, const PlanKey& k) {
  std::lock_guard<std::mutex> lock(g_plan_mu);
  if (g_plans.empty()) return;
  const auto it = g_plans.find(k);
  if (it != g_plans.end()) {
    p.plan_cfg = it->second.cfg;
    p.plan_split = it->second.split;
  }
}

// Dense problems of at most DECODE_MAX_M rows choose between the two decode kernels
// (BQ_CFG_GEMV, BQ_CFG_SKINNY); the rule takes the GEMV up to GEMV_RULE_M rows where it
// takes K. Measured on the 4096 x 4096 weight, cache-cold, both with non-temporal weight
// loads: GEMV / skinny 4.88 / 6.28 us at M = 1, 5.38 / 6.66 at 4, 5.81 / 6.55 at 5, 6.10 /
// 6.63 at 6, 6.40 / 6.71 at 7, 6.12 / 6.76 at 8.
constexpr int DECODE_MAX_M = 8;
constexpr int GEMV_RULE_M = 8;

// The GEMM view of a problem given as (M, N, K) or (N, H, W, C, O, KH, KW, stride, pad);
// false for a bad geometry. `tiled`: whether the tiled kernel runs it (a dense GEMM of at
// most 64 rows takes the GEMV / skinny kernels: nothing to choose).
static bool problem_view(const int64_t* pr, int n, PlanKey& key, GemmP& p, bool& conv, bool& tiled) {
  if (!pr) return false;
  p = GemmP{};
  if (n == 3) {
    const int64_t M = pr[0], N = pr[1], K = pr[2];
    if (M < 1 || N < 1 || K < 16 || K % 16 || M > 0x7fffffff || N > 0x7fffffff || K > KMAX_EXACT) return false;
    key = dense_key(M, N, K);
    p.M = (int)M; p.N = (int)N; p.K = (int)K;
    conv = false;
    tiled = M > 64;
    return true;
  }
  if (n != 9) return false;
  const int64_t N = pr[0], H = pr[1], W = pr[2], C = pr[3], O = pr[4], KH = pr[5], KW = pr[6], st = pr[7], pad = pr[8];
  if (N < 1 || H < 1 || W < 1 || C < 16 || C % 16 || O < 1 || KH < 1 || KW < 1 || st < 1 || pad < 0 ||
      H + 2 * pad < KH || W + 2 * pad < KW)
    return false;
  const int64_t OH = (H + 2 * pad - KH) / st + 1, OW = (W + 2 * pad - KW) / st + 1;
  const int64_t M = N * OH * OW, K = KH * KW * C;
  if (M > 0x7fffffff || O > 0x7fffffff || K > KMAX_EXACT) return false;
  key = conv_key(N, H, W, C, O, KH, KW, st, pad);
  p.M = (int)M; p.N = (int)O; p.K = (int)K;
  conv = !(KH == 1 && KW == 1 && st == 1 && pad == 0);  // a 1x1 conv runs the dense loader
  tiled = true;
  return true;
}

// The K split configuration `cfg` runs for this problem with a full-size workspace.
static int split_of(const GemmP& p, int cfg, bool conv, int planned) {
  const TileDims d = CFG_TILES[cfg];
  if (d.bm * d.bn > SPLIT_MAX_TILE) return 1;
  const long long tiles = (long long)((p.M + d.bm - 1) / d.bm) * ((p.N + d.bn - 1) / d.bn);
  const int S = pick_split(tiles, (p.K + BK - 1) / BK, conv, planned);
  const size_t need = SPLIT_CNT_BYTES + (size_t)tiles * S * d.bm * d.bn * 4;
  return (S > 1 && (need > SPLIT_WS_BYTES || tiles * 4 > (long long)SPLIT_CNT_BYTES)) ? 1 : S;
}

// The split-K workspace of bq_gemm_i8_noalloc: SPLIT_WS_BYTES of the library's own device
// memory, one copy on every GPU the library runs on, held until the process ends. In host
// code `scratch` names a host-side stand-in, never the device memory: the device address
// of each GPU's copy comes from hipGetSymbolAddress with that GPU current, and only that
// address is passed to kernels.
static __device__ __align__(256) unsigned char scratch[SPLIT_WS_BYTES];

constexpr int SCRATCH_MAX_DEVICES = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[SCRATCH_MAX_DEVICES];  // per device ordinal; null until set up

// The scratch address of the device `st` belongs to (not the calling thread's current
// device), set up on that device's first call: the symbol's address looked up once, with
// that device current. A static __device__ array is zero when the code object is loaded,
// so the tile counters (the part that must start at zero) need no clearing launch, and
// every split launch leaves them zero again.
static int noalloc_scratch(const char* what, hipStream_t st, void** out) {
  int dev = -1;
  hipError_t e = hipStreamGetDevice(st, &dev);
  if (e != hipSuccess) return set_error(BQ_ERR_DEVICE, "%s: hipStreamGetDevice: %s", what, hipGetErrorString(e));
  if (dev < 0 || dev >= SCRATCH_MAX_DEVICES)
    return set_error(BQ_ERR_DEVICE, "%s: device %d beyond the %d this library keeps scratch for", what, dev,
                     SCRATCH_MAX_DEVICES);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    int cur = -1;
    e = hipGetDevice(&cur);
    if (e != hipSuccess) return set_error(BQ_ERR_DEVICE, "%s: hipGetDevice: %s", what, hipGetErrorString(e));
    if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess)
      return set_error(BQ_ERR_DEVICE, "%s: hipSetDevice(%d): %s", what, dev, hipGetErrorString(e));
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (cur != dev) (void)hipSetDevice(cur);  // restoring what was current a moment ago
    if (e != hipSuccess || !ptr)
      return set_error(BQ_ERR_DEVICE, "%s: hipGetSymbolAddress(scratch): %s", what, hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return BQ_OK;
}

static int gemm_impl(const char* what, const int8_t* A, const int8_t* W, int64_t M, int64_t N, int64_t K,
                     const float* sA, const float* sW, const float* bias, const float* residual, int act,
                     float* out, int32_t* acc, void* ws, size_t ws_bytes, bool noalloc, bq_stream_t stream,
                     uint64_t* stamps = nullptr, int64_t stamps_cap = 0, int64_t* stamped = nullptr) {
  if (M < 0 || N < 0 || K < 0) return set_error(BQ_ERR_ARG, "%s: negative size", what);
  if (M > 0x7fffffff || N > 0x7fffffff || M * N > ((int64_t)1 << 40))
    return set_error(BQ_ERR_ARG, "%s: size too large", what);
  if (K > KMAX_EXACT)
    return set_error(BQ_ERR_UNSUPPORTED, "%s: K=%lld > %d: int32 accumulators could overflow", what, (long long)K,
                     KMAX_EXACT);
  if (M == 0 || N == 0) return BQ_OK;
  if (K % 16) return set_error(BQ_ERR_UNSUPPORTED, "%s: K=%lld is not a multiple of 16", what, (long long)K);
  if (!A || !W || !sA || !sW || !out) return set_error(BQ_ERR_ARG, "%s: null pointer", what);
  if (!aligned16(A) || !aligned16(W)) return set_error(BQ_ERR_ARG, "%s: A and W must be 16-byte aligned", what);
  const bool sa_per_tensor = (act & BQ_SCALE_A_PER_TENSOR) != 0;
  act &= ~BQ_SCALE_A_PER_TENSOR;
  if (act < BQ_ACT_NONE || act > BQ_ACT_GELU) return set_error(BQ_ERR_ARG, "%s: bad activation %d", what, act);
  GemmP p{};
  p.A = A; p.W = W; p.M = (int)M; p.N = (int)N; p.K = (int)K;
  p.sA = sA; p.sa_per_row = sa_per_tensor ? 0 : 1; p.sW = sW; p.bias = bias; p.res = residual; p.act = act;
  p.out = out; p.acc = acc;
  p.vec_ok = (N % 4 == 0) && aligned16(out) && aligned16(acc) && aligned16(residual);
  hipStream_t st = (hipStream_t)stream;
  if (stamps) {  // diagnostics: the tiled kernel, unsplit, one stamped workgroup a tile
    if (M <= 64) return set_error(BQ_ERR_UNSUPPORTED, "%s: phase stamps cover the tiled kernel (M > 64)", what);
    apply_plan(p, dense_key(M, N, K));
    const long long tiles = out_tiles(p, false);
    if (4 * tiles > stamps_cap)
      return set_error(BQ_ERR_ARG, "%s: %lld workgroups need %lld stamp words, %lld given", what, tiles, 4 * tiles,
                       (long long)stamps_cap);
    p.stamps = stamps;
    *stamped = tiles;
    launch_gemm<false>(p, st, Ws{nullptr, 0});
    return check_launch(what);
  }
  bool done = false;
  if (M <= DECODE_MAX_M) {
    // the decode shapes: the wave-reduction GEMV up to GEMV_RULE_M rows, the weight-streaming
    // MFMA kernel above; a plan may pick either for up to DECODE_MAX_M rows
    apply_plan(p, dense_key(M, N, K));
    bool gemv = M <= GEMV_RULE_M;
    if (p.plan_cfg == BQ_CFG_GEMV) gemv = true;
    else if (p.plan_cfg == BQ_CFG_SKINNY) gemv = false;
    if (gemv) done = launch_gemv_rows(p, st);
  }
  if (done) {
  } else if (M <= 64) {
    const unsigned grid = (unsigned)((N + SK_COLS - 1) / SK_COLS);
    switch ((M + 15) / 16) {
      case 1: skinny_i8_kernel<1, 8, 2><<<grid, 8 * 64, 0, st>>>(p); break;
      case 2: skinny_i8_kernel<2, 8, 2><<<grid, 8 * 64, 0, st>>>(p); break;
      case 3: skinny_i8_kernel<3, 8, 1><<<grid, 8 * 64, 0, st>>>(p); break;
      default: skinny_i8_kernel<4, 8, 1><<<grid, 8 * 64, 0, st>>>(p); break;
    }
  } else {
    if (noalloc) {
      const int rc = noalloc_scratch(what, st, &ws);
      if (rc != BQ_OK) return rc;
      ws_bytes = SPLIT_WS_BYTES;
    }
    apply_plan(p, dense_key(M, N, K));
    launch_gemm<false>(p, st, Ws{ws, ws_bytes});
  }
  return check_launch(what);
}

}  // namespace bq

using namespace bq;

extern "C" {

size_t bq_gemm_ws_bytes(void) { return SPLIT_WS_BYTES; }

int bq_gemm_i8(const int8_t* A, const int8_t* W, int64_t M, int64_t N, int64_t K, const float* sA,
               const float* sW, const float* bias, const float* residual, int act, float* out, int32_t* acc,
               void* ws, size_t ws_bytes, bq_stream_t stream) {
  return gemm_impl("bq_gemm_i8", A, W, M, N, K, sA, sW, bias, residual, act, out, acc, ws, ws_bytes, false,
                   stream);
}

int64_t bq_gemm_i8_phases(const int8_t* A, const int8_t* W, int64_t M, int64_t N, int64_t K, const float* sA,
                          const float* sW, const float* bias, float* out, uint64_t* stamps, int64_t stamps_cap,
                          bq_stream_t stream) {
  if (!stamps) return set_error(BQ_ERR_ARG, "bq_gemm_i8_phases: null stamps");
  int64_t n = 0;
  const int rc = gemm_impl("bq_gemm_i8_phases", A, W, M, N, K, sA, sW, bias, nullptr, BQ_ACT_NONE, out, nullptr,
                           nullptr, 0, false, stream, stamps, stamps_cap, &n);
  return rc != BQ_OK ? rc : n;
}

int bq_gemm_i8_noalloc(const int8_t* A, const int8_t* W, int64_t M, int64_t N, int64_t K, const float* sA,
                       const float* sW, const float* bias, const float* residual, int act, float* out,
                       int32_t* acc, bq_stream_t stream) {
  return gemm_impl("bq_gemm_i8_noalloc", A, W, M, N, K, sA, sW, bias, residual, act, out, acc, nullptr, 0, true,
                   stream);
}

int bq_linear_i8(const float* x, const int8_t* W, int64_t M, int64_t N, int64_t K, const float* sW,
                 const float* bias, const float* residual, int act, float* out, int8_t* qx, float* sx, void* ws,
                 size_t ws_bytes, bq_stream_t stream) {
  const char* what = "bq_linear_i8";
  if (M < 0 || N < 0 || K < 0) return set_error(BQ_ERR_ARG, "%s: negative size", what);
  if (M == 0 || N == 0) return BQ_OK;
  if (K % 16) return set_error(BQ_ERR_UNSUPPORTED, "%s: K=%lld is not a multiple of 16", what, (long long)K);
  if (!x || !W || !sW || !out) return set_error(BQ_ERR_ARG, "%s: null pointer", what);
  if (!aligned16(x) || !aligned16(W)) return set_error(BQ_ERR_ARG, "%s: x and W must be 16-byte aligned", what);
  if (act < BQ_ACT_NONE || act > BQ_ACT_GELU) return set_error(BQ_ERR_ARG, "%s: bad activation %d", what, act);
  if (M <= 4 && K <= 8192 && M * K * 4 < ((int64_t)1 << 31) && N <= 0x7fffffff && N * K < ((int64_t)1 << 31)) {
    if (qx && !aligned16(qx)) return set_error(BQ_ERR_ARG, "%s: qx must be 16-byte aligned", what);
    GemmP p{};
    p.X = x; p.qx = qx; p.sx = sx; p.W = W; p.M = (int)M; p.N = (int)N; p.K = (int)K;
    p.sa_per_row = 1; p.sW = sW; p.bias = bias; p.res = residual; p.act = act; p.out = out;
    hipStream_t st = (hipStream_t)stream;
    switch (M) {
      case 1: launch_gemv_fq<1>(p, st); break;
      case 2: launch_gemv_fq<2>(p, st); break;
      case 3: launch_gemv_fq<3>(p, st); break;
      default: launch_gemv_fq<4>(p, st); break;
    }
    return check_launch(what);
  }
  if (!qx || !sx) return set_error(BQ_ERR_ARG, "%s: qx and sx are needed (M=%lld > 4 quantizes into them)", what,
                                   (long long)M);
  const int rc = bq_quantize_rows(x, M, K, qx, sx, stream);
  if (rc != BQ_OK) return rc;
  return gemm_impl(what, qx, W, M, N, K, sx, sW, bias, residual, act, out, nullptr, ws, ws_bytes, false, stream);
}

// Checks one convolution's arguments and fills its kernel parameters (the tuned plan of its
// geometry applied). `dense`: a 1x1 stride-1 unpadded conv, which runs the dense loader on
// [N*H*W, C]. `empty`: no output rows (nothing to launch).
static int conv_setup(const char* what, const int8_t* x, int64_t N, int64_t H, int64_t W, int64_t C,
                      const int8_t* w, int64_t O, int64_t KH, int64_t KW, int64_t stride, int64_t pad,
                      const float* sA, const float* sW, const float* bias, const float* residual, int act,
                      float* out, int32_t* acc, const float* s_out, int8_t* q_out, float* amax, GemmP& p,
                      bool& dense, bool& empty) {
  empty = false;
  if (N < 0 || H < 1 || W < 1 || C < 1 || O < 1 || KH < 1 || KW < 1 || stride < 1 || pad < 0)
    return set_error(BQ_ERR_ARG, "%s: bad geometry", what);
  if (C % 16) return set_error(BQ_ERR_UNSUPPORTED, "%s: C=%lld is not a multiple of 16 (pad it)", what, (long long)C);
  const int64_t OH = (H + 2 * pad - KH) / stride + 1;
  const int64_t OW = (W + 2 * pad - KW) / stride + 1;
  if (H + 2 * pad < KH || W + 2 * pad < KW || OH < 1 || OW < 1)
    return set_error(BQ_ERR_ARG, "%s: the filter is larger than the input.", what);
  const int64_t M = N * OH * OW, K = KH * KW * C;
  if (M > 0x7fffffff || O > 0x7fffffff || N * H * W * C >= ((int64_t)1 << 31) || O * K >= ((int64_t)1 << 31))
    return set_error(BQ_ERR_ARG, "%s: size too large (activation and weight must each be < 2 GiB)", what);
  if (K > KMAX_EXACT)
    return set_error(BQ_ERR_UNSUPPORTED, "%s: KH*KW*C=%lld > %d: int32 accumulators could overflow", what,
                     (long long)K, KMAX_EXACT);
  if (M == 0) {
    empty = true;
    return BQ_OK;
  }
  if (!x || !w || !sA || !sW || (!out && !q_out)) return set_error(BQ_ERR_ARG, "%s: null pointer", what);
  if (!aligned16(x) || !aligned16(w)) return set_error(BQ_ERR_ARG, "%s: x and w must be 16-byte aligned", what);
  if (act < BQ_ACT_NONE || act > BQ_ACT_GELU) return set_error(BQ_ERR_ARG, "%s: bad activation %d", what, act);
  p = GemmP{};
  p.A = x; p.W = w; p.M = (int)M; p.N = (int)O; p.K = (int)K;
  p.sA = sA; p.sa_per_row = 0; p.sW = sW; p.bias = bias; p.res = residual; p.act = act;
  p.out = out; p.acc = acc;
  p.H = (int)H; p.Wd = (int)W; p.C = (int)C; p.OH = (int)OH; p.OW = (int)OW; p.KWd = (int)KW;
  p.stride = (int)stride; p.pad = (int)pad;
  const FastDiv dc = fast_div((uint32_t)C), dkw = fast_div((uint32_t)KW);
  p.c_mul = dc.mul; p.c_shift = dc.shift; p.kw_mul = dkw.mul; p.kw_shift = dkw.shift;
  const FastDiv dpl = fast_div((uint32_t)(OH * OW)), dow = fast_div((uint32_t)OW);
  p.plane_mul = dpl.mul; p.plane_shift = dpl.shift; p.ow_mul = dow.mul; p.ow_shift = dow.shift;
  p.Nimg_HWC = N * H * W * C;
  p.vec_ok = (O % 4 == 0) && aligned16(out) && aligned16(acc) && aligned16(residual) && ((uintptr_t)q_out & 3) == 0;
  p.s_out = s_out;
  p.q_out = q_out;
  p.amax = amax;
  apply_plan(p, conv_key(N, H, W, C, O, KH, KW, stride, pad));
  dense = KH == 1 && KW == 1 && stride == 1 && pad == 0;
  return BQ_OK;
}

static int conv_impl(const char* what, const int8_t* x, int64_t N, int64_t H, int64_t W, int64_t C,
                     const int8_t* w, int64_t O, int64_t KH, int64_t KW, int64_t stride, int64_t pad,
                     const float* sA, const float* sW, const float* bias, const float* residual, int act,
                     float* out, int32_t* acc, const float* s_out, int8_t* q_out, float* amax, void* ws,
                     size_t ws_bytes, bq_stream_t stream) {
  GemmP p;
  bool dense, empty;
  if (int r = conv_setup(what, x, N, H, W, C, w, O, KH, KW, stride, pad, sA, sW, bias, residual, act, out, acc,
                         s_out, q_out, amax, p, dense, empty))
    return r;
  if (empty) return BQ_OK;
  hipStream_t st = (hipStream_t)stream;
  if (dense)
    launch_gemm<false>(p, st, Ws{ws, ws_bytes});  // a 1x1 conv is the dense GEMM on [N*H*W, C]
  else
    launch_gemm<true>(p, st, Ws{ws, ws_bytes});
  return check_launch(what);
}

int bq_conv2d_i8_nchw_fq(const float* x, int64_t N, int64_t Cin, int64_t H, int64_t W, const float* s_x,
                         const int8_t* w, int64_t O, int64_t KH, int64_t KW, int64_t stride, int64_t pad,
                         const float* sW, const float* bias, const float* residual, int act, float* out,
                         int32_t* acc, const float* s_out, int8_t* q_out, float* absmax_parts, int64_t parts_cap,
                         int64_t* nparts, float* sx, void* ws, size_t ws_bytes, bq_stream_t stream) {
  const char* what = "bq_conv2d_i8_nchw_fq";
  if (Cin < 1 || Cin > 8) return set_error(BQ_ERR_UNSUPPORTED, "%s: %lld input channels (1 to 8)", what, (long long)Cin);
  if (N < 0 || H < 1 || W < 1 || N * Cin * H * W >= ((int64_t)1 << 31) / 4)
    return set_error(BQ_ERR_ARG, "%s: bad or too large input (the f32 input must be < 2 GiB)", what);
  GemmP p;
  bool dense, empty;
  // conv_setup checks the geometry (over the weight's 16 padded channels), the weight and the
  // epilogue; the f32 input and the weight scales stand in for the int8 input and its scale
  // in its pointer checks (non-null, 16-byte aligned; neither is read through A / sA), and an
  // empty batch returns before them
  if (int r = conv_setup(what, reinterpret_cast<const int8_t*>(x), N, H, W, 16, w, O, KH, KW, stride, pad, sW, sW,
                         bias, residual, act, out, acc, s_out, q_out, absmax_parts, p, dense, empty))
    return r;
  if (nparts) *nparts = 0;
  if (empty) return BQ_OK;
  if (O > 64 || O % 4 || !smallk_ok(p, true))
    return set_error(BQ_ERR_UNSUPPORTED, "%s: takes O <= 64 (O %% 4 == 0) and KH*KW*16 <= 256", what);
  if ((s_out != nullptr) != (q_out != nullptr) || (q_out && O % 16))
    return set_error(BQ_ERR_ARG, "%s: an int8 twin needs s_out, q_out and O %% 16 == 0", what);
  const long long grid = smallk_grid(p);
  if (absmax_parts && parts_cap < grid)
    return set_error(BQ_ERR_ARG, "%s: %lld partial maxima, room for %lld", what, grid, (long long)parts_cap);
  hipStream_t st = (hipStream_t)stream;
  p.A = nullptr;
  p.sA = nullptr;
  p.Nimg_HWC = N * Cin * H * W * 4;  // the f32 input's bytes (its buffer range)
  p.Xf = x;
  p.Cin = (int)Cin;
  p.sx_given = s_x;
  p.sx_out = sx;
  if (!s_x) {  // the dynamic scale: partial maxima of |x| first
    int np = 0;
    if (int r = absmax_parts_ws(what, x, N * Cin * H * W, ws, ws_bytes, st, &np)) return r;
    p.xparts = static_cast<const float*>(ws);
    p.nxparts = np;
  }
  if (Cin <= 4)
    launch_smallk_f32in<4>(p, st);
  else
    launch_smallk_f32in<8>(p, st);
  if (int r = check_launch(what)) return r;
  if (nparts && absmax_parts) *nparts = grid;
  return BQ_OK;
}

int64_t bq_conv2d_absmax_parts(int64_t N, int64_t H, int64_t W, int64_t C, int64_t O, int64_t KH, int64_t KW,
                               int64_t stride, int64_t pad) {
  if (N < 0 || H < 1 || W < 1 || C < 1 || O < 1 || KH < 1 || KW < 1 || stride < 1 || pad < 0 ||
      H + 2 * pad < KH || W + 2 * pad < KW)
    return set_error(BQ_ERR_ARG, "bq_conv2d_absmax_parts: bad geometry");
  const int64_t OH = (H + 2 * pad - KH) / stride + 1;
  const int64_t OW = (W + 2 * pad - KW) / stride + 1;
  if (N * OH * OW > 0x7fffffff || O > 0x7fffffff || KH * KW * C > KMAX_EXACT)
    return set_error(BQ_ERR_ARG, "bq_conv2d_absmax_parts: size too large");
  GemmP p{};
  p.M = (int)(N * OH * OW);
  p.N = (int)O;
  p.K = (int)(KH * KW * C);  // the small-K kernel's test reads K: the count is the launch's
  apply_plan(p, conv_key(N, H, W, C, O, KH, KW, stride, pad));
  return p.M == 0 ? 0 : out_tiles(p, !(KH == 1 && KW == 1 && stride == 1 && pad == 0));
}

int bq_conv2d_i8_nhwc_dq_ok(int64_t N, int64_t H, int64_t W, int64_t C, int64_t O, int64_t KH, int64_t KW,
                            int64_t stride, int64_t pad) {
  PlanKey key;
  GemmP p;
  bool conv, tiled;
  const int64_t pr[9] = {N, H, W, C, O, KH, KW, stride, pad};
  if (!problem_view(pr, 9, key, p, conv, tiled))
    return set_error(BQ_ERR_ARG, "bq_conv2d_i8_nhwc_dq_ok: bad geometry (C %% 16 == 0, N >= 1)");
  if (O % 16) return 0;
  apply_plan(p, key);
  p.q_out = reinterpret_cast<int8_t*>(&p);  // the twin alone (never dereferenced here)
  return choose_cfg(p, conv) == CFG_SMALLK ? 1 : 0;
}

int bq_plan_candidates(const int64_t* problem, int n, int32_t* cfgs, int32_t* splits, int cap) {
  PlanKey key;
  GemmP p;
  bool conv, tiled;
  if (!problem_view(problem, n, key, p, conv, tiled))
    return set_error(BQ_ERR_ARG, "bq_plan_candidates: bad problem (3 dense or 9 conv dimensions)");
  if (!tiled) {
    if (conv || p.M > DECODE_MAX_M) return 0;
    // the decode kernels: the rule's first, the GEMV only where it takes the shape
    const bool gemv_ok = p.K <= (p.M <= 4 ? 8192 : 4096);
    const bool rule_gemv = p.M <= GEMV_RULE_M && gemv_ok;
    int cnt = 0;
    int32_t c[2];
    c[cnt++] = rule_gemv ? BQ_CFG_GEMV : BQ_CFG_SKINNY;
    if (gemv_ok) c[cnt++] = rule_gemv ? BQ_CFG_SKINNY : BQ_CFG_GEMV;
    for (int i = 0; i < cnt && i < cap; ++i) {
      if (cfgs) cfgs[i] = c[i];
      if (splits) splits[i] = 1;
    }
    return cnt;
  }
  std::pair<int, int> out[64];
  int cnt = 0;
  const int rule = choose_cfg(p, conv);
  out[cnt++] = {rule, rule == CFG_SMALLK ? 1 : split_of(p, rule, conv, 0)};
  if (rule != CFG_SMALLK && smallk_ok(p, conv)) out[cnt++] = {CFG_SMALLK, 1};
  // 3 (four waves on 256x256) and 9 (64x64 with an 8-deep ring) never won a measurement
  static const int ids[] = {1, 2, 4, 5, 6, 7, 8, 10, 11, 12, 13, 14, 15, 16, 17};
  for (int cfg : ids) {
    if (cfg == 16 && conv) continue;  // dense only
    const TileDims d = CFG_TILES[cfg];
    const int KT = (p.K + BK - 1) / BK;
    const int tries[] = {1, 2, 4, 8};
    for (int want : tries) {
      if (want > 1 && (d.bm * d.bn > SPLIT_MAX_TILE || KT < 2 * want)) break;
      const std::pair<int, int> c{cfg, split_of(p, cfg, conv, want)};
      if (c.second != want) continue;  // the workspace cannot hold this split
      bool dup = false;
      for (int i = 0; i < cnt; ++i) dup |= out[i] == c;
      if (!dup && cnt < 64) out[cnt++] = c;
    }
  }
  for (int i = 0; i < cnt && i < cap; ++i) {
    if (cfgs) cfgs[i] = out[i].first;
    if (splits) splits[i] = out[i].second;
  }
  return cnt;
}

int bq_plan_set(const int64_t* problem, int n, int32_t cfg, int32_t split) {
  PlanKey key;
  GemmP p;
  bool conv, tiled;
  if (!problem_view(problem, n, key, p, conv, tiled))
    return set_error(BQ_ERR_ARG, "bq_plan_set: bad problem (3 dense or 9 conv dimensions)");
  std::lock_guard<std::mutex> lock(g_plan_mu);
  if (cfg == 0) {
    g_plans.erase(key);
    return BQ_OK;
  }
  if (!tiled) {
    if (p.M > DECODE_MAX_M || (cfg != BQ_CFG_GEMV && cfg != BQ_CFG_SKINNY) || split != 1)
      return set_error(BQ_ERR_ARG, "bq_plan_set: a GEMM of at most 64 rows has no tiled kernel to plan (up to %d "
                       "rows: BQ_CFG_GEMV or BQ_CFG_SKINNY, split 1)", DECODE_MAX_M);
    if (cfg == BQ_CFG_GEMV && p.K > (p.M <= 4 ? 8192 : 4096))
      return set_error(BQ_ERR_ARG, "bq_plan_set: the GEMV takes K <= %d at M = %d", p.M <= 4 ? 8192 : 4096, p.M);
    g_plans[key] = Plan{cfg, split};
    return BQ_OK;
  }
  if (cfg == CFG_SMALLK) {
    if (!smallk_ok(p, conv) || split != 1)
      return set_error(BQ_ERR_ARG, "bq_plan_set: BQ_CFG_SMALLK takes a problem of N <= 64 (N %% 4 == 0) and "
                       "K <= 256, split 1");
    g_plans[key] = Plan{cfg, split};
    return BQ_OK;
  }
  if (cfg < 1 || cfg >= NCFG || cfg == 3 || cfg == 9 || (cfg == 16 && conv) || split < 1 || split > 64)
    return set_error(BQ_ERR_ARG, "bq_plan_set: bad configuration %d / split %d", cfg, split);
  g_plans[key] = Plan{cfg, split};
  return BQ_OK;
}

int bq_plan_clear(void) {
  std::lock_guard<std::mutex> lock(g_plan_mu);
  g_plans.clear();
  return BQ_OK;
}

int bq_conv2d_i8_nhwc(const int8_t* x, int64_t N, int64_t H, int64_t W, int64_t C, const int8_t* w,
                      int64_t O, int64_t KH, int64_t KW, int64_t stride, int64_t pad, const float* sA,
                      const float* sW, const float* bias, const float* residual, int act, float* out,
                      int32_t* acc, float* absmax_parts, void* ws, size_t ws_bytes, bq_stream_t stream) {
  return conv_impl("bq_conv2d_i8_nhwc", x, N, H, W, C, w, O, KH, KW, stride, pad, sA, sW, bias, residual, act, out,
                   acc, nullptr, nullptr, absmax_parts, ws, ws_bytes, stream);
}

int bq_conv2d_i8_nhwc_q(const int8_t* x, int64_t N, int64_t H, int64_t W, int64_t C, const int8_t* w,
                        int64_t O, int64_t KH, int64_t KW, int64_t stride, int64_t pad, const float* sA,
                        const float* sW, const float* bias, const float* residual, int act, float* out,
                        int32_t* acc, const float* s_out, int8_t* q_out, float* absmax_parts, void* ws,
                        size_t ws_bytes, bq_stream_t stream) {
  if (!s_out || !q_out) return set_error(BQ_ERR_ARG, "bq_conv2d_i8_nhwc_q: null s_out or q_out");
  if (O % 16) return set_error(BQ_ERR_UNSUPPORTED, "bq_conv2d_i8_nhwc_q: O=%lld is not a multiple of 16", (long long)O);
  return conv_impl("bq_conv2d_i8_nhwc_q", x, N, H, W, C, w, O, KH, KW, stride, pad, sA, sW, bias, residual, act,
                   out, acc, s_out, q_out, absmax_parts, ws, ws_bytes, stream);
}

int bq_conv2d_i8_nhwc_dq(const int8_t* x, int64_t N, int64_t H, int64_t W, int64_t C, const int8_t* w, int64_t O,
                         int64_t KH, int64_t KW, int64_t stride, int64_t pad, const float* sA, const float* sW,
                         const float* bias, const float* residual, int act, int8_t* q_out, float* s_out, float* parts,
                         int64_t parts_cap, bq_stream_t stream) {
  const char* what = "bq_conv2d_i8_nhwc_dq";
  if (O % 16) return set_error(BQ_ERR_UNSUPPORTED, "%s: O=%lld is not a multiple of 16", what, (long long)O);
  GemmP p;
  bool dense, empty;
  if (int r = conv_setup(what, x, N, H, W, C, w, O, KH, KW, stride, pad, sA, sW, bias, residual, act, nullptr,
                         nullptr, nullptr, q_out, nullptr, p, dense, empty))
    return r;
  if (empty) return BQ_OK;  // an empty batch: nothing launched, the pointers may be null
  if (!s_out || !parts) return set_error(BQ_ERR_ARG, "%s: null s_out or parts", what);
  // where the small-K kernel runs the twin alone (the rule's pick, or a plan's): its pass with
  // no store is cheaper than an f32 output and a quantize pass over it
  if (choose_cfg(p, !dense) != CFG_SMALLK)
    return set_error(BQ_ERR_UNSUPPORTED, "%s: the small-K kernel does not take this layer's twin", what);
  const long long grid = smallk_grid(p);
  if (parts_cap < grid)
    return set_error(BQ_ERR_ARG, "%s: %lld partial maxima, room for %lld", what, grid, (long long)parts_cap);
  hipStream_t st = (hipStream_t)stream;
  GemmP p1 = p;  // pass 1: every output computed, only each workgroup's max |y| stored
  p1.q_out = nullptr;
  p1.amax = parts;
  GemmP p2 = p;  // pass 2: the same outputs again, stored as the twin at the scale of pass 1's maxima
  p2.oparts = parts;
  p2.noparts = (int)grid;
  p2.sout_write = s_out;
  if (dense) {
    launch_smallk<false>(p1, st);
    if (int r = check_launch(what)) return r;
    launch_smallk<false>(p2, st);
  } else {
    launch_smallk<true>(p1, st);
    if (int r = check_launch(what)) return r;
    launch_smallk<true>(p2, st);
  }
  return check_launch(what);
}

int bq_conv2d_i8_nhwc_pair(const int8_t* x, int64_t N, int64_t H, int64_t W, int64_t C, const float* sA,
                           const bq_conv_desc* a, const bq_conv_desc* b, void* ws, size_t ws_bytes,
                           bq_stream_t stream) {
  const char* what = "bq_conv2d_i8_nhwc_pair";
  if (!a || !b) return set_error(BQ_ERR_ARG, "%s: null descriptor", what);
  if (b->amax) return set_error(BQ_ERR_UNSUPPORTED, "%s: the second conv takes no absmax_parts", what);
  for (const bq_conv_desc* d : {a, b})
    if ((d->s_out != nullptr) != (d->q_out != nullptr) || (d->q_out && d->O % 16))
      return set_error(BQ_ERR_ARG, "%s: an int8 twin needs s_out, q_out and O %% 16 == 0", what);
  GemmP p[2];
  bool dense[2], empty[2];
  for (int i = 0; i < 2; ++i) {
    const bq_conv_desc& d = i ? *b : *a;
    if (int r = conv_setup(what, x, N, H, W, C, d.w, d.O, d.KH, d.KW, d.stride, d.pad, sA, d.sW, d.bias, d.residual,
                           d.act, d.out, nullptr, d.s_out, d.q_out, d.amax, p[i], dense[i], empty[i]))
      return r;
  }
  hipStream_t st = (hipStream_t)stream;
  const Ws w{ws, ws_bytes};
  if (!empty[0] && !empty[1] && !dense[0] && !dense[1] && launch_conv_pair(p[0], p[1], st, w))
    return check_launch(what);
  for (int i = 0; i < 2; ++i) {  // separate launches, one after the other on the stream
    if (empty[i]) continue;
    if (dense[i]) launch_gemm<false>(p[i], st, w);
    else launch_gemm<true>(p[i], st, w);
    if (int r = check_launch(what)) return r;
  }
  return BQ_OK;
}

}  // extern "C"
