/*
 * libbq — int8 (W8A8) inference kernels for AMD Instinct MI355X (gfx950).
 *
 * The C ABI of the drop-in boundary. Every pointer argument except `ws` is caller-owned
 * device memory (for example `torch.Tensor.data_ptr()`); the library allocates nothing
 * (scratch memory is the caller's `ws`). Every call enqueues on `stream` (a hipStream_t
 * handle; NULL = the null stream) and returns without a host synchronisation.
 *
 * Return value: BQ_OK (0) or a negative BQ_ERR_*; the message of the last failure on
 * the calling thread is bq_last_error(). No C++ exception crosses this boundary.
 *
 * Arithmetic (one rule for weights and activations):
 *   s = float32(max|v| / 127)                 correctly rounded
 *   q = clip(rint(v / s), -127, 127)          of the exact quotient, round half to even
 *   s == 0 (all-zero row / tensor)  ->  q = 0
 *   acc = sum_k qa * qw                        exact int32
 *   y = ((f32(acc) * sA) * sW[n]) + bias[n], then + residual, then the activation,
 *       one float32 rounding per operation.
 *
 * Reference interfaces replaced (paths into playidea-lab/borch):
 *   quantizers   borch-ts/src/quant.ts:23-103, kernels.ts:2024-2081
 *   GEMM         borch-ts/src/kernels.ts:1782-1857 (matmulInt8), called where the numpy
 *                core runs nn.Linear / F.linear (borch/_nn.py:397-415, 4675-4677)
 *   conv         borch-ts/src/kernels.ts:2084-2302 (convForwardInt8) + 5834-5914
 *                (sumSplitsConv), called from Tensor.convNDFusedInt8 (tensor.ts:11869-11958)
 *   depthwise    borch-ts/src/kernels.ts:5932-5968 (depthwiseForward, f32 in the
 *                reference) and borch-ts/wasm/src/lib.rs:598-641 (dwconv_rows)
 */
#ifndef BQ_H
#define BQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* bq_stream_t; /* a hipStream_t; NULL = the null stream */

#define BQ_OK 0
#define BQ_ERR_ARG (-1)         /* bad pointer, size, alignment or shape */
#define BQ_ERR_DEVICE (-2)      /* no device, or not gfx950 */
#define BQ_ERR_LAUNCH (-3)      /* the kernel launch failed */
#define BQ_ERR_UNSUPPORTED (-4) /* a shape this library does not take */

#define BQ_ACT_NONE 0
#define BQ_ACT_RELU 1
#define BQ_ACT_SILU 2
#define BQ_ACT_GELU 3 /* erf form, f32: (y * 0.5) * (1 + erf(y * sqrt(1/2))) */

/* OR-ed into bq_gemm_i8's `act`: sA is one activation scale for the whole A (f32 [1])
 * instead of one per row, as the reference's matmulInt8(scaled) takes it (Scale[0],
 * borch-ts/src/kernels.ts:1818-1827) after a per-tensor quantize (bq_quantize_tensor). */
#define BQ_SCALE_A_PER_TENSOR 0x100

/* Library version, (major << 16) | minor. */
int bq_version(void);

/* The message of the last failing call on this thread ("" if none). */
const char* bq_last_error(void);

/* 1 if `device` is a gfx950 (MI350/MI355X) the kernels were built for, else 0 with the
 * reason in bq_last_error(). Replaces the capability gate Device.subgroupInt8
 * (borch-ts/src/device.ts:466-482, refused by name at nn.ts:6771-6773). */
int bq_device_ok(int device);

/* Per-row dynamic activation quantization: x f32 [M, K] row-major -> q int8 [M, K],
 * s f32 [M]. One pass over x. Replaces absMaxAtomic + quantizeActivationInt8
 * (borch-ts/src/kernels.ts:2024-2081) with per-row scales. x, q: 16-byte aligned. */
int bq_quantize_rows(const float* x, int64_t M, int64_t K, int8_t* q, float* s,
                     bq_stream_t stream);

/* bq_quantize_rows of act(x) (BQ_ACT_*, one f32 evaluation per element, the epilogue's
 * operation order) without storing act(x): a transformer MLP's second input, where the
 * reference runs the activation pass and then the quantize (kernels.ts:2024-2081). y
 * (nullable) f32 [M, K] also receives act(x) (16-byte aligned). */
int bq_quantize_rows_act(const float* x, int64_t M, int64_t K, int act, int8_t* q, float* s, float* y,
                         bq_stream_t stream);

/* LayerNorm over each row, then bq_quantize_rows of the result, in one pass (the
 * normalised row is not stored):
 *   y = ((x - mean) * rstd) * gamma + beta, mean = sum(x) / K, var = sum((x - mean)^2) / K,
 *   rstd = 1 / sqrt(var + eps), f32, one rounding per operation (gamma, beta f32 [K],
 *   nullable: 1 and 0); q int8 [M, K], s f32 [M] = the per-row scales of y.
 * y (nullable) f32 [M, K] also receives the normalised rows. K % 4 == 0, K <= 4096; x,
 * gamma, beta, y 16-byte aligned. Replaces layerNormRows (borch-ts/src/kernels.ts:2935-2986)
 * followed by the activation quantize of the next Linear (kernels.ts:2024-2081). */
int bq_layernorm_quantize_rows(const float* x, int64_t M, int64_t K, const float* gamma, const float* beta, float eps,
                               int8_t* q, float* s, float* y, bq_stream_t stream);

/* Per-output-channel weight quantization of a Linear weight W f32 [N, K] -> q int8
 * [N, K], s f32 [N]. Replaces quantizeInt8PerChannel (borch-ts/src/quant.ts:23-53); the
 * same kernel and rule as bq_quantize_rows. */
int bq_quantize_weight_per_channel(const float* w, int64_t N, int64_t K, int8_t* q,
                                   float* s, bq_stream_t stream);

/* Rounding rules of bq_quantize_weight_host. */
#define BQ_ROUND_EXACT 0          /* this library's rule: the bytes of bq_quantize_weight_per_channel */
#define BQ_ROUND_REFERENCE 1      /* quant.ts:35-41 (Linear): double scale, w * (1/scale), Math.round */
#define BQ_ROUND_REFERENCE_CONV 2 /* quant.ts:88-96 (conv): f32 scale, w / scale in double, Math.round */

/* Per-output-channel weight quantization on the HOST (every pointer is host memory):
 * w f32 [N, K] row-major -> q int8 [N, Kpad] (columns K..Kpad-1 zero), s f32 [N], with
 * `rule` one of BQ_ROUND_*. BQ_ROUND_EXACT gives the bytes and scales of
 * bq_quantize_weight_per_channel; BQ_ROUND_REFERENCE the bytes of borch-ts's Linear packer
 * (scale = peak / 127 in double, stored as f32; q = Math.round(w * (1 / scale)), a tie
 * toward +inf; it differs from the exact rule on some near-ties as well as ties);
 * BQ_ROUND_REFERENCE_CONV those of its conv packer (f32 scale, Math.round(w / scale): it
 * differs from the exact rule on exact ties only). Rows are split over `nthreads` host
 * threads (<= 0: all hardware threads). Replaces quantizeInt8PerChannel
 * (borch-ts/src/quant.ts:23-53), which Tensor.inWindowInt8 runs on the host before the
 * upload (tensor.ts:1681-1705), and the scale and rounding of
 * quantizeConvWeightInt8TapMajor (quant.ts:80-96). */
int bq_quantize_weight_host(const float* w, int64_t N, int64_t K, int64_t Kpad, int rule, int8_t* q, float* s,
                            int nthreads);

/* Bytes of `ws` that bq_quantize_tensor / bq_quantize_nhwc need for n elements. */
size_t bq_quantize_tensor_ws_bytes(int64_t n);

/* Per-tensor quantization of x f32 [n] -> q int8 [n], s f32 [1]. Two kernels: partial
 * maxima into ws, then quantize. Replaces absMaxAtomic + quantizeActivationInt8
 * (borch-ts/src/kernels.ts:2024-2081). */
int bq_quantize_tensor(const float* x, int64_t n, int8_t* q, float* s, void* ws,
                       size_t ws_bytes, bq_stream_t stream);

/* Per-tensor quantization of a channels-last activation x f32 [P, C] (P = N*H*W pixels)
 * into q int8 [P, Cpad], channels C..Cpad-1 zero, s f32 [1]. The conv input
 * (tensor.ts:11909-11921; kernels.ts:2057-2081 packs NC/4HW4, this packs NHWC). */
int bq_quantize_nhwc(const float* x, int64_t P, int64_t C, int64_t Cpad, int8_t* q, float* s,
                     void* ws, size_t ws_bytes, bq_stream_t stream);

/* The same quantization with the scale taken from partial maxima a producer already wrote:
 * absmax_parts f32 [nparts] whose maximum is max|x| (bq_conv2d_i8_nhwc's per-tile output
 * maxima). One pass over x, no max pass; the scale is bit-identical to bq_quantize_nhwc's
 * (a maximum does not depend on how it is split). The reference's producer-side shortcut
 * is the calibrated twin (tensor.ts:11909-11913); this is its dynamic-scale counterpart. */
int bq_quantize_nhwc_parts(const float* x, int64_t P, int64_t C, int64_t Cpad, const float* absmax_parts,
                           int64_t nparts, int8_t* q, float* s, bq_stream_t stream);

/* Per-tensor quantization of a per-(image, channel) scaled activation: the value quantized
 * is fl(x[n, p, c] * cs[n, c]) (one f32 multiply, never stored), x f32 [N*HW, C]
 * channels-last, cs f32 [N, C] (a squeeze-excite's sigmoid gates), into q int8
 * [N*HW, Cpad] (channels C..Cpad-1 zero). The scale is s_given[0] when s_given is non-null
 * (calibrated; one pass), else float32(max|fl(x*cs)| / 127) into s[0]: from absmax_parts
 * f32 [nparts] whose maximum is max|fl(x*cs)| when given (one pass; bq_se_gate_nhwc writes
 * them), else two passes with partial maxima in ws (bq_quantize_tensor_ws_bytes(N*HW*C)
 * bytes). The same bytes as quantizing the stored product. C and Cpad multiples of 4; x, cs
 * 16-byte aligned. */
int bq_quantize_nhwc_chscale(const float* x, int64_t N, int64_t HW, int64_t C, int64_t Cpad, const float* cs,
                             int8_t* q, float* s, const float* s_given, const float* absmax_parts, int64_t nparts,
                             void* ws, size_t ws_bytes, bq_stream_t stream);

/* The same quantization with a given (calibrated) scale s f32 [1]: one pass, no maximum.
 * The static-scale input of borch-ts (int8.inMax, tensor.ts:11912-11913; calibrateInt8
 * nn.ts:6790-6824). Values beyond the calibrated range clamp to +-127. */
int bq_quantize_nhwc_scaled(const float* x, int64_t P, int64_t C, int64_t Cpad, const float* s, int8_t* q,
                            bq_stream_t stream);

/* bq_quantize_nhwc and bq_quantize_nhwc_scaled for an NCHW input x f32 [N, C, HW] (a
 * network's input image, channels padded, Cpad > C, Cpad % 16 == 0, q 16-byte aligned): the
 * same bytes and scale as permuting x to channels-last first, without the permute. The
 * reference's conv input quantization reads its NCHW tensors directly
 * (borch-ts/src/kernels.ts:2057-2081 from NCHW into NC/4HW4; tensor.ts:11909-11921). */
int bq_quantize_nchw(const float* x, int64_t N, int64_t C, int64_t HW, int64_t Cpad, int8_t* q, float* s, void* ws,
                     size_t ws_bytes, bq_stream_t stream);
int bq_quantize_nchw_scaled(const float* x, int64_t N, int64_t C, int64_t HW, int64_t Cpad, const float* s, int8_t* q,
                            bq_stream_t stream);

/* Bytes of the split-K workspace `ws` that bq_gemm_i8 / bq_conv2d_i8_nhwc(_q) can use, for
 * any shape (about 6.5 MiB). With it, a grid that would leave most CUs idle (few output
 * tiles, long K: e.g. the late layers of a CIFAR ResNet at small batch) is split along K
 * into several workgroups per tile; the int32 partial tiles are added exactly by the last
 * workgroup of each tile, in the same launch, so results are bit-identical to the unsplit
 * kernel. `ws` must be zero-filled before its first use; every call leaves its counters
 * zero again. Calls that share one `ws` must not run concurrently (use one per stream).
 * ws == NULL (or ws_bytes smaller than this) runs the unsplit kernel. The reference splits
 * K with f32 slabs and a second pass (convInt8Split / sumSplitsConv,
 * borch-ts/src/kernels.ts:2120-2127, 5860-5914). */
size_t bq_gemm_ws_bytes(void);

/* W8A8 GEMM with the fused dequant epilogue, Linear layout (x @ W.T):
 *   A int8 [M, K] (per-row scales sA f32 [M], or one sA f32 [1] for the whole A with
 *   act | BQ_SCALE_A_PER_TENSOR), W int8 [N, K] (per-channel sW f32 [N]),
 *   out f32 [M, N] = ((f32(A @ W.T) * sA[m]) * sW[n]) + bias[n] (bias nullable), then
 *   + residual[m, n] (f32 [M, N], nullable: a transformer's skip connection), then the
 *   activation `act` (BQ_ACT_*). `acc` (nullable) receives the exact int32 [M, N].
 * K % 16 == 0 and K <= 133152 (K * 127^2 < 2^31: the int32 sums are exact for any
 * operands); A, W 16-byte aligned. ws: the split-K workspace (nullable, see
 * bq_gemm_ws_bytes). Replaces matmulInt8(M,K,N,scaled)
 * (borch-ts/src/kernels.ts:1808-1852), which took only whole 32s. */
int bq_gemm_i8(const int8_t* A, const int8_t* W, int64_t M, int64_t N, int64_t K,
               const float* sA, const float* sW, const float* bias, const float* residual, int act,
               float* out, int32_t* acc, void* ws, size_t ws_bytes, bq_stream_t stream);

/* The dynamic-quant W8A8 Linear: out f32 [M, N] = bq_gemm_i8 of the per-row quantization of
 * x f32 [M, K] (bq_quantize_rows' rule and bytes) against W int8 [N, K] / sW, with bias,
 * residual and act as bq_gemm_i8. The quantized rows and scales are written to qx int8
 * [M, K] and sx f32 [M]. M <= 4, K <= 8192: one launch, the quantization fused into the
 * GEMV (every workgroup quantizes the rows into its own LDS while its weight loads are in
 * flight; qx and sx are then optional, nullable). Otherwise bq_quantize_rows into qx / sx,
 * then bq_gemm_i8 (ws: its split-K workspace). K % 16 == 0; x, W, qx 16-byte aligned.
 * Replaces the reference's Linear forward: the activation quantize (kernels.ts:2024-2081)
 * followed by matmulInt8(scaled) (kernels.ts:1808-1852), here with per-row scales. */
int bq_linear_i8(const float* x, const int8_t* W, int64_t M, int64_t N, int64_t K, const float* sW,
                 const float* bias, const float* residual, int act, float* out, int8_t* qx, float* sx, void* ws,
                 size_t ws_bytes, bq_stream_t stream);

/* bq_gemm_i8 that allocates nothing and takes no workspace: the same arguments without
 * ws / ws_bytes, the same kernels and bit-identical results. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). Its split-K workspace is
 * the library's own static device array of bq_gemm_ws_bytes() bytes (about 6.5 MiB), one
 * copy per GPU, held until the process ends. That size covers the K split the rule picks
 * for every shape, so no shape is refused for its size; every other limit is
 * bq_gemm_i8's. The copy used is that of the GPU `stream` belongs to; the first call on a
 * GPU looks up its address (no launch: the array is zero when the library is loaded, and
 * every launch leaves its tile counters zero again), so a caller that captures a graph
 * makes one call on each GPU before the capture. All calls on one GPU share that GPU's
 * copy: calls that overlap on one GPU (two streams, or two threads) race and give wrong
 * results. */
int bq_gemm_i8_noalloc(const int8_t* A, const int8_t* W, int64_t M, int64_t N, int64_t K, const float* sA,
                       const float* sW, const float* bias, const float* residual, int act, float* out,
                       int32_t* acc, bq_stream_t stream);

/* Diagnostics, no counterpart in the reference: bq_gemm_i8 (no residual, no activation, no
 * int32 output, no K split) on the tiled kernel (M > 64) that also records, for each
 * workgroup, four words at stamps[4 * i .. 4 * i + 3] (i: the workgroup's tile order): the
 * steady wall clock (100 MHz, hipDeviceAttributeWallClockRate) at entry, after its main loop
 * and after its last output store completed, then its hardware id (bits 3:0 CU, 5:4 SE,
 * 9:6 XCC, as HIP's __smid). Returns the number of workgroups stamped, or a negative
 * BQ_ERR_* (stamps_cap, in words, too small: BQ_ERR_ARG). For measuring where a launch's
 * time goes (the start of each XCD, prologue and main loop, the output stores). */
int64_t bq_gemm_i8_phases(const int8_t* A, const int8_t* W, int64_t M, int64_t N, int64_t K, const float* sA,
                          const float* sW, const float* bias, float* out, uint64_t* stamps, int64_t stamps_cap,
                          bq_stream_t stream);

/* Implicit-GEMM int8 convolution, NHWC, groups 1, dilation 1:
 *   x int8 [N, H, W, C] (C % 16 == 0, per-tensor scale sA f32 [1]),
 *   w int8 [O, KH, KW, C] (per-channel scale sW f32 [O]),
 *   out f32 [N, OH, OW, O] = ((f32(acc) * sA) * sW[o]) + bias[o] + residual, then act.
 * bias, residual (f32 [N, OH, OW, O]) and acc (int32 [N*OH*OW, O]) are nullable;
 * KH*KW*C <= 133152 (exact int32 sums). ws: the split-K workspace (nullable, see
 * bq_gemm_ws_bytes). absmax_parts (nullable, bq_conv2d_absmax_parts floats) receives
 * max|out| of each output tile: the next conv's bq_quantize_nhwc_parts then needs no max
 * pass over this output.
 * Replaces convForwardInt8 (+ sumSplitsConv) and its ConvEpilogue
 * (borch-ts/src/kernels.ts:2156-2302, 4230-4244, 5860-5914), which took stride 1, k <= 3,
 * C % 32 and O % 16 only. */
int bq_conv2d_i8_nhwc(const int8_t* x, int64_t N, int64_t H, int64_t W, int64_t C,
                      const int8_t* w, int64_t O, int64_t KH, int64_t KW, int64_t stride,
                      int64_t pad, const float* sA, const float* sW, const float* bias,
                      const float* residual, int act, float* out, int32_t* acc,
                      float* absmax_parts, void* ws, size_t ws_bytes, bq_stream_t stream);

/* A conv of an f32 NCHW input x [N, Cin, H, W] (a network's image, Cin <= 8; x 16-byte aligned) with its
 * per-tensor quantization fused: bq_conv2d_i8_nhwc(_q) of quantize(x) into 16 padded NHWC
 * channels, bit for bit, in one launch. The scale is s_x[0] (calibrated) or, with s_x NULL,
 * float32(max|x| / 127) from partial maxima computed first into ws
 * (bq_quantize_tensor_ws_bytes(N*Cin*H*W) bytes; a second launch); sx (nullable) receives
 * it. w is packed over 16 channels ([O, KH*KW*16]); O <= 64 with O % 4 == 0 and
 * KH*KW*16 <= 256 (the small-K kernel), else BQ_ERR_UNSUPPORTED (nothing launched).
 * absmax_parts (nullable, room for parts_cap floats; 4096 always suffice) receives the
 * output's partial maxima and *nparts (nullable) their count. The rest as
 * bq_conv2d_i8_nhwc_q (s_out / q_out nullable, out nullable with q_out). Replaces the
 * reference's input quantize pass before its first conv (tensor.ts:11909-11921;
 * kernels.ts:2057-2081). */
int bq_conv2d_i8_nchw_fq(const float* x, int64_t N, int64_t Cin, int64_t H, int64_t W, const float* s_x,
                         const int8_t* w, int64_t O, int64_t KH, int64_t KW, int64_t stride, int64_t pad,
                         const float* sW, const float* bias, const float* residual, int act, float* out,
                         int32_t* acc, const float* s_out, int8_t* q_out, float* absmax_parts, int64_t parts_cap,
                         int64_t* nparts, float* sx, void* ws, size_t ws_bytes, bq_stream_t stream);

/* The number of floats bq_conv2d_i8_nhwc(_q) writes to a non-null `absmax_parts` for this
 * geometry (its output tile count), or a negative BQ_ERR_* for a bad geometry. */
int64_t bq_conv2d_absmax_parts(int64_t N, int64_t H, int64_t W, int64_t C, int64_t O, int64_t KH, int64_t KW,
                               int64_t stride, int64_t pad);

/* 1 if bq_conv2d_i8_nhwc_dq takes this conv under the plans in force (it launches rather than
 * returning BQ_ERR_UNSUPPORTED), 0 if not, a negative BQ_ERR_* for a bad geometry (C % 16
 * == 0, N >= 1). Host only: a caller decides before quantizing the conv's input which form
 * to run. The companion of bq_conv2d_i8_nhwc_dq, as bq_conv2d_absmax_parts is of the conv
 * (tensor.ts:11909-11921 decides there between the twin and the quantize pass). */
int bq_conv2d_i8_nhwc_dq_ok(int64_t N, int64_t H, int64_t W, int64_t C, int64_t O, int64_t KH, int64_t KW,
                            int64_t stride, int64_t pad);

/* Kernel choice by measurement. The GEMM and conv entry points pick a tiled-kernel
 * configuration (tile, ring depth) and a K split by rule; a plan overrides both for one
 * problem. Every configuration and split computes the same exact int32 sums and the same
 * epilogue, so a plan changes the time only, never a result. A problem is
 *   n == 3: a dense bq_gemm_i8 (M, N, K), or
 *   n == 9: a bq_conv2d_i8_nhwc(_q) (N, H, W, C, O, KH, KW, stride, pad), C the padded count.
 * bq_plan_candidates writes up to `cap` (configuration id, K split) pairs, the rules' pick
 * first, and returns how many there are (0: nothing to choose, as for a dense GEMM of 9 to
 * 64 rows; negative: a bad problem). A dense GEMM of at most 8 rows chooses between the two
 * decode kernels, BQ_CFG_GEMV and BQ_CFG_SKINNY (split 1). bq_plan_set records one (cfg == 0 removes the
 * problem's plan); bq_plan_clear removes all. A plan in force when bq_conv2d_absmax_parts
 * sizes a buffer must stay in force for the conv that fills it. Plans are process-wide;
 * set them before a graph capture (a captured launch keeps the choice it was made with).
 * Replaces Device.choose / runTuning (borch-ts/src/device.ts:2686-2700, 2834-2846), the
 * rule's pick first and the fastest cached per key, that compiled(..., {tune}) drives
 * (borch-ts/src/compile.ts:55-62). */
#define BQ_CFG_GEMV 32   /* dense, M <= 8: the v_dot4 wave-reduction GEMV (K <= 8192; 4096 above 4 rows;
                          * the rule's pick where it takes K) */
#define BQ_CFG_SKINNY 33 /* dense, M <= 8: the weight-streaming MFMA kernel */
#define BQ_CFG_SMALLK 18 /* dense or conv, N <= 256 with N % 4 == 0, K <= 256 (ceil(N/16) ceil(K/64) <= 16),
                          * M N < 2^29: the small-K kernel, weights in registers, 16 rows a wave-step
                          * (split 1; the rule's pick from 131072 rows, and from 65536 rows for the int8
                          * twin alone up to 160 columns and for an f32 output of at most 32 or 128 to
                          * 160 columns). Its absmax_parts count is its workgroups. */
int bq_plan_candidates(const int64_t* problem, int n, int32_t* cfgs, int32_t* splits, int cap);
int bq_plan_set(const int64_t* problem, int n, int32_t cfg, int32_t split);
int bq_plan_clear(void);

/* bq_conv2d_i8_nhwc that also writes the output's int8 twin with a calibrated scale:
 * q_out int8 [N, OH, OW, O] = clip(rint(y / s_out[0]), +-127) (exact quotient, half to even) of the final f32 y
 * (after residual and activation), the next conv's input with no quantize pass.
 * O % 16 == 0 (the twin is then the next layer's padded NHWC layout). `out` may be NULL
 * here: the twin alone is written (a consumer that reads nothing else). Replaces the
 * quantOut store of convForwardInt8 / sumSplitsConv (borch-ts/src/kernels.ts:2177-2190,
 * 5866-5898) and the Int8Twin hand-off (tensor.ts:11909-11910, 11954-11955). */
int bq_conv2d_i8_nhwc_q(const int8_t* x, int64_t N, int64_t H, int64_t W, int64_t C, const int8_t* w,
                        int64_t O, int64_t KH, int64_t KW, int64_t stride, int64_t pad, const float* sA,
                        const float* sW, const float* bias, const float* residual, int act, float* out,
                        int32_t* acc, const float* s_out, int8_t* q_out, float* absmax_parts, void* ws,
                        size_t ws_bytes, bq_stream_t stream);

/* The int8 twin of a conv's output at its dynamic per-tensor scale, the f32 output never
 * stored: q_out int8 [N, OH, OW, O] and s_out f32 [1] are, bit for bit, what
 * bq_conv2d_i8_nhwc (with its absmax_parts) followed by bq_quantize_nhwc_parts into O
 * channels gives (s_out = float32(max|y| / 127), q = clip(rint(y / s_out), +-127), exact
 * quotient, half to even). Two launches of the small-K kernel: the first computes every
 * output and stores only its workgroups' maxima into parts (room for parts_cap floats; 4096
 * always suffice), the second computes them again and stores the twin. O % 16 == 0. Only
 * where the small-K kernel runs the twin alone (BQ_CFG_SMALLK: the rule's pick, or a plan's),
 * else BQ_ERR_UNSUPPORTED with nothing launched (the caller takes the two-call form). An
 * empty batch is a no-op. Replaces the conv output's f32 store and the dynamic quantization the next conv's input
 * takes from it (borch-ts/src/tensor.ts:11909-11921: absMaxAtomic and quantizeActivationInt8,
 * kernels.ts:2024-2081, over convForwardInt8's output, kernels.ts:2156-2302). */
int bq_conv2d_i8_nhwc_dq(const int8_t* x, int64_t N, int64_t H, int64_t W, int64_t C, const int8_t* w,
                         int64_t O, int64_t KH, int64_t KW, int64_t stride, int64_t pad, const float* sA,
                         const float* sW, const float* bias, const float* residual, int act, int8_t* q_out,
                         float* s_out, float* parts, int64_t parts_cap, bq_stream_t stream);

/* One convolution of bq_conv2d_i8_nhwc_pair: its filter and epilogue, as the arguments of
 * the same name of bq_conv2d_i8_nhwc_q (s_out and q_out both NULL: no int8 twin, and then
 * `out` is required; `amax` as bq_conv2d_i8_nhwc's absmax_parts, first conv only). */
typedef struct bq_conv_desc {
  const int8_t* w;
  int64_t O, KH, KW, stride, pad;
  const float* sW;
  const float* bias;
  const float* residual;
  int act;
  float* out;
  const float* s_out;
  int8_t* q_out;
  float* amax;
} bq_conv_desc;

/* Two convolutions of one int8 input x [N, H, W, C] (scale sA) in one launch: a residual
 * block's first conv and its downsampling shortcut, which the reference dispatches as two
 * convForwardInt8 passes over the same input (borch-ts/src/kernels.ts:2084-2302; the block
 * of tests/browser/export_resnet18.py:34-43). Each result is bit-identical to that conv's
 * own bq_conv2d_i8_nhwc(_q) call; the second runs on the first's tile configuration and
 * never splits K. Configurations without a paired kernel run as two launches. */
int bq_conv2d_i8_nhwc_pair(const int8_t* x, int64_t N, int64_t H, int64_t W, int64_t C, const float* sA,
                           const bq_conv_desc* a, const bq_conv_desc* b, void* ws, size_t ws_bytes,
                           bq_stream_t stream);

/* Depthwise int8 convolution, NHWC (groups = C, channel multiplier 1):
 *   x int8 [N, H, W, C] (C % 4 == 0, per-tensor sA f32 [1]), w int8 [KH*KW, C]
 *   (per-channel sW f32 [C]), out f32 [N, OH, OW, C] with the same epilogue.
 * Replaces depthwiseForward (borch-ts/src/kernels.ts:5932-5968, f32 there) and
 * dwconv_rows (borch-ts/wasm/src/lib.rs:598-641). */
int bq_dwconv_i8_nhwc(const int8_t* x, int64_t N, int64_t H, int64_t W, int64_t C,
                      const int8_t* w, int64_t KH, int64_t KW, int64_t stride, int64_t pad,
                      const float* sA, const float* sW, const float* bias, int act,
                      float* out, int32_t* acc, bq_stream_t stream);

/* Softmax attention in f32, beside the int8 path (a transformer's heads between its int8
 * qkv and output projections): for every image b and head h,
 *   out[b, t, h*64 + d] = sum_u softmax_u((q_t . k_u) * (1/sqrt(64))) v[u, d]
 * with q, k, v read from the qkv projection's output qkv f32 [B, T, 3, H, 64] (q, k, v of a
 * token side by side, each [H, 64]) and out f32 [B, T, H * 64]. f32 throughout: the
 * exponentials exp(s - max) are summed against v and the result divided by their sum (the
 * reference divides each probability first; the f32 sums run in another order too): within
 * 1e-5 of the output's scale of the float64 result. dh == 64, T <= 256; qkv and out 16-byte
 * aligned.
 * Replaces scaled_dot_product_attention (borch/_nn.py:2143-2170; its softmax is softmaxRows,
 * borch-ts/src/kernels.ts:2483-2532) on that layout. */
int bq_attention_f32(const float* qkv, int64_t B, int64_t T, int64_t H, int64_t dh, float* out, bq_stream_t stream);

/* A classifier head in f32, beside the int8 path: the global average pool of a channels-last
 * activation x f32 [N, HW, C] and the Linear w f32 [O, C], b f32 [O] (nullable) after it:
 *   out f32 [N, O] = b + (sum over the HW pixels of x[n, :, c], pixel order) / HW . w[o, :]
 * one f32 rounding per operation. O * C <= 65536 (a small head: the pool and the product in
 * one launch). Replaces the mean over H, W and the f32 Linear of the configuration's head
 * (tests/browser/export_resnet18.py:56-59; borch/_nn.py:397-415). */
int bq_avgpool_linear_f32(const float* x, int64_t N, int64_t HW, int64_t C, const float* w, const float* b,
                          int64_t O, float* out, bq_stream_t stream);

/* Workspace bytes of bq_se_gate_nhwc for this size (per-chunk partial sums and maxima). */
size_t bq_se_gate_ws_bytes(int64_t N, int64_t HW, int64_t C);

/* The number of floats bq_se_gate_nhwc writes to a non-null `absmax_parts` (one per image). */
int64_t bq_se_gate_absmax_parts(int64_t N, int64_t C);

/* Squeeze-excite gates in f32 of a channels-last activation x f32 [N, HW, C] (C % 4 == 0):
 *   pooled = mean over HW (sum in a fixed order, then * f32(1/HW)),
 *   z = silu(w1 [S, C] . pooled + b1),  gate f32 [N, C] = sigmoid(w2 . z + b2)
 * with the expand weight w2 [C, S] passed transposed as w2t [S, C] (b1, b2 nullable). The
 * gate is then folded into the next conv's input quantization (bq_quantize_nhwc_chscale).
 * absmax_parts (nullable, bq_se_gate_absmax_parts floats) receives partial maxima of
 * |fl(x * gate)| (exact: the gate is positive and rounding monotonic, so per image and
 * channel it is fl(max|x| * gate)), the dynamic scale of that quantization without a pass
 * over x. Replaces the CPU runner's "se" node (meanRows, gemmBiasAct swish and sigmoid;
 * borch-ts/src/cpu/runner.ts:256-268, wasm/src/lib.rs:222-244). */
int bq_se_gate_nhwc(const float* x, int64_t N, int64_t HW, int64_t C, const float* w1, const float* b1, int64_t S,
                    const float* w2t, const float* b2, float* gate, float* absmax_parts, void* ws, size_t ws_bytes,
                    bq_stream_t stream);

/* Weight-only int8 (W8A32) Linear, any M: f32 x [M, K] against int8 W [N, K] with
 * per-channel sW [N]; out f32 [M, N] = act(y + bias[n] + residual[m, n]) with y the f32 sum
 * over k of x * f32(q) * sW[n] (bias, residual nullable; residual f32 [M, N]). M <= 16 (K <=
 * 8192): wave-reduction GEMV kernels, the effective weight f32(f32(q) * sW[n]) per element
 * and f32 FMA / f32-MFMA accumulation, as the reference. Otherwise a tiled bf16-MFMA kernel:
 * q is exact in bf16 and each x is split exactly into three bf16 pieces, so every product is
 * exact; the f32 accumulation is the only rounding before y = fl(sum * sW[n]). Either way
 * every output is within (K + 2) 2^-24 sum_k |x * w| + 2^-24 |y| of the exact result on the
 * effective weights w = f32(q) * sW. The int8 weight is read inside the kernel: no f32 copy
 * of it is written. K % 16 == 0; x and W 16-byte aligned; x and W each < 2 GiB.
 * Replaces matmul(..., weightInt8) (borch-ts/src/kernels.ts:2661-2753, the int8 read at
 * 2695-2708) and its routing (tensor.ts:2553-2575) for streamed / windowed weights
 * (Tensor.inWindowInt8, tensor.ts:1681-1705; stream_sequential(int8=True),
 * borch_webgpu/_stream.py:61-66). */
int bq_linear_w8a32(const float* x, const int8_t* W, int64_t M, int64_t N, int64_t K, const float* sW,
                    const float* bias, const float* residual, int act, float* out, bq_stream_t stream);

/* bq_linear_w8a32's decode-shape kernels alone (M <= 16, K <= 8192, no residual); the same
 * results. Kept for callers bound to it. */
int bq_gemv_w8a32(const float* x, const int8_t* W, int64_t M, int64_t N, int64_t K, const float* sW,
                  const float* bias, int act, float* out, bq_stream_t stream);

/* w f32 [N, K] = f32(q[n, k]) * s[n] (one rounding): the effective weights of a weight-only
 * packing, unpacked (a consumer that needs them in f32). Replaces dequantInt8
 * (borch-ts/src/kernels.ts:1264-1274). */
int bq_dequant_i8(const int8_t* q, int64_t N, int64_t K, const float* s, float* w, bq_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* BQ_H */
