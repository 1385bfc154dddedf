/*
 * libbqprobe — measurement probes for bench.py (not part of the drop-in boundary; no
 * counterpart in the reference). They measure what one MI355X sustains on the day, so that
 * the kernels' roofline fractions can be read against it as well as against the nominal
 * peaks:
 *   - the int8 MFMA rate on given operand bytes with no memory traffic in the loop (the
 *     MFMA pipe's clock falls with the power its operands draw);
 *   - the duration of a plain streaming read of a buffer (the floor of any kernel that must
 *     read those bytes once, launch and drain included).
 * Same conventions as bq.h: device pointers, a hipStream_t, 0 or a negative BQ_ERR_* code,
 * the message in bqp_last_error(), no host synchronisation.
 */
#ifndef BQ_PROBE_H
#define BQ_PROBE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The message of the last failing probe call on this thread ("" if none). */
const char* bqp_last_error(void);

/* Runs `blocks` workgroups of 8 waves on fragments loaded once from A[0 .. a_bytes) and
 * W[0 .. w_bytes), in one of the 256x256 GEMM tile's per-wave shapes:
 *   form 32: iters * 32 v_mfma_i32_32x32x32_i8 (4 x 2 accumulators, 4 fragment sets);
 *   form 16: iters * 64 v_mfma_i32_16x16x64_i8 (8 x 4 accumulators, 2 fragment sets).
 * Integer ops = blocks * 8 * iters * 2097152 either way. `sink` receives one int per lane
 * (blocks * 512 ints) so that nothing is optimised away. a_bytes and w_bytes must be
 * multiples of 16 and at least 4096; A and W 16-byte aligned. */
int bqp_mfma_rate(const int8_t* A, int64_t a_bytes, const int8_t* W, int64_t w_bytes, int form, int blocks,
                  int iters, int32_t* sink, void* stream);

/* Reads src[0 .. bytes) once: 256-thread workgroups, each lane issuing `chunks` 16-byte
 * loads (1..8) before it uses any, one int of XOR-folded data per workgroup into sink
 * (ceil(bytes / (4096 * chunks)) ints). bytes must be a multiple of 16; src 16-byte aligned. */
int bqp_stream_read(const void* src, int64_t bytes, int chunks, int32_t* sink, void* stream);

#ifdef __cplusplus
}
#endif

#endif
