// Host-side weight packing: the per-output-channel int8 quantization of a weight held in
// host memory, for weights that are packed on the host and then copied into a device
// window (Tensor.inWindowInt8 quantizes on the host before the upload,
// borch-ts/src/tensor.ts:1681-1705). Host code only; nothing here touches the GPU.
//
// Three rounding rules:
//   BQ_ROUND_EXACT          s = f32(peak / 127) (correctly rounded), q = rint(w / s) of the
//                           exact quotient, half to even: the bytes of
//                           bq_quantize_weight_per_channel on the device.
//   BQ_ROUND_REFERENCE      borch-ts/src/quant.ts:35-41 as JavaScript evaluates it: scale =
//                           peak / 127 in double (stored as f32), inv = 1 / scale in double,
//                           q = Math.round(w * inv) (a tie toward +inf).
//   BQ_ROUND_REFERENCE_CONV borch-ts/src/quant.ts:88-96: s = f32(peak / 127), q =
//                           Math.round(w / s) with the division in double by the stored f32
//                           scale.
#include <math.h>
#include <stdarg.h>
#include <string.h>

#include <algorithm>
#include <thread>
#include <vector>

#include "bq_common.h"

namespace {

// JavaScript Math.round: the nearest integer, a tie toward +inf. x - floor(x) is exact for
// every double, so the comparison decides a tie exactly.
inline double js_round(double x) {
  const double f = floor(x);
  return (x - f >= 0.5) ? f + 1.0 : f;
}

inline int8_t clamp127(double r) { return (int8_t)(r > 127.0 ? 127.0 : (r < -127.0 ? -127.0 : r)); }

void pack_rows(const float* w, int64_t K, int64_t Kpad, int rule, int8_t* q, float* s, int64_t r0, int64_t r1) {
  for (int64_t n = r0; n < r1; ++n) {
    const float* row = w + n * K;
    int8_t* qr = q + n * Kpad;
    float peak = 0.0f;
    for (int64_t k = 0; k < K; ++k) {
      const float a = fabsf(row[k]);
      if (a > peak) peak = a;
    }
    if (rule == BQ_ROUND_REFERENCE) {
      const double scale = (double)peak / 127.0;
      s[n] = (float)scale;
      if (scale == 0.0) {
        memset(qr, 0, (size_t)K);
      } else {
        const double inv = 1.0 / scale;
        for (int64_t k = 0; k < K; ++k) qr[k] = clamp127(js_round((double)row[k] * inv));
      }
    } else {
      // f32(peak / 127): the float division is correctly rounded (IEEE, no contraction);
      // for the conv rule the double quotient stored as f32 is the same value.
      const float sf = peak / 127.0f;
      s[n] = sf;
      if (sf == 0.0f) {
        memset(qr, 0, (size_t)K);
      } else {
        const double sd = (double)sf;
        if (rule == BQ_ROUND_EXACT) {
          // the double quotient of two floats rounds to an integer exactly as the real
          // quotient does (a non-tie cannot land on k + 1/2 at 53 bits)
          for (int64_t k = 0; k < K; ++k) qr[k] = clamp127(nearbyint((double)row[k] / sd));
        } else {
          for (int64_t k = 0; k < K; ++k) qr[k] = clamp127(js_round((double)row[k] / sd));
        }
      }
    }
    if (Kpad > K) memset(qr + K, 0, (size_t)(Kpad - K));
  }
}

}  // namespace

extern "C" int bq_quantize_weight_host(const float* w, int64_t N, int64_t K, int64_t Kpad, int rule, int8_t* q,
                                       float* s, int nthreads) {
  const char* what = "bq_quantize_weight_host";
  if (N < 0 || K < 0 || Kpad < K) return bq::set_error(BQ_ERR_ARG, "%s: bad sizes (N=%lld K=%lld Kpad=%lld)", what,
                                                       (long long)N, (long long)K, (long long)Kpad);
  if (rule != BQ_ROUND_EXACT && rule != BQ_ROUND_REFERENCE && rule != BQ_ROUND_REFERENCE_CONV)
    return bq::set_error(BQ_ERR_ARG, "%s: unknown rounding rule %d", what, rule);
  if (N == 0) return BQ_OK;
  if ((K && !w) || (Kpad && !q) || !s) return bq::set_error(BQ_ERR_ARG, "%s: null pointer", what);
  int t = nthreads > 0 ? nthreads : (int)std::thread::hardware_concurrency();
  t = std::max(1, std::min<int>(t, 64));
  // below about a million elements a thread costs more to start than it saves
  const int64_t by_size = std::max<int64_t>(1, (N * std::max<int64_t>(K, 1)) >> 20);
  t = (int)std::min<int64_t>({(int64_t)t, N, by_size});
  if (t == 1) {
    pack_rows(w, K, Kpad, rule, q, s, 0, N);
    return BQ_OK;
  }
  std::vector<std::thread> pool;
  pool.reserve(t);
  for (int i = 0; i < t; ++i) {
    const int64_t r0 = N * i / t, r1 = N * (i + 1) / t;
    pool.emplace_back(pack_rows, w, K, Kpad, rule, q, s, r0, r1);
  }
  for (auto& th : pool) th.join();
  return BQ_OK;
}
