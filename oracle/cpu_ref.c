/*
 * CPU baseline — TEST AND MEASUREMENT INFRASTRUCTURE ONLY (timed by bench.py's
 * cpu_baseline leg; never part of the product).
 *
 * A C restatement of the borch_cpu path's f32 kernels, whose only readable source is the
 * Rust wasm-SIMD module borch-ts/wasm/src/lib.rs (no rustc in this image, and the
 * compiled wasm blobs are off limits):
 *
 *   ref_gemm_bias_act  <- gemm_bias_act + micro<R> (lib.rs:508-584): C[m,n] = A[m,k]·B[k,n]
 *                         + bias[n], activation on the store; 4 rows x 16 columns of
 *                         4-wide accumulators held across all of k, then a 1-row tail;
 *                         n % 16 == 0. `madd` is mul-then-add (the strict module).
 *   ref_im2col_rows    <- im2col_rows (lib.rs:643-678): NHWC, columns tap-major then channel.
 *   ref_dwconv_rows    <- dwconv_rows (lib.rs:598-641): pixel -> 16 channels -> taps, the
 *                         valid tap range decided per row and column; c % 16 == 0.
 *
 * The threaded drivers slice rows across pthreads, as the reference's worker pool slices
 * a GEMM's rows (borch-ts/src/cpu/threads.ts, runner.ts:199-214). Activations: 0 none,
 * 1 relu (act_f32x4 of lib.rs).
 */
#include <pthread.h>
#include <stddef.h>
#include <string.h>

typedef float f32x4 __attribute__((vector_size(16)));

static inline f32x4 splat(float v) { return (f32x4){v, v, v, v}; }
static inline f32x4 ld(const float* p) { f32x4 v; memcpy(&v, p, 16); return v; }
static inline void st(float* p, f32x4 v) { memcpy(p, &v, 16); }
static inline f32x4 madd(f32x4 a, f32x4 b, f32x4 c) { return a * b + c; }
static inline f32x4 act4(f32x4 v, unsigned act) {
  if (act == 1) {
    f32x4 z = splat(0.f);
    return (f32x4){v[0] > 0 ? v[0] : z[0], v[1] > 0 ? v[1] : z[1], v[2] > 0 ? v[2] : z[2], v[3] > 0 ? v[3] : z[3]};
  }
  return v;
}

#define MICRO(R)                                                                                     \
  static void micro##R(size_t k, size_t n, const float* a, const float* b, float* c, size_t j,       \
                       const float* bias, unsigned act) {                                            \
    f32x4 acc[R][4];                                                                                 \
    for (int r = 0; r < R; ++r) acc[r][0] = acc[r][1] = acc[r][2] = acc[r][3] = splat(0.f);          \
    for (size_t p = 0; p < k; ++p) {                                                                 \
      const float* bp = b + p * n + j;                                                               \
      f32x4 b0 = ld(bp), b1 = ld(bp + 4), b2 = ld(bp + 8), b3 = ld(bp + 12);                         \
      for (int r = 0; r < R; ++r) {                                                                  \
        f32x4 s = splat(a[r * k + p]);                                                               \
        acc[r][0] = madd(s, b0, acc[r][0]);                                                          \
        acc[r][1] = madd(s, b1, acc[r][1]);                                                          \
        acc[r][2] = madd(s, b2, acc[r][2]);                                                          \
        acc[r][3] = madd(s, b3, acc[r][3]);                                                          \
      }                                                                                              \
    }                                                                                                \
    f32x4 z = splat(0.f);                                                                            \
    f32x4 bb0 = bias ? ld(bias + j) : z, bb1 = bias ? ld(bias + j + 4) : z;                          \
    f32x4 bb2 = bias ? ld(bias + j + 8) : z, bb3 = bias ? ld(bias + j + 12) : z;                     \
    for (int r = 0; r < R; ++r) {                                                                    \
      float* row = c + r * n + j;                                                                    \
      st(row, act4(acc[r][0] + bb0, act));                                                           \
      st(row + 4, act4(acc[r][1] + bb1, act));                                                       \
      st(row + 8, act4(acc[r][2] + bb2, act));                                                       \
      st(row + 12, act4(acc[r][3] + bb3, act));                                                      \
    }                                                                                                \
  }
MICRO(4)
MICRO(1)

void ref_gemm_bias_act(size_t m, size_t n, size_t k, const float* a, const float* b, float* c, const float* bias,
                       unsigned act) {
  size_t i = 0;
  for (; i + 4 <= m; i += 4)
    for (size_t j = 0; j < n; j += 16) micro4(k, n, a + i * k, b, c + i * n, j, bias, act);
  for (; i < m; ++i)
    for (size_t j = 0; j < n; j += 16) micro1(k, n, a + i * k, b, c + i * n, j, bias, act);
}

void ref_im2col_rows(size_t h, size_t w, size_t c, size_t k, size_t stride, size_t pad, size_t wo, size_t row0,
                     size_t rows, const float* inp, float* out) {
  const size_t kk = k * k;
  for (size_t r = 0; r < rows; ++r) {
    const size_t pix = row0 + r, oy = pix / wo, ox = pix % wo;
    float* row = out + r * kk * c;
    for (size_t ky = 0; ky < k; ++ky) {
      const long iy = (long)(oy * stride + ky) - (long)pad;
      for (size_t kx = 0; kx < k; ++kx) {
        const long ix = (long)(ox * stride + kx) - (long)pad;
        float* dst = row + (ky * k + kx) * c;
        const int inside = iy >= 0 && iy < (long)h && ix >= 0 && ix < (long)w;
        if (inside)
          memcpy(dst, inp + ((size_t)iy * w + (size_t)ix) * c, c * sizeof(float));
        else
          memset(dst, 0, c * sizeof(float));
      }
    }
  }
}

void ref_dwconv_rows(size_t h, size_t w, size_t c, size_t k, size_t stride, size_t pad, size_t wo, size_t oy0,
                     size_t oy1, const float* inp, const float* wt, float* out, const float* bias, unsigned act) {
  for (size_t oy = oy0; oy < oy1; ++oy) {
    const size_t y0 = oy * stride;
    const size_t ky_lo = pad > y0 ? pad - y0 : 0;
    const size_t ky_hi = (h + pad - y0) < k ? (h + pad - y0) : k;
    for (size_t ox = 0; ox < wo; ++ox) {
      const size_t x0 = ox * stride;
      const size_t kx_lo = pad > x0 ? pad - x0 : 0;
      const size_t kx_hi = (w + pad - x0) < k ? (w + pad - x0) : k;
      float* o = out + (oy * wo + ox) * c;
      for (size_t ch = 0; ch < c; ch += 16) {
        f32x4 a0 = ld(bias + ch), a1 = ld(bias + ch + 4), a2 = ld(bias + ch + 8), a3 = ld(bias + ch + 12);
        for (size_t ky = ky_lo; ky < ky_hi; ++ky) {
          const float* row_in = inp + (y0 + ky - pad) * w * c + ch;
          const float* row_w = wt + ky * k * c + ch;
          for (size_t kx = kx_lo; kx < kx_hi; ++kx) {
            const float* ip = row_in + (x0 + kx - pad) * c;
            const float* wp = row_w + kx * c;
            a0 = madd(ld(ip), ld(wp), a0);
            a1 = madd(ld(ip + 4), ld(wp + 4), a1);
            a2 = madd(ld(ip + 8), ld(wp + 8), a2);
            a3 = madd(ld(ip + 12), ld(wp + 12), a3);
          }
        }
        st(o + ch, act4(a0, act));
        st(o + ch + 4, act4(a1, act));
        st(o + ch + 8, act4(a2, act));
        st(o + ch + 12, act4(a3, act));
      }
    }
  }
}

/* ------------------------------------------------------------------ threaded drivers */

typedef struct {
  size_t m0, m1, n, k;
  const float *a, *b, *bias;
  float* c;
  unsigned act;
} gemm_task;

static void* gemm_worker(void* p) {
  gemm_task* t = (gemm_task*)p;
  if (t->m1 > t->m0)
    ref_gemm_bias_act(t->m1 - t->m0, t->n, t->k, t->a + t->m0 * t->k, t->b, t->c + t->m0 * t->n, t->bias, t->act);
  return 0;
}

#define MAX_THREADS 256

/* C = A·B + bias with rows sliced over `threads` pthreads (whole 4-row blocks per slice). */
void ref_gemm_threaded(int threads, size_t m, size_t n, size_t k, const float* a, const float* b, float* c,
                       const float* bias, unsigned act) {
  if (threads < 1) threads = 1;
  if (threads > MAX_THREADS) threads = MAX_THREADS;
  pthread_t th[MAX_THREADS];
  gemm_task task[MAX_THREADS];
  size_t blocks = (m + 3) / 4, per = (blocks + threads - 1) / threads;
  for (int t = 0; t < threads; ++t) {
    size_t m0 = t * per * 4, m1 = (t + 1) * per * 4;
    if (m0 > m) m0 = m;
    if (m1 > m) m1 = m;
    task[t] = (gemm_task){m0, m1, n, k, a, b, bias, c, act};
    pthread_create(&th[t], 0, gemm_worker, &task[t]);
  }
  for (int t = 0; t < threads; ++t) pthread_join(th[t], 0);
}

typedef struct {
  size_t img0, img1, h, w, c, k, stride, pad, ho, wo, cout, block;
  const float *inp, *wcol, *bias;
  float *out, *cols;
  unsigned act;
} conv_task;

static void* conv_worker(void* p) {
  conv_task* t = (conv_task*)p;
  const size_t pix = t->ho * t->wo, kc = t->k * t->k * t->c;
  for (size_t im = t->img0; im < t->img1; ++im) {
    const float* x = t->inp + im * t->h * t->w * t->c;
    float* y = t->out + im * pix * t->cout;
    for (size_t r0 = 0; r0 < pix; r0 += t->block) {
      size_t rows = pix - r0 < t->block ? pix - r0 : t->block;
      ref_im2col_rows(t->h, t->w, t->c, t->k, t->stride, t->pad, t->wo, r0, rows, x, t->cols);
      ref_gemm_bias_act(rows, t->cout, kc, t->cols, t->wcol, y + r0 * t->cout, t->bias, t->act);
    }
  }
  return 0;
}

/* NHWC conv: per image, per block of output rows, im2col_rows then gemm_bias_act (the
 * reference runner's conv step, runner.ts:180-224), images sliced over threads. `wcol`
 * is [k*k*c][cout] (cout % 16 == 0); `cols` is scratch of threads * block * k*k*c floats. */
void ref_conv2d_threaded(int threads, size_t n, size_t h, size_t w, size_t c, size_t k, size_t stride, size_t pad,
                         const float* inp, const float* wcol, size_t cout, const float* bias, unsigned act, float* out,
                         float* cols, size_t block) {
  if (threads < 1) threads = 1;
  if (threads > MAX_THREADS) threads = MAX_THREADS;
  const size_t ho = (h + 2 * pad - k) / stride + 1, wo = (w + 2 * pad - k) / stride + 1;
  pthread_t th[MAX_THREADS];
  conv_task task[MAX_THREADS];
  size_t per = (n + threads - 1) / threads;
  for (int t = 0; t < threads; ++t) {
    size_t i0 = t * per, i1 = (t + 1) * per;
    if (i0 > n) i0 = n;
    if (i1 > n) i1 = n;
    task[t] = (conv_task){i0, i1, h, w, c, k, stride, pad, ho, wo, cout, block, inp, wcol, bias, out,
                          cols + (size_t)t * block * k * k * c, act};
    pthread_create(&th[t], 0, conv_worker, &task[t]);
  }
  for (int t = 0; t < threads; ++t) pthread_join(th[t], 0);
}
