/*
 * TEST INFRASTRUCTURE ONLY -- the CPU oracle for the TensorForge GPU hot path.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * this library, and only as the checker (or as the timed CPU baseline).  The
 * product path (tensorforge_amd/) never links, imports or calls it.
 *
 * What it restates (citations are paths in the TensorForge reference tree):
 *
 *  tfo_matmul_fma    acc = +0.0f; for k in 0..K-1: acc = fmaf(A[m,k], B[k,n], acc)
 *                    The arithmetic of every reference GPU kernel (naive and
 *                    staged, any BK) and of the vectorized CPU pipeline: they are
 *                    bitwise identical to each other (docs/numerics.md:13-25, 53;
 *                    results/numerics/e1.csv rows gpu-naive, gpu-staged-bk8/16/32, cpu-vec-kr1/kr4).
 *                    Accumulator init +0.0 from lib/Conversion/TForgeToLinalg.cpp:31-35.
 *  tfo_matmul_nofma  acc = +0.0f; acc = acc + (float)(A[m,k] * B[k,n]), each product
 *                    rounded before the add: the reference's default CPU pipeline
 *                    (cpu-scalar in results/numerics/e1.csv; docs/numerics.md:15).
 *  tfo_matmul_scalar_mnk  the same arithmetic in the default pipeline's loop
 *                    order (one output at a time, k innermost), for timing.
 *  tfo_epilogue      y = C + bias[n]  (tforge.bias_add, lib/Conversion/TForgeToLinalg.cpp:113-133)
 *                    y = maximum(y, +0.0)  IEEE-754-2019 maximum: NaN -> NaN,
 *                        -0 -> +0 (tforge.relu, docs/dialect.md:26-30;
 *                        lib/Conversion/TForgeToLinalg.cpp:94-111)
 *                    y = y + R[m,n]  (tforge.add, lib/Conversion/TForgeToLinalg.cpp:76-92)
 *  tfo_mbr_vec6x16   a port of the reference's fastest CPU configuration,
 *                    "fuse-elementwise=1 reg-tile=6,16,4 vectorize=1"
 *                    (docs/stage6.md:9-18): a 6x16 register tile, K step 4, FMA,
 *                    fused bias+relu.  Its per-output k order is sequential, so it
 *                    is bitwise equal to tfo_matmul_fma + tfo_epilogue; it exists to
 *                    time the CPU baseline, and is itself checked against the
 *                    closed form.
 *
 * The sequential closed forms are parallelised over rows only (each output's
 * k order is untouched), so their bits do not depend on the thread count.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#ifdef _OPENMP
#include <omp.h>
#endif
#if defined(__AVX2__) && defined(__FMA__)
#include <immintrin.h>
#define TFO_HAVE_AVX2 1
#else
#define TFO_HAVE_AVX2 0
#endif

#define TFO_BIAS 1
#define TFO_RELU 2
#define TFO_RESID 4

static void set_threads(int threads) {
#ifdef _OPENMP
  omp_set_num_threads(threads > 0 ? threads : omp_get_num_procs());
#else
  (void)threads;
#endif
}

/* IEEE-754-2019 maximum(x, +0.0): NaN propagates, -0.0 < +0.0. */
static inline float relu_ieee(float x) {
  if (x != x) return x;
  return x > 0.0f ? x : 0.0f;
}

void tfo_matmul_fma(const float *A, const float *B, float *C, long M, long N, long K,
                    int threads) {
  set_threads(threads);
#pragma omp parallel for schedule(static)
  for (long m = 0; m < M; ++m) {
    float *c = C + m * N;
    for (long n = 0; n < N; ++n) c[n] = 0.0f;
    for (long k = 0; k < K; ++k) {
      const float a = A[m * K + k];
      const float *b = B + k * N;
      for (long n = 0; n < N; ++n) c[n] = fmaf(a, b[n], c[n]);
    }
  }
}

/* Built with -ffp-contract=off (see Makefile) so the product is rounded before
 * the add, as in the reference's scalar CPU code. */
void tfo_matmul_nofma(const float *A, const float *B, float *C, long M, long N, long K,
                      int threads) {
  set_threads(threads);
#pragma omp parallel for schedule(static)
  for (long m = 0; m < M; ++m) {
    float *c = C + m * N;
    for (long n = 0; n < N; ++n) c[n] = 0.0f;
    for (long k = 0; k < K; ++k) {
      const float a = A[m * K + k];
      const float *b = B + k * N;
      for (long n = 0; n < N; ++n) {
        float p = a * b[n];
        c[n] = c[n] + p;
      }
    }
  }
}

/* The same closed form in the reference's default CPU loop order: one output at
 * a time (m, n outer; k inner, B read down a column), scalar, no FMA
 * (--tforge-cpu-pipeline defaults; docs/stage4.md:63 times it at ~0.6 GFLOP/s).
 * Bitwise equal to tfo_matmul_nofma; it exists to time the scalar baseline. */
void tfo_matmul_scalar_mnk(const float *A, const float *B, float *C, long M, long N, long K) {
  for (long m = 0; m < M; ++m)
    for (long n = 0; n < N; ++n) {
      float acc = 0.0f;
      for (long k = 0; k < K; ++k) {
        float p = A[m * K + k] * B[k * N + n];
        acc = acc + p;
      }
      C[m * N + n] = acc;
    }
}

void tfo_epilogue(float *C, const float *bias, const float *R, long M, long N, int flags) {
  for (long m = 0; m < M; ++m) {
    float *c = C + m * N;
    for (long n = 0; n < N; ++n) {
      float y = c[n];
      if (flags & TFO_BIAS) y = y + bias[n];
      if (flags & TFO_RELU) y = relu_ieee(y);
      if (flags & TFO_RESID) y = y + R[m * N + n];
      c[n] = y;
    }
  }
}

/* Elementwise ops on their own (tforge.add / relu / bias_add), one IEEE op each. */
void tfo_add(const float *X, const float *Y, float *O, long count) {
  for (long i = 0; i < count; ++i) O[i] = X[i] + Y[i];
}
void tfo_relu(const float *X, float *O, long count) {
  for (long i = 0; i < count; ++i) O[i] = relu_ieee(X[i]);
}
void tfo_bias_add(const float *X, const float *bias, float *O, long M, long N) {
  for (long m = 0; m < M; ++m)
    for (long n = 0; n < N; ++n) O[m * N + n] = X[m * N + n] + bias[n];
}

/* ---- port of the reference's 6x16x4 vectorized CPU kernel (fused bias+relu) ---- */

static void tile_scalar(const float *A, const float *B, const float *bias, float *C,
                        long N, long K, long m0, long mr, long n0, long nr, int flags) {
  for (long i = 0; i < mr; ++i)
    for (long j = 0; j < nr; ++j) {
      float acc = 0.0f;
      for (long k = 0; k < K; ++k) acc = fmaf(A[(m0 + i) * K + k], B[k * N + n0 + j], acc);
      float y = acc;
      if (flags & TFO_BIAS) y = y + bias[n0 + j];
      if (flags & TFO_RELU) y = relu_ieee(y);
      C[(m0 + i) * N + n0 + j] = y;
    }
}

#if TFO_HAVE_AVX2
static inline __m256 relu8(__m256 y) {
  /* maximum(y, +0): lanes with y > 0 keep y, NaN lanes keep y, the rest are +0. */
  __m256 zero = _mm256_setzero_ps();
  __m256 keep = _mm256_or_ps(_mm256_cmp_ps(y, zero, _CMP_GT_OQ), _mm256_cmp_ps(y, y, _CMP_UNORD_Q));
  return _mm256_and_ps(keep, y);
}

static void tile6x16(const float *A, const float *B, const float *bias, float *C, long N,
                     long K, long m0, long n0, int flags) {
  __m256 c[6][2];
  for (int i = 0; i < 6; ++i) c[i][0] = c[i][1] = _mm256_setzero_ps();
  const float *a = A + m0 * K;
  long k = 0;
  for (; k + 4 <= K; k += 4) {
    for (int kk = 0; kk < 4; ++kk) {
      const float *b = B + (k + kk) * N + n0;
      __m256 b0 = _mm256_loadu_ps(b), b1 = _mm256_loadu_ps(b + 8);
      for (int i = 0; i < 6; ++i) {
        __m256 ai = _mm256_broadcast_ss(a + i * K + k + kk);
        c[i][0] = _mm256_fmadd_ps(ai, b0, c[i][0]);
        c[i][1] = _mm256_fmadd_ps(ai, b1, c[i][1]);
      }
    }
  }
  for (; k < K; ++k) {
    const float *b = B + k * N + n0;
    __m256 b0 = _mm256_loadu_ps(b), b1 = _mm256_loadu_ps(b + 8);
    for (int i = 0; i < 6; ++i) {
      __m256 ai = _mm256_broadcast_ss(a + i * K + k);
      c[i][0] = _mm256_fmadd_ps(ai, b0, c[i][0]);
      c[i][1] = _mm256_fmadd_ps(ai, b1, c[i][1]);
    }
  }
  __m256 bb0 = _mm256_setzero_ps(), bb1 = _mm256_setzero_ps();
  if (flags & TFO_BIAS) {
    bb0 = _mm256_loadu_ps(bias + n0);
    bb1 = _mm256_loadu_ps(bias + n0 + 8);
  }
  for (int i = 0; i < 6; ++i) {
    __m256 y0 = c[i][0], y1 = c[i][1];
    if (flags & TFO_BIAS) {
      y0 = _mm256_add_ps(y0, bb0);
      y1 = _mm256_add_ps(y1, bb1);
    }
    if (flags & TFO_RELU) {
      y0 = relu8(y0);
      y1 = relu8(y1);
    }
    _mm256_storeu_ps(C + (m0 + i) * N + n0, y0);
    _mm256_storeu_ps(C + (m0 + i) * N + n0 + 8, y1);
  }
}
#endif

int tfo_have_avx2(void) { return TFO_HAVE_AVX2; }

/* C = [relu](A @ B [+ bias]) with 6x16 register tiles; edge strips in scalar FMA. */
void tfo_mbr_vec6x16(const float *A, const float *B, const float *bias, float *C, long M,
                     long N, long K, int flags, int threads) {
  set_threads(threads);
  const long mfull = M - M % 6, nfull = N - N % 16;
#pragma omp parallel for schedule(static)
  for (long m0 = 0; m0 < mfull; m0 += 6) {
#if TFO_HAVE_AVX2
    for (long n0 = 0; n0 < nfull; n0 += 16) tile6x16(A, B, bias, C, N, K, m0, n0, flags);
#else
    for (long n0 = 0; n0 < nfull; n0 += 16) tile_scalar(A, B, bias, C, N, K, m0, 6, n0, 16, flags);
#endif
    if (nfull < N) tile_scalar(A, B, bias, C, N, K, m0, 6, nfull, N - nfull, flags);
  }
  if (mfull < M) tile_scalar(A, B, bias, C, N, K, mfull, M - mfull, 0, N, flags);
}

/* Median wall time (ns) of `reps` calls of tfo_mbr_vec6x16 (1 thread) after
 * `warmup` calls, steady clock, as the reference's CPU runner times
 * (runners/cpu/tforge-cpu-bench.cpp:255-263). */
static int cmp_d(const void *a, const void *b) {
  double x = *(const double *)a, y = *(const double *)b;
  return (x > y) - (x < y);
}
double tfo_time_mbr_vec6x16(const float *A, const float *B, const float *bias, float *C,
                            long M, long N, long K, int flags, int warmup, int reps) {
  double ts[1024];
  if (reps > 1024) reps = 1024;
  if (reps < 1) reps = 1;
  for (int i = 0; i < warmup; ++i) tfo_mbr_vec6x16(A, B, bias, C, M, N, K, flags, 1);
  for (int i = 0; i < reps; ++i) {
    struct timespec t0, t1;
    clock_gettime(CLOCK_MONOTONIC, &t0);
    tfo_mbr_vec6x16(A, B, bias, C, M, N, K, flags, 1);
    clock_gettime(CLOCK_MONOTONIC, &t1);
    ts[i] = (t1.tv_sec - t0.tv_sec) * 1e9 + (t1.tv_nsec - t0.tv_nsec);
  }
  qsort(ts, reps, sizeof(double), cmp_d);
  return reps % 2 ? ts[reps / 2] : 0.5 * (ts[reps / 2 - 1] + ts[reps / 2]);
}

/* Same for the scalar (m, n, k) no-FMA loop plus its separate epilogue (the
 * reference's default CPU pipeline), 1 thread. */
double tfo_time_scalar(const float *A, const float *B, const float *bias, float *C, long M,
                       long N, long K, int flags, int warmup, int reps) {
  double ts[1024];
  if (reps > 1024) reps = 1024;
  if (reps < 1) reps = 1;
  for (int i = 0; i < warmup + reps; ++i) {
    struct timespec t0, t1;
    clock_gettime(CLOCK_MONOTONIC, &t0);
    tfo_matmul_scalar_mnk(A, B, C, M, N, K);
    if (flags) tfo_epilogue(C, bias, 0, M, N, flags);
    clock_gettime(CLOCK_MONOTONIC, &t1);
    if (i >= warmup) ts[i - warmup] = (t1.tv_sec - t0.tv_sec) * 1e9 + (t1.tv_nsec - t0.tv_nsec);
  }
  qsort(ts, reps, sizeof(double), cmp_d);
  return reps % 2 ? ts[reps / 2] : 0.5 * (ts[reps / 2 - 1] + ts[reps / 2]);
}
