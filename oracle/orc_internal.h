/* orc_internal.h -- shared helpers of the oracle (test infrastructure). */
#ifndef MX_ORC_INTERNAL_H
#define MX_ORC_INTERNAL_H

#include "oracle.h"

#include <immintrin.h>
#include <math.h>
#include <stdint.h>
#include <string.h>

typedef void (*orc_task_fn)(void *arg, int w, int nw);
/* Call fn(arg, w, nw) once per pool worker and wait for all of them. */
void orc_run(orc_task_fn fn, void *arg);
/* Contiguous block [lo, hi) of n items for worker w of nw. */
void orc_range(int64_t n, int w, int nw, int64_t *lo, int64_t *hi);

/* hsum256 (host_kernels.hpp:617-623): lo+hi halves, then two hadds. */
static inline float orc_hsum256(__m256 v) {
  __m128 lo = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
  lo = _mm_hadd_ps(lo, lo);
  lo = _mm_hadd_ps(lo, lo);
  return _mm_cvtss_f32(lo);
}

/* exp2_avx2 (host_kernels.hpp:358-379): k = trunc(x), f = x - k, degree-7
 * Horner by FMA, times 2^k built in the exponent field. */
static inline __m256 orc_exp2_v(__m256 x) {
  const __m256i k = _mm256_cvttps_epi32(x);
  const __m256 f = _mm256_sub_ps(x, _mm256_cvtepi32_ps(k));
  __m256 p = _mm256_fmadd_ps(_mm256_set1_ps(1.5483275463e-05f), f,
                             _mm256_set1_ps(1.5669833174e-04f));
  p = _mm256_fmadd_ps(p, f, _mm256_set1_ps(1.3331825236e-03f));
  p = _mm256_fmadd_ps(p, f, _mm256_set1_ps(9.6164605538e-03f));
  p = _mm256_fmadd_ps(p, f, _mm256_set1_ps(5.5504156855e-02f));
  p = _mm256_fmadd_ps(p, f, _mm256_set1_ps(2.4022684109e-01f));
  p = _mm256_fmadd_ps(p, f, _mm256_set1_ps(6.9314717694e-01f));
  p = _mm256_fmadd_ps(p, f, _mm256_set1_ps(9.9999998955e-01f));
  const __m256i bits =
      _mm256_slli_epi32(_mm256_add_epi32(k, _mm256_set1_epi32(127)), 23);
  return _mm256_mul_ps(p, _mm256_castsi256_ps(bits));
}

/* The same polynomial for one lane, with the same operation order. */
static inline float orc_exp2_s(float x) {
  const int32_t k = (int32_t)x; /* trunc, like cvttps */
  const float f = x - (float)k;
  float p = fmaf(1.5483275463e-05f, f, 1.5669833174e-04f);
  p = fmaf(p, f, 1.3331825236e-03f);
  p = fmaf(p, f, 9.6164605538e-03f);
  p = fmaf(p, f, 5.5504156855e-02f);
  p = fmaf(p, f, 2.4022684109e-01f);
  p = fmaf(p, f, 6.9314717694e-01f);
  p = fmaf(p, f, 9.9999998955e-01f);
  uint32_t b = (uint32_t)(k + 127) << 23;
  float s;
  memcpy(&s, &b, 4);
  return p * s;
}

#endif
