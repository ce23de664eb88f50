/*
 * orc_numerics.c -- bf16 rounding, GELU, exp2 and the AIE eltwise kernels,
 * restated on the CPU. TEST INFRASTRUCTURE (the oracle); see oracle.h.
 *
 * Built with -ffp-contract=off: every FMA the reference's own build performs
 * (explicit _mm256_fmadd_ps, or a `p * u + c` that GCC contracts under
 * -march=x86-64-v3) is written here as fmaf/fma, and every unfused AIE
 * multiply-then-add stays unfused.
 */
#include "orc_internal.h"

#include <stdlib.h>

/* host_kernels.hpp:157-161 */
uint16_t orc_to_bf16(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

/* host_kernels.hpp:162-167 */
float orc_from_bf16(uint16_t h) {
  const uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

void orc_bf16_fill(uint16_t *dst, const float *src, size_t n) {
  for (size_t i = 0; i < n; ++i) dst[i] = orc_to_bf16(src[i]);
}

void orc_bf16_read(float *dst, const uint16_t *src, size_t n) {
  for (size_t i = 0; i < n; ++i) dst[i] = orc_from_bf16(src[i]);
}

void orc_round_bf16_inplace(float *x, size_t n) {
  for (size_t i = 0; i < n; ++i) x[i] = orc_from_bf16(orc_to_bf16(x[i]));
}

/* The AVX2 lane semantics of gelu_cpu's vector branch
 * (bert_encoder.cpp:547-570): u = min_ps(|v|, 4) and max_ps(v, 0), which
 * return their SECOND operand when the first is NaN. */
static inline float gelu8_lane(float v) {
  const float av = fabsf(v);
  const float u = av < 4.0f ? av : 4.0f;
  float pl = fmaf(-7.2340282171e-05f, u, 1.8179518005e-03f);
  pl = fmaf(pl, u, -1.7707383379e-02f);
  pl = fmaf(pl, u, 8.4577147641e-02f);
  pl = fmaf(pl, u, -1.9228671834e-01f);
  pl = fmaf(pl, u, 9.8431124458e-02f);
  pl = fmaf(pl, u, 3.6137852062e-01f);
  pl = fmaf(pl, u, -4.9454128936e-01f);
  pl = fmaf(pl, u, -1.3007010117e-04f);
  const float pos = v > 0.0f ? v : 0.0f;
  return pos + pl;
}

float orc_gelu8(float x) { return gelu8_lane(x); }

typedef struct { float *x; size_t n; int erf; } gelu_task;

static void gelu_worker(void *p, int w, int nw) {
  const gelu_task *t = (const gelu_task *)p;
  int64_t lo, hi;
  orc_range((int64_t)t->n, w, nw, &lo, &hi);
  if (t->erf) {
    for (int64_t i = lo; i < hi; ++i) t->x[i] = orc_gelu_erf_exact(t->x[i]);
  } else {
    for (int64_t i = lo; i < hi; ++i) t->x[i] = gelu8_lane(t->x[i]);
  }
}

void orc_gelu_poly_inplace(float *x, size_t n) {
  gelu_task t = {x, n, 0};
  orc_run(gelu_worker, &t);
}

/* app_state.hpp:116-120 */
float orc_gelu_erf_exact(float x) {
  const double xd = (double)x;
  return (float)(0.5 * xd * (1.0 + erf(xd * 0.70710678118654752440)));
}

void orc_gelu_erf_inplace(float *x, size_t n) {
  gelu_task t = {x, n, 1};
  orc_run(gelu_worker, &t);
}

void orc_exp2_poly(const float *x, float *y, size_t n) {
  size_t i = 0;
  for (; i + 8 <= n; i += 8)
    _mm256_storeu_ps(y + i, orc_exp2_v(_mm256_loadu_ps(x + i)));
  for (; i < n; ++i) y[i] = orc_exp2_s(x[i]);
}

/* ---- AIE kernel restatements --------------------------------------------- */

/* exp2_poly (kernels/exp2_poly.h:35-65): the same degree-7 table, each step a
 * multiply then an add (two roundings), k = trunc(x). */
static inline float aie_exp2(float x) {
  const int32_t k = (int32_t)x;
  const float f = x - (float)k;
  float p = 1.5483275463e-05f;
  p = p * f + 1.5669833174e-04f;
  p = p * f + 1.3331825236e-03f;
  p = p * f + 9.6164605538e-03f;
  p = p * f + 5.5504156855e-02f;
  p = p * f + 2.4022684109e-01f;
  p = p * f + 6.9314717694e-01f;
  p = p * f + 9.9999998955e-01f;
  const uint32_t b = (uint32_t)(k + 127) << 23;
  float s;
  memcpy(&s, &b, 4);
  return p * s;
}

static inline float bf(float x) { return orc_from_bf16(orc_to_bf16(x)); }

/* aie::reduce_add of a 16-lane fp32 accumulator, the last step of the AIE
 * kernels' sums (softmax.cc:115-145, layernorm.cc:85-142). The AIE API that
 * defines reduce_add is not part of the reference (it ships in the mlir-aie
 * wheel, mlir_aie_no_rtti 1.4.3.dev55+g10767b5), so its order is not known:
 * this adds lane 0 to lane 15 one after another. PARITY UNPINNED for this
 * order (a hardware reduction may well be a pairwise tree); everything ahead
 * of it -- which element lands in which lane, each lane's own in-order sum --
 * follows the kernel source. The GPU kernels use the same order, so they are
 * bit-exact against this restatement, not against the array. */
static float aie_reduce_add16(const float acc[16]) {
  float s = 0.0f;
  for (int l = 0; l < 16; ++l) s += acc[l];
  return s;
}

/* softmax.cc:76-160 with softmax_rne.cc's conv_even. The exponentials are
 * summed as the 16-lane accumulator holds them (:115-145): element j into
 * partial sum j % 16, in element order, then aie_reduce_add16. */
void orc_aie_softmax_bf16(const uint16_t *in, uint16_t *out, int64_t rows,
                          int64_t cols) {
  const float lo = bf(-1.0e30f);
  float *e = (float *)malloc((size_t)cols * sizeof(float));
  for (int64_t r = 0; r < rows; ++r) {
    const uint16_t *x = in + r * cols;
    uint16_t *o = out + r * cols;
    float m = -1.0e30f;
    for (int64_t j = 0; j < cols; ++j) {
      float v = orc_from_bf16(x[j]);
      v = v > lo ? v : lo;
      m = v > m ? v : m;
    }
    float acc[16] = {0};
    for (int64_t j = 0; j < cols; ++j) {
      float v = orc_from_bf16(x[j]);
      v = v > lo ? v : lo;
      float d = v - m;
      d = d > -100.0f ? d : -100.0f;
      float a = d * 1.4426950408889634f;
      a = a > -120.0f ? a : -120.0f;
      e[j] = bf(aie_exp2(a));
      acc[j % 16] += e[j];
    }
    const float sum = aie_reduce_add16(acc);
    const float inv = 1.0f / sum;
    for (int64_t j = 0; j < cols; ++j) o[j] = orc_to_bf16(e[j] * inv);
  }
  free(e);
}

/* layernorm.cc:65-75 */
static inline float fast_invsqrt(float x) {
  const float xhalf = 0.5f * x;
  int32_t i;
  memcpy(&i, &x, 4);
  i = 0x5f3759df - (i >> 1);
  float y;
  memcpy(&y, &i, 4);
  y = y * (1.5f - xhalf * y * y);
  y = y * (1.5f - xhalf * y * y);
  return y;
}

/* layernorm.cc:85-142 with layernorm_rne.cc's conv_even. */
void orc_aie_layernorm_bf16(const uint16_t *in, uint16_t *out, int64_t rows,
                            int64_t cols, const float *gamma,
                            const float *beta, float eps) {
  const float inv_cols = 1.0f / (float)cols;
  for (int64_t r = 0; r < rows; ++r) {
    const uint16_t *x = in + r * cols;
    uint16_t *o = out + r * cols;
    /* 16-lane accumulators, then one reduction, as the AIE vector code. */
    float acc[16] = {0};
    for (int64_t j = 0; j < cols; ++j) acc[j % 16] += orc_from_bf16(x[j]);
    const float mean = aie_reduce_add16(acc) * inv_cols;
    float acc2[16] = {0};
    for (int64_t j = 0; j < cols; ++j) {
      const float d = orc_from_bf16(x[j]) - mean;
      acc2[j % 16] += d * d;
    }
    const float var = aie_reduce_add16(acc2) * inv_cols;
    const float is = fast_invsqrt(var + eps);
    for (int64_t j = 0; j < cols; ++j) {
      const float d = orc_from_bf16(x[j]) - mean;
      const float y = (d * is) * gamma[j] + beta[j];
      o[j] = orc_to_bf16(y);
    }
  }
}

/* gelu_erf.cc:79-145 */
void orc_aie_gelu_erf_bf16(const uint16_t *in, uint16_t *out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    const float x = orc_from_bf16(in[i]);
    const float u = x * 0.70710678118654752440f;
    const float au = fabsf(u);
    const float t = 1.0f / (1.0f + 0.3275911f * au);
    float p = 1.061405429f;
    p = p * t + -1.453152027f;
    p = p * t + 1.421413741f;
    p = p * t + -0.284496736f;
    p = p * t + 0.254829592f;
    float z = (0.0f - u * u) * 1.4426950408889634f;
    z = z > -125.0f ? z : -125.0f;
    const float ex = aie_exp2(z);
    const float tp = t * p;
    const float eabs = 1.0f - tp * ex;
    const float y = x * 0.5f + (fabsf(x) * 0.5f) * eabs;
    out[i] = orc_to_bf16(y);
  }
}

/* gelu_poly.cc:77-176 (gelu_poly_rne.cc:55-67): multiply then add per step. */
void orc_aie_gelu_poly_bf16(const uint16_t *in, uint16_t *out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    const float x = orc_from_bf16(in[i]);
    const float ax = fabsf(x);
    const float u = ax < 4.0f ? ax : 4.0f;
    float p = -7.2340282171e-05f;
    p = p * u + 1.8179518005e-03f;
    p = p * u + -1.7707383379e-02f;
    p = p * u + 8.4577147641e-02f;
    p = p * u + -1.9228671834e-01f;
    p = p * u + 9.8431124458e-02f;
    p = p * u + 3.6137852062e-01f;
    p = p * u + -4.9454128936e-01f;
    p = p * u + -1.3007010117e-04f;
    out[i] = orc_to_bf16((x > 0.0f ? x : 0.0f) + p);
  }
}

void orc_narrow_f32_bf16(const float *in, uint16_t *out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = orc_to_bf16(in[i]);
}

/* One rounding, nearest-even, computed on the integer itself: keep the top
 * 8 significant bits of |v| and round the dropped ones. */
static uint16_t i32_to_bf16_once(int32_t v) {
  if (v == 0) return 0;
  const uint32_t sign = v < 0 ? 0x8000u : 0u;
  uint64_t a = v < 0 ? (uint64_t)(-(int64_t)v) : (uint64_t)v;
  int e = 63 - __builtin_clzll(a); /* floor(log2 a) */
  uint64_t mant;                   /* 8 significant bits incl. the leading 1 */
  if (e <= 7) {
    mant = a << (7 - e);
  } else {
    const int sh = e - 7;
    mant = a >> sh;
    const uint64_t rem = a & ((1ull << sh) - 1);
    const uint64_t half = 1ull << (sh - 1);
    if (rem > half || (rem == half && (mant & 1))) mant++;
    if (mant == 256) { mant = 128; e++; }
  }
  const uint32_t exp_field = (uint32_t)(e + 127);
  return (uint16_t)(sign | (exp_field << 7) | (uint32_t)(mant & 0x7F));
}

void orc_narrow_i32_bf16(const int32_t *in, uint16_t *out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = i32_to_bf16_once(in[i]);
}

void orc_narrow_i32_bf16_twice(const int32_t *in, uint16_t *out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = orc_to_bf16((float)in[i]);
}
