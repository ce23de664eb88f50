/*
 * orc_ops.c -- the host encoder's per-op kernels, restated. TEST
 * INFRASTRUCTURE (the oracle); see oracle.h for what pins each one.
 */
#include "orc_internal.h"

#include <stdlib.h>

/* ---- GEMM: hostconv::gemm_nt (conv_host.hpp:148-181) ---------------------- */
typedef struct {
  const float *A, *B, *bias;
  float *C;
  int64_t M, K, N;
} gemm_task;

enum { kMR = 8 };

static void gemm_worker(void *p, int w, int nw) {
  const gemm_task *t = (const gemm_task *)p;
  const int64_t N = t->N, K = t->K;
  float *acc = (float *)malloc((size_t)kMR * (size_t)N * sizeof(float));
  for (int64_t m0 = (int64_t)w * kMR; m0 < t->M; m0 += (int64_t)nw * kMR) {
    const int64_t mr = t->M - m0 < kMR ? t->M - m0 : kMR;
    memset(acc, 0, (size_t)mr * (size_t)N * sizeof(float));
    const float *abase = t->A + m0 * K;
    for (int64_t k = 0; k < K; ++k) {
      const float *brow = t->B + k * N;
      for (int64_t r = 0; r < mr; ++r) {
        const float a = abase[r * K + k];
        float *ar = acc + r * N;
        for (int64_t n = 0; n < N; ++n) ar[n] = fmaf(a, brow[n], ar[n]);
      }
    }
    for (int64_t r = 0; r < mr; ++r) {
      float *crow = t->C + (m0 + r) * N;
      const float *ar = acc + r * N;
      for (int64_t n = 0; n < N; ++n)
        crow[n] = ar[n] + (t->bias ? t->bias[n] : 0.0f);
    }
  }
  free(acc);
}

void orc_gemm_nt(const float *A, int64_t M, const float *B, int64_t K,
                 int64_t N, const float *bias, float *C) {
  gemm_task t = {A, B, bias, C, M, K, N};
  orc_run(gemm_worker, &t);
}

/* ---- LayerNorm ------------------------------------------------------------ */
typedef struct {
  float *x;
  const float *g, *b, *y, *res;
  int64_t rows, cols;
  float eps;
  double eps_d;
} ln_task;

/* layer_norm_cpu's AVX2 branch (bert_encoder.cpp:426-447). */
static void ln_row_avx2(float *row, int64_t H, const float *g, const float *b,
                        float eps) {
  __m256 s = _mm256_setzero_ps();
  for (int64_t j = 0; j < H; j += 8) s = _mm256_add_ps(s, _mm256_loadu_ps(row + j));
  const float mean = orc_hsum256(s) / (float)H;
  const __m256 mv = _mm256_set1_ps(mean);
  __m256 v = _mm256_setzero_ps();
  for (int64_t j = 0; j < H; j += 8) {
    const __m256 d = _mm256_sub_ps(_mm256_loadu_ps(row + j), mv);
    v = _mm256_fmadd_ps(d, d, v);
  }
  const float var = orc_hsum256(v) / (float)H;
  const __m256 is = _mm256_set1_ps(1.0f / sqrtf(var + eps));
  for (int64_t j = 0; j < H; j += 8) {
    const __m256 d = _mm256_sub_ps(_mm256_loadu_ps(row + j), mv);
    const __m256 y = _mm256_fmadd_ps(_mm256_mul_ps(d, is), _mm256_loadu_ps(g + j),
                                     _mm256_loadu_ps(b + j));
    _mm256_storeu_ps(row + j, y);
  }
}

static void ln_worker(void *p, int w, int nw) {
  const ln_task *t = (const ln_task *)p;
  int64_t lo, hi;
  orc_range(t->rows, w, nw, &lo, &hi);
  for (int64_t r = lo; r < hi; ++r)
    ln_row_avx2(t->x + r * t->cols, t->cols, t->g, t->b, t->eps);
}

void orc_layer_norm_rows(float *x, int64_t rows, int64_t cols,
                         const float *gamma, const float *beta, float eps) {
  ln_task t = {x, gamma, beta, NULL, NULL, rows, cols, eps, 0.0};
  orc_run(ln_worker, &t);
}

/* layernorm_rows (npu_ops.cpp:449-468). */
static void ln64_worker(void *p, int w, int nw) {
  const ln_task *t = (const ln_task *)p;
  const int64_t d = t->cols;
  for (int64_t r = w; r < t->rows; r += nw) {
    float *row = t->x + r * d;
    double sm = 0.0;
    for (int64_t j = 0; j < d; ++j) sm += row[j];
    const float mean = (float)(sm / (double)d);
    double sv = 0.0;
    for (int64_t j = 0; j < d; ++j) {
      const double dd = (double)row[j] - (double)mean;
      sv = fma(dd, dd, sv);
    }
    const float var = (float)(sv / (double)d);
    const float is = 1.0f / sqrtf(var + (float)t->eps_d);
    for (int64_t j = 0; j < d; ++j)
      row[j] = fmaf((row[j] - mean) * is, t->g[j], t->b[j]);
  }
}

void orc_layernorm_rows_f64(float *x, int64_t rows, int64_t cols,
                            const float *gamma, const float *beta, double eps) {
  ln_task t = {x, gamma, beta, NULL, NULL, rows, cols, 0.0f, eps};
  orc_run(ln64_worker, &t);
}

typedef struct { float *x; const float *y, *r; size_t n; } add_task;

static void add_worker(void *p, int w, int nw) {
  const add_task *t = (const add_task *)p;
  int64_t lo, hi;
  orc_range((int64_t)t->n, w, nw, &lo, &hi);
  for (int64_t i = lo; i < hi; ++i) t->x[i] = t->y[i] + t->r[i];
}

void orc_add_into(float *x, const float *y, const float *residual, size_t n) {
  add_task t = {x, y, residual, n};
  orc_run(add_worker, &t);
}

/* ---- softmax -------------------------------------------------------------- */
typedef struct {
  float *x;
  const float *mask;
  int64_t rows, cols, rpm;
} sm_task;

/* softmax_cpu's AVX2 branch (bert_encoder.cpp:495-520). */
static void sm_poly_row(float *row, int64_t S) {
  __m256 mx = _mm256_loadu_ps(row);
  for (int64_t j = 8; j < S; j += 8) mx = _mm256_max_ps(mx, _mm256_loadu_ps(row + j));
  __m128 m4 = _mm_max_ps(_mm256_castps256_ps128(mx), _mm256_extractf128_ps(mx, 1));
  m4 = _mm_max_ps(m4, _mm_movehl_ps(m4, m4));
  m4 = _mm_max_ss(m4, _mm_movehdup_ps(m4));
  const __m256 mv = _mm256_set1_ps(_mm_cvtss_f32(m4));
  const __m256 log2e = _mm256_set1_ps(1.4426950408889634f);
  const __m256 argfloor = _mm256_set1_ps(-120.0f);
  __m256 sum = _mm256_setzero_ps();
  for (int64_t j = 0; j < S; j += 8) {
    const __m256 a = _mm256_mul_ps(_mm256_sub_ps(_mm256_loadu_ps(row + j), mv), log2e);
    const __m256 e = orc_exp2_v(_mm256_max_ps(a, argfloor));
    _mm256_storeu_ps(row + j, e);
    sum = _mm256_add_ps(sum, e);
  }
  const __m256 inv = _mm256_set1_ps(1.0f / orc_hsum256(sum));
  for (int64_t j = 0; j < S; j += 8)
    _mm256_storeu_ps(row + j, _mm256_mul_ps(_mm256_loadu_ps(row + j), inv));
}

static void sm_poly_worker(void *p, int w, int nw) {
  const sm_task *t = (const sm_task *)p;
  int64_t lo, hi;
  orc_range(t->rows, w, nw, &lo, &hi);
  for (int64_t r = lo; r < hi; ++r) {
    float *row = t->x + r * t->cols;
    if (t->mask) {
      const float *mk = t->mask + (r / t->rpm) * t->cols;
      for (int64_t j = 0; j < t->cols; ++j) row[j] += mk[j];
    }
    sm_poly_row(row, t->cols);
  }
}

void orc_softmax_rows_poly(float *x, int64_t rows, int64_t cols,
                           const float *add_mask, int64_t rows_per_mask_row) {
  if (cols % 8 != 0) abort(); /* the reference's seq is a multiple of 8 */
  sm_task t = {x, add_mask, rows, cols, rows_per_mask_row > 0 ? rows_per_mask_row : 1};
  orc_run(sm_poly_worker, &t);
}

/* npu_ops.cpp:591-599 softmax_row, then the 1/sum applied by av_row. */
static float sm_exact_row(float *sc, int64_t n) {
  float mx = sc[0];
  for (int64_t j = 1; j < n; ++j) mx = sc[j] > mx ? sc[j] : mx;
  float sum = 0.0f;
  for (int64_t j = 0; j < n; ++j) {
    sc[j] = expf(sc[j] - mx);
    sum += sc[j];
  }
  return sum > 0.0f ? 1.0f / sum : 0.0f;
}

static void sm_exact_worker(void *p, int w, int nw) {
  const sm_task *t = (const sm_task *)p;
  int64_t lo, hi;
  orc_range(t->rows, w, nw, &lo, &hi);
  for (int64_t r = lo; r < hi; ++r) {
    float *row = t->x + r * t->cols;
    if (t->mask) {
      const float *mk = t->mask + (r / t->rpm) * t->cols;
      for (int64_t j = 0; j < t->cols; ++j) row[j] += mk[j];
    }
    const float inv = sm_exact_row(row, t->cols);
    for (int64_t j = 0; j < t->cols; ++j) row[j] *= inv;
  }
}

void orc_softmax_rows_exact(float *x, int64_t rows, int64_t cols,
                            const float *add_mask, int64_t rows_per_mask_row) {
  sm_task t = {x, add_mask, rows, cols, rows_per_mask_row > 0 ? rows_per_mask_row : 1};
  orc_run(sm_exact_worker, &t);
}

/* ---- BERT host attention: qk_impl / av_impl ------------------------------- */
typedef struct {
  const float *qkv, *sc;
  float *out;
  int64_t B, S, H, hd;
} att_task;

/* qk_impl, AVX2 branch (bert_encoder.cpp:1019-1045). */
static void qk_worker(void *p, int w, int nw) {
  const att_task *t = (const att_task *)p;
  const int64_t d = t->H * t->hd, S = t->S, nv = t->hd / 8;
  for (int64_t pr = w; pr < t->B * t->H; pr += nw) {
    const int64_t b = pr / t->H, h = pr % t->H;
    for (int64_t i = 0; i < S; ++i) {
      const float *q = t->qkv + (b * S + i) * 3 * d + h * t->hd;
      float *dst = t->out + (pr * S + i) * S;
      __m256 qv[32];
      for (int64_t v = 0; v < nv; ++v) qv[v] = _mm256_loadu_ps(q + v * 8);
      for (int64_t j = 0; j < S; ++j) {
        const float *k = t->qkv + (b * S + j) * 3 * d + d + h * t->hd;
        __m256 s = _mm256_mul_ps(qv[0], _mm256_loadu_ps(k));
        for (int64_t v = 1; v < nv; ++v)
          s = _mm256_fmadd_ps(qv[v], _mm256_loadu_ps(k + v * 8), s);
        dst[j] = orc_hsum256(s);
      }
    }
  }
}

void orc_qk(const float *qkv, int64_t B, int64_t S, int64_t H, int64_t hd,
            float *scores) {
  if (hd % 8 != 0 || hd / 8 > 32) abort();
  att_task t = {qkv, NULL, scores, B, S, H, hd};
  orc_run(qk_worker, &t);
}

/* av_impl, AVX2 branch (bert_encoder.cpp:1100-1114). */
static void av_worker(void *p, int w, int nw) {
  const att_task *t = (const att_task *)p;
  const int64_t d = t->H * t->hd, S = t->S, nv = t->hd / 8;
  for (int64_t pr = w; pr < t->B * t->H; pr += nw) {
    const int64_t b = pr / t->H, h = pr % t->H;
    for (int64_t i = 0; i < S; ++i) {
      const float *a = t->sc + (pr * S + i) * S;
      float *o = t->out + (b * S + i) * d + h * t->hd;
      __m256 acc[32];
      for (int64_t v = 0; v < nv; ++v) acc[v] = _mm256_setzero_ps();
      for (int64_t j = 0; j < S; ++j) {
        const float *v = t->qkv + (b * S + j) * 3 * d + 2 * d + h * t->hd;
        const __m256 aj = _mm256_set1_ps(a[j]);
        for (int64_t k = 0; k < nv; ++k)
          acc[k] = _mm256_fmadd_ps(aj, _mm256_loadu_ps(v + k * 8), acc[k]);
      }
      for (int64_t v = 0; v < nv; ++v) _mm256_storeu_ps(o + v * 8, acc[v]);
    }
  }
}

void orc_av(const float *scores, const float *qkv, int64_t B, int64_t S,
            int64_t H, int64_t hd, float *ctx) {
  if (hd % 8 != 0 || hd / 8 > 32) abort();
  att_task t = {qkv, scores, ctx, B, S, H, hd};
  orc_run(av_worker, &t);
}

/* ---- whisper::attention (npu_ops.cpp:478-644, the in-place branch) -------- */
typedef struct {
  const float *q, *kv;
  float *out;
  int64_t q_stride, kv_stride, n_q, n_kv, d_model, heads, hd;
  float scale;
} watt_task;

static void watt_worker(void *p, int w, int nw) {
  const watt_task *t = (const watt_task *)p;
  float *sc = (float *)malloc((size_t)t->n_kv * sizeof(float));
  for (int64_t i = w; i < t->n_q; i += nw) {
    for (int64_t h = 0; h < t->heads; ++h) {
      const float *qh = t->q + i * t->q_stride + h * t->hd;
      for (int64_t j = 0; j < t->n_kv; ++j) {
        const float *kj = t->kv + j * t->kv_stride + h * t->hd;
        int64_t s = 0;
        __m256 a = _mm256_setzero_ps();
        for (; s + 8 <= t->hd; s += 8)
          a = _mm256_fmadd_ps(_mm256_loadu_ps(qh + s), _mm256_loadu_ps(kj + s), a);
        float acc = orc_hsum256(a);
        for (; s < t->hd; ++s) acc = fmaf(qh[s], kj[s], acc);
        sc[j] = acc * t->scale;
      }
      const float inv = sm_exact_row(sc, t->n_kv);
      float *o = t->out + i * t->d_model + h * t->hd;
      for (int64_t s = 0; s < t->hd; ++s) o[s] = 0.0f;
      for (int64_t j = 0; j < t->n_kv; ++j) {
        const float a = sc[j] * inv;
        const float *vj = t->kv + j * t->kv_stride + t->d_model + h * t->hd;
        int64_t s = 0;
        const __m256 av = _mm256_set1_ps(a);
        for (; s + 8 <= t->hd; s += 8)
          _mm256_storeu_ps(o + s, _mm256_fmadd_ps(av, _mm256_loadu_ps(vj + s),
                                                  _mm256_loadu_ps(o + s)));
        for (; s < t->hd; ++s) o[s] = fmaf(a, vj[s], o[s]);
      }
    }
  }
  free(sc);
}

void orc_whisper_attention(const float *q, int64_t q_stride, const float *kv,
                           int64_t kv_stride, int64_t n_q, int64_t n_kv,
                           int64_t d_model, int64_t heads, int64_t head_dim,
                           float scale, float *out) {
  watt_task t = {q, kv, out, q_stride, kv_stride, n_q, n_kv, d_model, heads,
                 head_dim, scale};
  orc_run(watt_worker, &t);
}

/* ---- embedding sum + mask (embed_service.cpp:29-64) ----------------------- */
void orc_embed_sum(const int32_t *ids, const float *attn_mask, int64_t B,
                   int64_t S, int64_t hidden, const float *word,
                   const float *pos, const float *type0, float *emb,
                   float *add_mask) {
  for (int64_t b = 0; b < B; ++b)
    for (int64_t s = 0; s < S; ++s) {
      const int64_t r = b * S + s;
      const float m = attn_mask[r];
      add_mask[r] = m > 0.0f ? 0.0f : -1.0e30f;
      const float *wv = word + (int64_t)ids[r] * hidden;
      const float *pv = pos + s * hidden;
      float *dst = emb + r * hidden;
      for (int64_t c = 0; c < hidden; ++c) dst[c] = wv[c] + pv[c] + type0[c];
    }
}

/* ---- pool_rows (app_state.hpp:335-374) ------------------------------------ */
int orc_pool_rows(const float *h, const float *am, int64_t B, int64_t S,
                  int64_t hidden, int cls_pool, int l2_normalize, float *out) {
  double *acc = (double *)malloc((size_t)hidden * sizeof(double));
  int rc = 0;
  for (int64_t b = 0; b < B && rc == 0; ++b) {
    const float *amb = am + b * S;
    const float *hb = h + b * S * hidden;
    if (cls_pool) {
      if (amb[0] == 0.0f) { rc = -1; break; }
      for (int64_t c = 0; c < hidden; ++c) acc[c] = hb[c];
    } else {
      float denom = 0.0f;
      for (int64_t s = 0; s < S; ++s) denom += amb[s];
      denom = denom > 1e-9f ? denom : 1e-9f;
      for (int64_t c = 0; c < hidden; ++c) acc[c] = 0.0;
      for (int64_t s = 0; s < S; ++s) {
        const float m = amb[s];
        if (m == 0.0f) continue;
        const float *hr = hb + s * hidden;
        for (int64_t c = 0; c < hidden; ++c) acc[c] += (double)(hr[c] * m);
      }
      for (int64_t c = 0; c < hidden; ++c) acc[c] /= (double)denom;
    }
    float *o = out + b * hidden;
    if (l2_normalize) {
      double nrm = 0.0;
      for (int64_t c = 0; c < hidden; ++c) nrm = fma(acc[c], acc[c], nrm);
      nrm = sqrt(nrm > 1e-24 ? nrm : 1e-24);
      for (int64_t c = 0; c < hidden; ++c) o[c] = (float)(acc[c] / nrm);
    } else {
      for (int64_t c = 0; c < hidden; ++c) o[c] = (float)acc[c];
    }
  }
  free(acc);
  return rc;
}

/* ---- ViT im2col (vit/image.cpp:731-748) and head (vit/head.cpp:16-49) ----- */
void orc_vit_patches(const float *chw, int64_t img, int64_t patch, float *rows) {
  const int64_t n = img / patch, pd = 3 * patch * patch;
  for (int64_t p = 0; p < n; ++p)
    for (int64_t q = 0; q < n; ++q) {
      float *dst = rows + (p * n + q) * pd;
      for (int64_t c = 0; c < 3; ++c)
        for (int64_t i = 0; i < patch; ++i)
          for (int64_t j = 0; j < patch; ++j)
            dst[(c * patch + i) * patch + j] =
                chw[(c * img + p * patch + i) * img + q * patch + j];
    }
}

void orc_head_matvec(const float *head, const float *bias, const float *cls_row,
                     int64_t d_model, int64_t num_labels, float *logits) {
  for (int64_t j = 0; j < num_labels; ++j) {
    double acc = bias ? (double)bias[j] : 0.0;
    for (int64_t t = 0; t < d_model; ++t)
      acc = fma((double)cls_row[t], (double)head[t * num_labels + j], acc);
    logits[j] = (float)acc;
  }
}

/* ---- hostb::host_b_kn's untile (host_b.hpp:206-243) ----------------------- */
int orc_untile_b_panel(const uint16_t *panel, int64_t K, int64_t N, int64_t tile_k,
                       int64_t tile_n, int64_t mac_s, int64_t mac_t, uint16_t *kn) {
  if (K <= 0 || N <= 0 || tile_k <= 0 || tile_n <= 0 || mac_s <= 0 || mac_t <= 0) return -1;
  if (K % tile_k || N % tile_n || tile_k % mac_s || tile_n % mac_t) return -1;
  const int64_t kblocks = K / tile_k, nblocks = N / tile_n;
  const int64_t rows = tile_k / mac_s, cols = tile_n / mac_t;
  size_t src = 0; /* the container is read strictly in order */
  for (int64_t bk = 0; bk < kblocks; ++bk)
    for (int64_t bn = 0; bn < nblocks; ++bn)
      for (int64_t r = 0; r < rows; ++r)
        for (int64_t c = 0; c < cols; ++c)
          for (int64_t si = 0; si < mac_s; ++si) {
            uint16_t *dst = kn + (bk * tile_k + r * mac_s + si) * N + bn * tile_n + c * mac_t;
            for (int64_t ti = 0; ti < mac_t; ++ti) dst[ti] = panel[src++];
          }
  return 0;
}

/* npue::gemm_b_panel's I4 branch (common/int4_panel.hpp:183-246): walk the
 * flat run's six axes (k-block, n-block, row group, column group, row, column)
 * so each element's (k, n) is known; element f is nibble f % 2 (low first) of
 * byte f / 2, sign-extended; q = clip(nearbyint(t * gscale[k / g][n]), +-127)
 * stays at flat index f. */
int orc_widen_i4_panel(const uint8_t *packed, int64_t K, int64_t N, int64_t tile_k,
                       int64_t tile_n, int64_t mac_s, int64_t mac_t, const float *gscale,
                       int64_t int4_group, int8_t *out) {
  if (K <= 0 || N <= 0 || (K * N) % 2 || tile_k <= 0 || tile_n <= 0 || mac_s <= 0 ||
      mac_t <= 0 || int4_group < 0)
    return -1;
  if (K % tile_k || N % tile_n || tile_k % mac_s || tile_n % mac_t) return -1;
  const int64_t g = int4_group == 0 ? K : int4_group;
  const int64_t kblocks = K / tile_k, nblocks = N / tile_n;
  const int64_t rows = tile_k / mac_s, cols = tile_n / mac_t;
  int64_t f = 0;
  for (int64_t bk = 0; bk < kblocks; ++bk)
    for (int64_t bn = 0; bn < nblocks; ++bn)
      for (int64_t r = 0; r < rows; ++r)
        for (int64_t c = 0; c < cols; ++c)
          for (int64_t si = 0; si < mac_s; ++si) {
            const int64_t k = bk * tile_k + r * mac_s + si;
            const float *grow = gscale + (k / g) * N;
            for (int64_t ti = 0; ti < mac_t; ++ti, ++f) {
              const int64_t n = bn * tile_n + c * mac_t + ti;
              const uint8_t b = packed[f >> 1];
              const int nv = (f & 1) ? (int)(b >> 4) : (int)(b & 0x0F);
              const float t = (float)(nv > 7 ? nv - 16 : nv);
              float q = nearbyintf(t * grow[n]);
              if (q > 127.0f)
                q = 127.0f;
              else if (q < -127.0f)
                q = -127.0f;
              out[f] = (int8_t)q;
            }
          }
  return 0;
}

/* ---- int8 W8A8 (host_kernels.hpp:263-320, 529-600) ------------------------ */
typedef struct {
  const float *a, *ias;
  int8_t *q;
  float *sc;
  int64_t rows, K;
} quant_task;

static void quant_worker(void *p, int w, int nw) {
  const quant_task *t = (const quant_task *)p;
  for (int64_t r = w; r < t->rows; r += nw) {
    const float *x = t->a + r * t->K;
    int8_t *q = t->q + r * t->K;
    float mx = 0.0f;
    for (int64_t j = 0; j < t->K; ++j) {
      const float v = fabsf(x[j] * t->ias[j]);
      if (v > mx) mx = v;
    }
    const float sc = mx > 0.0f ? mx / 127.0f : 1.0f;
    t->sc[r] = sc;
    const float inv = 1.0f / sc;
    for (int64_t j = 0; j < t->K; ++j) {
      float v = (x[j] * t->ias[j]) * inv;
      v = v < -127.0f ? -127.0f : (v > 127.0f ? 127.0f : v);
      q[j] = (int8_t)nearbyintf(v);
    }
  }
}

void orc_quantise_a_int8(const float *a, int64_t rows, int64_t K, const float *ias,
                         int8_t *q, float *a_scale) {
  quant_task t = {a, ias, q, a_scale, rows, K};
  orc_run(quant_worker, &t);
}

typedef struct {
  const int8_t *A, *W;
  int32_t *C;
  int64_t M, K, N;
} gemm_i8_task;

static void gemm_i8_worker(void *p, int w, int nw) {
  const gemm_i8_task *t = (const gemm_i8_task *)p;
  const int64_t N = t->N, N32 = N / 32 * 32;
  for (int64_t m = w; m < t->M; m += nw) {
    int32_t *c = t->C + m * N;
    const int8_t *a = t->A + m * t->K;
    /* 32 columns at a time in four int32 accumulators (integer sums are exact
     * in any order), the rest one column at a time */
    for (int64_t n = 0; n < N32; n += 32) {
      __m256i c0 = _mm256_setzero_si256(), c1 = c0, c2 = c0, c3 = c0;
      for (int64_t k = 0; k < t->K; ++k) {
        const __m256i av = _mm256_set1_epi32(a[k]);
        const int8_t *wr = t->W + k * N + n;
        c0 = _mm256_add_epi32(c0, _mm256_mullo_epi32(av, _mm256_cvtepi8_epi32(
                                                             _mm_loadl_epi64((const __m128i *)wr))));
        c1 = _mm256_add_epi32(c1, _mm256_mullo_epi32(av, _mm256_cvtepi8_epi32(_mm_loadl_epi64(
                                                             (const __m128i *)(wr + 8)))));
        c2 = _mm256_add_epi32(c2, _mm256_mullo_epi32(av, _mm256_cvtepi8_epi32(_mm_loadl_epi64(
                                                             (const __m128i *)(wr + 16)))));
        c3 = _mm256_add_epi32(c3, _mm256_mullo_epi32(av, _mm256_cvtepi8_epi32(_mm_loadl_epi64(
                                                             (const __m128i *)(wr + 24)))));
      }
      _mm256_storeu_si256((__m256i *)(c + n), c0);
      _mm256_storeu_si256((__m256i *)(c + n + 8), c1);
      _mm256_storeu_si256((__m256i *)(c + n + 16), c2);
      _mm256_storeu_si256((__m256i *)(c + n + 24), c3);
    }
    for (int64_t n = N32; n < N; ++n) c[n] = 0;
    for (int64_t k = 0; k < t->K; ++k) {
      const int32_t av = a[k];
      const int8_t *wr = t->W + k * N;
      for (int64_t n = N32; n < N; ++n) c[n] += av * (int32_t)wr[n];
    }
  }
}

void orc_gemm_i8(const int8_t *Aq, int64_t M, int64_t K, const int8_t *Wq, int64_t N,
                 int32_t *C) {
  gemm_i8_task t = {Aq, Wq, C, M, K, N};
  orc_run(gemm_i8_worker, &t);
}

typedef struct {
  const int32_t *C;
  const float *sa, *ws, *bias;
  float *out;
  int64_t rows, N;
} deq_task;

static void deq_worker(void *p, int w, int nw) {
  const deq_task *t = (const deq_task *)p;
  for (int64_t r = w; r < t->rows; r += nw) {
    const float sa = t->sa[r];
    for (int64_t n = 0; n < t->N; ++n)
      t->out[r * t->N + n] = fmaf((float)t->C[r * t->N + n] * sa, t->ws[n], t->bias[n]);
  }
}

void orc_dequantise_c(const int32_t *C, int64_t rows, int64_t N, const float *a_scale,
                      const float *wscale, const float *bias, float *out) {
  deq_task t = {C, a_scale, wscale, bias, out, rows, N};
  orc_run(deq_worker, &t);
}

void orc_gemm_i8_dequant(const float *A, int64_t M, int64_t K, const float *ias,
                         const int8_t *Wq, const float *wscale, const float *bias,
                         int64_t N, float *out) {
  int8_t *q = (int8_t *)malloc((size_t)(M * K));
  float *sa = (float *)malloc((size_t)M * sizeof(float));
  int32_t *c = (int32_t *)malloc((size_t)(M * N) * sizeof(int32_t));
  orc_quantise_a_int8(A, M, K, ias, q, sa);
  orc_gemm_i8(q, M, K, Wq, N, c);
  orc_dequantise_c(c, M, N, sa, wscale, bias, out);
  free(q);
  free(sa);
  free(c);
}

/* ---- the narrowed C (c_elem_bytes == 2) ----------------------------------- */

typedef struct {
  const uint16_t *C;
  const float *sa, *ws, *bias;
  float *out;
  uint16_t *dst;
  int64_t rows, N;
  int gated;
} cbf_task;

static void deq_bf16_worker(void *p, int w, int nw) {
  const cbf_task *t = (const cbf_task *)p;
  for (int64_t r = w; r < t->rows; r += nw) {
    const float sa = t->sa[r];
    for (int64_t n = 0; n < t->N; ++n)
      t->out[r * t->N + n] =
          fmaf(orc_from_bf16(t->C[r * t->N + n]) * sa, t->ws[n], t->bias[n]);
  }
}

void orc_dequantise_c_bf16(const uint16_t *C, int64_t rows, int64_t N, const float *a_scale,
                           const float *wscale, const float *bias, float *out) {
  cbf_task t = {C, a_scale, wscale, bias, out, NULL, rows, N, 0};
  orc_run(deq_bf16_worker, &t);
}

static void bias_bf16_worker(void *p, int w, int nw) {
  const cbf_task *t = (const cbf_task *)p;
  for (int64_t r = w; r < t->rows; r += nw)
    for (int64_t n = 0; n < t->N; ++n)
      t->out[r * t->N + n] = orc_from_bf16(t->C[r * t->N + n]) + t->bias[n];
}

void orc_bias_c_bf16(const uint16_t *C, int64_t rows, int64_t N, const float *bias,
                     float *out) {
  cbf_task t = {C, NULL, NULL, bias, out, NULL, rows, N, 0};
  orc_run(bias_bf16_worker, &t);
}

void orc_dequant_act_bf16(const uint16_t *C, int64_t rows, int64_t N, int gated,
                          const float *bias, uint16_t *dst) {
  float *v = (float *)malloc((size_t)(rows * N) * sizeof(float));
  orc_bias_c_bf16(C, rows, N, bias, v);
  if (!gated) {
    orc_gelu_poly_inplace(v, (size_t)(rows * N));
    orc_bf16_fill(dst, v, (size_t)(rows * N));
  } else {
    const int64_t f = N / 2;
    float *g = (float *)malloc((size_t)(rows * f) * sizeof(float));
    orc_glu(v, rows, f, gated, g);
    orc_bf16_fill(dst, g, (size_t)(rows * f));
    free(g);
  }
  free(v);
}
