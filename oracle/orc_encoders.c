/*
 * orc_encoders.c -- whole encoder stacks on the host, restated from the
 * reference's host branches. TEST INFRASTRUCTURE (the oracle); see oracle.h.
 */
#include "orc_internal.h"

#include <math.h>
#include <stdlib.h>

static float *falloc(size_t n) { return (float *)malloc(n * sizeof(float)); }

/* ---- the array datapath's arithmetic (orc_set_array_arith) ---------------- */

static int g_arr = 0;

int orc_set_array_arith(int flags) {
  const int prev = g_arr;
  g_arr = flags;
  return prev;
}

/* One bf16-datapath GEMM of the stack: gemm_nt on the host's fp32 A, or the
 * array's form -- A rounded to bf16 (ORC_ARR_A_BF16), the accumulator rounded
 * to bf16 before the bias (ORC_ARR_C_BF16). gemm_nt adds the bias after the
 * whole k chain, so acc then + bias is the same sum. */
static void gemm_site(const float *A, int64_t rows, const float *W, int64_t K, int64_t N,
                      const float *bias, float *out) {
  if (!g_arr) {
    orc_gemm_nt(A, rows, W, K, N, bias, out);
    return;
  }
  float *a = NULL;
  if (g_arr & ORC_ARR_A_BF16) {
    a = falloc((size_t)(rows * K));
    memcpy(a, A, (size_t)(rows * K) * sizeof(float));
    orc_round_bf16_inplace(a, (size_t)(rows * K));
  }
  if (!(g_arr & ORC_ARR_C_BF16)) {
    orc_gemm_nt(a ? a : A, rows, W, K, N, bias, out);
  } else {
    orc_gemm_nt(a ? a : A, rows, W, K, N, NULL, out);
    uint16_t *c = (uint16_t *)malloc((size_t)(rows * N) * sizeof(uint16_t));
    orc_bf16_fill(c, out, (size_t)(rows * N));
    orc_bias_c_bf16(c, rows, N, bias, out);
    free(c);
  }
  free(a);
}

/* One int8-datapath GEMM: quantise -> exact int32 product -> dequantise_c,
 * from the int32 C or (ORC_ARR_C_BF16) from narrow_i32_bf16 of it. */
static void gemm_i8_site(const float *A, int64_t M, int64_t K, const float *ias,
                         const int8_t *Wq, const float *wscale, const float *bias, int64_t N,
                         float *out) {
  if (!(g_arr & ORC_ARR_C_BF16)) {
    orc_gemm_i8_dequant(A, M, K, ias, Wq, wscale, bias, N, out);
    return;
  }
  int8_t *q = (int8_t *)malloc((size_t)(M * K));
  float *sa = falloc((size_t)M);
  int32_t *c = (int32_t *)malloc((size_t)(M * N) * sizeof(int32_t));
  uint16_t *cb = (uint16_t *)malloc((size_t)(M * N) * sizeof(uint16_t));
  orc_quantise_a_int8(A, M, K, ias, q, sa);
  orc_gemm_i8(q, M, K, Wq, N, c);
  orc_narrow_i32_bf16(c, cb, M * N);
  orc_dequantise_c_bf16(cb, M, N, sa, wscale, bias, out);
  free(q);
  free(sa);
  free(c);
  free(cb);
}

/* Q, K, V or a context rounded to bf16 (ORC_ARR_ATTN_BF16). */
static void attn_bf16(float *x, size_t n) {
  if (g_arr & ORC_ARR_ATTN_BF16) orc_round_bf16_inplace(x, n);
}

/* BertEncoder::run, every op on the host (bert_encoder.cpp:1419-1598 with
 * gemm_on_array() false, host_ln/host_sm/host_gelu true, attn_ null). */
void orc_bert_run(const orc_encoder *m, float *x, const float *add_mask,
                  int64_t B, int64_t S, int64_t layers_to_run) {
  const int64_t d = m->hidden, f = m->ffn, H = m->heads, hd = m->head_dim;
  const int64_t rows = B * S;
  const int64_t L = layers_to_run < 0 || layers_to_run > m->layers ? m->layers
                                                                   : layers_to_run;
  const float eps = 1e-12f; /* hard-coded in layer_norm_cpu (:438) */
  const int64_t fu = m->gated ? 2 * f : f; /* FFN-up width: up | gate when gated */
  float *qkv = falloc((size_t)(rows * 3 * d));
  float *scores = falloc((size_t)(B * H * S * S));
  float *ctx = falloc((size_t)(rows * d));
  float *proj = falloc((size_t)(rows * d));
  float *up = falloc((size_t)(rows * fu));
  float *gated = m->gated ? falloc((size_t)(rows * f)) : NULL;
  float *residual = falloc((size_t)(rows * d));

  orc_layer_norm_rows(x, rows, d, m->emb_ln_g, m->emb_ln_b, eps);
  for (int64_t l = 0; l < L; ++l) {
    memcpy(residual, x, (size_t)(rows * d) * sizeof(float));
    gemm_site(x, rows, m->w_qkv + l * d * 3 * d, d, 3 * d, m->b_qkv + l * 3 * d, qkv);
    if (m->rope_cos) orc_rope_qkv(qkv, rows, S, H, hd, m->rope_cos, m->rope_sin);
    attn_bf16(qkv, (size_t)(rows * 3 * d));
    orc_qk(qkv, B, S, H, hd, scores);
    orc_softmax_rows_poly(scores, B * H * S, S, add_mask, H * S);
    orc_av(scores, qkv, B, S, H, hd, ctx);
    attn_bf16(ctx, (size_t)(rows * d));
    gemm_site(ctx, rows, m->w_ao + l * d * d, d, d, m->b_ao + l * d, proj);
    orc_add_into(x, proj, residual, (size_t)(rows * d));
    orc_layer_norm_rows(x, rows, d, m->ln1_g + l * d, m->ln1_b + l * d, eps);
    memcpy(residual, x, (size_t)(rows * d) * sizeof(float));
    gemm_site(x, rows, m->w_up + l * d * fu, d, fu, m->b_up + l * fu, up);
    if (m->gated) {
      orc_glu(up, rows, f, (int)m->gated, gated);
    } else {
      orc_gelu_poly_inplace(up, (size_t)(rows * f));
    }
    gemm_site(m->gated ? gated : up, rows, m->w_down + l * f * d, f, d, m->b_down + l * d,
              proj);
    orc_add_into(x, proj, residual, (size_t)(rows * d));
    orc_layer_norm_rows(x, rows, d, m->ln2_g + l * d, m->ln2_b + l * d, eps);
  }
  free(qkv);
  free(scores);
  free(ctx);
  free(proj);
  free(up);
  free(gated);
  free(residual);
}

/* ---- RoPE and the gated FFN (the nomic / gte BERT archs) ------------------ */

void orc_rope_tables(int64_t S, int64_t hd, double theta, const float *inv_freq,
                     float *cos_t, float *sin_t) {
  const int64_t half = hd / 2;
  double *inv = (double *)malloc((size_t)half * sizeof(double));
  for (int64_t j = 0; j < half; ++j)
    inv[j] = inv_freq ? (double)inv_freq[j] : 1.0 / pow(theta, (2.0 * (double)j) / (double)hd);
  for (int64_t s = 0; s < S; ++s)
    for (int64_t j = 0; j < half; ++j) {
      const double ang = (double)s * inv[j];
      const float c = (float)cos(ang), sn = (float)sin(ang);
      cos_t[s * hd + j] = cos_t[s * hd + half + j] = c;
      sin_t[s * hd + j] = sin_t[s * hd + half + j] = sn;
    }
  free(inv);
}

typedef struct {
  float *qkv;
  const float *c, *sn;
  int64_t rows, S, H, hd;
} rope_task;

static void rope_rotate(float *v, const float *c, const float *sn, int64_t half) {
  for (int64_t j = 0; j < half; ++j) {
    const float x1 = v[j], x2 = v[j + half];
    v[j] = x1 * c[j] - x2 * sn[j];
    v[j + half] = x2 * c[j] + x1 * sn[j];
  }
}

static void rope_worker(void *p, int w, int nw) {
  const rope_task *t = (const rope_task *)p;
  const int64_t d = t->H * t->hd, half = t->hd / 2;
  for (int64_t r = w; r < t->rows; r += nw) {
    const int64_t s = r % t->S;
    float *row = t->qkv + r * 3 * d;
    for (int64_t h = 0; h < t->H; ++h) {
      rope_rotate(row + h * t->hd, t->c + s * t->hd, t->sn + s * t->hd, half);
      rope_rotate(row + d + h * t->hd, t->c + s * t->hd, t->sn + s * t->hd, half);
    }
  }
}

void orc_rope_qkv(float *qkv, int64_t rows, int64_t S, int64_t H, int64_t hd,
                  const float *cos_t, const float *sin_t) {
  rope_task t = {qkv, cos_t, sin_t, rows, S, H, hd};
  orc_run(rope_worker, &t);
}

typedef struct {
  const float *up;
  float *out;
  int64_t rows, f;
  int act;
} glu_task;

static void glu_worker(void *p, int w, int nw) {
  const glu_task *t = (const glu_task *)p;
  for (int64_t r = w; r < t->rows; r += nw) {
    const float *lo = t->up + r * 2 * t->f, *hi = lo + t->f;
    float *dst = t->out + r * t->f;
    for (int64_t j = 0; j < t->f; ++j) {
      if (t->act == 2) {
        dst[j] = lo[j] * orc_gelu_erf_exact(hi[j]);
      } else {
        float a = (0.0f - hi[j]) * 1.4426950408889634f;
        if (a < -120.0f) a = -120.0f;
        dst[j] = lo[j] * (hi[j] / (1.0f + orc_exp2_s(a)));
      }
    }
  }
}

void orc_glu(const float *up, int64_t rows, int64_t f, int act, float *out) {
  glu_task t = {up, out, rows, f, act};
  orc_run(glu_worker, &t);
}

/* BertEncoder::run on an int8 container, the GEMMs on the array
 * (bert_encoder.cpp:741-924 int8 branch), everything else on the host. */
void orc_bert_run_i8(const orc_encoder *m, const orc_i8_operands *q, float *x,
                     const float *add_mask, int64_t B, int64_t S, int64_t layers_to_run) {
  const int64_t d = m->hidden, f = m->ffn, H = m->heads, hd = m->head_dim;
  const int64_t rows = B * S;
  const int64_t L = layers_to_run < 0 || layers_to_run > m->layers ? m->layers
                                                                   : layers_to_run;
  const float eps = 1e-12f;
  const int64_t fu = m->gated ? 2 * f : f; /* FFN-up width: up | gate when gated */
  const int64_t Ks[4] = {d, d, d, f}, Ns[4] = {3 * d, d, fu, d};
  float *qkv = falloc((size_t)(rows * 3 * d));
  float *scores = falloc((size_t)(B * H * S * S));
  float *ctx = falloc((size_t)(rows * d));
  float *proj = falloc((size_t)(rows * d));
  float *up = falloc((size_t)(rows * fu));
  float *gated = m->gated ? falloc((size_t)(rows * f)) : NULL;
  float *residual = falloc((size_t)(rows * d));
#define GEMM_I8(i, A, bias, out)                                                          \
  gemm_i8_site((A), rows, Ks[i], q->ias[i] + l * Ks[i], q->wq[i] + l * Ks[i] * Ns[i], \
               q->wscale[i] + l * Ns[i], (bias), Ns[i], (out))
  orc_layer_norm_rows(x, rows, d, m->emb_ln_g, m->emb_ln_b, eps);
  for (int64_t l = 0; l < L; ++l) {
    memcpy(residual, x, (size_t)(rows * d) * sizeof(float));
    GEMM_I8(0, x, m->b_qkv + l * 3 * d, qkv);
    if (m->rope_cos) orc_rope_qkv(qkv, rows, S, H, hd, m->rope_cos, m->rope_sin);
    attn_bf16(qkv, (size_t)(rows * 3 * d));
    orc_qk(qkv, B, S, H, hd, scores);
    orc_softmax_rows_poly(scores, B * H * S, S, add_mask, H * S);
    orc_av(scores, qkv, B, S, H, hd, ctx);
    attn_bf16(ctx, (size_t)(rows * d));
    GEMM_I8(1, ctx, m->b_ao + l * d, proj);
    orc_add_into(x, proj, residual, (size_t)(rows * d));
    orc_layer_norm_rows(x, rows, d, m->ln1_g + l * d, m->ln1_b + l * d, eps);
    memcpy(residual, x, (size_t)(rows * d) * sizeof(float));
    GEMM_I8(2, x, m->b_up + l * fu, up);
    if (m->gated) {
      orc_glu(up, rows, f, (int)m->gated, gated);
    } else {
      orc_gelu_poly_inplace(up, (size_t)(rows * f));
    }
    GEMM_I8(3, m->gated ? gated : up, m->b_down + l * d, proj);
    orc_add_into(x, proj, residual, (size_t)(rows * d));
    orc_layer_norm_rows(x, rows, d, m->ln2_g + l * d, m->ln2_b + l * d, eps);
  }
#undef GEMM_I8
  free(qkv);
  free(scores);
  free(ctx);
  free(proj);
  free(up);
  free(gated);
  free(residual);
}

/* VitEncoder::run (vit/encoder.cpp:347-431) / WhisperEncoder::run
 * (whisper/encoder.cpp:156-213) body, host branch: pre-LN, the whole
 * sequence in one chunk (chunking by the design's rows does not change a
 * row's arithmetic: every op is row-wise except attention, which always sees
 * the whole sequence). */
void orc_preln_run(const orc_encoder *m, float *x, int64_t B, int64_t S,
                   double eps, float scale, int64_t layers_to_run) {
  const int64_t d = m->hidden, f = m->ffn;
  const int64_t rows = B * S;
  const int64_t L = layers_to_run < 0 || layers_to_run > m->layers ? m->layers
                                                                   : layers_to_run;
  float *norm = falloc((size_t)(rows * d));
  float *qkv = falloc((size_t)(rows * 3 * d));
  float *ctx = falloc((size_t)(rows * d));
  float *proj = falloc((size_t)(rows * d));
  float *up = falloc((size_t)(rows * f));
  for (int64_t l = 0; l < L; ++l) {
    memcpy(norm, x, (size_t)(rows * d) * sizeof(float));
    orc_layernorm_rows_f64(norm, rows, d, m->ln1_g + l * d, m->ln1_b + l * d, eps);
    orc_gemm_nt(norm, rows, m->w_qkv + l * d * 3 * d, d, 3 * d, m->b_qkv + l * 3 * d, qkv);
    for (int64_t b = 0; b < B; ++b) {
      const float *base = qkv + b * S * 3 * d;
      orc_whisper_attention(base, 3 * d, base + d, 3 * d, S, S, d, m->heads,
                            m->head_dim, scale, ctx + b * S * d);
    }
    orc_gemm_nt(ctx, rows, m->w_ao + l * d * d, d, d, m->b_ao + l * d, proj);
    for (int64_t i = 0; i < rows * d; ++i) x[i] += proj[i];
    memcpy(norm, x, (size_t)(rows * d) * sizeof(float));
    orc_layernorm_rows_f64(norm, rows, d, m->ln2_g + l * d, m->ln2_b + l * d, eps);
    orc_gemm_nt(norm, rows, m->w_up + l * d * f, d, f, m->b_up + l * f, up);
    orc_gelu_erf_inplace(up, (size_t)(rows * f));
    orc_gemm_nt(up, rows, m->w_down + l * f * d, f, d, m->b_down + l * d, proj);
    for (int64_t i = 0; i < rows * d; ++i) x[i] += proj[i];
  }
  if (m->fin_ln_g) orc_layernorm_rows_f64(x, rows, d, m->fin_ln_g, m->fin_ln_b, eps);
  free(norm);
  free(qkv);
  free(ctx);
  free(proj);
  free(up);
}

/* whisper/features.cpp:390-469 */
typedef struct {
  const float *in, *w, *bias;
  float *out;
  int64_t cin, T_in, T_out, stride, hidden;
} conv_task;

static void conv_worker(void *p, int w, int nw) {
  const conv_task *t = (const conv_task *)p;
  int64_t lo, hi;
  orc_range(t->hidden, w, nw, &lo, &hi);
  for (int64_t o = lo; o < hi; ++o) {
    const float *wo = t->w + o * t->cin * 3;
    for (int64_t tt = 0; tt < t->T_out; ++tt) {
      const int64_t centre = tt * t->stride;
      float acc = t->bias[o];
      for (int64_t c = 0; c < t->cin; ++c) {
        const float *wc = wo + c * 3;
        for (int64_t k = 0; k < 3; ++k) {
          const int64_t ti = centre + k - 1;
          if (ti < 0 || ti >= t->T_in) continue;
          acc = fmaf(wc[k], t->in[c * t->T_in + ti], acc);
        }
      }
      t->out[o * t->T_out + tt] = orc_gelu_erf_exact(acc);
    }
  }
}

void orc_conv_front_end(const float *mel, int64_t n_mels, int64_t T,
                        const float *w1, const float *b1, const float *w2,
                        const float *b2, int64_t hidden, float *out) {
  const int64_t T2 = T / 2;
  float *h1 = falloc((size_t)(hidden * T));
  float *h2 = falloc((size_t)(hidden * T2));
  conv_task c1 = {mel, w1, b1, h1, n_mels, T, T, 1, hidden};
  orc_run(conv_worker, &c1);
  conv_task c2 = {h1, w2, b2, h2, hidden, T, T2, 2, hidden};
  orc_run(conv_worker, &c2);
  for (int64_t o = 0; o < hidden; ++o)
    for (int64_t t = 0; t < T2; ++t) out[t * hidden + o] = h2[o * T2 + t];
  free(h1);
  free(h2);
}
