/* oracle_san.c -- the oracle (oracle/*.c, test infrastructure) under
 * AddressSanitizer and UndefinedBehaviorSanitizer. TEST PROGRAM: built by
 * tests/test_sanitize_cpu.py with gcc -fsanitize=address,undefined together
 * with the oracle's sources. Runs each op family on small shapes and the edge
 * shapes the tests use (one row, one token, masked rows, a fully masked
 * sequence, ragged tilings, refused tilings), single- and multi-threaded and
 * on per-lane pools. Prints "oracle ok". */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

static uint32_t g_state = 12345u;

static float frand(void) {
  g_state = g_state * 1664525u + 1013904223u;
  return ((float)(g_state >> 8) / 16777216.0f - 0.5f) * 0.1f;
}

static float *rnd(size_t n) {
  float *p = (float *)malloc(n * sizeof(float));
  for (size_t i = 0; i < n; ++i) p[i] = frand();
  return p;
}

static float *ones(size_t n) {
  float *p = (float *)malloc(n * sizeof(float));
  for (size_t i = 0; i < n; ++i) p[i] = 1.0f;
  return p;
}

/* A tiny BERT: d 64, 2 heads of 32, f 128 (gated: w_up [d, 2f]); the
   sequence is 8, a multiple of 8 as the polynomial softmax takes. */
static void bert_case(int gated, int rope, int threads) {
  const int64_t L = 2, d = 64, H = 2, hd = 32, f = 128, B = 3, S = 8;
  const int64_t fu = gated ? 2 * f : f;
  orc_encoder m;
  memset(&m, 0, sizeof m);
  m.layers = L;
  m.hidden = d;
  m.heads = H;
  m.head_dim = hd;
  m.ffn = f;
  m.w_qkv = rnd((size_t)(L * d * 3 * d));
  m.b_qkv = rnd((size_t)(L * 3 * d));
  m.w_ao = rnd((size_t)(L * d * d));
  m.b_ao = rnd((size_t)(L * d));
  m.w_up = rnd((size_t)(L * d * fu));
  m.b_up = rnd((size_t)(L * fu));
  m.w_down = rnd((size_t)(L * f * d));
  m.b_down = rnd((size_t)(L * d));
  m.ln1_g = ones((size_t)(L * d));
  m.ln1_b = rnd((size_t)(L * d));
  m.ln2_g = ones((size_t)(L * d));
  m.ln2_b = rnd((size_t)(L * d));
  m.emb_ln_g = ones((size_t)d);
  m.emb_ln_b = rnd((size_t)d);
  m.gated = gated;
  float *cos_t = NULL, *sin_t = NULL;
  if (rope) {
    cos_t = (float *)malloc((size_t)(S * hd) * sizeof(float));
    sin_t = (float *)malloc((size_t)(S * hd) * sizeof(float));
    orc_rope_tables(S, hd, 10000.0, NULL, cos_t, sin_t);
    m.rope_cos = cos_t;
    m.rope_sin = sin_t;
  }
  /* ids, mask with a fully masked last sequence and a one-token one */
  int32_t ids[24];
  float am[24], word[100 * 64], pos[8 * 64], type0[64];
  for (int i = 0; i < 24; ++i) ids[i] = (int32_t)(i * 7 % 100);
  for (int b = 0; b < B; ++b)
    for (int s = 0; s < S; ++s) am[b * S + s] = (b == 0) ? 1.0f : (b == 1 && s == 0 ? 1.0f : 0.0f);
  for (int i = 0; i < 100 * 64; ++i) word[i] = frand();
  for (int i = 0; i < 8 * 64; ++i) pos[i] = frand();
  for (int i = 0; i < 64; ++i) type0[i] = frand();
  float *emb = (float *)malloc((size_t)(B * S * d) * sizeof(float));
  float add_mask[24];
  orc_set_threads(threads);
  orc_embed_sum(ids, am, B, S, d, word, pos, type0, emb, add_mask);
  orc_bert_run(&m, emb, add_mask, B, S, -1);
  float pooled[3 * 64];
  (void)orc_pool_rows(emb, am, B, S, d, 0, 1, pooled);
  (void)orc_pool_rows(emb, am, B, S, d, 1, 0, pooled); /* CLS of a masked row: refused */
  if (!gated && !rope) {
    /* the int8 datapath on the same stack */
    int8_t *wq[4];
    float *ws[4], *ias[4];
    const int64_t K[4] = {d, d, d, f}, N[4] = {3 * d, d, f, d};
    orc_i8_operands q;
    for (int i = 0; i < 4; ++i) {
      wq[i] = (int8_t *)malloc((size_t)(L * K[i] * N[i]));
      for (int64_t j = 0; j < L * K[i] * N[i]; ++j) wq[i][j] = (int8_t)((j * 37) % 255 - 127);
      ws[i] = ones((size_t)(L * N[i]));
      ias[i] = ones((size_t)(L * K[i]));
      q.wq[i] = wq[i];
      q.wscale[i] = ws[i];
      q.ias[i] = ias[i];
    }
    orc_embed_sum(ids, am, B, S, d, word, pos, type0, emb, add_mask);
    orc_bert_run_i8(&m, &q, emb, add_mask, B, S, 1);
    for (int i = 0; i < 4; ++i) {
      free(wq[i]);
      free(ws[i]);
      free(ias[i]);
    }
  }
  /* a per-lane pool runs the same stack */
  if (orc_lane_begin(2) != 0 || orc_lane_begin(2) != -1) {
    printf("lane pool refused\n");
    exit(1);
  }
  orc_embed_sum(ids, am, B, S, d, word, pos, type0, emb, add_mask);
  orc_bert_run(&m, emb, add_mask, B, S, 1);
  orc_lane_end();
  orc_lane_end(); /* a second end is a no-op */
  free(emb);
  free(cos_t);
  free(sin_t);
  free((void *)m.w_qkv);
  free((void *)m.b_qkv);
  free((void *)m.w_ao);
  free((void *)m.b_ao);
  free((void *)m.w_up);
  free((void *)m.b_up);
  free((void *)m.w_down);
  free((void *)m.b_down);
  free((void *)m.ln1_g);
  free((void *)m.ln1_b);
  free((void *)m.ln2_g);
  free((void *)m.ln2_b);
  free((void *)m.emb_ln_g);
  free((void *)m.emb_ln_b);
}

static void preln_case(void) {
  const int64_t L = 1, d = 64, f = 128, B = 2, S = 3;
  orc_encoder m;
  memset(&m, 0, sizeof m);
  m.layers = L;
  m.hidden = d;
  m.heads = 2;
  m.head_dim = 32;
  m.ffn = f;
  m.w_qkv = rnd((size_t)(d * 3 * d));
  m.b_qkv = rnd((size_t)(3 * d));
  m.w_ao = rnd((size_t)(d * d));
  m.b_ao = rnd((size_t)d);
  m.w_up = rnd((size_t)(d * f));
  m.b_up = rnd((size_t)f);
  m.w_down = rnd((size_t)(f * d));
  m.b_down = rnd((size_t)d);
  m.ln1_g = ones((size_t)d);
  m.ln1_b = rnd((size_t)d);
  m.ln2_g = ones((size_t)d);
  m.ln2_b = rnd((size_t)d);
  m.fin_ln_g = ones((size_t)d);
  m.fin_ln_b = rnd((size_t)d);
  float *x = rnd((size_t)(B * S * d));
  orc_preln_run(&m, x, B, S, 1e-5, 0.125f, -1);
  /* conv front end, ViT patches, head */
  float *mel = rnd(4 * 8), *w1 = rnd((size_t)(d * 4 * 3)), *b1 = rnd((size_t)d);
  float *w2 = rnd((size_t)(d * d * 3)), *b2 = rnd((size_t)d), *out = rnd((size_t)(4 * d));
  orc_conv_front_end(mel, 4, 8, w1, b1, w2, b2, d, out);
  float *px = rnd(3 * 32 * 32), *rows = rnd(4 * 3 * 16 * 16);
  orc_vit_patches(px, 32, 16, rows);
  float *head = rnd((size_t)(d * 10)), *hb = rnd(10), logits[10];
  orc_head_matvec(head, hb, x, d, 10, logits);
  free(x);
  free(mel);
  free(w1);
  free(b1);
  free(w2);
  free(b2);
  free(out);
  free(px);
  free(rows);
  free(head);
  free(hb);
  free((void *)m.w_qkv);
  free((void *)m.b_qkv);
  free((void *)m.w_ao);
  free((void *)m.b_ao);
  free((void *)m.w_up);
  free((void *)m.b_up);
  free((void *)m.w_down);
  free((void *)m.b_down);
  free((void *)m.ln1_g);
  free((void *)m.ln1_b);
  free((void *)m.ln2_g);
  free((void *)m.ln2_b);
  free((void *)m.fin_ln_g);
  free((void *)m.fin_ln_b);
}

static void ops_case(void) {
  /* elementwise and row ops at one row, ragged counts and special values */
  float x[40];
  for (int i = 0; i < 40; ++i) x[i] = frand() * 100.0f;
  x[3] = INFINITY;
  x[4] = -INFINITY;
  x[5] = NAN;
  uint16_t b16[40], o16[40];
  int32_t i32[40];
  for (int i = 0; i < 40; ++i) i32[i] = (int32_t)((uint32_t)i * 123456789u);
  orc_gelu_poly_inplace(x, 40);
  orc_gelu_erf_inplace(x, 40);
  orc_narrow_f32_bf16(x, b16, 40);
  orc_narrow_i32_bf16(i32, b16, 40);
  orc_narrow_i32_bf16_twice(i32, b16, 40);
  orc_aie_gelu_erf_bf16(b16, o16, 40);
  orc_aie_gelu_poly_bf16(b16, o16, 40);
  float g[8] = {1, 1, 1, 1, 1, 1, 1, 1}, be[8] = {0};
  orc_aie_softmax_bf16(b16, o16, 5, 8);
  orc_aie_layernorm_bf16(b16, o16, 5, 8, g, be, 1e-5f);
  /* the polynomial softmax takes a multiple of 8 columns (the sequence) and
     one mask row per rows_per_mask_row rows */
  float s[32];
  for (int i = 0; i < 32; ++i) s[i] = frand();
  float mask[16] = {0, -1e30f, 0, 0, -1e30f, -1e30f, 0, 0, 0, 0, 0, 0, 0, 0, 0, -1e30f};
  orc_softmax_rows_poly(s, 4, 8, mask, 2);
  orc_softmax_rows_exact(s, 4, 6, NULL, 1);
  orc_softmax_rows_exact(s, 4, 8, mask, 2);
  orc_layer_norm_rows(s, 3, 8, g, be, 1e-12f);
  orc_layernorm_rows_f64(s, 3, 8, g, be, 1e-5);
  /* GEMM, int8 halves */
  float *A = rnd(7 * 24), *W = rnd(24 * 9), *C = rnd(7 * 9), bias[9] = {0};
  orc_gemm_nt(A, 7, W, 24, 9, bias, C);
  orc_gemm_nt(A, 1, W, 24, 9, NULL, C);
  int8_t q[7 * 24], wq[24 * 9];
  float sa[7], ias[24], ws[9];
  int32_t acc[7 * 9];
  for (int i = 0; i < 24; ++i) ias[i] = 1.0f;
  for (int i = 0; i < 9; ++i) ws[i] = 0.01f;
  for (int i = 0; i < 24 * 9; ++i) wq[i] = (int8_t)(i % 255 - 127);
  orc_quantise_a_int8(A, 7, 24, ias, q, sa);
  orc_gemm_i8(q, 7, 24, wq, 9, acc);
  orc_dequantise_c(acc, 7, 9, sa, ws, bias, C);
  orc_gemm_i8_dequant(A, 7, 24, ias, wq, ws, bias, 9, C);
  /* RoPE and GLU */
  float *qkv = rnd(5 * 3 * 64), ct[5 * 32], st[5 * 32], up[5 * 256], gl[5 * 128];
  float inv[16];
  for (int i = 0; i < 16; ++i) inv[i] = 1.0f / (float)(i + 1);
  orc_rope_tables(5, 32, 0.0, inv, ct, st);
  orc_rope_qkv(qkv, 5, 5, 2, 32, ct, st);
  for (int i = 0; i < 5 * 256; ++i) up[i] = frand();
  orc_glu(up, 5, 128, 1, gl);
  orc_glu(up, 5, 128, 2, gl);
  /* panels: ragged tilings and refused ones */
  uint16_t panel[96 * 64], kn[96 * 64];
  for (int i = 0; i < 96 * 64; ++i) panel[i] = (uint16_t)i;
  if (orc_untile_b_panel(panel, 96, 64, 32, 32, 4, 8, kn) != 0 ||
      orc_untile_b_panel(panel, 96, 64, 48, 64, 8, 8, kn) != 0 ||
      orc_untile_b_panel(panel, 96, 64, 40, 64, 8, 8, kn) != -1 ||
      orc_untile_b_panel(panel, 0, 64, 32, 32, 4, 8, kn) != -1) {
    printf("untile returns\n");
    exit(1);
  }
  uint8_t packed[96 * 64 / 2];
  int8_t wide[96 * 64];
  float gs[96 * 64];
  for (int i = 0; i < 96 * 64 / 2; ++i) packed[i] = (uint8_t)(i * 29);
  for (int i = 0; i < 96 * 64; ++i) gs[i] = 1.5f + (float)(i % 7);
  if (orc_widen_i4_panel(packed, 96, 64, 32, 32, 4, 8, gs, 24, wide) != 0 ||
      orc_widen_i4_panel(packed, 96, 64, 32, 32, 4, 8, gs, 0, wide) != 0 ||
      orc_widen_i4_panel(packed, 96, 64, 32, 32, 4, 8, gs, 7, wide) != 0 ||
      orc_widen_i4_panel(packed, 95, 1, 95, 1, 1, 1, gs, 0, wide) != -1 ||
      orc_widen_i4_panel(packed, 96, 64, 32, 32, 4, 8, gs, -1, wide) != -1) {
    printf("widen returns\n");
    exit(1);
  }
  free(A);
  free(W);
  free(C);
  free(qkv);
}

int main(void) {
  ops_case();
  bert_case(0, 0, 1);
  bert_case(0, 0, 4);
  bert_case(1, 1, 3);
  bert_case(2, 1, 2);
  preln_case();
  orc_set_threads(1);
  printf("oracle ok\n");
  return 0;
}
