/*
 * oracle.h -- CPU restatement of the reference's host (CPU-fallback) encoder
 * path. TEST INFRASTRUCTURE ONLY.
 *
 * This library is the checker: tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product path (libmx_encoder.so) never links
 * or calls it, and there is no CPU fallback in the product.
 *
 * Written in plain C from the reference's algorithms (the reference's C++ does
 * not build here: it needs XRT, and common/json_min.hpp does not compile
 * against this GCC's libstdc++). Each function names the reference file:line
 * it restates. Compiled with the reference's own host flags
 * (-O2 -march=x86-64-v3, runtime/CMakeLists.txt:302) so the AVX2 branches are
 * the ones restated and timed.
 *
 * Parity pins (what checks each function against something other than itself)
 * are listed per function below; tests/test_oracle_*.py hold the checks.
 *
 * Every weight operand is fp32 [K, N] row-major holding bf16-exact values (the
 * reference widens its bf16 container operands exactly, common/host_b.hpp:
 * 74-224). Every tensor argument is a plain host pointer.
 */
#ifndef MX_ORACLE_H
#define MX_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- threads -------------------------------------------------------------
 * One persistent pool, like app::Pool (runtime/src/pool.cpp:28-110). Rows are
 * independent in every op below, so the partition never changes a bit. */
void orc_set_threads(int n);
int orc_threads(void);
/* A pool of n workers for the calling thread alone (one --pipeline lane,
 * runtime/include/runtime/run_setup.hpp:465-477): until orc_lane_end, every
 * op this thread runs uses it. Returns 0, or -1 if the thread already has
 * one. */
int orc_lane_begin(int n);
void orc_lane_end(void);

/* ---- bf16 -----------------------------------------------------------------
 * to_bf16: (u + 0x7FFF + ((u >> 16) & 1)) >> 16 on the fp32 bits
 * (runtime/include/common/host_kernels.hpp:157-161). Pinned bit-exact against
 * oracle/_ref (the reference header compiled as-is) over all 2^32 inputs. */
uint16_t orc_to_bf16(float x);
float orc_from_bf16(uint16_t h);
void orc_bf16_fill(uint16_t *dst, const float *src, size_t n);
void orc_bf16_read(float *dst, const uint16_t *src, size_t n);
/* Round every element to the nearest bf16 value, kept as fp32. */
void orc_round_bf16_inplace(float *x, size_t n);

/* ---- GELU -----------------------------------------------------------------
 * gelu8: max(x,0) + p(min(|x|,4)), degree-8 Horner in fp32 FMA
 * (host_kernels.hpp:325-352; bert_encoder.cpp:532-580 gelu_cpu).
 * Pinned bit-exact against oracle/_ref's gelu8 (scalar and AVX2 forms), and
 * against 0.5x(1+erf(x/sqrt2)) to the fit's stated accuracy.
 * gelu_erf_exact: 0.5 x (1 + erf(x / sqrt 2)) in double, rounded once
 * (runtime/include/common/app_state.hpp:116-120); pinned against Python's
 * math.erf. */
float orc_gelu8(float x);
void orc_gelu_poly_inplace(float *x, size_t n);   /* gelu_cpu            */
float orc_gelu_erf_exact(float x);
void orc_gelu_erf_inplace(float *x, size_t n);    /* npu_ops.cpp:470-476 */

/* ---- exp2 polynomial (exp2_avx2, host_kernels.hpp:358-379) ----------------
 * 2^x = 2^k * p(f), k = trunc(x), f = x - k, degree-7 Horner. Pinned
 * bit-exact against oracle/_ref's exp2_avx2. */
void orc_exp2_poly(const float *x, float *y, size_t n);

/* ---- softmax --------------------------------------------------------------
 * softmax_cpu (bert_encoder.cpp:481-530): per row r of `cols` scores, add
 * mask row add_mask[(r / rows_per_mask_row) * cols ...], then
 * e_j = exp2_poly(max((x_j - max) * log2e, -120)), out = e_j * (1/sum).
 * rows_per_mask_row = heads * seq for BERT. add_mask may be NULL.
 * Pinned against an fp64 softmax (closed form) to 1e-6 and, per element,
 * against oracle/_ref's exp2_avx2. */
void orc_softmax_rows_poly(float *x, int64_t rows, int64_t cols,
                           const float *add_mask, int64_t rows_per_mask_row);
/* whisper::attention's softmax_row (npu_ops.cpp:591-599): max-subtracted
 * std::exp, sum in fp32, scaled by 1/sum (0 if sum is 0). Pinned against
 * an fp64 softmax. */
void orc_softmax_rows_exact(float *x, int64_t rows, int64_t cols,
                            const float *add_mask, int64_t rows_per_mask_row);

/* ---- LayerNorm ------------------------------------------------------------
 * layer_norm_cpu (bert_encoder.cpp:416-463), AVX2 branch: 8-lane fp32 mean and
 * variance partials, hsum256, biased variance, 1/sqrt(var + eps), then
 * fma(d*is, gamma, beta). `cols` must be a multiple of 8 (the reference
 * enforces hidden % 8 == 0, app_state.hpp:380-631). Pinned against a two-pass
 * fp64 LayerNorm. The reference hard-codes eps = 1e-12 for BERT. */
void orc_layer_norm_rows(float *x, int64_t rows, int64_t cols,
                         const float *gamma, const float *beta, float eps);
/* layernorm_rows (npu_ops.cpp:449-468): double sum and variance, fp32
 * normalise. Used by the ViT and Whisper encoders. */
void orc_layernorm_rows_f64(float *x, int64_t rows, int64_t cols,
                            const float *gamma, const float *beta, double eps);
/* x <- y + residual, elementwise (add_into, bert_encoder.cpp:1183-1194). */
void orc_add_into(float *x, const float *y, const float *residual, size_t n);

/* ---- GEMM -----------------------------------------------------------------
 * hostconv::gemm_nt (runtime/include/common/conv_host.hpp:148-181):
 * C[M,N] = A[M,K] @ B[K,N] + bias[N]; per element a sequential k-ordered FMA
 * chain from 0, bias added last. bias may be NULL (zero). Pinned bit-exact
 * against oracle/_ref's gemm_nt and against an fp64 product. */
void orc_gemm_nt(const float *A, int64_t M, const float *B, int64_t K,
                 int64_t N, const float *bias, float *C);

/* ---- host attention (BERT) ------------------------------------------------
 * qk_impl (bert_encoder.cpp:995-1052): scores[((b*H+h)*S + i)*S + j] =
 * q_i . k_j over head_dim, no scale (folded into Q), AVX2 8-wide FMA + hsum.
 * av_impl (bert_encoder.cpp:1062-1126): ctx[b*S+i, h*hd..] = sum_j p_ij v_j.
 * qkv is [B*S, 3*hidden] as Q|K|V. head_dim must be a multiple of 8. Pinned
 * against an fp64 brute-force attention on small shapes. */
void orc_qk(const float *qkv, int64_t B, int64_t S, int64_t H, int64_t hd,
            float *scores);
void orc_av(const float *scores, const float *qkv, int64_t B, int64_t S,
            int64_t H, int64_t hd, float *ctx);

/* whisper::attention (npu_ops.cpp:478-644), the no-softmax-design branch:
 * per query row and head, scores = (q.k) * scale, exact max-subtracted
 * softmax, ctx = sum p v. q row stride q_stride, K|V rows at kv (K at 0,
 * V at d_model) with stride kv_stride. No mask. Pinned against fp64. */
void orc_whisper_attention(const float *q, int64_t q_stride, const float *kv,
                           int64_t kv_stride, int64_t n_q, int64_t n_kv,
                           int64_t d_model, int64_t heads, int64_t head_dim,
                           float scale, float *out);

/* ---- embedding sum, mask, pooling -----------------------------------------
 * EmbedService::chunk / BertEncoder::encode (embed_service.cpp:29-64;
 * bert_encoder.cpp:1367-1417): emb[b*S+s] = word[id] + pos[s] + type[0]
 * (summed left to right in fp32); cam = mask (1/0); cmask = m > 0 ? 0 : -1e30.
 * Pinned by exact indexing invariants (tests). */
void orc_embed_sum(const int32_t *ids, const float *attn_mask, int64_t B,
                   int64_t S, int64_t hidden, const float *word,
                   const float *pos, const float *type0, float *emb,
                   float *add_mask);
/* app::pool_rows (runtime/include/common/app_state.hpp:335-374): CLS (row 0;
 * returns -1 if position 0 is masked) or mean (in-order double accumulation of
 * h*m, denominator max(sum m, 1e-9f)); optional L2 (double, clamp 1e-24 on the
 * squared norm). Pinned against the reference's own goldens: HF
 * last_hidden_state -> hf.pool.mean / hf.out.embedding / st.embedding
 * (the reference/goldens boundary .npz files). Returns 0 on success. */
int orc_pool_rows(const float *h, const float *attn_mask, int64_t B, int64_t S,
                  int64_t hidden, int cls_pool, int l2_normalize, float *out);

/* ---- AIE kernel restatements (bf16 in/out; the accelerator ops the GPU
 * kernels replace). bf16 narrowing here is RNE (the *_rne.cc variants and
 * narrow_*.cc all set conv_even). The softmax and LayerNorm sums end in
 * aie::reduce_add over 16 lanes, whose order the reference does not define
 * (the AIE API is outside it): lane 0 to 15 in turn is ASSUMED -- parity
 * unpinned for that one step (orc_numerics.c, aie_reduce_add16). -------- */
/* softmax.cc:76-160 (softmax_rne.cc:42-52): per row of `cols`: x = max(x,
 * -1e30) (in bf16); m = max; d = max(x - m, -100); arg = max(d*log2e, -120);
 * e = bf16(exp2_poly(arg)); sum over e in fp32; inv = 1/sum; out =
 * bf16(e*inv). */
void orc_aie_softmax_bf16(const uint16_t *in, uint16_t *out, int64_t rows,
                          int64_t cols);
/* layernorm.cc:85-142 (layernorm_rne.cc): fp32 two-pass stats of the bf16 row,
 * inv_std = fast_invsqrt(var + eps) (bit-trick seed + 2 Newton steps,
 * layernorm.cc:65-75), out = bf16((x-mean)*inv_std*gamma + beta). */
void orc_aie_layernorm_bf16(const uint16_t *in, uint16_t *out, int64_t rows,
                            int64_t cols, const float *gamma,
                            const float *beta, float eps);
/* gelu_erf.cc:79-145: 0.5x + 0.5|x| * (1 - t*P(t)*2^max(-u^2 log2e, -125)),
 * u = x/sqrt2, t = 1/(1+p|u|), A&S 7.1.26; bf16 RNE out. */
void orc_aie_gelu_erf_bf16(const uint16_t *in, uint16_t *out, int64_t n);
/* gelu_poly_rne.cc / gelu_poly.cc:77-176: gelu8 on the widened bf16 value,
 * bf16 RNE out. */
void orc_aie_gelu_poly_bf16(const uint16_t *in, uint16_t *out, int64_t n);
/* narrow_f32_bf16.cc:51-90: fp32 -> bf16, round to nearest even. The GPU
 * kernel is pinned to the host's to_bf16 integer formula. */
void orc_narrow_f32_bf16(const float *in, uint16_t *out, int64_t n);
/* narrow_i32_bf16.cc:66-95: int32 -> bf16 in ONE rounding (RNE on the
 * integer). Note the reference's host stand-in (--sim-c-bf16,
 * host_kernels.hpp:583-610) rounds twice (int32 -> fp32 -> bf16); the two
 * differ only for |v| > 2^24. This function is the single rounding; pinned
 * against exact integer arithmetic. */
void orc_narrow_i32_bf16(const int32_t *in, uint16_t *out, int64_t n);
/* The two-rounding host form, for the tests that state the difference. */
void orc_narrow_i32_bf16_twice(const int32_t *in, uint16_t *out, int64_t n);

/* ---- whole encoders --------------------------------------------------------
 * Every per-layer tensor is contiguous over layers: w_qkv is [L, d, 3d],
 * b_qkv [L, 3d], w_ao [L, d, d], w_up [L, d, f], w_down [L, f, d], LN
 * gamma/beta [L, d]. Q's block of w_qkv/b_qkv already carries 1/sqrt(hd)
 * (tools/pack/pack_npue.py:2630,2747), so attention uses scale 1. */
typedef struct {
  int64_t layers, hidden, heads, head_dim, ffn;
  const float *w_qkv, *b_qkv, *w_ao, *b_ao, *w_up, *b_up, *w_down, *b_down;
  const float *ln1_g, *ln1_b, *ln2_g, *ln2_b;
  const float *emb_ln_g, *emb_ln_b; /* BERT only: the embedding LayerNorm   */
  const float *fin_ln_g, *fin_ln_b; /* pre-LN only: the final LayerNorm     */
  /* The RoPE / gated-FFN BERT archs (nomic_bert_rope_swiglu,
   * gte_new_rope_geglu; app_state.hpp:440-550), BERT only. gated: 0 plain
   * GELU FFN, 1 SwiGLU (SiLU gate), 2 exact-erf GeGLU; w_up is then [d, 2f]
   * (up half first, gate half second) and b_up [2f]. rope_cos/rope_sin:
   * [S, head_dim] tables (orc_rope_tables), null = no RoPE. */
  int64_t gated;
  const float *rope_cos, *rope_sin;
} orc_encoder;

/* The RoPE tables of BertEncoder::apply_rope_qkv (bert_encoder.cpp:926-950):
 * cos/sin [S, head_dim], angle s * inv_freq_j in double, rounded once to
 * fp32, the half duplicated (column j and half + j equal). inv_freq from the
 * container's rope_inv_freq when given (gte), else gemma_rope_tables
 * (encoders/gemma_kernels.cpp:114-136): inv_freq_j = 1 / theta^(2j/hd) in
 * double (nomic). Pinned against oracle/_ref's gemma_rope_tables and by the
 * rotation invariants in the tests. */
void orc_rope_tables(int64_t S, int64_t head_dim, double theta, const float *inv_freq,
                     float *cos_t, float *sin_t);
/* apply_rope_qkv's rotation (bert_encoder.cpp:951-990) of Q and K (never V)
 * in a fused [rows, 3*H*hd] buffer, position s = row % S: per head, pairs
 * (j, j + half): o1 = x1*c - x2*s, o2 = x2*c + x1*s with every product
 * rounded (the AVX2 form: two multiplies and a subtract/add, no FMA). Pinned
 * by the complex-rotation closed form and the relative-position property. */
void orc_rope_qkv(float *qkv, int64_t rows, int64_t S, int64_t H, int64_t hd,
                  const float *cos_t, const float *sin_t);
/* swiglu_cpu (bert_encoder.cpp:582-627): up [rows, 2f] = lo | hi ->
 * out [rows, f]. act 1 (SiLU): a = max((-hi) * log2e, -120), out = lo *
 * (hi / (1 + exp2_avx2(a))); act 2 (exact-erf GeLU): out = lo *
 * gelu_erf_exact(hi). Pinned: exp2_avx2 against oracle/_ref, SiLU and GeLU
 * against their closed forms. */
void orc_glu(const float *up, int64_t rows, int64_t f, int act, float *out);

/* BertEncoder::run, host branch (bert_encoder.cpp:1419-1598): embedding LN,
 * then per layer QKV GEMM (-> apply_rope_qkv when m->rope_cos) -> qk ->
 * softmax_cpu (mask) -> av -> attn-out GEMM -> add_into + layer_norm_cpu ->
 * FFN-up GEMM -> gelu_cpu (or swiglu_cpu when m->gated) -> FFN-down GEMM ->
 * add_into + layer_norm_cpu. eps 1e-12 (hard-coded, :438/:456). x_io is
 * [B*S, hidden] fp32, updated in place (emb_in -> final hidden). add_mask is
 * [B, S] (0 / -1e30). layers_to_run < 0 means all. */
void orc_bert_run(const orc_encoder *m, float *x_io, const float *add_mask,
                  int64_t B, int64_t S, int64_t layers_to_run);

/* VitEncoder::run / WhisperEncoder::run layer body (vit/encoder.cpp:222-431;
 * whisper/encoder.cpp:114-213): pre-LN, layernorm_rows (double stats, eps),
 * whisper::attention per sequence (scale as given; 1 when folded into Q),
 * gelu_erf_exact, residual adds, final LayerNorm. x_io is [B*S, hidden]. */
void orc_preln_run(const orc_encoder *m, float *x_io, int64_t B, int64_t S,
                   double eps, float scale, int64_t layers_to_run);

/* Whisper's conv front end (whisper/features.cpp:390-469): conv1 (k3, p1) +
 * gelu_erf_exact, conv2 (k3, s2, p1) + gelu_erf_exact, permuted to
 * [T/2, hidden]. mel is [n_mels, T] channel-major; w1 [hidden, n_mels, 3],
 * w2 [hidden, hidden, 3] (PyTorch Conv1d layout). out is [T/2, hidden]. */
void orc_conv_front_end(const float *mel, int64_t n_mels, int64_t T,
                        const float *w1, const float *b1, const float *w2,
                        const float *b2, int64_t hidden, float *out);

/* ViT patch embedding input (vit/encoder.cpp:288-332 consumes it): im2col of
 * [3, H, W] pixels into [n_patches, 3*p*p] rows in (c, ky, kx) order, the
 * PyTorch Conv2d weight order. */
void orc_vit_patches(const float *pixels, int64_t img, int64_t patch,
                     float *rows);

/* head_matvec (runtime/src/vit/head.cpp:16-49): logits[j] = bias[j] +
 * sum_t cls[t] * head[t*num_labels + j], double accumulation. */
void orc_head_matvec(const float *head, const float *bias, const float *cls_row,
                     int64_t d_model, int64_t num_labels, float *logits);

/* ---- int8 W8A8: the array datapath's host halves --------------------------
 * quantise_a_int8 (host_kernels.hpp:263-320): per row, mx = max_j |a*ias|,
 * sc = mx > 0 ? mx/127 : 1, q = rint(clamp((a*ias)*(1/sc), -127, 127)) (the
 * AVX2 order: two rounded multiplies, clamp, nearest-even; the scalar tail
 * rounds before clamping, which gives the same integer). a_scale[r] = sc.
 * Pinned bit-exact against oracle/_ref's quantise_a_int8.
 * gemm_i8: C[M,N] = sum_k Aq[m,k] * Wq[k,n] in exact integer arithmetic (the
 * AIE int8 MMAC accumulates int32 exactly, tools/lib/gemm_i8.py:54-57; K*127^2
 * < 2^31 keeps it exact). Pinned against a 64-bit integer product.
 * dequantise_c (host_kernels.hpp:529-600, the int32-C AVX2 form):
 * out = fma(float(C) * sa[r], wscale[n], bias[n]). Pinned bit-exact against
 * oracle/_ref's dequantise_c.
 * gemm_i8_dequant: quantise -> gemm_i8 -> dequantise_c, the array branch of
 * BertEncoder::gemm (bert_encoder.cpp:741-924) for an int8 design. */
void orc_quantise_a_int8(const float *a, int64_t rows, int64_t K, const float *ias,
                         int8_t *q, float *a_scale);
void orc_gemm_i8(const int8_t *Aq, int64_t M, int64_t K, const int8_t *Wq, int64_t N,
                 int32_t *C);
void orc_dequantise_c(const int32_t *C, int64_t rows, int64_t N, const float *a_scale,
                      const float *wscale, const float *bias, float *out);
void orc_gemm_i8_dequant(const float *A, int64_t M, int64_t K, const float *ias,
                         const int8_t *Wq, const float *wscale, const float *bias,
                         int64_t N, float *out);

/* ---- the narrowed C of the array designs (c_elem_bytes == 2) -------------
 * The export default narrows C to bf16 on the core ("c_bf16": true,
 * tools/data/npu_targets.json:10; design.cpp:255) and the host finishes from
 * the bf16 value:
 * orc_dequantise_c_bf16: dequantise_c's 2-byte branch (host_kernels.hpp:
 * 529-560), out = fma(from_bf16(C) * sa[r], wscale[n], bias[n]) (the AVX2
 * form; the scalar tail is contracted to the same FMA at the reference's
 * -O2 -march=x86-64-v3). Pinned bit-exact against oracle/_ref's dequantise_c
 * with c_bytes = 2.
 * orc_bias_c_bf16: the bf16-C branch of BertEncoder::gemm (bert_encoder.cpp:
 * 874-900), out = from_bf16(C) + bias[n] in fp32. Pinned by the closed form
 * (an exact widening and one IEEE add).
 * orc_dequant_act_bf16: BertEncoder::dequant_act_bf16 (bert_encoder.cpp:
 * 633-712) for a 2-byte C: v = from_bf16(C) + bias in fp32, then gelu8
 * (gated 0) or the gated halves (1 SiLU / 2 exact-erf GeLU, as orc_glu,
 * out_n = N/2), then bf16_fill into dst [rows, out_n]. bert_encoder.cpp does
 * not build here; pinned by composing oracle/_ref's gelu8 and to_bf16 on
 * the closed-form v (tests), and the gated halves by orc_glu's own pins. */
void orc_dequantise_c_bf16(const uint16_t *C, int64_t rows, int64_t N, const float *a_scale,
                           const float *wscale, const float *bias, float *out);
void orc_bias_c_bf16(const uint16_t *C, int64_t rows, int64_t N, const float *bias,
                     float *out);
void orc_dequant_act_bf16(const uint16_t *C, int64_t rows, int64_t N, int gated,
                          const float *bias, uint16_t *dst);

/* The arithmetic of the array datapath in the whole-stack restatements
 * (orc_bert_run, orc_bert_run_i8), a bit set; 0 (the default) is the host
 * fallback. ORC_ARR_A_BF16: every bf16-datapath GEMM rounds its A to bf16
 * first (BertEncoder::gemm's bf16_fill, bert_encoder.cpp:776-782).
 * ORC_ARR_C_BF16: the narrowed C -- bf16 GEMMs give from_bf16(bf16(acc)) +
 * bias (orc_bias_c_bf16), int8 GEMMs dequantise narrow_i32_bf16(acc)
 * (orc_dequantise_c_bf16). ORC_ARR_ATTN_BF16: Q, K, V after the QKV GEMM (and
 * RoPE) and the attention context are rounded to bf16 (the array attention's
 * bf16 operands, attention_npu, bert_encoder.cpp:1151-1181). Returns the
 * previous setting. Not thread-safe: set it between runs. */
#define ORC_ARR_A_BF16 1
#define ORC_ARR_C_BF16 2
#define ORC_ARR_ATTN_BF16 4
int orc_set_array_arith(int flags);

/* The int8 operands of a BERT stack: per layer and GEMM (qkv, attn_out,
 * ffn_up, ffn_down) the [K, N] int8 weight, its [N] column scale and the [K]
 * reciprocal smoothing 1/asmooth (the reference reciprocates once, :764-772). */
typedef struct {
  const int8_t *wq[4];        /* each [layers][K*N]                         */
  const float *wscale[4];     /* each [layers][N]                           */
  const float *ias[4];        /* each [layers][K]                           */
} orc_i8_operands;

/* BertEncoder::run on an int8 container with gemm on the array and every
 * other op on the host, unfused (bert_encoder.cpp:1419-1598 with
 * fuse_ffn_epilogue off): each GEMM is gemm_i8_dequant; attention, GELU and
 * LayerNorm as orc_bert_run. The fused forms (add_norm_quant :1197-1300,
 * dequant_act_quant host_kernels.hpp:405-500) compute the same values in
 * one pass: LayerNorm then quantise, dequantise then GELU then quantise. */
void orc_bert_run_i8(const orc_encoder *m, const orc_i8_operands *q, float *x_io,
                     const float *add_mask, int64_t B, int64_t S, int64_t layers_to_run);

/* ---- the .npue container's B panels --------------------------------------
 * hostb::host_b_kn's untile (common/host_b.hpp:74-224, the BF16 branch of the
 * loop at :206-243): a [K, N] operand stored as (tile_k, tile_n) tiles in k,n
 * order, each tile as (mac_s, mac_t) sub-tiles, back to row-major [K, N] bf16
 * bits (the widening to fp32 is orc_bf16_read). Returns 0, or -1 for a shape
 * host_b_kn refuses (K % tile_k, N % tile_n, tile_k % mac_s, tile_n % mac_t,
 * a non-positive dimension). Pinned bit-exact against oracle/_ref's
 * host_b_kn reading the same container file, and as the exact inverse of the
 * tiling written as reshapes and transposes (tools/lib/npue.py:491-556). */
int orc_untile_b_panel(const uint16_t *panel, int64_t K, int64_t N, int64_t tile_k,
                       int64_t tile_n, int64_t mac_s, int64_t mac_t, uint16_t *kn);

/* int4 storage over the int8 datapath: npue::gemm_b_panel's I4 branch
 * (common/int4_panel.hpp:77-246). packed holds K * N / 2 bytes of the
 * container's flat run (two values per byte, even index in the low nibble);
 * gscale is F32 [ceil(K / g), N], g = int4_group (0: g = K). Writes the int8
 * run of the same tiling: out[f] = clip(nearbyint(t * gscale[k / g][n]),
 * -127, 127) for the sign-extended nibble t of element f at (k, n). Returns 0,
 * or -1 for a shape gemm_b_panel refuses (odd nibble count, a tiling that does
 * not divide, int4_group < 0). Pinned bit-exact against oracle/_ref's
 * gemm_b_panel reading the same container, and against the packer's
 * arithmetic written as numpy (tools/lib/npue.py fold_i4, :394-430). */
int orc_widen_i4_panel(const uint8_t *packed, int64_t K, int64_t N, int64_t tile_k,
                       int64_t tile_n, int64_t mac_s, int64_t mac_t, const float *gscale,
                       int64_t int4_group, int8_t *out);

#ifdef __cplusplus
}
#endif
#endif
