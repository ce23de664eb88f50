/*
 * mx_encoder.h -- C ABI of the MI355X (gfx950) encoder backend.
 *
 * The drop-in boundary for the reference runtime's encoder-layer hot path: the
 * per-op placement layer (--npu-ops codes gemm, attn, softm, layn, gelu) gains
 * a GPU backend, and every op the reference dispatches to its accelerator
 * through npu::Design (runtime/include/runtime/design.hpp:199-263) has an
 * entry point here. Each declaration names the reference interface it
 * replaces.
 *
 * Conventions
 *   - Every function returns an int status: MX_OK (0) or a negative MX_E_*.
 *     Nothing throws across the ABI. mx_last_error() returns the calling
 *     thread's message for its last failure, naming what was refused (the
 *     reference's refusals are std::runtime_error with a named reason,
 *     runtime/src/entry.cpp:74-77).
 *   - Tensor arguments are DEVICE pointers (from mx_alloc, or any device
 *     allocation on the context's GPU) unless the name ends in _host.
 *   - Operations on one mx_stream run in order; distinct streams may run
 *     concurrently (one per --pipeline lane, runtime/include/runtime/
 *     run_setup.hpp:778-874). Op calls are asynchronous; mx_sync() waits.
 *   - Weights staged with mx_stage_weight belong to the context; activations
 *     belong to the caller.
 *   - bf16 tensors are uint16_t bit patterns. Every fp32 -> bf16 narrowing is
 *     round-to-nearest-even by the reference's integer formula
 *     (u + 0x7FFF + ((u >> 16) & 1)) >> 16 (common/host_kernels.hpp:157-161),
 *     bit for bit, NaN behaviour included.
 */
#ifndef MX_ENCODER_H
#define MX_ENCODER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MX_OK 0
#define MX_E_INVALID (-1)     /* an argument was refused (shape, pointer, code) */
#define MX_E_DEVICE (-2)      /* a HIP call failed                             */
#define MX_E_UNSUPPORTED (-3) /* valid request this backend does not implement */
#define MX_E_STATE (-4)       /* object not ready (e.g. missing weights)       */
#define MX_E_DATA (-5)        /* the data itself was refused (e.g. CLS masked) */

typedef enum { MX_F32 = 0, MX_BF16 = 1, MX_I32 = 2, MX_I8 = 3 } mx_dtype;

/* GEMM epilogues: applied to acc + bias in fp32 before narrowing. */
typedef enum {
  MX_EPI_NONE = 0,
  MX_EPI_GELU_POLY = 1, /* gelu8 / gelu_cpu (bert_encoder.cpp:532-580)        */
  MX_EPI_GELU_ERF = 2   /* 0.5x(1+erf(x/sqrt2)) (app_state.hpp:116-120)       */
} mx_epilogue;
/* A flag OR'ed into a GEMM epilogue: the narrowed C of the array designs
 * (c_elem_bytes == 2, runtime/src/design.cpp:255; the export default,
 * tools/data/npu_targets.json:10). The finished accumulator is rounded to bf16
 * first -- fp32 to nearest even, int32 in one rounding of the integer -- and
 * the bias is added (bf16 datapath: from_bf16(c) + bias, bert_encoder.cpp:
 * 874-900) or the dequantisation applied (int8: fma(from_bf16(c) * a_scale,
 * wscale, bias), host_kernels.hpp:529-560) to that value, then the activation
 * (dequant_act_bf16, bert_encoder.cpp:633-712). No residual; for an fp32 C on
 * the bf16 datapath, no activation (the reference activates on the way into
 * the next bf16 A); on the int8 datapath not with the raw int32 C. Shapes the
 * direct-to-LDS kernel does not take (K % 32, misalignment, no bias) are
 * refused. */
#define MX_EPI_NARROW_C 32

typedef enum {
  MX_GELU_POLY = 0,   /* gelu_cpu / gelu_poly_rne.cc: degree-8 fit            */
  MX_GELU_ERF = 1,    /* exact-erf GELU (gelu_erf_exact)                      */
  MX_GELU_ERF_AS = 2  /* gelu_erf.cc: A&S 7.1.26 erf with exp2_poly           */
} mx_gelu_variant;

typedef enum {
  MX_SOFTMAX_POLY = 0,  /* softmax_cpu: exp2 poly, -120 argument floor       */
  MX_SOFTMAX_EXACT = 1, /* whisper::attention softmax_row: max-subtracted exp */
  MX_SOFTMAX_AIE = 2    /* softmax_rne.cc: bf16 in/out, three clamps, exps
                           narrowed to bf16 before the sum                    */
} mx_softmax_variant;

typedef struct mx_ctx mx_ctx;
typedef struct mx_stream mx_stream;
typedef struct mx_encoder mx_encoder;

typedef struct {
  int device;
  int compute_units;
  int clock_mhz;          /* peak engine clock                               */
  int64_t hbm_bytes;
  char arch[32];          /* "gfx950"                                        */
  double bf16_dense_tflops; /* compute_units * 4096 FLOP/clk * clock         */
} mx_device_props;

/* ---- library, device, streams, memory ------------------------------------ */

/* Message of the calling thread's last failed call ("" if none). */
const char *mx_last_error(void);
int mx_version(void);

/* Replaces npu::Device (runtime/include/runtime/device.hpp:28-39): opens GPU
 * `device`. Refuses a device that is not gfx950. */
int mx_create(int device, mx_ctx **out);
void mx_destroy(mx_ctx *ctx);
int mx_device_props_get(mx_ctx *ctx, mx_device_props *out);

/* One stream per --pipeline lane (run_setup.hpp:778-874; the reference's
 * lanes share one device under npu_mu, GPU lanes are independent streams). */
int mx_stream_create(mx_ctx *ctx, mx_stream **out);
void mx_stream_destroy(mx_stream *s);
/* Wait for every op issued on s. The reference's dispatch is synchronous
 * (Design::dispatch_only, runtime/src/design.cpp:502-532); a caller wanting
 * those semantics calls mx_sync after each op. Reports (MX_E_DATA) and clears
 * the data refusals that mx_encoder_embed_async calls left on s. */
int mx_sync(mx_stream *s);
/* The stream's hipStream_t, for callers that interleave their own work. */
void *mx_stream_handle(mx_stream *s);

/* Device buffers (Design::stage_alloc / slot_ptr, design.hpp:236-240, without
 * the host mapping: the GPU path keeps activations resident). */
int mx_alloc(mx_ctx *ctx, size_t bytes, void **dev);
int mx_free(mx_ctx *ctx, void *dev);
int mx_copy_h2d(mx_stream *s, void *dev_dst, const void *host_src, size_t bytes);
int mx_copy_d2h(mx_stream *s, void *host_dst, const void *dev_src, size_t bytes);

/* Replaces Design::stage (design.hpp:236) of a GEMM B operand: the [K, N]
 * row-major weight (host memory, fp32 holding any value -- it is rounded to
 * bf16 here by to_bf16 -- or bf16 bits) is copied once into a
 * context-owned, MFMA-ready [N, K] bf16 panel. *slot >= 1 on success. */
int mx_stage_weight(mx_ctx *ctx, const void *kn_host, int dtype, int64_t K,
                    int64_t N, int *slot);
int mx_release_weight(mx_ctx *ctx, int slot);

/* ---- per-op entry points (the accelerator ops of --npu-ops) --------------- */

/* gemm: replaces BertEncoder::gemm's array branch (bert_encoder.cpp:741-924)
 * and NpuGemm::run (runtime/src/whisper/npu_ops.cpp:200-288).
 * C[M, N] = epilogue(A[M, K] @ W + bias) (+ residual), W = slot `wslot`
 * ([K, N] as staged), bf16 A with row stride lda (elements), fp32 accumulate,
 * fp32 bias (nullable), optional fp32 residual [M, N] with stride ldc (may
 * alias C when c_dtype is MX_F32; the pre-LN encoders' x += proj), C fp32 or
 * bf16 (RNE) with row stride ldc. K % 8 == 0, lda % 8 == 0, 16-byte aligned A.
 * epilogue | MX_EPI_NARROW_C: the array design's narrowed C (see above). */
int mx_gemm(mx_stream *s, const uint16_t *A, int64_t M, int64_t K, int64_t lda,
            int wslot, const float *bias, int epilogue, const float *residual,
            void *C, int c_dtype, int64_t ldc);
/* The same with the weight panel given directly: Wt is [N, K] bf16 on the
 * device (row stride K). */
int mx_gemm_wt(mx_stream *s, const uint16_t *A, int64_t M, int64_t K,
               int64_t lda, const uint16_t *Wt, int64_t N, const float *bias,
               int epilogue, const float *residual, void *C, int c_dtype,
               int64_t ldc);

/* The GEMM kernel configuration mx_gemm / mx_gemm_wt choose for an [M, K] x
 * [K, N] product with aligned operands (no counterpart in the reference,
 * whose array GEMM has one fixed tiling per design): "lds_*" names the
 * direct-to-LDS pipelined kernel and its block tile, "staged_*" the
 * register-staged kernel used when K % 32 != 0 or an operand is not
 * vector-aligned. */
const char *mx_gemm_plan(int64_t M, int64_t N, int64_t K);

/* The plan for a C of c_dtype (MX_F32 / MX_BF16), with (residual != 0) or
 * without a residual, on the bf16 (int8 = 0, mx_gemm) or int8 (int8 = 1,
 * mx_gemm_i8) datapath: "lds_<BM>x<BN>x<slab K>_w<wave tile>_ns<slots>_..."
 * (no counterpart in the reference). */
const char *mx_gemm_plan_for(int64_t M, int64_t N, int64_t K, int c_dtype, int residual,
                             int int8);

/* attn (+softm fused): replaces the host qk/softmax_cpu/av triple
 * (bert_encoder.cpp:995-1135, :481-530), BertEncoder::attention_npu /
 * NpuAttention::run (runtime/src/whisper/attention_npu.cpp:177) and
 * whisper::attention (npu_ops.cpp:478-644). One pass per (sequence, head,
 * 128-query tile), scores never leave the chip.
 * qkv: bf16 [B*S, >=3*H*hd] rows of Q|K|V (head h at h*hd of each block), row
 * stride ld_qkv. scale multiplies q.k (1 when folded into Q). add_mask:
 * fp32 [B, S] additive (0 / -1e30), nullable. kv_len: int32 [B], keys at or
 * past kv_len[b] are skipped (must be masked anyway; nullable = S).
 * ctx: bf16 [B*S, H*hd], row stride ld_ctx. hd in {32, 64}. */
int mx_attention(mx_stream *s, const uint16_t *qkv, int64_t ld_qkv, int64_t B,
                 int64_t S, int64_t H, int64_t hd, float scale,
                 const float *add_mask, const int32_t *kv_len, uint16_t *ctx,
                 int64_t ld_ctx);

/* softm: replaces add_additive_mask + eltwise(softmax) (bert_encoder.cpp:
 * 465-475, :322-368) and NpuEltwise::softmax (whisper/eltwise.cpp:110-138):
 * in-place row softmax of `rows` rows of `cols`, row stride row_stride;
 * mask row add_mask[(r / rows_per_mask_row) * cols] added first (nullable).
 * dtype MX_F32 or MX_BF16 (MX_SOFTMAX_AIE needs MX_BF16). cols <= 4096. */
int mx_softmax_rows(mx_stream *s, void *x, int dtype, int64_t rows,
                    int64_t cols, int64_t row_stride, const float *add_mask,
                    int64_t rows_per_mask_row, int variant);

/* layn: replaces layer_norm / layer_norm_cpu / add_norm_bf16
 * (bert_encoder.cpp:370-463, :1304-1361) and layernorm_rows (npu_ops.cpp:
 * 449-468). z = x (+ y); out = (z - mean) / sqrt(var + eps) * gamma + beta,
 * biased variance, fp32 statistics. x, y: fp32 or bf16 (y nullable); outputs
 * out_f32 (nullable, may alias x when x is fp32) and/or out_bf16 (nullable).
 * Row stride = cols for every tensor. */
int mx_layernorm(mx_stream *s, const void *x, int x_dtype, const void *y,
                 int y_dtype, const float *gamma, const float *beta, float eps,
                 int64_t rows, int64_t cols, float *out_f32, uint16_t *out_bf16);

/* layn on the accelerator's own arithmetic: replaces the K2r LayerNorm kernel
 * (kernels/layernorm.cc:65-142 built with layernorm_rne.cc:42-52's
 * conv_even rounding) that eltwise(layn) dispatches on the array. bf16
 * x [rows, cols] -> bf16 out (may alias x), row stride cols; 16 fp32 partial
 * sums per pass (column j into sum j % 16, in column order) added in order,
 * the biased variance about that mean, fast_invsqrt (the 0x5f3759df estimate
 * and two Newton steps) of var + eps, y = (d * inv_std) * gamma + beta
 * rounded to bf16 to nearest even, every operation rounded on its own.
 * cols % 16 == 0 and cols <= 4096 (MX_E_UNSUPPORTED otherwise), rows <= 2^28;
 * x, out, gamma and beta 16-byte aligned. */
int mx_layernorm_aie(mx_stream *s, const uint16_t *x, const float *gamma, const float *beta,
                     float eps, int64_t rows, int64_t cols, uint16_t *out);

/* gelu: replaces gelu_cpu / eltwise(gelu) (bert_encoder.cpp:532-580),
 * gelu_erf_inplace (npu_ops.cpp:470-476) and NpuEltwise::gelu. Elementwise,
 * in place allowed (x == y with equal dtypes). */
int mx_gelu(mx_stream *s, const void *x, int x_dtype, void *y, int y_dtype,
            int64_t n, int variant);

/* The GEMM output epilogues of kernels/narrow_f32_bf16.cc:51-123 and
 * kernels/narrow_i32_bf16.cc:66-126 as standalone passes: fp32 -> bf16 by the
 * to_bf16 formula; int32 -> bf16 in ONE round-to-nearest-even rounding. */
int mx_narrow_f32_bf16(mx_stream *s, const float *in, uint16_t *out, int64_t n);
int mx_narrow_i32_bf16(mx_stream *s, const int32_t *in, uint16_t *out, int64_t n);

/* The callers either side of the encoder: EmbedService::chunk's embedding
 * sum and mask (runtime/src/server/embed_service.cpp:29-64) and
 * app::pool_rows (common/app_state.hpp:335-374).
 * embed_sum: emb[b*S+s] = word[ids] + pos[s] + type0 (fp32, left to right);
 * add_mask = m > 0 ? 0 : -1e30; kv_len[b] = 1 + last s with m != 0 (every
 * row pool_rows weights, negative weights included; keys before it with
 * m <= 0 are masked), or S when no m > 0 (the row attends uniformly like the
 * reference's all -1e30 row). Every
 * output nullable except emb. Ids outside [0, vocab) are refused by the
 * kernel (MX_E_DATA after the stream drains). */
int mx_embed_sum(mx_stream *s, const int32_t *ids, const float *attn_mask,
                 int64_t B, int64_t S, int64_t hidden, const float *word,
                 int64_t vocab, const float *pos, const float *type0,
                 float *emb, float *add_mask, int32_t *kv_len);
/* pool_rows: CLS (row 0; MX_E_DATA if position 0 is masked) or mean (in-order
 * double accumulation, denominator max(sum m, 1e-9f)), then optional L2
 * (double, clamp 1e-24). Bit-exact with the host form. Synchronises s. */
int mx_pool_rows(mx_stream *s, const float *h, const float *attn_mask,
                 int64_t B, int64_t S, int64_t hidden, int cls_pool,
                 int l2_normalize, float *out);

/* ---- the int8 (W8A8) datapath ---------------------------------------------
 * The reference's int8 design (a_elem_bytes == 1): A is quantised per row to
 * int8 on the way in, the array multiplies int8 x int8 into exact int32, and
 * C is dequantised with the row's scale, the column's weight scale and the
 * bias (BertEncoder::gemm's int8 branch, bert_encoder.cpp:741-924). The
 * container carries per operand the int8 [K, N] weight, `.wscale` [N] and the
 * SmoothQuant factor `.asmooth` [K] (bert_encoder.cpp:40-160); A is scaled by
 * ias = 1 / asmooth before it is quantised. */

/* Design::stage of an int8 design's B operand: [K, N] row-major int8 (host),
 * wscale [N] and asmooth [K] (host fp32). Stored as an [N, K] int8 panel with
 * wscale and ias = 1/asmooth (one fp32 division per element, as the reference
 * reciprocates, bert_encoder.cpp:764-772) on the device. K % 16 == 0. */
int mx_stage_weight_i8(mx_ctx *ctx, const int8_t *kn_host, const float *wscale_host,
                       const float *asmooth_host, int64_t K, int64_t N, int *slot);
/* The same from a container's pre-tiled I8 operand (block_panel layout, the
 * tiling of mx_stage_weight_panel), untiled on the GPU. */
int mx_stage_weight_panel_i8(mx_ctx *ctx, const int8_t *panel_host, const float *wscale_host,
                             const float *asmooth_host, int64_t K, int64_t N, int64_t tile_k,
                             int64_t tile_n, int64_t mac_s, int64_t mac_t, int *slot);
/* The same from a container's I4 operand (int4 storage over the int8
 * datapath; npue::gemm_b_panel's I4 branch, common/int4_panel.hpp:77-246):
 * packed_host holds K * N / 2 bytes of the block_panel run, two values per
 * byte (element f in nibble f % 2 of byte f / 2, low nibble first), gscale_host
 * the .gscale sidecar F32 [ceil(K / g), N] with g = int4_group (0: g = K).
 * Each nibble t (sign-extended) becomes q = clip(rint(t * gscale[k / g][n]),
 * -127, 127) on the GPU -- the int8 panel an I8 container carries -- which is
 * then staged as mx_stage_weight_panel_i8 stages it. Refusals as the
 * reference's: an odd nibble count, no tiling, int4_group < 0. */
int mx_stage_weight_panel_i4(mx_ctx *ctx, const uint8_t *packed_host, const float *gscale_host,
                             int64_t int4_group, const float *wscale_host,
                             const float *asmooth_host, int64_t K, int64_t N, int64_t tile_k,
                             int64_t tile_n, int64_t mac_s, int64_t mac_t, int *slot);
/* The widening alone, device to device on stream s: the I4 run (K * N / 2
 * bytes) and gscale in, the int8 run of the same tiling out (K * N bytes,
 * the bytes gemm_b_panel hands Design::stage, int4_panel.hpp:183-246). */
int mx_widen_panel_i4(mx_stream *s, const uint8_t *packed, const float *gscale,
                      int64_t int4_group, int64_t K, int64_t N, int64_t tile_k, int64_t tile_n,
                      int64_t mac_s, int64_t mac_t, int8_t *out);
/* The device vectors of a staged int8 operand: wscale [N] and ias [K] (the
 * ias to quantise this GEMM's A with). */
int mx_weight_i8_scales(mx_ctx *ctx, int slot, const float **wscale, const float **ias);

/* quantise_a_int8 (common/host_kernels.hpp:263-320): per row of a (fp32 or
 * bf16, [rows, K] contiguous), t = a * ias, sc = max|t| > 0 ? max|t| / 127 : 1,
 * q = rint(clamp(t * (1/sc), -127, 127)); a_scale[row] = sc. Bit-identical to
 * the host for finite input. K % 4 == 0, K <= 8192. */
int mx_quantise_a_int8(mx_stream *s, const void *a, int a_dtype, int64_t rows, int64_t K,
                       const float *ias, int8_t *q, float *a_scale);

/* gemm on an int8 design: Aq int8 [M, K] (row stride lda) with its a_scale [M]
 * times the int8 operand in `wslot`, exact int32 accumulation, then
 * dequantise_c (host_kernels.hpp:529-600) fused: y = fma(float(acc) *
 * a_scale[m], wscale[n], bias[n]) (bias nullable), bit-identical to the host's
 * int32-C form; then the epilogue (dequant_act_quant's activation, :405-500),
 * the optional fp32 residual, and C as fp32 or bf16. c_dtype MX_I32 stores
 * the raw int32 accumulators (the design's C before dequantise_c; no bias,
 * residual or epilogue). K % 64 == 0, 256 <= K <= 133144 (K * 127^2 < 2^31),
 * N % 4 == 0, lda % 16 == 0, 16-byte aligned A, C, bias and wscale.
 * epilogue | MX_EPI_NARROW_C: the design's narrowed C -- the int32 product
 * rounded to bf16 once (narrow_i32_bf16) before dequantise_c's 2-byte branch
 * (host_kernels.hpp:529-560) -- no residual, not with MX_I32 C. */
int mx_gemm_i8(mx_stream *s, const int8_t *A, const float *a_scale, int64_t M, int64_t K,
               int64_t lda, int wslot, const float *bias, int epilogue, const float *residual,
               void *C, int c_dtype, int64_t ldc);
/* The same with the operand given directly: Wt int8 [N, K] (row stride K),
 * wscale [N] on the device. */
int mx_gemm_i8_wt(mx_stream *s, const int8_t *A, const float *a_scale, int64_t M, int64_t K,
                  int64_t lda, const int8_t *Wt, const float *wscale, int64_t N,
                  const float *bias, int epilogue, const float *residual, void *C, int c_dtype,
                  int64_t ldc);

/* add_norm_quant (bert_encoder.cpp:1197-1300): the residual LayerNorm of
 * mx_layernorm (x fp32, y fp32 or bf16 nullable, out_f32 nullable and may
 * alias x) whose output is quantised in the same pass for the next int8 GEMM
 * (that GEMM's ias) into q [rows, cols] and a_scale [rows], as
 * mx_quantise_a_int8 would quantise out_f32. cols % 4 == 0, cols <= 4096. */
int mx_layernorm_i8(mx_stream *s, const float *x, const void *y, int y_dtype,
                    const float *gamma, const float *beta, float eps, int64_t rows,
                    int64_t cols, float *out_f32, const float *ias, int8_t *q,
                    float *a_scale);

/* ---- the RoPE and gated-FFN BERT archs ---------------------------------------
 * nomic_bert_rope_swiglu and gte_new_rope_geglu (app_state.hpp:440-550): the
 * BERT stack with rotary positions on Q and K after the QKV GEMM and a gated
 * FFN (FFN-up [d, 2f] = up | gate, then lo * act(hi) into FFN-down). */
typedef enum {
  MX_GATED_NONE = 0,     /* the plain GELU FFN                                */
  MX_GATED_SILU = 1,     /* SwiGLU: lo * silu(hi), the exp2 polynomial (nomic) */
  MX_GATED_GELU_ERF = 2  /* GeGLU: lo * gelu_erf(hi) (gte)                     */
} mx_gated;

/* apply_rope_qkv's tables (bert_encoder.cpp:926-950), on the host: cos/sin
 * [S, hd] fp32 (host memory), angle s * inv_freq_j in double rounded once,
 * the half duplicated; inv_freq_host [hd/2] (the container's rope_inv_freq,
 * gte) or, when null, gemma_rope_tables' inv_freq_j = 1/theta^(2j/hd)
 * (encoders/gemma_kernels.cpp:114-136, nomic). hd even. */
int mx_rope_tables(int64_t S, int64_t hd, double theta, const float *inv_freq_host,
                   float *cos_host, float *sin_host);
/* apply_rope_qkv (bert_encoder.cpp:951-990): Q and K (never V) of bf16
 * [B*S, ld_qkv] Q|K|V rows rotated in place, position s = row % S, pairs
 * (j, j + hd/2) of each head: o1 = x1*c - x2*s, o2 = x2*c + x1*s (each
 * product rounded, as the host's AVX2 form), narrowed once to bf16.
 * cos_t/sin_t: device fp32 [S, hd]. hd % 4 == 0. */
int mx_rope_qkv(mx_stream *s, uint16_t *qkv, int64_t ld_qkv, int64_t B, int64_t S,
                int64_t H, int64_t hd, const float *cos_t, const float *sin_t);
/* swiglu_cpu (bert_encoder.cpp:582-627): up [rows, 2f] = lo | hi (fp32 or
 * bf16) -> out [rows, f] (fp32 or bf16) = lo * act(hi), act MX_GATED_SILU
 * (x / (1 + exp2_poly(max(-x log2e, -120))), bit-identical to the host for
 * fp32 input) or MX_GATED_GELU_ERF. f % 4 == 0. */
int mx_glu(mx_stream *s, const void *up, int up_dtype, void *out, int out_dtype, int64_t rows,
           int64_t f, int act);

/* ---- placement registry (common/npu_ops_flag.hpp:75-214) ------------------ */

/* parse_npu_ops: comma list of codes (spaces ignored, empty items skipped);
 * an unknown code is refused by name with the list of valid ones, and the
 * set is replaced only on success. The codes and their meaning are the
 * reference's; "on the accelerator" means on this GPU. */
int mx_ops_parse(const char *list);
/* op_on_array(code): 1 if listed, 0 if not. */
int mx_op_on_gpu(const char *code);
/* The codes this build knows, comma-joined in table order. */
const char *mx_op_codes(void);
/* refuse_removed_op_flags (npu_ops_flag.hpp:238-268): MX_E_INVALID naming the
 * replacement when `flag` is one of the removed flags, else MX_OK. */
int mx_ops_check_flag(const char *flag);

/* ---- the encoder stack ----------------------------------------------------- */

typedef enum {
  MX_ARCH_BERT = 0,  /* post-LN (BertEncoder::run, bert_encoder.cpp:1419-1598) */
  MX_ARCH_PRELN = 1  /* pre-LN + final LN (VitEncoder::run, vit/encoder.cpp:
                        222-431; WhisperEncoder::run, whisper/encoder.cpp:
                        114-213)                                             */
} mx_arch;

typedef struct {
  int arch;           /* mx_arch                                             */
  int64_t layers, hidden, heads, head_dim, ffn;
  float ln_eps;       /* BERT: 1e-12 (hard-coded in the reference); ViT 1e-12;
                         Whisper 1e-5                                         */
  float attn_scale;   /* 1 when 1/sqrt(hd) is folded into Q (the packer's
                         convention)                                          */
  int gelu;           /* MX_GELU_POLY (BERT host path) or MX_GELU_ERF         */
  int cls_pool;       /* embed(): 1 = CLS, 0 = mean                           */
  int l2_normalize;   /* embed(): L2-normalise the pooled vector              */
  int64_t vocab, max_pos; /* embed(): word and position table rows (BERT)     */
  int front;          /* pre-LN front end: MX_FRONT_NONE (run() only), VIT or
                         WHISPER (mx_encoder_vit / mx_encoder_whisper)        */
  int64_t image, patch, labels; /* ViT: image side, patch side, head labels   */
  int64_t mels, frames;         /* Whisper: mel bins and input frames         */
  int gated_ffn;      /* BERT: mx_gated; gated -> "layer.{i}.ffn_up" is
                         [hidden, 2*ffn] (up half first) and its bias [2*ffn] */
  int rope;           /* BERT: rotary positions on Q and K (no position
                         table is needed then, but embed() still adds
                         "embeddings.position", as EmbedService::chunk does) */
  double rope_theta;  /* rope: the base when no "rope.inv_freq" [hd/2] tensor
                         is set (nomic); gte sets the frequencies instead     */
} mx_encoder_desc;

typedef enum { MX_FRONT_NONE = 0, MX_FRONT_VIT = 1, MX_FRONT_WHISPER = 2 } mx_front;

/* Replaces the BertEncoder + Design set wiring of setup_encoder
 * (run_setup.hpp:483-877). Tensors are then given by name with
 * mx_encoder_set, using the container's names (runtime/src/model.cpp:
 * 214-380): "layer.{i}.qkv", "layer.{i}.qkv.bias", "layer.{i}.attn_out",
 * "layer.{i}.attn_out.bias", "layer.{i}.ffn_up", "layer.{i}.ffn_up.bias",
 * "layer.{i}.ffn_down", "layer.{i}.ffn_down.bias", "layer.{i}.ln1.weight",
 * "layer.{i}.ln1.bias", "layer.{i}.ln2.weight", "layer.{i}.ln2.bias",
 * "embeddings.ln.weight", "embeddings.ln.bias", "embeddings.word",
 * "embeddings.position", "embeddings.token_type" (BERT), "final_ln.weight",
 * "final_ln.bias" (pre-LN). GEMM operands are [K, N] (fp32 values rounded
 * to bf16 by to_bf16, or bf16 bits); everything else fp32.
 * An int8 design's operands (BertEncoder::stage_all, bert_encoder.cpp:40-160)
 * are set as MX_I8 [K, N] with "layer.{i}.<gemm>.wscale" [N] and
 * "layer.{i}.<gemm>.asmooth" [K] beside them; the stack then runs the int8
 * datapath (each GEMM's A quantised per row by mx_layernorm_i8 or
 * mx_quantise_a_int8, the GEMM dequantising in its epilogue). Every GEMM
 * operand of a stack must be of one kind (mx_encoder_ready refuses a mix). */
int mx_encoder_create(mx_ctx *ctx, const mx_encoder_desc *desc,
                      mx_encoder **out);
void mx_encoder_destroy(mx_encoder *enc);
/* A --pipeline lane's encoder (run_setup.hpp:778-874): the same weights,
 * borrowed from a ready `enc`, with a workspace of its own, so lanes on
 * different streams run concurrently. It must be destroyed before `enc`;
 * setting a tensor on it is refused (the weights are the parent's). */
int mx_encoder_clone(mx_encoder *enc, mx_encoder **out);
int mx_encoder_set(mx_encoder *enc, const char *name, const void *host,
                   int dtype, int64_t count);
/* Every tensor the architecture needs has been set: MX_OK, else MX_E_STATE
 * naming the first missing one. Then builds what the stack derives on the
 * device: the gated FFN's interleaved FFN-up operands and, with RoPE, the
 * cos/sin tables for max_pos positions. */
int mx_encoder_ready(mx_encoder *enc);

/* BertEncoder::run (bert_encoder.cpp:1419-1598) with every op on the GPU,
 * activations resident: x_io fp32 [B*S, hidden] (device) goes in as the
 * embedding sum (BERT) or the front end's output (pre-LN) and comes out as
 * the final hidden state. add_mask fp32 [B, S] (nullable: no mask); kv_len
 * int32 [B] (nullable). Requires every code of the path (gemm, attn, softm,
 * layn, gelu) to be placed on the GPU, or no code at all (then the whole
 * stack is the GPU's by construction); a partial placement is refused by
 * name -- the per-op entry points above serve it. */
int mx_encoder_run(mx_encoder *enc, mx_stream *s, float *x_io,
                   const float *add_mask, const int32_t *kv_len, int64_t B,
                   int64_t S);
/* EmbedService::chunk minus the tokenizer (embed_service.cpp:29-64): ids and
 * the 1/0 attention mask (device, [B, S]) -> embedding sum -> run -> pool ->
 * out [B, hidden] (device). BERT only. Synchronises s. */
int mx_encoder_embed(mx_encoder *enc, mx_stream *s, const int32_t *ids,
                     const float *attn_mask, int64_t B, int64_t S, float *out);
/* mx_encoder_embed without its closing wait: no counterpart in the reference
 * (chunk() returns the pooled rows). For callers that queue the next batch
 * while this one runs, on one stream. The call enqueues the same work and
 * returns once it is queued; out is complete when s is synchronised. The
 * refusals the kernels raise on the data (a token id outside the vocabulary,
 * CLS pooling on a masked first token) stay in s's flag until it is next
 * read: by mx_sync(s), which reports them (MX_E_DATA) and clears it, or by a
 * synchronous call on s, which reports them as its own. Refusals of the
 * arguments come back from this call, as from mx_encoder_embed. ids,
 * attn_mask and out must stay valid until s is synchronised, and one
 * encoder's calls must share one stream (they share its workspace; a batch
 * larger than any before waits for the device before the workspace grows). */
int mx_encoder_embed_async(mx_encoder *enc, mx_stream *s, const int32_t *ids,
                           const float *attn_mask, int64_t B, int64_t S, float *out);

/* The static scratch of mx_encoder_embed_static: device memory that every GPU
 * the library runs on holds from mx_create until the process ends. */
#define MX_STATIC_SCRATCH_BYTES ((size_t)128 << 20)
/* mx_encoder_embed without allocating: no counterpart in the reference. For
 * callers that cannot allocate device memory (tight serving loops, harnesses
 * that forbid hipMalloc). The call is allocation-free and host-synchronous: it
 * reads the packed row count and the refusal flag back, so it cannot run
 * under HIP graph capture (a capturing stream is refused, MX_E_STATE, before
 * any launch or copy). The same inputs, output and refusals as
 * mx_encoder_embed, bit for bit the same pooled rows; its workspace is carved
 * from the library's static scratch (MX_STATIC_SCRATCH_BYTES per GPU) instead
 * of the encoder's own. The workspace is, in 256-byte pieces, the mask [B, S]
 * fp32, kv_len [B] and the plan [2B + 1] int32, then per computed row (the
 * packed row count with token packing, else B*S) its position int32, xb / ctx
 * / proj bf16 [hidden], qkv bf16 [3 hidden], up bf16 [ffn] (2 ffn gated, plus
 * the gated product [ffn]), emb fp32 [hidden] and on the int8 datapath xq
 * int8 [max(hidden, ffn)] and its scale fp32 (there up, the gated product and
 * proj are fp32); a batch whose workspace exceeds the scratch is refused
 * (MX_E_INVALID, naming both sizes). Also refused: timing on (its events are
 * created on demand) and an encoder whose device tables are stale
 * (MX_E_STATE: call mx_encoder_ready after the last tensor is set;
 * mx_encoder_from_npue and mx_encoder_clone return ready encoders). Every
 * call on one GPU shares that GPU's scratch, so a call holds the GPU's guard
 * (mx_static_guard_hold) from its first use of the scratch until it has
 * synchronised s: a call that overlaps it on the same GPU, from any encoder,
 * stream or thread, is refused (MX_E_STATE, naming the overlap) instead of
 * racing. Synchronises s. */
int mx_encoder_embed_static(mx_encoder *enc, mx_stream *s, const int32_t *ids,
                            const float *attn_mask, int64_t B, int64_t S, float *out);

/* The per-GPU guard of the static scratch (no counterpart in the reference;
 * for callers that cannot allocate and serialise their own use of the
 * scratch, and for tests of the overlap refusal). mx_static_guard_hold takes
 * device's guard as an mx_encoder_embed_static call does for its duration:
 * MX_E_STATE, naming the overlap, if a call or a hold already has it. While it
 * is held, mx_encoder_embed_static on that device is refused the same way.
 * mx_static_guard_release gives it back (MX_E_STATE if it is not held).
 * Host-only: neither touches the GPU. */
int mx_static_guard_hold(int device);
int mx_static_guard_release(int device);

/* How many device allocations (hipMalloc calls) the library has made in this
 * process: contexts' streams, staged weights, encoder workspaces, mx_alloc.
 * mx_encoder_embed_static adds none. Host-only. */
int64_t mx_device_allocations(void);

/* Token packing in mx_encoder_embed (on by default): the only rows of a
 * sequence that reach its pooled row are those before kv_len (every later
 * row is masked: never attended as a key, never pooled), so embed computes
 * only those -- each sequence's rows packed back to back, the GEMMs and
 * LayerNorms over the packed row count, attention per sequence over its own
 * rows. The pooled output is the padded computation's, bit for bit;
 * EmbedService::chunk (embed_service.cpp:29-64) computes the padded batch,
 * which off restores. The packed row count stays on the device: the
 * launches are sized for B*S rows and every row-wise kernel stops at the
 * count, so the host does not wait in the middle of the call (it is read
 * back instead with timing on, in mx_encoder_embed_static and on a stream's
 * first packed call, whose GEMM tiles have no earlier count to go by). The call
 * still synchronises its stream once, at its end, to read the refusal flag.
 * mx_encoder_run always computes every row (it returns them all). */
int mx_encoder_set_packing(mx_encoder *enc, int on);

/* CLS pruning in mx_encoder_embed (on by default; no counterpart in the
 * reference, which runs every row through every layer): with CLS pooling
 * only each sequence's first row of the last layer reaches the pooled output,
 * and in that layer only attention reads the other rows (as keys and values).
 * So the last layer's QKV GEMM runs over all rows, its attention computes the
 * first query of each sequence (over all its keys), and its attention-out
 * GEMM, LayerNorms and FFN run over the B first rows alone. Every query and
 * every row-wise operation is computed on its own, so the pooled output is
 * the unpruned computation's, bit for bit. mx_encoder_vit without a hidden
 * state to return prunes its last layer the same way (only the CLS rows reach
 * the head, after the final LayerNorm, which then runs over those rows alone).
 * Mean pooling, mx_encoder_run and mx_encoder_whisper are not affected; off
 * restores the last layer over every row. */
int mx_encoder_set_cls_pruning(mx_encoder *enc, int on);

/* The gated FFN (swiglu_cpu, bert_encoder.cpp:582-627) fused into FFN-up's
 * GEMM epilogue (on by default): FFN-up's operand is kept a second time with
 * its lo and hi rows interleaved, and the GEMM writes lo * act(hi) directly,
 * the [M, 2f] intermediate never reaching memory. The output is the unfused
 * GEMM-then-glu pair's, bit for bit; off runs that pair. No counterpart in
 * the reference, whose host path runs the two steps. */
int mx_encoder_set_fusion(mx_encoder *enc, int on);

/* The narrowed C of the array designs (off by default): c_elem_bytes == 2
 * (runtime/src/design.cpp:255), the export default ("c_bf16": true,
 * tools/data/npu_targets.json:10). Every GEMM of the BERT stack rounds its
 * finished accumulator to bf16 before the bias or the dequantisation
 * (MX_EPI_NARROW_C), as BertEncoder::gemm's array branch then computes on the
 * host (bert_encoder.cpp:741-924): the QKV result from_bf16(c) + bias; the
 * attention-out and FFN-down results from_bf16(c) + bias kept in fp32 for the
 * residual LayerNorm (:874-900); FFN-up through dequant_act_bf16 (:633-712:
 * from_bf16(c) + bias, GELU or the gated halves combined in fp32, one
 * rounding to bf16); on an int8 container fma(from_bf16(c) * a_scale, wscale,
 * bias) (dequantise_c's and dequant_act_quant's 2-byte branches,
 * host_kernels.hpp:405-560). The gated FFN then runs unfused. Off: the
 * accumulator enters the epilogue in fp32 (int32) as it is. BERT encoders
 * only (MX_E_UNSUPPORTED otherwise). */
int mx_encoder_set_narrowed_c(mx_encoder *enc, int on);

/* VitEncoder::run + head_matvec (runtime/src/vit/encoder.cpp:222-431,
 * runtime/src/vit/head.cpp:16-49), every step on the GPU: pixels fp32
 * [B, 3, image, image] (device) -> im2col patch rows (c, ky, kx order) -> patch
 * GEMM + bias -> [CLS; patches] + positions -> the pre-LN layers and final
 * LayerNorm -> CLS rows -> head GEMM + bias -> logits fp32 [B, labels]
 * (device). hidden (nullable, device, fp32 [B*(np+1), hidden]) receives the
 * final hidden state; without it the last layer is CLS-pruned
 * (mx_encoder_set_cls_pruning). Tensors: "patch_embed.weight" [3*patch^2, hidden],
 * "patch_embed.bias", "cls_token" [hidden], "position" [np+1, hidden],
 * "head.weight" [hidden, labels] (label fastest, as head.cpp reads it),
 * "head.bias" [labels]. image % patch == 0, patch % 8 == 0, image % 4 == 0.
 * Synchronises s. */
int mx_encoder_vit(mx_encoder *enc, mx_stream *s, const float *pixels,
                   int64_t B, float *logits, float *hidden);
/* WhisperEncoder::run (runtime/src/whisper/encoder.cpp:114-213) with the conv
 * front end of whisper/features.cpp:390-469 on the GPU: mel fp32
 * [B, mels, frames] (device) -> conv1 (k3, pad 1) + exact-erf GELU -> conv2
 * (k3, stride 2, pad 1) + GELU -> + positions -> the pre-LN layers and final
 * LayerNorm -> hidden fp32 [B*frames/2, hidden] (device). Each convolution is
 * one GEMM per sample over a time-major bf16 copy padded by a zero frame on
 * each side (its im2col rows overlap, nothing is copied). Tensors:
 * "conv1.weight" [hidden, mels, 3] and "conv2.weight" [hidden, hidden, 3]
 * (Conv1d layout), "conv1.bias", "conv2.bias", "position" [frames/2, hidden].
 * frames even, 3*mels and 3*hidden multiples of 32. Synchronises s. */
int mx_encoder_whisper(mx_encoder *enc, mx_stream *s, const float *mel,
                       int64_t B, float *hidden);

/* BertEncoder::Timings (runtime/include/encoders/bert_encoder.hpp:72-87) as
 * hipEvent times of the last run, in milliseconds, when timing is on (one
 * event pair around every launch, on the stream the kernels run on). The
 * gemm_site_* arrays split the GEMMs by layer site: [0] QKV, [1] attention
 * out, [2] FFN up, [3] FFN down. */
typedef struct {
  double gemm_ms, attn_ms, ln_ms, other_ms, total_ms;
  int64_t gemm_launches, attn_launches, ln_launches, other_launches;
  double gemm_flop, attn_flop; /* algorithmic FLOPs of the last run           */
  double gemm_site_ms[4], gemm_site_flop[4];
  int64_t gemm_site_launches[4];
} mx_timings;
int mx_encoder_set_timing(mx_encoder *enc, int on);
int mx_encoder_timings(mx_encoder *enc, mx_timings *out);

/* ---- the embedding service ----------------------------------------------
 * EmbedService::embed (runtime/src/server/embed_service.cpp:12-108) minus the
 * tokenizer: n sequences of token ids (host int32 [n, seq]) and their 1/0
 * attention masks (host fp32 [n, seq]) -> pooled rows (host fp32
 * [n, hidden]). The request is cut into chunks of `batch` sequences (plan(),
 * :12-27), taken by `lanes` workers -- each a thread with its own stream,
 * device buffers and encoder clone -- and each chunk is chunk() (:29-64):
 * embedding sum, the encoder, pooling, into its rows of out_host. The first
 * failing chunk stops the rest and its refusal is returned (:80-92). Results
 * do not depend on the lane count or the chunk size. One call at a time per
 * service; `enc` must outlive it.
 * A lane keeps two chunks in flight: inputs staged in pinned host slots and
 * copied by DMA, the embed queued without a wait, the pooled rows copied back
 * while the lane's next chunk runs. Lanes overlap on the GPU only on hardware
 * queues of their own: HIP maps streams onto GPU_MAX_HW_QUEUES queues (4 by
 * default), and two lanes whose streams share one run one after the other --
 * create the service before other long-lived streams, or keep lanes plus the
 * process's other live streams within that count. */
typedef struct mx_embed_service mx_embed_service;
int mx_embed_service_create(mx_encoder *enc, int lanes, int64_t batch, int64_t seq,
                            mx_embed_service **out);
void mx_embed_service_destroy(mx_embed_service *svc);
int mx_embed_service_embed(mx_embed_service *svc, const int32_t *ids_host,
                           const float *mask_host, int64_t n, float *out_host);

/* ---- the .npue weight container ------------------------------------------
 * npue::File (runtime/include/runtime/model.hpp, runtime/src/model.cpp:
 * 214-380): the container is mapped read-only; the 64-byte header is checked
 * (magic "NPUE", version 1, data_offset 4096-aligned, file size = data_offset
 * + data_length) and the JSON directory read. Refusals name the file and the
 * reason, like the reference's std::runtime_error messages. */
typedef struct mx_npue mx_npue;
typedef struct {
  char dtype[8];               /* "BF16", "F32", "I8", "I4", "U8", ...       */
  int ndim;                    /* of padded_shape (at most 4 kept)           */
  int64_t padded_shape[4], logical_shape[4];
  int block_panel;             /* layout.kind == "block_panel"               */
  int64_t tile_k, tile_n, mac_s, mac_t; /* the layout, when block_panel       */
  const void *data;            /* into the mapping; valid until close        */
  uint64_t nbytes;
} mx_npue_tensor_info;
int mx_npue_open(const char *path, mx_npue **out);
void mx_npue_close(mx_npue *f);
/* File::config_string (model.cpp:374-379): the value's text -- a JSON string
 * unescaped, a number or literal as written, an object or array as its raw
 * JSON. Copies at most len-1 bytes plus a NUL into buf (nullable); returns
 * the full length, or MX_E_INVALID naming a missing key. */
int mx_npue_config(const mx_npue *f, const char *key, char *buf, size_t len);
int mx_npue_tensor_count(const mx_npue *f);
const char *mx_npue_tensor_name(const mx_npue *f, int index);
/* File::info + File::raw (model.cpp:352-364). */
int mx_npue_tensor(const mx_npue *f, const char *name, mx_npue_tensor_info *out);

/* Design::stage (design.hpp:236) of a container's pre-tiled GEMM operand: the
 * bf16 bytes exactly as the container stores them -- a [K, N] operand tiled
 * (tile_k, tile_n) in k,n order, each tile in (mac_s, mac_t) sub-tiles
 * (tools/lib/npue.py:491-556) -- are copied to the GPU once and untiled there
 * into the MFMA-ready [N, K] panel. The same element lands where
 * hostb::host_b_kn (common/host_b.hpp:74-224) puts it; that function's
 * shape refusals are kept (K % tile_k, N % tile_n, tile_k % mac_s,
 * tile_n % mac_t). */
int mx_stage_weight_panel(mx_ctx *ctx, const uint16_t *panel_host, int64_t K, int64_t N,
                          int64_t tile_k, int64_t tile_n, int64_t mac_s, int64_t mac_t,
                          int *slot);
/* mx_encoder_set for a pre-tiled container operand ("layer.{i}.qkv", ...). */
int mx_encoder_set_panel(mx_encoder *enc, const char *name, const uint16_t *panel_host,
                         int64_t K, int64_t N, int64_t tile_k, int64_t tile_n,
                         int64_t mac_s, int64_t mac_t);
/* setup_encoder for a BERT container (run_setup.hpp:483-877 with
 * app::set_model_shape, app_state.hpp:380-620, and BertEncoder::stage_all,
 * bert_encoder.cpp:40-160). Three archs load:
 *  - "bert_abs_gelu_postln": absolute positions; a plain FFN, or a gated one
 *    when the config says gated_ffn true;
 *  - "nomic_bert_rope_swiglu": needs position_embedding_type "rope",
 *    gated_ffn true, swiglu_halves "fc11_up|fc12_gate" and a positive
 *    rope_theta;
 *  - "gte_new_rope_geglu": needs position_embedding_type "rope", gated_ffn
 *    true, glu_halves beginning "up_first|gate_second", rope_inv_freq (an
 *    array of head_dim/2 numbers) and an activation key.
 * Any other arch is refused by name. A gated container's gate activation is
 * its "activation" key ("silu" or "gelu", the exact erf form; missing means
 * silu except on gte; anything else is refused). Geometry from num_layers /
 * hidden / num_heads / head_dim / intermediate / max_seq_len; pooling "cls"
 * or "mean"; l2_normalize (default true); LayerNorm eps 1e-12 and the
 * polynomial GELU of a plain FFN (gelu_cpu), as BertEncoder hard-codes them.
 * Every tensor is set from the mapping: pre-tiled BF16 GEMM operands through
 * mx_encoder_set_panel, and an --int8 pack's pre-tiled I8 operands with their
 * .wscale/.asmooth through the int8 staging of mx_stage_weight_panel_i8, and
 * an --int4 pack's I4 operands (with .gscale and config int4_group) widened
 * on the GPU and staged likewise (mx_stage_weight_panel_i4). A "host" container (F32
 * row-major operands) is refused for the GEMM, as the reference refuses
 * --npu-ops gemm on one (bert_encoder.cpp:79-87). The encoder is ready on
 * MX_OK. */
int mx_encoder_from_npue(mx_ctx *ctx, const mx_npue *f, mx_encoder **out);

#ifdef __cplusplus
}
#endif
#endif
