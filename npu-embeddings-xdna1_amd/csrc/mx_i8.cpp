// mx_i8.cpp -- the int8 (W8A8) datapath's C ABI: staging an int8 design's B
// operand with its scales, the int8 GEMM with dequantise_c fused, and the two
// activation quantisers (quantise_a_int8 and add_norm_quant). Every entry
// validates its arguments and refuses by name, like the bf16 entries in
// mx_abi.cpp.
#include "mx_internal.hpp"
#include "mx_kernels.hpp"

#include <cstring>
#include <string>
#include <vector>

namespace mx {

namespace {

bool aligned(const void *p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// The largest K whose int8 products cannot overflow the int32 accumulator:
// K * 127^2 <= 2^31 - 1 (the reference's exactness condition, tools/lib/
// gemm_i8.py:54-57).
constexpr int64_t kMaxI8K = 2147483647LL / (127 * 127);

template <typename T>
int upload(const T *host, size_t count, T **dev, const char *what) {
  void *p = nullptr;
  hipError_t e = dev_malloc((void **)&p, count * sizeof(T));
  if (e != hipSuccess) return hip_fail(e, what);
  e = mx::upload(p, host, count * sizeof(T));
  if (e != hipSuccess) {
    (void)hipFree(p);
    return hip_fail(e, what);
  }
  *dev = static_cast<T *>(p);
  return MX_OK;
}

}  // namespace

void free_i8(I8Operand &op) {
  if (op.wq) (void)hipFree(op.wq);
  if (op.wscale) (void)hipFree(op.wscale);
  if (op.ias) (void)hipFree(op.ias);
  op = I8Operand{};
}

int stage_i8(mx_ctx *ctx, const int8_t *kn_host, const float *wscale_host,
             const float *asmooth_host, int64_t K, int64_t N, int64_t tile_k, int64_t tile_n,
             int64_t mac_s, int64_t mac_t, I8Operand *out) {
  if (!kn_host || !wscale_host || !asmooth_host)
    return fail(MX_E_INVALID, "stage_weight_i8: null operand, wscale or asmooth");
  if (K <= 0 || N <= 0) return fail(MX_E_INVALID, "stage_weight_i8: zero dimension");
  if (K % 16)
    return fail(MX_E_INVALID, "stage_weight_i8: K = " + std::to_string(K) +
                                  " is not a multiple of 16 (the int8 GEMM reads K in "
                                  "16-byte chunks)");
  if (tile_k > 0) {
    const int rc = check_panel("stage_weight_i8", K, N, tile_k, tile_n, mac_s, mac_t);
    if (rc) return rc;
  }
  int rc = use_device(ctx);
  if (rc) return rc;
  // 1/asmooth once, in fp32, as BertEncoder::gemm reciprocates it
  // (bert_encoder.cpp:764-772).
  std::vector<float> ias(static_cast<size_t>(K));
  for (int64_t k = 0; k < K; ++k) ias[k] = 1.0f / asmooth_host[k];
  I8Operand op;
  rc = upload(wscale_host, static_cast<size_t>(N), &op.wscale, "stage_weight_i8: wscale");
  if (!rc) rc = upload(ias.data(), ias.size(), &op.ias, "stage_weight_i8: asmooth");
  const size_t n = static_cast<size_t>(K) * N;
  if (!rc && tile_k <= 0) {
    std::vector<int8_t> panel(n);
    for (int64_t k = 0; k < K; ++k)
      for (int64_t j = 0; j < N; ++j)
        panel[static_cast<size_t>(j) * K + k] = kn_host[static_cast<size_t>(k) * N + j];
    rc = upload(panel.data(), n, &op.wq, "stage_weight_i8: operand");
  } else if (!rc) {
    int8_t *tiled = nullptr;
    rc = upload(kn_host, n, &tiled, "stage_weight_i8: panel");
    if (!rc) {
      void *wq = nullptr;
      SetupStream st;
      hipError_t e = dev_malloc((void **)&wq, n);
      if (e == hipSuccess) {
        op.wq = static_cast<int8_t *>(wq);
        e = mxk::untile_panel_i8(tiled, K, N, (int)tile_k, (int)tile_n, (int)mac_s, (int)mac_t,
                                 op.wq, st.s);
      }
      if (e == hipSuccess) e = st.finish();
      (void)hipFree(tiled);
      if (e != hipSuccess) rc = hip_fail(e, "stage_weight_i8: untile");
    }
  }
  if (rc) {
    free_i8(op);
    return rc;
  }
  *out = op;
  return MX_OK;
}

// The checks gemm_b_panel makes of an I4 operand before it widens it
// (int4_panel.hpp:87-173): a two-dimensional [K, N] with an even number of
// nibbles, a block_panel tiling, int4_group >= 0 (0: one group over K) and a
// gscale of ceil(K / group) rows.
int check_i4(const std::string &what, int64_t K, int64_t N, int64_t group, int64_t tile_k,
             int64_t tile_n, int64_t mac_s, int64_t mac_t) {
  if (K <= 0 || N <= 0 || (K * N) % 2)
    return fail(MX_E_INVALID, what + ": I4 payload of [" + std::to_string(K) + "," +
                                  std::to_string(N) + "] holds an odd number of nibbles; two "
                                  "int4 values make a byte");
  int rc = check_panel(what, K, N, tile_k, tile_n, mac_s, mac_t);
  if (rc) return rc;
  if (group < 0)
    return fail(MX_E_INVALID, what + ": int4_group is " + std::to_string(group) +
                                  "; rows per group must be >= 0, where 0 means one group over "
                                  "the whole K");
  return MX_OK;
}

int stage_i4(mx_ctx *ctx, const uint8_t *packed_host, const float *gscale_host, int64_t group,
             const float *wscale_host, const float *asmooth_host, int64_t K, int64_t N,
             int64_t tile_k, int64_t tile_n, int64_t mac_s, int64_t mac_t, I8Operand *out) {
  if (!packed_host || !gscale_host || !wscale_host || !asmooth_host)
    return fail(MX_E_INVALID, "stage_weight_panel_i4: null payload, gscale, wscale or asmooth");
  int rc = check_i4("stage_weight_panel_i4", K, N, group, tile_k, tile_n, mac_s, mac_t);
  if (rc) return rc;
  if (K % 16)
    return fail(MX_E_INVALID, "stage_weight_panel_i4: K = " + std::to_string(K) +
                                  " is not a multiple of 16 (the int8 GEMM reads K in "
                                  "16-byte chunks)");
  rc = use_device(ctx);
  if (rc) return rc;
  const int64_t g = group == 0 ? K : group, G = (K + g - 1) / g;
  uint8_t *packed = nullptr;
  float *gs = nullptr;
  int8_t *tiled = nullptr;
  rc = upload(packed_host, static_cast<size_t>(K * N / 2), &packed,
              "stage_weight_panel_i4: payload");
  if (!rc) rc = upload(gscale_host, static_cast<size_t>(G * N), &gs,
                       "stage_weight_panel_i4: gscale");
  if (!rc) {
    void *p = nullptr;
    const hipError_t e = dev_malloc((void **)&p, static_cast<size_t>(K) * N);
    if (e != hipSuccess) rc = hip_fail(e, "stage_weight_panel_i4: hipMalloc");
    tiled = static_cast<int8_t *>(p);
  }
  if (!rc) {
    SetupStream st;
    hipError_t e = mxk::widen_i4_panel(packed, K, N, (int)tile_k, (int)tile_n, (int)mac_s,
                                       (int)mac_t, gs, g, tiled, st.s);
    if (e == hipSuccess) e = st.finish();
    if (e != hipSuccess) rc = hip_fail(e, "stage_weight_panel_i4: widen");
  }
  if (packed) (void)hipFree(packed);
  if (gs) (void)hipFree(gs);
  // The widened run is exactly an I8 container's run: the scales as
  // stage_i8 stages them (1/asmooth once, in fp32), the run untiled into the
  // [N, K] panel.
  I8Operand op;
  if (!rc) {
    std::vector<float> ias(static_cast<size_t>(K));
    for (int64_t k = 0; k < K; ++k) ias[k] = 1.0f / asmooth_host[k];
    rc = upload(wscale_host, static_cast<size_t>(N), &op.wscale,
                "stage_weight_panel_i4: wscale");
    if (!rc) rc = upload(ias.data(), ias.size(), &op.ias, "stage_weight_panel_i4: asmooth");
  }
  if (!rc) {
    void *wq = nullptr;
    SetupStream st;
    hipError_t e = dev_malloc((void **)&wq, static_cast<size_t>(K) * N);
    if (e == hipSuccess) {
      op.wq = static_cast<int8_t *>(wq);
      e = mxk::untile_panel_i8(tiled, K, N, (int)tile_k, (int)tile_n, (int)mac_s, (int)mac_t,
                               op.wq, st.s);
    }
    if (e == hipSuccess) e = st.finish();
    if (e != hipSuccess) rc = hip_fail(e, "stage_weight_panel_i4: untile");
  }
  if (tiled) (void)hipFree(tiled);
  if (rc) {
    free_i8(op);
    return rc;
  }
  *out = op;
  return MX_OK;
}

int gemm_i8_checked(mx_stream *s, const int8_t *A, const float *a_scale, int64_t M, int64_t K,
                    int64_t lda, const int8_t *Wt, const float *wscale, int64_t N,
                    const float *bias, int epilogue, const float *residual, void *C,
                    int c_dtype, int64_t ldc, const Live &live) {
  // The 32-bit row offsets come first: a shape the kernel cannot address is
  // refused whatever else is wrong with the call.
  if (!mxk::lds_offsets_fit(lda, K, 1))
    return fail(MX_E_UNSUPPORTED, "gemm_i8: lda " + std::to_string(lda) + " / K " +
                                      std::to_string(K) + " -- the int8 GEMM addresses a tile's "
                                      "rows by 32-bit byte offsets (lda and K below 2^24)");
  if (!s) return fail(MX_E_INVALID, "gemm_i8: null stream");
  if (!A || !Wt || !C) return fail(MX_E_INVALID, "gemm_i8: null A, weight or C");
  if (M <= 0 || N <= 0 || K <= 0) return fail(MX_E_INVALID, "gemm_i8: zero dimension");
  if (M > INT32_MAX / 2 || N > INT32_MAX / 2)
    return fail(MX_E_INVALID, "gemm_i8: dimension beyond 2^30");
  if (K > kMaxI8K)
    return fail(MX_E_INVALID, "gemm_i8: K = " + std::to_string(K) +
                                  " can overflow the int32 accumulator (K * 127^2 >= 2^31)");
  if (K % 64 || K < 256)
    return fail(MX_E_UNSUPPORTED, "gemm_i8: K = " + std::to_string(K) +
                                      " -- the int8 GEMM reads K in 64-deep slabs, at least "
                                      "four of them (K % 64 == 0, K >= 256)");
  if (lda < K || lda % 16)
    return fail(MX_E_INVALID, "gemm_i8: lda " + std::to_string(lda) +
                                  " is below K or not a multiple of 16");
  if (N % 4) return fail(MX_E_UNSUPPORTED, "gemm_i8: N % 4 != 0");
  if (ldc < N) return fail(MX_E_INVALID, "gemm_i8: ldc < N");
  const bool narrow = (epilogue & MX_EPI_NARROW_C) != 0;
  const int act = epilogue & ~MX_EPI_NARROW_C;
  if (act < MX_EPI_NONE || act > MX_EPI_GELU_ERF)
    return fail(MX_E_INVALID, "gemm_i8: unknown epilogue " + std::to_string(epilogue));
  if (c_dtype != MX_F32 && c_dtype != MX_BF16 && c_dtype != MX_I32)
    return fail(MX_E_INVALID, "gemm_i8: C dtype must be MX_F32, MX_BF16 or MX_I32");
  if (narrow && (residual || c_dtype == MX_I32))
    return fail(MX_E_UNSUPPORTED, "gemm_i8: a narrowed C takes no residual and is not the raw "
                                  "MX_I32 product");
  if (c_dtype == MX_I32) {
    if (bias || residual || epilogue != MX_EPI_NONE)
      return fail(MX_E_INVALID, "gemm_i8: MX_I32 C is the raw accumulator -- no bias, "
                                "residual or epilogue");
  } else if (!a_scale || !wscale) {
    return fail(MX_E_INVALID, "gemm_i8: dequantisation needs a_scale and wscale");
  }
  if (!aligned(A, 16) || !aligned(Wt, 16) || !aligned(C, 16))
    return fail(MX_E_INVALID, "gemm_i8: A, the weight panel and C must be 16-byte aligned");
  if (ldc % (c_dtype == MX_BF16 ? 8 : 4))
    return fail(MX_E_INVALID, "gemm_i8: ldc must keep C rows 16-byte aligned");
  if ((bias && !aligned(bias, 16)) || (wscale && !aligned(wscale, 16)) ||
      (a_scale && !aligned(a_scale, 4)) || (residual && !aligned(residual, 16)))
    return fail(MX_E_INVALID, "gemm_i8: bias, wscale and residual must be 16-byte aligned");
  mxk::GemmI8Args a{A,
                    lda,
                    Wt,
                    M,
                    N,
                    K,
                    c_dtype == MX_I32 ? nullptr : a_scale,
                    c_dtype == MX_I32 ? nullptr : wscale,
                    bias,
                    epilogue,
                    residual,
                    C,
                    c_dtype == MX_BF16 ? 1 : c_dtype == MX_I32 ? 2 : 0,
                    ldc,
                    live.dev,
                    live.hint};
  const hipError_t e = mxk::gemm_i8(a, s->stream);
  return e == hipSuccess ? MX_OK : hip_fail(e, "gemm_i8 launch");
}

int quantise_checked(mx_stream *s, const void *a, int a_dtype, int64_t lda, int64_t rows,
                     int64_t K, const float *ias, int8_t *q, int64_t ldq, float *a_scale,
                     const Live &live) {
  if (!s) return fail(MX_E_INVALID, "quantise_a_int8: null stream");
  if (!a || !ias || !q || !a_scale)
    return fail(MX_E_INVALID, "quantise_a_int8: null a, ias, q or a_scale");
  if (rows <= 0 || K <= 0) return fail(MX_E_INVALID, "quantise_a_int8: zero dimension");
  if (a_dtype != MX_F32 && a_dtype != MX_BF16)
    return fail(MX_E_INVALID, "quantise_a_int8: a must be MX_F32 or MX_BF16");
  if (K % 4 || mxk::quant_groups(K) == 0)
    return fail(MX_E_UNSUPPORTED, "quantise_a_int8: K = " + std::to_string(K) +
                                      " (a multiple of 4, at most 8192)");
  if (lda < K || lda % 4 || ldq < K || ldq % 4)
    return fail(MX_E_INVALID, "quantise_a_int8: row strides below K or not multiples of 4");
  if (!aligned(a, a_dtype == MX_F32 ? 16 : 8) || !aligned(ias, 16) || !aligned(q, 4))
    return fail(MX_E_INVALID, "quantise_a_int8: a, ias or q misaligned");
  if (rows > (int64_t)INT32_MAX * 4)
    return fail(MX_E_INVALID, "quantise_a_int8: too many rows");
  const hipError_t e = mxk::quantise_rows(a, a_dtype == MX_BF16, lda, rows, K, ias, q, ldq,
                                          a_scale, s->stream, live.dev);
  return e == hipSuccess ? MX_OK : hip_fail(e, "quantise_a_int8 launch");
}

int layernorm_i8_checked(mx_stream *s, const float *x, const void *y, int y_dtype,
                         const float *gamma, const float *beta, float eps, int64_t rows,
                         int64_t cols, float *out_f32, const float *ias, int8_t *q,
                         float *a_scale, const Live &live) {
  if (!s) return fail(MX_E_INVALID, "layernorm_i8: null stream");
  if (!x || !gamma || !beta || !ias || !q || !a_scale)
    return fail(MX_E_INVALID, "layernorm_i8: null x, gamma, beta, ias, q or a_scale");
  if (rows <= 0 || cols <= 0) return fail(MX_E_INVALID, "layernorm_i8: zero dimension");
  if (y && y_dtype != MX_F32 && y_dtype != MX_BF16)
    return fail(MX_E_INVALID, "layernorm_i8: y must be MX_F32 or MX_BF16");
  if (cols % 4 || cols > 4096)
    return fail(MX_E_UNSUPPORTED, "layernorm_i8: cols = " + std::to_string(cols) +
                                      " (a multiple of 4, at most 4096)");
  if (!(eps >= 0.0f)) return fail(MX_E_INVALID, "layernorm_i8: bad eps");
  if (!aligned(x, 16) || (y && !aligned(y, y_dtype == MX_F32 ? 16 : 8)) || !aligned(gamma, 16) ||
      !aligned(beta, 16) || !aligned(ias, 16) || (out_f32 && !aligned(out_f32, 16)) ||
      !aligned(q, 4))
    return fail(MX_E_INVALID, "layernorm_i8: misaligned tensor");
  if (rows > (int64_t)INT32_MAX * 4) return fail(MX_E_INVALID, "layernorm_i8: too many rows");
  const hipError_t e = mxk::layernorm_quant(x, y, y_dtype == MX_BF16, gamma, beta, eps, rows, cols,
                                            out_f32, ias, q, a_scale, s->stream, live.dev);
  return e == hipSuccess ? MX_OK : hip_fail(e, "layernorm_i8 launch");
}

}  // namespace mx

using namespace mx;

namespace {

int push_slot(mx_ctx *ctx, const I8Operand &op, int64_t K, int64_t N, int *slot) {
  std::lock_guard<std::mutex> lk(ctx->mu);
  WeightSlot w;
  w.K = K;
  w.N = N;
  w.wq = op.wq;
  w.wscale = op.wscale;
  w.ias = op.ias;
  ctx->slots.push_back(w);
  *slot = static_cast<int>(ctx->slots.size());
  return MX_OK;
}

int i8_slot(mx_ctx *ctx, int wslot, WeightSlot *out, const char *who) {
  std::lock_guard<std::mutex> lk(ctx->mu);
  if (wslot < 1 || wslot > static_cast<int>(ctx->slots.size()) ||
      (!ctx->slots[wslot - 1].wq && !ctx->slots[wslot - 1].wt))
    return fail(MX_E_INVALID, std::string(who) + ": no weight staged in slot " +
                                  std::to_string(wslot));
  if (!ctx->slots[wslot - 1].wq)
    return fail(MX_E_INVALID, std::string(who) + ": slot " + std::to_string(wslot) +
                                  " holds a bf16 operand; the int8 GEMM needs one staged by "
                                  "mx_stage_weight_i8");
  *out = ctx->slots[wslot - 1];
  return MX_OK;
}

}  // namespace

extern "C" {

int mx_stage_weight_i8(mx_ctx *ctx, const int8_t *kn_host, const float *wscale_host,
                       const float *asmooth_host, int64_t K, int64_t N, int *slot) {
  clear_error();
  if (!ctx || !slot) return fail(MX_E_INVALID, "mx_stage_weight_i8: null argument");
  I8Operand op;
  const int rc = stage_i8(ctx, kn_host, wscale_host, asmooth_host, K, N, 0, 0, 0, 0, &op);
  if (rc) return rc;
  return push_slot(ctx, op, K, N, slot);
}

int mx_stage_weight_panel_i8(mx_ctx *ctx, const int8_t *panel_host, const float *wscale_host,
                             const float *asmooth_host, int64_t K, int64_t N, int64_t tile_k,
                             int64_t tile_n, int64_t mac_s, int64_t mac_t, int *slot) {
  clear_error();
  if (!ctx || !slot) return fail(MX_E_INVALID, "mx_stage_weight_panel_i8: null argument");
  if (tile_k <= 0)
    return fail(MX_E_INVALID, "mx_stage_weight_panel_i8: the block_panel layout needs a "
                              "positive tile_k");
  I8Operand op;
  const int rc = stage_i8(ctx, panel_host, wscale_host, asmooth_host, K, N, tile_k, tile_n,
                          mac_s, mac_t, &op);
  if (rc) return rc;
  return push_slot(ctx, op, K, N, slot);
}

int mx_stage_weight_panel_i4(mx_ctx *ctx, const uint8_t *packed_host, const float *gscale_host,
                             int64_t int4_group, const float *wscale_host,
                             const float *asmooth_host, int64_t K, int64_t N, int64_t tile_k,
                             int64_t tile_n, int64_t mac_s, int64_t mac_t, int *slot) {
  clear_error();
  if (!ctx || !slot) return fail(MX_E_INVALID, "mx_stage_weight_panel_i4: null argument");
  I8Operand op;
  const int rc = stage_i4(ctx, packed_host, gscale_host, int4_group, wscale_host, asmooth_host,
                          K, N, tile_k, tile_n, mac_s, mac_t, &op);
  if (rc) return rc;
  return push_slot(ctx, op, K, N, slot);
}

int mx_widen_panel_i4(mx_stream *s, const uint8_t *packed, const float *gscale,
                      int64_t int4_group, int64_t K, int64_t N, int64_t tile_k, int64_t tile_n,
                      int64_t mac_s, int64_t mac_t, int8_t *out) {
  clear_error();
  if (!s || !packed || !gscale || !out)
    return fail(MX_E_INVALID, "mx_widen_panel_i4: null argument");
  int rc = check_i4("mx_widen_panel_i4", K, N, int4_group, tile_k, tile_n, mac_s, mac_t);
  if (rc) return rc;
  const hipError_t e = mxk::widen_i4_panel(packed, K, N, (int)tile_k, (int)tile_n, (int)mac_s,
                                           (int)mac_t, gscale, int4_group == 0 ? K : int4_group,
                                           out, s->stream);
  return e == hipSuccess ? MX_OK : hip_fail(e, "mx_widen_panel_i4");
}

int mx_weight_i8_scales(mx_ctx *ctx, int slot, const float **wscale, const float **ias) {
  clear_error();
  if (!ctx || !wscale || !ias) return fail(MX_E_INVALID, "mx_weight_i8_scales: null argument");
  WeightSlot w;
  const int rc = i8_slot(ctx, slot, &w, "mx_weight_i8_scales");
  if (rc) return rc;
  *wscale = w.wscale;
  *ias = w.ias;
  return MX_OK;
}

int mx_gemm_i8(mx_stream *s, const int8_t *A, const float *a_scale, int64_t M, int64_t K,
               int64_t lda, int wslot, const float *bias, int epilogue, const float *residual,
               void *C, int c_dtype, int64_t ldc) {
  clear_error();
  if (!s) return fail(MX_E_INVALID, "gemm_i8: null stream");
  WeightSlot w;
  const int rc = i8_slot(s->ctx, wslot, &w, "gemm_i8");
  if (rc) return rc;
  if (w.K != K)
    return fail(MX_E_INVALID, "gemm_i8: A has K = " + std::to_string(K) + " but slot " +
                                  std::to_string(wslot) + " holds a [" + std::to_string(w.K) +
                                  ", " + std::to_string(w.N) + "] operand");
  return gemm_i8_checked(s, A, a_scale, M, K, lda, w.wq, w.wscale, w.N, bias, epilogue, residual,
                         C, c_dtype, ldc);
}

int mx_gemm_i8_wt(mx_stream *s, const int8_t *A, const float *a_scale, int64_t M, int64_t K,
                  int64_t lda, const int8_t *Wt, const float *wscale, int64_t N,
                  const float *bias, int epilogue, const float *residual, void *C, int c_dtype,
                  int64_t ldc) {
  clear_error();
  return gemm_i8_checked(s, A, a_scale, M, K, lda, Wt, wscale, N, bias, epilogue, residual, C,
                         c_dtype, ldc);
}

int mx_quantise_a_int8(mx_stream *s, const void *a, int a_dtype, int64_t rows, int64_t K,
                       const float *ias, int8_t *q, float *a_scale) {
  clear_error();
  return quantise_checked(s, a, a_dtype, K, rows, K, ias, q, K, a_scale);
}

int mx_layernorm_i8(mx_stream *s, const float *x, const void *y, int y_dtype,
                    const float *gamma, const float *beta, float eps, int64_t rows,
                    int64_t cols, float *out_f32, const float *ias, int8_t *q,
                    float *a_scale) {
  clear_error();
  return layernorm_i8_checked(s, x, y, y_dtype, gamma, beta, eps, rows, cols, out_f32, ias, q,
                              a_scale);
}

}  // extern "C"
