// mx_abi.cpp -- the C ABI: device, streams, memory, weight staging and the
// per-op entry points (validated, refused by name). The error state and the
// placement registry are host-only code in mx_host.cpp.
#include "mx_internal.hpp"
#include "mx_kernels.hpp"

#include <algorithm>
#include <cctype>
#include <cmath>
#include <cstring>
#include <set>
#include <sstream>

namespace mx {

int hip_fail(hipError_t e, const char *what) {
  return fail(MX_E_DEVICE, std::string(what) + ": " + hipGetErrorName(e) + " (" +
                               hipGetErrorString(e) + ")");
}

int use_device(const mx_ctx *ctx) {
  if (!ctx) return fail(MX_E_INVALID, "null context");
  const hipError_t e = hipSetDevice(ctx->device);
  return e == hipSuccess ? MX_OK : hip_fail(e, "hipSetDevice");
}

static inline uint16_t to_bf16(float x) {
  uint32_t u;
  std::memcpy(&u, &x, 4);
  return static_cast<uint16_t>((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

int stage_panel(mx_ctx *ctx, const void *kn_host, int dtype, int64_t K, int64_t N,
                uint16_t **out) {
  if (!kn_host) return fail(MX_E_INVALID, "stage_weight: null host operand");
  if (K <= 0 || N <= 0) return fail(MX_E_INVALID, "stage_weight: zero dimension");
  if (K % 8) {
    return fail(MX_E_INVALID, "stage_weight: K = " + std::to_string(K) +
                                  " is not a multiple of 8 (the GEMM reads K in 16-byte "
                                  "chunks; the reference enforces hidden % 8 == 0 too)");
  }
  if (dtype != MX_F32 && dtype != MX_BF16)
    return fail(MX_E_INVALID, "stage_weight: dtype must be MX_F32 or MX_BF16");
  std::vector<uint16_t> panel(static_cast<size_t>(K) * N);
  for (int64_t k = 0; k < K; ++k)
    for (int64_t n = 0; n < N; ++n) {
      const size_t src = static_cast<size_t>(k) * N + n;
      panel[static_cast<size_t>(n) * K + k] =
          dtype == MX_F32 ? to_bf16(static_cast<const float *>(kn_host)[src])
                          : static_cast<const uint16_t *>(kn_host)[src];
    }
  int rc = use_device(ctx);
  if (rc) return rc;
  void *p = nullptr;
  hipError_t e = dev_malloc((void **)&p, panel.size() * 2);
  if (e != hipSuccess) return hip_fail(e, "stage_weight: hipMalloc");
  e = upload(p, panel.data(), panel.size() * 2);
  if (e != hipSuccess) {
    (void)hipFree(p);
    return hip_fail(e, "stage_weight: upload");
  }
  *out = static_cast<uint16_t *>(p);
  return MX_OK;
}

int check_panel(const std::string &what, int64_t K, int64_t N, int64_t tile_k, int64_t tile_n,
                int64_t mac_s, int64_t mac_t) {
  if (K <= 0 || N <= 0) return fail(MX_E_INVALID, what + ": GEMM operand with a zero dimension");
  if (tile_k <= 0 || tile_n <= 0 || mac_s <= 0 || mac_t <= 0)
    return fail(MX_E_INVALID, what + ": the block_panel layout needs positive tile_k, tile_n, "
                                     "mac_s and mac_t");
  if (K % tile_k || N % tile_n || tile_k % mac_s || tile_n % mac_t)
    return fail(MX_E_INVALID, what + ": layout (" + std::to_string(tile_k) + "," +
                                  std::to_string(tile_n) + ") mac (" + std::to_string(mac_s) +
                                  "," + std::to_string(mac_t) + ") does not tile [" +
                                  std::to_string(K) + "," + std::to_string(N) + "]");
  if ((tile_k + 2) * tile_n * 2 > 65536)
    return fail(MX_E_UNSUPPORTED, what + ": a " + std::to_string(tile_k) + " x " +
                                      std::to_string(tile_n) +
                                      " tile does not fit the untile kernel's 64 KB of LDS");
  if (K % 8)
    return fail(MX_E_INVALID, what + ": K = " + std::to_string(K) +
                                  " is not a multiple of 8 (the GEMM reads K in 16-byte chunks)");
  return MX_OK;
}

int stage_tiled_panel(mx_ctx *ctx, const uint16_t *panel_host, int64_t K, int64_t N,
                      int64_t tile_k, int64_t tile_n, int64_t mac_s, int64_t mac_t,
                      uint16_t **out) {
  if (!panel_host) return fail(MX_E_INVALID, "stage_weight_panel: null panel");
  int rc = check_panel("stage_weight_panel", K, N, tile_k, tile_n, mac_s, mac_t);
  if (rc) return rc;
  rc = use_device(ctx);
  if (rc) return rc;
  const size_t bytes = static_cast<size_t>(K) * N * 2;
  void *tiled = nullptr, *wt = nullptr;
  hipError_t e = dev_malloc((void **)&tiled, bytes);
  if (e != hipSuccess) return hip_fail(e, "stage_weight_panel: hipMalloc");
  e = dev_malloc((void **)&wt, bytes);
  if (e != hipSuccess) {
    (void)hipFree(tiled);
    return hip_fail(e, "stage_weight_panel: hipMalloc");
  }
  {
    SetupStream st;
    e = st.h2d(tiled, panel_host, bytes);
    if (e == hipSuccess)
      e = mxk::untile_panel(static_cast<const uint16_t *>(tiled), K, N, (int)tile_k,
                            (int)tile_n, (int)mac_s, (int)mac_t, static_cast<uint16_t *>(wt),
                            st.s);
    if (e == hipSuccess) e = st.finish();
  }
  (void)hipFree(tiled);
  if (e != hipSuccess) {
    (void)hipFree(wt);
    return hip_fail(e, "stage_weight_panel: untile");
  }
  *out = static_cast<uint16_t *>(wt);
  return MX_OK;
}

static bool aligned(const void *p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

int gemm_checked(mx_stream *s, const uint16_t *A, int64_t M, int64_t K, int64_t lda,
                 const uint16_t *Wt, int64_t N, const float *bias, int epilogue,
                 const float *residual, void *C, int c_dtype, int64_t ldc, const Live &live) {
  if (!s) return fail(MX_E_INVALID, "gemm: null stream");
  if (!A || !Wt || !C) return fail(MX_E_INVALID, "gemm: null A, weight or C");
  if (M <= 0 || N <= 0 || K <= 0) return fail(MX_E_INVALID, "gemm: zero dimension");
  if (M > INT32_MAX / 2 || N > INT32_MAX / 2 || K > INT32_MAX / 2)
    return fail(MX_E_INVALID, "gemm: dimension beyond 2^30");
  if (K % 8 || lda % 8)
    return fail(MX_E_INVALID, "gemm: K (" + std::to_string(K) + ") and lda (" +
                                  std::to_string(lda) + ") must be multiples of 8");
  if (lda < K) return fail(MX_E_INVALID, "gemm: lda < K");
  if (ldc < N) return fail(MX_E_INVALID, "gemm: ldc < N");
  if (!aligned(A, 16) || !aligned(Wt, 16))
    return fail(MX_E_INVALID, "gemm: A and the weight panel must be 16-byte aligned");
  const bool narrow = (epilogue & MX_EPI_NARROW_C) != 0;
  const int act = epilogue & ~MX_EPI_NARROW_C;
  if (act < MX_EPI_NONE || act > MX_EPI_GELU_ERF)
    return fail(MX_E_INVALID, "gemm: unknown epilogue " + std::to_string(epilogue));
  if (c_dtype != MX_F32 && c_dtype != MX_BF16)
    return fail(MX_E_INVALID, "gemm: C dtype must be MX_F32 or MX_BF16");
  if (narrow && (residual || (c_dtype == MX_F32 && act != MX_EPI_NONE)))
    return fail(MX_E_UNSUPPORTED, "gemm: a narrowed C takes no residual, and an fp32 one no "
                                  "activation");
  mxk::GemmArgs a{A, lda, Wt, M, N, K, bias, epilogue, residual, C, c_dtype == MX_BF16 ? 1 : 0,
                  ldc, live.dev, live.hint};
  const hipError_t e = mxk::gemm(a, s->stream);
  if (narrow && e == hipErrorInvalidValue)
    return fail(MX_E_UNSUPPORTED, "gemm: a narrowed C runs on the direct-to-LDS kernel only "
                                  "(K % 32 == 0, K >= 128, N % 4 == 0, a bias, 16-byte aligned "
                                  "operands)");
  return e == hipSuccess ? MX_OK : hip_fail(e, "gemm launch");
}

int attention_checked(mx_stream *s, const uint16_t *qkv, int64_t ld_qkv, int64_t B, int64_t S,
                      int64_t H, int64_t hd, float scale, const float *add_mask,
                      const int32_t *kv_len, uint16_t *ctx, int64_t ld_ctx,
                      const int32_t *seq_start, const int32_t *order, int64_t q_rows) {
  if (!s) return fail(MX_E_INVALID, "attention: null stream");
  if (!qkv || !ctx) return fail(MX_E_INVALID, "attention: null qkv or ctx");
  if (B <= 0 || S <= 0 || H <= 0) return fail(MX_E_INVALID, "attention: zero dimension");
  if (hd != 32 && hd != 64)
    return fail(MX_E_UNSUPPORTED, "attention: head_dim " + std::to_string(hd) +
                                      " (this kernel is built for 32 and 64)");
  if (ld_qkv < 3 * H * hd || ld_qkv % 8)
    return fail(MX_E_INVALID, "attention: qkv row stride " + std::to_string(ld_qkv) +
                                  " cannot hold Q|K|V of " + std::to_string(H * hd) +
                                  " each, or is not a multiple of 8");
  if (ld_qkv >= ((int64_t)1 << 24))
    return fail(MX_E_UNSUPPORTED, "attention: qkv row stride " + std::to_string(ld_qkv) +
                                      " (a 64-key tile is addressed by 32-bit offsets: < 2^24)");
  if (ld_ctx < H * hd || ld_ctx % 4)
    return fail(MX_E_INVALID, "attention: ctx row stride too small or not a multiple of 4");
  if (!aligned(qkv, 16) || !aligned(ctx, 8))
    return fail(MX_E_INVALID, "attention: qkv must be 16-byte and ctx 8-byte aligned");
  if (B * H * ((S + 127) / 128) > INT32_MAX || S > INT32_MAX / 4)
    return fail(MX_E_INVALID, "attention: grid too large");
  if (!std::isfinite(scale)) return fail(MX_E_INVALID, "attention: non-finite scale");
  if (seq_start && !kv_len)
    return fail(MX_E_INVALID, "attention: packed rows need kv_len");
  if (order && !kv_len) return fail(MX_E_INVALID, "attention: a launch order needs kv_len");
  if (q_rows < 0) return fail(MX_E_INVALID, "attention: negative query count");
  mxk::AttnArgs a{qkv, ld_qkv, B,      S,        H,     hd,   scale, add_mask,
                  kv_len, ctx,  ld_ctx, seq_start, order, q_rows};
  const hipError_t e = mxk::attention(a, s->stream);
  return e == hipSuccess ? MX_OK : hip_fail(e, "attention launch");
}

void rope_tables_host(int64_t S, int64_t hd, double theta, const float *inv_freq, float *cos_t,
                      float *sin_t) {
  const int64_t half = hd / 2;
  std::vector<double> inv(static_cast<size_t>(half));
  for (int64_t j = 0; j < half; ++j)
    inv[j] = inv_freq ? static_cast<double>(inv_freq[j])
                      : 1.0 / std::pow(theta, (2.0 * static_cast<double>(j)) /
                                                  static_cast<double>(hd));
  for (int64_t p = 0; p < S; ++p)
    for (int64_t j = 0; j < half; ++j) {
      const double ang = static_cast<double>(p) * inv[j];
      const float c = static_cast<float>(std::cos(ang)), sn = static_cast<float>(std::sin(ang));
      cos_t[p * hd + j] = cos_t[p * hd + half + j] = c;
      sin_t[p * hd + j] = sin_t[p * hd + half + j] = sn;
    }
}

int rope_checked(mx_stream *s, uint16_t *qkv, int64_t ld_qkv, int64_t B, int64_t S, int64_t H,
                 int64_t hd, const float *cos_t, const float *sin_t, int64_t rows,
                 const int32_t *row_pos, const Live &live) {
  if (!s) return fail(MX_E_INVALID, "rope_qkv: null stream");
  if (!qkv || !cos_t || !sin_t) return fail(MX_E_INVALID, "rope_qkv: null qkv or table");
  if (B <= 0 || S <= 0 || H <= 0 || hd <= 0) return fail(MX_E_INVALID, "rope_qkv: zero dimension");
  if (hd % 4)
    return fail(MX_E_UNSUPPORTED, "rope_qkv: head_dim " + std::to_string(hd) +
                                      " (the kernel rotates two pairs at a time: hd % 4 == 0)");
  if (ld_qkv < 2 * H * hd || ld_qkv % 2)
    return fail(MX_E_INVALID, "rope_qkv: row stride cannot hold Q|K or is odd");
  if (!aligned(qkv, 4) || !aligned(cos_t, 8) || !aligned(sin_t, 8))
    return fail(MX_E_INVALID, "rope_qkv: misaligned qkv or table");
  if (B * S > INT32_MAX) return fail(MX_E_INVALID, "rope_qkv: too many rows");
  const hipError_t e = mxk::rope_qkv(qkv, ld_qkv, rows < 0 ? B * S : rows, (int)S, (int)H,
                                     (int)hd, cos_t, sin_t, s->stream, row_pos, live.dev);
  return e == hipSuccess ? MX_OK : hip_fail(e, "rope_qkv launch");
}

int glu_checked(mx_stream *s, const void *up, int up_dtype, void *out, int out_dtype,
                int64_t rows, int64_t f, int act, const Live &live) {
  if (!s) return fail(MX_E_INVALID, "glu: null stream");
  if (!up || !out) return fail(MX_E_INVALID, "glu: null up or out");
  if (rows <= 0 || f <= 0) return fail(MX_E_INVALID, "glu: zero dimension");
  if (f % 4) return fail(MX_E_UNSUPPORTED, "glu: f % 4 != 0");
  if ((up_dtype != MX_F32 && up_dtype != MX_BF16) || (out_dtype != MX_F32 && out_dtype != MX_BF16))
    return fail(MX_E_INVALID, "glu: dtypes must be MX_F32 or MX_BF16");
  if (act != MX_GATED_SILU && act != MX_GATED_GELU_ERF)
    return fail(MX_E_INVALID, "glu: act must be MX_GATED_SILU or MX_GATED_GELU_ERF");
  if (!aligned(up, up_dtype == MX_F32 ? 16 : 8) || !aligned(out, out_dtype == MX_F32 ? 16 : 8))
    return fail(MX_E_INVALID, "glu: misaligned up or out");
  const hipError_t e = mxk::glu(up, up_dtype == MX_BF16, out, out_dtype == MX_BF16, rows, f, act,
                                s->stream, live.dev);
  return e == hipSuccess ? MX_OK : hip_fail(e, "glu launch");
}

int take_data_error(mx_stream *s, int *flags) {
  int h[2] = {0, 0};
  hipError_t e = hipMemcpyAsync(h, s->err_dev, sizeof(h), hipMemcpyDeviceToHost, s->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(s->stream);
  if (e != hipSuccess) return hip_fail(e, "reading the refusal flag");
  *flags = h[0];
  if (h[1] > 0) s->last_rows = h[1];
  if (h[0]) {
    e = hipMemsetAsync(s->err_dev, 0, sizeof(int), s->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(s->stream);
    if (e != hipSuccess) return hip_fail(e, "clearing the refusal flag");
  }
  return MX_OK;
}

}  // namespace mx

using namespace mx;

extern "C" {

int mx_create(int device, mx_ctx **out) {
  clear_error();
  if (!out) return fail(MX_E_INVALID, "mx_create: null out");
  *out = nullptr;
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess) return hip_fail(e, "hipGetDeviceCount");
  if (device < 0 || device >= n)
    return fail(MX_E_INVALID, "mx_create: device " + std::to_string(device) + " of " +
                                  std::to_string(n) + " visible");
  hipDeviceProp_t p;
  e = hipGetDeviceProperties(&p, device);
  if (e != hipSuccess) return hip_fail(e, "hipGetDeviceProperties");
  if (std::strncmp(p.gcnArchName, "gfx950", 6) != 0)
    return fail(MX_E_UNSUPPORTED, std::string("mx_create: device is ") + p.gcnArchName +
                                      "; this backend is built for gfx950 (MI355X) only");
  // The static scratch's address on this device (mx_encoder_embed_static),
  // looked up once with the device current; the caller's current device is
  // restored.
  int prev = 0;
  e = hipGetDevice(&prev);
  if (e == hipSuccess) e = hipSetDevice(device);
  if (e != hipSuccess) return hip_fail(e, "mx_create: hipSetDevice");
  const int rc = static_scratch_init(device);
  e = hipSetDevice(prev);
  if (rc) return rc;
  if (e != hipSuccess) return hip_fail(e, "mx_create: restoring the current device");
  auto *c = new mx_ctx();
  c->device = device;
  c->props.device = device;
  c->props.compute_units = p.multiProcessorCount;
  c->props.clock_mhz = p.clockRate / 1000;
  c->props.hbm_bytes = static_cast<int64_t>(p.totalGlobalMem);
  std::snprintf(c->props.arch, sizeof c->props.arch, "%s", p.gcnArchName);
  c->props.bf16_dense_tflops =
      static_cast<double>(p.multiProcessorCount) * 4096.0 * (p.clockRate * 1e3) / 1e12;
  *out = c;
  return MX_OK;
}

void mx_destroy(mx_ctx *ctx) {
  if (!ctx) return;
  if (use_device(ctx) == MX_OK)
    for (auto &w : ctx->slots) {
      if (w.wt) (void)hipFree(w.wt);
      I8Operand op{w.wq, w.wscale, w.ias};
      free_i8(op);
    }
  delete ctx;
}

int mx_device_props_get(mx_ctx *ctx, mx_device_props *out) {
  if (!ctx || !out) return fail(MX_E_INVALID, "mx_device_props_get: null argument");
  *out = ctx->props;
  return MX_OK;
}

int mx_stream_create(mx_ctx *ctx, mx_stream **out) {
  clear_error();
  if (!out) return fail(MX_E_INVALID, "mx_stream_create: null out");
  *out = nullptr;
  int rc = use_device(ctx);
  if (rc) return rc;
  auto *s = new mx_stream();
  s->ctx = ctx;
  hipError_t e = hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    delete s;
    return hip_fail(e, "hipStreamCreate");
  }
  e = dev_malloc((void **)&s->err_dev, 2 * sizeof(int));
  if (e == hipSuccess) e = hipMemsetAsync(s->err_dev, 0, 2 * sizeof(int), s->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(s->stream);
  if (e != hipSuccess) {
    (void)hipStreamDestroy(s->stream);
    delete s;
    return hip_fail(e, "stream refusal flag");
  }
  *out = s;
  return MX_OK;
}

void mx_stream_destroy(mx_stream *s) {
  if (!s) return;
  if (use_device(s->ctx) == MX_OK) {
    (void)hipStreamSynchronize(s->stream);
    (void)hipFree(s->err_dev);
    (void)hipStreamDestroy(s->stream);
  }
  delete s;
}

int mx_sync(mx_stream *s) {
  clear_error();
  if (!s) return fail(MX_E_INVALID, "mx_sync: null stream");
  // The refusals of asynchronous calls (mx_encoder_embed_async) wait in the
  // stream's flag until here.
  int flags = 0;
  const int rc = take_data_error(s, &flags);
  if (rc) return rc;
  if (flags & 1)
    return fail(MX_E_DATA, "mx_sync: an asynchronous embed on this stream met a token id "
                           "outside the vocabulary (its row was embedded as zeros)");
  if (flags & 2)
    return fail(MX_E_DATA, "mx_sync: an asynchronous embed on this stream CLS-pooled a "
                           "sequence whose first token is masked");
  return MX_OK;
}

void *mx_stream_handle(mx_stream *s) { return s ? static_cast<void *>(s->stream) : nullptr; }

int mx_alloc(mx_ctx *ctx, size_t bytes, void **dev) {
  if (!dev) return fail(MX_E_INVALID, "mx_alloc: null out");
  int rc = use_device(ctx);
  if (rc) return rc;
  const hipError_t e = dev_malloc(dev, bytes ? bytes : 1);
  return e == hipSuccess ? MX_OK : hip_fail(e, "hipMalloc");
}

int mx_free(mx_ctx *ctx, void *dev) {
  int rc = use_device(ctx);
  if (rc) return rc;
  const hipError_t e = hipFree(dev);
  return e == hipSuccess ? MX_OK : hip_fail(e, "hipFree");
}

int mx_copy_h2d(mx_stream *s, void *dst, const void *src, size_t bytes) {
  if (!s || (!dst && bytes) || (!src && bytes)) return fail(MX_E_INVALID, "mx_copy_h2d: null");
  const hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, s->stream);
  return e == hipSuccess ? MX_OK : hip_fail(e, "hipMemcpyAsync H2D");
}

int mx_copy_d2h(mx_stream *s, void *dst, const void *src, size_t bytes) {
  if (!s || (!dst && bytes) || (!src && bytes)) return fail(MX_E_INVALID, "mx_copy_d2h: null");
  const hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, s->stream);
  return e == hipSuccess ? MX_OK : hip_fail(e, "hipMemcpyAsync D2H");
}

int mx_stage_weight(mx_ctx *ctx, const void *kn_host, int dtype, int64_t K, int64_t N,
                    int *slot) {
  clear_error();
  if (!ctx || !slot) return fail(MX_E_INVALID, "mx_stage_weight: null argument");
  uint16_t *p = nullptr;
  const int rc = stage_panel(ctx, kn_host, dtype, K, N, &p);
  if (rc) return rc;
  std::lock_guard<std::mutex> lk(ctx->mu);
  ctx->slots.push_back(WeightSlot{p, K, N});
  *slot = static_cast<int>(ctx->slots.size());
  return MX_OK;
}

int mx_stage_weight_panel(mx_ctx *ctx, const uint16_t *panel_host, int64_t K, int64_t N,
                          int64_t tile_k, int64_t tile_n, int64_t mac_s, int64_t mac_t,
                          int *slot) {
  clear_error();
  if (!ctx || !slot) return fail(MX_E_INVALID, "mx_stage_weight_panel: null argument");
  uint16_t *p = nullptr;
  const int rc = stage_tiled_panel(ctx, panel_host, K, N, tile_k, tile_n, mac_s, mac_t, &p);
  if (rc) return rc;
  std::lock_guard<std::mutex> lk(ctx->mu);
  ctx->slots.push_back(WeightSlot{p, K, N});
  *slot = static_cast<int>(ctx->slots.size());
  return MX_OK;
}

int mx_release_weight(mx_ctx *ctx, int slot) {
  if (!ctx) return fail(MX_E_INVALID, "mx_release_weight: null context");
  std::lock_guard<std::mutex> lk(ctx->mu);
  if (slot < 1 || slot > static_cast<int>(ctx->slots.size()) ||
      (!ctx->slots[slot - 1].wt && !ctx->slots[slot - 1].wq))
    return fail(MX_E_INVALID, "mx_release_weight: no weight in slot " + std::to_string(slot));
  int rc = use_device(ctx);
  if (rc) return rc;
  WeightSlot &w = ctx->slots[slot - 1];
  if (w.wt) (void)hipFree(w.wt);
  I8Operand op{w.wq, w.wscale, w.ias};
  free_i8(op);
  w = WeightSlot{};
  return MX_OK;
}

int mx_gemm(mx_stream *s, const uint16_t *A, int64_t M, int64_t K, int64_t lda, int wslot,
            const float *bias, int epilogue, const float *residual, void *C, int c_dtype,
            int64_t ldc) {
  clear_error();
  if (!s) return fail(MX_E_INVALID, "gemm: null stream");
  WeightSlot w;
  {
    std::lock_guard<std::mutex> lk(s->ctx->mu);
    if (wslot < 1 || wslot > static_cast<int>(s->ctx->slots.size()) ||
        (!s->ctx->slots[wslot - 1].wt && !s->ctx->slots[wslot - 1].wq))
      return fail(MX_E_INVALID, "gemm: no weight staged in slot " + std::to_string(wslot));
    w = s->ctx->slots[wslot - 1];
    if (!w.wt)
      return fail(MX_E_INVALID, "gemm: slot " + std::to_string(wslot) +
                                    " holds an int8 operand; it is multiplied by mx_gemm_i8");
  }
  if (w.K != K)
    return fail(MX_E_INVALID, "gemm: A has K = " + std::to_string(K) + " but slot " +
                                  std::to_string(wslot) + " holds a [" + std::to_string(w.K) +
                                  ", " + std::to_string(w.N) + "] operand");
  return gemm_checked(s, A, M, K, lda, w.wt, w.N, bias, epilogue, residual, C, c_dtype, ldc);
}

int mx_gemm_wt(mx_stream *s, const uint16_t *A, int64_t M, int64_t K, int64_t lda,
               const uint16_t *Wt, int64_t N, const float *bias, int epilogue,
               const float *residual, void *C, int c_dtype, int64_t ldc) {
  clear_error();
  return gemm_checked(s, A, M, K, lda, Wt, N, bias, epilogue, residual, C, c_dtype, ldc);
}

const char *mx_gemm_plan(int64_t M, int64_t N, int64_t K) {
  return mxk::gemm_config_name(M, N, K);
}

const char *mx_gemm_plan_for(int64_t M, int64_t N, int64_t K, int c_dtype, int residual,
                             int int8) {
  return mxk::gemm_plan_name(M, N, K, c_dtype == MX_BF16, residual != 0, int8 != 0);
}

int mx_attention(mx_stream *s, const uint16_t *qkv, int64_t ld_qkv, int64_t B, int64_t S,
                 int64_t H, int64_t hd, float scale, const float *add_mask,
                 const int32_t *kv_len, uint16_t *ctx, int64_t ld_ctx) {
  clear_error();
  return attention_checked(s, qkv, ld_qkv, B, S, H, hd, scale, add_mask, kv_len, ctx, ld_ctx);
}

int mx_softmax_rows(mx_stream *s, void *x, int dtype, int64_t rows, int64_t cols,
                    int64_t row_stride, const float *add_mask, int64_t rows_per_mask_row,
                    int variant) {
  clear_error();
  if (!s || !x) return fail(MX_E_INVALID, "softmax: null stream or tensor");
  if (rows <= 0 || cols <= 0) return fail(MX_E_INVALID, "softmax: zero dimension");
  if (cols > 4096)
    return fail(MX_E_UNSUPPORTED, "softmax: rows of " + std::to_string(cols) +
                                      " (this kernel holds a row in one wave, <= 4096)");
  if (row_stride < cols) return fail(MX_E_INVALID, "softmax: row stride narrower than a row");
  if (dtype != MX_F32 && dtype != MX_BF16)
    return fail(MX_E_INVALID, "softmax: dtype must be MX_F32 or MX_BF16");
  if (variant < MX_SOFTMAX_POLY || variant > MX_SOFTMAX_AIE)
    return fail(MX_E_INVALID, "softmax: unknown variant " + std::to_string(variant));
  if (variant == MX_SOFTMAX_AIE && dtype != MX_BF16)
    return fail(MX_E_INVALID, "softmax: the AIE variant is bf16 in and out");
  if (variant == MX_SOFTMAX_AIE && add_mask)
    return fail(MX_E_INVALID,
                "softmax: the AIE variant takes scores with the mask already added "
                "(add_additive_mask runs before it, in fp32)");
  if (add_mask && rows_per_mask_row <= 0)
    return fail(MX_E_INVALID, "softmax: rows_per_mask_row must be positive with a mask");
  const hipError_t e =
      mxk::softmax_rows(x, dtype == MX_BF16, rows, cols, row_stride, add_mask,
                        rows_per_mask_row > 0 ? rows_per_mask_row : 1, variant, s->stream);
  return e == hipSuccess ? MX_OK : hip_fail(e, "softmax launch");
}

int mx_layernorm(mx_stream *s, const void *x, int x_dtype, const void *y, int y_dtype,
                 const float *gamma, const float *beta, float eps, int64_t rows, int64_t cols,
                 float *out_f32, uint16_t *out_bf16) {
  clear_error();
  if (!s || !x || !gamma || !beta) return fail(MX_E_INVALID, "layernorm: null argument");
  if (!out_f32 && !out_bf16) return fail(MX_E_INVALID, "layernorm: no output given");
  if (rows <= 0 || cols <= 0) return fail(MX_E_INVALID, "layernorm: zero dimension");
  if (rows > INT32_MAX) return fail(MX_E_INVALID, "layernorm: more than 2^31 rows");
  if ((x_dtype != MX_F32 && x_dtype != MX_BF16) || (y && y_dtype != MX_F32 && y_dtype != MX_BF16))
    return fail(MX_E_INVALID, "layernorm: dtypes must be MX_F32 or MX_BF16");
  if (!(eps >= 0.0f) || !std::isfinite(eps)) return fail(MX_E_INVALID, "layernorm: bad eps");
  if (out_f32 && static_cast<const void *>(out_f32) == x && x_dtype != MX_F32)
    return fail(MX_E_INVALID, "layernorm: out_f32 aliases a bf16 input");
  const hipError_t e = mxk::layernorm(x, x_dtype == MX_BF16, y, y_dtype == MX_BF16, gamma, beta,
                                      eps, rows, cols, out_f32, out_bf16, s->stream);
  return e == hipSuccess ? MX_OK : hip_fail(e, "layernorm launch");
}

int mx_layernorm_aie(mx_stream *s, const uint16_t *x, const float *gamma, const float *beta,
                     float eps, int64_t rows, int64_t cols, uint16_t *out) {
  clear_error();
  if (!s || !x || !gamma || !beta || !out)
    return fail(MX_E_INVALID, "layernorm_aie: null argument");
  if (rows <= 0 || cols <= 0) return fail(MX_E_INVALID, "layernorm_aie: zero dimension");
  // one 64-lane workgroup per 4 rows: at most 2^26 workgroups
  if (rows > ((int64_t)1 << 28)) return fail(MX_E_INVALID, "layernorm_aie: more than 2^28 rows");
  if (cols % 16 || cols > 4096)
    return fail(MX_E_UNSUPPORTED, "layernorm_aie: cols " + std::to_string(cols) +
                                      " is not a multiple of 16 up to 4096 (the kernel's "
                                      "16-lane vectors)");
  if (!(eps >= 0.0f) || !std::isfinite(eps)) return fail(MX_E_INVALID, "layernorm_aie: bad eps");
  if (!aligned(x, 16) || !aligned(out, 16) || !aligned(gamma, 16) || !aligned(beta, 16))
    return fail(MX_E_INVALID, "layernorm_aie: x, out, gamma and beta must be 16-byte aligned");
  const hipError_t e = mxk::layernorm_aie(x, gamma, beta, eps, rows, cols, out, s->stream);
  return e == hipSuccess ? MX_OK : hip_fail(e, "layernorm_aie launch");
}

int mx_gelu(mx_stream *s, const void *x, int x_dtype, void *y, int y_dtype, int64_t n,
            int variant) {
  clear_error();
  if (!s || !x || !y) return fail(MX_E_INVALID, "gelu: null argument");
  if (n <= 0) return fail(MX_E_INVALID, "gelu: empty tensor");
  if ((x_dtype != MX_F32 && x_dtype != MX_BF16) || (y_dtype != MX_F32 && y_dtype != MX_BF16))
    return fail(MX_E_INVALID, "gelu: dtypes must be MX_F32 or MX_BF16");
  if (x == y && x_dtype != y_dtype)
    return fail(MX_E_INVALID, "gelu: in place needs equal dtypes");
  if (variant < MX_GELU_POLY || variant > MX_GELU_ERF_AS)
    return fail(MX_E_INVALID, "gelu: unknown variant " + std::to_string(variant));
  const hipError_t e =
      mxk::gelu(x, x_dtype == MX_BF16, y, y_dtype == MX_BF16, n, variant, s->stream);
  return e == hipSuccess ? MX_OK : hip_fail(e, "gelu launch");
}

int mx_narrow_f32_bf16(mx_stream *s, const float *in, uint16_t *out, int64_t n) {
  clear_error();
  if (!s || !in || !out) return fail(MX_E_INVALID, "narrow_f32_bf16: null argument");
  if (n < 0) return fail(MX_E_INVALID, "narrow_f32_bf16: negative count");
  if (n == 0) return MX_OK;
  const hipError_t e = mxk::narrow_f32_bf16(in, out, n, s->stream);
  return e == hipSuccess ? MX_OK : hip_fail(e, "narrow_f32_bf16 launch");
}

int mx_narrow_i32_bf16(mx_stream *s, const int32_t *in, uint16_t *out, int64_t n) {
  clear_error();
  if (!s || !in || !out) return fail(MX_E_INVALID, "narrow_i32_bf16: null argument");
  if (n < 0) return fail(MX_E_INVALID, "narrow_i32_bf16: negative count");
  if (n == 0) return MX_OK;
  const hipError_t e = mxk::narrow_i32_bf16(in, out, n, s->stream);
  return e == hipSuccess ? MX_OK : hip_fail(e, "narrow_i32_bf16 launch");
}

int mx_rope_tables(int64_t S, int64_t hd, double theta, const float *inv_freq, float *cos_t,
                   float *sin_t) {
  clear_error();
  if (!cos_t || !sin_t) return fail(MX_E_INVALID, "rope_tables: null table");
  if (S <= 0 || hd <= 0 || hd % 2)
    return fail(MX_E_INVALID, "rope_tables: S > 0 and an even head_dim wanted");
  if (!inv_freq && !(theta > 0.0))
    return fail(MX_E_INVALID, "rope_tables: a non-positive rope_theta and no inv_freq");
  rope_tables_host(S, hd, theta, inv_freq, cos_t, sin_t);
  return MX_OK;
}

int mx_rope_qkv(mx_stream *s, uint16_t *qkv, int64_t ld_qkv, int64_t B, int64_t S, int64_t H,
                int64_t hd, const float *cos_t, const float *sin_t) {
  clear_error();
  return rope_checked(s, qkv, ld_qkv, B, S, H, hd, cos_t, sin_t);
}

int mx_glu(mx_stream *s, const void *up, int up_dtype, void *out, int out_dtype, int64_t rows,
           int64_t f, int act) {
  clear_error();
  return glu_checked(s, up, up_dtype, out, out_dtype, rows, f, act);
}

int mx_embed_sum(mx_stream *s, const int32_t *ids, const float *attn_mask, int64_t B, int64_t S,
                 int64_t hidden, const float *word, int64_t vocab, const float *pos,
                 const float *type0, float *emb, float *add_mask, int32_t *kv_len) {
  clear_error();
  if (!s || !ids || !attn_mask || !word || !pos || !type0 || !emb)
    return fail(MX_E_INVALID, "embed_sum: null argument");
  if (B <= 0 || S <= 0 || hidden <= 0 || vocab <= 0)
    return fail(MX_E_INVALID, "embed_sum: zero dimension");
  hipError_t e = mxk::embed_sum(ids, B, S, hidden, word, vocab, pos, type0, emb, s->err_dev,
                                s->stream);
  if (e == hipSuccess && (add_mask || kv_len))
    e = mxk::mask_build(attn_mask, B, S, add_mask, kv_len, s->stream);
  if (e != hipSuccess) return hip_fail(e, "embed_sum launch");
  int flags = 0;
  const int rc = take_data_error(s, &flags);
  if (rc) return rc;
  if (flags & 1)
    return fail(MX_E_DATA, "embed_sum: a token id is outside [0, " + std::to_string(vocab) +
                               ") (its row was written as zeros)");
  return MX_OK;
}

int mx_pool_rows(mx_stream *s, const float *h, const float *attn_mask, int64_t B, int64_t S,
                 int64_t hidden, int cls_pool, int l2_normalize, float *out) {
  clear_error();
  if (!s || !h || !attn_mask || !out) return fail(MX_E_INVALID, "pool_rows: null argument");
  if (B <= 0 || S <= 0 || hidden <= 0) return fail(MX_E_INVALID, "pool_rows: zero dimension");
  if (hidden > 4096) return fail(MX_E_UNSUPPORTED, "pool_rows: hidden > 4096");
  const hipError_t e =
      mxk::pool_rows(h, attn_mask, B, S, hidden, cls_pool, l2_normalize, out, s->err_dev,
                     s->stream);
  if (e != hipSuccess) return hip_fail(e, "pool_rows launch");
  int flags = 0;
  const int rc = take_data_error(s, &flags);
  if (rc) return rc;
  if (flags & 2)
    return fail(MX_E_DATA, "CLS pooling on a sequence whose first token is masked");
  return MX_OK;
}

}  // extern "C"
