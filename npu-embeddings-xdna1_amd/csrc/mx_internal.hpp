// mx_internal.hpp -- host-side objects behind the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>
#include <string>
#include <vector>

#include "mx_host.hpp"

namespace mx {

int hip_fail(hipError_t e, const char *what);

// Every device allocation of the library goes through here, so that it is
// counted (mx_device_allocations).
inline hipError_t dev_malloc(void **p, size_t bytes) {
  count_device_allocation();
  return hipMalloc(p, bytes);
}

// One-off set-up work (weight uploads and reshapes, table uploads) runs on a
// stream made for it and destroyed when the work is done. The library never
// uses HIP's null stream: once created it holds one of the process's
// GPU_MAX_HW_QUEUES hardware queues (4 by default) for good, and streams that
// share a hardware queue run one after the other.
struct SetupStream {
  hipStream_t s = nullptr;
  hipError_t e = hipSuccess;
  SetupStream() { e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking); }
  ~SetupStream() {
    if (s) {
      (void)hipStreamSynchronize(s);
      (void)hipStreamDestroy(s);
    }
  }
  SetupStream(const SetupStream &) = delete;
  SetupStream &operator=(const SetupStream &) = delete;
  hipError_t h2d(void *dst, const void *src, size_t bytes) {
    return e != hipSuccess ? e : hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, s);
  }
  // Wait for everything queued on it.
  hipError_t finish() { return e != hipSuccess ? e : hipStreamSynchronize(s); }
};

// A host -> device copy that is complete when it returns (on a set-up stream).
inline hipError_t upload(void *dst, const void *src, size_t bytes) {
  SetupStream st;
  const hipError_t e = st.h2d(dst, src, bytes);
  return e != hipSuccess ? e : st.finish();
}

struct WeightSlot {
  uint16_t *wt = nullptr;  // [N, K] bf16 (a bf16 operand)
  int64_t K = 0, N = 0;
  int8_t *wq = nullptr;     // [N, K] int8 (an int8 operand; wt is then null)
  float *wscale = nullptr;  // int8: per-column scale [N]
  float *ias = nullptr;     // int8: 1 / asmooth [K]
};

}  // namespace mx

struct mx_ctx {
  int device = 0;
  mx_device_props props{};
  std::mutex mu;
  std::vector<mx::WeightSlot> slots;  // index = slot - 1
};

struct mx_stream {
  mx_ctx *ctx = nullptr;
  hipStream_t stream = nullptr;
  // Two device words: [0] the flags of kernels that refuse data, [1] the last
  // packed row total a pass planned on this stream.
  int *err_dev = nullptr;
  // Word 1 as last read with the flags (host): the GEMM tile hint of the next
  // packed pass on this stream.
  int last_rows = 0;
};

namespace mx {

// Make ctx's device current for the calling thread.
int use_device(const mx_ctx *ctx);
// Copy a [K, N] host weight (fp32 values or bf16 bits) into a new [N, K] bf16
// device panel.
int stage_panel(mx_ctx *ctx, const void *kn_host, int dtype, int64_t K, int64_t N,
                uint16_t **out);
// The live rows of a launch whose row count is known on the device only
// (token packing's packed total, left on the device so the host never waits
// for it): dev points at the count (the launch's M is then the bound its
// buffers hold), hint is the row count its GEMM tile is chosen for (every
// tile gives the same bits; the choice moves the time only). Default: M rows.
struct Live {
  const int32_t *dev = nullptr;
  int64_t hint = 0;
};
// Validated launches shared by the per-op entry points and the encoder.
int gemm_checked(mx_stream *s, const uint16_t *A, int64_t M, int64_t K, int64_t lda,
                 const uint16_t *Wt, int64_t N, const float *bias, int epilogue,
                 const float *residual, void *C, int c_dtype, int64_t ldc,
                 const Live &live = Live{});
int attention_checked(mx_stream *s, const uint16_t *qkv, int64_t ld_qkv, int64_t B, int64_t S,
                      int64_t H, int64_t hd, float scale, const float *add_mask,
                      const int32_t *kv_len, uint16_t *ctx, int64_t ld_ctx,
                      const int32_t *seq_start = nullptr, const int32_t *order = nullptr,
                      int64_t q_rows = 0);
// An int8 operand on the device: the [K, N] weight as an [N, K] int8 panel
// (from row-major int8, or untiled from a container's block panel when tile_k
// > 0), wscale [N] copied, ias = 1 / asmooth [K] computed once in fp32.
struct I8Operand {
  int8_t *wq = nullptr;
  float *wscale = nullptr, *ias = nullptr;
};
int stage_i8(mx_ctx *ctx, const int8_t *kn_host, const float *wscale_host,
             const float *asmooth_host, int64_t K, int64_t N, int64_t tile_k, int64_t tile_n,
             int64_t mac_s, int64_t mac_t, I8Operand *out);
void free_i8(I8Operand &op);
// The same from a container's I4 run (K * N / 2 bytes) and its .gscale
// ([ceil(K / group), N], group 0 = K): widened on the GPU to the int8 run of
// the same tiling (gemm_b_panel's I4 branch, int4_panel.hpp:77-246), then
// staged as an I8 operand.
int check_i4(const std::string &what, int64_t K, int64_t N, int64_t group, int64_t tile_k,
             int64_t tile_n, int64_t mac_s, int64_t mac_t);
int stage_i4(mx_ctx *ctx, const uint8_t *packed_host, const float *gscale_host, int64_t group,
             const float *wscale_host, const float *asmooth_host, int64_t K, int64_t N,
             int64_t tile_k, int64_t tile_n, int64_t mac_s, int64_t mac_t, I8Operand *out);
int gemm_i8_checked(mx_stream *s, const int8_t *A, const float *a_scale, int64_t M, int64_t K,
                    int64_t lda, const int8_t *Wt, const float *wscale, int64_t N,
                    const float *bias, int epilogue, const float *residual, void *C,
                    int c_dtype, int64_t ldc, const Live &live = Live{});
int quantise_checked(mx_stream *s, const void *a, int a_dtype, int64_t lda, int64_t rows,
                     int64_t K, const float *ias, int8_t *q, int64_t ldq, float *a_scale,
                     const Live &live = Live{});
int layernorm_i8_checked(mx_stream *s, const float *x, const void *y, int y_dtype,
                         const float *gamma, const float *beta, float eps, int64_t rows,
                         int64_t cols, float *out_f32, const float *ias, int8_t *q,
                         float *a_scale, const Live &live = Live{});
// The RoPE / gated-FFN archs: host tables, and validated launches.
void rope_tables_host(int64_t S, int64_t hd, double theta, const float *inv_freq, float *cos_t,
                      float *sin_t);
// rows / row_pos: packed rows (rows < 0: the dense B*S).
int rope_checked(mx_stream *s, uint16_t *qkv, int64_t ld_qkv, int64_t B, int64_t S, int64_t H,
                 int64_t hd, const float *cos_t, const float *sin_t, int64_t rows = -1,
                 const int32_t *row_pos = nullptr, const Live &live = Live{});
int glu_checked(mx_stream *s, const void *up, int up_dtype, void *out, int out_dtype,
                int64_t rows, int64_t f, int act, const Live &live = Live{});
// Read and clear the stream's data-refusal flag (synchronises the stream);
// word 1, the last packed row total, goes to s->last_rows.
int take_data_error(mx_stream *s, int *flags);
// The static device scratch of mx_encoder_embed_static (mx_static.hip): its
// address on each device is looked up once, by mx_create with that device
// current (static_scratch_init), and handed out by static_scratch.
int static_scratch_init(int device);
int static_scratch(int device, void **ptr);
size_t static_scratch_bytes();

// The context and width of an encoder (for mx_service.cpp).
mx_ctx *encoder_ctx(const mx_encoder *enc);
int64_t encoder_hidden(const mx_encoder *enc);

// Check a block_panel tiling of a [K, N] operand; MX_OK or a refusal naming it.
int check_panel(const std::string &what, int64_t K, int64_t N, int64_t tile_k, int64_t tile_n,
                int64_t mac_s, int64_t mac_t);
// Copy a pre-tiled bf16 [K, N] operand to the GPU and untile it into a new
// [N, K] panel (synchronous).
int stage_tiled_panel(mx_ctx *ctx, const uint16_t *panel_host, int64_t K, int64_t N,
                      int64_t tile_k, int64_t tile_n, int64_t mac_s, int64_t mac_t,
                      uint16_t **out);

}  // namespace mx
