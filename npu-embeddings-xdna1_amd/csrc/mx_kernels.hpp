// mx_kernels.hpp -- host-side launchers of the gfx950 kernels. Shapes and
// pointers are validated by the C ABI layer before any of these is called;
// each launcher only picks a kernel variant and a grid.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mxk {

hipError_t narrow_f32_bf16(const float *in, uint16_t *out, int64_t n, hipStream_t s);
hipError_t narrow_i32_bf16(const int32_t *in, uint16_t *out, int64_t n, hipStream_t s);
hipError_t gelu(const void *x, int x_bf, void *y, int y_bf, int64_t n, int variant,
                hipStream_t s);
hipError_t layernorm(const void *x, int x_bf, const void *y, int y_bf, const float *gamma,
                     const float *beta, float eps, int64_t rows, int64_t cols, float *out_f32,
                     uint16_t *out_bf16, hipStream_t s);
hipError_t softmax_rows(void *x, int bf, int64_t rows, int64_t cols, int64_t stride,
                        const float *mask, int64_t rows_per_mask_row, int variant,
                        hipStream_t s);
hipError_t embed_sum(const int32_t *ids, int64_t B, int64_t S, int64_t d, const float *word,
                     int64_t vocab, const float *pos, const float *type0, float *emb, int *err,
                     hipStream_t s);
hipError_t mask_build(const float *attn_mask, int64_t B, int64_t S, float *add_mask,
                      int32_t *kv_len, hipStream_t s);
hipError_t pool_rows(const float *h, const float *attn_mask, int64_t B, int64_t S, int64_t d,
                     int cls, int l2, float *out, int *err, hipStream_t s);

// Front ends (k_front.hip).
hipError_t vit_patches(const float *px, int64_t B, int img, int p, uint16_t *rows, hipStream_t s);
hipError_t vit_assemble(const float *patch, const float *cls, const float *pos, int64_t B, int np,
                        int d, float *x, hipStream_t s);
hipError_t gather_rows_bf16(const float *x, int64_t stride, int64_t n, int d, uint16_t *out,
                            hipStream_t s);
hipError_t mel_time_major(const float *mel, int64_t B, int mels, int T, uint16_t *out,
                          hipStream_t s);

// C[M,N] = epi(A[M,K] @ Wt[N,K]^T + bias) (+ residual); see k_gemm.hip.
struct GemmArgs {
  const uint16_t *A;
  int64_t lda;
  const uint16_t *Wt;  // [N, K], row stride K
  int64_t M, N, K;
  const float *bias;      // [N] or null
  int epilogue;           // mx_epilogue
  const float *residual;  // fp32, row stride ldc, or null
  void *C;
  int c_bf16;
  int64_t ldc;
};
hipError_t gemm(const GemmArgs &a, hipStream_t s);

// Container operand tiled (tile_k, tile_n) with (mac_s, mac_t) sub-tiles ->
// [N, K] panel (k_panel.hip). Shapes checked by the caller.
hipError_t untile_panel(const uint16_t *panel, int64_t K, int64_t N, int tile_k, int tile_n,
                        int mac_s, int mac_t, uint16_t *wt, hipStream_t s);
// Tile configuration the launcher would pick (for tests and reports).
const char *gemm_config_name(int64_t M, int64_t N, int64_t K);

struct AttnArgs {
  const uint16_t *qkv;
  int64_t ld_qkv;
  int64_t B, S, H, hd;
  float scale;
  const float *add_mask;  // [B, S] or null
  const int32_t *kv_len;  // [B] or null
  uint16_t *ctx;
  int64_t ld_ctx;
};
hipError_t attention(const AttnArgs &a, hipStream_t s);

}  // namespace mxk
