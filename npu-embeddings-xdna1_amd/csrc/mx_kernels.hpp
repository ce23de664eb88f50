// mx_kernels.hpp -- host-side launchers of the gfx950 kernels. Shapes and
// pointers are validated by the C ABI layer before any of these is called;
// each launcher only picks a kernel variant and a grid.
//
// rows_dev (nullable) on the row-wise launchers: the live row count, an int on
// the device that an earlier kernel of the stream wrote (token packing's
// packed total); the grid covers `rows`, the bound the buffers hold, and the
// kernels skip the rows at or past the live count.
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
                     uint16_t *out_bf16, hipStream_t s, const int32_t *rows_dev = nullptr);
// The accelerator LayerNorm (kernels/layernorm.cc:85-142, conv_even): bf16
// [rows, cols] in and out (out may alias x), cols % 16 == 0, cols <= 4096,
// 16-byte aligned x, out, gamma and beta.
hipError_t layernorm_aie(const uint16_t *x, const float *gamma, const float *beta, float eps,
                         int64_t rows, int64_t cols, uint16_t *out, hipStream_t s);
hipError_t softmax_rows(void *x, int bf, int64_t rows, int64_t cols, int64_t stride,
                        const float *mask, int64_t rows_per_mask_row, int variant,
                        hipStream_t s);
hipError_t embed_sum(const int32_t *ids, int64_t B, int64_t S, int64_t d, const float *word,
                     int64_t vocab, const float *pos, const float *type0, float *emb, int *err,
                     hipStream_t s);
hipError_t mask_build(const float *attn_mask, int64_t B, int64_t S, float *add_mask,
                      int32_t *kv_len, hipStream_t s);
// seq_start (nullable): the packed layout of the rows (pack_plan). compact
// (CLS pooling only): h holds just each sequence's first row, row b.
hipError_t pool_rows(const float *h, const float *attn_mask, int64_t B, int64_t S, int64_t d,
                     int cls, int l2, float *out, int *err, hipStream_t s,
                     const int32_t *seq_start = nullptr, bool compact = false);
// Each sequence's first row (seq_start[b], or b * S) of x fp32 and ctx bf16
// ([*, d], d % 4 == 0) into row b of xc and ctxc.
hipError_t gather_cls(const float *x, const uint16_t *ctx, const int32_t *seq_start, int64_t B,
                      int64_t S, int64_t d, float *xc, uint16_t *ctxc, hipStream_t s);
// Token packing: seq_start[0..B] = exclusive scan of kv_len (seq_start[B] =
// packed rows) and, when order is non-null, order[0..B) = the sequence
// indices by decreasing kv_len (attention's launch order); the embedding sum
// of the rows s < kv_len[b] into packed row seq_start[b] + s, with
// row_pos[packed row] = s. total_out (nullable): a second copy of seq_start[B].
hipError_t pack_plan(const int32_t *kv_len, int64_t B, int32_t *seq_start, int32_t *order,
                     hipStream_t s, int32_t *total_out = nullptr);
hipError_t embed_sum_packed(const int32_t *ids, int64_t B, int64_t S, int64_t d,
                            const float *word, int64_t vocab, const float *pos,
                            const float *type0, const int32_t *kv_len, const int32_t *seq_start,
                            float *emb, int32_t *row_pos, int *err, hipStream_t s);

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
  // rows_dev (nullable): the live row count on the device (<= M, which is then
  // the bound the buffers hold); m_hint (> 0): the row count the tile is
  // chosen for instead of M -- every tile runs the same MFMA chain over K for
  // each element, so the choice moves the time only, never a bit of C.
  const int32_t *rows_dev = nullptr;
  int64_t m_hint = 0;
};
hipError_t gemm(const GemmArgs &a, hipStream_t s);

// Internal epilogues beyond mx_epilogue (bf16 C, no residual, on both
// datapaths): the gated FFN fused into FFN-up. The GEMM's N = 2f rows of Wt
// (and the bias, wscale) come in glu_interleave's order -- groups of 16, the
// first 8 from the lo half, the next 8 the matching rows of the hi half -- and
// C is [M, f] = lo * act(hi), each product of the two bf16-rounded GEMM
// outputs, as the GEMM followed by glu() computes it. f % 32 == 0.
constexpr int EPI_GLU_SILU = 8, EPI_GLU_GELU = 9;
// An epilogue flag on both datapaths (MX_EPI_NARROW_C): the accumulator is
// rounded to bf16 before the bias or the dequantisation, as the array designs
// that narrow C on the core compute (no residual; the LDS-pipelined kernel).
constexpr int EPI_NARROW_C = 32;
// Wt [2f, row_bytes] (or a [2f] vector, row_bytes 4) -> the interleaved row
// order above. row_bytes % 4 == 0.
hipError_t glu_interleave(const void *src, void *dst, int64_t f, int64_t row_bytes,
                          hipStream_t s);

// The LDS-pipelined kernel's tile for an M x N product (0: 256x256, 1: 256x192,
// 2: 128x256, 3: 128x128; deep: the 256 x 256 tile would run on 128-byte
// slabs) and the resident blocks of a persistent launch.
int gemm_lds_tile(int64_t M, int64_t N, bool deep);
// The row count a launch's tile is chosen for: the hint when one is given
// (and below M), else M.
inline int64_t gemm_pick_rows(int64_t M, int64_t hint) { return hint > 0 && hint < M ? hint : M; }
int cu_count();
// Blocks of a persistent launch over ntiles tiles with `grid` resident: at
// most one per tile, rounded up to a whole number per XCD (a multiple of 8)
// so the kernel's XCD-chunked tile order applies even when the tiles do not
// fill the chip -- consecutive tiles share an A row-panel in one XCD's L2
// instead of landing on eight different L2s. Surplus blocks exit at once.
inline int persistent_grid(int ntiles, int grid) {
  int g = ntiles < grid ? ntiles : grid;
  if (g >= 16 && (g & 7)) g = (g + 7) & ~7;
  return g;
}
// The fewest blocks (a multiple of 8, at most `grid`) that walk `ntiles` tiles
// in as many rounds as `grid` blocks would: ceil(ntiles / rounds). The
// makespan in tiles is the same. The persistent kernels apply it on the device
// to the live tile count (the packed row count is known only there): at the
// packed bge-base rows the QKV (621 tiles), FFN-up (828) and N = 768 (207)
// GEMMs run on 208 of the 256 launched blocks, the rest exit at once, and one
// lane's step is 1.5 % faster with the same bits (each tile's arithmetic does
// not depend on the block that runs it). tests/cpu_checks/balanced_grid.cpp
// checks the rounds, the XCD multiple and the minimality for every tile count
// up to 20,000.
__host__ __device__ inline int balanced_grid(int ntiles, int grid) {
  if (ntiles <= 0 || grid <= 0) return grid;
  const int rounds = (ntiles + grid - 1) / grid;
  int g = (ntiles + rounds - 1) / rounds;
  if (g >= 16 && (g & 7)) g = (g + 7) & ~7;
  return g < grid ? g : grid;
}
// The LDS-pipelined kernel addresses a lane's operand row within a tile as a
// 32-bit byte offset from the tile origin: row r (< 256) of A at r * lda * esz
// and of Wt at r * K * esz, plus at most 128 bytes of K. Both must stay below
// 2^32, i.e. lda * esz and K * esz below 2^24.
inline bool lds_offsets_fit(int64_t lda, int64_t K, int esz) {
  const int64_t lim = (int64_t)1 << 24;
  return lda * esz < lim && K * esz < lim;
}

// int8 W8A8 (k_gemm_i8.hip): C[M,N] = epi(fma(float(Aq @ Wq^T) * a_scale[m],
// wscale[n], bias[n])) (+ residual), or the raw int32 product (c_dtype 2).
// Requires K % 64 == 0, K >= 256, N % 4 == 0, lda % 16 == 0, 16-byte aligned
// operands and vectors.
struct GemmI8Args {
  const int8_t *A;
  int64_t lda;
  const int8_t *Wt;  // [N, K], row stride K
  int64_t M, N, K;
  const float *a_scale;  // [M]
  const float *wscale;   // [N]
  const float *bias;     // [N] or null
  int epilogue;          // mx_epilogue
  const float *residual; // fp32, row stride ldc, or null
  void *C;
  int c_dtype;  // 0 fp32, 1 bf16, 2 int32 (raw accumulators)
  int64_t ldc;
  const int32_t *rows_dev = nullptr;  // as GemmArgs
  int64_t m_hint = 0;
};
hipError_t gemm_i8(const GemmI8Args &a, hipStream_t s);
// Whether the 256 x 256 tile runs on 128-byte slabs for this call.
bool gemm_i8_deep(const GemmI8Args &a);

// quantise_a_int8 over rows of K (k_quant.hip): a fp32 or bf16 (row stride
// lda), ias [K] -> q int8 (row stride ldq) and a_scale [rows]. K % 4 == 0,
// K <= 8192.
hipError_t quantise_rows(const void *a, int a_bf, int64_t lda, int64_t rows, int64_t K,
                         const float *ias, int8_t *q, int64_t ldq, float *a_scale,
                         hipStream_t s, const int32_t *rows_dev = nullptr);
// add_norm_quant: LayerNorm(x + y) -> out_f32 (nullable) and its quantisation
// with ias -> q, a_scale. cols % 4 == 0, cols <= 4096.
hipError_t layernorm_quant(const float *x, const void *y, int y_bf, const float *gamma,
                           const float *beta, float eps, int64_t rows, int64_t cols,
                           float *out_f32, const float *ias, int8_t *q, float *a_scale,
                           hipStream_t s, const int32_t *rows_dev = nullptr);
int quant_groups(int64_t K);

// The RoPE / gated-FFN archs (k_glu.hip): in-place RoPE of Q and K in bf16
// fused rows (tables [S, hd]); lo | hi -> lo * act(hi) (act 1 SiLU, 2 GELU).
// row_pos (nullable): each row's position (packed rows), else row % S.
hipError_t rope_qkv(uint16_t *qkv, int64_t ld, int64_t rows, int S, int H, int hd,
                    const float *cos_t, const float *sin_t, hipStream_t s,
                    const int32_t *row_pos = nullptr, const int32_t *rows_dev = nullptr);
hipError_t glu(const void *in, int in_bf, void *out, int out_bf, int64_t rows, int64_t f, int act,
               hipStream_t s, const int32_t *rows_dev = nullptr);

// Container operand tiled (tile_k, tile_n) with (mac_s, mac_t) sub-tiles ->
// [N, K] panel (k_panel.hip). Shapes checked by the caller.
hipError_t untile_panel(const uint16_t *panel, int64_t K, int64_t N, int tile_k, int tile_n,
                        int mac_s, int mac_t, uint16_t *wt, hipStream_t s);
hipError_t untile_panel_i8(const int8_t *panel, int64_t K, int64_t N, int tile_k, int tile_n,
                           int mac_s, int mac_t, int8_t *wt, hipStream_t s);
// An I4 container run (K * N / 2 bytes, two values per byte, low nibble
// first) -> the int8 run of the same tiling, each value widened by its
// group's gscale ([ceil(K / group), N] fp32): int4_panel.hpp:183-246.
hipError_t widen_i4_panel(const uint8_t *packed, int64_t K, int64_t N, int tile_k, int tile_n,
                          int mac_s, int mac_t, const float *gscale, int64_t group, int8_t *out,
                          hipStream_t s);
// The plan the launcher would pick (for tests and reports): tile, slab depth
// in K elements, wave tile and ring slots, e.g.
// "lds_256x256x64_w64x128_ns2_persistent". gemm_config_name is the bf16
// datapath's plan for an fp32 C without a residual.
const char *gemm_plan_name(int64_t M, int64_t N, int64_t K, bool c_bf16, bool residual,
                           bool i8);
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
  // Packed rows (nullable): sequence b's rows start at seq_start[b] and only
  // its kv_len[b] rows exist (queries and keys past it are neither read nor
  // written).
  const int32_t *seq_start = nullptr;
  // Launch order (nullable): the B sequence indices, longest kv_len first;
  // the blocks of order[0] are dispatched first.
  const int32_t *order = nullptr;
  // 0: every query; else only the first q_rows queries of each sequence are
  // computed and stored (their keys and values are all of the sequence's).
  int64_t q_rows = 0;
};
hipError_t attention(const AttnArgs &a, hipStream_t s);

}  // namespace mxk
