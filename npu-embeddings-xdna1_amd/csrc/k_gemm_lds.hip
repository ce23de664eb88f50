// k_gemm_lds.hip -- the bf16 instantiations of the persistent LDS-pipelined
// GEMM (the kernel body and its design are in k_gemm_lds.hpp): 64-byte slabs
// (32 K) for every tile and epilogue, and the 256 x 256 tile with 128-byte
// slabs (64 K, two slots) for a bf16 C without a residual or an fp32 C with
// one.
#include "k_gemm_lds.hpp"

using namespace mxlds;

namespace {

template <int BM, int BN, int WGM, int WGN, int NS, int EPI, bool RES, bool CBF, int RB>
__global__ __launch_bounds__(WGM *WGN * 64) void gemm_lds_k(
    const uint16_t *__restrict__ A, int64_t lda, const uint16_t *__restrict__ Wt, int M, int N,
    int K, const float *__restrict__ bias, const float *residual, void *C, int64_t ldc,
    int tiles_m, int tiles_n, const int32_t *rows_dev) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  gemm_lds_body<BM, BN, WGM, WGN, NS, EPI, RES, CBF, false, false, RB>(
      A, lda, Wt, M, N, K, bias, residual, C, ldc, tiles_m, tiles_n, nullptr, nullptr, smem,
      rows_dev);
}

}  // namespace

namespace mxk {

template <int BM, int BN, int WGM, int WGN, int NS, int EPI, bool RES, bool CBF, int RB = 64>
hipError_t gemm_lds_launch_t(const GemmArgs &a, int grid, hipStream_t s) {
  using Cfg = LdsCfg<BM, BN, WGM, WGN, NS, false, stg_kind(CBF, RES), RB>;
  auto kern = gemm_lds_k<BM, BN, WGM, WGN, NS, EPI, RES, CBF, RB>;
  static bool attr_set = false;
  if (!attr_set) {
    const hipError_t e = hipFuncSetAttribute(
        (const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, Cfg::LDS);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  const int tiles_m = (int)((a.M + BM - 1) / BM), tiles_n = (int)((a.N + BN - 1) / BN);
  const int ntiles = tiles_m * tiles_n;
  const int g = mxk::persistent_grid(ntiles, grid);
  kern<<<g, Cfg::NT, Cfg::LDS, s>>>((const uint16_t *)a.A, a.lda, (const uint16_t *)a.Wt,
                                    (int)a.M, (int)a.N, (int)a.K, a.bias, a.residual, a.C, a.ldc,
                                    tiles_m, tiles_n, a.rows_dev);
  return hipGetLastError();
}

// One tile configuration, every epilogue variant. `grid` = resident blocks
// (one per CU).
template <int BM, int BN, int WGM, int WGN, int NS>
hipError_t gemm_lds_launch(const GemmArgs &a, int grid, hipStream_t s) {
  if (a.epilogue >= EPI_GLU_SILU) {
    // The fused gated FFN pairs a wave's column blocks: an even number of
    // them, a bf16 C.
    if constexpr ((BN / WGN) % 64 == 0) {
      if (!a.c_bf16 || a.residual) return hipErrorInvalidValue;
      if (a.epilogue == EPI_GLU_SILU)
        return gemm_lds_launch_t<BM, BN, WGM, WGN, NS, EPI_GLU_SILU, false, true>(a, grid, s);
      if (a.epilogue == EPI_GLU_GELU)
        return gemm_lds_launch_t<BM, BN, WGM, WGN, NS, EPI_GLU_GELU, false, true>(a, grid, s);
    }
    return hipErrorInvalidValue;
  }
#define MX_LDS_EPI(E)                                                                        \
  if (a.epilogue == E) {                                                                     \
    if (a.residual)                                                                          \
      return a.c_bf16 ? gemm_lds_launch_t<BM, BN, WGM, WGN, NS, E, true, true>(a, grid, s)   \
                      : gemm_lds_launch_t<BM, BN, WGM, WGN, NS, E, true, false>(a, grid, s); \
    return a.c_bf16 ? gemm_lds_launch_t<BM, BN, WGM, WGN, NS, E, false, true>(a, grid, s)    \
                    : gemm_lds_launch_t<BM, BN, WGM, WGN, NS, E, false, false>(a, grid, s);  \
  }
  MX_LDS_EPI(0)
  MX_LDS_EPI(1)
  MX_LDS_EPI(2)
#undef MX_LDS_EPI
  return hipErrorInvalidValue;
}

// The 256 x 256 tile on 128-byte slabs: a bf16 C without a residual (the
// fused gated FFN included) or an fp32 C with one (their compact staging is
// what leaves LDS room for two 64 KB slots).
hipError_t gemm_lds_deep_launch(const GemmArgs &a, int grid, hipStream_t s) {
  if (a.c_bf16 && !a.residual) {
    switch (a.epilogue) {
      case 0: return gemm_lds_launch_t<256, 256, 4, 2, 2, 0, false, true, 128>(a, grid, s);
      case 1: return gemm_lds_launch_t<256, 256, 4, 2, 2, 1, false, true, 128>(a, grid, s);
      case 2: return gemm_lds_launch_t<256, 256, 4, 2, 2, 2, false, true, 128>(a, grid, s);
      case EPI_GLU_SILU:
        return gemm_lds_launch_t<256, 256, 4, 2, 2, EPI_GLU_SILU, false, true, 128>(a, grid, s);
      case EPI_GLU_GELU:
        return gemm_lds_launch_t<256, 256, 4, 2, 2, EPI_GLU_GELU, false, true, 128>(a, grid, s);
      default: return hipErrorInvalidValue;
    }
  }
  if (!a.c_bf16 && a.residual) {
    switch (a.epilogue) {
      case 0: return gemm_lds_launch_t<256, 256, 4, 2, 2, 0, true, false, 128>(a, grid, s);
      case 1: return gemm_lds_launch_t<256, 256, 4, 2, 2, 1, true, false, 128>(a, grid, s);
      case 2: return gemm_lds_launch_t<256, 256, 4, 2, 2, 2, true, false, 128>(a, grid, s);
      default: return hipErrorInvalidValue;
    }
  }
  return hipErrorInvalidValue;
}

// The 128 x 128 tile on 128-byte slabs (two 32 KB slots: the LDS of the
// 64-byte form's four, half the barriers per K) for a bf16 C without a
// residual.
hipError_t gemm_lds_128_deep_launch(const GemmArgs &a, int grid, hipStream_t s) {
  if (!a.c_bf16 || a.residual) return hipErrorInvalidValue;
  switch (a.epilogue) {
    case 0: return gemm_lds_launch_t<128, 128, 2, 2, 2, 0, false, true, 128>(a, grid, s);
    case 1: return gemm_lds_launch_t<128, 128, 2, 2, 2, 1, false, true, 128>(a, grid, s);
    case 2: return gemm_lds_launch_t<128, 128, 2, 2, 2, 2, false, true, 128>(a, grid, s);
    case EPI_GLU_SILU:
      return gemm_lds_launch_t<128, 128, 2, 2, 2, EPI_GLU_SILU, false, true, 128>(a, grid, s);
    case EPI_GLU_GELU:
      return gemm_lds_launch_t<128, 128, 2, 2, 2, EPI_GLU_GELU, false, true, 128>(a, grid, s);
    default: return hipErrorInvalidValue;
  }
}

// A narrowed C (EPI_NARROW_C; no residual): the 256 x 256 tile on 64-byte
// slabs, or the 128 x 128 tile where the product is too small for it; a bf16
// C with any activation, or an fp32 C without one (the BERT projections and
// the gated FFN's halves, which the host adds the bias to in fp32).
hipError_t gemm_lds_nc_launch(const GemmArgs &a, int grid, hipStream_t s) {
  if (a.residual) return hipErrorInvalidValue;
  const int e = a.epilogue & ~EPI_NARROW_C;
  constexpr int NC = EPI_NARROW_C;
#define MX_LDS_NC(BM, BN, WGM, WGN, NS)                                                   \
  if (a.c_bf16) {                                                                         \
    switch (e) {                                                                          \
      case 0: return gemm_lds_launch_t<BM, BN, WGM, WGN, NS, NC, false, true>(a, grid, s); \
      case 1:                                                                             \
        return gemm_lds_launch_t<BM, BN, WGM, WGN, NS, NC | 1, false, true>(a, grid, s);   \
      case 2:                                                                             \
        return gemm_lds_launch_t<BM, BN, WGM, WGN, NS, NC | 2, false, true>(a, grid, s);   \
      default: return hipErrorInvalidValue;                                               \
    }                                                                                     \
  }                                                                                       \
  if (e == 0) return gemm_lds_launch_t<BM, BN, WGM, WGN, NS, NC, false, false>(a, grid, s); \
  return hipErrorInvalidValue;
  if (gemm_lds_tile(gemm_pick_rows(a.M, a.m_hint), a.N, false) == 0) {
    MX_LDS_NC(256, 256, 2, 4, 3)
  }
  MX_LDS_NC(128, 128, 2, 2, 4)
#undef MX_LDS_NC
}

template hipError_t gemm_lds_launch<256, 256, 2, 4, 3>(const GemmArgs &, int, hipStream_t);
template hipError_t gemm_lds_launch<128, 256, 2, 4, 4>(const GemmArgs &, int, hipStream_t);
template hipError_t gemm_lds_launch<128, 128, 2, 2, 4>(const GemmArgs &, int, hipStream_t);
template hipError_t gemm_lds_launch<256, 192, 4, 2, 4>(const GemmArgs &, int, hipStream_t);

}  // namespace mxk
