// k_gemm_i8.hip -- the int8 (W8A8) instantiations of the persistent
// LDS-pipelined GEMM (kernel body and design in k_gemm_lds.hpp): exact int32
// accumulation in v_mfma_i32_32x32x32_i8 with dequantise_c fused into the
// epilogue, or the raw int32 accumulators.
#include "k_gemm_lds.hpp"

using namespace mxlds;

namespace {

// OUT: 0 fp32 C, 1 bf16 C, 2 raw int32 C. RB: bytes (= int8 K) per slab row.
template <int BM, int BN, int WGM, int WGN, int NS, int EPI, bool RES, int OUT, int RB>
__global__ __launch_bounds__(WGM *WGN * 64) void gemm_i8_k(
    const int8_t *__restrict__ A, int64_t lda, const int8_t *__restrict__ Wt, int M, int N,
    int K, const float *__restrict__ a_scale, const float *__restrict__ wscale,
    const float *__restrict__ bias, const float *residual, void *C, int64_t ldc, int tiles_m,
    int tiles_n, const int32_t *rows_dev) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  gemm_lds_body<BM, BN, WGM, WGN, NS, EPI, RES, OUT == 1, true, OUT == 2, RB>(
      A, lda, Wt, M, N, K, bias, residual, C, ldc, tiles_m, tiles_n, a_scale, wscale, smem,
      rows_dev);
}

template <int BM, int BN, int WGM, int WGN, int NS, int EPI, bool RES, int OUT, int RB = 64>
hipError_t launch_t(const mxk::GemmI8Args &a, int grid, hipStream_t s) {
  using Cfg = LdsCfg<BM, BN, WGM, WGN, NS, true, stg_kind(OUT == 1, RES), RB>;
  auto kern = gemm_i8_k<BM, BN, WGM, WGN, NS, EPI, RES, OUT, RB>;
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
  kern<<<g, Cfg::NT, Cfg::LDS, s>>>(a.A, a.lda, a.Wt, (int)a.M, (int)a.N, (int)a.K, a.a_scale,
                                    a.wscale, a.bias, a.residual, a.C, a.ldc, tiles_m, tiles_n,
                                    a.rows_dev);
  return hipGetLastError();
}

template <int BM, int BN, int WGM, int WGN, int NS>
hipError_t launch(const mxk::GemmI8Args &a, int grid, hipStream_t s) {
  if (a.c_dtype == 2) return launch_t<BM, BN, WGM, WGN, NS, 0, false, 2>(a, grid, s);
  if (a.epilogue >= mxk::EPI_GLU_SILU) {
    // The fused gated FFN pairs a wave's column blocks: an even number of
    // them, a bf16 C.
    if constexpr ((BN / WGN) % 64 == 0) {
      if (a.c_dtype != 1 || a.residual) return hipErrorInvalidValue;
      if (a.epilogue == mxk::EPI_GLU_SILU)
        return launch_t<BM, BN, WGM, WGN, NS, mxk::EPI_GLU_SILU, false, 1>(a, grid, s);
      if (a.epilogue == mxk::EPI_GLU_GELU)
        return launch_t<BM, BN, WGM, WGN, NS, mxk::EPI_GLU_GELU, false, 1>(a, grid, s);
    }
    return hipErrorInvalidValue;
  }
#define MX_I8_EPI(E)                                                                 \
  if (a.epilogue == E) {                                                             \
    if (a.residual)                                                                  \
      return a.c_dtype == 1 ? launch_t<BM, BN, WGM, WGN, NS, E, true, 1>(a, grid, s) \
                            : launch_t<BM, BN, WGM, WGN, NS, E, true, 0>(a, grid, s);  \
    return a.c_dtype == 1 ? launch_t<BM, BN, WGM, WGN, NS, E, false, 1>(a, grid, s)  \
                          : launch_t<BM, BN, WGM, WGN, NS, E, false, 0>(a, grid, s);   \
  }
  MX_I8_EPI(0)
  MX_I8_EPI(1)
  MX_I8_EPI(2)
#undef MX_I8_EPI
  return hipErrorInvalidValue;
}

// The 256 x 256 tile on 128-byte slabs (128 int8 of K, two slots): a bf16 C
// without a residual.
hipError_t launch_deep(const mxk::GemmI8Args &a, int grid, hipStream_t s) {
  if (a.c_dtype == 1 && !a.residual) {
    switch (a.epilogue) {
      case 0: return launch_t<256, 256, 4, 2, 2, 0, false, 1, 128>(a, grid, s);
      case 1: return launch_t<256, 256, 4, 2, 2, 1, false, 1, 128>(a, grid, s);
      case 2: return launch_t<256, 256, 4, 2, 2, 2, false, 1, 128>(a, grid, s);
      case mxk::EPI_GLU_SILU:
        return launch_t<256, 256, 4, 2, 2, mxk::EPI_GLU_SILU, false, 1, 128>(a, grid, s);
      case mxk::EPI_GLU_GELU:
        return launch_t<256, 256, 4, 2, 2, mxk::EPI_GLU_GELU, false, 1, 128>(a, grid, s);
      default: return hipErrorInvalidValue;
    }
  }
  return hipErrorInvalidValue;
}

// A narrowed C (EPI_NARROW_C: the int32 product rounded to bf16 once before
// the dequantisation; no residual, not the raw product): the 256 x 256 tile,
// or the 128 x 128 tile where the product is too small for it.
hipError_t launch_nc(const mxk::GemmI8Args &a, int grid, hipStream_t s) {
  if (a.residual || a.c_dtype == 2) return hipErrorInvalidValue;
  const int e = a.epilogue & ~EPI_NARROW_C;
  constexpr int NC = EPI_NARROW_C;
#define MX_I8_NC(BM, BN, WGM, WGN, NS)                                                        \
  switch (e) {                                                                                \
    case 0:                                                                                   \
      return a.c_dtype == 1 ? launch_t<BM, BN, WGM, WGN, NS, NC, false, 1>(a, grid, s)        \
                            : launch_t<BM, BN, WGM, WGN, NS, NC, false, 0>(a, grid, s);       \
    case 1:                                                                                   \
      return a.c_dtype == 1 ? launch_t<BM, BN, WGM, WGN, NS, NC | 1, false, 1>(a, grid, s)    \
                            : launch_t<BM, BN, WGM, WGN, NS, NC | 1, false, 0>(a, grid, s);   \
    case 2:                                                                                   \
      return a.c_dtype == 1 ? launch_t<BM, BN, WGM, WGN, NS, NC | 2, false, 1>(a, grid, s)    \
                            : launch_t<BM, BN, WGM, WGN, NS, NC | 2, false, 0>(a, grid, s);   \
    default: return hipErrorInvalidValue;                                                     \
  }
  if (mxk::gemm_lds_tile(mxk::gemm_pick_rows(a.M, a.m_hint), a.N, false) == 0) {
    MX_I8_NC(256, 256, 2, 4, 3)
  }
  MX_I8_NC(128, 128, 2, 2, 4)
#undef MX_I8_NC
}

}  // namespace

namespace mxk {

// (An fp32 C with a residual stays on 64-byte slabs on this datapath: with the
// dequantisation vectors its 128-byte-slab form spills registers.)
bool gemm_i8_deep(const GemmI8Args &a) {
  return a.c_dtype == 1 && !a.residual && a.K % 128 == 0 && a.K >= 256;
}

hipError_t gemm_i8(const GemmI8Args &a, hipStream_t s) {
  const int grid = cu_count();
  if (a.epilogue & EPI_NARROW_C) return launch_nc(a, grid, s);
  const bool deep = gemm_i8_deep(a);
  int t = gemm_lds_tile(gemm_pick_rows(a.M, a.m_hint), a.N, deep);
  if (t == 1 && a.epilogue >= EPI_GLU_SILU) t = 0;  // 96-column waves cannot pair blocks
  switch (t) {
    case 0: return deep ? launch_deep(a, grid, s) : launch<256, 256, 2, 4, 3>(a, grid, s);
    case 1: return launch<256, 192, 4, 2, 4>(a, grid, s);
    case 2: return launch<128, 256, 2, 4, 4>(a, grid, s);
    default: return launch<128, 128, 2, 2, 4>(a, grid, s);
  }
}

}  // namespace mxk
