// k_gemm.hip -- the unified bf16 GEMM of the encoder path on gfx950 MFMA.
//
// C[M, N] = epilogue(A[M, K] @ W[K, N] + bias) (+ residual), A bf16 row-major,
// W held as its transpose Wt[N, K] (K contiguous, the layout mx_stage_weight
// writes once) so both operands are read the same way. fp32 accumulation in
// v_mfma_f32_32x32x16_bf16; one rounding to bf16 (the host's to_bf16
// formula) at the very end when C is bf16 -- the single-narrowing contract of
// kernels/narrow_f32_bf16.cc, here fused into the store.
//
// Tiling: a BM x BN block tile over (BM/WM) x (BN/WN) waves, each wave owning
// a WM x WN sub-tile of (WM/32) x (WN/32) MFMA tiles. K advances BK at a time
// through two LDS buffers: the next K-slab is fetched from HBM into registers
// while the MFMAs consume the current one, then written to the other buffer,
// so there is one barrier per slab. LDS rows are padded by 16 bytes, which
// makes the 16-byte fragment reads of 8 consecutive rows hit distinct banks.
//
// Blocks are numbered so that each XCD (workgroups go round-robin over the 8
// XCDs) owns a contiguous run of tiles in row-major (m, n) order: the blocks
// resident on one XCD share A row-panels and the whole of W in its L2.
#include "mx_common.hpp"
#include "mx_kernels.hpp"

using namespace mxd;

namespace {

template <int BM, int BN, int BK, int WM, int WN>
struct GemmCfg {
  static constexpr int NWM = BM / WM, NWN = BN / WN;
  static constexpr int NT = NWM * NWN * 64;
  static constexpr int LDK = BK + 8;  // padded LDS row, elements
  static constexpr int TM = WM / 32, TN = WN / 32;
  static constexpr int CPR = BK / 8;  // 16-byte chunks per row
  static constexpr int A_PER_T = BM * CPR / NT;
  static constexpr int B_PER_T = BN * CPR / NT;
  static constexpr int LDS_BYTES = 2 * (BM + BN) * LDK * 2;
  static_assert(BM * CPR % NT == 0 && BN * CPR % NT == 0, "chunks must divide threads");
  static_assert(WM % 32 == 0 && WN % 32 == 0 && BK % 16 == 0, "MFMA tile shape");
};

template <int BM, int BN, int BK, int WM, int WN>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * 64) void gemm_bf16_k(
    const uint16_t *__restrict__ A, int64_t lda, const uint16_t *__restrict__ Wt, int M, int N,
    int K, const float *__restrict__ bias, int epi, const float *residual, void *C, int c_bf16,
    int64_t ldc, int tiles_m, int tiles_n, const int32_t *rows_dev) {
  using Cfg = GemmCfg<BM, BN, BK, WM, WN>;
  constexpr int LDK = Cfg::LDK, NT = Cfg::NT, CPR = Cfg::CPR;
  constexpr int TM = Cfg::TM, TN = Cfg::TN;
  __shared__ __attribute__((aligned(16))) uint16_t smA[2][BM * LDK];
  __shared__ __attribute__((aligned(16))) uint16_t smB[2][BN * LDK];

  // XCD-aware tile order.
  const int total = tiles_m * tiles_n;
  int tile = blockIdx.x;
  if ((total & 7) == 0) tile = (blockIdx.x & 7) * (total >> 3) + (blockIdx.x >> 3);
  const int tm = tile / tiles_n, tn = tile - tm * tiles_n;
  const int m0 = tm * BM, n0 = tn * BN;
  M = (int)live_rows(M, rows_dev);
  if (m0 >= M) return;  // the whole block: a tile past the live rows

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / Cfg::NWN, wn = wave - wm * Cfg::NWN;

  uint4 ra[Cfg::A_PER_T], rb[Cfg::B_PER_T];
  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < Cfg::A_PER_T; ++i) {
      const int c = tid + i * NT, r = c / CPR, kc = (c - r * CPR) * 8;
      const int gr = m0 + r, gk = k0 + kc;
      ra[i] = (gr < M && gk < K) ? *(const uint4 *)(A + (int64_t)gr * lda + gk)
                                 : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < Cfg::B_PER_T; ++i) {
      const int c = tid + i * NT, r = c / CPR, kc = (c - r * CPR) * 8;
      const int gr = n0 + r, gk = k0 + kc;
      rb[i] = (gr < N && gk < K) ? *(const uint4 *)(Wt + (int64_t)gr * K + gk)
                                 : make_uint4(0, 0, 0, 0);
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < Cfg::A_PER_T; ++i) {
      const int c = tid + i * NT, r = c / CPR, kc = (c - r * CPR) * 8;
      *(uint4 *)&smA[buf][r * LDK + kc] = ra[i];
    }
#pragma unroll
    for (int i = 0; i < Cfg::B_PER_T; ++i) {
      const int c = tid + i * NT, r = c / CPR, kc = (c - r * CPR) * 8;
      *(uint4 *)&smB[buf][r * LDK + kc] = rb[i];
    }
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int nk = (K + BK - 1) / BK;
  gload(0);
  sstore(0);
  __syncthreads();
  const int frow = lane & 31, fk = (lane >> 5) * 8;
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) gload((kt + 1) * BK);
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      bf16x8 af[TM], bfr[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        af[i] = *(const bf16x8 *)&smA[cur][(wm * WM + i * 32 + frow) * LDK + kk * 16 + fk];
#pragma unroll
      for (int j = 0; j < TN; ++j)
        bfr[j] = *(const bf16x8 *)&smB[cur][(wn * WN + j * 32 + frow) * LDK + kk * 16 + fk];
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) sstore(cur ^ 1);
    __syncthreads();
  }

  // Epilogue. 32x32 accumulator layout: lane holds column (lane & 31) and rows
  // 8*(r/4) + 4*(lane/32) + (r%4), r = 0..15.
  const int rbase = (lane >> 5) * 4;
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int col = n0 + wn * WN + j * 32 + (lane & 31);
    if (col >= N) continue;
    const float bj = bias ? bias[col] : 0.0f;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm * WM + i * 32 + (r >> 2) * 8 + rbase + (r & 3);
        if (row >= M) continue;
        float v = gemm_epilogue(acc[i][j][r] + bj, epi);
        const int64_t off = (int64_t)row * ldc + col;
        if (residual) v += residual[off];
        if (c_bf16)
          ((uint16_t *)C)[off] = f2bf(v);
        else
          ((float *)C)[off] = v;
      }
    }
  }
}

template <int BM, int BN, int BK, int WM, int WN>
hipError_t launch(const mxk::GemmArgs &a, hipStream_t s) {
  using Cfg = GemmCfg<BM, BN, BK, WM, WN>;
  const int tiles_m = (int)((a.M + BM - 1) / BM), tiles_n = (int)((a.N + BN - 1) / BN);
  const int blocks = tiles_m * tiles_n;
  gemm_bf16_k<BM, BN, BK, WM, WN><<<blocks, Cfg::NT, 0, s>>>(
      a.A, a.lda, a.Wt, (int)a.M, (int)a.N, (int)a.K, a.bias, a.epilogue, a.residual, a.C,
      a.c_bf16, a.ldc, tiles_m, tiles_n, a.rows_dev);
  return hipGetLastError();
}

}  // namespace

namespace mxk {

// The persistent LDS-pipelined kernel (k_gemm_lds.hip) serves every call it
// can: K a multiple of 32 and at least 128 (four slabs, the deepest ring), N a
// multiple of 4, a bias, and C, bias and residual aligned for 16-byte vector
// access; the register-staged kernel above serves the rest.
template <int BM, int BN, int WGM, int WGN, int NS>
hipError_t gemm_lds_launch(const GemmArgs &a, int grid, hipStream_t s);
hipError_t gemm_lds_deep_launch(const GemmArgs &a, int grid, hipStream_t s);
hipError_t gemm_lds_128_deep_launch(const GemmArgs &a, int grid, hipStream_t s);
hipError_t gemm_lds_nc_launch(const GemmArgs &a, int grid, hipStream_t s);

namespace {

enum GemmPath {
  PATH_STAGED,
  PATH_LDS_256x256,
  PATH_LDS_256x192,
  PATH_LDS_128x256,
  PATH_LDS_128x128,
  PATH_LDS_256x256_DEEP,
  PATH_LDS_128x128_DEEP
};

// The 256 x 256 tile on 128-byte slabs: a bf16 C without a residual or an
// fp32 C with one, K a multiple of 64.
bool deep_ok(const GemmArgs &a) {
  return ((a.c_bf16 && !a.residual) || (!a.c_bf16 && a.residual)) && a.K % 64 == 0;
}

bool lds_path_ok(const GemmArgs &a) {
  const uintptr_t c = (uintptr_t)a.C;
  return a.K % 32 == 0 && a.K >= 128 && a.N % 4 == 0 && a.lda % 8 == 0 && a.bias &&
         lds_offsets_fit(a.lda, a.K, 2) &&
         a.ldc % (a.c_bf16 ? 8 : 4) == 0 && c % 16 == 0 && (uintptr_t)a.bias % 16 == 0 &&
         (!a.residual || (uintptr_t)a.residual % 16 == 0);
}

GemmPath pick(const GemmArgs &a) {
  if (!lds_path_ok(a)) return PATH_STAGED;
  static const GemmPath paths[] = {PATH_LDS_256x256, PATH_LDS_256x192, PATH_LDS_128x256,
                                   PATH_LDS_128x128};
  const bool deep = deep_ok(a);
  const int64_t m = gemm_pick_rows(a.M, a.m_hint);
  int t = gemm_lds_tile(m, a.N, deep);
  if (t == 1 && a.epilogue >= EPI_GLU_SILU) t = 0;  // 96-column waves cannot pair blocks
  if (t == 0 && deep) return PATH_LDS_256x256_DEEP;
  // The 128 x 128 tile on 128-byte slabs keeps one slab in flight ahead, the
  // 64-byte form three: a launch of a few tiles per XCD (the CLS-pruned last
  // layer's 64-row GEMMs) waits on every slab's load and runs faster with
  // three ahead. Both run the same MFMA chain over K for every element.
  if (t == 3 && deep && a.c_bf16 && !a.residual &&
      ((m + 127) / 128) * ((a.N + 127) / 128) * 8 > cu_count())
    return PATH_LDS_128x128_DEEP;
  return paths[t];
}

}  // namespace

// The tile with the least estimated time: rounds of tiles over the CUs (the
// last round costs a whole one) times the tile's area over its relative
// throughput per unit area, measured on MI355X on the encoder's GEMM shapes
// when every tile count is a whole number of rounds (256 x 256: 1.0, 256 x
// 192: 0.88, 128 x 256: 0.86, 128 x 128: 0.65; the 256 x 256 tile on
// 128-byte slabs: 1.1). The 256 x 192 tile wins where N = 768 leaves 256 x
// 256 tiles at 1.5 rounds; small problems take the small tiles that spread
// over the most CUs.
int gemm_lds_tile(int64_t M, int64_t N, bool deep) {
  struct Cand {
    int bm, bn;
    double eff;
  };
  const Cand cands[] = {{256, 256, deep ? 1.1 : 1.0}, {256, 192, 0.88}, {128, 256, 0.86},
                        {128, 128, 0.65}};
  const int64_t G = cu_count();
  int best = 3;
  double best_t = 0.0;
  for (int i = 0; i < 4; ++i) {
    const Cand &c = cands[i];
    const int64_t tiles = ((M + c.bm - 1) / c.bm) * ((N + c.bn - 1) / c.bn);
    const double t = (double)((tiles + G - 1) / G) * c.bm * c.bn / c.eff;
    if (best_t == 0.0 || t < best_t) {
      best = i;
      best_t = t;
    }
  }
  return best;
}

// Resident blocks of the persistent kernel: one per CU of the current device.
int cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cached[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}


const char *gemm_plan_name(int64_t M, int64_t N, int64_t K, bool c_bf16, bool residual,
                           bool i8) {
  static const float aligned_probe[4] __attribute__((aligned(16))) = {0, 0, 0, 0};
  if (i8) {
    // The int8 kernels are the same tiles with slabs of 64 (or, deep, 128) int8.
    GemmI8Args a{};
    a.M = M;
    a.N = N;
    a.K = K;
    a.c_dtype = c_bf16 ? 1 : 0;
    a.residual = residual ? aligned_probe : nullptr;
    const bool deep = gemm_i8_deep(a);
    switch (gemm_lds_tile(M, N, deep)) {
      case 0:
        return deep ? "lds_256x256x128_w64x128_ns2_persistent"
                    : "lds_256x256x64_w128x64_ns3_persistent";
      case 1: return "lds_256x192x64_w64x96_ns4_persistent";
      case 2: return "lds_128x256x64_w64x64_ns4_persistent";
      default: return "lds_128x128x64_w64x64_ns4_persistent";
    }
  }
  GemmArgs a{};
  a.M = M;
  a.N = N;
  a.K = K;
  a.lda = K;
  a.ldc = N;
  a.bias = aligned_probe;
  a.residual = residual ? aligned_probe : nullptr;
  a.C = (void *)aligned_probe;
  a.c_bf16 = c_bf16 ? 1 : 0;
  switch (pick(a)) {
    case PATH_LDS_256x256_DEEP: return "lds_256x256x64_w64x128_ns2_persistent";
    case PATH_LDS_128x128_DEEP: return "lds_128x128x64_w64x64_ns2_persistent";
    case PATH_LDS_256x256: return "lds_256x256x32_w128x64_ns3_persistent";
    case PATH_LDS_256x192: return "lds_256x192x32_w64x96_ns4_persistent";
    case PATH_LDS_128x256: return "lds_128x256x32_w64x64_ns4_persistent";
    case PATH_LDS_128x128: return "lds_128x128x32_w64x64_ns4_persistent";
    default: return "staged_128x128x64_w64x64";
  }
}

const char *gemm_config_name(int64_t M, int64_t N, int64_t K) {
  return gemm_plan_name(M, N, K, false, false, false);
}

hipError_t gemm(const GemmArgs &a, hipStream_t s) {
  if (a.epilogue & EPI_NARROW_C) {
    if (!lds_path_ok(a) || a.residual) return hipErrorInvalidValue;
    return gemm_lds_nc_launch(a, cu_count(), s);
  }
  const GemmPath p = pick(a);
  // The fused gated FFN exists only on the LDS-pipelined kernel.
  if (a.epilogue >= EPI_GLU_SILU && (p == PATH_STAGED || a.N % 64)) return hipErrorInvalidValue;
  switch (p) {
    case PATH_LDS_256x256_DEEP: return gemm_lds_deep_launch(a, cu_count(), s);
    case PATH_LDS_128x128_DEEP: return gemm_lds_128_deep_launch(a, cu_count(), s);
    case PATH_LDS_256x256: return gemm_lds_launch<256, 256, 2, 4, 3>(a, cu_count(), s);
    case PATH_LDS_256x192: return gemm_lds_launch<256, 192, 4, 2, 4>(a, cu_count(), s);
    case PATH_LDS_128x256: return gemm_lds_launch<128, 256, 2, 4, 4>(a, cu_count(), s);
    case PATH_LDS_128x128: return gemm_lds_launch<128, 128, 2, 2, 4>(a, cu_count(), s);
    default: return launch<128, 128, 64, 64, 64>(a, s);
  }
}

}  // namespace mxk
