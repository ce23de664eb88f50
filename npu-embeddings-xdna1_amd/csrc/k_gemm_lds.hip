// k_gemm_lds.hip -- the encoder's bf16 GEMM, pipelined through LDS by direct
// global->LDS loads (gfx950 global_load_lds_dwordx4).
//
// C[M, N] = epilogue(A[M, K] @ W[K, N] + bias) (+ residual), A bf16 row-major,
// W held as Wt[N, K] (K contiguous), fp32 accumulation in
// v_mfma_f32_32x32x16_bf16, one to_bf16 rounding at the store when C is bf16.
//
// Pipeline. The K axis advances BK = 32 at a time through an NS-slot LDS ring.
// Each slab is fetched straight into LDS by global_load_lds_dwordx4 (every lane
// moves 16 bytes; one wave instruction fills 1 KB of LDS), NS - 1 slabs ahead
// of the one the MFMAs consume, so no VGPR holds staged tiles and ~NS-1 slab
// times of HBM latency are covered. The loads are issued from inline assembly:
// the compiler's own wait insertion would otherwise put vmcnt(0) -- a wait on
// every prefetch -- before each LDS read. Each wave waits for its own loads of
// the slab it is about to read (vmcnt = loads it issued since), then all waves
// meet at one barrier per slab; the barrier also proves every wave has left
// the slot the next prefetch overwrites.
//
// LDS image. A slab is rows of 32 bf16 = 64 bytes = four 16-byte chunks. Chunk
// c of row r is stored at position c ^ ((r >> 1) & 3) of its row, so the eight
// lanes of one ds_read_b128 phase (rows r..r+7, same logical chunk) hit eight
// different 16-byte bank groups. The direct load writes lane l's 16 bytes at
// LDS offset 16*l of its 1 KB window, so the swizzle is applied to the GLOBAL
// address each lane fetches: lane l fills row l/4, position l%4, i.e. logical
// chunk (l%4) ^ (((l/4) >> 1) & 3).
//
// Operand roles. The MFMA's first operand is the W tile and its second the A
// tile, so the 32x32 accumulator holds C^T: each lane owns one row m of C and
// runs of four consecutive columns, stored as 8-byte (bf16) or 16-byte (fp32)
// vectors instead of 2- or 4-byte scalars.
//
// Edges. Rows past M (or N) are fetched from a clamped, in-bounds row and never
// stored. K must be a multiple of 32 (the launcher routes anything else to the
// register-staged kernel in k_gemm.hip).
//
// Blocks are numbered so that each XCD (workgroups go round-robin over the 8
// XCDs) owns a contiguous run of tiles in row-major (m, n) order.
#include "mx_common.hpp"
#include "mx_kernels.hpp"

using namespace mxd;

namespace {

constexpr int BK = 32;
constexpr int ROWB = BK * 2;  // bytes per LDS row

template <int BM, int BN, int WGM, int WGN, int NS>
struct LdsCfg {
  static constexpr int NW = WGM * WGN;          // waves
  static constexpr int NT = NW * 64;            // threads
  static constexpr int WM = BM / WGM, WN = BN / WGN;  // wave tile
  static constexpr int TM = WM / 32, TN = WN / 32;    // 32x32 MFMA tiles per wave
  static constexpr int A_BYTES = BM * ROWB, B_BYTES = BN * ROWB;
  static constexpr int SLOT = A_BYTES + B_BYTES;
  static constexpr int A_LOADS = A_BYTES / 1024 / NW;  // 1 KB wave loads per wave per slab
  static constexpr int B_LOADS = B_BYTES / 1024 / NW;
  static constexpr int LOADS = A_LOADS + B_LOADS;
  static constexpr int LDS = NS * SLOT;
  static_assert(WM % 32 == 0 && WN % 32 == 0, "wave tile must be whole MFMA tiles");
  static_assert(A_BYTES % (1024 * NW) == 0 && B_BYTES % (1024 * NW) == 0,
                "each wave must issue whole 1 KB loads");
  static_assert(LDS <= 160 * 1024, "gfx950 LDS is 160 KB");
  static_assert(NS >= 2 && LOADS * (NS - 1) < 64, "vmcnt holds at most 63");
};

// s_waitcnt vmcnt(N), other counters untouched.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// One wave-wide direct load: 64 lanes x 16 bytes from `src` (per lane) into
// LDS bytes [lds, lds + 1024) in lane order.
__device__ __forceinline__ void dma16(const void *src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off"
               ::"s"(lds), "v"(src)
               : "memory");
}

// Epilogue variants are compile-time: EPI (mx_epilogue), RES (fp32 residual
// added after the activation), CBF (bf16 C).
template <int BM, int BN, int WGM, int WGN, int NS, int EPI, bool RES, bool CBF>
__global__ __launch_bounds__(WGM *WGN * 64) void gemm_lds_k(
    const uint16_t *__restrict__ A, int64_t lda, const uint16_t *__restrict__ Wt, int M, int N,
    int K, const float *__restrict__ bias, const float *residual, void *C, int64_t ldc,
    int tiles_m, int tiles_n) {
  using Cfg = LdsCfg<BM, BN, WGM, WGN, NS>;
  constexpr int TM = Cfg::TM, TN = Cfg::TN;
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];

  const int total = tiles_m * tiles_n;
  int tile = blockIdx.x;
  if ((total & 7) == 0) tile = (blockIdx.x & 7) * (total >> 3) + (blockIdx.x >> 3);
  const int tm = tile / tiles_n, tn = tile - tm * tiles_n;
  const int m0 = tm * BM, n0 = tn * BN;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WGN, wn = wave - wm * WGN;
  const int li = lane & 31, g = lane >> 5;

  // Per-lane source pointers of this wave's loads (row within its 1 KB window
  // = lane / 4, logical chunk = swizzled lane % 4). Rows are clamped in bounds.
  const int lrow = lane >> 2;
  const int lchunk = (lane & 3) ^ ((lrow >> 1) & 3);
  const uint16_t *srcA[Cfg::A_LOADS];
  const uint16_t *srcB[Cfg::B_LOADS];
#pragma unroll
  for (int i = 0; i < Cfg::A_LOADS; ++i) {
    int r = m0 + (wave * Cfg::A_LOADS + i) * 16 + lrow;
    r = r < M ? r : M - 1;
    srcA[i] = A + (int64_t)r * lda + lchunk * 8;
  }
#pragma unroll
  for (int i = 0; i < Cfg::B_LOADS; ++i) {
    int r = n0 + (wave * Cfg::B_LOADS + i) * 16 + lrow;
    r = r < N ? r : N - 1;
    srcB[i] = Wt + (int64_t)r * K + lchunk * 8;
  }
  const uint32_t lds0 = (uint32_t)(uintptr_t)smem;
  auto issue = [&](int kt) {
    const uint32_t slot = lds0 + (uint32_t)((kt % NS) * Cfg::SLOT);
    const int k0 = kt * BK;
#pragma unroll
    for (int i = 0; i < Cfg::A_LOADS; ++i)
      dma16(srcA[i] + k0, slot + (uint32_t)((wave * Cfg::A_LOADS + i) * 1024));
#pragma unroll
    for (int i = 0; i < Cfg::B_LOADS; ++i)
      dma16(srcB[i] + k0, slot + Cfg::A_BYTES + (uint32_t)((wave * Cfg::B_LOADS + i) * 1024));
  };

  const int nk = K / BK;
#pragma unroll
  for (int s = 0; s < NS - 1; ++s)
    if (s < nk) issue(s);

  // The bias of this lane's columns, fetched while the first slabs land:
  // column n = n0 + wn*WN + 32*j + 8*q + 4*g + e.
  const int cbase = n0 + wn * Cfg::WN + g * 4;
  const bool cols_full = n0 + BN <= N;
  float4 bv[TN][4];
#pragma unroll
  for (int j = 0; j < TN; ++j)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int col = cbase + j * 32 + q * 8;
      float4 b = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (bias) {
        if (cols_full) {
          b = *(const float4 *)(bias + col);
        } else {
          if (col + 0 < N) b.x = bias[col + 0];
          if (col + 1 < N) b.y = bias[col + 1];
          if (col + 2 < N) b.z = bias[col + 2];
          if (col + 3 < N) b.w = bias[col + 3];
        }
      }
      bv[j][q] = b;
    }

  f32x16 acc[TN][TM];
#pragma unroll
  for (int j = 0; j < TN; ++j)
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[j][i][r] = 0.0f;

  // Fragment addressing: lane (row li, k-half g) reads logical chunk 2*kk + g
  // of its row, at its swizzled position.
  const int swz = (li >> 1) & 3;  // (row >> 1) & 3 with row = 32*x + li
  const int pos0 = ((0 + g) ^ swz) * 16, pos1 = ((2 + g) ^ swz) * 16;
  const int rowA = (wm * Cfg::WM + li) * ROWB, rowB = (wn * Cfg::WN + li) * ROWB;

  for (int kt = 0; kt < nk; ++kt) {
    // This wave's loads of slab kt are done once at most the loads of the
    // slabs issued after it (up to NS - 2 of them) are outstanding. The bias
    // loads were issued after the first NS - 1 slabs, so the first wait
    // covers them too.
    const int ahead = nk - 1 - kt < NS - 2 ? nk - 1 - kt : NS - 2;
    if (kt == 0) {
      wait_vmcnt<0>();
    } else if (ahead >= NS - 2) {
      wait_vmcnt<Cfg::LOADS *(NS - 2)>();
    } else if (NS > 2 && ahead == NS - 3) {
      wait_vmcnt<(NS > 2 ? Cfg::LOADS * (NS - 3) : 0)>();
    } else {
      wait_vmcnt<0>();
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's LDS reads are done
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (kt + NS - 1 < nk) issue(kt + NS - 1);

    const uint8_t *slot = smem + (kt % NS) * Cfg::SLOT;
    bf16x8 fa[2][TM], fb[2][TN];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const int pos = kk ? pos1 : pos0;
#pragma unroll
      for (int j = 0; j < TN; ++j)
        fb[kk][j] = *(const bf16x8 *)(slot + Cfg::A_BYTES + rowB + j * 32 * ROWB + pos);
#pragma unroll
      for (int i = 0; i < TM; ++i)
        fa[kk][i] = *(const bf16x8 *)(slot + rowA + i * 32 * ROWB + pos);
    }
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int i = 0; i < TM; ++i)
          acc[j][i] =
              __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[kk][j], fa[kk][i], acc[j][i], 0, 0, 0);
  }

  // Epilogue. acc[j][i] is the C^T tile: lane owns C row m = m0 + wm*WM +
  // 32*i + li and columns cbase + 32*j + 8*q + e (register r = 4*q + e).
  const bool interior = cols_full && m0 + BM <= M;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int row = m0 + wm * Cfg::WM + i * 32 + li;
    const bool row_ok = interior || row < M;
    const int64_t roff = (int64_t)(row_ok ? row : 0) * ldc;
    float4 rv[TN][4];
    if (RES) {
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int col = cbase + j * 32 + q * 8;
          rv[j][q] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
          if (interior || (row_ok && col + 4 <= N)) {
            rv[j][q] = *(const float4 *)(residual + roff + col);
          } else if (row_ok) {
            if (col + 0 < N) rv[j][q].x = residual[roff + col + 0];
            if (col + 1 < N) rv[j][q].y = residual[roff + col + 1];
            if (col + 2 < N) rv[j][q].z = residual[roff + col + 2];
          }
        }
    }
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int col = cbase + j * 32 + q * 8;
        float v[4] = {acc[j][i][q * 4 + 0] + bv[j][q].x, acc[j][i][q * 4 + 1] + bv[j][q].y,
                      acc[j][i][q * 4 + 2] + bv[j][q].z, acc[j][i][q * 4 + 3] + bv[j][q].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = gemm_epilogue(v[e], EPI);
        if (RES) {
          v[0] += rv[j][q].x;
          v[1] += rv[j][q].y;
          v[2] += rv[j][q].z;
          v[3] += rv[j][q].w;
        }
        if (interior || (row_ok && col + 4 <= N)) {
          if (CBF) {
            uint2 w;
            w.x = pack_bf2(v[0], v[1]);
            w.y = pack_bf2(v[2], v[3]);
            *(uint2 *)((uint16_t *)C + roff + col) = w;
          } else {
            *(float4 *)((float *)C + roff + col) = make_float4(v[0], v[1], v[2], v[3]);
          }
        } else if (row_ok) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if (col + e < N) {
              if (CBF)
                ((uint16_t *)C)[roff + col + e] = f2bf(v[e]);
              else
                ((float *)C)[roff + col + e] = v[e];
            }
          }
        }
      }
  }
}

}  // namespace

namespace mxk {

template <int BM, int BN, int WGM, int WGN, int NS, int EPI, bool RES, bool CBF>
hipError_t gemm_lds_launch_t(const GemmArgs &a, hipStream_t s) {
  using Cfg = LdsCfg<BM, BN, WGM, WGN, NS>;
  auto kern = gemm_lds_k<BM, BN, WGM, WGN, NS, EPI, RES, CBF>;
  static bool attr_set = false;
  if (!attr_set) {
    const hipError_t e = hipFuncSetAttribute((const void *)kern,
                                             hipFuncAttributeMaxDynamicSharedMemorySize,
                                             Cfg::LDS);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  const int tiles_m = (int)((a.M + BM - 1) / BM), tiles_n = (int)((a.N + BN - 1) / BN);
  kern<<<tiles_m * tiles_n, Cfg::NT, Cfg::LDS, s>>>(a.A, a.lda, a.Wt, (int)a.M, (int)a.N,
                                                     (int)a.K, a.bias, a.residual, a.C, a.ldc,
                                                     tiles_m, tiles_n);
  return hipGetLastError();
}

// One tile configuration, every epilogue variant.
template <int BM, int BN, int WGM, int WGN, int NS>
hipError_t gemm_lds_launch(const GemmArgs &a, hipStream_t s) {
#define MX_LDS_EPI(E)                                                                  \
  if (a.epilogue == E) {                                                               \
    if (a.residual)                                                                    \
      return a.c_bf16 ? gemm_lds_launch_t<BM, BN, WGM, WGN, NS, E, true, true>(a, s)   \
                      : gemm_lds_launch_t<BM, BN, WGM, WGN, NS, E, true, false>(a, s); \
    return a.c_bf16 ? gemm_lds_launch_t<BM, BN, WGM, WGN, NS, E, false, true>(a, s)    \
                    : gemm_lds_launch_t<BM, BN, WGM, WGN, NS, E, false, false>(a, s);  \
  }
  MX_LDS_EPI(0)
  MX_LDS_EPI(1)
  MX_LDS_EPI(2)
#undef MX_LDS_EPI
  return hipErrorInvalidValue;
}

template hipError_t gemm_lds_launch<256, 256, 2, 4, 3>(const GemmArgs &, hipStream_t);
template hipError_t gemm_lds_launch<128, 256, 2, 4, 4>(const GemmArgs &, hipStream_t);
template hipError_t gemm_lds_launch<128, 128, 2, 2, 4>(const GemmArgs &, hipStream_t);

}  // namespace mxk
