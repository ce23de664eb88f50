// k_gemm_lds.hpp -- the encoder's GEMM on gfx950: a persistent kernel whose
// operand tiles reach LDS by direct global->LDS loads (global_load_lds_dwordx4)
// through a ring of slabs. One template serves both datapaths of the
// reference's array GEMM (the bf16 and the int8 design, bert_encoder.cpp:
// 741-924); k_gemm_lds.hip instantiates the bf16 kernels, k_gemm_i8.hip the
// int8 ones.
//
// bf16: C[M, N] = epilogue(A[M, K] @ W[K, N] + bias) (+ residual), A bf16
// row-major, W held as Wt[N, K] (K contiguous), fp32 accumulation in
// v_mfma_f32_32x32x16_bf16, one round-to-nearest-even narrowing (the hardware
// conversion) at the store when C is bf16.
//
// int8 (W8A8): A and Wt are int8, the accumulation is exact int32 in
// v_mfma_i32_32x32x32_i8, and the epilogue is dequantise_c
// (host_kernels.hpp:529-600, its int32-C form) fused:
//   y = fma(float(acc) * a_scale[row], wscale[col], bias[col])
// rounded exactly as the host's _mm256_fmadd_ps(_mm256_mul_ps(cf, sa), ws, b),
// then the activation and the store. RAW stores the int32 accumulators
// themselves (the design's C before dequantisation).
//
// Narrowed C (EPI | EPI_NARROW_C): the array designs that narrow C on the core
// (c_elem_bytes == 2, the export default) round the finished accumulator to
// bf16 -- fp32 to nearest even (narrow_f32_bf16), int32 in one rounding of the
// integer (narrow_i32_bf16) -- and the host adds the bias or dequantises from
// that bf16 value (host_kernels.hpp:529-560, bert_encoder.cpp:633-712,
// :874-900). With the bit set, the epilogue reads the accumulator through the
// same rounding before anything else.
//
// Grid. One block per CU walks a list of BM x BN output tiles; its slabs
// (RB = 64 or 128 bytes of K per row: 32 or 64 bf16, 64 or 128 int8; 128-byte
// rows make every load request a whole 128-byte line and halve the barriers
// per K, and need two 64 KB slots for a 256 x 256 tile) form one sequence across tile
// boundaries, so the ring keeps loading the next tile's first slabs while the
// current tile drains: no per-tile prologue latency, no block relaunch.
// Workgroups go round-robin over the 8 XCDs, so the blocks of XCD x
// (blockIdx % 8 == x) share the x-th eighth of the tiles (row-major over
// (m, n)) and walk it together: they share A row-panels and W in that XCD's
// L2, and every XCD gets the same share of the work even when the tiles do
// not fill whole rounds.
//
// Ring. NS slots; slab s + NS is fetched into slot s % NS as soon as every read
// of slab s is done, i.e. ~NS - 1 slabs ahead of its use. The loads are issued
// from inline assembly: the compiler's own wait insertion would otherwise put
// vmcnt(0) -- a wait on every prefetch -- before each LDS read. Each load is
// addressed as a scalar base (the operand's tile origin plus the slab's depth)
// and a 32-bit per-lane offset fixed for the tile, so issuing a slab costs a
// few scalar adds: building 64-bit addresses per load (quarter-rate integer
// multiplies on the vector ALU, right after the barrier) cost up to a tenth
// of the kernel. Each wave waits
// for its own loads of the slab it is about to read (vmcnt = loads it issued
// since; loads complete in issue order), then all waves meet at one barrier
// per slab. The first slab of each tile also moves the tile's epilogue
// vectors into per-tile-parity LDS copies (a few lanes of one extra load per
// wave and vector: the bias; for int8 also wscale and the rows' a_scale), so
// they are on chip for the epilogue without a compiler-tracked load; the
// waits do not count those loads, which only makes them stricter.
//
// Fragments. A slab is RB/32 k-steps of 32 bytes of K. Two register sets
// alternate: each k-step's MFMAs run while the next k-step is read from LDS
// into the other set (in the order the MFMAs consume it, one ds_read after
// each of the first MFMAs, pinned by sched_group_barrier). The barrier sits
// before the slab's last k-step, when every read of the slab has been issued.
//
// LDS image. A slab is rows of RB bytes = RB/16 16-byte chunks. gfx950
// serves a ds_read_b128 sixteen lanes (256 bytes, all 64 banks) per cycle; the
// sixteen lanes of one phase read rows r..r+15 at the same logical chunk.
// Chunk c of row r is stored at position chunk_pos(c, r) of its row, which
// puts those sixteen 16-byte reads in sixteen different bank groups. The
// direct load writes lane l's 16 bytes at LDS offset 16*l of its 1 KB window,
// so the swizzle is applied to the GLOBAL address each lane fetches: lane l
// fills row l/(RB/16), position l%(RB/16), i.e. the logical chunk that
// chunk_pos maps there. A lane's MFMA operand is one 16-byte chunk (8 bf16 or
// 16 int8), read at the same chunk index for A and W, so both operands pair
// the same K values.
//
// Operand roles. The MFMA's first operand is the W tile and its second the A
// tile, so the 32x32 accumulator holds C^T: each lane owns one row of C and
// runs of four consecutive columns.
//
// Epilogue. Per 32 x 32 accumulator block a wave adds the bias (dequantises),
// applies the activation, writes the block to its private LDS staging area
// (packed bf16 in swizzled 64-byte rows for a bf16 C, else fp32 rows padded
// by 16 bytes) and reads it back row-major, so every global store (and
// residual load) of a wave covers whole 128-byte (fp32) or 64-byte (bf16) row
// segments instead of 16-byte pieces of 32 rows.
//
// Requirements (the launchers check them; bf16 shapes outside them go to
// k_gemm.hip's kernel): K a multiple of the slab depth and at least NS slabs,
// N % 4 == 0, a bias (bf16; optional for int8), 16-byte aligned operands.
// Rows past M (or N) are fetched from a clamped, in-bounds row and never
// stored.
#pragma once

#include "mx_common.hpp"
#include "mx_kernels.hpp"

namespace mxlds {

using namespace mxd;

// The epilogue bit of a narrowed C (see above); the rest of EPI is the
// activation (mx_epilogue) or a fused gated FFN (8, 9).
constexpr int EPI_NARROW_C = mxk::EPI_NARROW_C;

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

constexpr int STG_ROWB = 144;  // staging row: 32 fp32 + 16 bytes of padding

// The epilogue's staging per wave (stg_kind): 1 packed bf16 32-row blocks (a
// bf16 C without a residual), 2 KB; 2 fp32 16-row half blocks (an fp32 C with
// a residual), 2.25 KB; 0 fp32 32-row blocks (the rest), 4.5 KB. RB: bytes of
// K per slab row, 64 or 128.
constexpr int stg_kind(bool cbf, bool res) { return cbf && !res ? 1 : (res && !cbf ? 2 : 0); }

template <int BM, int BN, int WGM, int WGN, int NS, bool I8, int STG, int RB = 64>
struct LdsCfg {
  static constexpr int NW = WGM * WGN;                // waves
  static constexpr int NT = NW * 64;                  // threads
  static constexpr int WM = BM / WGM, WN = BN / WGN;  // wave tile
  static constexpr int TM = WM / 32, TN = WN / 32;    // 32x32 MFMA tiles per wave
  static constexpr int ESZ = I8 ? 1 : 2;              // operand element bytes
  static constexpr int BKE = RB / ESZ;                // K elements per slab
  static constexpr int KSTEPS = RB / 32;              // MFMA k-steps (32 bytes of K) per slab
  static constexpr int PR = 1024 / RB;                // slab rows per 1 KB piece
  static constexpr int CPR = RB / 16;                 // 16-byte chunks per slab row
  static constexpr int A_BYTES = BM * RB, B_BYTES = BN * RB;
  static constexpr int SLOT = A_BYTES + B_BYTES;
  // A slab is PIECES 1 KB wave loads of PR rows each, A's first; wave w
  // issues pieces w, w + NW, ...: LOADS_HI of them if w < NHI, else LOADS_LO
  // (a 256 x 192 slab is 28 pieces: four waves issue 4, four issue 3).
  static constexpr int A_PIECES = A_BYTES / 1024, PIECES = (A_BYTES + B_BYTES) / 1024;
  static constexpr int LOADS_LO = PIECES / NW, LOADS_HI = (PIECES + NW - 1) / NW;
  static constexpr int NHI = PIECES % NW == 0 ? NW : PIECES % NW;
  static constexpr int BIAS_PER_WAVE = BN / NW;        // floats each wave's bias piece moves
  static constexpr int ROWS_PER_WAVE = BM / NW;        // a_scale rows each wave moves
  static constexpr int STG_WAVE = STG == 1 ? 32 * 64 : (STG == 2 ? 16 : 32) * STG_ROWB;
  static constexpr int STG_OFF = NS * SLOT;
  static constexpr int BIAS_OFF = STG_OFF + NW * STG_WAVE;
  static constexpr int WS_OFF = BIAS_OFF + 2 * BN * 4;  // int8: wscale, two parities
  static constexpr int SA_OFF = WS_OFF + 2 * BN * 4;    // int8: a_scale, two parities
  static constexpr int LDS = I8 ? SA_OFF + 2 * BM * 4 : BIAS_OFF + 2 * BN * 4;
  static_assert(WM % 32 == 0 && WN % 32 == 0, "wave tile must be whole MFMA tiles");
  static_assert(A_BYTES % 1024 == 0 && B_BYTES % 1024 == 0, "slabs are whole 1 KB pieces");
  static_assert(BIAS_PER_WAVE % 4 == 0 && BIAS_PER_WAVE <= 256, "bias piece: 16-byte lanes");
  static_assert(ROWS_PER_WAVE <= 64, "a_scale piece: one row per lane");
  static_assert(LDS <= 160 * 1024, "gfx950 LDS is 160 KB");
  static_assert(RB == 64 || RB == 128, "slab rows of 64 or 128 bytes");
  static_assert(NS >= 2 && LOADS_HI * (NS - 2) < 64, "vmcnt holds at most 63");
};

// Position of logical 16-byte chunk c in slab row r (an involution in c).
// Sixteen lanes of a ds_read_b128 phase read rows r..r+15 at one logical
// chunk; a row of RB bytes spans RB/4 banks, so row r starts at bank
// 16 * (r % 4) (RB = 64) or 32 * (r % 2) (RB = 128), and the XOR spreads the
// sixteen reads over all 64 banks.
template <int RB>
__device__ __forceinline__ int chunk_pos(int c, int r) {
  return RB == 64 ? c ^ ((r >> 2) & 3) : c ^ ((r >> 1) & 7);
}

// s_waitcnt vmcnt(N), other counters untouched.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// One wave-wide direct load: each active lane moves 16 bytes from `src` into
// LDS byte lds + 16 * lane.
__device__ __forceinline__ void dma16(const void *src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds), "v"(src)
               : "memory");
}

// The same with 4 bytes per lane, into LDS byte lds + 4 * lane.
__device__ __forceinline__ void dma4(const void *src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, off" ::"s"(lds), "v"(src)
               : "memory");
}

// The 16-byte load addressed as a wave-uniform base (SGPRs) plus a 32-bit
// per-lane byte offset: the per-slab advance is a scalar add.
__device__ __forceinline__ void dma16s(uint64_t base, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds), "v"(voff),
               "s"(base)
               : "memory");
}

__device__ __forceinline__ uint64_t uniform64(uint64_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return ((uint64_t)hi << 32) | lo;
}

// Wait until this wave's loads of the next slab have landed: at most the
// loads of the `later` slabs issued after it (LOADS each) may stay in flight,
// plus `extra` younger operations (the stores of an epilogue issued after that
// slab's loads). vmcnt counts loads and stores in issue order.
template <int LOADS, int NS, int EXTRA>
__device__ __forceinline__ void wait_slab(int ahead, bool extra) {
  if (ahead >= NS - 2) {
    if (extra)
      wait_vmcnt<LOADS *(NS - 2) + EXTRA>();
    else
      wait_vmcnt<LOADS *(NS - 2)>();
  } else if (NS > 3 && ahead == NS - 3) {
    if (extra)
      wait_vmcnt<(NS > 3 ? LOADS * (NS - 3) : 0) + EXTRA>();
    else
      wait_vmcnt<(NS > 3 ? LOADS * (NS - 3) : 0)>();
  } else {
    if (extra)
      wait_vmcnt<EXTRA>();
    else
      wait_vmcnt<0>();
  }
}

// The datapath's MFMA, fragment and accumulator types.
template <bool I8>
struct Path;
template <>
struct Path<false> {
  typedef bf16x8 frag;
  typedef f32x16 acc;
  static __device__ __forceinline__ acc mfma(frag w, frag a, acc c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(w, a, c, 0, 0, 0);
  }
};
template <>
struct Path<true> {
  typedef i32x4 frag;
  typedef i32x16 acc;
  static __device__ __forceinline__ acc mfma(frag w, frag a, acc c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(w, a, c, 0, 0, 0);
  }
};

// The kernel body. EPI: mx_epilogue; RES: add the fp32 residual; CBF: bf16 C
// (else fp32); I8: the int8 datapath; RAW (int8 only): store the int32
// accumulators, no bias, scales or activation.
template <int BM, int BN, int WGM, int WGN, int NS, int EPI, bool RES, bool CBF, bool I8,
          bool RAW, int RB = 64>
__device__ __forceinline__ void gemm_lds_body(
    const void *__restrict__ A, int64_t lda, const void *__restrict__ Wt, int M, int N, int K,
    const float *__restrict__ bias, const float *residual, void *C, int64_t ldc, int tiles_m,
    int tiles_n, const float *__restrict__ a_scale, const float *__restrict__ wscale,
    uint8_t *smem, const int32_t *rows_dev) {
  constexpr bool STG_BF = CBF && !RES;
  using Cfg = LdsCfg<BM, BN, WGM, WGN, NS, I8, stg_kind(CBF, RES), RB>;
  using PT = Path<I8>;
  typedef typename PT::frag frag_t;
  typedef typename PT::acc acc_t;
  static_assert(I8 || !RAW, "RAW is the int8 datapath's");
  static_assert(!RAW || (EPI == 0 && !RES && !CBF), "RAW stores the accumulators as they are");
  constexpr int TM = Cfg::TM, TN = Cfg::TN, ESZ = Cfg::ESZ;
  constexpr bool NC = (EPI & EPI_NARROW_C) != 0;
  constexpr int EPB = EPI & ~EPI_NARROW_C;
  // EPB 8 / 9: the gated FFN fused (GLU), C = lo * act(hi) in bf16 (act 1
  // SiLU, 2 exact-erf GELU), Wt's rows interleaved in groups of 16 (8 lo, 8
  // hi): each 32-column accumulator block gives 16 columns of C.
  constexpr bool GLU = EPB >= 8;
  constexpr int GACT = EPB - 7, EPA = GLU ? 0 : EPB;
  static_assert(!GLU || (EPB <= 9 && CBF && !RES && !RAW && !NC), "GLU: bf16 C, no residual");
  static_assert(!NC || (!RES && !RAW), "a narrowed C: no residual, not the raw product");
  static_assert(!GLU || TN % 2 == 0, "GLU pairs a wave's column blocks");
  // The bf16 kernel always has a bias (the launcher routes others away); the
  // int8 kernel takes it as optional.
  const bool has_bias = !RAW && (!I8 || bias != nullptr);

  // The live rows (M is then the bound A and C hold): the tile rows past them
  // are not walked.
  if (rows_dev) {
    M = (int)live_rows(M, rows_dev);
    tiles_m = (M + BM - 1) / BM;
  }
  // This block's tiles: t(i) = first + i * stride, i < my_tiles. With a grid
  // that is a multiple of 8, XCD x owns tiles [x*chunk, (x+1)*chunk) and its
  // G/8 blocks interleave over them. G: the launched blocks balanced over the
  // live tiles (mxk::balanced_grid); the blocks past it exit here.
  const int ntiles = tiles_m * tiles_n;
  const int G = mxk::balanced_grid(ntiles, (int)gridDim.x);
  if ((int)blockIdx.x >= G) return;
  int first = (int)blockIdx.x, stride = G, end = ntiles;
  if ((G & 7) == 0 && G >= 16) {
    const int chunk = (ntiles + 7) >> 3, x = (int)(blockIdx.x & 7);
    first = x * chunk + (int)(blockIdx.x >> 3);
    stride = G >> 3;
    end = min(ntiles, (x + 1) * chunk);
  }
  if (first >= end) return;
  const int my_tiles = (end - 1 - first) / stride + 1;
  const int nk = K / Cfg::BKE;
  const int nslab = my_tiles * nk;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WGN, wn = wave - wm * WGN;
  const int li = lane & 31, g = lane >> 5;

  // Load addressing: lane fills position lpos of row lrow of a PR-row piece,
  // i.e. it fetches the logical chunk stored there; rows are clamped in
  // bounds.
  const int lrow = lane / Cfg::CPR, lpos = lane % Cfg::CPR;
  const uint32_t lds0 = (uint32_t)(uintptr_t)smem;
  const uint8_t *Ab = (const uint8_t *)A;
  const uint8_t *Wb = (const uint8_t *)Wt;
  // Issue cursor: the next slab to issue is tile is_ti, depth is_kt, tile origin
  // (is_m0, is_n0).
  int is_ti = 0, is_kt = 0, is_m0 = 0, is_n0 = 0;
  auto tile_origin = [&](int ti, int &m0, int &n0) {
    const int t = first + ti * stride;
    const int tm = t / tiles_n;
    m0 = tm * BM;
    n0 = (t - tm * tiles_n) * BN;
  };
  tile_origin(0, is_m0, is_n0);
  // Per issue tile: each piece's per-lane byte offset from its operand's tile
  // origin (rows clamped in bounds), and the two origins as scalars. When the
  // waves split A's pieces evenly (SPLIT), load k of every wave is an A piece
  // iff k < A_PIECES / NW, known at compile time, and only the two origins
  // are kept; otherwise each load keeps its own.
  constexpr bool SPLIT = Cfg::A_PIECES % Cfg::NW == 0;
  uint32_t poff[Cfg::LOADS_HI];
  uint64_t pbase[Cfg::LOADS_HI];
  uint64_t abase = 0, bbase = 0;
  auto is_a = [&](int k) {
    return SPLIT ? k < Cfg::A_PIECES / Cfg::NW : wave + Cfg::NW * k < Cfg::A_PIECES;
  };
  auto set_tile = [&](int m0, int n0) {
#pragma unroll
    for (int k = 0; k < Cfg::LOADS_HI; ++k) {
      const int p = wave + Cfg::NW * k;
      if (is_a(k)) {
        const int tr = p * Cfg::PR + lrow;  // slab row within A's part
        int r = m0 + tr;
        r = (r < M ? r : M - 1) - m0;
        poff[k] = (uint32_t)(r * lda * ESZ + chunk_pos<RB>(lpos, tr) * 16);
      } else {
        const int tr = (p - Cfg::A_PIECES) * Cfg::PR + lrow;  // within W's part
        int r = n0 + tr;
        r = (r < N ? r : N - 1) - n0;
        poff[k] = (uint32_t)((int64_t)r * K * ESZ + chunk_pos<RB>(lpos, tr) * 16);
      }
    }
    abase = uniform64((uint64_t)(uintptr_t)(Ab + (int64_t)m0 * lda * ESZ));
    bbase = uniform64((uint64_t)(uintptr_t)(Wb + (int64_t)n0 * K * ESZ));
    if (!SPLIT) {
#pragma unroll
      for (int k = 0; k < Cfg::LOADS_HI; ++k) pbase[k] = is_a(k) ? abase : bbase;
    }
  };
  set_tile(is_m0, is_n0);
  // Issue the loads of slab is_s, then advance the cursor.
  uint32_t is_slot = 0;  // byte offset of slot is_s % NS
  uint64_t is_kb = 0;    // byte depth of slab is_kt
  auto issue = [&]() {
    const int ti = is_ti, kt = is_kt, n0 = is_n0, m0 = is_m0;
    const uint32_t slot = lds0 + is_slot;
#pragma unroll
    for (int k = 0; k < Cfg::LOADS_HI; ++k) {
      const int p = wave + Cfg::NW * k;  // wave-uniform
      if (k < Cfg::LOADS_LO || p < Cfg::PIECES)
        dma16s((SPLIT ? (is_a(k) ? abase : bbase) : pbase[k]) + is_kb, poff[k],
               slot + (uint32_t)(p * 1024));
    }
    // Epilogue vectors, on a tile's first slab: lanes 0 .. BIAS_PER_WAVE/4 - 1
    // move 16 bytes each of the columns from n0 + wave * BIAS_PER_WAVE (clamped
    // in bounds; a column >= N is never stored); for int8, lanes
    // 0 .. ROWS_PER_WAVE - 1 move one row's a_scale each (clamped likewise).
    // The other lanes are inactive for these loads and write nothing.
    if (kt == 0) {
      const uint32_t par = (uint32_t)(ti & 1);
      if (has_bias || (I8 && !RAW)) {
        if (lane < Cfg::BIAS_PER_WAVE / 4) {
          int c = n0 + wave * Cfg::BIAS_PER_WAVE + lane * 4;
          c = c < N ? c : N - 4;
          const uint32_t off = par * BN * 4 + (uint32_t)(wave * Cfg::BIAS_PER_WAVE * 4);
          if (has_bias) dma16(bias + c, lds0 + Cfg::BIAS_OFF + off);
          if (I8 && !RAW) dma16(wscale + c, lds0 + Cfg::WS_OFF + off);
        }
      }
      if (I8 && !RAW && lane < Cfg::ROWS_PER_WAVE) {
        int r = m0 + wave * Cfg::ROWS_PER_WAVE + lane;
        r = r < M ? r : M - 1;
        dma4(a_scale + r,
             lds0 + Cfg::SA_OFF + par * BM * 4 + (uint32_t)(wave * Cfg::ROWS_PER_WAVE * 4));
      }
    }
    is_slot = is_slot + Cfg::SLOT == NS * Cfg::SLOT ? 0 : is_slot + Cfg::SLOT;
    is_kb += RB;
    if (++is_kt == nk) {
      is_kt = 0;
      is_kb = 0;
      ++is_ti;
      if (is_ti < my_tiles) {
        tile_origin(is_ti, is_m0, is_n0);
        set_tile(is_m0, is_n0);
      }
    }
  };

  constexpr bool SAME_LOADS_P = Cfg::LOADS_HI == Cfg::LOADS_LO;
  static_assert(Cfg::LOADS_HI * (NS - 1) < 64, "vmcnt holds at most 63");
  acc_t acc[TN][TM];
#pragma unroll
  for (int j = 0; j < TN; ++j)
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[j][i][r] = 0;
  // Accumulator element r of block (j, i) as the epilogue reads it: as it is,
  // or (NC) rounded to bf16 first.
  auto accf = [&](int j, int i, int r) -> float {
    if constexpr (I8) {
      if constexpr (NC) return bf2f(i32_to_bf16((int)acc[j][i][r]));
      return (float)acc[j][i][r];
    } else {
      if constexpr (NC) return bf2f(f2bf(acc[j][i][r]));
      return acc[j][i][r];
    }
  };

  // Fragment addressing: at k-step kk lane (row li, k-half g) reads logical
  // chunk 2*kk + g of its row, at its swizzled position (rows 32*x + li all
  // share li's swizzle).
  constexpr int KS = Cfg::KSTEPS;
  static_assert(KS % 2 == 0, "the last k-step of a slab is in set 1");
  int pos[KS];
#pragma unroll
  for (int kk = 0; kk < KS; ++kk) pos[kk] = chunk_pos<RB>(2 * kk + g, li) * 16;
  const int rowA = (wm * Cfg::WM + li) * RB, rowB = (wn * Cfg::WN + li) * RB;

  frag_t fa0[TM], fb0[TN], fa1[TM], fb1[TN];
  // Reads in the order the MFMAs consume them: fb[0], fa[0..TM), fb[1..TN);
  // read x of that order for x in [x0, x1).
  auto read_part = [&](uint32_t soff, int pos, frag_t *fa, frag_t *fb, int x0, int x1) {
    const uint8_t *slot = smem + soff;
#pragma unroll
    for (int x = 0; x < TM + TN; ++x) {
      if (x < x0 || x >= x1) continue;
      if (x == 0)
        fb[0] = *(const frag_t *)(slot + Cfg::A_BYTES + rowB + pos);
      else if (x <= TM)
        fa[x - 1] = *(const frag_t *)(slot + rowA + (x - 1) * 32 * RB + pos);
      else
        fb[x - TM] = *(const frag_t *)(slot + Cfg::A_BYTES + rowB + (x - TM) * 32 * RB + pos);
    }
  };
  auto read_set = [&](uint32_t soff, int pos, frag_t *fa, frag_t *fb) {
    read_part(soff, pos, fa, fb, 0, TM + TN);
  };
  auto mfma_set = [&](const frag_t *fa, const frag_t *fb) {
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int i = 0; i < TM; ++i) acc[j][i] = PT::mfma(fb[j], fa[i], acc[j][i]);
  };
  // MFMAs and the LDS reads of the other set, one read after each of the
  // first TM + TN MFMAs.
  auto interleave = []() {
#pragma unroll
    for (int x = 0; x < TM + TN; ++x) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
    }
    __builtin_amdgcn_sched_group_barrier(0x008, TM * TN - (TM + TN), 0);
  };

  // The epilogue of a bf16 C without a residual, block by block (k = j * TM
  // + i): each column block's bias (and wscale) is read once for its TM row
  // blocks; a block goes through the bias (dequantisation), the activation and
  // the bf16 narrowing in registers, then crosses the wave's 2 KB staging
  // area. The round trips are software-pipelined: block k is written right
  // after block k - 1's read-back is issued (a wave's LDS operations execute
  // in order, so the write cannot overtake the read), and only block k - 1's
  // global stores wait for its read-back, while block k's arithmetic runs
  // under it.
  auto epilogue_bf = [&](int ti) {
    int m0, n0;
    tile_origin(ti, m0, n0);
    const float *bl = (const float *)(smem + Cfg::BIAS_OFF + (ti & 1) * BN * 4);
    const float *wsl = (const float *)(smem + Cfg::WS_OFF + (ti & 1) * BN * 4);
    const float *sal = (const float *)(smem + Cfg::SA_OFF + (ti & 1) * BM * 4);
    uint8_t *stg = smem + Cfg::STG_OFF + wave * Cfg::STG_WAVE;
    // C's columns per accumulator column (GLU: half).
    constexpr int CD = GLU ? 2 : 1;
    const int NC = N / CD;
    // Staging: lane (li, g) writes its 8 bytes of chunk q of row li at
    // position q ^ ((li >> 2) & 3); lane l reads chunk c = l & 3 of rows
    // r * 16 + l / 4, 16 bytes each, and stores them. Block k covers C's
    // columns [cl, cl + 32) of row block i (GLU: column blocks 2j and 2j + 1
    // of the accumulators).
    auto store = [&](int k, const uint4 *w) {
      const int j = k / TM, i = k % TM;
      const int rbase = m0 + wm * Cfg::WM + i * 32;
      const int cl = (n0 + wn * Cfg::WN) / CD + j * 32;
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int row = r * 16 + (lane >> 2), c = lane & 3;
        const int grow = rbase + row, gcol = cl + c * 8;
        if (grow < M && gcol < NC) {
          const int64_t off = (int64_t)grow * ldc + gcol;
          if (gcol + 8 <= NC)
            *(uint4 *)((uint16_t *)C + off) = w[r];
          else  // N % 8 == 4: four columns left
            *(uint2 *)((uint16_t *)C + off) = make_uint2(w[r].x, w[r].y);
        }
      }
    };
    // The epilogue's value of accumulator (j, i) element q * 4 + e: the bias
    // (dequantisation) added, before the activation.
    auto pre = [&](int j, int i, int q, int e, float bb, float ww, float sa) {
      if (I8) return __builtin_fmaf(__fmul_rn(accf(j, i, q * 4 + e), sa), ww, bb);
      return accf(j, i, q * 4 + e) + bb;
    };
    float4 b[4], w[4];
    uint4 wv[2];
    constexpr int NB = TM * TN / CD;  // staged blocks
#pragma unroll
    for (int k = 0; k < NB; ++k) {
      const int j = k / TM, i = k % TM;
      uint32_t pk[8];  // columns 8q + 4g + 2h, +1 of row li: pk[2q + h]
      if constexpr (GLU) {
        // Columns 16u + e (lo) and 16u + 8 + e (hi) of accumulator block
        // 2j + jj give C's column 8(2jj + u) + e: each pair rounds to bf16 as
        // the unfused GEMM's C does, then lo * act(hi) rounds once more.
        const float sa = I8 ? sal[wm * Cfg::WM + i * 32 + li] : 0.0f;
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
          const int ja = 2 * j + jj;
          const int cl = wn * Cfg::WN + ja * 32;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            b[q] = has_bias ? *(const float4 *)(bl + cl + q * 8 + g * 4)
                            : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (I8) w[q] = *(const float4 *)(wsl + cl + q * 8 + g * 4);
          }
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const float bl4[4] = {b[2 * u].x, b[2 * u].y, b[2 * u].z, b[2 * u].w};
            const float bh4[4] = {b[2 * u + 1].x, b[2 * u + 1].y, b[2 * u + 1].z,
                                  b[2 * u + 1].w};
            const float wl4[4] = {w[2 * u].x, w[2 * u].y, w[2 * u].z, w[2 * u].w};
            const float wh4[4] = {w[2 * u + 1].x, w[2 * u + 1].y, w[2 * u + 1].z,
                                  w[2 * u + 1].w};
            float o[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const uint32_t h = pack_bf2_hw(pre(ja, i, 2 * u, e, bl4[e], wl4[e], sa),
                                             pre(ja, i, 2 * u + 1, e, bh4[e], wh4[e], sa));
              o[e] = bf2f(h & 0xFFFFu) * glu_act<GACT>(bf2f(h >> 16));
            }
            pk[2 * (2 * jj + u)] = pack_bf2(o[0], o[1]);
            pk[2 * (2 * jj + u) + 1] = pack_bf2(o[2], o[3]);
          }
        }
      } else {
        if (i == 0) {
          const int cl = wn * Cfg::WN + j * 32;  // tile-local first column
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            b[q] = has_bias ? *(const float4 *)(bl + cl + q * 8 + g * 4)
                            : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (I8) w[q] = *(const float4 *)(wsl + cl + q * 8 + g * 4);
          }
        }
        const float sa = I8 ? sal[wm * Cfg::WM + i * 32 + li] : 0.0f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float bb[4] = {b[q].x, b[q].y, b[q].z, b[q].w};
          const float ww[4] = {w[q].x, w[q].y, w[q].z, w[q].w};
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e)
            v[e] = gemm_epilogue(pre(j, i, q, e, bb[e], ww[e], sa), EPA);
          pk[2 * q] = pack_bf2_hw(v[0], v[1]);
          pk[2 * q + 1] = pack_bf2_hw(v[2], v[3]);
        }
      }
#pragma unroll
      for (int q = 0; q < 4; ++q)
        *(uint2 *)(stg + li * 64 + ((q ^ ((li >> 2) & 3)) * 16 + g * 8)) =
            make_uint2(pk[2 * q], pk[2 * q + 1]);
      if (k > 0) store(k - 1, wv);
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int row = r * 16 + (lane >> 2), c = lane & 3;
        wv[r] = *(const uint4 *)(stg + row * 64 + ((c ^ ((row >> 2) & 3)) * 16));
      }
    }
    store(NB - 1, wv);
  };

  // The epilogue of an fp32 C with a residual (C = epi(A W + b) + R, R may be
  // C itself), block by block (k = i * TN + j), each block staged as two
  // 16-row halves (2.25 KB per wave, which leaves LDS for two 64 KB slots):
  // block k + 1's residual rows are loaded while block k goes through the
  // bias (dequantisation), the activation and the staging, so the loads'
  // latency is paid once per tile instead of once per block. Rows of
  // different blocks are disjoint, so loading block k + 1's residual before
  // storing block k is exact also in place.
  auto epilogue_res = [&](int ti) {
    int m0, n0;
    tile_origin(ti, m0, n0);
    const float *bl = (const float *)(smem + Cfg::BIAS_OFF + (ti & 1) * BN * 4);
    const float *wsl = (const float *)(smem + Cfg::WS_OFF + (ti & 1) * BN * 4);
    const float *sal = (const float *)(smem + Cfg::SA_OFF + (ti & 1) * BM * 4);
    uint8_t *stg = smem + Cfg::STG_OFF + wave * Cfg::STG_WAVE;
    // Half h of a block: lane l reads (and stores) row 16h + l / 4, columns
    // (l % 4) * 8 + 4 * part .. + 3, part = 0, 1.
    auto load_res = [&](int k, float4 *rv) {
      const int i = k / TN, j = k % TN;
      const int rbase = m0 + wm * Cfg::WM + i * 32;
      const int cl = wn * Cfg::WN + j * 32;
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int part = 0; part < 2; ++part) {
          const int grow = rbase + h * 16 + (lane >> 2);
          const int gcol = n0 + cl + (lane & 3) * 8 + part * 4;
          rv[h * 2 + part] = grow < M && gcol < N
                                 ? *(const float4 *)(residual + (int64_t)grow * ldc + gcol)
                                 : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
    };
    float4 rcur[4], rnext[4];
    load_res(0, rcur);
#pragma unroll
    for (int k = 0; k < TM * TN; ++k) {
      const int i = k / TN, j = k % TN;
      if (k + 1 < TM * TN) load_res(k + 1, rnext);
      const int rbase = m0 + wm * Cfg::WM + i * 32;
      const int cl = wn * Cfg::WN + j * 32;
      const float sa = I8 ? sal[wm * Cfg::WM + i * 32 + li] : 0.0f;
      float4 vq[4];  // columns 8q + 4g .. + 3 of row li
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float4 b = has_bias ? *(const float4 *)(bl + cl + q * 8 + g * 4)
                                  : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        float4 v;
        if (I8) {
          const float4 w = *(const float4 *)(wsl + cl + q * 8 + g * 4);
          v.x = gemm_epilogue(
              __builtin_fmaf(__fmul_rn((float)acc[j][i][q * 4 + 0], sa), w.x, b.x), EPB);
          v.y = gemm_epilogue(
              __builtin_fmaf(__fmul_rn((float)acc[j][i][q * 4 + 1], sa), w.y, b.y), EPB);
          v.z = gemm_epilogue(
              __builtin_fmaf(__fmul_rn((float)acc[j][i][q * 4 + 2], sa), w.z, b.z), EPB);
          v.w = gemm_epilogue(
              __builtin_fmaf(__fmul_rn((float)acc[j][i][q * 4 + 3], sa), w.w, b.w), EPB);
        } else {
          v.x = gemm_epilogue(acc[j][i][q * 4 + 0] + b.x, EPB);
          v.y = gemm_epilogue(acc[j][i][q * 4 + 1] + b.y, EPB);
          v.z = gemm_epilogue(acc[j][i][q * 4 + 2] + b.z, EPB);
          v.w = gemm_epilogue(acc[j][i][q * 4 + 3] + b.w, EPB);
        }
        vq[q] = v;
      }
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        if ((li >> 4) == h) {
#pragma unroll
          for (int q = 0; q < 4; ++q)
            *(float4 *)(stg + (li & 15) * STG_ROWB + (q * 8 + g * 4) * 4) = vq[q];
        }
        asm volatile("" ::: "memory");
#pragma unroll
        for (int part = 0; part < 2; ++part) {
          const int row = lane >> 2, c4 = (lane & 3) * 8 + part * 4;
          float4 x = *(const float4 *)(stg + row * STG_ROWB + c4 * 4);
          const int grow = rbase + h * 16 + row, gcol = n0 + cl + c4;
          if (grow < M && gcol < N) {
            const float4 r = rcur[h * 2 + part];
            x.x += r.x;
            x.y += r.y;
            x.z += r.z;
            x.w += r.w;
            *(float4 *)((float *)C + (int64_t)grow * ldc + gcol) = x;
          }
        }
        asm volatile("" ::: "memory");
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) rcur[r] = rnext[r];
    }
  };

  // The epilogue of this block's ti-th tile.
  auto epilogue = [&](int ti) {
    if constexpr (CBF && !RES) {
      epilogue_bf(ti);
      return;
    }
    if constexpr (RES && !CBF) {
      epilogue_res(ti);
      return;
    }
    int m0, n0;
    tile_origin(ti, m0, n0);
    const float *bl = (const float *)(smem + Cfg::BIAS_OFF + (ti & 1) * BN * 4);
    const float *wsl = (const float *)(smem + Cfg::WS_OFF + (ti & 1) * BN * 4);
    const float *sal = (const float *)(smem + Cfg::SA_OFF + (ti & 1) * BM * 4);
    uint8_t *stg = smem + Cfg::STG_OFF + wave * Cfg::STG_WAVE;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int rbase = m0 + wm * Cfg::WM + i * 32;
      float sa = 0.0f;
      if (I8 && !RAW) sa = sal[wm * Cfg::WM + i * 32 + li];
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int cl = wn * Cfg::WN + j * 32;  // tile-local first column
        // acc layout -> staging rows (lane li's row, columns 8q + 4g + e).
        // bf16 C without a residual stages packed bf16 (2 KB per block): lane
        // (li, g) writes its four columns 8q + 4g .. +3 of row li as 8 bytes,
        // 16-byte chunk q of the 64-byte row stored at q ^ ((li >> 2) & 3), so
        // the writes of 16 rows and the reads of 4 rows x 4 chunks each cover
        // all 64 banks once. Everything else stages fp32 rows (the residual is
        // added before the one rounding).
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          float4 v;
          if (RAW) {
            v.x = __int_as_float((int)acc[j][i][q * 4 + 0]);
            v.y = __int_as_float((int)acc[j][i][q * 4 + 1]);
            v.z = __int_as_float((int)acc[j][i][q * 4 + 2]);
            v.w = __int_as_float((int)acc[j][i][q * 4 + 3]);
          } else if (I8) {
            const float4 b = has_bias ? *(const float4 *)(bl + cl + q * 8 + g * 4)
                                      : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            const float4 w = *(const float4 *)(wsl + cl + q * 8 + g * 4);
            v.x = gemm_epilogue(__builtin_fmaf(__fmul_rn(accf(j, i, q * 4 + 0), sa), w.x, b.x),
                                EPB);
            v.y = gemm_epilogue(__builtin_fmaf(__fmul_rn(accf(j, i, q * 4 + 1), sa), w.y, b.y),
                                EPB);
            v.z = gemm_epilogue(__builtin_fmaf(__fmul_rn(accf(j, i, q * 4 + 2), sa), w.z, b.z),
                                EPB);
            v.w = gemm_epilogue(__builtin_fmaf(__fmul_rn(accf(j, i, q * 4 + 3), sa), w.w, b.w),
                                EPB);
          } else {
            const float4 b = *(const float4 *)(bl + cl + q * 8 + g * 4);
            v.x = gemm_epilogue(accf(j, i, q * 4 + 0) + b.x, EPB);
            v.y = gemm_epilogue(accf(j, i, q * 4 + 1) + b.y, EPB);
            v.z = gemm_epilogue(accf(j, i, q * 4 + 2) + b.z, EPB);
            v.w = gemm_epilogue(accf(j, i, q * 4 + 3) + b.w, EPB);
          }
          if (STG_BF) {
            const uint2 w = make_uint2(pack_bf2_hw(v.x, v.y), pack_bf2_hw(v.z, v.w));
            *(uint2 *)(stg + li * 64 + ((q ^ ((li >> 2) & 3)) * 16 + g * 8)) = w;
          } else {
            *(float4 *)(stg + li * STG_ROWB + (q * 8 + g * 4) * 4) = v;
          }
        }
        asm volatile("" ::: "memory");
        if (STG_BF) {
          // 8 bf16 per lane; 4 lanes per 32-column row.
#pragma unroll
          for (int r = 0; r < 2; ++r) {
            const int row = r * 16 + (lane >> 2), c = lane & 3;
            const uint4 w = *(const uint4 *)(stg + row * 64 + ((c ^ ((row >> 2) & 3)) * 16));
            const int grow = rbase + row, gcol = n0 + cl + c * 8;
            if (grow < M && gcol < N) {
              const int64_t off = (int64_t)grow * ldc + gcol;
              if (gcol + 8 <= N)
                *(uint4 *)((uint16_t *)C + off) = w;
              else  // N % 8 == 4: four columns left
                *(uint2 *)((uint16_t *)C + off) = make_uint2(w.x, w.y);
            }
          }
        } else if (CBF) {
          // 8 fp32 per lane -> 16 bytes of bf16; 4 lanes per 32-column row.
#pragma unroll
          for (int r = 0; r < 2; ++r) {
            const int row = r * 16 + (lane >> 2), c8 = (lane & 3) * 8;
            const float4 x0 = *(const float4 *)(stg + row * STG_ROWB + c8 * 4);
            const float4 x1 = *(const float4 *)(stg + row * STG_ROWB + c8 * 4 + 16);
            const int grow = rbase + row, gcol = n0 + cl + c8;
            if (grow < M && gcol < N) {
              float y[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
              const int64_t off = (int64_t)grow * ldc + gcol;
              const bool full = gcol + 8 <= N;  // else N % 8 == 4: four columns left
              if (RES) {
                const float4 r0 = *(const float4 *)(residual + off);
                y[0] += r0.x;
                y[1] += r0.y;
                y[2] += r0.z;
                y[3] += r0.w;
                if (full) {
                  const float4 r1 = *(const float4 *)(residual + off + 4);
                  y[4] += r1.x;
                  y[5] += r1.y;
                  y[6] += r1.z;
                  y[7] += r1.w;
                }
              }
              uint4 w;
              w.x = pack_bf2_hw(y[0], y[1]);
              w.y = pack_bf2_hw(y[2], y[3]);
              w.z = pack_bf2_hw(y[4], y[5]);
              w.w = pack_bf2_hw(y[6], y[7]);
              if (full)
                *(uint4 *)((uint16_t *)C + off) = w;
              else
                *(uint2 *)((uint16_t *)C + off) = make_uint2(w.x, w.y);
            }
          }
        } else {
          // 4 fp32 (or raw int32) per lane; 8 lanes per 32-column row.
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int row = r * 8 + (lane >> 3), c4 = (lane & 7) * 4;
            float4 x = *(const float4 *)(stg + row * STG_ROWB + c4 * 4);
            const int grow = rbase + row, gcol = n0 + cl + c4;
            if (grow < M && gcol < N) {
              const int64_t off = (int64_t)grow * ldc + gcol;
              if (RES) {
                const float4 rv = *(const float4 *)(residual + off);
                x.x += rv.x;
                x.y += rv.y;
                x.z += rv.z;
                x.w += rv.w;
              }
              *(float4 *)((float *)C + off) = x;
            }
          }
        }
        asm volatile("" ::: "memory");
      }
    }
  };

  // Prologue: slabs 0 .. NS-1 in flight; k-step 0 of slab 0 into set 0. Only
  // slab 0 is waited for here (with the tile's epilogue vectors, issued with
  // it): this wave's loads of slabs 1 .. NS-1 -- all in the first tile, which
  // has at least NS slabs, so no epilogue vectors among them -- stay in
  // flight, and the main loop waits for slab 1 before its first barrier.
#pragma unroll
  for (int s = 0; s < NS; ++s)
    if (s < nslab) issue();
  if (nslab >= NS) {
    if (SAME_LOADS_P || wave < Cfg::NHI)
      wait_vmcnt<Cfg::LOADS_HI *(NS - 1)>();
    else
      wait_vmcnt<Cfg::LOADS_LO *(NS - 1)>();
  } else {
    wait_vmcnt<0>();
  }
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  read_set(0, pos[0], fa0, fb0);

  // An epilogue issues EPI_STORES global stores per wave (one per staged row
  // group of each 32 x 32 block) when its tile lies wholly inside C, where
  // every store is taken. Those stores are younger than the loads of the next
  // NS - 1 slabs, so the waits for those slabs leave them in flight instead of
  // stalling the next tile on the previous one's write acknowledgements. An
  // edge tile (or a residual epilogue, whose loads the compiler waits on)
  // keeps the exact wait.
  constexpr int EPI_STORES = RES ? 0 : (GLU ? 1 : CBF ? 2 : 4) * TM * TN;
  static_assert(Cfg::LOADS_HI * (NS - 2) + EPI_STORES < 64, "vmcnt holds at most 63");
  constexpr bool SAME_LOADS = Cfg::LOADS_HI == Cfg::LOADS_LO;
  int epi_left = 0;
  int ep_kt = 0, ep_ti = 0;  // tile and depth of slab s
  uint32_t rd_slot = 0;      // byte offset of slab s's slot
  for (int s = 0; s < nslab; ++s) {
    // k-steps 0 .. KS-2 of slab s: each one's MFMAs run while the next
    // k-step's fragments are read into the other set.
#pragma unroll
    for (int kk = 0; kk + 1 < KS; ++kk) {
      if (kk % 2 == 0) {
        mfma_set(fa0, fb0);
        read_set(rd_slot, pos[kk + 1], fa1, fb1);
      } else {
        mfma_set(fa1, fb1);
        read_set(rd_slot, pos[kk + 1], fa0, fb0);
      }
      interleave();
      __builtin_amdgcn_sched_barrier(0);
    }
    // Every read of slab s is now issued. Wait for them and for this wave's
    // loads of slab s + 1 (the slabs issued after it, at most NS - 2, may stay
    // in flight), then meet: slab s + 1 is in LDS and slot s % NS is free.
    const uint32_t nx_slot = rd_slot + Cfg::SLOT == NS * Cfg::SLOT ? 0 : rd_slot + Cfg::SLOT;
    const int ahead = nslab - 2 - s;
    const bool stores_young = EPI_STORES > 0 && epi_left > 0;
    if (ahead >= NS - 2 && !stores_young) {
      if (SAME_LOADS || wave < Cfg::NHI)
        wait_vmcnt<Cfg::LOADS_HI *(NS - 2)>();
      else
        wait_vmcnt<Cfg::LOADS_LO *(NS - 2)>();
    } else if (SAME_LOADS || wave < Cfg::NHI) {
      wait_slab<Cfg::LOADS_HI, NS, EPI_STORES>(ahead, stores_young);
    } else {
      wait_slab<Cfg::LOADS_LO, NS, EPI_STORES>(ahead, stores_young);
    }
    if (epi_left > 0) --epi_left;
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    // The last k-step of slab s (set 1: KS is even); k-step 0 of slab s + 1
    // is read meanwhile, in consumption order (after the last slab, slab s
    // again: in bounds, unused): the first TM reads beside the j = 0 MFMAs,
    // the rest after the loads of slab s + NS are issued -- those keep the
    // matrix pipe busy while the scalar unit addresses the loads.
    const uint32_t rs = s + 1 < nslab ? nx_slot : rd_slot;
#pragma unroll
    for (int i = 0; i < TM; ++i) acc[0][i] = PT::mfma(fb1[0], fa1[i], acc[0][i]);
    read_part(rs, pos[0], fa0, fb0, 0, TM);
#pragma unroll
    for (int x = 0; x < TM; ++x) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (s + NS < nslab) issue();  // slab s + NS
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 1; j < TN; ++j)
#pragma unroll
      for (int i = 0; i < TM; ++i) acc[j][i] = PT::mfma(fb1[j], fa1[i], acc[j][i]);
    read_part(rs, pos[0], fa0, fb0, TM, TM + TN);
    {
      constexpr int NM = TM * (TN - 1), NR = TN, NP = NM < NR ? NM : NR;
#pragma unroll
      for (int x = 0; x < NP; ++x) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      if (NM > NP) __builtin_amdgcn_sched_group_barrier(0x008, NM - NP, 0);
      if (NR > NP) __builtin_amdgcn_sched_group_barrier(0x100, NR - NP, 0);
    }
    rd_slot = nx_slot;
    if (++ep_kt == nk) {
      ep_kt = 0;
      {
        int m0, n0;
        tile_origin(ep_ti, m0, n0);
        epi_left = (m0 + BM <= M && n0 + BN <= N) ? NS - 1 : 0;
      }
      epilogue(ep_ti++);
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[j][i][r] = 0;
    }
  }
}

}  // namespace mxlds
