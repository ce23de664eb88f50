// k_attn.hip -- fused masked attention on gfx950 MFMA: QK^T, additive-mask
// softmax and PV in one pass per (sequence, head, 128-query tile); the score
// matrix never reaches HBM. Two kernels share the design below: attn_dma_k
// (K, V and the mask reach LDS by direct loads through a ring of slots, and
// V^T is read with the transposing ds_read_b64_tr_b16) and attn_fwd_k (a qkv
// too long for 32-bit row offsets: K and V staged through registers, V
// transposed on the way into LDS).
//
// Each of the 4 waves owns 32 queries and computes the TRANSPOSED score tile
// S^T = K Q^T with v_mfma_f32_32x32x16_bf16 (keys on rows, queries on
// columns), so every lane holds 16 scores of ONE query: the row max and sum of
// the online softmax are lane-local plus one exchange with lane^32, and the
// rescale of the running output is a per-lane scalar. The output is kept as
// O^T = V^T P^T: the probabilities go straight from the score accumulator into
// the B operand (converted to bf16) -- the keys a lane holds are a fixed
// permutation of the MFMA's k index, and the A operand (V^T, from LDS) is read
// in that same permutation, so no shuffle is needed.
//
// K is staged row-major in LDS, V transposed (Vt[hd][key], via a 4x4 register
// transpose on the way in), both double-buffered with the mask tile; the next
// 64-key tile is fetched into registers while the current one is consumed.
// Softmax runs in the log2 domain (scores * scale * log2e, mask * log2e) with
// the hardware exp2. Keys at or past kv_len[b] are skipped (whole tiles) or
// given -inf (inside the last tile); -1e30 mask entries stay finite, so a row
// whose keys are all masked attends uniformly, as the host softmax does.
//
// VALU economy (the softmax, not the MFMAs, bounds this kernel): a key tile
// whose mask entries are all zero -- a block-uniform flag set while the tile
// is staged -- skips the per-score mask add and takes its max on the raw
// scores (scale > 0), and each probability is one FMA into exp2. The running
// max m moves (and O and l are rescaled) only when a tile's max exceeds it by
// more than 8 in log2 units, so probabilities stay below 2^8 and most tiles
// skip the rescale; the result O / l is the same quotient.
#include "mx_common.hpp"
#include "mx_kernels.hpp"

using namespace mxd;

namespace {

constexpr int BQ = 128, BKV = 64;

template <int HD>
__global__ __launch_bounds__(256, 3) void attn_fwd_k(const uint16_t *__restrict__ qkv, int64_t ldq,
                                                  int S, int H, float scale_log2e,
                                                  const float *__restrict__ add_mask,
                                                  const int32_t *__restrict__ kv_len,
                                                  uint16_t *__restrict__ ctx, int64_t ldo,
                                                  int n_qblk, int force_logits,
                                                  const int32_t *__restrict__ seq_start,
                                                  const int32_t *__restrict__ order) {
  constexpr int KS = HD + 8;   // K row stride in LDS (elements)
  constexpr int VS = BKV + 4;  // Vt row stride in LDS (elements)
  constexpr int KCH = BKV * HD / 8 / 256;  // 16-byte K chunks per thread (1 or 2)
  constexpr int VBLK = (BKV / 4) * (HD / 4);  // 4x4 V blocks per tile (128 or 256)
  constexpr int NKK = HD / 16;
  constexpr int NHT = HD / 32;
  static_assert(KCH >= 1, "tile too small");
  __shared__ __attribute__((aligned(16))) uint16_t sK[2][BKV * KS];
  __shared__ __attribute__((aligned(16))) uint16_t sV[2][HD * VS];
  __shared__ float sM[2][BKV];
  __shared__ int sF[2];  // 1 if the staged tile has a nonzero mask entry

  // Block -> (sequence, query block, head). With an order (sequences by
  // decreasing kv_len), the blocks of the longest sequences are dispatched
  // first and the short ones fill in behind them; otherwise sequence-major.
  const int blk = blockIdx.x;
  int qb, h, b;
  if (order) {
    h = blk % H;
    const int t = blk / H;
    qb = t % n_qblk;
    b = order[t / n_qblk];
  } else {
    qb = blk % n_qblk;
    const int bh = blk / n_qblk;
    h = bh % H;
    b = bh / H;
  }
  const int d = H * HD;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 5, li = lane & 31;
  int kvl = kv_len ? kv_len[b] : S;
  kvl = kvl < 1 ? 1 : (kvl > S ? S : kvl);
  // Dense rows: sequence b is rows b*S .. b*S + S - 1, every query is
  // computed and keys past kv_len are read but weighted 0. Packed rows: only
  // the sequence's kv_len rows exist, so queries and keys stop there (a key
  // past it would be the next sequence's row).
  const int64_t row0 = seq_start ? (int64_t)seq_start[b] : (int64_t)b * S;
  const int lim = seq_start ? kvl : S;
  if (qb * BQ >= lim) return;
  const uint16_t *base = qkv + row0 * ldq;

  // Q fragments: B operand of S^T = K Q^T (column = query, k = head dim).
  const int q = qb * BQ + wave * 32 + li;
  bf16x8 qf[NKK];
#pragma unroll
  for (int kk = 0; kk < NKK; ++kk) {
    uint4 v = make_uint4(0, 0, 0, 0);
    if (q < lim) v = *(const uint4 *)(base + (int64_t)q * ldq + h * HD + kk * 16 + g * 8);
    qf[kk] = __builtin_bit_cast(bf16x8, v);
  }

  // Register staging of one K/V/mask tile.
  uint4 rk[KCH];
  uint2 rv[4];
  float rm = 0.0f;
  const int vkb = tid & 15, vhb = tid >> 4;  // 4x4 block: keys vkb*4.., dims vhb*4..
  auto gload = [&](int t) {
    const int k0 = t * BKV;
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      const int c = tid + i * 256, key = c / (HD / 8), c8 = (c % (HD / 8)) * 8;
      rk[i] = (k0 + key < lim)
                  ? *(const uint4 *)(base + (int64_t)(k0 + key) * ldq + d + h * HD + c8)
                  : make_uint4(0, 0, 0, 0);
    }
    if (tid < VBLK) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = k0 + vkb * 4 + r;
        rv[r] = key < lim ? *(const uint2 *)(base + (int64_t)key * ldq + 2 * d + h * HD + vhb * 4)
                        : make_uint2(0, 0);
      }
    }
    if (tid < BKV) {
      const int key = k0 + tid;
      rm = key < kvl ? (add_mask ? add_mask[(int64_t)b * S + key] * 1.4426950408889634f : 0.0f)
                     : -INFINITY;
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      const int c = tid + i * 256, key = c / (HD / 8), c8 = (c % (HD / 8)) * 8;
      *(uint4 *)&sK[buf][key * KS + c8] = rk[i];
    }
    if (tid < VBLK) {
      // rows r (keys) x 4 dims -> 4 dims x 4 keys
      const uint32_t r0l = rv[0].x, r0h = rv[0].y, r1l = rv[1].x, r1h = rv[1].y;
      const uint32_t r2l = rv[2].x, r2h = rv[2].y, r3l = rv[3].x, r3h = rv[3].y;
      uint2 c0, c1, c2, c3;
      c0.x = (r0l & 0xFFFFu) | (r1l << 16);
      c0.y = (r2l & 0xFFFFu) | (r3l << 16);
      c1.x = (r0l >> 16) | (r1l & 0xFFFF0000u);
      c1.y = (r2l >> 16) | (r3l & 0xFFFF0000u);
      c2.x = (r0h & 0xFFFFu) | (r1h << 16);
      c2.y = (r2h & 0xFFFFu) | (r3h << 16);
      c3.x = (r0h >> 16) | (r1h & 0xFFFF0000u);
      c3.y = (r2h >> 16) | (r3h & 0xFFFF0000u);
      uint16_t *vt = &sV[buf][(vhb * 4) * VS + vkb * 4];
      *(uint2 *)(vt) = c0;
      *(uint2 *)(vt + VS) = c1;
      *(uint2 *)(vt + 2 * VS) = c2;
      *(uint2 *)(vt + 3 * VS) = c3;
    }
    if (tid < BKV) {  // exactly wave 0
      sM[buf][tid] = rm;
      const bool any = __ballot(rm != 0.0f) != 0;
      if (tid == 0) sF[buf] = any || force_logits;
    }
  };

  f32x16 o[NHT];
#pragma unroll
  for (int t = 0; t < NHT; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[t][r] = 0.0f;
  float m_run = -INFINITY, l_run = 0.0f;

  const int ntile = (kvl + BKV - 1) / BKV;
  // A wave whose 32 queries all lie past the sequence's rows (the last query
  // block of a packed sequence) only helps stage K/V and meets the barriers;
  // its SIMD time goes to the other blocks on the CU.
  const bool live = qb * BQ + wave * 32 < lim;
  gload(0);
  sstore(0);
  __syncthreads();
  for (int t = 0; t < ntile; ++t) {
    const int cur = t & 1;
    if (t + 1 < ntile) gload(t + 1);
    if (!live) {
      if (t + 1 < ntile) sstore(cur ^ 1);
      __syncthreads();
      continue;
    }

    // S^T for the two 32-key halves of the tile.
    f32x16 sc[2];
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
#pragma unroll
      for (int r = 0; r < 16; ++r) sc[sub][r] = 0.0f;
#pragma unroll
      for (int kk = 0; kk < NKK; ++kk) {
        const bf16x8 kf = *(const bf16x8 *)&sK[cur][(sub * 32 + li) * KS + kk * 16 + g * 8];
        sc[sub] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[kk], sc[sub], 0, 0, 0);
      }
    }
    // Tile max of this lane's query, in log2 units. A tile with a nonzero
    // mask entry turns its scores into logits first (scale and mask); a
    // mask-free tile keeps the raw scores and scales the max.
    float mx = -INFINITY, cc;
    if (sF[cur]) {
#pragma unroll
      for (int sub = 0; sub < 2; ++sub)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = sub * 32 + (r >> 2) * 8 + g * 4 + (r & 3);
          const float v = __builtin_fmaf(sc[sub][r], scale_log2e, sM[cur][key]);
          sc[sub][r] = v;
          mx = fmaxf(mx, v);
        }
      cc = 1.0f;
    } else {
#pragma unroll
      for (int sub = 0; sub < 2; ++sub)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sc[sub][r]);
      mx *= scale_log2e;
      cc = scale_log2e;
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    if (mx > m_run + 8.0f) {
      const float alpha = __builtin_amdgcn_exp2f(m_run - mx);
      m_run = mx;
      l_run *= alpha;
#pragma unroll
      for (int ht = 0; ht < NHT; ++ht)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[ht][r] *= alpha;
    }

    // Probabilities exp2(s * cc - m) -> bf16 B operands, one per 16-key chunk.
    bf16x8 pk[4];
    float ps = 0.0f;
#pragma unroll
    for (int ch = 0; ch < 4; ++ch) {
      const int sub = ch >> 1, c = ch & 1;
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) {
        const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[sub][c * 8 + jj], cc, -m_run));
        ps += p;
        pk[ch][jj] = (__bf16)p;
      }
    }
    l_run += ps;

    // O^T += V^T P^T over the tile's 4 chunks of 16 keys.
#pragma unroll
    for (int ch = 0; ch < 4; ++ch) {
      const int sub = ch >> 1, c = ch & 1;
      const int kb = sub * 32 + c * 16 + g * 4;
#pragma unroll
      for (int ht = 0; ht < NHT; ++ht) {
        const uint16_t *vr = &sV[cur][(ht * 32 + li) * VS];
        const uint2 lo = *(const uint2 *)(vr + kb);
        const uint2 hi = *(const uint2 *)(vr + kb + 8);
        const uint4 vv = make_uint4(lo.x, lo.y, hi.x, hi.y);
        o[ht] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, vv), pk[ch],
                                                        o[ht], 0, 0, 0);
      }
    }

    if (t + 1 < ntile) sstore(cur ^ 1);
    __syncthreads();
  }

  const float l = l_run + __shfl_xor(l_run, 32);
  const float inv = 1.0f / l;
  if (q < lim) {
    uint16_t *dst = ctx + (row0 + q) * ldo + h * HD;
#pragma unroll
    for (int ht = 0; ht < NHT; ++ht)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int hd0 = ht * 32 + r4 * 8 + g * 4;
        uint2 w;
        w.x = pack_bf2(o[ht][r4 * 4 + 0] * inv, o[ht][r4 * 4 + 1] * inv);
        w.y = pack_bf2(o[ht][r4 * 4 + 2] * inv, o[ht][r4 * 4 + 3] * inv);
        *(uint2 *)(dst + hd0) = w;
      }
  }
}


// ---- K, V and the mask through a ring of LDS slots ------------------------------
//
// The same block and wave roles and the same softmax as attn_fwd_k, with the
// key tiles staged differently: K, V and the tile's mask row go global -> LDS
// by direct loads (global_load_lds_dwordx4 / _dword, issued from inline
// assembly so the compiler adds no waits) into a ring of NSL slots, NSL - 1
// tiles ahead, and V stays row-major in LDS: the PV operand V^T is read with
// ds_read_b64_tr_b16, which hands each lane of a 16-lane group one column of
// the 4 x 16 bf16 block the group addresses (lane j of the group receives
// element j % 4 of group lane 4e + j / 4's 8 bytes, e = 0..3). No registers
// hold K or V in flight and no VALU transposes them.
//
// LDS rows are head_dim bf16: 128 bytes (head_dim 64) or 64 bytes (32).
// 16-byte chunk c of K row r is stored at c ^ ((r >> 1) & 7) (128-byte rows)
// or c ^ ((r >> 2) & 3) (64-byte rows), so sixteen ds_read_b128 rows r..r+15
// hit sixteen bank groups. V chunks of 128-byte rows are stored at
// c ^ ((r & 2) << 1): the 32 lanes of a ds_read_b64_tr_b16 phase read rows
// k0..k0+3 of two 16-column groups, row parity picks a 32-bank half and the
// XOR separates rows k0 and k0 + 2; 64-byte rows k0..k0+3 already start in
// four different 16-bank quarters. Rows past the sequence's last are fetched
// from that last row (in bounds) and carry probability 0.
constexpr int NSL = 3;

__device__ __forceinline__ void dma16o(uint64_t base, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds), "v"(voff),
               "s"(base)
               : "memory");
}
__device__ __forceinline__ void dma4o(uint64_t base, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, %2" ::"s"(lds), "v"(voff),
               "s"(base)
               : "memory");
}
__device__ __forceinline__ uint64_t uni64(uint64_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return ((uint64_t)hi << 32) | lo;
}
template <int N>
__device__ __forceinline__ void vm_wait() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

typedef short v4s __attribute__((ext_vector_type(4)));

template <int HD>
__global__ __launch_bounds__(256, 3) void attn_dma_k(const uint16_t *__restrict__ qkv,
                                                   int64_t ldq, int S, int H, float scale_log2e,
                                                   const float *__restrict__ add_mask,
                                                   const int32_t *__restrict__ kv_len,
                                                   uint16_t *__restrict__ ctx, int64_t ldo,
                                                   int n_qblk, int force_logits,
                                                   const int32_t *__restrict__ seq_start,
                                                   const int32_t *__restrict__ order) {
  constexpr int NKK = HD / 16, NHT = HD / 32;
  constexpr int ROWB = HD * 2, TILE = BKV * ROWB;  // bytes per row and per operand tile
  constexpr int SLOT = 2 * TILE + BKV * 4;         // K, V, mask row
  constexpr int CPR = ROWB / 16, PR = 1024 / ROWB;  // chunks per row, rows per 1 KB piece
  constexpr int NP = TILE / 1024 / 4;               // pieces per wave and operand (2 or 1)
  constexpr int LOADS = 2 * NP;                     // this wave's K and V loads per tile
  static_assert(HD == 64 || HD == 32, "head_dim 64 or 32");
  __shared__ __attribute__((aligned(1024))) uint8_t sm[NSL * SLOT];

  const int blk = blockIdx.x;
  int qb, h, b;
  if (order) {
    h = blk % H;
    const int t = blk / H;
    qb = t % n_qblk;
    b = order[t / n_qblk];
  } else {
    qb = blk % n_qblk;
    const int bh = blk / n_qblk;
    h = bh % H;
    b = bh / H;
  }
  const int d = H * HD;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5, li = lane & 31;
  int kvl = kv_len ? kv_len[b] : S;
  kvl = kvl < 1 ? 1 : (kvl > S ? S : kvl);
  const int64_t row0 = seq_start ? (int64_t)seq_start[b] : (int64_t)b * S;
  const int lim = seq_start ? kvl : S;
  if (qb * BQ >= lim) return;
  const uint16_t *base = qkv + row0 * ldq;
  const bool live = qb * BQ + wave * 32 < lim;

  // Q fragments (B operand of S^T = K Q^T), waited for before the loop.
  const int q = qb * BQ + wave * 32 + li;
  bf16x8 qf[NKK];
#pragma unroll
  for (int kk = 0; kk < NKK; ++kk) {
    uint4 v = make_uint4(0, 0, 0, 0);
    if (q < lim) v = *(const uint4 *)(base + (int64_t)q * ldq + h * HD + kk * 16 + g * 8);
    qf[kk] = __builtin_bit_cast(bf16x8, v);
  }
#pragma unroll
  for (int kk = 0; kk < NKK; ++kk) asm volatile("" ::"v"(qf[kk]));

  // Key tile t -> slot t % NSL: wave w moves K rows and V rows 8p .. 8p + 7
  // for pieces p = w and w + 4 (1 KB each: lane l fills row 8p + l / 8,
  // position l % 8); wave 0 also the tile's 64 mask entries.
  const uint64_t kb64 = uni64((uint64_t)(uintptr_t)(base + d + h * HD));
  const uint64_t vb64 = uni64((uint64_t)(uintptr_t)(base + 2 * d + h * HD));
  const uint64_t mb64 = add_mask ? uni64((uint64_t)(uintptr_t)(add_mask + (int64_t)b * S)) : 0;
  const uint32_t lds0 = (uint32_t)(uintptr_t)sm;
  const uint32_t rowbytes = (uint32_t)(ldq * 2);
  const int prow = lane / CPR, ppos = lane % CPR;
  auto swz_k = [](int r) { return HD == 64 ? (r >> 1) & 7 : (r >> 2) & 3; };
  auto swz_v = [](int r) { return HD == 64 ? (r & 2) << 1 : 0; };
  auto issue = [&](int t) {
    const uint32_t slot = lds0 + (uint32_t)((t % NSL) * SLOT);
#pragma unroll
    for (int x = 0; x < NP; ++x) {
      const int p = wave + 4 * x;
      const int row = p * PR + prow;
      int key = t * BKV + row;
      key = key < lim ? key : lim - 1;
      const uint32_t roff = (uint32_t)key * rowbytes;
      dma16o(kb64, roff + (uint32_t)((ppos ^ swz_k(row)) * 16), slot + p * 1024);
      dma16o(vb64, roff + (uint32_t)((ppos ^ swz_v(row)) * 16), slot + TILE + p * 1024);
    }
    if (wave == 0 && add_mask) {
      int key = t * BKV + lane;
      key = key < S ? key : S - 1;
      dma4o(mb64, (uint32_t)key * 4, slot + 2 * TILE);
    }
  };
  // This wave's loads of one tile complete in issue order; the wait for tile
  // t leaves tile t + 1's (issued after it) in flight.
  const bool mwave = wave == 0 && add_mask != nullptr;
  auto wait_next = [&](bool one_more_in_flight) {
    if (one_more_in_flight) {
      if (mwave)
        vm_wait<LOADS + 1>();
      else
        vm_wait<LOADS>();
    } else {
      vm_wait<0>();
    }
  };

  f32x16 o[NHT];
#pragma unroll
  for (int t = 0; t < NHT; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[t][r] = 0.0f;
  float m_run = -INFINITY, l_run = 0.0f;

  // Fixed per-lane LDS offsets: K fragment rows sub * 32 + li, chunk 2kk + g;
  // the V^T transposed reads (group G = lane / 16, e, qq below).
  const int swk = swz_k(li);  // rows sub * 32 + li share li's swizzle
  const int G = lane >> 4, e4 = (lane & 15) >> 2, qq = lane & 3;
  // swz_v(16ch + 4(G >> 1) + e4) = swz_v(e4), as a multiple of 4 chunks
  const int swv = swz_v(e4) >> 2;
  const int vrow = 4 * (G >> 1) + e4;

  const int ntile = (kvl + BKV - 1) / BKV;
  issue(0);
  if (ntile > 1) issue(1);
  wait_next(ntile > 1);
  __syncthreads();
  for (int t = 0; t < ntile; ++t) {
    if (t + 2 < ntile) issue(t + 2);
    const uint8_t *sl = sm + (t % NSL) * SLOT;
    if (live) {
      f32x16 sc[2];
#pragma unroll
      for (int sub = 0; sub < 2; ++sub) {
#pragma unroll
        for (int r = 0; r < 16; ++r) sc[sub][r] = 0.0f;
#pragma unroll
        for (int kk = 0; kk < NKK; ++kk) {
          const bf16x8 kf = *(const bf16x8 *)(sl + (sub * 32 + li) * ROWB +
                                              (((2 * kk + g) ^ swk) * 16));
          sc[sub] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[kk], sc[sub], 0, 0, 0);
        }
      }
      // The tile needs logits (mask added, keys past kv_len at -inf) if it
      // reaches past kv_len or has a nonzero mask entry.
      const float *smk = (const float *)(sl + 2 * TILE);
      bool masked = (t + 1) * BKV > kvl || force_logits;
      if (add_mask) masked = masked || __ballot(smk[lane] != 0.0f) != 0;
      float mx = -INFINITY, cc;
      if (masked) {
#pragma unroll
        for (int sub = 0; sub < 2; ++sub)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = sub * 32 + (r >> 2) * 8 + g * 4 + (r & 3);
            const float mv = t * BKV + key < kvl
                                 ? (add_mask ? smk[key] * 1.4426950408889634f : 0.0f)
                                 : -INFINITY;
            const float v = __builtin_fmaf(sc[sub][r], scale_log2e, mv);
            sc[sub][r] = v;
            mx = fmaxf(mx, v);
          }
        cc = 1.0f;
      } else {
#pragma unroll
        for (int sub = 0; sub < 2; ++sub)
#pragma unroll
          for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sc[sub][r]);
        mx *= scale_log2e;
        cc = scale_log2e;
      }
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      if (mx > m_run + 8.0f) {
        const float alpha = __builtin_amdgcn_exp2f(m_run - mx);
        m_run = mx;
        l_run *= alpha;
#pragma unroll
        for (int ht = 0; ht < NHT; ++ht)
#pragma unroll
          for (int r = 0; r < 16; ++r) o[ht][r] *= alpha;
      }
      bf16x8 pk[4];
      float ps = 0.0f;
#pragma unroll
      for (int ch = 0; ch < 4; ++ch) {
        const int sub = ch >> 1, c = ch & 1;
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
          const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[sub][c * 8 + jj], cc, -m_run));
          ps += p;
          pk[ch][jj] = (__bf16)p;
        }
      }
      l_run += ps;
      // O^T += V^T P^T: lane (hd row li, half g) needs keys 16ch + 4g + 0..3
      // and 16ch + 8 + 4g + 0..3 of its hd column; group G of the transposed
      // read covers hd columns 32ht + 16(G & 1) + 0..15 and keys
      // 16ch + 4(G >> 1) + 0..3 (+ 8), its lane 4e + qq addressing row
      // 16ch + 4(G >> 1) + e, columns 32ht + 16(G & 1) + 4qq .. + 3.
      const uint8_t *vs = sl + TILE;
#pragma unroll
      for (int ch = 0; ch < 4; ++ch) {
#pragma unroll
        for (int ht = 0; ht < NHT; ++ht) {
          const int chunk = ((4 * ht) ^ (4 * swv)) + 2 * (G & 1) + (qq >> 1);
          const uint8_t *a = vs + (16 * ch + vrow) * ROWB + chunk * 16 + (qq & 1) * 8;
          const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) v4s *)(uintptr_t)(uint32_t)(uintptr_t)a);
          const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) v4s *)(uintptr_t)(uint32_t)(uintptr_t)(a + 8 * ROWB));
          const short vv8 __attribute__((ext_vector_type(8))) = {lo[0], lo[1], lo[2], lo[3],
                                                                   hi[0], hi[1], hi[2], hi[3]};
          o[ht] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, vv8),
                                                          pk[ch], o[ht], 0, 0, 0);
        }
      }
    }
    // Tile t + 1 in LDS (tile t + 2's loads may stay in flight), then meet:
    // every read of slot t % NSL is done before iteration t + 1 refills it.
    if (t + 1 < ntile) wait_next(t + 2 < ntile);
    __syncthreads();
  }

  const float l = l_run + __shfl_xor(l_run, 32);
  const float inv = 1.0f / l;
  if (q < lim) {
    uint16_t *dst = ctx + (row0 + q) * ldo + h * HD;
#pragma unroll
    for (int ht = 0; ht < NHT; ++ht)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int hd0 = ht * 32 + r4 * 8 + g * 4;
        uint2 w;
        w.x = pack_bf2(o[ht][r4 * 4 + 0] * inv, o[ht][r4 * 4 + 1] * inv);
        w.y = pack_bf2(o[ht][r4 * 4 + 2] * inv, o[ht][r4 * 4 + 3] * inv);
        *(uint2 *)(dst + hd0) = w;
      }
  }
}

}  // namespace

namespace mxk {

hipError_t attention(const AttnArgs &a, hipStream_t s) {
  const int n_qblk = (int)((a.S + BQ - 1) / BQ);
  const int64_t blocks = a.B * a.H * n_qblk;
  const float sl2e = a.scale * 1.4426950408889634f;
  const int force_logits = a.scale > 0.0f ? 0 : 1;  // raw-score max needs scale > 0
  // The direct-load kernel addresses K/V rows by 32-bit byte offsets from the
  // sequence's first row.
  const bool off32 = (int64_t)a.S * a.ld_qkv * 2 < ((int64_t)1 << 31);
  if (a.hd == 64 && off32)
    attn_dma_k<64><<<(unsigned)blocks, 256, 0, s>>>(a.qkv, a.ld_qkv, (int)a.S, (int)a.H, sl2e,
                                                   a.add_mask, a.kv_len, a.ctx, a.ld_ctx, n_qblk,
                                                   force_logits, a.seq_start, a.order);
  else if (a.hd == 32 && off32)
    attn_dma_k<32><<<(unsigned)blocks, 256, 0, s>>>(a.qkv, a.ld_qkv, (int)a.S, (int)a.H, sl2e,
                                                   a.add_mask, a.kv_len, a.ctx, a.ld_ctx, n_qblk,
                                                   force_logits, a.seq_start, a.order);
  else if (a.hd == 64)
    attn_fwd_k<64><<<(unsigned)blocks, 256, 0, s>>>(a.qkv, a.ld_qkv, (int)a.S, (int)a.H, sl2e,
                                                   a.add_mask, a.kv_len, a.ctx, a.ld_ctx, n_qblk,
                                                   force_logits, a.seq_start, a.order);
  else if (a.hd == 32)
    attn_fwd_k<32><<<(unsigned)blocks, 256, 0, s>>>(a.qkv, a.ld_qkv, (int)a.S, (int)a.H, sl2e,
                                                   a.add_mask, a.kv_len, a.ctx, a.ld_ctx, n_qblk,
                                                   force_logits, a.seq_start, a.order);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace mxk
