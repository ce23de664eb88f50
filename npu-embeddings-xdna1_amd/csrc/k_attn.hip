// k_attn.hip -- fused masked attention on gfx950 MFMA: QK^T, additive-mask
// softmax and PV in one pass per (sequence, head, 128-query block); the score
// matrix never reaches HBM. A block is 4 waves. With head_dim 64 the key tiles
// are 32 keys and four blocks share a CU (four waves per SIMD: 104 VGPRs, a
// 33 KB ring); waves in flight are what hide this kernel's latency, and the
// 64-key tiles' 156 VGPRs and 49 KB ring allowed only three (0.60 against
// 0.55 ms per bge-base batch). With head_dim 32 a 32-key tile is less than a
// 1 KB load per wave, and the tiles stay 64 keys, three blocks per CU. (8-wave
// blocks of 256 queries, which halve the K/V tiles staged per query, measured
// slower on the bge-base batch: 0.85 against 0.68 ms per batch -- fewer,
// larger blocks leave more query waves idle on short sequences, and at two
// blocks per CU the kernel spills.)
//
// Each wave owns 32 queries and computes the TRANSPOSED score tile
// S^T = K Q^T with v_mfma_f32_32x32x16_bf16 (keys on rows, queries on
// columns), so every lane holds 16 scores of ONE query: the row max and sum of
// the online softmax are lane-local plus one exchange with lane^32, and the
// rescale of the running output is a per-lane scalar. The output is kept as
// O^T = V^T P^T: the probabilities go straight from the score accumulator into
// the B operand (converted to bf16) -- the keys a lane holds are a fixed
// permutation of the MFMA's k index, and the A operand (V^T) is read in that
// same permutation, so no shuffle is needed.
//
// Staging. K, V and the tile's mask row go global -> LDS by direct loads
// (global_load_lds_dwordx4 / _dword, issued from inline assembly so the
// compiler adds no waits) into a ring of NSL slots, two key tiles ahead; no
// registers hold K or V in flight. (Four slots with the fourth spare measured
// faster than three, 0.56 against 0.58 ms per bge-base batch; issuing three
// tiles ahead into all four was no faster than two.) V stays row-major in LDS: the PV
// operand V^T is read with ds_read_b64_tr_b16, which hands each lane of a
// 16-lane group one column of the 4 x 16 bf16 block the group addresses (lane
// j of the group receives element j % 4 of group lane 4e + j / 4's 8 bytes,
// e = 0..3), i.e. four consecutive keys of one head-dim column.
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
//
// Softmax runs in the log2 domain (scores * scale * log2e, mask * log2e) with
// the hardware exp2. Keys at or past kv_len[b] are skipped (whole tiles) or
// given -inf (inside the last tile); -1e30 mask entries stay finite, so a row
// whose keys are all masked attends uniformly, as the host softmax does.
//
// VALU economy (the softmax, not the MFMAs, bounds this kernel): a key tile
// that reaches no further than kv_len and whose mask entries are all zero (a
// wave ballot over the staged mask row) skips the per-score mask add (scale >
// 0), and each probability is one FMA into exp2. Only the first key tile
// takes a maximum: it fixes the reference point m of the exponentials, and a
// later tile pays for a maximum, a rescale of O and l and a second pass of
// exponentials only when its probabilities sum past 2^24 -- so most tiles
// carry no max, no cross-lane exchange and no rescale; the result O / l is
// the same quotient. The row sum adds the bf16 probabilities two at a time
// (v_dot2c_f32_bf16 against 1.0).
#include "mx_common.hpp"
#include "mx_kernels.hpp"

using namespace mxd;

namespace {

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

// NW waves of 32 queries per block (BQ = 32 NW queries share each staged K/V
// tile), key tiles of BKV (32 or 64) keys in a ring of NSL slots, and WPS
// waves per SIMD as the second launch bound.
template <int HD, int NW, int BKV, int NSL, int WPS>
__global__ __launch_bounds__(NW * 64, WPS) void attn_dma_k(const uint16_t *__restrict__ qkv,
                                                   int64_t ldq, int S, int H, float scale_log2e,
                                                   const float *__restrict__ add_mask,
                                                   const int32_t *__restrict__ kv_len,
                                                   uint16_t *__restrict__ ctx, int64_t ldo,
                                                   int n_qblk, int force_logits,
                                                   const int32_t *__restrict__ seq_start,
                                                   const int32_t *__restrict__ order,
                                                   int q_lim) {
  constexpr int NKK = HD / 16, NHT = HD / 32;
  constexpr int ROWB = HD * 2, TILE = BKV * ROWB;  // bytes per row and per operand tile
  constexpr int SLOT = 2 * TILE + BKV * 4;         // K, V, mask row
  constexpr int CPR = ROWB / 16, PR = 1024 / ROWB;  // chunks per row, rows per 1 KB piece
  constexpr int BQ = 32 * NW;                       // queries per block
  constexpr int NP = TILE / 1024 / NW;              // pieces per wave and operand
  constexpr int LOADS = 2 * NP;                     // this wave's K and V loads per tile
  static_assert(HD == 64 || HD == 32, "head_dim 64 or 32");
  static_assert(NP >= 1 && NP * NW * 1024 == TILE, "each wave moves whole 1 KB pieces");
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
  // Queries at or past q_lim (the first q_lim of each sequence are asked for)
  // are neither computed nor stored; their waves still stage K and V.
  const int qend = lim < q_lim ? lim : q_lim;
  const bool live = qb * BQ + wave * 32 < qend;

  const int q = qb * BQ + wave * 32 + li;

  // Key tile t -> slot t % NSL: wave w moves the K and V rows of 1 KB pieces
  // p = w, w + NW, ... (PR rows each: lane l fills row PR p + l / CPR,
  // 16-byte position l % CPR); wave 0 also the tile's BKV mask entries.
  const uint64_t kb64 = uni64((uint64_t)(uintptr_t)(base + d + h * HD));
  const uint64_t vb64 = uni64((uint64_t)(uintptr_t)(base + 2 * d + h * HD));
  const uint64_t mb64 = add_mask ? uni64((uint64_t)(uintptr_t)(add_mask + (int64_t)b * S)) : 0;
  const uint32_t lds0 = (uint32_t)(uintptr_t)sm;
  const uint64_t rowbytes = (uint64_t)ldq * 2;
  const int prow = lane / CPR, ppos = lane % CPR;
  auto swz_k = [](int r) { return HD == 64 ? (r >> 1) & 7 : (r >> 2) & 3; };
  auto swz_v = [](int r) { return HD == 64 ? (r & 2) << 1 : 0; };
  // Addresses: a 64-bit scalar base at the tile's first row plus a 32-bit
  // per-lane offset within the tile's 64 rows (any sequence length). A live
  // tile starts below kv_len <= lim <= S, so the clamped rows stay at or past
  // its first.
  auto issue = [&](int t) {
    const uint32_t slot = lds0 + (uint32_t)((t % NSL) * SLOT);
    const uint64_t toff = (uint64_t)(t * BKV) * rowbytes;
#pragma unroll
    for (int x = 0; x < NP; ++x) {
      const int p = wave + NW * x;
      const int row = p * PR + prow;
      int key = t * BKV + row;
      key = key < lim ? key : lim - 1;
      const uint32_t roff = (uint32_t)((uint64_t)(key - t * BKV) * rowbytes);
      dma16o(kb64 + toff, roff + (uint32_t)((ppos ^ swz_k(row)) * 16), slot + p * 1024);
      dma16o(vb64 + toff, roff + (uint32_t)((ppos ^ swz_v(row)) * 16), slot + TILE + p * 1024);
    }
    if (wave == 0 && add_mask && lane < BKV) {
      int key = t * BKV + lane;
      key = key < S ? key : S - 1;
      dma4o(mb64 + (uint64_t)(t * BKV) * 4, (uint32_t)(key - t * BKV) * 4, slot + 2 * TILE);
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
  // Q fragments (B operand of S^T = K Q^T), loaded after the first key tiles'
  // loads are issued so the two latencies overlap, and waited for before the
  // loop (the wait drains every load of this wave, tile 1's included).
  bf16x8 qf[NKK];
#pragma unroll
  for (int kk = 0; kk < NKK; ++kk) {
    uint4 v = make_uint4(0, 0, 0, 0);
    if (q < lim) v = *(const uint4 *)(base + (int64_t)q * ldq + h * HD + kk * 16 + g * 8);
    qf[kk] = __builtin_bit_cast(bf16x8, v);
  }
#pragma unroll
  for (int kk = 0; kk < NKK; ++kk) asm volatile("" ::"v"(qf[kk]));
  wait_next(ntile > 1);
  __syncthreads();
  for (int t = 0; t < ntile; ++t) {
    if (t + 2 < ntile) issue(t + 2);
    const uint8_t *sl = sm + (t % NSL) * SLOT;
    if (live) {
      // A 64-key tile's second 32 keys all at or past kv_len (the last tile of
      // a sequence whose length is <= 32 past a multiple of 64): their scores,
      // probabilities and PV products are skipped -- each would be exp2(-inf)
      // = 0. A 32-key tile is its first half alone.
      const bool h1 = BKV == 64 && t * BKV + 32 < kvl;
      // The staged mask entry this lane tests, read first: its latency runs
      // under the score MFMAs instead of after them.
      const float *smk = (const float *)(sl + 2 * TILE);
      // (unused, and never written, without a mask; a 32-key row has 32)
      float mword = lane < BKV ? smk[lane] : 0.0f;
      // Each half's chain starts from an immediate zero accumulator; a
      // skipped second half is left unset (nothing reads it), so no register
      // copies merge it with the computed one. With both halves live their
      // two chains alternate, each k-step's fragments read one step ahead, so
      // neither the LDS reads nor a chain's dependent MFMAs stall the wave.
      f32x16 sc[2];
      auto kfrag = [&](int sub, int kk) {
        return *(const bf16x8 *)(sl + (sub * 32 + li) * ROWB + (((2 * kk + g) ^ swk) * 16));
      };
      if (h1) {
        bf16x8 ka = kfrag(0, 0), kb = kfrag(1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // k-step 0's two reads
#pragma unroll
        for (int kk = 0; kk < NKK; ++kk) {
          bf16x8 na = ka, nb = kb;
          if (kk + 1 < NKK) {
            na = kfrag(0, kk + 1);
            nb = kfrag(1, kk + 1);
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // the next k-step's reads
          }
          sc[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka, qf[kk], kk == 0 ? f32x16{} : sc[0],
                                                          0, 0, 0);
          sc[1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kb, qf[kk], kk == 0 ? f32x16{} : sc[1],
                                                          0, 0, 0);
          __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // then this k-step's MFMAs
          ka = na;
          kb = nb;
        }
      } else {
#pragma unroll
        for (int kk = 0; kk < NKK; ++kk)
          sc[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kfrag(0, kk), qf[kk],
                                                          kk == 0 ? f32x16{} : sc[0], 0, 0, 0);
      }
      // The tile needs logits (mask added, keys past kv_len at -inf) if it
      // reaches past kv_len or has a nonzero mask entry.
      bool masked = (t + 1) * BKV > kvl || force_logits;
      asm volatile("" : "+v"(mword));  // first read of the mask entry: after the MFMAs
      if (add_mask) masked = masked || __ballot(mword != 0.0f) != 0;
      float cc;
      if (masked) {
        // Lane (li, g) holds keys sub * 32 + 8 rr + 4 g + e of accumulator
        // element 4 rr + e: four consecutive mask entries, one 16-byte LDS
        // read. All BKV entries of the staged row are written (the loads clamp
        // to the sequence's last key), so the reads are unconditional; keys at
        // or past kv_len take -inf by a select.
#pragma unroll
        for (int sub = 0; sub < 2; ++sub) {
          if (sub == 1 && !h1) continue;
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) {
            const int key0 = sub * 32 + rr * 8 + g * 4;
            float4 m4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (add_mask) m4 = *(const float4 *)(smk + key0);
            const float mk[4] = {m4.x, m4.y, m4.z, m4.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int r = rr * 4 + e;
              const float mv =
                  t * BKV + key0 + e < kvl ? mk[e] * 1.4426950408889634f : -INFINITY;
              sc[sub][r] = __builtin_fmaf(sc[sub][r], scale_log2e, mv);
            }
          }
        }
        cc = 1.0f;
      } else {
        cc = scale_log2e;
      }
      // The query's largest logit in this tile (both lanes of the query).
      auto tile_max = [&]() {
        float mx = -INFINITY;
#pragma unroll
        for (int sub = 0; sub < 2; ++sub) {
          if (sub == 1 && !h1) continue;
#pragma unroll
          for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sc[sub][r]);
        }
        mx *= cc;
        return fmaxf(mx, __shfl_xor(mx, 32));
      };
      // Probabilities p = 2^(logit - m_run), rounded to bf16 in pairs for the
      // PV MFMA; the row sum adds the bf16 pairs (v_dot2c_f32_bf16 with 1.0),
      // so the normaliser is the sum of the very weights PV applies.
      bf16x8 pk[4];
      float ps;
      auto exps = [&]() {
        typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
        const bf16x2_t one = {(__bf16)1.0f, (__bf16)1.0f};
        ps = 0.0f;
#pragma unroll
        for (int ch = 0; ch < 4; ++ch) {
          const int sub = ch >> 1, c = ch & 1;
          if (sub == 1 && !h1) continue;
#pragma unroll
          for (int jj = 0; jj < 8; jj += 2) {
            bf16x2_t pr;
            pr[0] = (__bf16)__builtin_amdgcn_exp2f(
                __builtin_fmaf(sc[sub][c * 8 + jj], cc, -m_run));
            pr[1] = (__bf16)__builtin_amdgcn_exp2f(
                __builtin_fmaf(sc[sub][c * 8 + jj + 1], cc, -m_run));
            pk[ch][jj] = pr[0];
            pk[ch][jj + 1] = pr[1];
            ps = __builtin_amdgcn_fdot2_f32_bf16(pr, one, ps, false);
          }
        }
      };
      // The reference point m_run is the first tile's maximum and moves only
      // when a later tile's probabilities sum past 2^24 (or overflow): then
      // that tile's maximum is taken, O and l are rescaled and the tile's
      // probabilities recomputed. Below that bound every p is at most 2^24,
      // far inside fp32 and bf16 range, and O / l is the same quotient.
      if (t == 0) m_run = tile_max();
      exps();
      if (__ballot(!(ps <= 16777216.0f)) != 0) {
        const float mn = fmaxf(m_run, tile_max());
        const float alpha = __builtin_amdgcn_exp2f(m_run - mn);
        m_run = mn;
        l_run *= alpha;
#pragma unroll
        for (int ht = 0; ht < NHT; ++ht)
#pragma unroll
          for (int r = 0; r < 16; ++r) o[ht][r] *= alpha;
        exps();
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
        if (ch >= 2 && !h1) continue;
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
  if (q < qend) {
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
  constexpr int nw = 4, bq = 32 * nw;
  const int64_t qs = a.q_rows > 0 && a.q_rows < a.S ? a.q_rows : a.S;
  const int n_qblk = (int)((qs + bq - 1) / bq);
  const int64_t blocks = a.B * a.H * n_qblk;
  const float sl2e = a.scale * 1.4426950408889634f;
  const int force_logits = a.scale > 0.0f ? 0 : 1;  // raw-score max needs scale > 0
  // head_dim 64: 32-key tiles, a 4-slot ring, four blocks per CU; head_dim 32:
  // 64-key tiles, 3 slots, three blocks per CU.
  if (a.hd == 64)
    attn_dma_k<64, nw, 32, 4, 4><<<(unsigned)blocks, 64 * nw, 0, s>>>(
        a.qkv, a.ld_qkv, (int)a.S, (int)a.H, sl2e, a.add_mask, a.kv_len, a.ctx, a.ld_ctx,
        n_qblk, force_logits, a.seq_start, a.order, (int)qs);
  else if (a.hd == 32)
    attn_dma_k<32, nw, 64, 3, 3><<<(unsigned)blocks, 64 * nw, 0, s>>>(
        a.qkv, a.ld_qkv, (int)a.S, (int)a.H, sl2e, a.add_mask, a.kv_len, a.ctx, a.ld_ctx,
        n_qblk, force_logits, a.seq_start, a.order, (int)qs);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace mxk
