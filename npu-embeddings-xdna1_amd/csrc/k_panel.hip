// k_panel.hip -- a container's pre-tiled GEMM operand, untiled on the GPU into
// the MFMA-ready [N, K] panel the GEMM reads.
//
// The container stores a [K, N] operand as tiles of tile_k x tile_n in
// (k-block, n-block) order, and each tile as (tile_k/mac_s, tile_n/mac_t)
// sub-tiles of mac_s x mac_t, row-major inside (tools/lib/npue.py:491-556):
// flat element e of tile (bk, bn) is
//   e = ((ri * (tile_n/mac_t) + ci) * mac_s + si) * mac_t + ti,
//   k = bk*tile_k + ri*mac_s + si,  n = bn*tile_n + ci*mac_t + ti,
// the placement hostb::host_b_kn walks (common/host_b.hpp:206-243).
//
// One workgroup per tile: the tile's contiguous run of the container is read
// in order (coalesced) and scattered into LDS as [n][k]; each row n of the
// tile then leaves as tile_k consecutive bf16 of the panel row (coalesced).
// A pure permutation of bf16 or int8 elements -- every element is copied, none
// is converted. An int4 run is first widened to the int8 run (widen_i4_k).
#include "mx_common.hpp"
#include "mx_kernels.hpp"

namespace {

template <typename T>
__global__ __launch_bounds__(256) void untile_panel_k(const T *__restrict__ panel, int64_t K,
                                                      int64_t N, int tk, int tn, int ms, int mt,
                                                      T *__restrict__ wt) {
  extern __shared__ uint8_t lds[];
  T *tile = (T *)lds;  // [tn][tk + 2]
  const int pitch = tk + 2;
  const int64_t nb = N / tn;
  const int64_t b = blockIdx.x;  // k,n order: b = bk * nb + bn
  const int64_t bk = b / nb, bn = b - bk * nb;
  const T *src = panel + b * (int64_t)tk * tn;
  const int c0 = tn / mt, elems = tk * tn;
  for (int e = threadIdx.x; e < elems; e += blockDim.x) {
    int q = e;
    const int ti = q % mt;
    q /= mt;
    const int si = q % ms;
    q /= ms;
    const int ci = q % c0;
    const int ri = q / c0;
    tile[(ci * mt + ti) * pitch + ri * ms + si] = src[e];
  }
  __syncthreads();
  for (int e = threadIdx.x; e < elems; e += blockDim.x) {
    const int nn = e / tk, kk = e - nn * tk;
    wt[(bn * tn + nn) * K + bk * tk + kk] = tile[nn * pitch + kk];
  }
}

// int4 weight storage over the int8 datapath (common/int4_panel.hpp:77-246,
// the I4 branch of npue::gemm_b_panel). The container's flat tiled run holds
// two values per byte, element f in nibble f % 2 (the low one first) of byte
// f / 2, sign-extended from 4 bits to t in [-8, 7]. With (k, n) the element's
// place in the [K, N] operand (the placement above),
//   q = clip(rint(t * gscale[k / group][n]), -127, 127)
// (rint: round half to even; t * gscale one fp32 rounding, no fused multiply)
// is written at the same flat index: the int8 panel an I8 container of that
// tiling carries, which untile_panel_k<int8_t> then turns into [N, K]. One
// thread per byte (two elements), so the packed run is read once, coalesced.
__global__ __launch_bounds__(256) void widen_i4_k(const uint8_t *__restrict__ packed, int64_t K,
                                                  int64_t N, int tk, int tn, int ms, int mt,
                                                  const float *__restrict__ gscale,
                                                  int64_t group, int8_t *__restrict__ out) {
#pragma clang fp contract(off)
  const int64_t nbytes = K * N / 2;
  const int64_t tile = (int64_t)tk * tn, nb = N / tn;
  const int c0 = tn / mt;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < nbytes;
       i += (int64_t)gridDim.x * blockDim.x) {
    const uint32_t byte = packed[i];
    int8_t pair[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int64_t f = 2 * i + h;
      const int64_t b = f / tile;
      int e = (int)(f - b * tile);
      const int ti = e % mt;
      e /= mt;
      const int si = e % ms;
      e /= ms;
      const int ci = e % c0;
      const int ri = e / c0;
      const int64_t bk = b / nb, bn = b - bk * nb;
      const int64_t k = bk * tk + ri * ms + si, n = bn * tn + ci * mt + ti;
      const int nv = (int)((byte >> (4 * h)) & 0xFu);
      const float t = (float)(nv > 7 ? nv - 16 : nv);
      float q = __builtin_rintf(t * gscale[(k / group) * N + n]);
      q = q > 127.0f ? 127.0f : (q < -127.0f ? -127.0f : q);
      pair[h] = (int8_t)(int)q;
    }
    *(char2 *)(out + 2 * i) = make_char2(pair[0], pair[1]);
  }
}

}  // namespace

namespace mxk {

hipError_t widen_i4_panel(const uint8_t *packed, int64_t K, int64_t N, int tile_k, int tile_n,
                          int mac_s, int mac_t, const float *gscale, int64_t group, int8_t *out,
                          hipStream_t s) {
  const int64_t bytes = K * N / 2;
  const int64_t blocks = (bytes + 255) / 256;
  widen_i4_k<<<(unsigned)(blocks < 65536 ? blocks : 65536), 256, 0, s>>>(
      packed, K, N, tile_k, tile_n, mac_s, mac_t, gscale, group, out);
  return hipGetLastError();
}


hipError_t untile_panel(const uint16_t *panel, int64_t K, int64_t N, int tile_k, int tile_n,
                        int mac_s, int mac_t, uint16_t *wt, hipStream_t s) {
  const int64_t tiles = (K / tile_k) * (N / tile_n);
  const size_t lds = (size_t)(tile_k + 2) * tile_n * 2;
  untile_panel_k<uint16_t><<<(unsigned)tiles, 256, lds, s>>>(panel, K, N, tile_k, tile_n, mac_s,
                                                             mac_t, wt);
  return hipGetLastError();
}

hipError_t untile_panel_i8(const int8_t *panel, int64_t K, int64_t N, int tile_k, int tile_n,
                           int mac_s, int mac_t, int8_t *wt, hipStream_t s) {
  const int64_t tiles = (K / tile_k) * (N / tile_n);
  const size_t lds = (size_t)(tile_k + 2) * tile_n;
  untile_panel_k<int8_t><<<(unsigned)tiles, 256, lds, s>>>(panel, K, N, tile_k, tile_n, mac_s,
                                                           mac_t, wt);
  return hipGetLastError();
}

}  // namespace mxk
