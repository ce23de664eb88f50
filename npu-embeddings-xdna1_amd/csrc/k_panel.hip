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
// is converted.
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

}  // namespace

namespace mxk {

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
