// k_quant.hip -- the int8 datapath's activation quantisation on gfx950:
// quantise_a_int8 (host_kernels.hpp:263-320) as a standalone pass, and
// add_norm_quant (bert_encoder.cpp:1197-1300): the residual LayerNorm whose
// output is quantised for the next int8 GEMM in the same pass.
//
// Per row r of K values a (scaled per column by ias = 1/asmooth):
//   t_j = a_j * ias_j                 (one rounded multiply)
//   mx  = max_j |t_j|,  sc = mx > 0 ? mx / 127 : 1,  inv = 1 / sc
//   q_j = rint(clamp(t_j * inv, -127, 127))   (nearest-even)
// with correctly rounded division, the host's operation order, and no fused
// multiply-add, so q and sc are bit-identical to the host's for finite input.
//
// One wave per row; the row stays in registers between the maximum and the
// quantisation: NQ groups of 256 columns, four consecutive columns per lane
// (16-byte fp32 / 8-byte bf16 loads, 4-byte int8 stores). Columns past K
// (K % 256 != 0) are masked out of every reduction.
#include "mx_common.hpp"
#include "mx_kernels.hpp"

using namespace mxd;

namespace {

// ST: streaming (nontemporal) loads, for data dead once read.
template <bool ST = false>
__device__ __forceinline__ float4 load4(const void *p, bool bf, int64_t off) {
  if (bf) {
    const uint2 u = ST ? ld_stream8((const uint16_t *)p + off)
                       : *(const uint2 *)((const uint16_t *)p + off);
    return make_float4(bf2f(u.x & 0xFFFFu), bf2f(u.x >> 16), bf2f(u.y & 0xFFFFu), bf2f(u.y >> 16));
  }
  if (ST) {
    const uint4 u = ld_stream16((const float *)p + off);
    return make_float4(__uint_as_float(u.x), __uint_as_float(u.y), __uint_as_float(u.z),
                       __uint_as_float(u.w));
  }
  return *(const float4 *)((const float *)p + off);
}

__device__ __forceinline__ float4 mul4(float4 a, float4 b) {
  return make_float4(__fmul_rn(a.x, b.x), __fmul_rn(a.y, b.y), __fmul_rn(a.z, b.z),
                     __fmul_rn(a.w, b.w));
}

__device__ __forceinline__ float absmax4(float m, float4 t) {
  return fmaxf(fmaxf(fmaxf(m, fabsf(t.x)), fmaxf(fabsf(t.y), fabsf(t.z))), fabsf(t.w));
}

__device__ __forceinline__ int q8(float t, float inv) {
  const float v = fminf(fmaxf(__fmul_rn(t, inv), -127.0f), 127.0f);
  return (int)__builtin_rintf(v);
}

// Quantise the NQ groups t (already a * ias) of one row: the scale and the
// int8 codes (lane's four columns per group packed into one 32-bit store).
template <int NQ>
__device__ __forceinline__ void quantise_row(const float4 *t, float mx, int K, int lane,
                                             int8_t *qrow, float *scale_out) {
  mx = wave_max(mx);
  const float sc = mx > 0.0f ? mx / 127.0f : 1.0f;
  const float inv = 1.0f / sc;
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    const int c = i * 256 + lane * 4;
    if (c < K) {
      const uint32_t w = (uint32_t)(q8(t[i].x, inv) & 0xFF) |
                         ((uint32_t)(q8(t[i].y, inv) & 0xFF) << 8) |
                         ((uint32_t)(q8(t[i].z, inv) & 0xFF) << 16) |
                         ((uint32_t)(q8(t[i].w, inv) & 0xFF) << 24);
      *(uint32_t *)(qrow + c) = w;
    }
  }
  if (lane == 0) *scale_out = sc;
}

template <int NQ, bool IN_BF>
__global__ __launch_bounds__(256) void quantise_rows_k(const void *__restrict__ a, int64_t lda,
                                                       int64_t rows, int K,
                                                       const float *__restrict__ ias,
                                                       int8_t *__restrict__ q, int64_t ldq,
                                                       float *__restrict__ a_scale,
                                                       const int32_t *rows_dev) {
  const int lane = threadIdx.x & 63;
  const int64_t row = blockIdx.x * (int64_t)(blockDim.x / 64) + (threadIdx.x >> 6);
  if (row >= live_rows(rows, rows_dev)) return;
  float4 t[NQ];
  float mx = 0.0f;
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    const int c = i * 256 + lane * 4;
    if (c < K) {
      t[i] = mul4(load4(a, IN_BF, row * lda + c), *(const float4 *)(ias + c));
      mx = absmax4(mx, t[i]);
    } else {
      t[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
  }
  quantise_row<NQ>(t, mx, K, lane, q + row * ldq, a_scale + row);
}

// add_norm_quant: z = x (+ y); x_out = (z - mean) / sqrt(var + eps) * gamma +
// beta (fp32 statistics, the LayerNorm of k_elem.hip), then the quantisation
// of x_out * ias. x_out is written to out_f32 (nullable; may alias x).
// ST: the in-place residual form (out_f32 == x, y given) streams x, y and the
// new x, as the bf16 datapath's residual LayerNorm does (k_elem.hip).
template <int NQ, bool ST>
__global__ __launch_bounds__(256) void layernorm_quant_k(
    const float *__restrict__ x, const void *__restrict__ y, int y_bf,
    const float *__restrict__ gamma, const float *__restrict__ beta, float eps, int64_t rows,
    int cols, float *out_f32, const float *__restrict__ ias, int8_t *__restrict__ q,
    float *__restrict__ a_scale, const int32_t *rows_dev) {
  const int lane = threadIdx.x & 63;
  const int64_t row = blockIdx.x * (int64_t)(blockDim.x / 64) + (threadIdx.x >> 6);
  if (row >= live_rows(rows, rows_dev)) return;
  // gamma, beta and the next GEMM's ias are read with the row, so their
  // latency runs under its loads instead of after the two reductions.
  float4 gm[NQ], bt[NQ], ia[NQ];
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    const int c = i * 256 + lane * 4;
    if (c < cols) {
      gm[i] = *(const float4 *)(gamma + c);
      bt[i] = *(const float4 *)(beta + c);
      ia[i] = *(const float4 *)(ias + c);
    }
  }
  float4 v[NQ];
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    const int c = i * 256 + lane * 4;
    v[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (c < cols) {
      const int64_t off = row * cols + c;
      v[i] = load4<ST>(x, false, off);
      if (y) {
        const float4 w = load4<ST>(y, y_bf, off);
        v[i].x += w.x;
        v[i].y += w.y;
        v[i].z += w.z;
        v[i].w += w.w;
      }
    }
    s += (v[i].x + v[i].y) + (v[i].z + v[i].w);
  }
  const float mean = wave_sum(s) / (float)cols;
  float qs = 0.0f;
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    if (i * 256 + lane * 4 < cols) {
      const float a = v[i].x - mean, b = v[i].y - mean, c = v[i].z - mean, d = v[i].w - mean;
      qs = __builtin_fmaf(a, a, qs);
      qs = __builtin_fmaf(b, b, qs);
      qs = __builtin_fmaf(c, c, qs);
      qs = __builtin_fmaf(d, d, qs);
    }
  }
  const float var = wave_sum(qs) / (float)cols;
  const float is = 1.0f / sqrtf(var + eps);
  float mx = 0.0f;
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    const int c = i * 256 + lane * 4;
    if (c < cols) {
      float4 r;
      r.x = __builtin_fmaf((v[i].x - mean) * is, gm[i].x, bt[i].x);
      r.y = __builtin_fmaf((v[i].y - mean) * is, gm[i].y, bt[i].y);
      r.z = __builtin_fmaf((v[i].z - mean) * is, gm[i].z, bt[i].z);
      r.w = __builtin_fmaf((v[i].w - mean) * is, gm[i].w, bt[i].w);
      if (out_f32) {
        if (ST)
          st_stream16(out_f32 + row * cols + c,
                      make_uint4(__float_as_uint(r.x), __float_as_uint(r.y),
                                 __float_as_uint(r.z), __float_as_uint(r.w)));
        else
          *(float4 *)(out_f32 + row * cols + c) = r;
      }
      v[i] = mul4(r, ia[i]);
      mx = absmax4(mx, v[i]);
    }
  }
  quantise_row<NQ>(v, mx, cols, lane, q + row * cols, a_scale + row);
}

}  // namespace

namespace mxk {

int quant_groups(int64_t K) {
  const int64_t g = (K + 255) / 256;
  static const int sizes[] = {1, 2, 3, 4, 5, 6, 8, 12, 16, 20, 24, 32};
  for (int s : sizes)
    if (g <= s) return s;
  return 0;
}

hipError_t quantise_rows(const void *a, int a_bf, int64_t lda, int64_t rows, int64_t K,
                         const float *ias, int8_t *q, int64_t ldq, float *a_scale,
                         hipStream_t s, const int32_t *rows_dev) {
  const int g = (int)((rows + 3) / 4);
#define MX_Q_CASE(nq)                                                                         \
  case nq:                                                                                    \
    if (a_bf)                                                                                 \
      quantise_rows_k<nq, true><<<g, 256, 0, s>>>(a, lda, rows, (int)K, ias, q, ldq, a_scale, \
                                                  rows_dev);                                  \
    else                                                                                      \
      quantise_rows_k<nq, false><<<g, 256, 0, s>>>(a, lda, rows, (int)K, ias, q, ldq,         \
                                                   a_scale, rows_dev);                        \
    return hipGetLastError();
  switch (quant_groups(K)) {
    MX_Q_CASE(1)
    MX_Q_CASE(2)
    MX_Q_CASE(3)
    MX_Q_CASE(4)
    MX_Q_CASE(5)
    MX_Q_CASE(6)
    MX_Q_CASE(8)
    MX_Q_CASE(12)
    MX_Q_CASE(16)
    MX_Q_CASE(20)
    MX_Q_CASE(24)
    MX_Q_CASE(32)
    default:
      return hipErrorInvalidValue;
  }
#undef MX_Q_CASE
}

hipError_t layernorm_quant(const float *x, const void *y, int y_bf, const float *gamma,
                           const float *beta, float eps, int64_t rows, int64_t cols,
                           float *out_f32, const float *ias, int8_t *q, float *a_scale,
                           hipStream_t s, const int32_t *rows_dev) {
  const int g = (int)((rows + 3) / 4);
  const bool st = y && out_f32 && out_f32 == x;
#define MX_LQ_CASE(nq)                                                                    \
  case nq:                                                                                \
    if (st)                                                                               \
      layernorm_quant_k<nq, true><<<g, 256, 0, s>>>(x, y, y_bf, gamma, beta, eps, rows,   \
                                                    (int)cols, out_f32, ias, q, a_scale,  \
                                                    rows_dev);                            \
    else                                                                                  \
      layernorm_quant_k<nq, false><<<g, 256, 0, s>>>(x, y, y_bf, gamma, beta, eps, rows,  \
                                                     (int)cols, out_f32, ias, q, a_scale, \
                                                     rows_dev);                           \
    return hipGetLastError();
  switch (quant_groups(cols)) {
    MX_LQ_CASE(1)
    MX_LQ_CASE(2)
    MX_LQ_CASE(3)
    MX_LQ_CASE(4)
    MX_LQ_CASE(5)
    MX_LQ_CASE(6)
    MX_LQ_CASE(8)
    MX_LQ_CASE(12)
    MX_LQ_CASE(16)
    default:
      return hipErrorInvalidValue;
  }
#undef MX_LQ_CASE
}

}  // namespace mxk
