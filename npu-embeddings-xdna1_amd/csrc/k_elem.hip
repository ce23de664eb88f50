// k_elem.hip -- the HBM-bound kernels of the encoder path on gfx950:
// narrowing (fp32/int32 -> bf16), GELU, row LayerNorm with the residual add
// fused, row softmax, the embedding sum + mask, and pooling.
//
// Every kernel is a coalesced streaming pass: one wave per row for the row ops
// (rows of <= 2048 values live in registers, reductions by wave shuffles), 16-
// or 8-byte accesses for the elementwise ops, grid-stride loops sized to fill
// the 256 CUs.
#include "mx_common.hpp"
#include "mx_kernels.hpp"

using namespace mxd;

namespace {

constexpr int kElemThreads = 256;

inline int grid_for(int64_t work_items, int per_block) {
  int64_t g = (work_items + per_block - 1) / per_block;
  if (g < 1) g = 1;
  if (g > 65536) g = 65536;
  return (int)g;
}

// ---- narrowing --------------------------------------------------------------

// Streaming 16-byte accesses both ways: each value is read and written once
// (fp32 -> bf16 over FFN-up's 17,455 x 3,072: 52 us against 55 with cached
// accesses; int32 -> bf16 54 against 56).
__global__ void narrow_f32_vec_k(const float4 *__restrict__ in, uint4 *__restrict__ out,
                                 int64_t n8) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n8;
       i += (int64_t)gridDim.x * blockDim.x) {
    const uint4 ua = ld_stream16(in + 2 * i), ub = ld_stream16(in + 2 * i + 1);
    const float a[4] = {__uint_as_float(ua.x), __uint_as_float(ua.y), __uint_as_float(ua.z),
                        __uint_as_float(ua.w)};
    const float b[4] = {__uint_as_float(ub.x), __uint_as_float(ub.y), __uint_as_float(ub.z),
                        __uint_as_float(ub.w)};
    uint4 o;
    o.x = pack_bf2(a[0], a[1]);
    o.y = pack_bf2(a[2], a[3]);
    o.z = pack_bf2(b[0], b[1]);
    o.w = pack_bf2(b[2], b[3]);
    st_stream16(out + i, o);
  }
}

__global__ void narrow_f32_scalar_k(const float *__restrict__ in, uint16_t *__restrict__ out,
                                    int64_t lo, int64_t n) {
  for (int64_t i = lo + blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    out[i] = f2bf(in[i]);
}

// i32_to_bf16 (mx_common.hpp): int32 -> bf16 in one rounding of the integer.

__global__ void narrow_i32_vec_k(const int4 *__restrict__ in, uint4 *__restrict__ out,
                                 int64_t n8) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n8;
       i += (int64_t)gridDim.x * blockDim.x) {
    const uint4 a = ld_stream16(in + 2 * i), b = ld_stream16(in + 2 * i + 1);
    uint4 o;
    o.x = (uint32_t)i32_to_bf16((int32_t)a.x) | ((uint32_t)i32_to_bf16((int32_t)a.y) << 16);
    o.y = (uint32_t)i32_to_bf16((int32_t)a.z) | ((uint32_t)i32_to_bf16((int32_t)a.w) << 16);
    o.z = (uint32_t)i32_to_bf16((int32_t)b.x) | ((uint32_t)i32_to_bf16((int32_t)b.y) << 16);
    o.w = (uint32_t)i32_to_bf16((int32_t)b.z) | ((uint32_t)i32_to_bf16((int32_t)b.w) << 16);
    st_stream16(out + i, o);
  }
}

__global__ void narrow_i32_scalar_k(const int32_t *__restrict__ in, uint16_t *__restrict__ out,
                                    int64_t lo, int64_t n) {
  for (int64_t i = lo + blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    out[i] = i32_to_bf16(in[i]);
}

// ---- GELU -------------------------------------------------------------------

// gelu_erf.cc:79-145: A&S 7.1.26 erf with the AIE exp2, unfused steps.
__device__ __forceinline__ float gelu_erf_as(float x) {
  const float u = mul_rn(x, 0.70710678118654752440f);
  const float au = fabsf(u);
  const float t = __fdiv_rn(1.0f, add_rn(1.0f, mul_rn(0.3275911f, au)));
  float p = 1.061405429f;
  p = add_rn(mul_rn(p, t), -1.453152027f);
  p = add_rn(mul_rn(p, t), 1.421413741f);
  p = add_rn(mul_rn(p, t), -0.284496736f);
  p = add_rn(mul_rn(p, t), 0.254829592f);
  float z = mul_rn(sub_rn(0.0f, mul_rn(u, u)), 1.4426950408889634f);
  z = z > -125.0f ? z : -125.0f;
  const float ex = exp2_poly_aie(z);
  const float eabs = sub_rn(1.0f, mul_rn(mul_rn(t, p), ex));
  return add_rn(mul_rn(x, 0.5f), mul_rn(mul_rn(fabsf(x), 0.5f), eabs));
}

__device__ __forceinline__ float gelu_variant(float v, int variant) {
  if (variant == 0) return gelu_poly(v);
  if (variant == 1) return gelu_erf(v);
  return gelu_erf_as(v);
}

// Eight elements per thread per step in 16-byte accesses (a bf16 chunk is one
// 16-byte load or store, an fp32 chunk two), the variant fixed at compile
// time; in place is safe (each chunk is read whole before it is written).
// fp32 input is read, and its bf16 result written, with streaming accesses
// (53 us against 55 at FFN-up's 17,455 x 3,072); bf16 input, which the GEMM
// before it has just written and the last-level cache still holds, stays on
// cached accesses (32.7 us against 36 with streaming ones).
template <bool IN_BF, bool OUT_BF, int VAR>
__global__ __launch_bounds__(256) void gelu_vec_k(const void *__restrict__ x,
                                                  void *__restrict__ y, int64_t n8) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n8;
       i += (int64_t)gridDim.x * blockDim.x) {
    float v[8];
    if (IN_BF) {
      const uint4 w = ((const uint4 *)x)[i];
      const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[2 * e] = bf2f(u[e] & 0xFFFFu);
        v[2 * e + 1] = bf2f(u[e] >> 16);
      }
    } else {
      const uint4 a = ld_stream16((const float4 *)x + 2 * i),
                  b = ld_stream16((const float4 *)x + 2 * i + 1);
      v[0] = __uint_as_float(a.x), v[1] = __uint_as_float(a.y);
      v[2] = __uint_as_float(a.z), v[3] = __uint_as_float(a.w);
      v[4] = __uint_as_float(b.x), v[5] = __uint_as_float(b.y);
      v[6] = __uint_as_float(b.z), v[7] = __uint_as_float(b.w);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = gelu_variant(v[e], VAR);
    if (OUT_BF) {
      const uint4 o = make_uint4(pack_bf2(v[0], v[1]), pack_bf2(v[2], v[3]),
                                 pack_bf2(v[4], v[5]), pack_bf2(v[6], v[7]));
      if (IN_BF)
        ((uint4 *)y)[i] = o;
      else
        st_stream16((uint4 *)y + i, o);
    } else {
      ((float4 *)y)[2 * i] = make_float4(v[0], v[1], v[2], v[3]);
      ((float4 *)y)[2 * i + 1] = make_float4(v[4], v[5], v[6], v[7]);
    }
  }
}

// The elements from lo on, one per thread (tails and unaligned tensors).
template <bool IN_BF, bool OUT_BF>
__global__ void gelu_k(const void *__restrict__ x, void *__restrict__ y, int64_t lo, int64_t n,
                       int variant) {
  for (int64_t i = lo + blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const float v = IN_BF ? bf2f(((const uint16_t *)x)[i]) : ((const float *)x)[i];
    const float r = gelu_variant(v, variant);
    if (OUT_BF)
      ((uint16_t *)y)[i] = f2bf(r);
    else
      ((float *)y)[i] = r;
  }
}

// ---- LayerNorm: one wave per row, NP pairs of columns per lane --------------

template <int NP>
__global__ __launch_bounds__(256) void layernorm_wave_k(
    const void *__restrict__ x, int x_bf, const void *__restrict__ y, int y_bf,
    const float *__restrict__ gamma, const float *__restrict__ beta, float eps,
    int64_t rows, float *out_f32, uint16_t *out_bf16, const int32_t *rows_dev) {
  constexpr int cols = NP * 128;
  const int lane = threadIdx.x & 63;
  const int64_t row = blockIdx.x * (int64_t)(blockDim.x / 64) + (threadIdx.x >> 6);
  if (row >= live_rows(rows, rows_dev)) return;
  float v[2 * NP];
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    const int64_t off = row * cols + i * 128 + lane * 2;
    float a0, a1;
    if (x_bf) {
      const uint32_t p = *(const uint32_t *)((const uint16_t *)x + off);
      a0 = bf2f(p & 0xFFFFu);
      a1 = bf2f(p >> 16);
    } else {
      const float2 p = *(const float2 *)((const float *)x + off);
      a0 = p.x;
      a1 = p.y;
    }
    if (y) {
      if (y_bf) {
        const uint32_t p = *(const uint32_t *)((const uint16_t *)y + off);
        a0 += bf2f(p & 0xFFFFu);
        a1 += bf2f(p >> 16);
      } else {
        const float2 p = *(const float2 *)((const float *)y + off);
        a0 += p.x;
        a1 += p.y;
      }
    }
    v[2 * i] = a0;
    v[2 * i + 1] = a1;
  }
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < 2 * NP; ++i) s += v[i];
  const float mean = wave_sum(s) / (float)cols;
  float q = 0.0f;
#pragma unroll
  for (int i = 0; i < 2 * NP; ++i) {
    const float d = v[i] - mean;
    q = __builtin_fmaf(d, d, q);
  }
  const float var = wave_sum(q) / (float)cols;
  const float is = 1.0f / sqrtf(var + eps);
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    const int c = i * 128 + lane * 2;
    const float2 g = *(const float2 *)(gamma + c);
    const float2 b = *(const float2 *)(beta + c);
    const float r0 = __builtin_fmaf((v[2 * i] - mean) * is, g.x, b.x);
    const float r1 = __builtin_fmaf((v[2 * i + 1] - mean) * is, g.y, b.y);
    const int64_t off = row * cols + c;
    if (out_f32) *(float2 *)(out_f32 + off) = make_float2(r0, r1);
    if (out_bf16) *(uint32_t *)(out_bf16 + off) = pack_bf2(r0, r1);
  }
}

// The same with four consecutive values per lane per access (16-byte fp32 /
// 8-byte bf16 loads and stores): NQ quads of 256 columns.
//
// ST: the residual LayerNorm of a post-LN layer, x <- LN(x + y) in place. x's
// old value and y (the GEMM result) are dead once read, and the new x is next
// read by the following residual LayerNorm, a GEMM and attention later. Their
// accesses stream (nontemporal), so the 160 MB this kernel moves at 17,455
// rows x 768 does not evict the GEMMs' operands from the caches: the kernel
// itself takes 1-2 us longer, but the GEMMs and attention around it gain more
// (bge-base b64 x s512, two lanes: 15,950-16,013 -> 16,561-16,629 seq/s). The
// bf16 copy, the next GEMM's A operand, stays on cached stores (streaming it
// gave 16,111-16,230).
template <bool ST>
__device__ __forceinline__ float4 ld4(const void *p, int bf, int64_t off) {
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

template <int NQ, bool ST>
__global__ __launch_bounds__(256) void layernorm_wave4_k(
    const void *__restrict__ x, int x_bf, const void *__restrict__ y, int y_bf,
    const float *__restrict__ gamma, const float *__restrict__ beta, float eps,
    int64_t rows, float *out_f32, uint16_t *out_bf16, const int32_t *rows_dev) {
  constexpr int cols = NQ * 256;
  const int lane = threadIdx.x & 63;
  const int64_t row = blockIdx.x * (int64_t)(blockDim.x / 64) + (threadIdx.x >> 6);
  if (row >= live_rows(rows, rows_dev)) return;
  // gamma and beta are read with the row, so their latency runs under its
  // loads instead of after the two reductions.
  float4 gm[NQ], bt[NQ];
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    gm[i] = *(const float4 *)(gamma + i * 256 + lane * 4);
    bt[i] = *(const float4 *)(beta + i * 256 + lane * 4);
  }
  float4 v[NQ];
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    const int64_t off = row * cols + i * 256 + lane * 4;
    v[i] = ld4<ST>(x, x_bf, off);
    if (y) {
      const float4 w = ld4<ST>(y, y_bf, off);
      v[i].x += w.x;
      v[i].y += w.y;
      v[i].z += w.z;
      v[i].w += w.w;
    }
  }
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < NQ; ++i) s += (v[i].x + v[i].y) + (v[i].z + v[i].w);
  const float mean = wave_sum(s) / (float)cols;
  float q = 0.0f;
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    const float a = v[i].x - mean, b = v[i].y - mean, c = v[i].z - mean, d = v[i].w - mean;
    q = __builtin_fmaf(a, a, q);
    q = __builtin_fmaf(b, b, q);
    q = __builtin_fmaf(c, c, q);
    q = __builtin_fmaf(d, d, q);
  }
  const float var = wave_sum(q) / (float)cols;
  const float is = 1.0f / sqrtf(var + eps);
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    const int c = i * 256 + lane * 4;
    float4 r;
    r.x = __builtin_fmaf((v[i].x - mean) * is, gm[i].x, bt[i].x);
    r.y = __builtin_fmaf((v[i].y - mean) * is, gm[i].y, bt[i].y);
    r.z = __builtin_fmaf((v[i].z - mean) * is, gm[i].z, bt[i].z);
    r.w = __builtin_fmaf((v[i].w - mean) * is, gm[i].w, bt[i].w);
    const int64_t off = row * cols + c;
    if (out_f32) {
      if (ST)
        st_stream16(out_f32 + off, make_uint4(__float_as_uint(r.x), __float_as_uint(r.y),
                                              __float_as_uint(r.z), __float_as_uint(r.w)));
      else
        *(float4 *)(out_f32 + off) = r;
    }
    if (out_bf16) *(uint2 *)(out_bf16 + off) = make_uint2(pack_bf2(r.x, r.y), pack_bf2(r.z, r.w));
  }
}

// Any width: one 256-thread block per row, two passes through global memory.
__global__ __launch_bounds__(256) void layernorm_any_k(
    const void *__restrict__ x, int x_bf, const void *__restrict__ y, int y_bf,
    const float *__restrict__ gamma, const float *__restrict__ beta, float eps,
    int64_t rows, int64_t cols, float *out_f32, uint16_t *out_bf16, const int32_t *rows_dev) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  if (row >= live_rows(rows, rows_dev)) return;
  auto load = [&](int64_t c) {
    const int64_t off = row * cols + c;
    float a = x_bf ? bf2f(((const uint16_t *)x)[off]) : ((const float *)x)[off];
    if (y) a += y_bf ? bf2f(((const uint16_t *)y)[off]) : ((const float *)y)[off];
    return a;
  };
  auto block_sum = [&](float s) {
    s = wave_sum(s);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    return red[0] + red[1] + red[2] + red[3];
  };
  float s = 0.0f;
  for (int64_t c = threadIdx.x; c < cols; c += 256) s += load(c);
  const float mean = block_sum(s) / (float)cols;
  float q = 0.0f;
  for (int64_t c = threadIdx.x; c < cols; c += 256) {
    const float d = load(c) - mean;
    q = __builtin_fmaf(d, d, q);
  }
  const float var = block_sum(q) / (float)cols;
  const float is = 1.0f / sqrtf(var + eps);
  for (int64_t c = threadIdx.x; c < cols; c += 256) {
    const float r = __builtin_fmaf((load(c) - mean) * is, gamma[c], beta[c]);
    if (out_f32) out_f32[row * cols + c] = r;
    if (out_bf16) out_bf16[row * cols + c] = f2bf(r);
  }
}

// ---- LayerNorm with the accelerator kernel's arithmetic ---------------------
// kernels/layernorm.cc:85-142 under layernorm_rne.cc's conv_even: bf16 in and
// out; 16 fp32 partial sums per pass (column j into sum j % 16, in column
// order), the 16 added in order (aie::reduce_add's order is not defined by
// the reference; lane 0 to 15 in turn is an assumption shared with the
// oracle); the biased variance about that mean;
// fast_invsqrt of var + eps (the 0x5f3759df estimate and two Newton steps,
// layernorm.cc:65-75); y = (d * inv_std) * gamma + beta narrowed to bf16 to
// nearest even. Every product and sum rounds on its own (no FMA).
// One wave normalises 4 rows: the rows reach LDS by 16-byte loads, lanes
// 16r .. 16r + 15 keep row r's 16 partial sums (lane 16r + l is sum l), each
// of them adds the 16 in order itself, and the results leave in 16-byte
// stores. The 4 rows are in LDS before any is written, so out may alias x.
__device__ __forceinline__ float fast_invsqrt_aie(float x) {
  const float xhalf = mul_rn(0.5f, x);
  int i = __float_as_int(x);
  i = 0x5f3759df - (i >> 1);
  float y = __int_as_float(i);
  y = mul_rn(y, sub_rn(1.5f, mul_rn(mul_rn(xhalf, y), y)));
  y = mul_rn(y, sub_rn(1.5f, mul_rn(mul_rn(xhalf, y), y)));
  return y;
}

__global__ __launch_bounds__(64) void layernorm_aie_k(const uint16_t *__restrict__ x,
                                                      const float *__restrict__ gamma,
                                                      const float *__restrict__ beta, float eps,
                                                      float inv_cols, int64_t rows, int cols,
                                                      uint16_t *out) {
  extern __shared__ __attribute__((aligned(16))) uint16_t srow[];  // [4][cols]
  const int lane = threadIdx.x;
  const int64_t r0 = (int64_t)blockIdx.x * 4;
  const int nr = rows - r0 < 4 ? (int)(rows - r0) : 4;
  const int cpr = cols / 8;  // 16-byte chunks per row
  for (int c = lane; c < nr * cpr; c += 64) {
    const int r = c / cpr, k = c - r * cpr;
    *(uint4 *)(srow + r * cols + k * 8) = *(const uint4 *)(x + (r0 + r) * cols + k * 8);
  }
  __syncthreads();
  const int r = lane >> 4, l = lane & 15, lead = lane & ~15;
  const bool live = r < nr;
  const uint16_t *xr = srow + (live ? r : 0) * cols;
  float acc = 0.0f;
  if (live)
    for (int j = l; j < cols; j += 16) acc = add_rn(acc, bf2f(xr[j]));
  float sum = 0.0f;
#pragma unroll
  for (int q = 0; q < 16; ++q) sum = add_rn(sum, __shfl(acc, lead + q));
  const float mean = mul_rn(sum, inv_cols);
  float acc2 = 0.0f;
  if (live)
    for (int j = l; j < cols; j += 16) {
      const float d = sub_rn(bf2f(xr[j]), mean);
      acc2 = add_rn(acc2, mul_rn(d, d));
    }
  float vs = 0.0f;
#pragma unroll
  for (int q = 0; q < 16; ++q) vs = add_rn(vs, __shfl(acc2, lead + q));
  const float inv_std = fast_invsqrt_aie(add_rn(mul_rn(vs, inv_cols), eps));
  if (!live) return;
  for (int k = l; k < cpr; k += 16) {
    const uint4 raw = *(const uint4 *)(xr + k * 8);
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
    const float4 g0 = *(const float4 *)(gamma + k * 8), g1 = *(const float4 *)(gamma + k * 8 + 4);
    const float4 b0 = *(const float4 *)(beta + k * 8), b1 = *(const float4 *)(beta + k * 8 + 4);
    const float g[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
    const float b[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float y2[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const float d = sub_rn(bf2f(h ? w[e] >> 16 : w[e] & 0xFFFFu), mean);
        y2[h] = add_rn(mul_rn(mul_rn(d, inv_std), g[2 * e + h]), b[2 * e + h]);
      }
      o[e] = pack_bf2(y2[0], y2[1]);
    }
    *(uint4 *)(out + (r0 + r) * cols + k * 8) = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// ---- softmax: one wave per row, NV values per lane (cols <= 64 * NV) --------

template <int NV>
__global__ __launch_bounds__(256) void softmax_wave_k(void *x, int bf, int64_t rows,
                                                      int64_t cols, int64_t stride,
                                                      const float *__restrict__ mask,
                                                      int64_t rpm, int variant) {
  const int lane = threadIdx.x & 63;
  const int64_t row = blockIdx.x * (int64_t)(blockDim.x / 64) + (threadIdx.x >> 6);
  if (row >= rows) return;
  const float *mk = mask ? mask + (row / rpm) * cols : nullptr;
  float v[NV];
  float m = -INFINITY;
  const float lo_aie = bf2f(f2bf(-1.0e30f));
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int64_t c = lane + 64 * i;
    float a = -INFINITY;
    if (c < cols) {
      a = bf ? bf2f(((const uint16_t *)x)[row * stride + c]) : ((const float *)x)[row * stride + c];
      if (variant == 2) {
        a = a > lo_aie ? a : lo_aie;  // softmax.cc clamp 1, in bf16
      } else if (mk) {
        a += mk[c];
      }
      m = fmaxf(m, a);
    }
    v[i] = a;
  }
  m = wave_max(m);
  if (variant == 2) m = fmaxf(m, -1.0e30f);  // softmax.cc's running max starts at -1e30
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int64_t c = lane + 64 * i;
    float e = 0.0f;
    if (c < cols) {
      if (variant == 0) {
        float a = (v[i] - m) * 1.4426950408889634f;
        a = a > -120.0f ? a : -120.0f;
        e = exp2_poly_neg(a);
      } else if (variant == 1) {
        e = expf(v[i] - m);
      } else {
        float d = v[i] - m;
        d = d > -100.0f ? d : -100.0f;
        float a = mul_rn(d, 1.4426950408889634f);
        a = a > -120.0f ? a : -120.0f;
        e = bf2f(f2bf(exp2_poly_aie_neg(a)));
      }
      if (variant != 2) s += e;
    }
    v[i] = e;
  }
  if (variant == 2) {
    // softmax.cc:115-145's 16-lane accumulator: column j into partial sum
    // j % 16 in column order (columns l, l + 16, l + 32, l + 48 of each
    // 64-column group sit in lanes l .. l + 48), then the 16 in order (the
    // assumed order of aie::reduce_add, as in the oracle). Lanes 0 .. 15 hold
    // the partial sums; every lane adds them itself.
    float part = 0.0f;
    const int l = lane & 15;
#pragma unroll
    for (int i = 0; i < NV; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float t = __shfl(v[i], l + 16 * q);
        if (64 * i + 16 * q + l < cols) part = add_rn(part, t);
      }
    s = 0.0f;
#pragma unroll
    for (int q = 0; q < 16; ++q) s = add_rn(s, __shfl(part, q));
  } else {
    s = wave_sum(s);
  }
  const float inv = variant == 1 ? (s > 0.0f ? 1.0f / s : 0.0f) : 1.0f / s;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int64_t c = lane + 64 * i;
    if (c < cols) {
      const float r = v[i] * inv;
      if (bf)
        ((uint16_t *)x)[row * stride + c] = f2bf(r);
      else
        ((float *)x)[row * stride + c] = r;
    }
  }
}

// The poly (0) and exact (1) softmax on 16-byte accesses: one wave per NR
// rows, whose loads are all issued before the first row's reductions (a row
// of 512 bf16 is 1 KB, too little in flight alone); lane l holds the
// 8-column chunks l, l + 64, ... of each row (cols <= 512 * NC). cols and the
// row stride multiples of 8, 16-byte aligned rows and mask. bf16 rows are
// read and written with streaming accesses (each is touched once): 141-146 us
// against 155-157 with cached ones at 393,216 x 512. fp32 rows stay cached,
// which measured faster for them (292-296 us against 319-325). The mask rows,
// re-read by every head, always go through the caches.
template <int NC, int NR, bool BF, int VAR>
__global__ __launch_bounds__(256) void softmax_vec_k(void *x, int64_t rows, int64_t cols,
                                                     int64_t stride,
                                                     const float *__restrict__ mask,
                                                     int64_t rpm) {
  const int lane = threadIdx.x & 63;
  const int64_t row0 = (blockIdx.x * (int64_t)(blockDim.x / 64) + (threadIdx.x >> 6)) * NR;
  if (row0 >= rows) return;
  float v[NR][NC][8];
  // The mask row of row0 + r: one division per wave (row0 / rpm, the rest
  // carried), not one per row -- a 64-bit division is dozens of vector
  // instructions.
  int64_t mrow = 0, mrem = 0;
  if (mask) {
    mrow = row0 / rpm;
    mrem = row0 - mrow * rpm;
  }
  // The mask entries are read with the rows (added to them right away), so
  // their latency runs under the row loads instead of after them.
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const int64_t row = row0 + r;
    if (r > 0 && ++mrem == rpm) {
      mrem = 0;
      ++mrow;
    }
    const float *mk = mask && row < rows ? mask + mrow * cols : nullptr;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int64_t c0 = 8 * (lane + 64 * (int64_t)i);
      float4 ma = make_float4(0.0f, 0.0f, 0.0f, 0.0f), mb = ma;
      if (mk && c0 < cols) {
        ma = *(const float4 *)(mk + c0);
        mb = *(const float4 *)(mk + c0 + 4);
      }
      const float mm[8] = {ma.x, ma.y, ma.z, ma.w, mb.x, mb.y, mb.z, mb.w};
      if (row < rows && c0 < cols) {
        if (BF) {
          const uint4 w = ld_stream16((const uint16_t *)x + row * stride + c0);
          const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            v[r][i][2 * e] = bf2f(u[e] & 0xFFFFu);
            v[r][i][2 * e + 1] = bf2f(u[e] >> 16);
          }
        } else {
          const float *p = (const float *)x + row * stride + c0;
          const float4 a = *(const float4 *)p, b = *(const float4 *)(p + 4);
          v[r][i][0] = a.x, v[r][i][1] = a.y, v[r][i][2] = a.z, v[r][i][3] = a.w;
          v[r][i][4] = b.x, v[r][i][5] = b.y, v[r][i][6] = b.z, v[r][i][7] = b.w;
        }
        if (mk) {
#pragma unroll
          for (int e = 0; e < 8; ++e) v[r][i][e] += mm[e];
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const int64_t row = row0 + r;
    if (row >= rows) break;
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int64_t c0 = 8 * (lane + 64 * (int64_t)i);
      if (c0 < cols) {
#pragma unroll
        for (int e = 0; e < 8; ++e) m = fmaxf(m, v[r][i][e]);
      }
    }
    m = wave_max(m);
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int64_t c0 = 8 * (lane + 64 * (int64_t)i);
      if (c0 < cols) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float ex;
          if (VAR == 0) {
            float a = (v[r][i][e] - m) * 1.4426950408889634f;
            a = a > -120.0f ? a : -120.0f;
            ex = exp2_poly_neg(a);
          } else {
            ex = expf(v[r][i][e] - m);
          }
          v[r][i][e] = ex;
          sum += ex;
        }
      }
    }
    sum = wave_sum(sum);
    const float inv = VAR == 1 ? (sum > 0.0f ? 1.0f / sum : 0.0f) : 1.0f / sum;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int64_t c0 = 8 * (lane + 64 * (int64_t)i);
      if (c0 < cols) {
        float o[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = v[r][i][e] * inv;
        if (BF) {  // the hardware conversion: the same bits for every non-NaN value
          st_stream16((uint16_t *)x + row * stride + c0,
                      make_uint4(pack_bf2_hw(o[0], o[1]), pack_bf2_hw(o[2], o[3]),
                                 pack_bf2_hw(o[4], o[5]), pack_bf2_hw(o[6], o[7])));
        } else {
          float *p = (float *)x + row * stride + c0;
          *(float4 *)p = make_float4(o[0], o[1], o[2], o[3]);
          *(float4 *)(p + 4) = make_float4(o[4], o[5], o[6], o[7]);
        }
      }
    }
  }
}

// ---- embedding sum + mask ---------------------------------------------------

__global__ __launch_bounds__(256) void embed_sum_k(const int32_t *__restrict__ ids, int64_t rows,
                                                   int64_t S, int64_t d,
                                                   const float *__restrict__ word, int64_t vocab,
                                                   const float *__restrict__ pos,
                                                   const float *__restrict__ type0,
                                                   float *__restrict__ emb, int *err) {
  const int lane = threadIdx.x & 63;
  const int64_t r = blockIdx.x * (int64_t)(blockDim.x / 64) + (threadIdx.x >> 6);
  if (r >= rows) return;
  const int32_t id = ids[r];
  const int64_t s = r % S;
  if (id < 0 || id >= vocab) {
    if (lane == 0) atomicOr(err, 1);
    for (int64_t c = lane; c < d; c += 64) emb[r * d + c] = 0.0f;
    return;
  }
  const float *wv = word + (int64_t)id * d;
  const float *pv = pos + s * d;
  for (int64_t c = lane; c < d; c += 64) emb[r * d + c] = (wv[c] + pv[c]) + type0[c];
}

// kv_len[b] = 1 + the last position with m != 0: every row pooling reads
// (pool_rows weights every row with m != 0, negative ones included) and every
// key attention can weight (m > 0) lies before it. A row with no m > 0 attends
// uniformly over all S keys, as the reference's all -1e30 row does, so it
// keeps S.
__global__ __launch_bounds__(256) void mask_k(const float *__restrict__ am, int64_t S,
                                              float *add_mask, int32_t *kv_len) {
  __shared__ int last_pos, last_nz;
  if (threadIdx.x == 0) last_pos = last_nz = 0;
  __syncthreads();
  const int64_t b = blockIdx.x;
  int pos = 0, nz = 0;
  for (int64_t s = threadIdx.x; s < S; s += blockDim.x) {
    const float m = am[b * S + s];
    if (add_mask) add_mask[b * S + s] = m > 0.0f ? 0.0f : -1.0e30f;
    if (m > 0.0f) pos = (int)s + 1;
    if (m != 0.0f) nz = (int)s + 1;
  }
  atomicMax(&last_pos, pos);
  atomicMax(&last_nz, nz);
  __syncthreads();
  if (threadIdx.x == 0 && kv_len) kv_len[b] = last_pos > 0 ? last_nz : (int32_t)S;
}

// ---- token packing: only the rows pooling can see ---------------------------
// Sequence b keeps its rows s < kv_len[b] (every row past it is masked: it is
// never attended as a key and its output is never pooled). seq_start is the
// exclusive scan of kv_len, seq_start[B] the packed row count; packed row
// seq_start[b] + s is dense row b*S + s, and row_pos records its position s.

// One block: seq_start (thread 0, an exclusive prefix sum of kv_len) and the
// attention launch order -- the sequence indices by decreasing kv_len, ties by
// index: order[rank(b)] = b with rank(b) = #{b' : kv_len[b'] > kv_len[b], or
// equal and b' < b}, a permutation by construction. Past ORDER_MAX_B sequences
// the quadratic ranking is skipped and the order is the identity.
constexpr int64_t ORDER_MAX_B = 8192;
__global__ __launch_bounds__(256) void pack_plan_k(const int32_t *__restrict__ kv_len, int64_t B,
                                                   int32_t *__restrict__ seq_start,
                                                   int32_t *__restrict__ order,
                                                   int32_t *__restrict__ total_out) {
  if (threadIdx.x == 0) {
    int32_t acc = 0;
    for (int64_t b = 0; b < B; ++b) {
      seq_start[b] = acc;
      acc += kv_len[b];
    }
    seq_start[B] = acc;
    if (total_out) *total_out = acc;
  }
  if (!order) return;
  for (int64_t b = threadIdx.x; b < B; b += blockDim.x) {
    int64_t rank = b;
    if (B <= ORDER_MAX_B) {
      const int32_t lb = kv_len[b];
      rank = 0;
      for (int64_t o = 0; o < B; ++o) {
        const int32_t lo = kv_len[o];
        rank += (lo > lb) || (lo == lb && o < b);
      }
    }
    order[rank] = (int32_t)b;
  }
}

template <bool V4>
__global__ __launch_bounds__(256) void embed_sum_packed_k(
    const int32_t *__restrict__ ids, int64_t rows, int64_t S, int64_t d,
    const float *__restrict__ word, int64_t vocab, const float *__restrict__ pos,
    const float *__restrict__ type0, const int32_t *__restrict__ kv_len,
    const int32_t *__restrict__ seq_start, float *__restrict__ emb, int32_t *__restrict__ row_pos,
    int *err) {
  const int lane = threadIdx.x & 63;
  const int64_t r = blockIdx.x * (int64_t)(blockDim.x / 64) + (threadIdx.x >> 6);
  if (r >= rows) return;
  const int64_t b = r / S, s = r - b * S;
  if (s >= kv_len[b]) return;
  const int64_t p = seq_start[b] + s;
  if (lane == 0) row_pos[p] = (int32_t)s;
  const int32_t id = ids[r];
  if (id < 0 || id >= vocab) {
    if (lane == 0) atomicOr(err, 1);
    for (int64_t c = lane; c < d; c += 64) emb[p * d + c] = 0.0f;
    return;
  }
  const float *wv = word + (int64_t)id * d;
  const float *pv = pos + s * d;
  if (V4) {  // d % 4 == 0 and 16-byte aligned rows: four columns per lane
    for (int64_t c = 4 * lane; c < d; c += 256) {
      const float4 w = *(const float4 *)(wv + c), q = *(const float4 *)(pv + c);
      const float4 t = *(const float4 *)(type0 + c);
      *(float4 *)(emb + p * d + c) =
          make_float4((w.x + q.x) + t.x, (w.y + q.y) + t.y, (w.z + q.z) + t.z, (w.w + q.w) + t.w);
    }
  } else {
    for (int64_t c = lane; c < d; c += 64) emb[p * d + c] = (wv[c] + pv[c]) + type0[c];
  }
}

// ---- pooling (app_state.hpp:335-374), bit-exact with the host form ----------

// One block per sequence, one column per thread (d <= 1024; beyond, the
// threads take the columns in rounds). Each column's sum runs over s in
// order, in double, as the host's does. The mask row reaches LDS a chunk at a
// time; the rows' loads are issued POOL_U at a time ahead of their adds (a
// masked row's load reads the buffer's first element instead, and its term
// is an exact +0.0: the running sum starts at +0.0 and can never be -0.0, so
// adding it is the host's skip), which keeps the in-order chain from waiting
// on one load per row. Every thread forms the float denominator itself, in
// the same order.
constexpr int POOL_U = 16, POOL_CH = 1024;

__global__ __launch_bounds__(1024) void pool_k(const float *__restrict__ h,
                                               const float *__restrict__ am, int64_t S,
                                               int64_t d, int cls, int l2, float *out,
                                               int *err, const int32_t *__restrict__ seq_start,
                                               int compact) {
  extern __shared__ double acc[];
  __shared__ double nrm_s;
  __shared__ __align__(16) float msk[POOL_CH];
  const int64_t b = blockIdx.x;
  const float *amb = am + b * S;
  // Packed rows: the loop below reads row s only where the mask is nonzero,
  // i.e. only rows s < kv_len[b], the ones packing kept. compact (CLS
  // pooling): h holds only the sequences' first rows, row b for sequence b.
  const float *hb = h + (compact ? b : seq_start ? (int64_t)seq_start[b] : b * S) * d;
  if (cls) {
    if (amb[0] == 0.0f) {
      if (threadIdx.x == 0) atomicOr(err, 2);
      for (int64_t c = threadIdx.x; c < d; c += blockDim.x) out[b * d + c] = 0.0f;
      return;
    }
    for (int64_t c = threadIdx.x; c < d; c += blockDim.x) acc[c] = (double)hb[c];
  } else {
    const int64_t rounds = (d + blockDim.x - 1) / blockDim.x;
    for (int64_t rd = 0; rd < rounds; ++rd) {
      const int64_t c = rd * blockDim.x + threadIdx.x;
      const bool live = c < d;
      double a = 0.0;
      float den = 0.0f;
      for (int64_t sb = 0; sb < S; sb += POOL_CH) {
        const int n = (int)(S - sb < POOL_CH ? S - sb : POOL_CH);
        __syncthreads();
        for (int i = threadIdx.x; i < n; i += blockDim.x) msk[i] = amb[sb + i];
        __syncthreads();
        for (int i0 = 0; i0 < n; i0 += POOL_U) {
          float m[POOL_U], v[POOL_U];
#pragma unroll
          for (int q = 0; q < POOL_U / 4; ++q) {  // in bounds: POOL_CH % POOL_U == 0
            const float4 x = *(const float4 *)(msk + i0 + 4 * q);
            m[4 * q] = x.x;
            m[4 * q + 1] = x.y;
            m[4 * q + 2] = x.z;
            m[4 * q + 3] = x.w;
          }
#pragma unroll
          for (int u = 0; u < POOL_U; ++u) {
            m[u] = i0 + u < n ? m[u] : 0.0f;
            const float *p = live && m[u] != 0.0f ? hb + (sb + i0 + u) * d + c : h;
            v[u] = *p;
          }
#pragma unroll
          for (int u = 0; u < POOL_U; ++u) {
            if (i0 + u < n) den += m[u];
            a += m[u] != 0.0f ? (double)(mul_rn(v[u], m[u])) : 0.0;
          }
        }
      }
      if (live) acc[c] = a / (double)(den > 1e-9f ? den : 1e-9f);
    }
  }
  __syncthreads();
  if (l2) {
    if (threadIdx.x == 0) {
      // In column order, POOL_U values read ahead of their FMAs.
      double n = 0.0;
      int64_t c0 = 0;
      for (; c0 + POOL_U <= d; c0 += POOL_U) {
        double x[POOL_U];
#pragma unroll
        for (int u = 0; u < POOL_U; ++u) x[u] = acc[c0 + u];
#pragma unroll
        for (int u = 0; u < POOL_U; ++u) n = __builtin_fma(x[u], x[u], n);
      }
      for (; c0 < d; ++c0) n = __builtin_fma(acc[c0], acc[c0], n);
      nrm_s = sqrt(n > 1e-24 ? n : 1e-24);
    }
    __syncthreads();
    const double nrm = nrm_s;
    for (int64_t c = threadIdx.x; c < d; c += blockDim.x) out[b * d + c] = (float)(acc[c] / nrm);
  } else {
    for (int64_t c = threadIdx.x; c < d; c += blockDim.x) out[b * d + c] = (float)acc[c];
  }
}

}  // namespace

namespace mxk {

hipError_t narrow_f32_bf16(const float *in, uint16_t *out, int64_t n, hipStream_t s) {
  int64_t done = 0;
  if (((uintptr_t)in % 16 == 0) && ((uintptr_t)out % 16 == 0) && n >= 8) {
    const int64_t n8 = n / 8;
    narrow_f32_vec_k<<<grid_for(n8, kElemThreads), kElemThreads, 0, s>>>(
        (const float4 *)in, (uint4 *)out, n8);
    done = n8 * 8;
  }
  if (done < n)
    narrow_f32_scalar_k<<<grid_for(n - done, kElemThreads), kElemThreads, 0, s>>>(in, out, done,
                                                                                  n);
  return hipGetLastError();
}

hipError_t narrow_i32_bf16(const int32_t *in, uint16_t *out, int64_t n, hipStream_t s) {
  int64_t done = 0;
  if (((uintptr_t)in % 16 == 0) && ((uintptr_t)out % 16 == 0) && n >= 8) {
    const int64_t n8 = n / 8;
    narrow_i32_vec_k<<<grid_for(n8, kElemThreads), kElemThreads, 0, s>>>((const int4 *)in,
                                                                        (uint4 *)out, n8);
    done = n8 * 8;
  }
  if (done < n)
    narrow_i32_scalar_k<<<grid_for(n - done, kElemThreads), kElemThreads, 0, s>>>(in, out, done,
                                                                                  n);
  return hipGetLastError();
}

template <bool IB, bool OB>
void gelu_vec_launch(const void *x, void *y, int64_t n8, int variant, hipStream_t s) {
  const int g = grid_for(n8, kElemThreads);
  if (variant == 0)
    gelu_vec_k<IB, OB, 0><<<g, kElemThreads, 0, s>>>(x, y, n8);
  else if (variant == 1)
    gelu_vec_k<IB, OB, 1><<<g, kElemThreads, 0, s>>>(x, y, n8);
  else
    gelu_vec_k<IB, OB, 2><<<g, kElemThreads, 0, s>>>(x, y, n8);
}

hipError_t gelu(const void *x, int x_bf, void *y, int y_bf, int64_t n, int variant,
                hipStream_t s) {
  int64_t done = 0;
  if ((uintptr_t)x % 16 == 0 && (uintptr_t)y % 16 == 0 && n >= 8) {
    const int64_t n8 = n / 8;
    if (x_bf && y_bf)
      gelu_vec_launch<true, true>(x, y, n8, variant, s);
    else if (x_bf)
      gelu_vec_launch<true, false>(x, y, n8, variant, s);
    else if (y_bf)
      gelu_vec_launch<false, true>(x, y, n8, variant, s);
    else
      gelu_vec_launch<false, false>(x, y, n8, variant, s);
    done = n8 * 8;
  }
  if (done < n) {
    const int g = grid_for(n - done, kElemThreads);
    if (x_bf && y_bf)
      gelu_k<true, true><<<g, kElemThreads, 0, s>>>(x, y, done, n, variant);
    else if (x_bf)
      gelu_k<true, false><<<g, kElemThreads, 0, s>>>(x, y, done, n, variant);
    else if (y_bf)
      gelu_k<false, true><<<g, kElemThreads, 0, s>>>(x, y, done, n, variant);
    else
      gelu_k<false, false><<<g, kElemThreads, 0, s>>>(x, y, done, n, variant);
  }
  return hipGetLastError();
}

hipError_t layernorm(const void *x, int x_bf, const void *y, int y_bf, const float *gamma,
                     const float *beta, float eps, int64_t rows, int64_t cols, float *out_f32,
                     uint16_t *out_bf16, hipStream_t s, const int32_t *rows_dev) {
  const int rpb = 4;  // rows (waves) per block
  const int g = (int)((rows + rpb - 1) / rpb);
  bool aligned = ((uintptr_t)x % 8 == 0) && (!y || (uintptr_t)y % 8 == 0) &&
                 ((uintptr_t)gamma % 8 == 0) && ((uintptr_t)beta % 8 == 0) &&
                 (!out_f32 || (uintptr_t)out_f32 % 8 == 0) &&
                 (!out_bf16 || (uintptr_t)out_bf16 % 4 == 0);
  const bool aligned16 = ((uintptr_t)x % (x_bf ? 8 : 16) == 0) &&
                         (!y || (uintptr_t)y % (y_bf ? 8 : 16) == 0) &&
                         ((uintptr_t)gamma % 16 == 0) && ((uintptr_t)beta % 16 == 0) &&
                         (!out_f32 || (uintptr_t)out_f32 % 16 == 0) &&
                         (!out_bf16 || (uintptr_t)out_bf16 % 8 == 0);
  // The post-LN residual form (x <- LN(x + y) in place) streams its accesses.
  const bool st = y && out_f32 && (const void *)out_f32 == x;
  if (aligned16 && cols % 256 == 0) {
#define MX_LN4_CASE(nq)                                                                   \
  case nq:                                                                                \
    if (st)                                                                               \
      layernorm_wave4_k<nq, true><<<g, 256, 0, s>>>(x, x_bf, y, y_bf, gamma, beta, eps,   \
                                                    rows, out_f32, out_bf16, rows_dev);   \
    else                                                                                  \
      layernorm_wave4_k<nq, false><<<g, 256, 0, s>>>(x, x_bf, y, y_bf, gamma, beta, eps,  \
                                                     rows, out_f32, out_bf16, rows_dev);  \
    return hipGetLastError();
    switch (cols / 256) {
      MX_LN4_CASE(1)
      MX_LN4_CASE(2)
      MX_LN4_CASE(3)
      MX_LN4_CASE(4)
      MX_LN4_CASE(5)
      MX_LN4_CASE(6)
      MX_LN4_CASE(8)
      default:
        break;
    }
#undef MX_LN4_CASE
  }
  if (aligned && cols % 128 == 0 && rows <= (int64_t)1 << 36) {
#define MX_LN_CASE(np)                                                                     \
  case np:                                                                                 \
    layernorm_wave_k<np><<<g, 256, 0, s>>>(x, x_bf, y, y_bf, gamma, beta, eps, rows,      \
                                           out_f32, out_bf16, rows_dev);                  \
    return hipGetLastError();
    switch (cols / 128) {
      MX_LN_CASE(1)
      MX_LN_CASE(2)
      MX_LN_CASE(3)
      MX_LN_CASE(4)
      MX_LN_CASE(5)
      MX_LN_CASE(6)
      MX_LN_CASE(7)
      MX_LN_CASE(8)
      MX_LN_CASE(10)
      MX_LN_CASE(12)
      MX_LN_CASE(16)
      default:
        break;
    }
#undef MX_LN_CASE
  }
  layernorm_any_k<<<(unsigned)rows, 256, 0, s>>>(x, x_bf, y, y_bf, gamma, beta, eps, rows, cols,
                                                 out_f32, out_bf16, rows_dev);
  return hipGetLastError();
}

hipError_t layernorm_aie(const uint16_t *x, const float *gamma, const float *beta, float eps,
                         int64_t rows, int64_t cols, uint16_t *out, hipStream_t s) {
  const int64_t g = (rows + 3) / 4;
  const size_t lds = (size_t)4 * cols * 2;
  const float inv_cols = 1.0f / (float)cols;
  layernorm_aie_k<<<(unsigned)g, 64, lds, s>>>(x, gamma, beta, eps, inv_cols, rows, (int)cols,
                                               out);
  return hipGetLastError();
}

template <int NC, bool BF>
hipError_t softmax_vec_launch(void *x, int64_t rows, int64_t cols, int64_t stride,
                              const float *mask, int64_t rpm, int variant, hipStream_t s) {
  // rows per wave (bf16): 32 values per lane held at most; an fp32 row moves
  // twice the bytes and runs fastest alone
  constexpr int NR = !BF || NC >= 4 ? 1 : 4 / NC;
  const int64_t g = (rows + 4 * NR - 1) / (4 * NR);
  if (variant == 0)
    softmax_vec_k<NC, NR, BF, 0><<<(unsigned)g, 256, 0, s>>>(x, rows, cols, stride, mask, rpm);
  else
    softmax_vec_k<NC, NR, BF, 1><<<(unsigned)g, 256, 0, s>>>(x, rows, cols, stride, mask, rpm);
  return hipGetLastError();
}

hipError_t softmax_rows(void *x, int bf, int64_t rows, int64_t cols, int64_t stride,
                        const float *mask, int64_t rpm, int variant, hipStream_t s) {
  const int g = (int)((rows + 3) / 4);
  // 16-byte chunks where the rows allow them (the accelerator form keeps the
  // strided layout, whose 16-lane summation order it reproduces)
  if (variant != 2 && cols % 8 == 0 && stride % 8 == 0 && (uintptr_t)x % 16 == 0 &&
      (!mask || (uintptr_t)mask % 16 == 0) && cols <= 4096) {
    const int64_t nc = (cols + 511) / 512;
#define MX_SMV_CASE(NC)                                                                   \
  if (nc <= NC)                                                                           \
    return bf ? softmax_vec_launch<NC, true>(x, rows, cols, stride, mask, rpm, variant, s) \
              : softmax_vec_launch<NC, false>(x, rows, cols, stride, mask, rpm, variant, s);
    MX_SMV_CASE(1)
    MX_SMV_CASE(2)
    MX_SMV_CASE(4)
    MX_SMV_CASE(8)
#undef MX_SMV_CASE
  }
  const int64_t nv = (cols + 63) / 64;
#define MX_SM_CASE(NV)                                                                      \
  if (nv <= NV) {                                                                           \
    softmax_wave_k<NV><<<g, 256, 0, s>>>(x, bf, rows, cols, stride, mask, rpm, variant);   \
    return hipGetLastError();                                                               \
  }
  MX_SM_CASE(2)
  MX_SM_CASE(4)
  MX_SM_CASE(8)
  MX_SM_CASE(16)
  MX_SM_CASE(32)
  MX_SM_CASE(64)
#undef MX_SM_CASE
  return hipErrorInvalidValue;
}

hipError_t embed_sum(const int32_t *ids, int64_t B, int64_t S, int64_t d, const float *word,
                     int64_t vocab, const float *pos, const float *type0, float *emb, int *err,
                     hipStream_t s) {
  const int64_t rows = B * S;
  embed_sum_k<<<(unsigned)((rows + 3) / 4), 256, 0, s>>>(ids, rows, S, d, word, vocab, pos,
                                                         type0, emb, err);
  return hipGetLastError();
}

hipError_t mask_build(const float *am, int64_t B, int64_t S, float *add_mask, int32_t *kv_len,
                      hipStream_t s) {
  mask_k<<<(unsigned)B, 256, 0, s>>>(am, S, add_mask, kv_len);
  return hipGetLastError();
}

hipError_t pool_rows(const float *h, const float *am, int64_t B, int64_t S, int64_t d, int cls,
                     int l2, float *out, int *err, hipStream_t s, const int32_t *seq_start,
                     bool compact) {
  if (compact && !cls) return hipErrorInvalidValue;
  const int nt = d >= 1024 ? 1024 : (int)((d + 63) / 64 * 64);
  pool_k<<<(unsigned)B, nt, (size_t)d * sizeof(double), s>>>(h, am, S, d, cls, l2, out, err,
                                                             seq_start, compact ? 1 : 0);
  return hipGetLastError();
}

// Sequence b's first row (seq_start[b], or b * S) of the fp32 residual
// stream x and of the bf16 attention context ctx, both [*, d], into row b of
// xc and ctxc. One block per sequence; d % 4 == 0, 16-byte aligned rows.
__global__ __launch_bounds__(256) void gather_cls_k(const float *__restrict__ x,
                                                    const uint16_t *__restrict__ ctx,
                                                    const int32_t *__restrict__ seq_start,
                                                    int64_t S, int64_t d, float *__restrict__ xc,
                                                    uint16_t *__restrict__ ctxc) {
  const int64_t b = blockIdx.x;
  const int64_t r = seq_start ? (int64_t)seq_start[b] : b * S;
  for (int64_t c = (int64_t)threadIdx.x * 4; c < d; c += (int64_t)blockDim.x * 4) {
    *(float4 *)(xc + b * d + c) = *(const float4 *)(x + r * d + c);
    *(uint2 *)(ctxc + b * d + c) = *(const uint2 *)(ctx + r * d + c);
  }
}

hipError_t gather_cls(const float *x, const uint16_t *ctx, const int32_t *seq_start, int64_t B,
                      int64_t S, int64_t d, float *xc, uint16_t *ctxc, hipStream_t s) {
  if (d % 4) return hipErrorInvalidValue;
  gather_cls_k<<<(unsigned)B, 256, 0, s>>>(x, ctx, seq_start, S, d, xc, ctxc);
  return hipGetLastError();
}

hipError_t pack_plan(const int32_t *kv_len, int64_t B, int32_t *seq_start, int32_t *order,
                     hipStream_t s, int32_t *total_out) {
  pack_plan_k<<<1, 256, 0, s>>>(kv_len, B, seq_start, order, total_out);
  return hipGetLastError();
}

hipError_t embed_sum_packed(const int32_t *ids, int64_t B, int64_t S, int64_t d,
                            const float *word, int64_t vocab, const float *pos,
                            const float *type0, const int32_t *kv_len, const int32_t *seq_start,
                            float *emb, int32_t *row_pos, int *err, hipStream_t s) {
  const int64_t rows = B * S;
  const bool v4 = d % 4 == 0 && (uintptr_t)word % 16 == 0 && (uintptr_t)pos % 16 == 0 &&
                  (uintptr_t)type0 % 16 == 0 && (uintptr_t)emb % 16 == 0;
  if (v4)
    embed_sum_packed_k<true><<<(unsigned)((rows + 3) / 4), 256, 0, s>>>(
        ids, rows, S, d, word, vocab, pos, type0, kv_len, seq_start, emb, row_pos, err);
  else
    embed_sum_packed_k<false><<<(unsigned)((rows + 3) / 4), 256, 0, s>>>(
        ids, rows, S, d, word, vocab, pos, type0, kv_len, seq_start, emb, row_pos, err);
  return hipGetLastError();
}

}  // namespace mxk
