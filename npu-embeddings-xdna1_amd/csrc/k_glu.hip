// k_glu.hip -- the two ops of the RoPE / gated-FFN BERT archs (nomic_bert_rope_swiglu,
// gte_new_rope_geglu) on gfx950, both memory-bound passes:
//
// rope_qkv_k: BertEncoder::apply_rope_qkv (bert_encoder.cpp:951-990) on the
// bf16 fused Q|K|V rows, in place, Q and K only. Position s = row % S (or the
// packed row's recorded position); per
// head the pairs (j, j + hd/2) rotate by the table's angle:
//   o1 = x1*c - x2*s,  o2 = x2*c + x1*s
// each product rounded as the host's AVX2 form (no fused multiply-add), the
// result narrowed once to bf16. Each thread moves four adjacent pairs (two
// when head_dim % 8 != 0 or the rows are not 8-byte aligned).
//
// glu_k: swiglu_cpu (bert_encoder.cpp:582-627): FFN-up's [rows, 2f] output as
// lo | hi halves -> [rows, f] = lo * act(hi), act SiLU with the host's
// exp2 polynomial and -120 argument floor (x / (1 + 2^max(-x log2e, -120))),
// or exact-erf GELU. Four consecutive outputs per thread. The encoder fuses
// this pass into FFN-up's GEMM epilogue where it can (k_gemm_lds.hpp, GLU),
// over FFN-up's operands put in glu_interleave_k's row order once; the
// product and its roundings are the same (glu_act).
#include "mx_common.hpp"
#include "mx_kernels.hpp"

// Every product and sum in this file is rounded on its own, as the host's
// AVX2 forms are: hipcc would otherwise contract a multiply feeding an add
// (x1*c - x2*s, 1 + 2^a) into one fused multiply-add. The pragma governs the
// operators written here (the __fmul_rn family is compiled in HIP's headers,
// outside it, and would still be contracted). The explicit fmaf steps of the
// exp2 polynomial stay fused, as on the host.
#pragma clang fp contract(off)

using namespace mxd;

namespace {

// PAIRS adjacent pairs per thread (4: 8-byte loads of x1 and x2 and 16-byte
// table loads, for head_dim % 8 == 0; else 2), threads over (row, unit) flat.
template <int PAIRS>
__global__ __launch_bounds__(256) void rope_qkv_k(uint16_t *__restrict__ qkv, int64_t ld,
                                                  int64_t rows, int S, int H, int hd,
                                                  const float *__restrict__ cos_t,
                                                  const float *__restrict__ sin_t,
                                                  const int32_t *__restrict__ row_pos,
                                                  const int32_t *rows_dev) {
  const int half = hd / 2, d = H * hd;
  const int per_head = half / PAIRS;  // thread units per head
  const int units = 2 * H * per_head;
  const int64_t total = live_rows(rows, rows_dev) * units;
  for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = t / units;
    const int u = (int)(t - row * units);
    const int s = row_pos ? row_pos[row] : (int)(row % S);
    const int which = u / (H * per_head);  // 0: Q, 1: K
    const int rem = u - which * H * per_head;
    const int h = rem / per_head, j = (rem - h * per_head) * PAIRS;
    uint16_t *v = qkv + row * ld + which * d + h * hd;
    const float *cs = cos_t + (int64_t)s * hd + j, *sn = sin_t + (int64_t)s * hd + j;
    float a[PAIRS], b[PAIRS], c[PAIRS], si[PAIRS];
    if constexpr (PAIRS == 4) {
      const uint2 p1 = *(const uint2 *)(v + j), p2 = *(const uint2 *)(v + j + half);
      const float4 c4 = *(const float4 *)cs, s4 = *(const float4 *)sn;
      const uint32_t w1[2] = {p1.x, p1.y}, w2[2] = {p2.x, p2.y};
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        a[2 * k] = bf2f(w1[k] & 0xFFFFu);
        a[2 * k + 1] = bf2f(w1[k] >> 16);
        b[2 * k] = bf2f(w2[k] & 0xFFFFu);
        b[2 * k + 1] = bf2f(w2[k] >> 16);
      }
      c[0] = c4.x, c[1] = c4.y, c[2] = c4.z, c[3] = c4.w;
      si[0] = s4.x, si[1] = s4.y, si[2] = s4.z, si[3] = s4.w;
    } else {
      const uint32_t p1 = *(const uint32_t *)(v + j), p2 = *(const uint32_t *)(v + j + half);
      const float2 c2 = *(const float2 *)cs, s2 = *(const float2 *)sn;
      a[0] = bf2f(p1 & 0xFFFFu), a[1] = bf2f(p1 >> 16);
      b[0] = bf2f(p2 & 0xFFFFu), b[1] = bf2f(p2 >> 16);
      c[0] = c2.x, c[1] = c2.y;
      si[0] = s2.x, si[1] = s2.y;
    }
    uint32_t o1[PAIRS / 2], o2[PAIRS / 2];
#pragma unroll
    for (int k = 0; k < PAIRS / 2; ++k) {
      const int e = 2 * k;
      o1[k] = pack_bf2(a[e] * c[e] - b[e] * si[e], a[e + 1] * c[e + 1] - b[e + 1] * si[e + 1]);
      o2[k] = pack_bf2(b[e] * c[e] + a[e] * si[e], b[e + 1] * c[e + 1] + a[e + 1] * si[e + 1]);
    }
    if constexpr (PAIRS == 4) {
      *(uint2 *)(v + j) = make_uint2(o1[0], o1[1]);
      *(uint2 *)(v + j + half) = make_uint2(o2[0], o2[1]);
    } else {
      *(uint32_t *)(v + j) = o1[0];
      *(uint32_t *)(v + j + half) = o2[0];
    }
  }
}

__device__ __forceinline__ float4 load4(const void *p, bool bf, int64_t off) {
  if (bf) {
    const uint2 u = *(const uint2 *)((const uint16_t *)p + off);
    return make_float4(bf2f(u.x & 0xFFFFu), bf2f(u.x >> 16), bf2f(u.y & 0xFFFFu), bf2f(u.y >> 16));
  }
  return *(const float4 *)((const float *)p + off);
}

template <bool IN_BF, bool OUT_BF, int ACT>
__global__ __launch_bounds__(256) void glu_k(const void *__restrict__ in, void *__restrict__ out,
                                             int64_t rows, int64_t f, const int32_t *rows_dev) {
  const int64_t q4 = f / 4, total = live_rows(rows, rows_dev) * q4;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / q4, j = (i - r * q4) * 4;
    const float4 lo = load4(in, IN_BF, r * 2 * f + j), hi = load4(in, IN_BF, r * 2 * f + f + j);
    float4 o;
    o.x = lo.x * glu_act<ACT>(hi.x);
    o.y = lo.y * glu_act<ACT>(hi.y);
    o.z = lo.z * glu_act<ACT>(hi.z);
    o.w = lo.w * glu_act<ACT>(hi.w);
    const int64_t oo = r * f + j;
    if (OUT_BF)
      *(uint2 *)((uint16_t *)out + oo) = make_uint2(pack_bf2(o.x, o.y), pack_bf2(o.z, o.w));
    else
      *(float4 *)((float *)out + oo) = o;
  }
}

// Row n of dst = row orig(n) of src, in groups of 16: the first 8 from the lo
// half (rows 8G ..), the next 8 the matching rows of the hi half (f + 8G ..).
// One block per row, 4-byte words.
__global__ __launch_bounds__(256) void glu_interleave_k(const uint32_t *__restrict__ src,
                                                        uint32_t *__restrict__ dst, int64_t f,
                                                        int64_t words) {
  const int64_t n = blockIdx.x, G = n >> 4, r = n & 15;
  const int64_t orig = r < 8 ? 8 * G + r : f + 8 * G + (r - 8);
  for (int64_t w = threadIdx.x; w < words; w += blockDim.x)
    dst[n * words + w] = src[orig * words + w];
}

}  // namespace

namespace mxk {

hipError_t glu_interleave(const void *src, void *dst, int64_t f, int64_t row_bytes,
                          hipStream_t s) {
  if (f <= 0 || f % 8 || row_bytes <= 0 || row_bytes % 4) return hipErrorInvalidValue;
  glu_interleave_k<<<(unsigned)(2 * f), 256, 0, s>>>((const uint32_t *)src, (uint32_t *)dst, f,
                                                     row_bytes / 4);
  return hipGetLastError();
}

hipError_t rope_qkv(uint16_t *qkv, int64_t ld, int64_t rows, int S, int H, int hd,
                    const float *cos_t, const float *sin_t, hipStream_t s,
                    const int32_t *row_pos, const int32_t *rows_dev) {
  // Four pairs where their 8- and 16-byte accesses are aligned.
  const bool wide = hd % 8 == 0 && ld % 4 == 0 && (uintptr_t)qkv % 8 == 0 &&
                    (uintptr_t)cos_t % 16 == 0 && (uintptr_t)sin_t % 16 == 0;
  const int pairs = wide ? 4 : 2;
  const int64_t total = rows * (2 * H * (hd / 2 / pairs));
  int64_t g = (total + 255) / 256;
  if (g > 65536) g = 65536;
  if (pairs == 4)
    rope_qkv_k<4><<<(unsigned)g, 256, 0, s>>>(qkv, ld, rows, S, H, hd, cos_t, sin_t, row_pos,
                                              rows_dev);
  else
    rope_qkv_k<2><<<(unsigned)g, 256, 0, s>>>(qkv, ld, rows, S, H, hd, cos_t, sin_t, row_pos,
                                              rows_dev);
  return hipGetLastError();
}

hipError_t glu(const void *in, int in_bf, void *out, int out_bf, int64_t rows, int64_t f, int act,
               hipStream_t s, const int32_t *rows_dev) {
  const int64_t total = rows * (f / 4);
  int64_t g = (total + 255) / 256;
  if (g > 65536) g = 65536;
#define MX_GLU(A)                                                                          \
  if (in_bf && out_bf)                                                                     \
    glu_k<true, true, A><<<(unsigned)g, 256, 0, s>>>(in, out, rows, f, rows_dev);          \
  else if (in_bf)                                                                          \
    glu_k<true, false, A><<<(unsigned)g, 256, 0, s>>>(in, out, rows, f, rows_dev);         \
  else if (out_bf)                                                                         \
    glu_k<false, true, A><<<(unsigned)g, 256, 0, s>>>(in, out, rows, f, rows_dev);         \
  else                                                                                     \
    glu_k<false, false, A><<<(unsigned)g, 256, 0, s>>>(in, out, rows, f, rows_dev);
  if (act == 1) {
    MX_GLU(1)
  } else {
    MX_GLU(2)
  }
#undef MX_GLU
  return hipGetLastError();
}

}  // namespace mxk
