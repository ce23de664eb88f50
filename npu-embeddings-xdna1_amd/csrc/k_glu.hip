// k_glu.hip -- the two ops of the RoPE / gated-FFN BERT archs (nomic_bert_rope_swiglu,
// gte_new_rope_geglu) on gfx950, both memory-bound passes:
//
// rope_qkv_k: BertEncoder::apply_rope_qkv (bert_encoder.cpp:951-990) on the
// bf16 fused Q|K|V rows, in place, Q and K only. Position s = row % S (or the
// packed row's recorded position); per
// head the pairs (j, j + hd/2) rotate by the table's angle:
//   o1 = x1*c - x2*s,  o2 = x2*c + x1*s
// each product rounded as the host's AVX2 form (no fused multiply-add), the
// result narrowed once to bf16. One block per row; each thread moves two
// adjacent pairs (4-byte bf16 loads of x1 and x2, 8-byte table loads).
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

__global__ __launch_bounds__(256) void rope_qkv_k(uint16_t *__restrict__ qkv, int64_t ld,
                                                  int S, int H, int hd,
                                                  const float *__restrict__ cos_t,
                                                  const float *__restrict__ sin_t,
                                                  const int32_t *__restrict__ row_pos) {
  const int64_t row = blockIdx.x;
  const int s = row_pos ? row_pos[row] : (int)(row % S), half = hd / 2, d = H * hd;
  const int per_head = half / 2;  // thread units (two pairs) per head
  const int units = 2 * H * per_head;
  uint16_t *base = qkv + row * ld;
  const float *cs = cos_t + (int64_t)s * hd, *sn = sin_t + (int64_t)s * hd;
  for (int u = threadIdx.x; u < units; u += blockDim.x) {
    const int which = u / (H * per_head);  // 0: Q, 1: K
    const int rem = u - which * H * per_head;
    const int h = rem / per_head, j = (rem - h * per_head) * 2;
    uint16_t *v = base + which * d + h * hd;
    const uint32_t p1 = *(const uint32_t *)(v + j), p2 = *(const uint32_t *)(v + j + half);
    const float2 c = *(const float2 *)(cs + j), si = *(const float2 *)(sn + j);
    const float a0 = bf2f(p1 & 0xFFFFu), a1 = bf2f(p1 >> 16);
    const float b0 = bf2f(p2 & 0xFFFFu), b1 = bf2f(p2 >> 16);
    const float o10 = a0 * c.x - b0 * si.x;
    const float o11 = a1 * c.y - b1 * si.y;
    const float o20 = b0 * c.x + a0 * si.x;
    const float o21 = b1 * c.y + a1 * si.y;
    *(uint32_t *)(v + j) = pack_bf2(o10, o11);
    *(uint32_t *)(v + j + half) = pack_bf2(o20, o21);
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
                                             int64_t rows, int64_t f) {
  const int64_t q4 = f / 4, total = rows * q4;
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
                    const int32_t *row_pos) {
  rope_qkv_k<<<(unsigned)rows, 256, 0, s>>>(qkv, ld, S, H, hd, cos_t, sin_t, row_pos);
  return hipGetLastError();
}

hipError_t glu(const void *in, int in_bf, void *out, int out_bf, int64_t rows, int64_t f, int act,
               hipStream_t s) {
  const int64_t total = rows * (f / 4);
  int64_t g = (total + 255) / 256;
  if (g > 65536) g = 65536;
#define MX_GLU(A)                                                                          \
  if (in_bf && out_bf) glu_k<true, true, A><<<(unsigned)g, 256, 0, s>>>(in, out, rows, f); \
  else if (in_bf) glu_k<true, false, A><<<(unsigned)g, 256, 0, s>>>(in, out, rows, f);     \
  else if (out_bf) glu_k<false, true, A><<<(unsigned)g, 256, 0, s>>>(in, out, rows, f);    \
  else glu_k<false, false, A><<<(unsigned)g, 256, 0, s>>>(in, out, rows, f);
  if (act == 1) {
    MX_GLU(1)
  } else {
    MX_GLU(2)
  }
#undef MX_GLU
  return hipGetLastError();
}

}  // namespace mxk
