// mx_common.hpp -- device helpers shared by the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mxd {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// fp32 -> bf16 by the reference's integer formula (host_kernels.hpp:157-161):
// round to nearest even on the bit pattern, NaN behaviour included (a NaN
// whose payload carries into the exponent becomes Inf or 0, as on the host).
__device__ __forceinline__ uint16_t f2bf(float x) {
  const uint32_t u = __float_as_uint(x);
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

__device__ __forceinline__ float bf2f(uint32_t h) { return __uint_as_float(h << 16); }

// int32 -> bf16 in one nearest-even rounding of the integer itself (the
// array's narrow_i32_bf16 kernel): keep the top 8 significant bits of |v|,
// round on the dropped bits.
__device__ __forceinline__ uint16_t i32_to_bf16(int32_t v) {
  if (v == 0) return 0;
  const uint32_t sign = v < 0 ? 0x8000u : 0u;
  const uint32_t a = v < 0 ? (uint32_t)(-(int64_t)v) : (uint32_t)v;
  int e = 31 - __clz(a);
  uint32_t mant;
  if (e <= 7) {
    mant = a << (7 - e);
  } else {
    const int sh = e - 7;
    mant = a >> sh;
    const uint32_t rem = a & ((1u << sh) - 1u);
    const uint32_t half = 1u << (sh - 1);
    if (rem > half || (rem == half && (mant & 1u))) ++mant;
    if (mant == 256u) {
      mant = 128u;
      ++e;
    }
  }
  return (uint16_t)(sign | ((uint32_t)(e + 127) << 7) | (mant & 0x7Fu));
}

// Two fp32 -> packed bf16 by the hardware conversion (v_cvt_pk_bf16_f32, round
// to nearest even): identical to f2bf for every non-NaN input; a NaN becomes a
// quiet NaN instead of f2bf's carry pattern. For results held to a tolerance
// (GEMM outputs), not for the bit-exact narrowing kernels.
__device__ __forceinline__ uint32_t pack_bf2_hw(float a, float b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  bf16x2_t v;
  v[0] = (__bf16)a;
  v[1] = (__bf16)b;
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ uint32_t pack_bf2(float a, float b) {
  return (uint32_t)f2bf(a) | ((uint32_t)f2bf(b) << 16);
}

// 16-byte streaming accesses: global loads and stores with the nontemporal
// hint, for data a kernel touches once and that no cache holds from an earlier
// kernel (the bf16 softmax rows, the narrowings, GELU over fp32 input, the
// residual LayerNorm's inputs and fp32 output). Where each is used, its kernel
// states what it measured against cached accesses.
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld_stream16(const void *p) {
  const u32x4_t v = __builtin_nontemporal_load((const u32x4_t *)p);
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void st_stream16(void *p, uint4 w) {
  const u32x4_t v = {w.x, w.y, w.z, w.w};
  __builtin_nontemporal_store(v, (u32x4_t *)p);
}
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint2 ld_stream8(const void *p) {
  const u32x2_t v = __builtin_nontemporal_load((const u32x2_t *)p);
  return make_uint2(v.x, v.y);
}

// The rows a launch runs over: `rows` (the launch's bound, what its buffers
// hold), or fewer when rows_dev is given -- a count an earlier kernel on the
// stream wrote on the device (token packing's packed row total), read here so
// that the host never waits for it. Clamped to [0, rows].
__device__ __forceinline__ int64_t live_rows(int64_t rows, const int32_t *rows_dev) {
  if (!rows_dev) return rows;
  const int64_t r = *rows_dev;
  return r < 0 ? 0 : (r < rows ? r : rows);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

// gelu8 with the lane semantics of the reference's AVX2 branch
// (bert_encoder.cpp:547-570): u = min(|v|, 4), degree-8 Horner by FMA, plus
// max(v, 0); a NaN input gives the polynomial at 4 (min_ps/max_ps return the
// second operand on NaN).
__device__ __forceinline__ float gelu_poly(float v) {
  const float av = fabsf(v);
  const float u = av < 4.0f ? av : 4.0f;
  float p = __builtin_fmaf(-7.2340282171e-05f, u, 1.8179518005e-03f);
  p = __builtin_fmaf(p, u, -1.7707383379e-02f);
  p = __builtin_fmaf(p, u, 8.4577147641e-02f);
  p = __builtin_fmaf(p, u, -1.9228671834e-01f);
  p = __builtin_fmaf(p, u, 9.8431124458e-02f);
  p = __builtin_fmaf(p, u, 3.6137852062e-01f);
  p = __builtin_fmaf(p, u, -4.9454128936e-01f);
  p = __builtin_fmaf(p, u, -1.3007010117e-04f);
  return (v > 0.0f ? v : 0.0f) + p;
}

// Exact-erf GELU, in fp32 (the host form rounds a double result once).
__device__ __forceinline__ float gelu_erf(float v) {
  return 0.5f * v * (1.0f + erff(v * 0.70710678118654752440f));
}

// Exact-erf GELU for the GEMM epilogues, where it runs while the matrix pipe
// idles: erfc(z), z = |x|/sqrt2, by Abramowitz & Stegun 7.1.26 (|error| <=
// 1.5e-7, the method of the reference's accelerator kernel, gelu_erf.cc:60-65)
// with the hardware reciprocal and exp2, about half the instructions of erff.
// Formed from erfc, GELU(x) = x - x erfc(z) / 2 for x >= 0 and x erfc(z) / 2
// below, so the negative side keeps its relative accuracy instead of
// cancelling in 1 + erf. +inf gives +inf; -inf and NaN give NaN, as the host's
// 0.5 x (1 + erf(x / sqrt2)) does.
__device__ __forceinline__ float gelu_erf_epi(float v) {
  const float z = fabsf(v) * 0.70710678118654752440f;
  const float t = __builtin_amdgcn_rcpf(__builtin_fmaf(0.3275911f, z, 1.0f));
  float p = __builtin_fmaf(1.061405429f, t, -1.453152027f);
  p = __builtin_fmaf(p, t, 1.421413741f);
  p = __builtin_fmaf(p, t, -0.284496736f);
  p = __builtin_fmaf(p, t, 0.254829592f);
  const float erfc = p * t * __builtin_amdgcn_exp2f(-(z * z) * 1.4426950408889634f);
  const float h = 0.5f * v * erfc;
  return v >= 0.0f ? (erfc == 0.0f ? v : v - h) : h;
}

// The GEMM epilogue activation (mx_epilogue): 0 none, 1 gelu_poly, 2 GELU erf.
__device__ __forceinline__ float gemm_epilogue(float v, int epi) {
  if (epi == 1) return gelu_poly(v);
  if (epi == 2) return gelu_erf_epi(v);
  return v;
}

// exp2_avx2 (host_kernels.hpp:358-379): k = trunc(x), f = x - k, degree-7
// Horner by FMA, times 2^k written into the exponent field. Bit-identical to
// the host lane for x in [-126, 127].
__device__ __forceinline__ float exp2_poly(float x) {
  const int k = (int)x;
  const float f = x - (float)k;
  float p = __builtin_fmaf(1.5483275463e-05f, f, 1.5669833174e-04f);
  p = __builtin_fmaf(p, f, 1.3331825236e-03f);
  p = __builtin_fmaf(p, f, 9.6164605538e-03f);
  p = __builtin_fmaf(p, f, 5.5504156855e-02f);
  p = __builtin_fmaf(p, f, 2.4022684109e-01f);
  p = __builtin_fmaf(p, f, 6.9314717694e-01f);
  p = __builtin_fmaf(p, f, 9.9999998955e-01f);
  return p * __uint_as_float((uint32_t)(k + 127) << 23);
}

// exp2_poly for x in [-120, 0], where the softmaxes clamp their argument: the
// same polynomial, scaled by v_ldexp_f32 (one instruction) instead of a
// multiply by 2^k built in the exponent field (three). p * 2^k is exact and
// normal there (p in (0.5, 1], k >= -120), so both give the same bits; every
// float in [-120, 0] was checked (tests/test_exp2_scaling_cpu.py).
__device__ __forceinline__ float exp2_poly_neg(float x) {
  const int k = (int)x;
  const float f = x - (float)k;
  float p = __builtin_fmaf(1.5483275463e-05f, f, 1.5669833174e-04f);
  p = __builtin_fmaf(p, f, 1.3331825236e-03f);
  p = __builtin_fmaf(p, f, 9.6164605538e-03f);
  p = __builtin_fmaf(p, f, 5.5504156855e-02f);
  p = __builtin_fmaf(p, f, 2.4022684109e-01f);
  p = __builtin_fmaf(p, f, 6.9314717694e-01f);
  p = __builtin_fmaf(p, f, 9.9999998955e-01f);
  return __builtin_amdgcn_ldexpf(p, k);
}

// swiglu_cpu's SiLU (bert_encoder.cpp:582-627): x / (1 + 2^max(-x log2e,
// -120)) with the exp2 polynomial above, each operation rounded on its own as
// the host's AVX2 form is (no multiply-add contraction of the polynomial's
// last product into the 1 + ...).
__device__ __forceinline__ float silu_host(float x) {
#pragma clang fp contract(off)
  float a = -x * 1.4426950408889634f;
  a = a < -120.0f ? -120.0f : a;
  return x / (1.0f + exp2_poly(a));
}

// The gated FFN's activation of the gate half: 1 SiLU, 2 exact-erf GELU.
// Contraction is off here too, so the GELU form rounds alike wherever it is
// inlined (the gated-FFN pass and the GEMM epilogue that fuses it).
template <int ACT>
__device__ __forceinline__ float glu_act(float hi) {
#pragma clang fp contract(off)
  if (ACT == 1) return silu_host(hi);
  return 0.5f * hi * (1.0f + erff(hi * 0.70710678118654752440f));
}

// A rounded product, sum and difference that the compiler may not fuse into a
// multiply-add. (HIP's __fmul_rn / __fadd_rn are plain x * y and x + y in its
// headers, compiled under the default contraction, so a product feeding a sum
// through them still becomes one FMA.) Contraction is off inside each; a
// product without the contract flag is never fused.
__device__ __forceinline__ float mul_rn(float a, float b) {
#pragma clang fp contract(off)
  return a * b;
}
__device__ __forceinline__ float add_rn(float a, float b) {
#pragma clang fp contract(off)
  return a + b;
}
__device__ __forceinline__ float sub_rn(float a, float b) {
#pragma clang fp contract(off)
  return a - b;
}

// The AIE exp2_poly (kernels/exp2_poly.h:35-65): the same table, each Horner
// step a rounded multiply then a rounded add (no FMA).
__device__ __forceinline__ float exp2_poly_aie(float x) {
  const int k = (int)x;
  const float f = sub_rn(x, (float)k);
  float p = 1.5483275463e-05f;
  p = add_rn(mul_rn(p, f), 1.5669833174e-04f);
  p = add_rn(mul_rn(p, f), 1.3331825236e-03f);
  p = add_rn(mul_rn(p, f), 9.6164605538e-03f);
  p = add_rn(mul_rn(p, f), 5.5504156855e-02f);
  p = add_rn(mul_rn(p, f), 2.4022684109e-01f);
  p = add_rn(mul_rn(p, f), 6.9314717694e-01f);
  p = add_rn(mul_rn(p, f), 9.9999998955e-01f);
  return mul_rn(p, __uint_as_float((uint32_t)(k + 127) << 23));
}

// exp2_poly_aie for x in [-120, 0] (the accelerator softmax's clamp), scaled
// by v_ldexp_f32: the same bits there, for the reason exp2_poly_neg gives;
// every float in [-120, 0] was checked (tests/test_exp2_scaling_cpu.py).
__device__ __forceinline__ float exp2_poly_aie_neg(float x) {
  const int k = (int)x;
  const float f = sub_rn(x, (float)k);
  float p = 1.5483275463e-05f;
  p = add_rn(mul_rn(p, f), 1.5669833174e-04f);
  p = add_rn(mul_rn(p, f), 1.3331825236e-03f);
  p = add_rn(mul_rn(p, f), 9.6164605538e-03f);
  p = add_rn(mul_rn(p, f), 5.5504156855e-02f);
  p = add_rn(mul_rn(p, f), 2.4022684109e-01f);
  p = add_rn(mul_rn(p, f), 6.9314717694e-01f);
  p = add_rn(mul_rn(p, f), 9.9999998955e-01f);
  return __builtin_amdgcn_ldexpf(p, k);
}

}  // namespace mxd
