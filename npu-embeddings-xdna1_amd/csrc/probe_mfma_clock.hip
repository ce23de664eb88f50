// probe_mfma_clock.hip -- a measurement program, not part of the library: the
// shader clock and the MFMA / LDS throughput a full-chip workload sustains on
// MI355X, for the GEMM's design. Built by build.py into
// _build/probe_mfma_clock; run it on the GPU and it prints one line per case.
//
// Every case runs one 8-wave block per CU for a few milliseconds; each wave
// brackets its loop with s_memtime (shader clock) and s_memrealtime (the
// 100 MHz constant counter), so clock = d(memtime) / d(memrealtime) * 100 MHz.
// Cases:
//   mfma low-entropy   v_mfma_f32_32x32x16_bf16 on register operands holding
//                      a few distinct small values, 8 independent accumulators
//   mfma random        the same on operands of random bf16 bit patterns
//   mfma+lds           the same MFMAs with 6 ds_read_b128 per 8 MFMAs (the
//                      encoder GEMM's 64 x 128 wave tile reads 6 fragments per
//                      8 MFMAs), random data in LDS
//   mfma+lds+dma       plus 2 KB of global->LDS direct loads per 8 MFMAs per
//                      wave (the GEMM's slab loads: 1 byte written per 3 read)
//                      from a 1 MB source that stays in L2
//   lds only           ds_read_b128 alone: the LDS read bandwidth per CU
// Then the library's own bf16 GEMM (through the C ABI, mx_gemm_wt) at the
// packed bge-base QKV shape (M 17455, N 2304, K 768, bias, bf16 C) on three
// operand distributions: constant, the encoder's (A ~ N(0, 1) as a LayerNorm
// output, W ~ N(0, 0.02)), and random bf16 bit patterns.
// All indexes stay inside their buffers: LDS offsets are masked to 64 KB
// (reads) and 32 KB (direct-load targets, a separate region), the global
// source window to its allocation.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <vector>

#include "mx_encoder.h"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr int LDS_READ = 65536, LDS_DMA = 32768;
constexpr size_t SRC_BYTES = (size_t)1 << 20;  // direct-load source: L2-resident, as the
                                                // GEMM's reused operand slabs mostly are

__device__ __forceinline__ unsigned mix(unsigned x) {
  x ^= x >> 16;
  x *= 0x7feb352dU;
  x ^= x >> 15;
  x *= 0x846ca68bU;
  x ^= x >> 16;
  return x;
}

// MODE: 0 mfma low-entropy, 1 mfma random, 2 mfma+lds, 3 mfma+lds+dma, 4 lds
template <int MODE>
__global__ __launch_bounds__(512) void probe_k(const uint8_t *src, float *out, long long *clk,
                                               int iters) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const unsigned seed = blockIdx.x * 512u + threadIdx.x;
  for (int i = threadIdx.x; i < LDS_READ / 4; i += 512) {
    // random bf16 pairs with exponents near 1.0, so the products stay finite
    const unsigned r = mix(seed * 131u + (unsigned)i);
    ((unsigned *)smem)[i] = (r & 0x807F807FU) | 0x3F003F00U;
  }
  __syncthreads();
  bf16x8 fa[6];
#pragma unroll
  for (int k = 0; k < 6; ++k) {
    if (MODE == 0) {
      u32x4 v = {0x3C003C00U + (unsigned)(k & 3), 0x3C003C00U, 0x3C003C00U, 0x3C003C00U};
      fa[k] = __builtin_bit_cast(bf16x8, v);
    } else {
      fa[k] = *(const bf16x8 *)(smem + ((lane * 16 + k * 1024) & (LDS_READ - 1)));
    }
  }
  f32x16 acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[j][r] = 0.0f;
  const uint32_t lds0 = (uint32_t)(uintptr_t)smem;
  const long long t0 = __builtin_amdgcn_s_memtime();
  const long long r0 = __builtin_amdgcn_s_memrealtime();
  int base = (wave * 4096 + lane * 16) & (LDS_READ - 1);
  size_t gofs = ((size_t)blockIdx.x * 8 + wave) * 2048;
  for (int it = 0; it < iters; ++it) {
    if (MODE == 3) {
      // two 1 KB direct loads per wave into the separate 32 KB region
#pragma unroll
      for (int d = 0; d < 2; ++d) {
        const uint8_t *g = src + ((gofs + (size_t)d * 1024) % SRC_BYTES) + lane * 16;
        const uint32_t dst = lds0 + LDS_READ + (uint32_t)(((wave * 2 + d) * 1024) & (LDS_DMA - 1));
        asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(dst), "v"(g)
                     : "memory");
      }
      gofs += 8 * 2048;
    }
    if (MODE != 4) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[j & 3], fa[4 + (j >> 2)], acc[j], 0,
                                                         0, 0);
        if (MODE >= 2 && j < 6)
          fa[j] = *(const bf16x8 *)(smem + ((base + j * 1024) & (LDS_READ - 1)));
      }
    } else {
#pragma unroll
      for (int j = 0; j < 6; ++j)
        fa[j] = *(const bf16x8 *)(smem + ((base + j * 1024) & (LDS_READ - 1)));
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      acc[0][0] += (float)fa[0][0];
    }
    if (MODE == 3) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    base = (base + 6144) & (LDS_READ - 1);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  const long long t1 = __builtin_amdgcn_s_memtime();
  const long long r1 = __builtin_amdgcn_s_memrealtime();
  float t = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) t += acc[j][r];
#pragma unroll
  for (int k = 0; k < 6; ++k) t += (float)fa[k][1];
  out[blockIdx.x * 512 + threadIdx.x] = t;
  if (lane == 0) {
    clk[(blockIdx.x * 8 + wave) * 2] = t1 - t0;
    clk[(blockIdx.x * 8 + wave) * 2 + 1] = r1 - r0;
  }
}

template <int MODE>
int run(const char *name, int iters, int blocks, const uint8_t *src, float *d_out,
        long long *d_clk) {
  const int lds = LDS_READ + (MODE == 3 ? LDS_DMA : 0);
  if (hipFuncSetAttribute((const void *)probe_k<MODE>, hipFuncAttributeMaxDynamicSharedMemorySize,
                          lds) != hipSuccess)
    return 1;
  hipEvent_t a, b;
  if (hipEventCreate(&a) != hipSuccess || hipEventCreate(&b) != hipSuccess) return 1;
  probe_k<MODE><<<blocks, 512, lds>>>(src, d_out, d_clk, iters / 10);  // warm-up
  if (hipEventRecord(a) != hipSuccess) return 1;
  probe_k<MODE><<<blocks, 512, lds>>>(src, d_out, d_clk, iters);
  if (hipEventRecord(b) != hipSuccess || hipEventSynchronize(b) != hipSuccess) return 1;
  float ms = 0.0f;
  if (hipEventElapsedTime(&ms, a, b) != hipSuccess) return 1;
  std::vector<long long> h((size_t)blocks * 16);
  if (hipMemcpy(h.data(), d_clk, h.size() * 8, hipMemcpyDeviceToHost) != hipSuccess) return 1;
  double tc = 0.0, tr = 0.0;
  for (int i = 0; i < blocks * 8; ++i) {
    tc += (double)h[2 * i];
    tr += (double)h[2 * i + 1];
  }
  const double ghz = tc / tr * 0.1;
  const double cycles = ms * 1e-3 * ghz * 1e9;
  const double mfma = MODE == 4 ? 0.0 : (double)blocks * 8 * iters * 8;
  const double tflops = mfma * 32768.0 / (ms * 1e-3) / 1e12;
  const double lds_rd = MODE < 2 ? 0.0 : (double)blocks * 8 * iters * 6 * 1024;
  const double lds_wr = MODE == 3 ? (double)blocks * 8 * iters * 2 * 1024 : 0.0;
  printf("%-18s %7.3f ms  clock %.3f GHz  %7.1f TFLOP/s  MFMA issue %5.1f%% of 1 per 32 clk  "
         "LDS read %5.1f B/clk/CU  LDS write %4.1f B/clk/CU\n",
         name, ms, ghz, tflops, MODE == 4 ? 0.0 : 100.0 * mfma / blocks / 4 / (cycles / 32.0),
         lds_rd / blocks / cycles, lds_wr / blocks / cycles);
  return hipEventDestroy(a) != hipSuccess || hipEventDestroy(b) != hipSuccess;
}

uint16_t to_bf16(float x) {
  uint32_t u;
  std::memcpy(&u, &x, 4);
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

// The library's GEMM at the packed QKV shape on one operand distribution:
// microseconds per launch over 20 launches (events on the library's stream).
int gemm_case(mx_ctx *ctx, mx_stream *st, const char *name, int dist) {
  const int64_t M = 17455, N = 2304, K = 768;
  std::vector<uint16_t> a((size_t)M * K), w((size_t)N * K);
  std::vector<float> bias((size_t)N, 0.01f);
  uint64_t x = 88172645463325252ULL;
  auto next = [&]() {
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    return x;
  };
  auto normal = [&]() {  // Box-Muller
    const double u1 = ((next() >> 11) + 1.0) / 9007199254740993.0;
    const double u2 = (next() >> 11) / 9007199254740992.0;
    return (float)(std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2));
  };
  for (auto &v : a)
    v = dist == 0 ? to_bf16(0.5f)
                  : dist == 1 ? to_bf16(normal())
                              : (uint16_t)((next() & 0x807F) | 0x3F00);
  for (auto &v : w)
    v = dist == 0 ? to_bf16(0.01f)
                  : dist == 1 ? to_bf16(0.02f * normal())
                              : (uint16_t)((next() & 0x807F) | 0x3C00);
  void *da = nullptr, *dw = nullptr, *db = nullptr, *dc = nullptr;
  if (mx_alloc(ctx, a.size() * 2, &da) || mx_alloc(ctx, w.size() * 2, &dw) ||
      mx_alloc(ctx, bias.size() * 4, &db) || mx_alloc(ctx, (size_t)M * N * 2, &dc) ||
      mx_copy_h2d(st, da, a.data(), a.size() * 2) || mx_copy_h2d(st, dw, w.data(), w.size() * 2) ||
      mx_copy_h2d(st, db, bias.data(), bias.size() * 4) || mx_sync(st)) {
    printf("gemm %s: %s\n", name, mx_last_error());
    return 1;
  }
  hipStream_t hs = (hipStream_t)mx_stream_handle(st);
  hipEvent_t e0, e1;
  if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) return 1;
  int rc = 0;
  for (int r = 0; r < 25 && !rc; ++r) {
    if (r == 5 && hipEventRecord(e0, hs) != hipSuccess) rc = 1;
    rc |= mx_gemm_wt(st, (const uint16_t *)da, M, K, K, (const uint16_t *)dw, N,
                     (const float *)db, MX_EPI_NONE, nullptr, dc, MX_BF16, N);
  }
  float ms = 0.0f;
  if (rc || hipEventRecord(e1, hs) != hipSuccess || hipEventSynchronize(e1) != hipSuccess ||
      hipEventElapsedTime(&ms, e0, e1) != hipSuccess) {
    printf("gemm %s: %s\n", name, rc ? mx_last_error() : "event failure");
    return 1;
  }
  const double us = ms * 1e3 / 20.0;
  printf("gemm QKV %-14s %7.1f us/launch  %7.1f TFLOP/s  (%s)\n", name, us,
         2.0 * M * N * K / (us * 1e-6) / 1e12, mx_gemm_plan_for(M, N, K, MX_BF16, 0, 0));
  rc |= mx_free(ctx, da) | mx_free(ctx, dw) | mx_free(ctx, db) | mx_free(ctx, dc);
  rc |= hipEventDestroy(e0) != hipSuccess || hipEventDestroy(e1) != hipSuccess;
  return rc;
}

}  // namespace

int main() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return 1;
  const int blocks = cus;
  uint8_t *src = nullptr;
  float *d_out = nullptr;
  long long *d_clk = nullptr;
  if (hipMalloc(&src, SRC_BYTES) != hipSuccess ||
      hipMalloc(&d_out, (size_t)blocks * 512 * 4) != hipSuccess ||
      hipMalloc(&d_clk, (size_t)blocks * 16 * 8) != hipSuccess)
    return 1;
  {
    std::vector<unsigned> h(SRC_BYTES / 4);
    unsigned x = 2463534242U;
    for (auto &v : h) {
      x ^= x << 13;
      x ^= x >> 17;
      x ^= x << 5;
      v = (x & 0x807F807FU) | 0x3F003F00U;
    }
    if (hipMemcpy(src, h.data(), SRC_BYTES, hipMemcpyHostToDevice) != hipSuccess) return 1;
  }
  printf("%d CUs, one 8-wave block per CU\n", blocks);
  int rc = 0;
  rc |= run<0>("mfma low-entropy", 20000, blocks, src, d_out, d_clk);
  rc |= run<1>("mfma random", 20000, blocks, src, d_out, d_clk);
  rc |= run<2>("mfma+lds", 20000, blocks, src, d_out, d_clk);
  rc |= run<3>("mfma+lds+dma", 20000, blocks, src, d_out, d_clk);
  rc |= run<4>("lds only", 20000, blocks, src, d_out, d_clk);
  rc |= run<0>("mfma low-entropy", 20000, blocks, src, d_out, d_clk);
  mx_ctx *ctx = nullptr;
  mx_stream *st = nullptr;
  if (mx_create(dev, &ctx) || mx_stream_create(ctx, &st)) {
    printf("mx_create: %s\n", mx_last_error());
    return 1;
  }
  rc |= gemm_case(ctx, st, "constant", 0);
  rc |= gemm_case(ctx, st, "encoder-like", 1);
  rc |= gemm_case(ctx, st, "random bits", 2);
  mx_stream_destroy(st);
  mx_destroy(ctx);
  if (hipFree(src) != hipSuccess || hipFree(d_out) != hipSuccess || hipFree(d_clk) != hipSuccess)
    rc = 1;
  return rc;
}
