// ref_shim.cpp -- C entry points over the reference's OWN host kernels, so the
// oracle's restatement can be checked against them. TEST INFRASTRUCTURE.
//
// Compiled by oracle/Makefile (target `ref`) directly against the headers in
// the reference checkout (runtime/include/common/host_kernels.hpp,
// runtime/include/common/conv_host.hpp) and runtime/src/pool.cpp; nothing of
// the reference is copied here. The output lives in oracle/_ref/ only.
#include "common/conv_host.hpp"
#include "common/host_kernels.hpp"
#include "runtime/pool.hpp"

#include <cstdint>
#include <memory>

extern "C" {

uint16_t ref_to_bf16(float x) { return app::to_bf16(x); }
float ref_from_bf16(uint16_t h) { return app::from_bf16(h); }

// bf16_fill over all 2^32 bit patterns in [lo, hi) (as uint32), written to
// out[i - lo]; the AVX2 form the reference ships.
void ref_bf16_fill_bits(uint32_t lo, uint64_t count, uint16_t *out) {
  const size_t chunk = 1 << 20;
  std::unique_ptr<float[]> buf(new float[chunk]);
  for (uint64_t done = 0; done < count; done += chunk) {
    const size_t n = static_cast<size_t>(count - done < chunk ? count - done : chunk);
    for (size_t i = 0; i < n; ++i) {
      const uint32_t u = lo + static_cast<uint32_t>(done + i);
      std::memcpy(&buf[i], &u, 4);
    }
    app::bf16_fill(out + done, buf.get(), n);
  }
}

void ref_bf16_fill(uint16_t *dst, const float *src, size_t n) { app::bf16_fill(dst, src, n); }

float ref_gelu8_scalar(float x) { return app::gelu8(x); }

void ref_gelu8_avx2(const float *x, float *y, size_t n) {
  size_t i = 0;
  for (; i + 8 <= n; i += 8)
    _mm256_storeu_ps(y + i, app::gelu8(_mm256_loadu_ps(x + i)));
  for (; i < n; ++i) y[i] = app::gelu8(x[i]);
}

void ref_exp2_avx2(const float *x, float *y, size_t n) {
  size_t i = 0;
  for (; i + 8 <= n; i += 8)
    _mm256_storeu_ps(y + i, app::exp2_avx2(_mm256_loadu_ps(x + i)));
  for (; i < n; ++i) {
    float tmp[8] = {x[i], 0, 0, 0, 0, 0, 0, 0}, out[8];
    _mm256_storeu_ps(out, app::exp2_avx2(_mm256_loadu_ps(tmp)));
    y[i] = out[0];
  }
}

float ref_hsum8(const float *v) { return app::hsum256(_mm256_loadu_ps(v)); }

void ref_gemm_nt(const float *A, int64_t M, const float *B, int64_t K, int64_t N,
                 const float *bias, float *C, int threads) {
  app::Pool pool(threads > 0 ? threads : 1);
  npue::hostconv::gemm_nt(A, M, B, K, N, bias, C, pool);
}

}  // extern "C"
