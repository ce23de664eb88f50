// ref_shim.cpp -- C entry points over the reference's OWN host kernels, so the
// oracle's restatement can be checked against them. TEST INFRASTRUCTURE.
//
// Compiled by oracle/Makefile (target `ref`) directly against the headers in
// the reference checkout (runtime/include/common/host_kernels.hpp,
// runtime/include/common/conv_host.hpp, runtime/include/common/host_b.hpp)
// and runtime/src/pool.cpp, runtime/src/model.cpp (the .npue reader) and
// runtime/src/encoders/gemma_kernels.cpp (the RoPE tables);
// nothing of the reference is copied here. The output lives in oracle/_ref/
// only.
#include "encoders/gemma_kernels.hpp"
#include "common/conv_host.hpp"
#include "common/host_b.hpp"
#include "common/host_kernels.hpp"
#include "runtime/model.hpp"
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

// ---- int8: quantise_a_int8 and dequantise_c (host_kernels.hpp:263-320,
// 529-600), rows serially --------------------------------------------------
static auto serial_rows = [](int64_t n, auto f) { f(0, n); };

void ref_quantise_a_int8(const float *a, int64_t rows, int64_t K, const float *ias, int8_t *q,
                         float *a_scale) {
  app::quantise_a_int8(a, rows, K, ias, q, a_scale, serial_rows);
}

// C must be 32-byte aligned with 32-byte rows (the reference's streaming
// loads require it and refuse otherwise): 0, or -1 when refused.
int ref_dequantise_c(const int32_t *c, int64_t rows, int64_t N, const float *a_scale,
                     const float *wscale, const float *bias, float *out) {
  try {
    app::dequantise_c(c, 4, rows, N, a_scale, wscale, bias, out, serial_rows);
    return 0;
  } catch (const std::exception &) {
    return -1;
  }
}

// The same for the 2-byte C of a design that narrows C on the core (c_bytes =
// 2, bf16 bits): 0, or -1 when refused.
int ref_dequantise_c_bf16(const uint16_t *c, int64_t rows, int64_t N, const float *a_scale,
                          const float *wscale, const float *bias, float *out) {
  try {
    app::dequantise_c(c, 2, rows, N, a_scale, wscale, bias, out, serial_rows);
    return 0;
  } catch (const std::exception &) {
    return -1;
  }
}

// ---- the .npue reader and B-panel untile (model.cpp, host_b.hpp) ----------
// Each returns a negative value when the reference throws; *err (when given)
// receives the exception text.
static void put_err(const std::exception &e, char *err, size_t len) {
  if (err && len) {
    std::strncpy(err, e.what(), len - 1);
    err[len - 1] = 0;
  }
}

// hostb::host_b_kn(File(path), name): fp32 [K, N] into out (cap floats).
long long ref_npue_host_b_kn(const char *path, const char *name, float *out, long long cap,
                             char *err, size_t len) {
  try {
    npue::File f(path);
    const std::vector<float> v = npue::hostb::host_b_kn(f, name);
    if (static_cast<long long>(v.size()) > cap) return -2;
    std::memcpy(out, v.data(), v.size() * sizeof(float));
    return static_cast<long long>(v.size());
  } catch (const std::exception &e) {
    put_err(e, err, len);
    return -1;
  }
}

// npue::gemm_b_panel(File(path), name, a_elem_bytes): the bytes Design::stage
// receives (an I4 payload widened to int8, int4_panel.hpp) into out (cap
// bytes); their count, or -1 when the reference refuses.
long long ref_npue_gemm_b_panel(const char *path, const char *name, long long a_elem_bytes,
                                void *out, long long cap, char *err, size_t len) {
  try {
    npue::File f(path);
    const npue::Panel p = npue::gemm_b_panel(f, name, static_cast<size_t>(a_elem_bytes));
    if (static_cast<long long>(p.bytes.bytes) > cap) return -2;
    std::memcpy(out, p.bytes.data, p.bytes.bytes);
    return static_cast<long long>(p.bytes.bytes);
  } catch (const std::exception &e) {
    put_err(e, err, len);
    return -1;
  }
}

// File::config_string(key) into buf; its length, or -1.
long long ref_npue_config(const char *path, const char *key, char *buf, size_t buflen,
                          char *err, size_t len) {
  try {
    npue::File f(path);
    const std::string v = f.config_string(key);
    if (buf && buflen) {
      const size_t n = v.size() < buflen - 1 ? v.size() : buflen - 1;
      std::memcpy(buf, v.data(), n);
      buf[n] = 0;
    }
    return static_cast<long long>(v.size());
  } catch (const std::exception &e) {
    put_err(e, err, len);
    return -1;
  }
}

// File(path) opens: 0, or -1 with the refusal in err.
int ref_npue_open(const char *path, char *err, size_t len) {
  try {
    npue::File f(path);
    return 0;
  } catch (const std::exception &e) {
    put_err(e, err, len);
    return -1;
  }
}

// File::info + File::raw: dtype, padded shape, layout numbers and the bytes.
int ref_npue_tensor(const char *path, const char *name, char *dtype, int64_t *padded,
                    int *ndim, int64_t *layout4, unsigned char *bytes, size_t cap,
                    unsigned long long *nbytes) {
  try {
    npue::File f(path);
    const npue::TensorInfo &t = f.info(name);
    std::strncpy(dtype, t.dtype.c_str(), 7);
    dtype[7] = 0;
    *ndim = static_cast<int>(t.padded_shape.size());
    for (size_t i = 0; i < t.padded_shape.size() && i < 4; ++i) padded[i] = t.padded_shape[i];
    layout4[0] = t.tile_k;
    layout4[1] = t.tile_n;
    layout4[2] = t.mac_s;
    layout4[3] = t.mac_t;
    const npue::Span s = f.raw(name);
    *nbytes = s.bytes;
    if (bytes && s.bytes <= cap) std::memcpy(bytes, s.data, s.bytes);
    return 0;
  } catch (const std::exception &) {
    return -1;
  }
}

}  // extern "C"

extern "C" {

// gemma_rope_tables (encoders/gemma_kernels.cpp:114-136): the RoPE cos/sin
// tables from a base, the form BertEncoder::apply_rope_qkv uses for nomic.
void ref_gemma_rope_tables(int64_t S, int64_t hd, double theta, float *cos_t, float *sin_t) {
  npue::gemma_rope_tables(S, hd, theta, cos_t, sin_t);
}

}  // extern "C"
