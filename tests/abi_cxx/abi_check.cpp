// abi_check.cpp -- a C++17 caller of the C ABI through include/mx_gpu_backend.hpp,
// compiled with g++ against include/ and linked to libmx_encoder.so (built by
// npu-embeddings-xdna1_amd/build.py), as the reference runtime would be.
// TEST PROGRAM.
//
//   abi_check cpu [<container.npue> <key> <value>]
//       The paths that need no GPU: the op registry with the reference's
//       refusals (npu_ops_flag.hpp:96-214, :238-268), the container reader's
//       refusals (model.cpp:214-380), null-argument refusals, plan names --
//       each failure surfacing as std::runtime_error("gpu: ...") through the
//       wrapper; with a container, its config read through the wrapper (the
//       value of <key> must be <value>). Prints "cpu ok".
//   abi_check gpu <container.npue> <ids.bin> <mask.bin> <B> <S> <out.bin>
//       One embed on GPU 0: the container loaded by mxgpu::Encoder, ids int32
//       [B, S] and the 1/0 mask fp32 [B, S] from the files, the pooled fp32
//       [B, hidden] written to out.bin. Prints "gpu ok".
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <string>
#include <vector>

#include "mx_gpu_backend.hpp"

namespace {

int failures = 0;

void expect(bool ok, const char *what) {
  if (!ok) {
    std::printf("FAIL: %s\n", what);
    ++failures;
  }
}

// The wrapper must turn `rc` into a runtime_error whose text holds `needle`.
void expect_refusal(int rc, const char *needle, const char *what) {
  try {
    mxgpu::check(rc);
    std::printf("FAIL: %s: no refusal\n", what);
    ++failures;
  } catch (const std::runtime_error &e) {
    const std::string m = e.what();
    if (m.rfind("gpu: ", 0) != 0 || m.find(needle) == std::string::npos) {
      std::printf("FAIL: %s: '%s' lacks '%s'\n", what, m.c_str(), needle);
      ++failures;
    }
  }
}

template <typename T>
std::vector<T> read_file(const char *path, size_t count) {
  std::vector<T> v(count);
  std::ifstream f(path, std::ios::binary);
  f.read(reinterpret_cast<char *>(v.data()), static_cast<std::streamsize>(count * sizeof(T)));
  if (!f) throw std::runtime_error(std::string("cannot read ") + path);
  return v;
}

int run_cpu(const char *container, const std::string &key, const std::string &value) {
  expect(mx_version() > 0, "mx_version");
  // The registry: codes, separators, unknown codes and removed flags.
  expect(mx_ops_parse(" gemm ,attn,, softm,layn , gelu,") == MX_OK, "ops_parse list");
  expect(mx_op_on_gpu("attn") == 1 && mx_op_on_gpu("flash") == 0, "op_on_gpu");
  expect_refusal(mx_ops_parse("gemm,flash"), "flash", "unknown op code");
  expect(mx_ops_parse("") == MX_OK && mx_op_on_gpu("gemm") == 0, "empty list: all host");
  expect_refusal(mx_ops_check_flag("--npu-eltwise"), "gelu,layn,softm", "removed flag");
  expect(mx_ops_check_flag("--npu-ops") == MX_OK, "current flag");
  // The container reader refuses a missing file by name, through the wrapper.
  try {
    mxgpu::Container c("/nonexistent/model.npue");
    std::printf("FAIL: opened a missing container\n");
    ++failures;
  } catch (const std::runtime_error &e) {
    expect(std::string(e.what()).find("cannot open") != std::string::npos, "missing container");
  }
  // Null arguments are refused before any device work.
  expect_refusal(mx_gemm_wt(nullptr, nullptr, 8, 8, 8, nullptr, 8, nullptr, 0, nullptr, nullptr,
                            MX_F32, 8),
                 "null", "gemm without a stream");
  expect_refusal(mx_encoder_embed(nullptr, nullptr, nullptr, nullptr, 1, 1, nullptr), "null",
                 "embed without an encoder");
  const char *plan = mx_gemm_plan_for(17455, 2304, 768, MX_BF16, 0, 0);
  expect(plan && std::strncmp(plan, "lds_", 4) == 0, "plan name");
  // A valid container: its config values through the wrapper, a missing key
  // refused by name.
  if (container) {
    mxgpu::Container c(container);
    expect(c.config(key) == value, "config value");
    expect(std::atoll(c.config("hidden").c_str()) > 0, "config hidden");
    try {
      (void)c.config("no_such_key");
      std::printf("FAIL: a missing config key was read\n");
      ++failures;
    } catch (const std::runtime_error &e) {
      expect(std::string(e.what()).find("no_such_key") != std::string::npos, "missing key");
    }
  }
  if (failures) return 1;
  std::printf("cpu ok\n");
  return 0;
}

int run_gpu(int argc, char **argv) {
  if (argc < 8) {
    std::printf("usage: abi_check gpu <container> <ids> <mask> <B> <S> <out>\n");
    return 2;
  }
  const int64_t B = std::atoll(argv[5]), S = std::atoll(argv[6]);
  const auto ids = read_file<int32_t>(argv[3], static_cast<size_t>(B * S));
  const auto mask = read_file<float>(argv[4], static_cast<size_t>(B * S));
  mxgpu::Backend be(0);
  mxgpu::Lane lane(be);
  mxgpu::Container file(argv[2]);
  const int64_t hidden = std::atoll(file.config("hidden").c_str());
  mxgpu::Encoder enc(be, file);
  mxgpu::Buffer d_ids(be, ids.size() * 4), d_mask(be, mask.size() * 4),
      d_out(be, static_cast<size_t>(B * hidden) * 4);
  lane.to_device(d_ids.get(), ids.data(), ids.size() * 4);
  lane.to_device(d_mask.get(), mask.data(), mask.size() * 4);
  enc.embed(lane, static_cast<const int32_t *>(d_ids.get()),
            static_cast<const float *>(d_mask.get()), B, S, static_cast<float *>(d_out.get()));
  std::vector<float> out(static_cast<size_t>(B * hidden));
  lane.to_host(out.data(), d_out.get(), out.size() * 4);
  lane.sync();
  // The queued embed gives the same rows once the lane is synchronised.
  mxgpu::Buffer d_out2(be, static_cast<size_t>(B * hidden) * 4);
  enc.embed_async(lane, static_cast<const int32_t *>(d_ids.get()),
                  static_cast<const float *>(d_mask.get()), B, S,
                  static_cast<float *>(d_out2.get()));
  lane.sync();
  std::vector<float> out2(out.size());
  lane.to_host(out2.data(), d_out2.get(), out2.size() * 4);
  lane.sync();
  if (std::memcmp(out.data(), out2.data(), out.size() * 4) != 0) {
    std::printf("FAIL: embed_async rows differ from embed's\n");
    ++failures;
  }
  // The embed service from host memory, two lanes in chunks of 3 sequences:
  // the same rows, whatever the chunking.
  {
    mxgpu::EmbedService svc(enc, 2, 3, S);
    std::vector<float> out3(out.size());
    svc.embed(ids.data(), mask.data(), B, out3.data());
    if (std::memcmp(out.data(), out3.data(), out.size() * 4) != 0) {
      std::printf("FAIL: the embed service's rows differ from embed's\n");
      ++failures;
    }
  }
  // A refusal on the live device also arrives as an exception.
  expect_refusal(mx_encoder_embed(enc.get(), lane.get(), static_cast<const int32_t *>(d_ids.get()),
                                  static_cast<const float *>(d_mask.get()), 0, S,
                                  static_cast<float *>(d_out.get())),
                 "", "embed of zero sequences");
  std::ofstream f(argv[7], std::ios::binary);
  f.write(reinterpret_cast<const char *>(out.data()),
          static_cast<std::streamsize>(out.size() * 4));
  if (!f) {
    std::printf("FAIL: cannot write %s\n", argv[7]);
    return 1;
  }
  if (failures) return 1;
  std::printf("gpu ok\n");
  return 0;
}

}  // namespace

int main(int argc, char **argv) {
  try {
    if (argc >= 2 && std::strcmp(argv[1], "cpu") == 0)
      return run_cpu(argc >= 5 ? argv[2] : nullptr, argc >= 5 ? argv[3] : "",
                     argc >= 5 ? argv[4] : "");
    if (argc >= 2 && std::strcmp(argv[1], "gpu") == 0) return run_gpu(argc, argv);
    std::printf("usage: abi_check cpu | gpu ...\n");
    return 2;
  } catch (const std::exception &e) {
    std::printf("FAIL: %s\n", e.what());
    return 1;
  }
}
