// npue_san.cpp -- the untrusted-input host code under AddressSanitizer and
// UndefinedBehaviorSanitizer. TEST PROGRAM: built by tests/test_sanitize_cpu.py
// with g++ -fsanitize=address,undefined from this file, csrc/mx_host.cpp (the
// error state and the --npu-ops registry) and csrc/mx_npue.cpp (the .npue
// reader and its JSON parser); no HIP is involved.
//
//   npue_san <file>...
// opens each container (runtime/src/model.cpp:214-380's refusals), reads a
// set of config keys, every tensor's record and every byte of its data, and
// closes it; then drives the registry (npu_ops_flag.hpp:96-268) with
// malformed lists. Prints "opened <n> refused <m>" and exits 0; a sanitizer
// finding aborts the process with a report instead.
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>

#include "mx_encoder.h"

namespace {

int touch(const mx_npue *f) {
  static const char *keys[] = {"arch", "hidden", "num_layers", "pooling", "activation",
                               "rope_inv_freq", "int4_group", "fusions", "", "nested"};
  char buf[256];
  for (const char *k : keys) (void)mx_npue_config(f, k, buf, sizeof buf);
  (void)mx_npue_config(f, "arch", buf, 1);  // truncating buffer
  const int n = mx_npue_tensor_count(f);
  if (n < 0) return 1;
  unsigned sum = 0;
  for (int i = 0; i < n; ++i) {
    const char *name = mx_npue_tensor_name(f, i);
    if (!name) return 1;
    mx_npue_tensor_info t;
    if (mx_npue_tensor(f, name, &t) != MX_OK) return 1;
    const unsigned char *p = static_cast<const unsigned char *>(t.data);
    for (uint64_t b = 0; b < t.nbytes; ++b) sum += p[b];
  }
  (void)mx_npue_tensor_name(f, n);       // past the end
  (void)mx_npue_tensor_name(f, -1);
  mx_npue_tensor_info t;
  (void)mx_npue_tensor(f, "absent", &t);
  volatile unsigned sink = sum;
  (void)sink;
  return 0;
}

}  // namespace

int main(int argc, char **argv) {
  int opened = 0, refused = 0;
  for (int a = 1; a < argc; ++a) {
    mx_npue *f = nullptr;
    if (mx_npue_open(argv[a], &f) != MX_OK) {
      if (std::strlen(mx_last_error()) == 0) {
        std::printf("FAIL: %s refused with no reason\n", argv[a]);
        return 1;
      }
      ++refused;
      continue;
    }
    ++opened;
    if (touch(f)) {
      std::printf("FAIL: %s opened but its records are inconsistent\n", argv[a]);
      return 1;
    }
    mx_npue_close(f);
  }
  static const char *lists[] = {"", ",", ",,,", " gemm ", "gemm,attn,softm,layn,gelu",
                                "gemm,,gemm", "GEMM", "gemm;attn", "\t\n", "unknown",
                                "gemm,attn,softm,layn,gelu,conv,mproj,fft,logit,x"};
  for (const char *l : lists) {
    (void)mx_ops_parse(l);
    (void)mx_op_on_gpu(l);
    (void)mx_ops_check_flag(l);
  }
  std::string longlist(100000, 'g');
  (void)mx_ops_parse(longlist.c_str());
  (void)mx_ops_parse(nullptr);
  (void)mx_op_on_gpu(nullptr);
  (void)mx_ops_check_flag(nullptr);
  std::printf("opened %d refused %d\n", opened, refused);
  return 0;
}
