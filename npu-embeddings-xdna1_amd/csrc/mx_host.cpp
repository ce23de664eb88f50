// mx_host.cpp -- the host-only part of the C ABI: the thread-local error
// message every refusal sets, the --npu-ops placement registry
// (runtime/include/common/npu_ops_flag.hpp:75-268), the per-device guard of
// the static scratch and the device-allocation count. No HIP here: the
// container reader (mx_npue.cpp) and this file build with any C++17 compiler,
// which is how the sanitizer build of the untrusted-input paths compiles them.
#include "mx_host.hpp"

#include <atomic>
#include <cctype>
#include <cstring>
#include <mutex>
#include <set>
#include <string>

namespace mx {

static thread_local std::string t_err;

void set_error(const std::string &msg) { t_err = msg; }
void clear_error() { t_err.clear(); }

int fail(int code, const std::string &msg) {
  set_error(msg);
  return code;
}

// ---- placement registry ---------------------------------------------------

struct OpCode {
  const char *code;
  const char *long_name;
};

// The reference's codes, in its table order (npu_ops_flag.hpp:105-142).
static const OpCode kOps[] = {
    {"gemm", "the per-layer GEMMs"},
    {"gelu", "GELU"},
    {"layn", "LayerNorm"},
    {"softm", "softmax"},
    {"conv", "conv1d (Whisper's audio front end)"},
    {"attn", "attention (QK^T, softmax, softmax.V fused)"},
    {"mproj", "Whisper's mel filter bank, as a GEMM"},
    {"fft", "Whisper's 400-point transform, as a GEMM"},
    {"logit", "the vocabulary projection, as a GEMM"},
};

static std::mutex g_ops_mu;
static std::set<std::string> g_ops;

static std::string codes_joined() {
  std::string s;
  for (const auto &o : kOps) {
    if (!s.empty()) s += ", ";
    s += o.code;
  }
  return s;
}

std::set<std::string> placed_ops() {
  std::lock_guard<std::mutex> lk(g_ops_mu);
  return g_ops;
}

// ---- the static scratch's per-device guard --------------------------------
// mx_encoder_embed_static holds its device's entry for the whole call (every
// such call is host-synchronous); a call that finds the entry held is refused
// instead of racing on the shared scratch.

static std::mutex g_static_mu;
static std::set<int> g_static_held;

int static_guard_enter(int device, const char *who) {
  std::lock_guard<std::mutex> lk(g_static_mu);
  if (!g_static_held.insert(device).second)
    return fail(MX_E_STATE, std::string(who) + ": the static scratch of device " +
                                std::to_string(device) +
                                " is in use by another call; calls that overlap on one GPU "
                                "share it and are refused");
  return MX_OK;
}

int static_guard_leave(int device) {
  std::lock_guard<std::mutex> lk(g_static_mu);
  return g_static_held.erase(device) ? MX_OK : MX_E_STATE;
}

// ---- device allocations ----------------------------------------------------

static std::atomic<int64_t> g_allocs{0};

void count_device_allocation() { g_allocs.fetch_add(1, std::memory_order_relaxed); }

}  // namespace mx

using namespace mx;

extern "C" {

const char *mx_last_error(void) { return t_err.c_str(); }

int mx_version(void) { return 1; }

int mx_ops_parse(const char *list) {
  clear_error();
  if (!list) return fail(MX_E_INVALID, "--npu-ops: null list");
  std::set<std::string> out;
  std::string item;
  auto commit = [&]() -> bool {
    std::string code;
    for (char c : item)
      if (!std::isspace(static_cast<unsigned char>(c))) code.push_back(c);
    item.clear();
    if (code.empty()) return true;
    bool known = false;
    for (const auto &o : kOps) known = known || code == o.code;
    if (!known) {
      set_error("--npu-ops: '" + code + "' is not an op this build knows. Valid codes: [" +
                codes_joined() +
                "]. Nothing listed means no op is placed on the accelerator.");
      return false;
    }
    out.insert(code);
    return true;
  };
  for (const char *p = list; *p; ++p) {
    if (*p == ',') {
      if (!commit()) return MX_E_INVALID;
      continue;
    }
    item.push_back(*p);
  }
  if (!commit()) return MX_E_INVALID;
  std::lock_guard<std::mutex> lk(g_ops_mu);
  g_ops = out;
  return MX_OK;
}

int mx_op_on_gpu(const char *code) {
  if (!code) return 0;
  std::lock_guard<std::mutex> lk(g_ops_mu);
  return g_ops.count(code) ? 1 : 0;
}

const char *mx_op_codes(void) {
  static const std::string s = codes_joined();
  return s.c_str();
}

int mx_static_guard_hold(int device) {
  clear_error();
  if (device < 0) return fail(MX_E_INVALID, "static_guard_hold: negative device");
  return static_guard_enter(device, "static_guard_hold");
}

int mx_static_guard_release(int device) {
  clear_error();
  if (device < 0) return fail(MX_E_INVALID, "static_guard_release: negative device");
  if (static_guard_leave(device))
    return fail(MX_E_STATE, "static_guard_release: the static scratch of device " +
                                std::to_string(device) + " is not held");
  return MX_OK;
}

int64_t mx_device_allocations(void) { return g_allocs.load(std::memory_order_relaxed); }

int mx_ops_check_flag(const char *flag) {
  clear_error();
  if (!flag) return MX_OK;
  static const std::pair<const char *, const char *> removed[] = {
      {"--npu-eltwise", "--npu-ops gelu,layn,softm"},
      {"--host-gelu", "--npu-ops without gelu"},
      {"--host-ln", "--npu-ops without layn"},
      {"--host-sm", "--npu-ops without softm"},
      {"--npu-extra-ops", "--npu-ops"},
  };
  for (const auto &r : removed)
    if (std::strcmp(flag, r.first) == 0)
      return fail(MX_E_INVALID, std::string(r.first) +
                                    " is gone: one flag now says which ops go on the "
                                    "accelerator, and an op is on the host when it is NOT "
                                    "listed. Use " +
                                    r.second + ".");
  return MX_OK;
}

}  // extern "C"
