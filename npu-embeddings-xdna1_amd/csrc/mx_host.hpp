// mx_host.hpp -- host-only declarations shared by every source behind the C
// ABI (no HIP): the error state, the placement registry's view and the
// container reader's tensor view.
#pragma once

#include <cstdint>
#include <set>
#include <string>
#include <vector>

#include "../../include/mx_encoder.h"

namespace mx {

// Thread-local last error, set by every failing entry point.
void set_error(const std::string &msg);
void clear_error();
int fail(int code, const std::string &msg);

// The static scratch's per-device guard (mx_encoder_embed_static): enter
// refuses with MX_E_STATE, naming `who`, when a call on that device holds it.
int static_guard_enter(int device, const char *who);
int static_guard_leave(int device);

// Every device allocation the library makes is counted (mx_device_allocations).
void count_device_allocation();

// The codes --npu-ops placed on the GPU (mx_ops_parse).
std::set<std::string> placed_ops();

// A container tensor as the loaders use it (mx_npue.cpp).
struct TensorRecView {
  bool found = false, has_layout = false, block_panel = false;
  std::string dtype;
  std::vector<int64_t> padded, logical;
  int64_t tile_k = 0, tile_n = 0, mac_s = 0, mac_t = 0;
  const void *data = nullptr;
  uint64_t nbytes = 0;
};
const TensorRecView npue_tensor(const mx_npue *f, const std::string &name);
bool npue_config(const mx_npue *f, const std::string &key, std::string &out);

}  // namespace mx
