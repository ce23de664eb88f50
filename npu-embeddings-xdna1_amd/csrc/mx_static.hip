// mx_static.hip -- the device scratch of mx_encoder_embed_static, the embed
// that allocates nothing: one file-scope array of MX_STATIC_SCRATCH_BYTES in
// device memory, which each GPU the library runs on holds (at its own
// address) from the library's first use of that GPU until the process ends.
//
// Host code never uses the array's name as an address: the name is a host
// stand-in. mx_create looks the device address up once per device, with that
// device current (static_scratch_init -> hipGetSymbolAddress), and every later
// use takes the looked-up pointer (static_scratch). Every call on one GPU
// shares the array and leaves its contents behind; nothing in it has to start
// at zero (each buffer carved from it is written before it is read), and
// calls that overlap on one GPU race.
#include "mx_internal.hpp"

static __device__ __align__(256) unsigned char scratch[MX_STATIC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void *g_ptr[kMaxDevices] = {};

}  // namespace

namespace mx {

int static_scratch_init(int device) {
  if (device < 0 || device >= kMaxDevices)
    return fail(MX_E_UNSUPPORTED, "static scratch: device " + std::to_string(device) +
                                      " is past the " + std::to_string(kMaxDevices) +
                                      " this library tracks");
  std::lock_guard<std::mutex> lk(g_mu);
  if (g_ptr[device]) return MX_OK;
  void *p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess) return hip_fail(e, "static scratch: hipGetSymbolAddress");
  if (!p) return fail(MX_E_DEVICE, "static scratch: hipGetSymbolAddress gave a null address");
  g_ptr[device] = p;
  return MX_OK;
}

int static_scratch(int device, void **ptr) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (device < 0 || device >= kMaxDevices || !g_ptr[device])
    return fail(MX_E_STATE, "static scratch: device " + std::to_string(device) +
                                " has no scratch address (mx_create looks it up)");
  *ptr = g_ptr[device];
  return MX_OK;
}

size_t static_scratch_bytes() { return MX_STATIC_SCRATCH_BYTES; }

}  // namespace mx
