// mla_scratch.hip — the library's one piece of device state: a fixed scratch
// area for the entry point that allocates nothing (mla_decode_attn_noalloc),
// holding the split-KV partials and the balanced plan between the decode and
// merge launches it makes.
//
// `scratch` is a file-scope __device__ array: each GPU the library runs on
// gets its own copy when the code object loads there, and keeps it until the
// process ends.  In host code its name is only a stand-in for the symbol, not
// a device address, so the address is looked up once per device, with that
// device current (hipGetSymbolAddress), and that pointer is what the launches
// receive.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#include "mla_scratch.h"

namespace swamla {
namespace {

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_ptr[kMaxDevices] = {};

}  // namespace

int scratch_area(void** ptr) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) return -1;
  if (dev < 0 || dev >= kMaxDevices) return -2;
  std::lock_guard<std::mutex> lock(g_mu);
  if (!g_ptr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return -1;
    g_ptr[dev] = p;
  }
  *ptr = g_ptr[dev];
  return 0;
}

}  // namespace swamla
