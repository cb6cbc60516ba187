// mla_scratch.hip — the library's one piece of device state: a fixed scratch
// area for the entry point that allocates nothing (mla_decode_attn_noalloc),
// holding the split-KV partials and the balanced plan between the decode and
// merge launches it makes, and the bookkeeping that orders calls from
// different streams so that they never share the area at once.
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
// per device: the area's address and a completion event of the last call
// (set up on the device's first call, kept to the end)
std::mutex g_mu[kMaxDevices];
void* g_ptr[kMaxDevices] = {};
hipEvent_t g_done[kMaxDevices] = {};
bool g_recorded[kMaxDevices] = {};

}  // namespace

ScratchUse::ScratchUse(void* stream) : stream_(stream) {
  if (hipGetDevice(&dev_) != hipSuccess) return;
  if (dev_ < 0 || dev_ >= kMaxDevices) {
    status = -2;
    dev_ = -1;
    return;
  }
  g_mu[dev_].lock();
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (!g_ptr[dev_]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return;
    if (hipEventCreateWithFlags(&g_done[dev_], hipEventDisableTiming) != hipSuccess) return;
    g_ptr[dev_] = p;
  }
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cs) != hipSuccess) return;
  capturing_ = cs != hipStreamCaptureStatusNone;
  // (also on the last call's own stream: a handle can be reused by a new
  // stream after the old one is destroyed)
  if (!capturing_ && g_recorded[dev_] && hipStreamWaitEvent(st, g_done[dev_], 0) != hipSuccess) return;
  area = g_ptr[dev_];
  status = 0;
}

void ScratchUse::launched() {
  if (status != 0 || capturing_) return;
  const hipStream_t st = static_cast<hipStream_t>(stream_);
  if (hipEventRecord(g_done[dev_], st) != hipSuccess) return;
  g_recorded[dev_] = true;
}

ScratchUse::~ScratchUse() {
  if (dev_ >= 0) g_mu[dev_].unlock();
}

}  // namespace swamla
