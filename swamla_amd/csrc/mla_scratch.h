// mla_scratch.h — layout of the per-device scratch area (mla_scratch.hip)
// used by mla_decode_attn_noalloc.
#pragma once

#include <stddef.h>
#include <stdint.h>

namespace swamla {

// Split-KV partials: o_part [rows, splits, H, R_pad] fp32 up to 16 MiB, then
// lse_part [rows, splits, H] fp32 (at most 1/64 of o_part's bytes, R_pad >= 64),
// then the balanced plan's chunk (one int32).
constexpr size_t kScratchPartBytes = size_t(16) << 20;
constexpr size_t kScratchLseBytes = kScratchPartBytes / 64;
constexpr size_t kScratchPlanOffset = kScratchPartBytes + kScratchLseBytes;
constexpr size_t kScratchBytes = kScratchPlanOffset + 256;

// One call's use of the calling thread's current device's scratch area, for
// the length of the call (constructor to destructor; host threads take turns
// on a device).  status: 0, and `area` holds the device address (looked up
// on the device's first call); -1 if the HIP runtime failed; -2 for a device
// ordinal past the ones tracked.  The constructor makes this call's stream
// wait for the completion event of the device's last call (on whichever
// stream it went to), so two calls never share the area at once; after its
// launches succeed the call marks launched(), which records its own event.
// Calls made while their stream is being captured into a graph neither wait
// nor record: their launches run at replay, and ordering replays that use the
// area on different streams is the caller's.
class ScratchUse {
 public:
  explicit ScratchUse(void* stream);
  ~ScratchUse();
  ScratchUse(const ScratchUse&) = delete;
  ScratchUse& operator=(const ScratchUse&) = delete;
  void launched();
  int status = -1;
  void* area = nullptr;

 private:
  int dev_ = -1;
  void* stream_ = nullptr;
  bool capturing_ = false;
};

}  // namespace swamla
