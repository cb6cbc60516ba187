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

// The calling thread's current device's scratch area (its device address,
// looked up on the device's first call).  0 on success; -1 if the HIP
// runtime failed; -2 for a device ordinal past the ones tracked.
int scratch_area(void** ptr);

}  // namespace swamla
