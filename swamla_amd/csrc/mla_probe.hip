// mla_probe.hip — the plain HBM read ceiling, a measurement kernel with no
// reference counterpart (bench.py reports it as roofline.ceiling_gbs beside
// the decode launch; the module never runs it).
//
// mla_read_probe streams a buffer once with 16-byte non-temporal loads, four
// independent loads in flight per lane per step (each wave reads whole 1 KB
// runs), and folds every word into a per-thread checksum stored at
// sink[thread], so the read is observable.  The bench rotates it over
// regions larger than the Infinity Cache, so the rate it reports is HBM's.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mla_args.h"

namespace swamla {
namespace {

typedef unsigned int rp_u32x4_t __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void mla_read_probe(const rp_u32x4_t* src, int64_t n16, uint32_t* sink) {
  const int64_t nt = static_cast<int64_t>(gridDim.x) * 256;
  int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t tid = i;
  uint32_t acc = 0;
  for (; i + 3 * nt < n16; i += 4 * nt) {
    const rp_u32x4_t v0 = __builtin_nontemporal_load(src + i);
    const rp_u32x4_t v1 = __builtin_nontemporal_load(src + i + nt);
    const rp_u32x4_t v2 = __builtin_nontemporal_load(src + i + 2 * nt);
    const rp_u32x4_t v3 = __builtin_nontemporal_load(src + i + 3 * nt);
    const rp_u32x4_t v = v0 ^ v1 ^ v2 ^ v3;
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  for (; i < n16; i += nt) {
    const rp_u32x4_t v = __builtin_nontemporal_load(src + i);
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  sink[tid] = acc;
}

}  // namespace

int launch_read_probe(const void* src, int64_t n16, uint32_t* sink, int grid, hipStream_t s) {
  hipLaunchKernelGGL(mla_read_probe, dim3(grid), dim3(256), 0, s, static_cast<const rp_u32x4_t*>(src), n16, sink);
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

}  // namespace swamla
