// Streaming-read calibration of the HBM roofline: reads a device buffer once
// with 16-byte loads (every lane keeps several loads in flight, grid-stride
// over the buffer) and folds the words into one XOR per workgroup, which it
// stores only if it equals a sentinel (so the loads are not removed).  The
// time of this kernel for a buffer the size of a workload's reads is the read
// bandwidth the part delivers in practice, the ceiling against which the
// decode kernel's bandwidth is compared (no counterpart in the reference).
// NT: non-temporal loads (the decode kernel's cache reads), which stream
// faster than ordinary ones on this part.
#include <stdint.h>

#include "capi.hpp"
#include "common.hpp"

namespace logo {

constexpr int kCalibUnroll = 4;

template <bool NT>
__global__ __launch_bounds__(256) void read_calibration_kernel(const u32x4* __restrict__ p, size_t n16,
                                                               uint32_t* sink) {
  uint32_t acc = 0;
  const size_t stride = (size_t)gridDim.x * 256 * kCalibUnroll;
  for (size_t base = (size_t)blockIdx.x * 256 * kCalibUnroll + threadIdx.x; base < n16; base += stride) {
    u32x4 v[kCalibUnroll];
#pragma unroll
    for (int u = 0; u < kCalibUnroll; ++u) {
      const size_t i = base + (size_t)u * 256;
      v[u] = i < n16 ? (NT ? __builtin_nontemporal_load(p + i) : p[i]) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < kCalibUnroll; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  if (acc == 0x9e3779b9u && threadIdx.x == 0) sink[blockIdx.x] = acc;
}

}  // namespace logo

using namespace logo;

extern "C" int logo_read_calibration(const void* buf, size_t bytes, void* sink, int grid, int nontemporal,
                                     void* stream) {
  LOGO_REQUIRE(buf && sink, "null pointer argument");
  LOGO_REQUIRE((reinterpret_cast<uintptr_t>(buf) & 15) == 0 && bytes % 16 == 0, "buffer must be 16-byte aligned");
  LOGO_REQUIRE(grid >= 1 && grid <= 65536, "grid must be in [1, 65536]");
  auto kern = nontemporal ? read_calibration_kernel<true> : read_calibration_kernel<false>;
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(256), 0, as_stream(stream), static_cast<const u32x4*>(buf),
                     bytes / 16, static_cast<uint32_t*>(sink));
  LOGO_LAUNCH_CHECK("read_calibration_kernel");
  return LOGO_OK;
}
