// Streaming-read bandwidth probe: the practical HBM read ceiling that the decode kernels are
// compared against next to the nominal 8 TB/s. No counterpart in the reference (measurement
// only).
//
// Each thread reads one 16-byte vector per grid-stride step and folds it into an xor that is
// kept live by a store that only happens for one specific value.
#include "common.h"

namespace sym {

__global__ __launch_bounds__(256) void hbm_read_probe_kernel(const uint4* __restrict__ p,
                                                              size_t n, uint32_t* __restrict__ sink) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  uint32_t acc = 0;
  for (; i < n; i += stride) {
    const uint4 v = p[i];
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  if (acc == 0x9E3779B9u) sink[0] = acc;
}

}  // namespace sym

using namespace sym;

extern "C" int sym_hbm_read_probe(const void* buf, size_t bytes, uint32_t* sink, void* stream) {
  SYM_REQUIRE(buf && sink, SYM_ERR_INVALID, "hbm_read_probe: null pointer argument");
  SYM_REQUIRE(bytes >= 16 && bytes % 16 == 0, SYM_ERR_INVALID,
              "hbm_read_probe: bytes=%zu must be a positive multiple of 16", bytes);
  (void)hipGetLastError();
  hipLaunchKernelGGL(hbm_read_probe_kernel, dim3(2048), dim3(256), 0, (hipStream_t)stream,
                     (const uint4*)buf, bytes / 16, sink);
  return sym_host::check_launch("hbm_read_probe_kernel");
}
