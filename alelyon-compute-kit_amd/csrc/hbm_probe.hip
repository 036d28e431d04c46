// The HBM read ceiling the GEMV kernels are measured against: one pass that
// reads a buffer with the loads the GEMV's code stream uses (16-byte raw
// buffer loads, non-temporal) and does nothing else, so its rate is what a
// plain streaming read reaches on this GPU. Benchmarks time it on the
// library's stream (ack_stream_timer); it is not part of the vq4 path.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "kernels.hpp"

namespace ackvq {
namespace {

constexpr int kProbeThreads = 512;
constexpr int kProbeBlocks = 2048;   // eight per compute unit
constexpr int kProbeUnroll = 4;      // 16-byte loads in flight per lane

__global__ __launch_bounds__(kProbeThreads) void k_read_probe(const uint32_t* data, uint32_t bytes,
                                                             uint32_t* sink) {
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(data), 0, int(bytes), 0x00020000);
  const uint32_t chunks = bytes / 16;
  const uint32_t stride = gridDim.x * blockDim.x;
  uint32_t acc = 0;
  for (uint32_t c = blockIdx.x * blockDim.x + threadIdx.x; c < chunks;
       c += kProbeUnroll * stride) {
    uint32_t v[kProbeUnroll][4];
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) {  // chunks past the end read as zero
      const auto q = __builtin_amdgcn_raw_buffer_load_b128(rs, (c + u * stride) * 16u, 0, 2);
      v[u][0] = q[0]; v[u][1] = q[1]; v[u][2] = q[2]; v[u][3] = q[3];
    }
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  }
  // keeps the loads alive; no buffer the probe is given holds this pattern
  // in every lane's fold, and a write here would change nothing measured
  if (acc == 0x9e3779b9u && threadIdx.x == 0 && sink != nullptr) sink[blockIdx.x % 4] = acc;
}

}  // namespace

hipError_t launch_read_probe(hipStream_t s, const void* data, uint64_t bytes, uint32_t* sink) {
  k_read_probe<<<kProbeBlocks, kProbeThreads, 0, s>>>(static_cast<const uint32_t*>(data),
                                                      uint32_t(bytes), sink);
  return hipGetLastError();
}

}  // namespace ackvq
