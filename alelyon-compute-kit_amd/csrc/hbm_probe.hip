// The HBM read ceiling the GEMV kernels are measured against: one pass that
// reads a buffer with the loads and the access pattern of the GEMV's code
// stream and does nothing else, so its rate is what a plain streaming read
// reaches on this GPU. Each of 256 blocks (one per compute unit) streams its
// own contiguous share of the buffer, 512 threads issuing 16-byte raw buffer
// loads (non-temporal), eight in flight per lane; this pattern measured
// 6.9-7.2 TB/s where a grid-stride loop over 2,048 blocks reached 6.1 TB/s.
// Benchmarks time it on the library's stream (ack_stream_timer); it is not
// part of the vq4 path.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "kernels.hpp"

namespace ackvq {
namespace {

constexpr int kProbeThreads = 512;
constexpr int kProbeBlocks = 256;    // one per compute unit
constexpr int kProbeUnroll = 8;      // 16-byte loads in flight per lane

__global__ __launch_bounds__(kProbeThreads) void k_read_probe(const uint32_t* data, uint32_t bytes,
                                                             uint32_t* sink) {
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(data), 0, int(bytes), 0x00020000);
  const uint32_t per = bytes / gridDim.x / 16 * 16;  // this block's share (the last 16-byte
  const uint32_t base = blockIdx.x * per;            // chunks of an uneven size are not read)
  uint32_t acc = 0;
  for (uint32_t o = threadIdx.x * 16u; o < per; o += kProbeUnroll * kProbeThreads * 16u) {
    uint32_t v[kProbeUnroll][4];
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) {  // past the share: the next block's, or zero
      const auto q = __builtin_amdgcn_raw_buffer_load_b128(rs, base + o + u * kProbeThreads * 16u, 0, 2);
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
