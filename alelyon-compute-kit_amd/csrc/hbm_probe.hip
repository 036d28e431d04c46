// The HBM read ceiling the GEMV kernels are measured against: one pass that
// reads a buffer with the loads and the access pattern of the GEMV's code
// stream and does nothing else, so its rate is what a plain streaming read
// reaches on this GPU. Each of 256 blocks (one per compute unit) streams its
// own contiguous share of the buffer, 512 threads issuing 16-byte raw buffer
// loads (non-temporal), eight in flight per lane; this pattern measured
// 6.9-7.2 TB/s where a grid-stride loop over 2,048 blocks reached 6.1 TB/s.
//
// Built as its own library (libackprobe.so), which only the benchmark's
// calibration loads: it is not part of the vq4 path or of libackvq.so.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

constexpr int kProbeThreads = 512;
constexpr int kProbeBlocks = 256;    // one per compute unit
constexpr int kProbeUnroll = 8;      // 16-byte loads in flight per lane

// sink is null at every launch: the store it guards never runs, but the
// compiler cannot know that, so the loads feeding `acc` stay.
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
  if (sink != nullptr && threadIdx.x == 0) sink[blockIdx.x] = acc;
}

}  // namespace

// Reads `bytes` (16 bytes to 2 GiB - 1) at the device address `data`
// `launches` times on a stream of its own, each launch bracketed by events;
// ms[i] receives launch i's time. Returns 0, or -1 for bad arguments, or the
// HIP error code of the failing call. Allocates nothing on the device.
extern "C" int32_t ack_probe_read_ms(const void* data, uint64_t bytes, uint32_t launches,
                                     float* ms) {
  if (data == nullptr || ms == nullptr || launches == 0 || bytes < 16 || bytes >= (1ull << 31))
    return -1;
  hipStream_t stream = nullptr;
  hipEvent_t start = nullptr, stop = nullptr;
  hipError_t e = hipStreamCreate(&stream);
  if (e == hipSuccess) e = hipEventCreate(&start);
  if (e == hipSuccess) e = hipEventCreate(&stop);
  for (uint32_t i = 0; e == hipSuccess && i < launches; ++i) {
    e = hipEventRecord(start, stream);
    if (e != hipSuccess) break;
    k_read_probe<<<kProbeBlocks, kProbeThreads, 0, stream>>>(static_cast<const uint32_t*>(data),
                                                            uint32_t(bytes), nullptr);
    e = hipGetLastError();
    if (e == hipSuccess) e = hipEventRecord(stop, stream);
    if (e == hipSuccess) e = hipEventSynchronize(stop);
    if (e == hipSuccess) e = hipEventElapsedTime(&ms[i], start, stop);
  }
  if (stop) (void)hipEventDestroy(stop);
  if (start) (void)hipEventDestroy(start);
  if (stream) (void)hipStreamDestroy(stream);
  return e == hipSuccess ? 0 : int32_t(e);
}
