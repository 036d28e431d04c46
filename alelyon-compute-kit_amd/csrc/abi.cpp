// C ABI of libackvq.so over HIP: device and buffer registry, transfers, and
// the vq4/v1 entry ack_vq with its admission order.
//
// Mirrors src/alelyon_compute_kit/_kit/src/ffi.rs for the entries the vq
// binding uses: handles are ids (device = counter, buffer = (device << 32) |
// sequence, ffi.rs:10-24) that are looked up under a lock and refused by name,
// never dereferenced; the last error is thread-local (ffi.rs:1290-1292,
// :3325-3339); ack_vq checks plan, device, poison, handles, capacities and
// aliases in the reference's order (ffi.rs:6037-6151) before anything reaches
// the device. Where the reference records a Vulkan dispatch into a deferred
// batch, this library enqueues on the device's HIP stream: ACK_OK means
// accepted, and ack_download (which waits on the stream) is the point where
// results exist -- the same contract.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdarg>
#include <cstddef>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/ack_vq.h"
#include "host_fit.hpp"
#include "kernels.hpp"
#include "plan.hpp"

namespace {

thread_local std::string t_last_error;

void set_error(const std::string& message) { t_last_error = message; }

struct BufferRec {
  void* ptr = nullptr;
  uint64_t bytes = 0;
  uint64_t id = 0;
};

struct Device {
  uint64_t id = 0;
  int hip_device = 0;
  hipStream_t stream = nullptr;
  hipEvent_t timer_start = nullptr;
  hipEvent_t timer_stop = nullptr;
  std::mutex mu;
  bool closed = false;
  bool poisoned = false;
  uint32_t next_buffer = 1;
  uint32_t policy = 0;
  std::unordered_map<uint32_t, BufferRec> buffers;
  std::string name;
  void* workspace = nullptr;
  size_t workspace_bytes = 0;
  void* scratch = nullptr;  // this GPU's copy of `scratch` (ack_vq_noalloc), or null
  uint32_t* arrivals = nullptr;  // gemv-direct's counters, zeroed at open (Operands::arrivals)
};

struct Registry {
  std::mutex mu;
  std::unordered_map<uint64_t, std::shared_ptr<Device>> devices;
};

Registry& registry() {
  static Registry* r = new Registry();  // never destroyed: outlives every caller
  return *r;
}

std::atomic<uint64_t> g_next_device{1};

uint64_t buffer_handle(uint64_t device, uint32_t seq) { return (device << 32) | seq; }

// device() of ffi.rs:1887-1902.
int32_t lookup_device(const AckDevice* handle, std::shared_ptr<Device>* out) {
  const uint64_t id = uint64_t(reinterpret_cast<uintptr_t>(handle));
  if (id == 0) return ACK_ERR_NULL;
  Registry& r = registry();
  std::lock_guard<std::mutex> lock(r.mu);
  auto it = r.devices.find(id);
  if (it == r.devices.end()) {
    set_error("device handle " + std::to_string(id) +
              " is not open (closed, never opened, or not a kit handle)");
    return ACK_ERR_CLOSED;
  }
  *out = it->second;
  return ACK_OK;
}

// buffer_of() of ffi.rs:1921-1944; caller holds dev.mu.
int32_t lookup_buffer(Device& dev, const AckBuffer* handle, BufferRec** out) {
  const uint64_t raw = uint64_t(reinterpret_cast<uintptr_t>(handle));
  if (raw == 0) return ACK_ERR_NULL;
  const uint64_t owner = raw >> 32;
  const uint32_t seq = uint32_t(raw & 0xffffffffu);
  char hex[32];
  std::snprintf(hex, sizeof hex, "%#llx", static_cast<unsigned long long>(raw));
  if (owner != dev.id) {
    set_error(std::string("buffer ") + hex + " belongs to device " + std::to_string(owner) +
              ", not device " + std::to_string(dev.id));
    return ACK_ERR_FOREIGN;
  }
  auto it = dev.buffers.find(seq);
  if (it == dev.buffers.end()) {
    set_error(std::string("buffer ") + hex + " is not live on device " + std::to_string(dev.id) +
              " (freed, or never allocated)");
    return ACK_ERR_FREED;
  }
  *out = &it->second;
  return ACK_OK;
}

// A device runtime failure. Errors after work was enqueued leave the device
// state unknown: the device is poisoned and refuses later calls, as the
// reference does after an ambiguous fence wait (ffi.rs:16-19).
int32_t hip_failure(Device& dev, const char* what, hipError_t err, bool poison) {
  set_error(std::string(what) + ": " + hipGetErrorString(err));
  if (poison) dev.poisoned = true;
  return ACK_ERR_DEVICE;
}

int32_t plan_code(ackvq::PlanError e) {
  switch (e) {
    case ackvq::PlanError::Capacity:
    case ackvq::PlanError::AddressLimit:
    case ackvq::PlanError::WorkLimit:
      return ACK_ERR_SIZE;
    default:
      return ACK_ERR_SHAPE;
  }
}

// Steps 1-3 of the check order: the plan block alone.
int32_t parse_plan(const uint8_t* plan, size_t plan_len, ackvq::Bounds bounds, ackvq::Plan* out) {
  if (plan == nullptr) {
    set_error("vq: null plan");
    return ACK_ERR_NULL;
  }
  if (plan_len != ackvq::kPushBytes) {
    set_error("vq: plan has " + std::to_string(plan_len) + " bytes, expected 32");
    return ACK_ERR_SIZE;
  }
  std::array<uint32_t, 8> words{};
  for (int i = 0; i < 8; ++i)
    words[i] = uint32_t(plan[4 * i]) | (uint32_t(plan[4 * i + 1]) << 8) |
               (uint32_t(plan[4 * i + 2]) << 16) | (uint32_t(plan[4 * i + 3]) << 24);
  ackvq::PlanError e = ackvq::plan_from_words(words, bounds, out);
  if (e != ackvq::PlanError::None) {
    set_error("vq: plan refused: " + ackvq::plan_error_name(e));
    return plan_code(e);
  }
  return ACK_OK;
}

size_t round_up(size_t bytes) { return (bytes + 255) / 256 * 256; }

// ---- the allocation-free entry's scratch ----------------------------------------
// ack_vq_noalloc takes the workspace of the paths that need one (the GEMV's
// split-k partials, gemv-direct's slice partials, onehot-mfma's nibble
// columns and split-k partials) from this array instead
// of allocating it. Every GPU the library runs on holds its own copy until
// the process ends. In host code `scratch` names a host-side stand-in, never
// a device address: the address is resolved per GPU with
// hipGetSymbolAddress (scratch_address) and only that pointer is passed on.
constexpr size_t kScratchBytes = size_t(16) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxGpus = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxGpus] = {};
bool g_scratch_done[kMaxGpus] = {};

// The scratch of a GPU belongs to one device handle at a time: the handle
// whose ack_vq_noalloc launch used it last, with an event recorded on that
// handle's stream after the launch. Calls on one handle are ordered by its
// stream; another handle's call is refused while the event is pending, so
// two handles never have work on one GPU's scratch at the same time. Claim,
// launch and record happen under g_scratch_mu.
struct ScratchOwner {
  uint64_t device = 0;      // id of the owning handle, 0 before the first use
  hipEvent_t done = nullptr;  // recorded after the owner's last launch
};
ScratchOwner g_scratch_owner[kMaxGpus];

// This GPU's `scratch`, resolved once per GPU with that GPU current (the
// caller has selected it). Null when resolution failed.
void* scratch_address(int hip_device) {
  if (hip_device < 0 || hip_device >= kMaxGpus) return nullptr;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_done[hip_device]) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) == hipSuccess) g_scratch_ptr[hip_device] = ptr;
    g_scratch_done[hip_device] = true;
  }
  return g_scratch_ptr[hip_device];
}

int32_t ensure_workspace(Device& dev, size_t bytes) {
  if (bytes <= dev.workspace_bytes) return ACK_OK;
  if (dev.workspace) {
    hipError_t e = hipStreamSynchronize(dev.stream);
    if (e != hipSuccess) return hip_failure(dev, "vq: workspace wait", e, true);
    (void)hipFree(dev.workspace);
    dev.workspace = nullptr;
    dev.workspace_bytes = 0;
  }
  hipError_t e = hipMalloc(&dev.workspace, bytes);
  if (e != hipSuccess) {
    dev.workspace = nullptr;
    return hip_failure(dev, "vq: workspace allocation", e, false);
  }
  dev.workspace_bytes = bytes;
  return ACK_OK;
}

// Steps 4-7 then the launch, shared by ack_vq, ack_vq_batch and
// ack_vq_noalloc (no_alloc: the workspace is the GPU's `scratch`, and a plan
// needing more than kScratchBytes of it is refused).
int32_t run_vq(const AckDevice* handle, const AckBuffer* const slots[6], const uint8_t* plan_bytes,
               size_t plan_len, uint32_t count, bool no_alloc = false) {
  ackvq::Plan plan;
  if (int32_t rc = parse_plan(plan_bytes, plan_len, ackvq::Bounds::Library, &plan)) return rc;
  std::shared_ptr<Device> dev;
  if (int32_t rc = lookup_device(handle, &dev)) return rc;
  std::lock_guard<std::mutex> lock(dev->mu);
  if (dev->closed) {
    set_error("device " + std::to_string(dev->id) + " is closed");
    return ACK_ERR_CLOSED;
  }
  if (dev->poisoned) {
    set_error("vq: device poisoned by an earlier ambiguous operation");
    return ACK_ERR_POISONED;
  }
  BufferRec* bufs[6];
  uint64_t capacities[6], ids[6];
  for (int i = 0; i < 6; ++i) {
    if (int32_t rc = lookup_buffer(*dev, slots[i], &bufs[i])) return rc;
    capacities[i] = bufs[i]->bytes;
    ids[i] = bufs[i]->id;
  }
  // Batched instances: every slot must hold `count` images; the status word
  // is shared.
  ackvq::Plan scaled = plan;
  if (count > 1) {
    for (int i = 0; i < 5; ++i) {
      const unsigned __int128 need = (unsigned __int128)plan.required_bytes[i] * count;
      scaled.required_bytes[i] = need > UINT64_MAX ? UINT64_MAX : uint64_t(need);
    }
  }
  int slot = 0;
  ackvq::PlanError e = ackvq::validate_buffers(scaled, capacities, ids, &slot);
  if (e == ackvq::PlanError::None) {
    const uint32_t limits[3] = {65535, 65535, 65535};
    e = ackvq::validate_dispatch(plan, limits);
  }
  if (e != ackvq::PlanError::None) {
    set_error("vq: plan refused: " + ackvq::plan_error_name(e, slot));
    return plan_code(e);
  }
  hipError_t he = hipSetDevice(dev->hip_device);
  if (he != hipSuccess) return hip_failure(*dev, "vq: device selection", he, false);

  ackvq::Operands o;
  o.arrivals = dev->arrivals;
  for (int i = 0; i < 4; ++i) {
    o.in[i] = bufs[i]->ptr;
    o.stride[i] = count > 1 ? plan.required_bytes[i] : 0;
  }
  o.out = bufs[4]->ptr;
  o.stride[4] = count > 1 ? plan.required_bytes[4] : 0;
  o.status = static_cast<uint32_t*>(bufs[5]->ptr);
  o.count = count;
  const uint32_t m = plan.m(), n = plan.n(), k = plan.k(), g = plan.group();
  switch (plan.op) {
    case ackvq::Op::Encode: he = ackvq::launch_encode(dev->stream, o, m, g); break;
    case ackvq::Op::Decode: he = ackvq::launch_decode(dev->stream, o, m, g); break;
    case ackvq::Op::AdamW: he = ackvq::launch_adamw(dev->stream, o, m, g); break;
    case ackvq::Op::Matmul: {
      const ackvq::MatmulPath path =
          ackvq::choose_matmul_path(m, n, k, g, plan.flags(), count, dev->policy);
      const size_t ws = ackvq::matmul_workspace_bytes(path, m, n, k, g, plan.flags(), count);
      void* work = nullptr;
      size_t work_bytes = 0;
      if (no_alloc) {
        if (ws > kScratchBytes) {
          set_error("vq noalloc: the product needs " + std::to_string(ws) +
                    " bytes of workspace, more than the " + std::to_string(kScratchBytes) +
                    "-byte scratch; use ack_vq");
          return ACK_ERR_SIZE;
        }
        if (dev->scratch == nullptr) {
          set_error("vq noalloc: the device address of the scratch array is unknown");
          return ACK_ERR_DEVICE;
        }
        work = dev->scratch;
        work_bytes = kScratchBytes;
        if (ws > 0) {  // the path writes the scratch: claim it, launch, mark the launch's end
          std::lock_guard<std::mutex> own_lock(g_scratch_mu);
          ScratchOwner& own = g_scratch_owner[dev->hip_device];
          if (own.device != 0 && own.device != dev->id && own.done != nullptr) {
            const hipError_t q = hipEventQuery(own.done);
            (void)hipGetLastError();  // a pending query must not read as a launch failure
            if (q == hipErrorNotReady) {
              set_error("vq noalloc: this GPU's scratch is in use by device handle " +
                        std::to_string(own.device) +
                        " (its enqueued ack_vq_noalloc work has not finished); synchronize "
                        "that handle first, or use ack_vq");
              return ACK_ERR_DEVICE;
            }
          }
          if (own.done == nullptr) {
            he = hipEventCreateWithFlags(&own.done, hipEventDisableTiming);
            if (he != hipSuccess) {
              own.done = nullptr;
              return hip_failure(*dev, "vq noalloc: scratch event", he, false);
            }
          }
          he = ackvq::launch_matmul(dev->stream, o, m, n, k, g, plan.flags(), path, work,
                                    work_bytes);
          if (he == hipSuccess) he = hipEventRecord(own.done, dev->stream);
          if (he != hipSuccess) return hip_failure(*dev, "vq: kernel launch refused", he, false);
          own.device = dev->id;
          return ACK_OK;
        }
      } else {
        if (int32_t rc = ensure_workspace(*dev, ws)) return rc;
        work = dev->workspace;
        work_bytes = dev->workspace_bytes;
      }
      he = ackvq::launch_matmul(dev->stream, o, m, n, k, g, plan.flags(), path, work, work_bytes);
      break;
    }
  }
  if (he != hipSuccess) return hip_failure(*dev, "vq: kernel launch refused", he, false);
  return ACK_OK;
}

// Shared prologue of the transfer and control entries.
int32_t enter(const AckDevice* handle, std::shared_ptr<Device>* dev,
              std::unique_lock<std::mutex>* lock, bool refuse_poisoned = true) {
  if (int32_t rc = lookup_device(handle, dev)) return rc;
  *lock = std::unique_lock<std::mutex>((*dev)->mu);
  if ((*dev)->closed) {
    set_error("device " + std::to_string((*dev)->id) + " is closed");
    return ACK_ERR_CLOSED;
  }
  if (refuse_poisoned && (*dev)->poisoned) {
    set_error("device poisoned by an earlier ambiguous operation");
    return ACK_ERR_POISONED;
  }
  hipError_t e = hipSetDevice((*dev)->hip_device);
  if (e != hipSuccess) return hip_failure(**dev, "device selection", e, false);
  return ACK_OK;
}

}  // namespace

extern "C" {

uint32_t ack_vq_schema(void) { return ackvq::kSchema; }

int32_t ack_vq(const AckDevice* dev, const AckBuffer* b0, const AckBuffer* b1, const AckBuffer* b2,
               const AckBuffer* b3, const AckBuffer* out, const AckBuffer* status,
               const uint8_t* plan, size_t plan_len) {
  const AckBuffer* slots[6] = {b0, b1, b2, b3, out, status};
  return run_vq(dev, slots, plan, plan_len, 1);
}

int32_t ack_vq_batch(const AckDevice* dev, const AckBuffer* b0, const AckBuffer* b1,
                     const AckBuffer* b2, const AckBuffer* b3, const AckBuffer* out,
                     const AckBuffer* status, const uint8_t* plan, size_t plan_len,
                     uint32_t count) {
  if (count == 0) {
    set_error("vq: batch count must be at least 1");
    return ACK_ERR_SHAPE;
  }
  const AckBuffer* slots[6] = {b0, b1, b2, b3, out, status};
  return run_vq(dev, slots, plan, plan_len, count);
}

int32_t ack_vq_noalloc(const AckDevice* dev, const AckBuffer* b0, const AckBuffer* b1,
                       const AckBuffer* b2, const AckBuffer* b3, const AckBuffer* out,
                       const AckBuffer* status, const uint8_t* plan, size_t plan_len) {
  const AckBuffer* slots[6] = {b0, b1, b2, b3, out, status};
  return run_vq(dev, slots, plan, plan_len, 1, true);
}

AckDevice* ack_open(void) {
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess || count == 0) {
    set_error(std::string("no HIP device: ") +
              (e != hipSuccess ? hipGetErrorString(e) : "device count is 0"));
    return nullptr;
  }
  int index = 0;
  if (const char* choice = std::getenv("ACK_DEVICE")) {
    if (std::strncmp(choice, "gpu:", 4) != 0 || choice[4] == '\0') {
      set_error(std::string("ACK_DEVICE=") + choice + " is not gpu:<index>");
      return nullptr;
    }
    char* end = nullptr;
    long v = std::strtol(choice + 4, &end, 10);
    if (*end != '\0' || v < 0 || v >= count) {
      set_error(std::string("ACK_DEVICE=") + choice + " names no device (" +
                std::to_string(count) + " present)");
      return nullptr;
    }
    index = int(v);
  }
  auto dev = std::make_shared<Device>();
  dev->hip_device = index;
  if ((e = hipSetDevice(index)) != hipSuccess ||
      (e = hipStreamCreateWithFlags(&dev->stream, hipStreamNonBlocking)) != hipSuccess ||
      (e = hipEventCreate(&dev->timer_start)) != hipSuccess ||
      (e = hipEventCreate(&dev->timer_stop)) != hipSuccess ||
      (e = hipMalloc(reinterpret_cast<void**>(&dev->arrivals),
                     ackvq::kDirectCounters * sizeof(uint32_t))) != hipSuccess ||
      (e = hipMemset(dev->arrivals, 0, ackvq::kDirectCounters * sizeof(uint32_t))) !=
          hipSuccess ||
      (e = hipDeviceSynchronize()) != hipSuccess) {
    set_error(std::string("device open: ") + hipGetErrorString(e));
    if (dev->arrivals) (void)hipFree(dev->arrivals);
    if (dev->timer_stop) (void)hipEventDestroy(dev->timer_stop);
    if (dev->timer_start) (void)hipEventDestroy(dev->timer_start);
    if (dev->stream) (void)hipStreamDestroy(dev->stream);
    return nullptr;
  }
  char name[256] = {0};
  hipDeviceProp_t prop;
  const bool have_prop = hipGetDeviceProperties(&prop, index) == hipSuccess;
  if (hipDeviceGetName(name, sizeof name, index) == hipSuccess && name[0] != '\0')
    dev->name = name;
  else
    dev->name = "HIP device " + std::to_string(index);
  if (have_prop) dev->name += std::string(" (") + prop.gcnArchName + ")";
  dev->scratch = scratch_address(index);  // `index` is current (hipSetDevice above)
  dev->id = g_next_device.fetch_add(1);
  Registry& r = registry();
  std::lock_guard<std::mutex> lock(r.mu);
  r.devices[dev->id] = dev;
  return reinterpret_cast<AckDevice*>(uintptr_t(dev->id));
}

int32_t ack_close(AckDevice* handle) {
  std::shared_ptr<Device> dev;
  if (int32_t rc = lookup_device(handle, &dev)) return rc;
  {
    std::lock_guard<std::mutex> lock(dev->mu);
    if (dev->closed) {
      set_error("device " + std::to_string(dev->id) + " is closed");
      return ACK_ERR_CLOSED;
    }
    if (!dev->buffers.empty()) {
      set_error("close refused: " + std::to_string(dev->buffers.size()) +
                " buffer(s) still allocated on this device");
      return ACK_ERR_LIVE_BUFFERS;
    }
    dev->closed = true;
    if (!dev->poisoned && hipSetDevice(dev->hip_device) == hipSuccess) {
      hipError_t e = hipStreamSynchronize(dev->stream);
      if (e != hipSuccess)
        set_error(std::string("close waited for enqueued work and it failed: ") +
                  hipGetErrorString(e));
      if (dev->workspace) (void)hipFree(dev->workspace);
      if (dev->arrivals) (void)hipFree(dev->arrivals);
      (void)hipEventDestroy(dev->timer_start);
      (void)hipEventDestroy(dev->timer_stop);
      (void)hipStreamDestroy(dev->stream);
    }
    dev->workspace = nullptr;
    dev->arrivals = nullptr;
  }
  Registry& r = registry();
  std::lock_guard<std::mutex> lock(r.mu);
  r.devices.erase(dev->id);
  return ACK_OK;
}

int32_t ack_device_name(const AckDevice* handle, char* out, size_t len) {
  if (out == nullptr || len == 0) return ACK_ERR_NULL;
  std::shared_ptr<Device> dev;
  if (int32_t rc = lookup_device(handle, &dev)) return rc;
  std::lock_guard<std::mutex> lock(dev->mu);
  if (dev->closed) {
    set_error("device " + std::to_string(dev->id) + " is closed");
    return ACK_ERR_CLOSED;
  }
  const size_t n = dev->name.size() < len - 1 ? dev->name.size() : len - 1;
  std::memcpy(out, dev->name.data(), n);
  out[n] = '\0';
  return ACK_OK;
}

// FNV-1a over a byte stream (the reference's identity hash, ffi.rs:1419).
static uint64_t fnv1a(uint64_t h, const void* data, size_t len) {
  const unsigned char* p = static_cast<const unsigned char*>(data);
  for (size_t i = 0; i < len; ++i) {
    h ^= p[i];
    h *= 0x00000100000001b3ull;
  }
  return h;
}
constexpr uint64_t kFnvBasis = 0xcbf29ce484222325ull;
// The kernel sources' hash, from the build (build.py); 0 in a build without it.
#ifndef ACK_SHADERS_ID
#define ACK_SHADERS_ID 0ull
#endif
static_assert(sizeof(AckAbiInfo) == 96, "the layout of ffi.rs AckAbiInfo");
static_assert(sizeof(AckDeviceInfo) == 616 && offsetof(AckDeviceInfo, identity) == 160,
              "the layout of ffi.rs AckDeviceInfo");
constexpr uint32_t kAbiLayoutVersion = 14;  // the AckAbiInfo layout's ABI version
constexpr uint32_t kDeviceInfoVersion = 1;

int32_t ack_abi_info(AckAbiInfo* out, size_t size) {
  if (out == nullptr) return ACK_ERR_NULL;
  if (size < sizeof(AckAbiInfo)) {
    set_error("AckAbiInfo of " + std::to_string(size) + " bytes is smaller than this library's " +
              std::to_string(sizeof(AckAbiInfo)));
    return ACK_ERR_ABI;
  }
  AckAbiInfo info;
  std::memset(&info, 0, sizeof info);  // no operator family, schema or capability: 0 (absent)
  info.size = sizeof(AckAbiInfo);
  info.version = kAbiLayoutVersion;
  info.shaders = ACK_SHADERS_ID;
  const char kName[] = "libackvq vq4/v1 gfx950";
  const uint64_t shaders = info.shaders;
  info.build = fnv1a(fnv1a(kFnvBasis, kName, sizeof kName - 1), &shaders, sizeof shaders);
  std::memcpy(out, &info, sizeof info);
  return ACK_OK;
}

int32_t ack_device_info(const AckDevice* handle, AckDeviceInfo* out, size_t size) {
  if (out == nullptr) return ACK_ERR_NULL;
  if (size < sizeof(AckDeviceInfo)) {
    set_error("AckDeviceInfo of " + std::to_string(size) + " bytes is smaller than this library's " +
              std::to_string(sizeof(AckDeviceInfo)));
    return ACK_ERR_ABI;
  }
  std::shared_ptr<Device> dev;
  std::unique_lock<std::mutex> lock;
  if (int32_t rc = enter(handle, &dev, &lock, false)) return rc;
  hipDeviceProp_t prop;
  hipError_t e = hipGetDeviceProperties(&prop, dev->hip_device);
  int chip = 0, wall_khz = 0, runtime = 0, driver = 0;
  hipUUID uuid;
  std::memset(&uuid, 0, sizeof uuid);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&chip, hipDeviceAttributePciChipId, dev->hip_device);
  if (e == hipSuccess)
    e = hipDeviceGetAttribute(&wall_khz, hipDeviceAttributeWallClockRate, dev->hip_device);
  if (e == hipSuccess) e = hipRuntimeGetVersion(&runtime);
  if (e == hipSuccess) e = hipDriverGetVersion(&driver);
  if (e == hipSuccess) e = hipDeviceGetUuid(&uuid, dev->hip_device);
  if (e != hipSuccess) return hip_failure(*dev, "device info", e, false);
  AckDeviceInfo info;
  std::memset(&info, 0, sizeof info);
  info.size = sizeof(AckDeviceInfo);
  info.version = kDeviceInfoVersion;
  // HIP's version number is major * 10^7 + minor * 10^5 + patch
  const uint32_t major = uint32_t(runtime / 10000000), minor = uint32_t(runtime / 100000 % 100),
                 patch = uint32_t(runtime % 100000);
  info.api_version = (major << 22) | ((minor & 0x3FFu) << 12) | (patch & 0xFFFu);
  info.driver_version_raw = uint32_t(driver);
  info.vendor_id = 0x1002;  // AMD
  info.device_id = uint32_t(chip);
  info.device_type = 2;  // discrete GPU
  std::memcpy(info.device_uuid, uuid.bytes, 16);
  // cooperative matrix (1), bf16 type (2), bf16 dot product (4), bf16 matrix
  // (8), bf16 16x16x16 (32), int16 (64), fp16 (128), fp16 16x16x16 (256)
  info.features = 1u | 2u | 4u | 8u | 32u | 64u | 128u | 256u;
  info.subgroup_size = uint32_t(prop.warpSize);
  info.timestamp_valid_bits = 64;
  info.timestamp_period_ns = wall_khz > 0 ? float(1e6 / wall_khz) : 0.0f;
  info.max_push_constant_bytes = 4096;  // kernel argument space
  info.device_local_bytes = uint64_t(prop.totalGlobalMem);
  info.max_storage_buffer_bytes = uint64_t(prop.totalGlobalMem);
  info.max_workgroup_invocations = uint32_t(prop.maxThreadsPerBlock);
  for (int i = 0; i < 3; ++i) {
    info.max_workgroup_count[i] = uint32_t(prop.maxGridSize[i]);
    info.max_workgroup_size[i] = uint32_t(prop.maxThreadsDim[i]);
  }
  const uint64_t shaders = ACK_SHADERS_ID;
  info.identity = fnv1a(fnv1a(kFnvBasis, reinterpret_cast<const char*>(&info) + 8, 152), &shaders,
                        sizeof shaders);
  std::snprintf(info.device_name, sizeof info.device_name, "%s", dev->name.c_str());
  std::snprintf(info.driver_name, sizeof info.driver_name, "HIP (ROCm)");
  std::snprintf(info.driver_info, sizeof info.driver_info, "HIP runtime %d, driver %d, %s", runtime,
                driver, prop.gcnArchName);
  std::memcpy(out, &info, sizeof info);
  return ACK_OK;
}

int32_t ack_last_error(char* out, size_t len) {
  if (out == nullptr || len == 0) return ACK_ERR_NULL;
  const size_t n = t_last_error.size() < len - 1 ? t_last_error.size() : len - 1;
  std::memcpy(out, t_last_error.data(), n);
  out[n] = '\0';
  return ACK_OK;
}

AckBuffer* ack_buffer_alloc(const AckDevice* handle, uint64_t bytes) {
  if (bytes == 0) {
    set_error("zero-byte buffer");
    return nullptr;
  }
  std::shared_ptr<Device> dev;
  std::unique_lock<std::mutex> lock;
  if (enter(handle, &dev, &lock)) return nullptr;
  if (dev->next_buffer == UINT32_MAX) {
    set_error("buffer handle space exhausted on this device; close and reopen");
    return nullptr;
  }
  void* ptr = nullptr;
  hipError_t e = hipMalloc(&ptr, bytes);
  if (e != hipSuccess) {
    set_error(std::string("buffer allocation of ") + std::to_string(bytes) +
              " bytes: " + hipGetErrorString(e));
    (void)hipGetLastError();
    return nullptr;
  }
  const uint32_t seq = dev->next_buffer++;
  BufferRec rec;
  rec.ptr = ptr;
  rec.bytes = bytes;
  rec.id = buffer_handle(dev->id, seq);
  dev->buffers[seq] = rec;
  return reinterpret_cast<AckBuffer*>(uintptr_t(rec.id));
}

int32_t ack_buffer_free(const AckDevice* handle, AckBuffer* buf) {
  std::shared_ptr<Device> dev;
  std::unique_lock<std::mutex> lock;
  if (int32_t rc = enter(handle, &dev, &lock, false)) return rc;
  BufferRec* rec = nullptr;
  if (int32_t rc = lookup_buffer(*dev, buf, &rec)) return rc;
  const uint32_t seq = uint32_t(uint64_t(reinterpret_cast<uintptr_t>(buf)) & 0xffffffffu);
  void* ptr = rec->ptr;
  dev->buffers.erase(seq);
  if (dev->poisoned) {
    set_error("buffer leaked, not freed: device poisoned by an earlier ambiguous operation");
    return ACK_ERR_POISONED;
  }
  // Work enqueued earlier may still read the allocation: hipFree waits for
  // the device, which keeps the free safe without a flush of its own.
  hipError_t e = hipFree(ptr);
  if (e != hipSuccess) return hip_failure(*dev, "buffer free", e, true);
  return ACK_OK;
}

int32_t ack_upload(const AckDevice* handle, const AckBuffer* buf, const uint8_t* data, size_t len) {
  if (data == nullptr) return ACK_ERR_NULL;
  std::shared_ptr<Device> dev;
  std::unique_lock<std::mutex> lock;
  if (int32_t rc = enter(handle, &dev, &lock)) return rc;
  BufferRec* rec = nullptr;
  if (int32_t rc = lookup_buffer(*dev, buf, &rec)) return rc;
  if (uint64_t(len) != rec->bytes) {
    set_error("upload of " + std::to_string(len) + " bytes into a " + std::to_string(rec->bytes) +
              "-byte buffer");
    return ACK_ERR_SIZE;
  }
  hipError_t e = hipMemcpyAsync(rec->ptr, data, len, hipMemcpyHostToDevice, dev->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(dev->stream);
  if (e != hipSuccess) return hip_failure(*dev, "upload", e, true);
  return ACK_OK;
}

int32_t ack_download(const AckDevice* handle, const AckBuffer* buf, uint8_t* data, size_t len) {
  if (data == nullptr) return ACK_ERR_NULL;
  std::shared_ptr<Device> dev;
  std::unique_lock<std::mutex> lock;
  if (int32_t rc = enter(handle, &dev, &lock)) return rc;
  BufferRec* rec = nullptr;
  if (int32_t rc = lookup_buffer(*dev, buf, &rec)) return rc;
  if (uint64_t(len) != rec->bytes) {
    set_error("download of " + std::to_string(len) + " bytes from a " +
              std::to_string(rec->bytes) + "-byte buffer");
    return ACK_ERR_SIZE;
  }
  hipError_t e = hipMemcpyAsync(data, rec->ptr, len, hipMemcpyDeviceToHost, dev->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(dev->stream);
  if (e != hipSuccess) return hip_failure(*dev, "download", e, true);
  return ACK_OK;
}

int32_t ack_buffer_copy(const AckDevice* handle, const AckBuffer* dst, uint64_t dst_offset,
                        const AckBuffer* src, uint64_t src_offset, uint64_t bytes) {
  std::shared_ptr<Device> dev;
  std::unique_lock<std::mutex> lock;
  if (int32_t rc = enter(handle, &dev, &lock)) return rc;
  BufferRec* d = nullptr;
  BufferRec* s = nullptr;
  if (int32_t rc = lookup_buffer(*dev, dst, &d)) return rc;
  if (int32_t rc = lookup_buffer(*dev, src, &s)) return rc;
  if (dst_offset > d->bytes || bytes > d->bytes - dst_offset || src_offset > s->bytes ||
      bytes > s->bytes - src_offset) {
    set_error("copy of " + std::to_string(bytes) + " bytes outside a buffer");
    return ACK_ERR_SIZE;
  }
  if (d->id == s->id && dst_offset < src_offset + bytes && src_offset < dst_offset + bytes) {
    set_error("copy ranges overlap within one buffer");
    return ACK_ERR_SHAPE;
  }
  if (bytes == 0) return ACK_OK;
  hipError_t e = hipMemcpyAsync(static_cast<char*>(d->ptr) + dst_offset,
                                static_cast<const char*>(s->ptr) + src_offset, bytes,
                                hipMemcpyDeviceToDevice, dev->stream);
  if (e != hipSuccess) return hip_failure(*dev, "copy", e, true);
  return ACK_OK;
}

int32_t ack_vq_sum_squares(const AckDevice* handle, const AckBuffer* x, uint64_t count,
                           const AckBuffer* out) {
  std::shared_ptr<Device> dev;
  std::unique_lock<std::mutex> lock;
  if (int32_t rc = enter(handle, &dev, &lock)) return rc;
  BufferRec* xb = nullptr;
  BufferRec* ob = nullptr;
  if (int32_t rc = lookup_buffer(*dev, x, &xb)) return rc;
  if (int32_t rc = lookup_buffer(*dev, out, &ob)) return rc;
  if (count > xb->bytes / sizeof(float) || ob->bytes < sizeof(double)) {
    set_error("sum of squares: " + std::to_string(count) + " values or the 8-byte result "
              "do not fit their buffers");
    return ACK_ERR_SIZE;
  }
  if (int32_t rc = ensure_workspace(*dev, 256 * sizeof(double))) return rc;
  hipError_t e = ackvq::launch_sum_squares(dev->stream, static_cast<const float*>(xb->ptr), count,
                                           static_cast<double*>(dev->workspace),
                                           static_cast<double*>(ob->ptr));
  if (e != hipSuccess) return hip_failure(*dev, "sum of squares", e, true);
  return ACK_OK;
}

int32_t ack_vq_scale(const AckDevice* handle, const AckBuffer* x, uint64_t count, float factor) {
  std::shared_ptr<Device> dev;
  std::unique_lock<std::mutex> lock;
  if (int32_t rc = enter(handle, &dev, &lock)) return rc;
  BufferRec* xb = nullptr;
  if (int32_t rc = lookup_buffer(*dev, x, &xb)) return rc;
  if (count > xb->bytes / sizeof(float)) {
    set_error("scale: " + std::to_string(count) + " values do not fit the buffer");
    return ACK_ERR_SIZE;
  }
  if (count == 0) return ACK_OK;
  hipError_t e = ackvq::launch_scale(dev->stream, static_cast<float*>(xb->ptr), count, factor);
  if (e != hipSuccess) return hip_failure(*dev, "scale", e, true);
  return ACK_OK;
}

int32_t ack_sync(const AckDevice* handle) {
  std::shared_ptr<Device> dev;
  std::unique_lock<std::mutex> lock;
  if (int32_t rc = enter(handle, &dev, &lock)) return rc;
  hipError_t e = hipStreamSynchronize(dev->stream);
  if (e != hipSuccess) return hip_failure(*dev, "sync", e, true);
  return ACK_OK;
}

int32_t ack_stream_timer(const AckDevice* handle, uint32_t phase, float* ms_out) {
  std::shared_ptr<Device> dev;
  std::unique_lock<std::mutex> lock;
  if (int32_t rc = enter(handle, &dev, &lock)) return rc;
  if (phase == 0) {
    hipError_t e = hipEventRecord(dev->timer_start, dev->stream);
    if (e != hipSuccess) return hip_failure(*dev, "timer start", e, false);
    return ACK_OK;
  }
  if (phase != 1 || ms_out == nullptr) {
    set_error("ack_stream_timer: phase must be 0 (start) or 1 (stop) with an output");
    return ACK_ERR_SHAPE;
  }
  hipError_t e = hipEventRecord(dev->timer_stop, dev->stream);
  if (e == hipSuccess) e = hipEventSynchronize(dev->timer_stop);
  if (e == hipSuccess) e = hipEventElapsedTime(ms_out, dev->timer_start, dev->timer_stop);
  if (e != hipSuccess) return hip_failure(*dev, "timer stop", e, true);
  return ACK_OK;
}

int32_t ack_vq_set_policy(const AckDevice* handle, uint32_t policy) {
  if (policy > 2) {
    set_error("ack_vq_set_policy: policy must be 0 (automatic), 1 (general) or 2 (any size)");
    return ACK_ERR_SHAPE;
  }
  std::shared_ptr<Device> dev;
  std::unique_lock<std::mutex> lock;
  if (int32_t rc = enter(handle, &dev, &lock)) return rc;
  dev->policy = policy;
  return ACK_OK;
}

int32_t ack_vq_plan_query(const uint8_t* plan, size_t plan_len, uint32_t bounds,
                          uint64_t* required_bytes6, uint32_t* work_items, uint32_t* dispatch3) {
  if (bounds > 1) {
    set_error("vq: bounds must be 0 (library) or 1 (reference)");
    return ACK_ERR_SHAPE;
  }
  ackvq::Plan p;
  if (int32_t rc = parse_plan(plan, plan_len, ackvq::Bounds(bounds), &p)) return rc;
  if (required_bytes6)
    for (int i = 0; i < 6; ++i) required_bytes6[i] = p.required_bytes[i];
  if (work_items) *work_items = p.work_items;
  if (dispatch3)
    for (int i = 0; i < 3; ++i) dispatch3[i] = p.dispatch[i];
  return ACK_OK;
}

int32_t ack_vq_plan_check_buffers(const uint8_t* plan, size_t plan_len,
                                  const uint64_t* capacities6, const uint64_t* ids6) {
  if (capacities6 == nullptr || ids6 == nullptr) return ACK_ERR_NULL;
  ackvq::Plan p;
  if (int32_t rc = parse_plan(plan, plan_len, ackvq::Bounds::Library, &p)) return rc;
  int slot = 0;
  ackvq::PlanError e = ackvq::validate_buffers(p, capacities6, ids6, &slot);
  if (e != ackvq::PlanError::None) {
    set_error("vq: plan refused: " + ackvq::plan_error_name(e, slot));
    return plan_code(e);
  }
  return ACK_OK;
}

int32_t ack_vq_batch_path_name(const uint8_t* plan, size_t plan_len, uint32_t count, char* out,
                               size_t len) {
  if (out == nullptr || len == 0) return ACK_ERR_NULL;
  if (count == 0) {
    set_error("vq path name: count must be at least 1");
    return ACK_ERR_SHAPE;
  }
  ackvq::Plan p;
  if (int32_t rc = parse_plan(plan, plan_len, ackvq::Bounds::Library, &p)) return rc;
  const char* name = "encode";
  if (p.op == ackvq::Op::Decode) name = "decode";
  if (p.op == ackvq::Op::AdamW) name = "adamw";
  if (p.op == ackvq::Op::Matmul)
    name = ackvq::matmul_path_name(
        ackvq::choose_matmul_path(p.m(), p.n(), p.k(), p.group(), p.flags(), count, 0));
  const size_t n = std::strlen(name) < len - 1 ? std::strlen(name) : len - 1;
  std::memcpy(out, name, n);
  out[n] = '\0';
  return ACK_OK;
}

int32_t ack_vq_path_name(const uint8_t* plan, size_t plan_len, char* out, size_t len) {
  return ack_vq_batch_path_name(plan, plan_len, 1, out, len);
}

int32_t ack_vq_host_encode(const float* values, uint64_t m, const float* book, uint32_t group,
                           uint32_t* codes_out) {
  if (values == nullptr || book == nullptr || codes_out == nullptr) return ACK_ERR_NULL;
  if (!(group == 8 || group == 16 || group == 32)) {
    set_error("vq host encode: group must be 8, 16 or 32");
    return ACK_ERR_SHAPE;
  }
  if (m == 0 || m > ackvq::kMaxValues) {
    set_error("vq host encode: element count must be in 1..2^28");
    return ACK_ERR_SIZE;
  }
  ackvq::host_encode64(values, m, book, group, codes_out);
  return ACK_OK;
}

int32_t ack_vq_host_fit_codebook(const float* values, uint64_t m, uint32_t group,
                                 uint32_t iterations, uint32_t sample_vectors, const float* init,
                                 float* book_out) {
  if (values == nullptr || book_out == nullptr) return ACK_ERR_NULL;
  if (!(group == 8 || group == 16 || group == 32)) {
    set_error("vq host fit: group must be 8, 16 or 32");
    return ACK_ERR_SHAPE;
  }
  if (m < group || m > ackvq::kMaxValues) {
    set_error("codebook calibration needs at least one complete vector");
    return ACK_ERR_SIZE;
  }
  if (iterations > 32 || sample_vectors < 16 || sample_vectors > 65536) {
    set_error("vq host fit: iterations must be in 0..32 and sample_vectors in 16..65536");
    return ACK_ERR_SHAPE;
  }
  ackvq::host_fit_codebook(values, m, group, iterations, sample_vectors, init, book_out);
  return ACK_OK;
}

int32_t ack_vq_matmul_dense(const AckDevice* handle, const AckBuffer* x, const AckBuffer* b_codes,
                            const AckBuffer* b_book, const AckBuffer* out, const AckBuffer* status,
                            const uint8_t* plan_bytes, size_t plan_len) {
  ackvq::Plan plan;
  if (int32_t rc = parse_plan(plan_bytes, plan_len, ackvq::Bounds::Library, &plan)) return rc;
  if (plan.op != ackvq::Op::Matmul) {
    set_error("vq dense matmul: plan op must be 2 (matmul)");
    return ACK_ERR_SHAPE;
  }
  std::shared_ptr<Device> dev;
  std::unique_lock<std::mutex> lock;
  if (int32_t rc = enter(handle, &dev, &lock)) return rc;
  // Slot 0 holds the dense m x k activations; slot 1 (A's codebook in op 2)
  // is not read and aliases slot 0. The output and status rules are op 2's.
  const AckBuffer* slots[6] = {x, x, b_codes, b_book, out, status};
  BufferRec* bufs[6];
  uint64_t capacities[6], ids[6];
  for (int i = 0; i < 6; ++i) {
    if (int32_t rc = lookup_buffer(*dev, slots[i], &bufs[i])) return rc;
    capacities[i] = bufs[i]->bytes;
    ids[i] = bufs[i]->id;
  }
  const uint32_t m = plan.m(), n = plan.n(), k = plan.k(), g = plan.group();
  ackvq::Plan dense = plan;
  dense.required_bytes[0] = uint64_t(m) * k * 4;
  dense.required_bytes[1] = 0;
  int slot = 0;
  ackvq::PlanError e = ackvq::validate_buffers(dense, capacities, ids, &slot);
  if (e != ackvq::PlanError::None) {
    set_error("vq dense matmul: plan refused: " + ackvq::plan_error_name(e, slot));
    return plan_code(e);
  }
  ackvq::Operands o;
  o.arrivals = dev->arrivals;
  for (int i = 0; i < 4; ++i) o.in[i] = bufs[i]->ptr;
  o.out = bufs[4]->ptr;
  o.status = static_cast<uint32_t*>(bufs[5]->ptr);
  const ackvq::MatmulPath path =
      ackvq::choose_dense_path(m, n, k, g, plan.flags(), 1, dev->policy);
  const size_t ws = ackvq::dense_workspace_bytes(path, m, n, k, g, plan.flags(), 1);
  if (int32_t rc = ensure_workspace(*dev, ws)) return rc;
  hipError_t he = ackvq::launch_matmul_dense(dev->stream, o, m, n, k, g, plan.flags(), path,
                                             dev->workspace, dev->workspace_bytes);
  if (he != hipSuccess) return hip_failure(*dev, "vq dense matmul: kernel launch refused", he, false);
  return ACK_OK;
}

int32_t ack_vq_dense_path_name(const uint8_t* plan, size_t plan_len, char* out, size_t len) {
  if (out == nullptr || len == 0) return ACK_ERR_NULL;
  ackvq::Plan p;
  if (int32_t rc = parse_plan(plan, plan_len, ackvq::Bounds::Library, &p)) return rc;
  if (p.op != ackvq::Op::Matmul) {
    set_error("vq dense matmul: plan op must be 2 (matmul)");
    return ACK_ERR_SHAPE;
  }
  const char* name = ackvq::matmul_path_name(
      ackvq::choose_dense_path(p.m(), p.n(), p.k(), p.group(), p.flags(), 1, 0));
  const size_t n = std::strlen(name) < len - 1 ? std::strlen(name) : len - 1;
  std::memcpy(out, name, n);
  out[n] = '\0';
  return ACK_OK;
}

int32_t ack_vq_fit_codebook(const AckDevice* handle, const AckBuffer* values,
                            const AckBuffer* init, const AckBuffer* book_out,
                            const AckBuffer* status, uint64_t m, uint32_t group,
                            uint32_t iterations, uint32_t sample_vectors) {
  if (!(group == 8 || group == 16 || group == 32)) {
    set_error("vq fit: group must be 8, 16 or 32");
    return ACK_ERR_SHAPE;
  }
  if (m < group || m > ackvq::kMaxValues) {
    set_error("codebook calibration needs at least one complete vector");
    return ACK_ERR_SIZE;
  }
  if (iterations > 32 || sample_vectors < 16 || sample_vectors > 65536) {
    set_error("vq fit: iterations must be in 0..32 and sample_vectors in 16..65536");
    return ACK_ERR_SHAPE;
  }
  std::shared_ptr<Device> dev;
  std::unique_lock<std::mutex> lock;
  if (int32_t rc = enter(handle, &dev, &lock)) return rc;
  const AckBuffer* slots[4] = {values, init, book_out, status};
  BufferRec* bufs[4] = {nullptr, nullptr, nullptr, nullptr};
  for (int i = 0; i < 4; ++i) {
    if (i == 1 && init == nullptr) continue;
    if (int32_t rc = lookup_buffer(*dev, slots[i], &bufs[i])) return rc;
  }
  const uint64_t need[4] = {m * 4, uint64_t(16) * group * 4, uint64_t(16) * group * 4, 4};
  for (int i = 0; i < 4; ++i) {
    if (bufs[i] != nullptr && bufs[i]->bytes < need[i]) {
      set_error("vq fit: buffer " + std::to_string(i) + " is too small");
      return ACK_ERR_SIZE;
    }
  }
  for (int w = 2; w < 4; ++w)
    for (int i = 0; i < w; ++i)
      if (bufs[i] != nullptr && bufs[w]->id == bufs[i]->id) {
        set_error("vq fit: write slot " + std::to_string(w) + " aliases slot " +
                  std::to_string(i));
        return ACK_ERR_SHAPE;
      }
  const uint64_t complete = m / group;
  const uint32_t count = uint32_t(complete < sample_vectors ? complete : sample_vectors);
  const size_t sample_bytes = round_up(size_t(count) * group * 4);
  const size_t idx_bytes = round_up(count);
  const size_t gap_bytes = round_up(size_t(count) * 17 * 8);
  const size_t book64_bytes = round_up(size_t(16) * group * 8);
  if (int32_t rc = ensure_workspace(*dev, sample_bytes + idx_bytes + 256 + gap_bytes + book64_bytes))
    return rc;
  char* ws = static_cast<char*>(dev->workspace);
  ackvq::FitArgs fit;
  fit.sample = reinterpret_cast<float*>(ws);
  fit.idx = reinterpret_cast<uint8_t*>(ws + sample_bytes);
  fit.flags = reinterpret_cast<uint32_t*>(ws + sample_bytes + idx_bytes);
  fit.gaps = reinterpret_cast<double*>(ws + sample_bytes + idx_bytes + 256);
  fit.book64 = reinterpret_cast<double*>(ws + sample_bytes + idx_bytes + 256 + gap_bytes);
  fit.book = static_cast<float*>(bufs[2]->ptr);
  fit.count = count;
  fit.complete = complete;
  fit.status = static_cast<uint32_t*>(bufs[3]->ptr);
  ackvq::FitWhole whole;
  whole.values = static_cast<const float*>(bufs[0]->ptr);
  const float* init_book = bufs[1] ? static_cast<const float*>(bufs[1]->ptr) : nullptr;
  hipError_t e = ackvq::launch_fit_sample_dense(dev->stream, whole.values, group, fit, init_book);
  if (e == hipSuccess)
    e = ackvq::launch_fit(dev->stream, fit, group, 1, iterations, init_book, whole, true);
  if (e != hipSuccess) return hip_failure(*dev, "vq fit: launch", e, true);
  return ACK_OK;
}

int32_t ack_vq_adamw_step(const AckDevice* handle, const AckBuffer* b0, const AckBuffer* b1,
                          const AckBuffer* b2, const AckBuffer* out_codes,
                          const AckBuffer* out_books, const AckBuffer* changed,
                          const AckBuffer* status, const uint8_t* plan_bytes, size_t plan_len,
                          uint32_t iterations, uint32_t sample_vectors) {
  ackvq::Plan plan;
  if (int32_t rc = parse_plan(plan_bytes, plan_len, ackvq::Bounds::Library, &plan)) return rc;
  if (plan.op != ackvq::Op::AdamW) {
    set_error("vq adamw step: plan op must be 3 (AdamW)");
    return ACK_ERR_SHAPE;
  }
  if (iterations > 32 || sample_vectors < 16 || sample_vectors > 65536) {
    set_error("vq adamw step: iterations must be in 0..32 and sample_vectors in 16..65536");
    return ACK_ERR_SHAPE;
  }
  const uint32_t m = plan.m(), g = plan.group();
  if (m < g) {
    set_error("codebook calibration needs at least one complete vector");
    return ACK_ERR_SIZE;
  }
  std::shared_ptr<Device> dev;
  std::unique_lock<std::mutex> lock;
  if (int32_t rc = enter(handle, &dev, &lock)) return rc;
  const AckBuffer* slots[7] = {b0, b1, b2, out_codes, out_books, changed, status};
  BufferRec* bufs[7];
  for (int i = 0; i < 7; ++i)
    if (int32_t rc = lookup_buffer(*dev, slots[i], &bufs[i])) return rc;
  const uint64_t words = ackvq::packed_words(m, g);
  const uint64_t need[7] = {plan.required_bytes[0], plan.required_bytes[1], plan.required_bytes[2],
                            3 * words * 4, 3ull * 16 * g * 4, 4, 4};
  for (int i = 0; i < 7; ++i) {
    if (bufs[i]->bytes < need[i]) {
      set_error("vq adamw step: buffer " + std::to_string(i) + " is too small");
      return ACK_ERR_SIZE;
    }
  }
  for (int w = 3; w < 7; ++w)
    for (int i = 0; i < w; ++i)
      if (bufs[w]->id == bufs[i]->id) {
        set_error("vq adamw step: write slot " + std::to_string(w) + " aliases slot " +
                  std::to_string(i));
        return ACK_ERR_SHAPE;
      }

  ackvq::AdamwInputs in;
  in.codes4 = static_cast<const uint32_t*>(bufs[0]->ptr);
  in.books4 = static_cast<const float*>(bufs[1]->ptr);
  in.coeffs = static_cast<const float*>(bufs[2]->ptr);
  in.m = m;
  in.group = g;
  uint32_t* st = static_cast<uint32_t*>(bufs[6]->ptr);
  hipStream_t s = dev->stream;

  // fit_codebook's strided sample of complete vectors (vq.py:206-207), the
  // three fits on the device, then the encode pass; no host round trip.
  const uint64_t complete = m / g;
  const uint32_t count = uint32_t(complete < sample_vectors ? complete : sample_vectors);
  const size_t sample_bytes = round_up(size_t(3) * count * g * 4);
  const size_t idx_bytes = round_up(size_t(3) * count);
  const size_t gap_bytes = round_up(size_t(3) * count * 17 * 8);
  const size_t book64_bytes = round_up(size_t(3) * 16 * g * 8);
  if (int32_t rc = ensure_workspace(*dev, sample_bytes + idx_bytes + 256 + gap_bytes + book64_bytes))
    return rc;
  char* ws = static_cast<char*>(dev->workspace);
  ackvq::FitArgs fit;
  fit.sample = reinterpret_cast<float*>(ws);
  fit.idx = reinterpret_cast<uint8_t*>(ws + sample_bytes);
  fit.flags = reinterpret_cast<uint32_t*>(ws + sample_bytes + idx_bytes);
  fit.gaps = reinterpret_cast<double*>(ws + sample_bytes + idx_bytes + 256);
  fit.book64 = reinterpret_cast<double*>(ws + sample_bytes + idx_bytes + 256 + gap_bytes);
  fit.book = static_cast<float*>(bufs[4]->ptr);
  fit.count = count;
  fit.complete = complete;
  fit.status = st;
  ackvq::FitWhole whole;
  whole.adamw = &in;

  hipError_t e = ackvq::launch_adamw_gather(s, in, count, const_cast<float*>(fit.sample),
                                               static_cast<uint32_t*>(bufs[5]->ptr), st, fit.book,
                                               fit.flags);
  if (e == hipSuccess) e = ackvq::launch_fit(s, fit, g, 3, iterations, in.books4, whole, true);
  if (e == hipSuccess)
    e = ackvq::launch_adamw_encode(s, in, fit.book, static_cast<uint32_t*>(bufs[3]->ptr),
                                   static_cast<uint32_t*>(bufs[5]->ptr), st);
  if (e != hipSuccess) return hip_failure(*dev, "vq adamw step: launch", e, true);
  return ACK_OK;
}

}  // extern "C"
