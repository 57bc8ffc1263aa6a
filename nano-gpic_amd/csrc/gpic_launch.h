// Host-side constants and helpers shared by the C-ABI entry points of libgpic_fp8.so.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

#include "../../include/gpic_fp8.h"

namespace gpic {

constexpr int kCastThreads = 256;                     // threads per workgroup of the streaming cast kernels
constexpr int kMaxParts = 1024;                       // at most this many partial maxima per amax pass
constexpr int kAmaxBlocks = 512;                      // workgroups of a flat amax pass
constexpr int kSwigluBlocks = 512;                    // workgroups of a SwiGLU pass
constexpr int kMaxCastBlocks = 8192;                  // workgroups of a streaming cast pass
constexpr int kCastTBlocks = 1024;                    // workgroups of a (persistent) transposing cast pass
constexpr int kSwigluCastTBlocks = 768;               // workgroups of the SwiGLU backward's recomputing cast (3 per CU)
constexpr size_t kCastWorkspaceBytes = 44 * 1024;     // partial maxima (4 KiB), the SwiGLU sigmoid table (24 KiB),
                                                      // the single-pass tagged partials (8 KiB), their epoch and
                                                      // counters (4 KiB + 4 KiB)

static inline bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

// The first statement of every entry point that launches kernels: clears the calling thread's last HIP error, so
// that the hipGetLastError() the entry point returns after its launches reports those launches and not an earlier,
// unrelated failure on the same thread.
static inline void status_scope() { (void)hipGetLastError(); }

// Device attributes the launches depend on, cached per device: each GPU of the process gets its own entry (the
// library may run on several), and a cache slot is written whole by whichever thread computes it first (all compute
// the same value). Devices past kMaxDevices are queried on every call.
constexpr int kMaxDevices = 64;
typedef std::atomic<int> DeviceCache[kMaxDevices];

static inline int current_device() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    dev = 0;
  }
  return dev;
}

// cache[dev] if set (>= 0), else compute(dev), stored for the next call.
template <class F>
static inline int per_device(DeviceCache &cache, F compute) {
  const int dev = current_device();
  if (dev < 0 || dev >= kMaxDevices) return compute(dev);
  int v = cache[dev].load(std::memory_order_relaxed);
  if (v < 0) {
    v = compute(dev);
    cache[dev].store(v, std::memory_order_relaxed);
  }
  return v;
}

// The device's compute units (256 on MI355X when the query fails).
static inline int device_cus(int dev) {
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) {
    (void)hipGetLastError();
    cus = 256;
  }
  return cus;
}

}  // namespace gpic
