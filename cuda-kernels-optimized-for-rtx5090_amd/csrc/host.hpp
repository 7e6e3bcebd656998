// Host-side helpers shared by the C-ABI launchers: return codes, device facts, a per-(device, stream) workspace and
// the tuning overrides used by parameter sweeps.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>
#include <map>
#include <mutex>
#include <utility>

namespace rw_host {

// Return codes of every launcher: 0 = success (also the no-op of an empty problem), -1 = invalid or unsupported
// argument, anything else = the hipError_t the runtime reported.
constexpr int kOk = 0;
constexpr int kInvalid = -1;

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Compute units of the current device, queried once per device.
inline int device_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    (void)hipGetLastError();
    return 256;
  }
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n > 0) return n;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) {
    (void)hipGetLastError();
    n = 256;
  }
  cache[dev].store(n, std::memory_order_relaxed);
  return n;
}

// A device buffer of at least `bytes` owned by the library for (current device, stream). Launches on one stream are
// ordered, so a buffer reused by consecutive launches on its stream is never read and written by two of them at once.
// It grows by reallocation (the runtime waits for work that may still use the old buffer) and lives until the process
// ends. Returns nullptr with *err set on failure.
// `purpose` keeps separate buffers for users that must not share one (a buffer whose contents carry over between
// launches); with `zeroed` a new buffer is cleared on `stream` before first use.
// The workspace table: (device, purpose, stream) -> (buffer, bytes).
struct WorkspaceTable {
  std::mutex mu;
  std::map<std::pair<std::pair<int, int>, hipStream_t>, std::pair<void*, size_t>> buffers;
};
inline WorkspaceTable& workspaces() {
  static WorkspaceTable table;
  return table;
}

inline void* stream_workspace(hipStream_t stream, size_t bytes, int* err, int purpose = 0, bool zeroed = false) {
  std::mutex& mu = workspaces().mu;
  auto& buffers = workspaces().buffers;
  *err = kOk;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    *err = (int)e;
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(mu);
  auto& slot = buffers[std::make_pair(std::make_pair(dev, purpose), stream)];
  if (slot.second >= bytes && slot.first) return slot.first;
  size_t want = bytes < (1u << 20) ? (1u << 20) : bytes;
  if (slot.first) {
    e = hipFree(slot.first);
    slot = {nullptr, 0};
    if (e != hipSuccess) {
      *err = (int)e;
      return nullptr;
    }
  }
  void* p = nullptr;
  e = hipMalloc(&p, want);
  if (e != hipSuccess) {
    *err = (int)e;
    return nullptr;
  }
  if (zeroed) {
    e = hipMemsetAsync(p, 0, want, stream);
    if (e != hipSuccess) {
      (void)hipFree(p);
      *err = (int)e;
      return nullptr;
    }
  }
  slot = {p, want};
  return p;
}

// Zeroes the current device's workspace for (purpose, stream), if one was allocated, on `stream`. Returns 0 or the
// hipError_t.
inline int clear_stream_workspace(hipStream_t stream, int purpose) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  std::lock_guard<std::mutex> lock(workspaces().mu);
  auto it = workspaces().buffers.find(std::make_pair(std::make_pair(dev, purpose), stream));
  if (it == workspaces().buffers.end() || !it->second.first) return kOk;
  return (int)hipMemsetAsync(it->second.first, 0, it->second.second, stream);
}

// Tuning overrides: slot i holds 0 (automatic choice) or a value the launcher uses instead of its own choice. They are
// process-wide and meant for parameter sweeps; the automatic choices are the tuned defaults.
constexpr int kTuneSlots = 16;
inline std::atomic<int>* tune_table() {
  static std::atomic<int> table[kTuneSlots];
  return table;
}
inline int tune_get(int slot) { return tune_table()[slot].load(std::memory_order_relaxed); }
inline int tune_set(int slot, int value) {
  if (slot < 0 || slot >= kTuneSlots) return kInvalid;
  tune_table()[slot].store(value, std::memory_order_relaxed);
  return kOk;
}

}  // namespace rw_host
