// Host-side helpers shared by the C-ABI launchers: return codes, device facts and the tuning overrides used by
// parameter sweeps and tests. The libraries allocate no device memory.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>

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
