// Bandwidth probes for the measurement (bench.py --ceiling): the practical HBM ceiling that the row kernels' rates are
// compared with. Not part of the reference's interface and not used by the ops.
//
// probe_copy: y = x over `bytes` (a multiple of 16), the access pattern of a 1R + 1W row kernel at its best: 16-byte
// non-temporal loads and stores, 4 vectors per lane in flight, a persistent grid of 8 workgroups of 256 threads per CU.
// probe_read: reads `bytes` (a multiple of 16) with 8 vectors per lane in flight and folds them into sink[0] (written
// only when the fold meets a value that the bench's data never produces, so the loads are kept).
#include <hip/hip_runtime.h>

#include "host.hpp"

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
constexpr int kThreads = 256;
constexpr int kBlocksPerCu = 8;

template <int U>
__global__ void __launch_bounds__(kThreads)
    probe_copy_kernel(const u32x4* __restrict__ x, u32x4* __restrict__ y, long long n) {
  const long long stride = (long long)gridDim.x * kThreads * U;
  for (long long base = (long long)blockIdx.x * kThreads * U + threadIdx.x; base < n; base += stride) {
    u32x4 r[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const long long i = base + (long long)u * kThreads;
      r[u] = i < n ? __builtin_nontemporal_load(x + i) : (u32x4){0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const long long i = base + (long long)u * kThreads;
      if (i < n) __builtin_nontemporal_store(r[u], y + i);
    }
  }
}

template <int U>
__global__ void __launch_bounds__(kThreads)
    probe_read_kernel(const u32x4* __restrict__ x, unsigned* __restrict__ sink, long long n) {
  const long long stride = (long long)gridDim.x * kThreads * U;
  unsigned acc = 0;
  for (long long base = (long long)blockIdx.x * kThreads * U + threadIdx.x; base < n; base += stride) {
    u32x4 r[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const long long i = base + (long long)u * kThreads;
      r[u] = i < n ? __builtin_nontemporal_load(x + i) : (u32x4){0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= r[u].x ^ r[u].y ^ r[u].z ^ r[u].w;
  }
  if (acc == 0x9e3779b9u) sink[0] = acc;
}

long long probe_grid(long long n, int per_block) {
  const long long need = (n + per_block - 1) / per_block;
  const long long full = (long long)rw_host::device_cus() * kBlocksPerCu;
  return need < full ? (need > 0 ? need : 1) : full;
}

}  // namespace

extern "C" int probe_copy(const void* x, void* y, long long bytes, hipStream_t stream) {
  if (bytes <= 0) return rw_host::kOk;
  if (bytes % 16 || !rw_host::aligned16(x) || !rw_host::aligned16(y)) return rw_host::kInvalid;
  const long long n = bytes / 16;
  hipLaunchKernelGGL(probe_copy_kernel<4>, dim3((unsigned)probe_grid(n, kThreads * 4)), dim3(kThreads), 0, stream,
                     (const u32x4*)x, (u32x4*)y, n);
  return (int)hipGetLastError();
}

extern "C" int probe_read(const void* x, long long bytes, unsigned* sink, hipStream_t stream) {
  if (bytes <= 0) return rw_host::kOk;
  if (bytes % 16 || !rw_host::aligned16(x) || !sink) return rw_host::kInvalid;
  const long long n = bytes / 16;
  hipLaunchKernelGGL(probe_read_kernel<8>, dim3((unsigned)probe_grid(n, kThreads * 8)), dim3(kThreads), 0, stream,
                     (const u32x4*)x, sink, n);
  return (int)hipGetLastError();
}
