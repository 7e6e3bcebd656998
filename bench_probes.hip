// Bandwidth probes of the measurement (bench.py --ceiling and --probes): structurally different kernels that move a
// given number of bytes through HBM with no arithmetic, so that the row kernels' rates can be set against what a plain
// copy, read or write reaches on the same part at the same size. Not part of the reference's interface and not used
// by the ops; bench.py builds this file into its own library (_build/libbench_probes.so).
//
// Every kernel moves 16-byte vectors; `bytes` (a multiple of 16) is what is read and what is written (a copy reads
// `bytes` from x and writes `bytes` to y). Families (probe_run's `family`):
//   kStride  persistent grid of blocks_per_cu workgroups of 256 threads per CU; each lane loads `unroll` vectors, then
//            stores them, and the grid strides over the buffer (the access pattern of a 1R + 1W row kernel).
//   kXcd     kStride with an XCD-aware block order: the hardware deals workgroup b to XCD b % 8, and the logical block
//            is chosen so that each XCD walks one contiguous eighth of the buffer (the grid is a multiple of 8).
//   kOneShot one workgroup per `unroll` * 256 vectors, no loop: the hardware dispatcher spreads the work.
//   kSlab    persistent; each workgroup owns one contiguous slab and streams it with the next `unroll` vectors loaded
//            before the current ones are stored (registers double-buffered).
//   kLds     kStride whose loads go straight to LDS (global_load_lds_dwordx4, no VGPRs) and come back with ds_read
//            before the stores; each wave uses its own LDS region.
//   kRow     persistent row groups as the row kernels run them: a workgroup owns rows of 256 * `unroll` vectors, loads
//            the next row while it exchanges one word per wave through LDS across a barrier for the current one, and
//            then stores it: the row kernels' structure with the arithmetic taken out.
//   kRead    kStride without the stores: each lane folds its vectors into one word, written to sink[0] only when the
//            fold meets a value the measurement's data never produces (so the loads are kept).
//   kWrite   kStride without the loads: each lane stores a constant vector.
// Cache policies (load_policy, store_policy) are the memory instructions' cache-policy bits: 0 none, 1 sc0, 2 nt,
// 16 sc1, 17 sc0 sc1, 18 nt sc1, 19 sc0 nt sc1. kStride takes every pair of {0, 2, 17, 18, 19} (loads) and
// {0, 2, 17, 18, 19} (stores); the other families use nt for both (what the row kernels issue). The kStride, kXcd,
// kRead and kWrite kernels access memory through buffer resources whose range is the buffer, so a lane past the end
// reads zero and its store is dropped; the other families compare each index with the end.
#include <hip/hip_runtime.h>

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
constexpr int kThreads = 256;
constexpr int kLdsMaxUnroll = 8;

enum Family { kStride = 0, kXcd = 1, kOneShot = 2, kSlab = 3, kLds = 4, kRow = 5, kRead = 6, kWrite = 7 };

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, long long bytes) {
  // raw buffer (stride 0): num_records counts bytes; the third word is the gfx9 raw-buffer format
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

// byte offset of vector base + u * 256 (below 2^31 for buffers of at most 1 GiB)
__device__ __forceinline__ int offset(long long base, int u) { return (int)((base + (long long)u * kThreads) * 16); }

__device__ __forceinline__ long long xcd_block(long long b, long long grid) {
  // grid is a multiple of 8: XCD b % 8 gets the logical blocks [(b % 8) * grid / 8, (b % 8 + 1) * grid / 8)
  return (b % 8) * (grid / 8) + b / 8;
}

template <int U, int LP, int SP, bool XCD>
__global__ void __launch_bounds__(kThreads) copy_stride(const u32x4* __restrict__ x, u32x4* __restrict__ y,
                                                        long long n) {
  const __amdgpu_buffer_rsrc_t rx = rsrc(x, n * 16), ry = rsrc(y, n * 16);
  const long long grid = gridDim.x;
  const long long b = XCD ? xcd_block(blockIdx.x, grid) : (long long)blockIdx.x;
  const long long stride = grid * kThreads * U;
  for (long long base = b * kThreads * U + threadIdx.x; base < n; base += stride) {
    u32x4 r[U];
#pragma unroll
    for (int u = 0; u < U; ++u) r[u] = __builtin_amdgcn_raw_buffer_load_b128(rx, offset(base, u), 0, LP);
#pragma unroll
    for (int u = 0; u < U; ++u) __builtin_amdgcn_raw_buffer_store_b128(r[u], ry, offset(base, u), 0, SP);
  }
}

template <int U>
__global__ void __launch_bounds__(kThreads) copy_oneshot(const u32x4* __restrict__ x, u32x4* __restrict__ y,
                                                         long long n) {
  const long long base = (long long)blockIdx.x * kThreads * U + threadIdx.x;
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

template <int U>
__global__ void __launch_bounds__(kThreads) copy_slab(const u32x4* __restrict__ x, u32x4* __restrict__ y, long long n) {
  const long long per = (n + gridDim.x - 1) / gridDim.x;
  const long long s0 = (long long)blockIdx.x * per;
  const long long s1 = s0 + per < n ? s0 + per : n;
  u32x4 a[U], c[U];
  long long base = s0 + threadIdx.x;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const long long i = base + (long long)u * kThreads;
    a[u] = i < s1 ? __builtin_nontemporal_load(x + i) : (u32x4){0u, 0u, 0u, 0u};
  }
  while (base < s1) {
    const long long next = base + (long long)kThreads * U;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const long long i = next + (long long)u * kThreads;
      c[u] = i < s1 ? __builtin_nontemporal_load(x + i) : (u32x4){0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const long long i = base + (long long)u * kThreads;
      if (i < s1) __builtin_nontemporal_store(a[u], y + i);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) a[u] = c[u];
    base = next;
  }
}

template <int U>
__global__ void __launch_bounds__(kThreads) copy_lds(const u32x4* __restrict__ x, u32x4* __restrict__ y, long long n) {
  static_assert(U <= kLdsMaxUnroll, "LDS region");
  __shared__ u32x4 buf[kThreads * U];
  const int wave = threadIdx.x / 64;
  const int lane = threadIdx.x % 64;
  // this wave's region: U blocks of 64 vectors; global_load_lds writes lane l's vector at the block's base + 16 * l
  u32x4* mine = buf + wave * 64 * U;
  const long long stride = (long long)gridDim.x * kThreads * U;
  for (long long base = (long long)blockIdx.x * kThreads * U + threadIdx.x; base < n; base += stride) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const long long i = base + (long long)u * kThreads;
      if (i < n)
        __builtin_amdgcn_global_load_lds(x + i, (__attribute__((address_space(3))) void*)(mine + u * 64), 16, 0, 2);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's LDS writes have landed
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const long long i = base + (long long)u * kThreads;
      if (i < n) __builtin_nontemporal_store(mine[u * 64 + lane], y + i);
    }
  }
}

template <int U>
__global__ void __launch_bounds__(kThreads) copy_rows(const u32x4* __restrict__ x, u32x4* __restrict__ y,
                                                      long long n) {
  constexpr long long kRow = (long long)kThreads * U;  // vectors per row
  __shared__ unsigned slot[2][kThreads / 64];
  const long long rows = (n + kRow - 1) / kRow;
  u32x4 cur[U], nxt[U];
  long long row = blockIdx.x;
  auto load = [&](u32x4 (&r)[U], long long rw) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const long long i = rw * kRow + (long long)u * kThreads + threadIdx.x;
      r[u] = (rw < rows && i < n) ? __builtin_nontemporal_load(x + i) : (u32x4){0u, 0u, 0u, 0u};
    }
  };
  load(cur, row);
  for (int parity = 0; row < rows; row += gridDim.x, parity ^= 1) {
    load(nxt, row + gridDim.x);
    unsigned fold = 0;
#pragma unroll
    for (int u = 0; u < U; ++u) fold ^= cur[u].x ^ cur[u].w;
    fold = __builtin_amdgcn_readfirstlane(fold);
    if (threadIdx.x % 64 == 0) slot[parity][threadIdx.x / 64] = fold;
    __syncthreads();  // the row's exchange, in place of a reduction's; slots alternate so one barrier per row suffices
    unsigned all = 0;
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) all ^= slot[parity][w];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const long long i = row * kRow + (long long)u * kThreads + threadIdx.x;
      u32x4 v = cur[u];
      v.y ^= all == 0x9e3779b9u ? 1u : 0u;  // keeps the exchange live; the measurement's data never folds to this
      if (i < n) __builtin_nontemporal_store(v, y + i);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) cur[u] = nxt[u];
  }
}

template <int U>
__global__ void __launch_bounds__(kThreads) read_stride(const u32x4* __restrict__ x, unsigned* __restrict__ sink,
                                                        long long n) {
  const __amdgpu_buffer_rsrc_t rx = rsrc(x, n * 16);
  const long long stride = (long long)gridDim.x * kThreads * U;
  unsigned acc = 0;
  for (long long base = (long long)blockIdx.x * kThreads * U + threadIdx.x; base < n; base += stride) {
    u32x4 r[U];
#pragma unroll
    for (int u = 0; u < U; ++u) r[u] = __builtin_amdgcn_raw_buffer_load_b128(rx, offset(base, u), 0, 2);
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= r[u].x ^ r[u].y ^ r[u].z ^ r[u].w;
  }
  if (acc == 0x9e3779b9u) sink[0] = acc;
}

template <int U, int SP>
__global__ void __launch_bounds__(kThreads) write_stride(u32x4* __restrict__ y, long long n) {
  const __amdgpu_buffer_rsrc_t ry = rsrc(y, n * 16);
  const long long stride = (long long)gridDim.x * kThreads * U;
  const u32x4 v = {1u, 2u, 3u, (unsigned)blockIdx.x};
  for (long long base = (long long)blockIdx.x * kThreads * U + threadIdx.x; base < n; base += stride) {
#pragma unroll
    for (int u = 0; u < U; ++u) __builtin_amdgcn_raw_buffer_store_b128(v, ry, offset(base, u), 0, SP);
  }
}

int device_cus() {
  static int cached[64] = {};
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  if (dev >= 0 && dev < 64 && cached[dev]) return cached[dev];
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) return 256;
  if (dev >= 0 && dev < 64) cached[dev] = cus;
  return cus;
}

// A persistent grid: enough workgroups for the work, at most blocks_per_cu per CU, a multiple of 8 when it is full.
long long persistent_grid(long long n, long long per_block, int blocks_per_cu) {
  const long long need = (n + per_block - 1) / per_block;
  const long long full = (long long)device_cus() * blocks_per_cu / 8 * 8;
  return need < full ? need : full;
}

template <int U, int LP, bool XCD>
int launch_stride_sp(int sp, dim3 grid, const u32x4* x, u32x4* y, long long n, hipStream_t s) {
  switch (sp) {
    case 0: hipLaunchKernelGGL((copy_stride<U, LP, 0, XCD>), grid, dim3(kThreads), 0, s, x, y, n); return 0;
    case 2: hipLaunchKernelGGL((copy_stride<U, LP, 2, XCD>), grid, dim3(kThreads), 0, s, x, y, n); return 0;
    case 17: hipLaunchKernelGGL((copy_stride<U, LP, 17, XCD>), grid, dim3(kThreads), 0, s, x, y, n); return 0;
    case 18: hipLaunchKernelGGL((copy_stride<U, LP, 18, XCD>), grid, dim3(kThreads), 0, s, x, y, n); return 0;
    case 19: hipLaunchKernelGGL((copy_stride<U, LP, 19, XCD>), grid, dim3(kThreads), 0, s, x, y, n); return 0;
    default: return -1;
  }
}

template <int U, bool XCD>
int launch_stride(int lp, int sp, dim3 grid, const u32x4* x, u32x4* y, long long n, hipStream_t s) {
  switch (lp) {
    case 0: return launch_stride_sp<U, 0, XCD>(sp, grid, x, y, n, s);
    case 2: return launch_stride_sp<U, 2, XCD>(sp, grid, x, y, n, s);
    case 17: return launch_stride_sp<U, 17, XCD>(sp, grid, x, y, n, s);
    case 18: return launch_stride_sp<U, 18, XCD>(sp, grid, x, y, n, s);
    case 19: return launch_stride_sp<U, 19, XCD>(sp, grid, x, y, n, s);
    default: return -1;
  }
}

}  // namespace

// Launches one probe on `stream` (nothing for bytes == 0). Returns 0, -1 for arguments no probe takes (an unknown
// family, unroll or policy pair, bytes not a multiple of 16, negative or beyond 1 GiB, blocks_per_cu outside [1, 32], a null buffer the family
// uses), or the HIP error of the launch.
extern "C" int probe_run(int family, int unroll, int blocks_per_cu, int load_policy, int store_policy, const void* xv,
                         void* yv, unsigned* sink, long long bytes, hipStream_t stream) {
  if (bytes == 0) return 0;
  if (bytes < 0 || bytes % 16 || bytes > (1LL << 30) || blocks_per_cu < 1 || blocks_per_cu > 32) return -1;
  const bool reads = family != kWrite, writes = family != kRead;
  if ((reads && !xv) || (writes && !yv) || (family == kRead && !sink)) return -1;
  const bool nt_only = family != kStride;
  if (nt_only && ((reads && load_policy != 2) || (writes && store_policy != 2))) return -1;
  const long long n = bytes / 16;
  const u32x4* x = static_cast<const u32x4*>(xv);
  u32x4* y = static_cast<u32x4*>(yv);
  const dim3 grid((unsigned)persistent_grid(n, (long long)kThreads * unroll, blocks_per_cu));
  int rc = -1;
  switch (family) {
    case kStride:
    case kXcd: {
      const bool xcd = family == kXcd;
      dim3 g = grid;
      if (xcd) g.x = g.x < 8 ? 8 : g.x / 8 * 8;  // the block order needs a multiple of 8; the grid strides over the rest
      switch (unroll) {
        case 2: rc = xcd ? launch_stride<2, true>(load_policy, store_policy, g, x, y, n, stream)
                         : launch_stride<2, false>(load_policy, store_policy, g, x, y, n, stream); break;
        case 4: rc = xcd ? launch_stride<4, true>(load_policy, store_policy, g, x, y, n, stream)
                         : launch_stride<4, false>(load_policy, store_policy, g, x, y, n, stream); break;
        case 8: rc = xcd ? launch_stride<8, true>(load_policy, store_policy, g, x, y, n, stream)
                         : launch_stride<8, false>(load_policy, store_policy, g, x, y, n, stream); break;
        case 16: rc = xcd ? launch_stride<16, true>(load_policy, store_policy, g, x, y, n, stream)
                          : launch_stride<16, false>(load_policy, store_policy, g, x, y, n, stream); break;
        default: return -1;
      }
      break;
    }
    case kOneShot: {
      const dim3 all((unsigned)((n + (long long)kThreads * unroll - 1) / ((long long)kThreads * unroll)));
      switch (unroll) {
        case 4: hipLaunchKernelGGL(copy_oneshot<4>, all, dim3(kThreads), 0, stream, x, y, n); rc = 0; break;
        case 8: hipLaunchKernelGGL(copy_oneshot<8>, all, dim3(kThreads), 0, stream, x, y, n); rc = 0; break;
        case 16: hipLaunchKernelGGL(copy_oneshot<16>, all, dim3(kThreads), 0, stream, x, y, n); rc = 0; break;
        default: return -1;
      }
      break;
    }
    case kSlab:
      switch (unroll) {
        case 4: hipLaunchKernelGGL(copy_slab<4>, grid, dim3(kThreads), 0, stream, x, y, n); rc = 0; break;
        case 8: hipLaunchKernelGGL(copy_slab<8>, grid, dim3(kThreads), 0, stream, x, y, n); rc = 0; break;
        default: return -1;
      }
      break;
    case kLds:
      switch (unroll) {
        case 2: hipLaunchKernelGGL(copy_lds<2>, grid, dim3(kThreads), 0, stream, x, y, n); rc = 0; break;
        case 4: hipLaunchKernelGGL(copy_lds<4>, grid, dim3(kThreads), 0, stream, x, y, n); rc = 0; break;
        case 8: hipLaunchKernelGGL(copy_lds<8>, grid, dim3(kThreads), 0, stream, x, y, n); rc = 0; break;
        default: return -1;
      }
      break;
    case kRow:
      switch (unroll) {
        case 4: hipLaunchKernelGGL(copy_rows<4>, grid, dim3(kThreads), 0, stream, x, y, n); rc = 0; break;
        case 8: hipLaunchKernelGGL(copy_rows<8>, grid, dim3(kThreads), 0, stream, x, y, n); rc = 0; break;
        default: return -1;
      }
      break;
    case kRead:
      switch (unroll) {
        case 4: hipLaunchKernelGGL(read_stride<4>, grid, dim3(kThreads), 0, stream, x, sink, n); rc = 0; break;
        case 8: hipLaunchKernelGGL(read_stride<8>, grid, dim3(kThreads), 0, stream, x, sink, n); rc = 0; break;
        default: return -1;
      }
      break;
    case kWrite:
      switch (unroll) {
        case 4: hipLaunchKernelGGL((write_stride<4, 2>), grid, dim3(kThreads), 0, stream, y, n); rc = 0; break;
        case 8: hipLaunchKernelGGL((write_stride<8, 2>), grid, dim3(kThreads), 0, stream, y, n); rc = 0; break;
        default: return -1;
      }
      break;
    default: return -1;
  }
  if (rc) return rc;
  return (int)hipGetLastError();
}
