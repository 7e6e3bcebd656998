// Row-wise softmax over the last dim of x[rows, cols] for fp32 (dtype 0) and bf16 (dtype 1) rows, every value
// accumulated in fp32 and each output rounded once (round to nearest even for bf16), behind the reference's C-ABI
// `launch` (softmax/kernel.cu:520-527, softmax/seed.cu:68-81).
//
// Tiers, chosen by row length in 16-byte vectors (4 fp32 or 8 bf16 elements), for rows whose length is a multiple of
// the vector width and whose x and y are 16-byte aligned:
//  - row tier (rows up to 16 waves x 64 lanes x 8 vectors = 32768 fp32 / 65536 bf16 columns): a group of WAVES waves
//    holds one row in registers, NV 16-byte vectors per lane. A max and a sum of exp(x - max) are reduced over the
//    group (DPP inside each wave, one LDS slot per wave across waves) and y = exp(x - max) / sum is written from the
//    registers: one HBM read and one write per element. Workgroups are persistent: each walks the rows with a stride
//    of the grid and loads its next row while it reduces and stores the current one.
//  - co-resident tier (longer rows, up to 64 chunks of 16384 elements): one pass over x for any number of rows; see
//    softmax_coop.
//  - stream tier (longer rows still): one workgroup per row, two passes, no workspace; see softmax_stream.
//  - generic tier (any length or alignment): one workgroup per row, three scalar passes (max, sum, write).
// The library allocates no device memory: the co-resident tier exchanges its chunk pairs through a static device
// table whose entries carry a per-launch tag, so nothing has to be cleared between launches; launches recorded into a
// HIP graph take fresh tags at every replay (see softmax_coop).
// The normalisation multiplies by the fp32 reciprocal of the row sum (the reference divides, softmax/kernel.cu:240;
// the two differ by at most 1.5 ulp in fp32 and are within the 1e-5 relative tolerance of the fp64 oracle).
#include <climits>
#include <cmath>
#include <mutex>

#include "host.hpp"
#include "rowwise.hpp"

using namespace rw;

namespace {

constexpr int kMaxNv = 8;       // 16-byte vectors a lane holds per row (32 fp32 / 64 bf16 values)
constexpr int kMaxWaves = 16;   // waves that share a row in the row tier (1024 threads)

template <int NV>
struct Regs {
  u32x4 v[NV];
};

// Lane t of a group of G lanes holds vectors t, t + G, ..., t + (NV - 1) G of the row: each load instruction of the
// group covers G * 16 contiguous bytes. Without FULL the index is clamped into the row (the duplicate is ignored), so
// the loads are issued unconditionally and the wait for them is not merged with a branch.
template <int G, int NV, bool FULL, bool NTL>
__device__ __forceinline__ void load_vectors(Regs<NV>& r, const void* base, long long first, long long count, int t) {
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    long long i = (long long)k * G + t;
    if constexpr (!FULL) i = i < count ? i : count - 1;
    r.v[k] = load16<NTL>(base, first + i);
  }
}

// exp(x - m) for the held vectors; returns the lane's sum over its valid elements (sequential order).
template <typename T, int G, int NV, bool FULL>
__device__ __forceinline__ float exp_and_sum(float (&f)[NV][T::V], float m, long long count, int t) {
  float s = 0.0f;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const bool ok = FULL || (long long)k * G + t < count;
#pragma unroll
    for (int i = 0; i < T::V; ++i) {
      f[k][i] = exp_to<T>(f[k][i] - m);
      s += ok ? f[k][i] : 0.0f;
    }
  }
  return s;
}

template <typename T, int G, int NV, bool FULL>
__device__ __forceinline__ float lane_max(const Regs<NV>& r, float (&f)[NV][T::V], long long count, int t) {
  float m = -INFINITY;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    unpack<T>(r.v[k], f[k]);
    const bool ok = FULL || (long long)k * G + t < count;
#pragma unroll
    for (int i = 0; i < T::V; ++i) m = ok ? fmaxf(m, f[k][i]) : m;
  }
  return m;
}

// y = f * (1 / s): one division per row and a product per element (within 1.5 ulp of f / s; an element-wise fp32
// division is a multi-instruction sequence that made these kernels compute-bound).
template <typename T, int G, int NV, bool FULL, bool NTS>
__device__ __forceinline__ void scale_store(float (&f)[NV][T::V], float s, void* base, long long first,
                                            long long count, int t, bool active) {
  const float inv = 1.0f / s;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const long long i = (long long)k * G + t;
    if (active && (FULL || i < count)) {
#pragma unroll
      for (int e = 0; e < T::V; ++e) f[k][e] = f[k][e] * inv;
      store16<NTS>(base, first + i, pack<T>(f[k]));
    }
  }
}

template <typename T, int WAVES, int NV, bool FULL, bool NTS>
__device__ __forceinline__ void softmax_row(const Regs<NV>& r, void* y, long long row, long long nvec, int t,
                                            bool active, float* slots0, float* slots1, int wave, int first) {
  constexpr int G = WAVES * kWave;
  float f[NV][T::V];
  float m = lane_max<T, G, NV, FULL>(r, f, nvec, t);
  m = group_reduce<WAVES>(m, OpMax{}, slots0, wave, first);
  float s = exp_and_sum<T, G, NV, FULL>(f, m, nvec, t);
  s = group_reduce<WAVES>(s, OpSum{}, slots1, wave, first);
  scale_store<T, G, NV, FULL, NTS>(f, s, y, row * nvec, nvec, t, active);
}

// Row tier. A block is max(WAVES, 4) waves; GROUPS = block waves / WAVES groups each walk their own rows. The loop
// trip count is uniform over the block (a group past the last row loads an in-bounds row and stores nothing), so the
// LDS barriers of a multi-wave group are reached by every wave.
template <typename T, int WAVES, int NV, bool FULL, bool NTL, bool NTS>
__global__ void __launch_bounds__((WAVES < 4 ? 4 : WAVES) * 64)
    softmax_rows(const void* __restrict__ x, void* __restrict__ y, long long rows, long long nvec) {
  constexpr int BW = WAVES < 4 ? 4 : WAVES;
  constexpr int GROUPS = BW / WAVES;
  constexpr int G = WAVES * kWave;
  __shared__ float slots[2][BW];
  const int wave = wave_id();
  const int first = (wave / WAVES) * WAVES;
  const int t = (int)threadIdx.x - first * kWave;
  const long long step = (long long)gridDim.x * GROUPS;
  long long base = (long long)blockIdx.x * GROUPS;
  if (base >= rows) return;
  const long long last = rows - 1;
  long long ra = base + wave / WAVES;
  Regs<NV> a, b;
  load_vectors<G, NV, FULL, NTL>(a, x, (ra < rows ? ra : last) * nvec, nvec, t);
  while (true) {
    const long long rb = ra + step;
    load_vectors<G, NV, FULL, NTL>(b, x, (rb < rows ? rb : last) * nvec, nvec, t);
    softmax_row<T, WAVES, NV, FULL, NTS>(a, y, ra, nvec, t, ra < rows, slots[0], slots[1], wave, first);
    base += step;
    if (base >= rows) break;
    ra = rb;
    const long long rc = ra + step;
    load_vectors<G, NV, FULL, NTL>(a, x, (rc < rows ? rc : last) * nvec, nvec, t);
    softmax_row<T, WAVES, NV, FULL, NTS>(b, y, ra, nvec, t, ra < rows, slots[0], slots[1], wave, first);
    base += step;
    if (base >= rows) break;
    ra = rc;
  }
}

// Stream tier (aligned rows too long for the co-resident tier, or when it is declined): one workgroup of WAVES waves
// per row, persistent over rows, two passes and no workspace. Pass 1 keeps each lane's online (max, sum of exp(x -
// max)) over its vectors, U of them in flight per lane, merged over the workgroup (M = max m, S = sum s * exp(m - M));
// pass 2 reads the row again and writes exp(x - M) * (1 / S): 2R + 1W, the second read mostly from the caches.
template <typename T, int WAVES, bool NTS>
__global__ void __launch_bounds__(WAVES * 64)
    softmax_stream(const void* __restrict__ x, void* __restrict__ y, long long rows, long long nvec) {
  constexpr int G = WAVES * kWave;
  constexpr int U = 4;
  __shared__ float slots[2][WAVES];
  const int t = (int)threadIdx.x;
  for (long long row = blockIdx.x; row < rows; row += gridDim.x) {
    const long long base = row * nvec;
    float m = -INFINITY, s = 0.0f;
    for (long long i0 = 0; i0 < nvec; i0 += (long long)G * U) {
      u32x4 r[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const long long i = i0 + (long long)u * G + t;
        r[u] = load16<false>(x, base + (i < nvec ? i : nvec - 1));  // clamped: issued unconditionally
      }
      float f[U][T::V];
      float cm = -INFINITY;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        unpack<T>(r[u], f[u]);
        const bool ok = i0 + (long long)u * G + t < nvec;
#pragma unroll
        for (int e = 0; e < T::V; ++e) cm = ok ? fmaxf(cm, f[u][e]) : cm;
      }
      if (cm > m) {  // rescale the running sum to the new maximum (-inf elements never raise it)
        s = m == -INFINITY ? 0.0f : s * expf(m - cm);
        m = cm;
      }
      if (m != -INFINITY) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const bool ok = i0 + (long long)u * G + t < nvec;
#pragma unroll
          for (int e = 0; e < T::V; ++e) s += ok ? exp_to<T>(f[u][e] - m) : 0.0f;
        }
      }
    }
    const float M = group_reduce<WAVES>(m, OpMax{}, slots[0], wave_id(), 0);
    const float S = group_reduce<WAVES>(m == -INFINITY ? 0.0f : s * expf(m - M), OpSum{}, slots[1], wave_id(), 0);
    const float inv = 1.0f / S;  // an all -inf row: M = -inf, S = 0, and every output NaN (as the fp64 reference)
    for (long long i = t; i < nvec; i += G) {
      float f[T::V];
      unpack<T>(load16<false>(x, base + i), f);
#pragma unroll
      for (int e = 0; e < T::V; ++e) f[e] = exp_to<T>(f[e] - M) * inv;
      store16<NTS>(y, base + i, pack<T>(f));
    }
    __syncthreads();  // the slots are written again by the next row's reductions
  }
}

// Co-resident tier: long rows in chunks of WAVES x 64 x NV vectors, one workgroup per chunk, every workgroup of a launch
// resident at once (the grid never exceeds the GPU's resident slots of this kernel): x is read once (1R + 1W). The
// grid is `groups` row groups of `chunks` workgroups; group g handles rows g, g + groups, ..., one row per iteration,
// so any number of rows keeps one pass over x. Per iteration, each workgroup holds its chunk in registers as
// e = exp(x - m) in fp32 (one exp per element), reduces it to its online-softmax pair (m, s = sum of e), and publishes
// the pair into its slot of the device-scope pair table; wave 0 polls the group's slots until every chunk's pair of
// this row is there, merges them in a fixed order (the online-softmax merge, the same lanes and order in every
// workgroup of the row, so all agree bit for bit; softmax/kernel.cu:121-152 is the reference's form of it), and the
// chunk is written as e * (exp(m - M) / S), within 3 fp32 ulp of the once-rounded value before the output's rounding.
//
// The pair table needs no clearing: each pair is two 64-bit words, (tag << 32 | m bits) and (tag << 32 | s bits),
// stored with device-coherent stores, and a word counts only when its tag is this launch's tag for the iteration.
// Every launch gets a fresh range of tags; tag 0, the table's load-time contents, is never handed out. An eager launch
// takes its range from the host, in [1, 2^31). A launch recorded into a HIP graph cannot: its kernel arguments are
// replayed as they were captured, and every replay would wait for the tags the previous replay left in the table. It
// takes its range on the device instead, at every replay, from a cell of its own that a one-wave kernel node just
// before it fills from a device counter (softmax_coop_cell), in [2^31, 2^32); so no two launches, eager or replayed,
// share a tag. The table is double-buffered by iteration parity: a chunk writes its slot of parity p again two
// iterations later, by which time every workgroup of its group has published the iteration in between, and so has
// read parity p. A launch on another stream that uses the same slots at the same time can only make a wait fail (its
// tags differ), never pass.
//
// The wait is bounded by time: after wait_ticks of the 100 MHz s_memrealtime clock with pairs still missing (other
// kernels holding CUs, so that the row's workgroups are not all resident) the workgroup takes the row's M and S from x
// itself (every thread an online max and sum over a share of the whole row), so the result stays within the tolerance
// either way; only the time suffers, by about one read of the row per waiting workgroup.
constexpr int kCoopMaxChunks = 64;   // a row's chunks: one slot each, polled by one lane each of one wave
constexpr int kCoopSlots = 4096;     // pair slots per parity: the most workgroups one launch may have
constexpr int kCoopCells = 4096;     // captured launches per device with a tag cell of their own
constexpr unsigned kDeviceTags = 0x80000000u;  // the top bit marks the tags handed out on the device
__device__ __align__(256) unsigned long long g_coop_pairs[2][kCoopSlots][2];
__device__ unsigned g_coop_cells[kCoopCells];     // each captured launch's first tag, refreshed at every replay
__device__ unsigned long long g_coop_device_next;  // tags handed out on the device so far

// The tag of iteration it of a launch whose first tag is tag0: host tags never reach the top bit (the host restarts
// its range before they would), device tags keep it and wrap within the top half.
__device__ __forceinline__ unsigned coop_tag(unsigned tag0, int it) {
  return (((tag0 & ~kDeviceTags) + (unsigned)it) & ~kDeviceTags) | (tag0 & kDeviceTags);
}

// Clears the pair table (before a launch whose tags restart after the tag counter wrapped).
__device__ __forceinline__ void coop_clear_table(unsigned first, unsigned stride) {
  unsigned long long* p = &g_coop_pairs[0][0][0];
  for (unsigned i = first; i < 2u * kCoopSlots * 2u; i += stride)
    __hip_atomic_store(p + i, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The kernel node ahead of a captured co-resident launch: takes `iters` fresh device tags and leaves the first in the
// launch's cell. When the range reaches the end of the device half of the tag space the table is cleared first, as the
// host does for its half, so that a pair left from the previous round of the counter can never match (another
// stream's launch using the table meanwhile can only see its wait fail).
__global__ void __launch_bounds__(256) softmax_coop_cell(int cell, unsigned iters) {
  __shared__ unsigned long long old;
  if (threadIdx.x == 0)
    old = __hip_atomic_fetch_add(&g_coop_device_next, (unsigned long long)iters, __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  const unsigned long long lo = old & ~(unsigned long long)kDeviceTags;
  if (lo + iters > (unsigned long long)kDeviceTags) coop_clear_table(threadIdx.x, 256);
  if (threadIdx.x == 0)
    __hip_atomic_store(&g_coop_cells[cell], kDeviceTags | (unsigned)lo, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// LOOP: some row group has more than one row (groups < rows); without it every workgroup takes one row, and the
// kernel is compiled without the loop (which costs registers: fewer resident workgroups).
template <typename T, int WAVES, int NV, bool NTL, bool NTS, bool LOOP>
__global__ void __launch_bounds__(WAVES * 64)
    softmax_coop(const void* __restrict__ x, void* __restrict__ y, long long rows, long long nvec, int chunks,
                 int groups, unsigned tag0, int cell, unsigned wait_ticks) {
  constexpr int G = WAVES * kWave;
  // a captured launch (cell >= 0) reads its first tag from its cell, filled by the kernel node just before it
  if (cell >= 0) tag0 = __hip_atomic_load(&g_coop_cells[cell], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  constexpr long long CH = (long long)G * NV;
  constexpr int PER = kCoopMaxChunks / kWave;
  __shared__ float slots[2][WAVES];
  __shared__ float ms[2];
  __shared__ int partial;  // the wait ended before every pair of the row was published
  const int c = (int)(blockIdx.x % (unsigned)chunks), group = (int)(blockIdx.x / (unsigned)chunks);
  const int first = c * (int)CH;  // < 2^31: at most kCoopMaxChunks chunks of CH vectors
  const int count = nvec - first < CH ? (int)(nvec - first) : (int)CH;
  const int t0 = (int)threadIdx.x;
  const int iters = (int)((rows - group + groups - 1) / groups);
  constexpr bool PREFETCH = LOOP && T::V == 8;
  Regs<NV> next;  // PREFETCH: the next row's raw chunk, loaded during the wait
  if constexpr (PREFETCH) load_vectors<G, NV, false, NTL>(next, x, group * nvec + first, count, t0);
  for (int it = 0; it < iters; ++it) {
    const long long row = group + (long long)it * groups;
    // the lane's offsets are formed anew each iteration (hoisted out of the loop they would hold NV 64-bit offsets in
    // registers for its whole length)
    int t = t0;
    if constexpr (LOOP) asm volatile("" : "+v"(t));
    const unsigned long long tag = (unsigned long long)coop_tag(tag0, it) << 32;
    unsigned long long(*table)[2] = g_coop_pairs[it & 1] + (long long)group * chunks;
    Regs<NV> r;
    if constexpr (PREFETCH) r = next;
    else load_vectors<G, NV, false, NTL>(r, x, row * nvec + first, count, t);
    float m = -INFINITY;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      float f[T::V];
      unpack<T>(r.v[k], f);
      const bool ok = k * G + t < count;
#pragma unroll
      for (int i = 0; i < T::V; ++i) m = ok ? fmaxf(m, f[i]) : m;
    }
    m = group_reduce<WAVES>(m, OpMax{}, slots[0], wave_id(), 0);
    // the registers take e = exp(x - m) (0 for an all -inf chunk) in place of x: one exp per element
    float e[NV][T::V];
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      float f[T::V];
      unpack<T>(r.v[k], f);
      const bool ok = k * G + t < count;
#pragma unroll
      for (int i = 0; i < T::V; ++i) {
        e[k][i] = ok && m != -INFINITY ? exp_to<T>(f[i] - m) : 0.0f;
        s += e[k][i];
      }
    }
    s = group_reduce<WAVES>(s, OpSum{}, slots[1], wave_id(), 0);
    // x is now held as e: the next row's loads go out before the wait and the stores, into the freed registers (bf16,
    // whose raw chunk is half the size of e; for fp32 the two together would halve the resident workgroups)
    if constexpr (PREFETCH)
      if (it + 1 < iters) load_vectors<G, NV, false, NTL>(next, x, (row + groups) * nvec + first, count, t);
    if (t == 0) {  // an all -inf chunk publishes (-inf, 0) and contributes nothing to the merge
      __hip_atomic_store(&table[c][0], tag | __float_as_uint(m), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&table[c][1], tag | __float_as_uint(s), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (wave_id() == 0) {
      const int lane = lane_id();
      unsigned long long wm[PER], ws[PER];
#pragma unroll
      for (int i = 0; i < PER; ++i) wm[i] = ws[i] = 0;
      const unsigned long long start = __builtin_amdgcn_s_memrealtime();
      bool complete = false;
      while (true) {
        bool have = true;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
          const int at = i * kWave + lane;
          if (at < chunks) {
            if ((wm[i] >> 32) != (tag >> 32))
              wm[i] = __hip_atomic_load(&table[at][0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if ((ws[i] >> 32) != (tag >> 32))
              ws[i] = __hip_atomic_load(&table[at][1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            have = have && (wm[i] >> 32) == (tag >> 32) && (ws[i] >> 32) == (tag >> 32);
          }
        }
        if (__ballot(!have) == 0) {
          complete = true;
          break;
        }
        // (the clock is a scalar read, so the decision is the wave's; readfirstlane states it)
        if (__builtin_amdgcn_readfirstlane((int)(__builtin_amdgcn_s_memrealtime() - start > wait_ticks))) break;
        __builtin_amdgcn_s_sleep(1);
      }
      float pm = -INFINITY, ps = 0.0f;
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        if (i * kWave + lane < chunks) {
          const float qm = __uint_as_float((unsigned)wm[i]), qs = __uint_as_float((unsigned)ws[i]);
          const float mm = fmaxf(pm, qm);
          if (mm != -INFINITY) {
            ps = ps * expf(pm - mm) + qs * expf(qm - mm);
            pm = mm;
          }
        }
      }
      const float M = wave_max(pm);
      const float S = wave_sum(M == -INFINITY ? ps : ps * expf(pm - M));
      if (lane == 0) {
        ms[0] = M;
        ms[1] = S;
        partial = complete ? 0 : 1;
      }
    }
    __syncthreads();
    if (partial) {
      // the row's M and S from x: an online max and sum per thread over its share of the row, merged over the block
      // (-inf elements add nothing; a NaN makes the sum NaN, as in the pairs)
      float tm = -INFINITY, ts = 0.0f;
      for (long long i = t; i < nvec; i += G) {
        float f[T::V];
        unpack<T>(load16<false>(x, row * nvec + i), f);
#pragma unroll
        for (int e = 0; e < T::V; ++e) {
          if (f[e] == -INFINITY) continue;
          if (f[e] > tm) {
            ts = ts * expf(tm - f[e]) + 1.0f;
            tm = f[e];
          } else {
            ts += expf(f[e] - tm);
          }
        }
      }
      const float RM = group_reduce<WAVES>(tm, OpMax{}, slots[0], wave_id(), 0);
      const float RS =
          group_reduce<WAVES>(tm == -INFINITY ? 0.0f : ts * expf(tm - RM), OpSum{}, slots[1], wave_id(), 0);
      __syncthreads();  // every wave has read ms and the slots before they are written
      if (t == 0) {
        ms[0] = RM;
        ms[1] = RS;
      }
      __syncthreads();
    }
    const float M = ms[0], S = ms[1];
    // y = e * exp(m - M) / S; an all -inf chunk (e = 0) gives 0, or NaN when the whole row is -inf (M = -inf)
    const float scale = m == -INFINITY ? (M == -INFINITY ? NAN : 0.0f) : expf(m - M) / S;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int i = k * G + t;
      if (i < count) {
        float f[T::V];
#pragma unroll
        for (int j = 0; j < T::V; ++j) f[j] = e[k][j] * scale;
        store16<NTS>(y, row * nvec + first + i, pack<T>(f));
      }
    }
    if constexpr (!LOOP) break;
    __syncthreads();  // ms, partial and the reduction slots are written again by the next row
  }
}

// Clears the pair table (before an eager launch whose tags restart after the host's tag counter wrapped).
__global__ void __launch_bounds__(256) softmax_coop_clear() {
  coop_clear_table(blockIdx.x * 256 + threadIdx.x, gridDim.x * 256);
}

// Generic tier: any row length and alignment; one 256-thread block per row (grid-strided), three scalar passes.
template <typename T>
__global__ void __launch_bounds__(256)
    softmax_generic(const void* __restrict__ x, void* __restrict__ y, long long rows, long long cols) {
  __shared__ float slots[2][4];
  const int wave = wave_id();
  for (long long row = blockIdx.x; row < rows; row += gridDim.x) {
    const long long o = row * cols;
    float m = -INFINITY;
    for (long long j = threadIdx.x; j < cols; j += 256) m = fmaxf(m, load_elem<T>(x, o + j));
    m = group_reduce<4>(m, OpMax{}, slots[0], wave, 0);
    float s = 0.0f;
    for (long long j = threadIdx.x; j < cols; j += 256) s += expf(load_elem<T>(x, o + j) - m);
    s = group_reduce<4>(s, OpSum{}, slots[1], wave, 0);
    for (long long j = threadIdx.x; j < cols; j += 256) store_elem<T>(y, o + j, expf(load_elem<T>(x, o + j) - m) / s);
    __syncthreads();  // slots are rewritten by the next row's reductions
  }
}

// ---- host side ------------------------------------------------------------------------------------------------------

// Tuning slots (0 = automatic), for sweeps and tests: row-tier waves per row, row-tier vectors per lane, row-tier
// resident blocks per CU, stream-tier waves, co-resident row groups (fewer forces more rows per workgroup), preferred
// tier (1 row, 2 stream, 3 generic, 4 co-resident; a tier that cannot take the rows is passed over for the automatic
// choice), non-temporal loads (1 on, 2 off), the co-resident tier's wait budget in 100 MHz ticks (tests force its
// fallback with 1).
enum { kTuneWaves = 0, kTuneNv = 1, kTuneBlocksPerCu = 2, kTuneStreamWaves = 3, kTuneCoopGroups = 4, kTuneTier = 5,
       kTuneNtLoads = 6, kTuneWaitTicks = 7 };
constexpr unsigned kCoopWaitTicks = 10000;  // 100 us: tens of times a row's arrival skew, a few launch lengths

int pow2_at_least(long long v) {
  int p = 1;
  while (p < v) p <<= 1;
  return p;
}

template <typename Kernel>
int blocks_per_cu(Kernel k, int threads) {
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k, threads, 0) != hipSuccess || n <= 0) {
    (void)hipGetLastError();
    n = 1;
  }
  return n;
}

template <typename T, int WAVES, int NV, bool FULL, bool NTL>
int launch_rows_k(const void* x, void* y, long long rows, long long nvec, hipStream_t stream) {
  constexpr int BW = WAVES < 4 ? 4 : WAVES;
  constexpr int GROUPS = BW / WAVES;
  auto kern = softmax_rows<T, WAVES, NV, FULL, NTL, true>;
  static int occ = 0;  // resident blocks per CU of this instantiation (idempotent cache)
  if (occ <= 0) occ = blocks_per_cu(kern, BW * kWave);
  // about 8 resident waves per CU by default: with two register sets per wave that keeps enough loads in flight,
  // and more waves only contend (measured on MI355X); rows of 8 waves take 16 (two blocks): [4096, 4096] fp32 as 8
  // waves x 2 vectors 24.61 -> 24.37 us (means of six fresh allocations each), [2048, 8192] as 8 waves x 4 vectors
  // 25.69 -> 25.12 us (interleaved runs on one box)
  int per_cu = rw_host::tune_get(kTuneBlocksPerCu);
  if (per_cu <= 0) per_cu = WAVES == 8 ? 2 : (8 / BW > 1 ? 8 / BW : 1);
  if (per_cu > occ) per_cu = occ;
  const long long need = (rows + GROUPS - 1) / GROUPS;
  long long grid = (long long)rw_host::device_cus() * per_cu;
  if (grid > need) grid = need;
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(BW * kWave), 0, stream, x, y, rows, nvec);
  return (int)hipGetLastError();
}

template <typename T, int WAVES, int NV, bool NTL>
int launch_rows_nv(const void* x, void* y, long long rows, long long nvec, hipStream_t stream) {
  if (nvec == (long long)WAVES * kWave * NV) return launch_rows_k<T, WAVES, NV, true, NTL>(x, y, rows, nvec, stream);
  return launch_rows_k<T, WAVES, NV, false, NTL>(x, y, rows, nvec, stream);
}

template <typename T, int WAVES, bool NTL>
int launch_rows_w(int nv, const void* x, void* y, long long rows, long long nvec, hipStream_t stream) {
  switch (nv) {
    case 1: return launch_rows_nv<T, WAVES, 1, NTL>(x, y, rows, nvec, stream);
    case 2: return launch_rows_nv<T, WAVES, 2, NTL>(x, y, rows, nvec, stream);
    case 4: return launch_rows_nv<T, WAVES, 4, NTL>(x, y, rows, nvec, stream);
    case 8: return launch_rows_nv<T, WAVES, 8, NTL>(x, y, rows, nvec, stream);
    case 16:  // (through the tuning slots: one or two waves holding a row of up to 8192 fp32 / 16384 bf16 elements)
      if constexpr (WAVES <= 2) return launch_rows_nv<T, WAVES, 16, NTL>(x, y, rows, nvec, stream);
      else return rw_host::kInvalid;
    default: return rw_host::kInvalid;
  }
}

template <typename T, bool NTL>
int launch_rows(int waves, int nv, const void* x, void* y, long long rows, long long nvec, hipStream_t stream) {
  switch (waves) {
    case 1: return launch_rows_w<T, 1, NTL>(nv, x, y, rows, nvec, stream);
    case 2: return launch_rows_w<T, 2, NTL>(nv, x, y, rows, nvec, stream);
    case 4: return launch_rows_w<T, 4, NTL>(nv, x, y, rows, nvec, stream);
    case 8: return launch_rows_w<T, 8, NTL>(nv, x, y, rows, nvec, stream);
    case 16: return launch_rows_w<T, 16, NTL>(nv, x, y, rows, nvec, stream);
    default: return rw_host::kInvalid;
  }
}

template <typename T, int WAVES>
int launch_stream_w(const void* x, void* y, long long rows, long long nvec, hipStream_t stream) {
  long long grid = (long long)rw_host::device_cus() * (16 / WAVES > 1 ? 16 / WAVES : 1);
  if (grid > rows) grid = rows;
  hipLaunchKernelGGL((softmax_stream<T, WAVES, true>), dim3((unsigned)grid), dim3(WAVES * kWave), 0, stream, x, y,
                     rows, nvec);
  return (int)hipGetLastError();
}

template <typename T>
int launch_stream(const void* x, void* y, long long rows, long long nvec, hipStream_t stream) {
  switch (rw_host::tune_get(kTuneStreamWaves)) {
    case 4: return launch_stream_w<T, 4>(x, y, rows, nvec, stream);
    case 8: return launch_stream_w<T, 8>(x, y, rows, nvec, stream);
    default: return launch_stream_w<T, 16>(x, y, rows, nvec, stream);
  }
}

// The co-resident tier's tags of eager launches: per device, the next unused one of the host's half of the tag space,
// [1, 2^31) (0 is never handed out: it is the pair table's contents at load). A launch takes one per iteration; when the
// range would pass 2^31 - 1, the table is cleared on the launch's stream and the tags start again at 1.
unsigned coop_tags(int dev, unsigned n, hipStream_t stream, int* err) {
  static std::mutex mu;
  static unsigned next[64];
  std::lock_guard<std::mutex> lock(mu);
  unsigned& nx = next[dev & 63];
  *err = rw_host::kOk;
  if (nx == 0 || (unsigned long long)nx + n > (unsigned long long)kDeviceTags) {
    hipLaunchKernelGGL(softmax_coop_clear, dim3(16), dim3(256), 0, stream);
    *err = (int)hipGetLastError();
    nx = 1;
  }
  const unsigned t = nx;
  nx += n;
  return t;
}

// A captured launch's tag cell: per device, cells are handed out once each, in capture order, and never reused (a
// graph may be replayed at any time). Returns -1 when the device's cells are used up; such a launch takes the stream
// tier, which keeps no state between launches.
int coop_cell(int dev) {
  static std::mutex mu;
  static int next[64];
  std::lock_guard<std::mutex> lock(mu);
  int& nx = next[dev & 63];
  if (nx >= kCoopCells) return -1;
  return nx++;
}

// Whether work issued to `stream` is being recorded into a graph (an error reads as not capturing: the launch then
// fails or runs as an eager one would).
bool capturing(hipStream_t stream) {
  hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &status) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  return status != hipStreamCaptureStatusNone;
}

// Co-resident tier: chunks of 4 waves x 64 lanes x 64 elements (16 fp32 or 8 bf16 vectors per lane), at most
// kCoopMaxChunks per row; one row per workgroup when every row's chunks fit on the GPU at once, else row groups
// walking several rows (a second instantiation: the loop costs registers). Returns 1, launching nothing, when one
// row's chunks do not fit on the GPU at once.
template <typename T, bool NTL>
int launch_coop(const void* x, void* y, long long rows, long long nvec, hipStream_t stream) {
  constexpr int WAVES = 4, NV1 = 64 / T::V, NVL = T::V == 4 ? 16 : 8;
  constexpr long long CH1 = (long long)WAVES * kWave * NV1, CHL = (long long)WAVES * kWave * NVL;
  auto one = softmax_coop<T, WAVES, NV1, NTL, true, false>;
  auto loop = softmax_coop<T, WAVES, NVL, NTL, true, true>;
  static int occ_one = 0, occ_loop = 0;  // resident blocks per CU of each instantiation (idempotent caches)
  if (occ_one <= 0) occ_one = blocks_per_cu(one, WAVES * kWave);
  if (occ_loop <= 0) occ_loop = blocks_per_cu(loop, WAVES * kWave);
  const int want = rw_host::tune_get(kTuneCoopGroups);
  const long long cus = rw_host::device_cus();
  long long chunks = (nvec + CH1 - 1) / CH1;
  long long slots = cus * occ_one;
  if (slots > kCoopSlots) slots = kCoopSlots;
  const bool single = chunks <= kCoopMaxChunks && rows * chunks <= slots && (want <= 0 || want >= rows);
  if (!single) {
    chunks = (nvec + CHL - 1) / CHL;
    slots = cus * occ_loop;
    if (slots > kCoopSlots) slots = kCoopSlots;
    if (chunks > kCoopMaxChunks || chunks > slots) return 1;
  }
  long long groups = single ? rows : slots / chunks;
  if (want > 0 && want < groups) groups = want;
  if (groups > rows) groups = rows;
  const long long iters = (rows + groups - 1) / groups;
  if (iters > 0x40000000LL) return 1;
  int dev = 0, err = (int)hipGetDevice(&dev);
  if (err != rw_host::kOk) return err;
  unsigned tag0 = 0;
  int cell = -1;
  if (capturing(stream)) {
    // recorded into a graph: the tags are taken on the device at every replay, by a kernel node ahead of the launch
    cell = coop_cell(dev);
    if (cell < 0) return 1;
    hipLaunchKernelGGL(softmax_coop_cell, dim3(1), dim3(256), 0, stream, cell, (unsigned)iters);
    err = (int)hipGetLastError();
  } else {
    tag0 = coop_tags(dev, (unsigned)iters, stream, &err);
  }
  if (err != rw_host::kOk) return err;
  const int budget = rw_host::tune_get(kTuneWaitTicks);
  const unsigned ticks = budget > 0 ? (unsigned)budget : kCoopWaitTicks;
  const dim3 grid((unsigned)(groups * chunks)), block(WAVES * kWave);
  if (single)
    hipLaunchKernelGGL(one, grid, block, 0, stream, x, y, rows, nvec, (int)chunks, (int)groups, tag0, cell, ticks);
  else
    hipLaunchKernelGGL(loop, grid, block, 0, stream, x, y, rows, nvec, (int)chunks, (int)groups, tag0, cell, ticks);
  return (int)hipGetLastError();
}

template <typename T>
int launch_generic(const void* x, void* y, long long rows, long long cols, hipStream_t stream) {
  long long grid = (long long)rw_host::device_cus() * 8;
  if (grid > rows) grid = rows;
  hipLaunchKernelGGL(softmax_generic<T>, dim3((unsigned)grid), dim3(256), 0, stream, x, y, rows, cols);
  return (int)hipGetLastError();
}

template <typename T>
int launch_typed(const void* x, void* y, long long rows, long long cols, hipStream_t stream) {
  const bool vec = cols % T::V == 0 && rw_host::aligned16(x) && rw_host::aligned16(y);
  const int tier = rw_host::tune_get(kTuneTier);
  if (!vec || tier == 3) return launch_generic<T>(x, y, rows, cols, stream);
  const long long nvec = cols / T::V;
  if (tier == 2) return launch_stream<T>(x, y, rows, nvec, stream);
  const bool ntl = rw_host::tune_get(kTuneNtLoads) == 1;
  if (tier != 4 && nvec <= (long long)kMaxWaves * kWave * kMaxNv) {
    // Row tier: 4 vectors per lane as long as 16 waves suffice, then up to 8; except that rows of 513 to 1024
    // vectors take 8 waves of 2 vectors rather than 4 waves of 4 (more waves with fewer loads each; [4096, 4096]
    // fp32 24.61 -> 24.37 us measured).
    auto auto_waves = [&] {
      const long long lanes = (nvec + 3) / 4;
      const int w = pow2_at_least((lanes + kWave - 1) / kWave);
      return w == 4 ? 8 : w > kMaxWaves ? kMaxWaves : w;
    };
    auto auto_nv = [&](int w) { return pow2_at_least((nvec + (long long)w * kWave - 1) / ((long long)w * kWave)); };
    int waves = rw_host::tune_get(kTuneWaves), nv = rw_host::tune_get(kTuneNv);
    if (waves <= 0) waves = auto_waves();
    if (nv <= 0) nv = auto_nv(waves);
    // a tuned shape the row kernel does not have (launch_rows below) is ignored: the automatic choice runs
    const bool shape = (waves == 1 || waves == 2 || waves == 4 || waves == 8 || waves == 16) &&
                       (nv == 1 || nv == 2 || nv == 4 || nv == 8 || (nv == 16 && waves <= 2));
    if (!shape) {
      waves = auto_waves();
      nv = auto_nv(waves);
    }
    if ((long long)waves * kWave * nv >= nvec) {
      return ntl ? launch_rows<T, true>(waves, nv, x, y, rows, nvec, stream)
                 : launch_rows<T, false>(waves, nv, x, y, rows, nvec, stream);
    }
  }
  const int rc =
      ntl ? launch_coop<T, true>(x, y, rows, nvec, stream) : launch_coop<T, false>(x, y, rows, nvec, stream);
  if (rc != 1) return rc;
  return launch_stream<T>(x, y, rows, nvec, stream);
}

}  // namespace

// softmax/kernel.cu:520 `launch`: dtype 0 = fp32, 1 = bf16. `threads` and `aux` are the reference's block-size hints
// for its CUDA tiers; they are accepted and not used (as softmax/seed.cu:70-71 does): the tier and shape are chosen
// from the row length. rows <= 0 or cols <= 0 is a successful no-op.
extern "C" int launch(const void* x, void* y, long long rows, long long cols, int dtype, int threads, int aux,
                      hipStream_t stream) {
  (void)threads;
  (void)aux;
  if (rows <= 0 || cols <= 0) return rw_host::kOk;
  if (dtype == 0) return launch_typed<F32>(x, y, rows, cols, stream);
  if (dtype == 1) return launch_typed<BF16>(x, y, rows, cols, stream);
  return rw_host::kInvalid;
}

// Tuning override for parameter sweeps (see the slot list above); 0 restores the automatic choice.
extern "C" int softmax_tune(int slot, int value) { return rw_host::tune_set(slot, value); }
