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
//  - co-resident tier (longer rows, when all of their chunks fit on the GPU at once): one pass; see softmax_coop.
//  - split tier (longer rows otherwise): a row is split into chunks of WAVES x 64 x NV vectors, one workgroup each.
//    Pass 1 reduces each chunk to its online-softmax pair (m, s = sum of exp(x - m)) in a workspace; pass 2 merges the
//    row's pairs (M = max m, S = sum of s * exp(m - M)) in every wave and writes exp(x - M) / S for its chunk,
//    re-reading the chunk (2R + 1W).
//  - generic tier (any length or alignment): one workgroup per row, three scalar passes (max, sum, write).
// The normalisation multiplies by the fp32 reciprocal of the row sum (the reference divides, softmax/kernel.cu:240;
// the two differ by at most 1.5 ulp in fp32 and are within the 1e-5 relative tolerance of the fp64 oracle).
#include <climits>
#include <cmath>

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
      f[k][i] = expf(f[k][i] - m);
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

// Split tier, pass 1: block b = row * chunks + c reduces vectors [c * CH, min((c + 1) * CH, nvec)) of its row to
// (m, s) and writes them to ws[b].
template <typename T, int WAVES, int NV, bool NTL>
__global__ void __launch_bounds__(WAVES * 64)
    softmax_split_stats(const void* __restrict__ x, float2* __restrict__ ws, long long nvec, long long chunks) {
  constexpr int G = WAVES * kWave;
  constexpr long long CH = (long long)G * NV;
  __shared__ float slots[2][WAVES];
  const long long b = blockIdx.x;
  const long long row = b / chunks, c = b - row * chunks;
  const long long first = c * CH;
  const long long count = nvec - first < CH ? nvec - first : CH;
  const int t = (int)threadIdx.x;
  Regs<NV> r;
  load_vectors<G, NV, false, NTL>(r, x, row * nvec + first, count, t);
  float f[NV][T::V];
  float m = lane_max<T, G, NV, false>(r, f, count, t);
  m = group_reduce<WAVES>(m, OpMax{}, slots[0], wave_id(), 0);
  float s = exp_and_sum<T, G, NV, false>(f, m, count, t);
  s = group_reduce<WAVES>(s, OpSum{}, slots[1], wave_id(), 0);
  // An all -inf chunk contributes nothing to the merge (its NaN sum must not reach it).
  if (t == 0) ws[b] = make_float2(m, m == -INFINITY ? 0.0f : s);
}

// Merge of a row's chunk pairs, computed identically (same lanes, same order) by every wave that needs it.
__device__ __forceinline__ void merge_pairs(const float2* __restrict__ p, long long chunks, float& M, float& S) {
  const int lane = lane_id();
  float m = -INFINITY, s = 0.0f;
  for (long long i = lane; i < chunks; i += kWave) {
    const float2 q = p[i];
    const float mm = fmaxf(m, q.x);
    if (mm != -INFINITY) {
      s = s * expf(m - mm) + q.y * expf(q.x - mm);
      m = mm;
    }
  }
  M = wave_max(m);
  S = wave_sum(M == -INFINITY ? s : s * expf(m - M));
}

// Split tier, pass 2: re-reads the chunk and writes exp(x - M) / S.
template <typename T, int WAVES, int NV, bool NTL, bool NTS>
__global__ void __launch_bounds__(WAVES * 64)
    softmax_split_apply(const void* __restrict__ x, void* __restrict__ y, const float2* __restrict__ ws,
                        long long nvec, long long chunks) {
  constexpr int G = WAVES * kWave;
  constexpr long long CH = (long long)G * NV;
  const long long b = blockIdx.x;
  const long long row = b / chunks, c = b - row * chunks;
  const long long first = c * CH;
  const long long count = nvec - first < CH ? nvec - first : CH;
  const int t = (int)threadIdx.x;
  Regs<NV> r;
  load_vectors<G, NV, false, NTL>(r, x, row * nvec + first, count, t);
  float M, S;
  merge_pairs(ws + row * chunks, chunks, M, S);
  float f[NV][T::V];
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    unpack<T>(r.v[k], f[k]);
#pragma unroll
    for (int e = 0; e < T::V; ++e) f[k][e] = expf(f[k][e] - M);
  }
  scale_store<T, G, NV, false, NTS>(f, S, y, row * nvec + first, count, t, true);
}

// Co-resident tier, for long rows whose chunks all fit on the GPU at once: the split tier's chunks, each held in its
// workgroup's registers across the exchange of the row's chunk pairs, so x is read once (1R + 1W). For fp32 the
// registers hold exp(x - m) after the first pass and the output is exp(x - m) * (exp(m - M) / S), within 3 ulp of
// the once-rounded value (outputs in the fp32 subnormal range, below 2^-126, are within a few 2^-149). The grid never
// exceeds what the GPU holds at once, so every workgroup of a row is resident (or waits only for other kernels to
// drain). A workgroup publishes its pair (m, s) as one device-coherent 64-bit store into the row's slot for it; a slot
// holding 0 is unpublished (no pair is 0: a chunk's s is >= 1 for a finite max, an all -inf chunk stores (-inf, 0)
// and a NaN chunk NaNs). Wave 0 polls the row's slots with device-coherent loads until all are published, merges them
// (the same lanes and order in every workgroup of the row, so all agree bit for bit) and hands M and S to the other
// waves; the chunk is then written from the registers. Last, a departure counter finds the row's last workgroup, which
// zeroes the row's slots and the counter for the next launch (the workspace starts zeroed). The wait is bounded
// (spin_limit polls): it always ends, even if a row's workgroups could not all run at once (other kernels holding
// CUs, or two such launches on two streams). A workgroup whose wait ends before every pair is published takes the
// row's M and S from x itself (every thread an online max and sum over a share of the whole row), so the result
// stays within the tolerance either way; only the time suffers.
constexpr unsigned kSpinLimit = 1u << 22;
constexpr int kCoopMaxChunks = 64;  // slots a row may have (one per lane of the polling wave)

__device__ __forceinline__ unsigned long long pair_bits(float m, float s) {
  return ((unsigned long long)__float_as_uint(s) << 32) | __float_as_uint(m);
}

template <typename T, int WAVES, int NV, bool NTL, bool NTS>
__global__ void __launch_bounds__(WAVES * 64)
    softmax_coop(const void* __restrict__ x, void* __restrict__ y, unsigned long long* __restrict__ pairs,
                 unsigned* __restrict__ departs, long long nvec, long long chunks, unsigned spin_limit) {
  constexpr int G = WAVES * kWave;
  constexpr long long CH = (long long)G * NV;
  constexpr int PER = kCoopMaxChunks / kWave;
  __shared__ float slots[2][WAVES];
  __shared__ float ms[2];
  __shared__ int partial;  // the wait ended before every pair of the row was published
  const long long b = blockIdx.x;
  const long long row = b / chunks, c = b - row * chunks;
  const long long first = c * CH;
  const long long count = nvec - first < CH ? nvec - first : CH;
  const int t = (int)threadIdx.x;
  Regs<NV> r;
  load_vectors<G, NV, false, NTL>(r, x, row * nvec + first, count, t);
  // the chunk's pair; exp(x - m) is not kept (the registers keep x for the second use)
  float m = -INFINITY;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    float f[T::V];
    unpack<T>(r.v[k], f);
    const bool ok = (long long)k * G + t < count;
#pragma unroll
    for (int i = 0; i < T::V; ++i) m = ok ? fmaxf(m, f[i]) : m;
  }
  m = group_reduce<WAVES>(m, OpMax{}, slots[0], wave_id(), 0);
  // fp32: the registers now take e = exp(x - m) (0 for an all -inf chunk) in place of x, and the output is e * (exp(m -
  // M) / S): one exp per element. bf16 (twice the elements per register) keeps x and evaluates exp(x - M) again.
  constexpr bool KEEP = T::V == 4;
  float s = 0.0f;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    float f[T::V];
    unpack<T>(r.v[k], f);
    const bool ok = (long long)k * G + t < count;
#pragma unroll
    for (int i = 0; i < T::V; ++i) {
      const float e = ok && m != -INFINITY ? expf(f[i] - m) : 0.0f;
      s += e;
      if constexpr (KEEP) r.v[k][i] = __float_as_uint(e);
    }
  }
  s = group_reduce<WAVES>(s, OpSum{}, slots[1], wave_id(), 0);
  unsigned long long* row_pairs = pairs + row * chunks;
  if (t == 0)  // an all -inf chunk has s = 0 and contributes nothing to the merge
    __hip_atomic_store(row_pairs + c, pair_bits(m, s), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (wave_id() == 0) {
    const int lane = lane_id();
    unsigned long long v[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) v[i] = 0;
    for (unsigned n = 0; n < spin_limit; ++n) {
      bool ready = true;
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const long long at = (long long)i * kWave + lane;
        if (at < chunks && v[i] == 0)
          v[i] = __hip_atomic_load(row_pairs + at, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        ready = ready && (at >= chunks || v[i] != 0);
      }
      if (__ballot(!ready) == 0) break;
      __builtin_amdgcn_s_sleep(1);
    }
    bool have = true;
#pragma unroll
    for (int i = 0; i < PER; ++i) have = have && ((long long)i * kWave + lane >= chunks || v[i] != 0);
    const bool complete = __ballot(!have) == 0;
    float pm = -INFINITY, ps = 0.0f;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      if ((long long)i * kWave + lane < chunks) {
        const float qm = __uint_as_float((unsigned)v[i]), qs = __uint_as_float((unsigned)(v[i] >> 32));
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
    const float RS = group_reduce<WAVES>(tm == -INFINITY ? 0.0f : ts * expf(tm - RM), OpSum{}, slots[1], wave_id(), 0);
    __syncthreads();  // every wave has read ms and the slots before they are written
    if (t == 0) {
      ms[0] = RM;
      ms[1] = RS;
    }
    __syncthreads();
  }
  const float M = ms[0], S = ms[1];
  if constexpr (KEEP) {
    // y = e * exp(m - M) / S; an all -inf chunk (e = 0) gives 0, or NaN when the whole row is -inf (M = -inf)
    const float scale = m == -INFINITY ? (M == -INFINITY ? NAN : 0.0f) : expf(m - M) / S;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const long long i = (long long)k * G + t;
      if (i < count) {
        float f[T::V];
#pragma unroll
        for (int e = 0; e < T::V; ++e) f[e] = __uint_as_float(r.v[k][e]) * scale;
        store16<NTS>(y, row * nvec + first + i, pack<T>(f));
      }
    }
  } else {
    float f[NV][T::V];
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      unpack<T>(r.v[k], f[k]);
#pragma unroll
      for (int e = 0; e < T::V; ++e) f[k][e] = expf(f[k][e] - M);
    }
    scale_store<T, G, NV, false, NTS>(f, S, y, row * nvec + first, count, t, true);
  }
  if (wave_id() == 0) {
    unsigned old = 0;
    if (lane_id() == 0) old = __hip_atomic_fetch_add(departs + row, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (__builtin_amdgcn_readfirstlane(old) == (unsigned)chunks - 1) {  // the row's last workgroup: clear for reuse
      for (long long at = lane_id(); at < chunks; at += kWave)
        __hip_atomic_store(row_pairs + at, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (lane_id() == 0) __hip_atomic_store(departs + row, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
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

// Tuning slots (0 = automatic): row-tier waves per row, row-tier vectors per lane, row-tier resident blocks per CU,
// split-tier waves, split-tier vectors per lane, forced tier (1 row, 2 split, 3 generic, 4 co-resident), non-temporal
// loads (1 on, 2 off), the co-resident tier's bound on its polls (tests force its fallback with a small one).
enum { kTuneWaves = 0, kTuneNv = 1, kTuneBlocksPerCu = 2, kTuneSplitWaves = 3, kTuneSplitNv = 4, kTuneTier = 5,
       kTuneNtLoads = 6, kTuneSpinLimit = 7 };

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
  // and more waves only contend (measured on MI355X)
  int per_cu = rw_host::tune_get(kTuneBlocksPerCu);
  if (per_cu <= 0) per_cu = 8 / BW > 1 ? 8 / BW : 1;
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

template <typename T, int WAVES, int NV, bool NTL>
int launch_split_k(const void* x, void* y, long long rows, long long nvec, hipStream_t stream) {
  constexpr long long CH = (long long)WAVES * kWave * NV;
  const long long chunks = (nvec + CH - 1) / CH;
  const long long blocks = rows * chunks;
  if (blocks > (long long)UINT_MAX) return rw_host::kInvalid;
  int err = 0;
  float2* ws = (float2*)rw_host::stream_workspace(stream, (size_t)blocks * sizeof(float2), &err);
  if (!ws) return err;
  hipLaunchKernelGGL((softmax_split_stats<T, WAVES, NV, NTL>), dim3((unsigned)blocks), dim3(WAVES * kWave), 0, stream,
                     x, ws, nvec, chunks);
  hipLaunchKernelGGL((softmax_split_apply<T, WAVES, NV, NTL, true>), dim3((unsigned)blocks), dim3(WAVES * kWave), 0,
                     stream, x, y, ws, nvec, chunks);
  return (int)hipGetLastError();
}

template <typename T, int WAVES, bool NTL>
int launch_split_w(int nv, const void* x, void* y, long long rows, long long nvec, hipStream_t stream) {
  switch (nv) {
    case 2: return launch_split_k<T, WAVES, 2, NTL>(x, y, rows, nvec, stream);
    case 4: return launch_split_k<T, WAVES, 4, NTL>(x, y, rows, nvec, stream);
    case 8: return launch_split_k<T, WAVES, 8, NTL>(x, y, rows, nvec, stream);
    default: return rw_host::kInvalid;
  }
}

template <typename T, bool NTL>
int launch_split(int waves, int nv, const void* x, void* y, long long rows, long long nvec, hipStream_t stream) {
  switch (waves) {
    case 4: return launch_split_w<T, 4, NTL>(nv, x, y, rows, nvec, stream);
    case 8: return launch_split_w<T, 8, NTL>(nv, x, y, rows, nvec, stream);
    case 16: return launch_split_w<T, 16, NTL>(nv, x, y, rows, nvec, stream);
    default: return rw_host::kInvalid;
  }
}

// Co-resident tier: chunks of 4 waves x 64 lanes x 16 vectors (16384 fp32 / 32768 bf16 elements), up to kCoopRows
// rows of up to kCoopMaxChunks chunks. Returns 1, launching nothing, when the rows' chunks do not all fit on the GPU
// at once. Workspace: the departure counters (a fixed region, so that launches of any shape agree on it), then the
// pair slots.
constexpr long long kCoopRows = 4096;
constexpr size_t kCoopCounterBytes = (size_t)kCoopRows * sizeof(unsigned);

template <typename T, bool NTL>
int launch_coop(const void* x, void* y, long long rows, long long nvec, hipStream_t stream) {
  constexpr int WAVES = 4, NV = 16;
  constexpr long long CH = (long long)WAVES * kWave * NV;
  long long chunks = (nvec + CH - 1) / CH;
  auto kern = softmax_coop<T, WAVES, NV, NTL, true>;
  static int occ = 0;  // resident blocks per CU of this instantiation (idempotent cache)
  if (occ <= 0) occ = blocks_per_cu(kern, WAVES * kWave);
  const long long blocks = rows * chunks;
  if (rows > kCoopRows || chunks > kCoopMaxChunks || blocks > (long long)rw_host::device_cus() * occ) return 1;
  int err = 0;
  char* ws = (char*)rw_host::stream_workspace(stream, kCoopCounterBytes + (size_t)blocks * 8, &err, 1, true);
  if (!ws) return err;
  unsigned* departs = (unsigned*)ws;
  unsigned long long* pairs = (unsigned long long*)(ws + kCoopCounterBytes);
  const int limit = rw_host::tune_get(kTuneSpinLimit);
  hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(WAVES * kWave), 0, stream, x, y, pairs, departs, nvec, chunks,
                     limit > 0 ? (unsigned)limit : kSpinLimit);
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
  const bool ntl = rw_host::tune_get(kTuneNtLoads) == 1;
  if (tier != 2 && nvec <= (long long)kMaxWaves * kWave * kMaxNv) {
    // Row tier: 4 vectors per lane as long as 16 waves suffice, then up to 8.
    int waves = rw_host::tune_get(kTuneWaves), nv = rw_host::tune_get(kTuneNv);
    if (waves <= 0) {
      const long long lanes = (nvec + 3) / 4;
      waves = pow2_at_least((lanes + kWave - 1) / kWave);
      if (waves > kMaxWaves) waves = kMaxWaves;
    }
    if (nv <= 0) nv = pow2_at_least((nvec + (long long)waves * kWave - 1) / ((long long)waves * kWave));
    if ((long long)waves * kWave * nv >= nvec) {
      return ntl ? launch_rows<T, true>(waves, nv, x, y, rows, nvec, stream)
                 : launch_rows<T, false>(waves, nv, x, y, rows, nvec, stream);
    }
    if (tier == 1) return rw_host::kInvalid;
  }
  if (tier == 0 || tier == 4) {
    const int rc =
        ntl ? launch_coop<T, true>(x, y, rows, nvec, stream) : launch_coop<T, false>(x, y, rows, nvec, stream);
    if (rc != 1) return rc;
    if (tier == 4) return rw_host::kInvalid;
  }
  int waves = rw_host::tune_get(kTuneSplitWaves), nv = rw_host::tune_get(kTuneSplitNv);
  if (waves <= 0) waves = 4;
  if (nv <= 0) nv = 8;
  return ntl ? launch_split<T, true>(waves, nv, x, y, rows, nvec, stream)
             : launch_split<T, false>(waves, nv, x, y, rows, nvec, stream);
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
