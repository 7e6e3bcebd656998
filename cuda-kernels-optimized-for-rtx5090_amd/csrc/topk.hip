// Row-wise top-k (largest, sorted descending, ties broken by the lowest index) of x[rows, cols] in fp32 (dtype 0) or
// bf16 (dtype 1), behind the reference's C-ABI `plan` and `launch` (topk/kernel.cu:520-570), for 1 <= k <= 1024.
//
// Order (topk/kernel.cu:1-3, :56-60): every element is ranked by the 64-bit composite (key << 32) | ~index, key = ~u
// for a set sign bit and u | 0x80000000 otherwise (u the fp32 bits; a bf16 element is widened first). Composites are
// distinct, a larger one comes first, and composite 0 means "no element". Values are decoded from the composites bit
// for bit, so x is read once.
//
// Two kernels on the caller's stream (the stream order publishes the first kernel's workspace writes to the second;
// a same-kernel hand-off would need an agent-scope release and acquire per workgroup, i.e. an L2 write-back and
// invalidate of an XCD per workgroup, which costs far more than a second launch):
//  - topk_chunks, one 256-thread workgroup per (chunk, row): the workgroup loads a block of its chunk (E elements per
//    lane, 16-byte loads, all in flight at once) into registers and admits the block's top-k into an LDS buffer:
//      seed   - for k <= 64 each wave ranks its 64 lane maxima (v_readlane broadcasts, no barrier) and takes the k-th;
//               k distinct elements lie at or above it, and the block takes the largest such wave seed;
//      admit  - if the composites >= the seed fit the buffer they are appended (one LDS atomic per wave: ballot,
//               popcount, mbcnt), otherwise 256-bin histograms over the register values narrow the range [lo, hi]
//               holding the k-th (bins (c - lo) >> s, adaptive to the data) until the rest fits;
//    then prunes the buffer to exactly its k largest with the same histogram narrowing over LDS. A chunk longer than
//    one register block repeats this per block, from the buffer's current k-th. With one chunk per row it sorts and
//    writes the outputs; otherwise it writes its k composites (smallest first) to the workspace.
//  - topk_merge, one workgroup per split row: streams the row's nchunks * k composites through the buffer from a floor
//    equal to the largest chunk minimum (each full list holds k composites at or above its minimum), prunes to k,
//    sorts (bitonic in LDS) and writes values and int64 indices.
#include <climits>
#include <cstdint>
#include <type_traits>

#include "host.hpp"
#include "rowwise.hpp"

using namespace rw;

namespace {

typedef unsigned long long u64;

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kBins = 256;
constexpr int kMaxK = 1024;
constexpr int kChunkBuf = 2048;   // chunk kernel buffer: k composites kept + a block's admissions
constexpr int kMergeBuf = 4096;   // merge kernel buffer: k kept + one 2048-composite tile
constexpr int kMergePer = 8;      // composites per lane per merge tile
constexpr int kMergeTile = kThreads * kMergePer;
constexpr int kSeedMaxK = 64;

static_assert(2 * kMaxK <= kChunkBuf, "a block's top-k must fit beside the kept k");
static_assert(kMaxK + kMergeTile <= kMergeBuf, "a merge tile must fit beside the kept k");

template <int CAP>
struct Smem {
  u64 buf[CAP];
  unsigned hist[kBins];
  unsigned wsum[kWaves];
  u64 red[kWaves];
  u64 thr;       // admit composites >= thr (>= 1: composite 0 is never admitted)
  int count;     // composites in buf
  int bin;       // narrowing: the bin holding the wanted rank
  int above;     // narrowing: composites in the bins above it
};

__device__ __forceinline__ u64 composite(uint32_t u, uint32_t index) {
  const uint32_t key = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((u64)key << 32) | (u64)(~index);
}
__device__ __forceinline__ uint32_t composite_bits(u64 c) {
  const uint32_t key = (uint32_t)(c >> 32);
  return (key & 0x80000000u) ? (key & 0x7fffffffu) : ~key;
}
__device__ __forceinline__ long long composite_index(u64 c) { return (long long)(uint32_t)~(uint32_t)c; }

// ---- wave / block primitives ---------------------------------------------------------------------------------------

template <int CTRL>
__device__ __forceinline__ u64 dpp64(u64 v) {
  const int lo = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)v, CTRL, 0xF, 0xF, false);
  const int hi = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)(v >> 32), CTRL, 0xF, 0xF, false);
  return ((u64)(uint32_t)hi << 32) | (uint32_t)lo;
}
__device__ __forceinline__ u64 readlane64(u64 v, int lane) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, lane);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), lane);
  return ((u64)hi << 32) | lo;
}
template <bool MAX>
__device__ __forceinline__ u64 pick64(u64 a, u64 b) { return MAX ? (a > b ? a : b) : (a < b ? a : b); }

template <bool MAX>
__device__ __forceinline__ u64 wave_ext64(u64 v) {
  v = pick64<MAX>(v, dpp64<kDppXor1>(v));
  v = pick64<MAX>(v, dpp64<kDppXor2>(v));
  v = pick64<MAX>(v, dpp64<kDppHalfMirror>(v));
  v = pick64<MAX>(v, dpp64<kDppMirror>(v));
  return pick64<MAX>(pick64<MAX>(readlane64(v, 0), readlane64(v, 16)), pick64<MAX>(readlane64(v, 32), readlane64(v, 48)));
}

// Block-wide max (MAX) or min of v; every thread returns it. Synchronizes the block.
template <bool MAX, typename S>
__device__ __forceinline__ u64 block_ext64(u64 v, S& s) {
  v = wave_ext64<MAX>(v);
  if (lane_id() == 0) s.red[wave_id()] = v;
  __syncthreads();
  u64 r = s.red[0];
#pragma unroll
  for (int i = 1; i < kWaves; ++i) r = pick64<MAX>(r, s.red[i]);
  __syncthreads();
  return r;
}

// Block-wide sum of a per-lane count; every thread returns it. Synchronizes the block.
template <typename S>
__device__ __forceinline__ int block_count(int v, S& s) {
  const float w = wave_sum((float)v);  // exact: the counts stay far below 2^24
  if (lane_id() == 0) s.wsum[wave_id()] = (unsigned)w;
  __syncthreads();
  unsigned r = 0;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) r += s.wsum[i];
  __syncthreads();
  return (int)r;
}

__device__ __forceinline__ int lanes_below(u64 mask) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

// Appends the lane's composites c with keep to buf: one LDS atomic per wave reserves the wave's total. Returns the
// buffer fill right after the wave's append (0 if it appended nothing); the largest over a block's appends is the
// block's final count.
template <int N, typename S>
__device__ __forceinline__ int append(S& s, const u64 (&c)[N], const bool (&keep)[N]) {
  u64 m[N];
  int total = 0;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    m[i] = __ballot(keep[i]);
    total += __popcll(m[i]);
  }
  if (total == 0) return 0;
  int base = 0;
  if (lane_id() == 0) base = atomicAdd(&s.count, total);
  base = __builtin_amdgcn_readfirstlane(base);
#pragma unroll
  for (int i = 0; i < N; ++i) {
    if (keep[i]) s.buf[base + lanes_below(m[i])] = c[i];
    base += __popcll(m[i]);
  }
  return base;
}

// One narrowing pass: histograms the composites in [lo, hi] (visited through `each`, which calls its argument once per
// composite of this lane) into 256 bins of width 2^sh from lo and moves [lo, hi] to the bin holding the r-th largest
// of the range; r becomes the rank within that bin. Returns the bin's population and adds the composites of the
// higher bins to `above`. Requires lo < hi and 1 <= r <= |[lo, hi]|. Synchronizes the block.
template <typename S, typename Each>
__device__ int narrow(S& s, const Each& each, u64& lo, u64& hi, int& r, int& above) {
  const int t = threadIdx.x;
  const int bits = 64 - __clzll(hi - lo);
  const int sh = bits > 8 ? bits - 8 : 0;
  const u64 l = lo, h = hi;
  s.hist[t] = 0;
  __syncthreads();
  each([&](u64 c) {
    if (c >= l && c <= h) atomicAdd(&s.hist[(int)((c - l) >> sh)], 1u);
  });
  __syncthreads();
  // thread t holds bin 255 - t: the inclusive count of the bins at or above it
  const unsigned mine = s.hist[kBins - 1 - t];
  unsigned incl = mine;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const unsigned o = __shfl_up(incl, d, kWave);
    if (lane_id() >= d) incl += o;
  }
  if (lane_id() == kWave - 1) s.wsum[wave_id()] = incl;
  __syncthreads();
  for (int w = 0; w < wave_id(); ++w) incl += s.wsum[w];
  if ((int)incl >= r && (int)(incl - mine) < r) {
    s.bin = kBins - 1 - t;
    s.above = (int)(incl - mine);
  }
  __syncthreads();
  const int b = s.bin;
  const int higher = s.above;
  const int pop = (int)s.hist[b];
  __syncthreads();
  r -= higher;
  above += higher;
  lo = l + ((u64)b << sh);
  const u64 top = lo + (((u64)1 << sh) - 1);
  hi = (b + 1 < kBins && top < h) ? top : h;
  return pop;
}

// The exact k-th largest of the n distinct composites buf[0, n) (1 <= k <= n). Every thread returns it; the block is
// synchronized on entry and return.
template <typename S>
__device__ u64 kth_largest(S& s, int n, int k) {
  const int t = threadIdx.x;
  auto each = [&](auto f) {
    for (int i = t; i < n; i += kThreads) f(s.buf[i]);
  };
  u64 mx = 0, mn = ~0ull;
  each([&](u64 c) {
    mx = c > mx ? c : mx;
    mn = c < mn ? c : mn;
  });
  u64 hi = block_ext64<true>(mx, s), lo = block_ext64<false>(mn, s);
  int r = k, above = 0;
  while (lo < hi) {
    if (r == 1) {
      u64 v = 0;
      each([&](u64 c) { v = (c >= lo && c <= hi && c > v) ? c : v; });
      return block_ext64<true>(v, s);
    }
    const int pop = narrow(s, each, lo, hi, r, above);
    if (pop == r) {  // every composite of the bin is wanted: the k-th is the bin's smallest
      u64 v = ~0ull;
      each([&](u64 c) { v = (c >= lo && c <= hi && c < v) ? c : v; });
      return block_ext64<false>(v, s);
    }
  }
  return lo;
}

// Keeps the composites >= floor of buf[0, n) in place (order not kept); returns their number. Rounds of 4 composites
// per lane: a round's survivors land below every composite not yet read.
template <typename S>
__device__ int keep_at_least(S& s, int n, u64 floor) {
  __syncthreads();
  if (threadIdx.x == 0) s.count = 0;
  __syncthreads();
  for (int r = 0; r < n; r += 4 * kThreads) {
    u64 c[4];
    bool keep[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = r + j * kThreads + (int)threadIdx.x;
      c[j] = i < n ? s.buf[i] : 0ull;
      keep[j] = i < n && c[j] >= floor;
    }
    __syncthreads();
    append<4>(s, c, keep);
    __syncthreads();
  }
  return s.count;
}

// Prunes the buffer to its k largest when it holds more, and raises the admission threshold to the k-th.
template <typename S>
__device__ void prune(S& s, int k) {
  __syncthreads();
  const int n = s.count;
  if (n <= k) return;
  const u64 kth = kth_largest(s, n, k);
  keep_at_least(s, n, kth);
  if (threadIdx.x == 0 && kth > s.thr) s.thr = kth;
  __syncthreads();
}

// Sorts buf[0, n) descending (bitonic over the next power of two >= 64, padded with 0).
template <typename S>
__device__ void sort_desc(S& s, int n) {
  int m = 64;
  while (m < n) m <<= 1;
  for (int i = n + (int)threadIdx.x; i < m; i += kThreads) s.buf[i] = 0ull;
  __syncthreads();
  for (int size = 2; size <= m; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = threadIdx.x; i < (m >> 1); i += kThreads) {
        const int lo = ((i & ~(stride - 1)) << 1) | (i & (stride - 1)), hi = lo + stride;
        const u64 a = s.buf[lo], b = s.buf[hi];
        const bool desc = (lo & size) == 0;
        if (desc ? a < b : a > b) {
          s.buf[lo] = b;
          s.buf[hi] = a;
        }
      }
      __syncthreads();
    }
  }
}

template <typename T> struct Fmt;
template <> struct Fmt<float> { static constexpr int W = 4; };      // elements per 16-byte vector
template <> struct Fmt<uint16_t> { static constexpr int W = 8; };

template <typename T>
__device__ __forceinline__ void write_outputs(void* values, long long* indices, long long row, int k, const u64* buf,
                                              int n) {
  for (int j = threadIdx.x; j < k; j += kThreads) {
    const u64 c = j < n ? buf[j] : 0ull;
    if constexpr (sizeof(T) == 4) static_cast<uint32_t*>(values)[row * k + j] = composite_bits(c);
    else static_cast<uint16_t*>(values)[row * k + j] = (uint16_t)(composite_bits(c) >> 16);
    indices[row * k + j] = composite_index(c);
  }
}

// ---- chunk kernel ----------------------------------------------------------------------------------------------------

// A register block: lane t of LANES holds vectors v * LANES + t (v < NV) of elements [b0, b1) of a row, W elements
// each.
template <typename T, bool VEC, int E, int LANES = kThreads>
struct Block {
  static constexpr int W = Fmt<T>::W;
  static constexpr int NV = E / W;
  static_assert(NV * W == E, "E must be a multiple of the vector width");
  u32x4 r[NV];
  int b0, b1;  // element offsets within the row (cols <= INT_MAX / 2)

  __device__ __forceinline__ void load(const T* row) {
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const int e0 = b0 + (v * LANES + (int)threadIdx.x) * W;
      if constexpr (VEC) {
        const int e = e0 < b1 ? e0 : b1 - W;  // an in-range duplicate, skipped by each_vec()
        r[v] = load16<true>(row + e, 0);
      } else {
        uint32_t u[W];
#pragma unroll
        for (int j = 0; j < W; ++j) {
          const int e = e0 + j;
          if constexpr (sizeof(T) == 4) u[j] = e < b1 ? reinterpret_cast<const uint32_t*>(row)[e] : 0u;
          else u[j] = e < b1 ? (uint32_t)reinterpret_cast<const uint16_t*>(row)[e] : 0u;
        }
        if constexpr (sizeof(T) == 4) r[v] = (u32x4){u[0], u[1], u[2], u[3]};
        else r[v] = (u32x4){u[0] | (u[1] << 16), u[2] | (u[3] << 16), u[4] | (u[5] << 16), u[6] | (u[7] << 16)};
      }
    }
  }

  // f(c, ok) for each vector of this lane: c[W] its composites, ok[W] whether each element lies in [b0, b1). Each call
  // recomputes the composites from the raw registers: the empty asm makes them opaque, so the compiler does not keep
  // E 64-bit composites alive across the selection passes.
  template <typename F>
  __device__ __forceinline__ void each_vec(F f) {
#pragma unroll
    for (int v = 0; v < NV; ++v) asm volatile("" : "+v"(r[v]));
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const int e0 = b0 + (v * LANES + (int)threadIdx.x) * W;
      const bool vin = e0 < b1;
      const uint32_t i0 = (uint32_t)e0;
      u64 c[W];
      bool ok[W];
#pragma unroll
      for (int j = 0; j < W; ++j) {
        uint32_t u;
        if constexpr (sizeof(T) == 4) {
          u = r[v][j];
        } else {
          const uint32_t w = r[v][j >> 1];
          u = (j & 1) ? (w & 0xffff0000u) : (w << 16);
        }
        ok[j] = VEC ? vin : (e0 + j < b1);
        c[j] = composite(u, i0 + (uint32_t)j);
      }
      f(c, ok);
    }
  }

  // f(composite) for every element of this lane in [b0, b1).
  template <typename F>
  __device__ __forceinline__ void each(F f) {
    each_vec([&](const u64 (&c)[W], const bool (&ok)[W]) {
#pragma unroll
      for (int j = 0; j < W; ++j)
        if (ok[j]) f(c[j]);
    });
  }
};

// Admits the block's top-k composites (among those >= the buffer's threshold) into the buffer, which holds at most k
// on entry: exactly the block's top-k, or a superset of them when it fits beside the kept k.
template <typename S, typename B>
__device__ void admit_block(S& s, B& blk, int k) {
  // lane maximum; for k <= 64 the wave's seed is the k-th largest of its lane maxima (k distinct elements at or above)
  u64 m = 0;
  blk.each([&](u64 c) { m = c > m ? c : m; });
  u64 seed = 1;
  if (k == 1) {
    seed = wave_ext64<true>(m);
  } else if (k <= kSeedMaxK) {
    int rank = 0;
#pragma unroll 8
    for (int j = 0; j < kWave; ++j) rank += readlane64(m, j) > m;
    const u64 hit = __ballot(m != 0 && rank == k - 1);
    if (hit) seed = readlane64(m, (int)__builtin_ctzll(hit));
  }
  const u64 hi = block_ext64<true>(m, s);
  const u64 seed_blk = block_ext64<true>(seed, s);
  u64 lo = seed_blk > s.thr ? seed_blk : s.thr;
  if (hi < lo) return;  // nothing here reaches the buffer's k-th
  int n = 0;
  blk.each([&](u64 c) { n += c >= lo; });
  n = block_count(n, s);
  int r = k < n ? k : n, above = 0;
  u64 h = hi;
  // narrow until the composites >= lo fit beside the buffer; [lo, h] keeps the block's r-th largest of the range
  while (s.count + n > kChunkBuf && lo < h) {
    const int pop = narrow(s, [&](auto f) { blk.each(f); }, lo, h, r, above);
    n = above + pop;
  }
  const u64 floor = lo;
  blk.each_vec([&](const u64 (&c)[B::W], const bool (&ok)[B::W]) {
    bool keep[B::W];
    bool any = false;
#pragma unroll
    for (int j = 0; j < B::W; ++j) {
      keep[j] = ok[j] && c[j] >= floor;
      any |= keep[j];
    }
    if (__ballot(any)) append<B::W>(s, c, keep);
  });
  __syncthreads();
}

template <typename T, bool VEC, int E>
__global__ void __launch_bounds__(kThreads)
    topk_chunks(const T* __restrict__ x, void* __restrict__ values, long long* __restrict__ indices,
                u64* __restrict__ work, long long cols, long long chunk, int nchunks, int k) {
  __shared__ Smem<kChunkBuf> s;
  const long long row = blockIdx.y;
  const int part = blockIdx.x;
  const int begin = (int)((long long)part * chunk);
  const int end = (int)(begin + chunk < cols ? begin + chunk : cols);
  const T* xr = x + row * cols;
  if (threadIdx.x == 0) {
    s.count = 0;
    s.thr = 1;
  }
  __syncthreads();
  constexpr int CH = kThreads * E;
  for (int b0 = begin; b0 < end; b0 += CH) {
    Block<T, VEC, E> blk;
    blk.b0 = b0;
    blk.b1 = end - b0 > CH ? b0 + CH : end;
    blk.load(xr);
    prune(s, k);  // at most k kept, threshold at the k-th
    admit_block(s, blk, k);
  }
  prune(s, k);
  const int n = s.count;
  if (nchunks == 1) {
    sort_desc(s, n);
    write_outputs<T>(values, indices, row, k, s.buf, n);
    return;
  }
  // the list with its smallest composite first (0 first when the chunk holds fewer than k elements)
  u64 mn = ~0ull;
  for (int j = threadIdx.x; j < k; j += kThreads) {
    const u64 v = j < n ? s.buf[j] : 0ull;
    mn = v < mn ? v : mn;
  }
  mn = block_ext64<false>(mn, s);
  if (threadIdx.x == 0) s.bin = 0;
  __syncthreads();
  for (int j = threadIdx.x; j < n; j += kThreads)
    if (s.buf[j] == mn) s.bin = j;
  __syncthreads();
  const int at = n < k ? n : s.bin;
  u64* wr = work + (row * nchunks + part) * (long long)k;
  for (int j = threadIdx.x; j < k; j += kThreads) {
    u64 v;
    if (j == 0) v = at < n ? s.buf[at] : 0ull;
    else if (j == at) v = s.buf[0];
    else v = j < n ? s.buf[j] : 0ull;
    wr[j] = v;
  }
}

// ---- wave kernels (k <= 64) ---------------------------------------------------------------------------------------

constexpr int kWaveCap = 512;                // wave-private candidate list (4 KB of LDS)
constexpr int kWaveM = kWaveCap / kWave;     // list entries per lane while pruning (held in registers)
constexpr int kWaveE = 32;                   // elements per lane per register block
constexpr int kWaveSub = kWave * kWaveE;     // 2048 elements per register block
constexpr int kWavePruneAt = kWaveCap / 2;   // prune after a block that leaves more than this

// Order-preserving 32-bit key of fp32 bits u (the upper half of a composite).
__device__ __forceinline__ uint32_t key_of(uint32_t u) { return u ^ ((uint32_t)((int32_t)u >> 31) | 0x80000000u); }

// The k-th largest (1 <= k <= the number of lanes with ok) of the wave's 32-bit values v (one per lane): a bitwise
// search from the highest bit where the valid minimum and maximum differ, keeping the largest prefix with at least k
// values at or above it (counted with ballots). Wave-uniform.
__device__ __forceinline__ uint32_t wave_kth32(uint32_t v, bool ok, int k) {
  const uint32_t mx = (uint32_t)wave_ext64<true>(ok ? v : 0u);
  const uint32_t mn = (uint32_t)wave_ext64<false>(ok ? v : 0xffffffffu);
  if (mx == mn) return mx;
  const int top = 31 - __builtin_clz(mx ^ mn);
  uint32_t p = mx & ~((2u << top) - 1u);
  for (int b = top; b >= 0; --b) {
    const uint32_t cand = p | (1u << b);
    if (__popcll(__ballot(ok && v >= cand)) >= k) p = cand;
  }
  return p;
}

// A wave's candidate list: composites buf[0, count) in LDS (count wave-uniform) and the admission key (composites
// whose key is below it cannot reach the row's top k). The row's waves share admission keys through a per-row word
// (`shared`, an atomic maximum): any wave's k-th key bounds the row's k-th key from below.
struct WaveList {
  u64* buf;
  int count;
  uint32_t thr_key;

  // Appends c where keep (positions from a ballot; no atomics).
  __device__ __forceinline__ void push(u64 c, bool keep) {
    const u64 m = __ballot(keep);
    if (keep) buf[count + lanes_below(m)] = c;
    count += __popcll(m);
  }

  // Keeps exactly the k largest (when more are held) and raises thr_key to the k-th's key. The list is held in
  // registers (8 per lane) for a bitwise search of the k-th key from the common prefix of the keys' range, then, only
  // when equal keys straddle it, of the k-th lower word (~index) among them; then it is rewritten in place.
  __device__ __forceinline__ void prune(int k) {
    __syncthreads();  // one-wave workgroup: orders the list's LDS writes before these reads
    if (count <= k) return;
    u64 v[kWaveM];
    bool ok[kWaveM];
    uint32_t kmx = 0, kmn = 0xffffffffu;
#pragma unroll
    for (int i = 0; i < kWaveM; ++i) {
      const int at = i * kWave + lane_id();
      ok[i] = at < count;
      v[i] = ok[i] ? buf[at] : 0ull;
      const uint32_t kk = (uint32_t)(v[i] >> 32);
      kmx = ok[i] && kk > kmx ? kk : kmx;
      kmn = ok[i] && kk < kmn ? kk : kmn;
    }
    kmx = (uint32_t)wave_ext64<true>(kmx);
    kmn = (uint32_t)wave_ext64<false>(kmn);
    uint32_t K = kmx;
    if (kmx != kmn) {
      const int top = 31 - __builtin_clz(kmx ^ kmn);
      K = kmx & ~((2u << top) - 1u);
      for (int b = top; b >= 0; --b) {
        const uint32_t cand = K | (1u << b);
        int cnt = 0;
#pragma unroll
        for (int i = 0; i < kWaveM; ++i) cnt += __popcll(__ballot(ok[i] && (uint32_t)(v[i] >> 32) >= cand));
        if (cnt >= k) K = cand;
      }
    }
    int gt = 0, eq = 0;
    uint32_t lmx = 0, lmn = 0xffffffffu;
#pragma unroll
    for (int i = 0; i < kWaveM; ++i) {
      const uint32_t kk = (uint32_t)(v[i] >> 32), lw = (uint32_t)v[i];
      const bool e = ok[i] && kk == K;
      gt += __popcll(__ballot(ok[i] && kk > K));
      eq += __popcll(__ballot(e));
      lmx = e && lw > lmx ? lw : lmx;
      lmn = e && lw < lmn ? lw : lmn;
    }
    lmx = (uint32_t)wave_ext64<true>(lmx);
    lmn = (uint32_t)wave_ext64<false>(lmn);
    const int r = k - gt;  // 1 <= r <= eq
    uint32_t L = lmn;
    if (r < eq) {
      const int top = 31 - __builtin_clz(lmx ^ lmn);
      L = lmx & ~((2u << top) - 1u);
      for (int b = top; b >= 0; --b) {
        const uint32_t cand = L | (1u << b);
        int cnt = 0;
#pragma unroll
        for (int i = 0; i < kWaveM; ++i)
          cnt += __popcll(__ballot(ok[i] && (uint32_t)(v[i] >> 32) == K && (uint32_t)v[i] >= cand));
        if (cnt >= r) L = cand;
      }
    }
    const u64 kth = ((u64)K << 32) | L;
    __syncthreads();
    count = 0;
#pragma unroll
    for (int i = 0; i < kWaveM; ++i) push(v[i], ok[i] && v[i] >= kth);
    thr_key = K > thr_key ? K : thr_key;
    __syncthreads();
  }

  // Writes the list (at most k <= 64 composites, one per lane) as a sorted output row or as a workspace list whose
  // smallest composite comes first (0 first when fewer than k are held).
  template <typename T>
  __device__ __forceinline__ void finish(void* values, long long* indices, u64* wr, long long row, int k,
                                         bool to_output) {
    __syncthreads();
    const int n = count;
    const int lane = lane_id();
    const u64 mine = lane < n ? buf[lane] : 0ull;
    if (to_output) {
      int rank = 0;
      for (int j = 0; j < n; ++j) rank += readlane64(mine, j) > mine;
      if (lane < n) {
        if constexpr (sizeof(T) == 4) static_cast<uint32_t*>(values)[row * k + rank] = composite_bits(mine);
        else static_cast<uint16_t*>(values)[row * k + rank] = (uint16_t)(composite_bits(mine) >> 16);
        indices[row * k + rank] = composite_index(mine);
      }
      return;
    }
    const u64 mn = wave_ext64<false>(lane < n ? mine : ~0ull);
    const int at = n < k ? n : (int)__builtin_ctzll(__ballot(lane < n && mine == mn));
    const u64 first_val = readlane64(mine, 0);
    const u64 at_val = at < n ? readlane64(mine, at) : 0ull;
    if (lane < k) wr[lane] = lane == 0 ? at_val : (lane == at ? first_val : (lane < n ? mine : 0ull));
  }
};

struct ListState {
  int count;
  uint32_t thr_key;
};

// The rare path: admits the row's elements [e0, e1) with key >= the admission key straight from memory, 64 at a time,
// pruning whenever the next 64 might not fit. Elements of [e0, e0 + 64 w) whose offset modulo w is below `done` were
// admitted already and are skipped. Out of line, so its code exists once.
template <typename T>
__device__ __noinline__ ListState admit_range(u64* buf, ListState st, const T* row, int e0, int e1, int w, int done,
                                              int k) {
  WaveList L;
  L.buf = buf;
  L.count = st.count;
  L.thr_key = st.thr_key;
  const int skip_end = e0 + kWave * w;
  for (int base = e0; base < e1; base += kWave) {
    if (L.count > kWaveCap - kWave) L.prune(k);
    const int e = base + lane_id();
    const bool ok = e < e1 && !(e < skip_end && (e - e0) % w < done);
    uint32_t u = 0;
    if (ok) {
      if constexpr (sizeof(T) == 4) u = reinterpret_cast<const uint32_t*>(row)[e];
      else u = (uint32_t)reinterpret_cast<const uint16_t*>(row)[e] << 16;
    }
    const uint32_t kk = key_of(u);
    L.push(((u64)kk << 32) | (u64)(~(uint32_t)e), ok && kk >= L.thr_key);
  }
  return ListState{L.count, L.thr_key};
}

// A register block of one wave: lane t holds vectors v * 64 + t (v < NV) of elements [b0, b1) of a row, W each;
// vector v covers the contiguous elements [b0 + 64 W v, b0 + 64 W (v + 1)).
template <typename T, bool VEC>
struct WaveBlock {
  static constexpr int W = Fmt<T>::W;
  static constexpr int NV = kWaveE / W;
  u32x4 r[NV];
  int b0, b1;

  __device__ __forceinline__ int first(int v) const { return b0 + (v * kWave + lane_id()) * W; }
  __device__ __forceinline__ bool valid(int v, int j) const { return VEC ? first(v) < b1 : first(v) + j < b1; }
  __device__ __forceinline__ uint32_t key(int v, int j) const {
    uint32_t u;
    if constexpr (sizeof(T) == 4) {
      u = r[v][j];
    } else {
      const uint32_t w = r[v][j >> 1];
      u = (j & 1) ? (w & 0xffff0000u) : (w << 16);
    }
    return key_of(u);
  }
  // Loads vector v of the block [nb0, nb1) (an in-range duplicate when nb0 >= nb1: loaded, never used).
  __device__ __forceinline__ void load_vec(const T* row, int v, int nb0, int nb1) {
    const int e0 = nb0 + (v * kWave + lane_id()) * W;
    if constexpr (VEC) {
      const int last = nb1 - W;
      r[v] = load16<true>(row + (e0 < nb1 ? e0 : (last > 0 ? last : 0)), 0);
    } else {
      uint32_t u[W];
#pragma unroll
      for (int j = 0; j < W; ++j) {
        const int e = e0 + j;
        if constexpr (sizeof(T) == 4) u[j] = e < nb1 ? reinterpret_cast<const uint32_t*>(row)[e] : 0u;
        else u[j] = e < nb1 ? (uint32_t)reinterpret_cast<const uint16_t*>(row)[e] : 0u;
      }
      if constexpr (sizeof(T) == 4) r[v] = (u32x4){u[0], u[1], u[2], u[3]};
      else r[v] = (u32x4){u[0] | (u[1] << 16), u[2] | (u[3] << 16), u[4] | (u[5] << 16), u[6] | (u[7] << 16)};
    }
  }
};

__device__ __forceinline__ uint32_t load_shared_key(const unsigned* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void publish_key(unsigned* p, uint32_t key) {
  if (lane_id() == 0) __hip_atomic_fetch_max(p, key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// k <= 64: one 64-lane workgroup (one wave) per (chunk, row). The wave streams its chunk in register blocks of 2048
// elements through a single register set: as soon as a 16-byte slice has been filtered, its registers load the same
// slice of the next block, so the next block is in flight while the rest of this one is filtered. Admission compares
// 32-bit keys against the admission key -- the largest of the wave's own bound, the first block's lane-maxima seed
// (the k-th largest lane maximum has k distinct elements at or above it) and the row's shared word, which every wave
// of the row raises to its k-th key -- and builds composites only for admitted elements. `shared` (the caller's
// per-row counter, zero on entry) is left at the row's bound; the merge (or the single wave of an unsplit row)
// zeroes it.
template <typename T, bool VEC>
__global__ void __launch_bounds__(kWave)
    topk_wave(const T* __restrict__ x, void* __restrict__ values, long long* __restrict__ indices,
              u64* __restrict__ work, unsigned* __restrict__ shared, long long cols, long long chunk, int nchunks,
              int k) {
  __shared__ u64 list[kWaveCap];
  const long long row = blockIdx.y;
  const int part = blockIdx.x;
  const int begin = (int)((long long)part * chunk);
  const int end = (int)(begin + chunk < cols ? begin + chunk : cols);
  const T* xr = x + row * cols;
  unsigned* row_key = shared + row;
  WaveList L;
  L.buf = list;
  L.count = 0;
  L.thr_key = 0u;
  using B = WaveBlock<T, VEC>;
  B blk;
  blk.b0 = begin;
  blk.b1 = end - begin > kWaveSub ? begin + kWaveSub : end;
#pragma unroll
  for (int v = 0; v < B::NV; ++v) blk.load_vec(xr, v, blk.b0, blk.b1);
  bool seeded = false;
  uint32_t row_bound = load_shared_key(row_key);
  while (true) {
    if (!seeded) {
      uint32_t m = 0;
      bool has = false;
#pragma unroll
      for (int v = 0; v < B::NV; ++v)
#pragma unroll
        for (int j = 0; j < B::W; ++j)
          if (blk.valid(v, j)) {
            const uint32_t kk = blk.key(v, j);
            m = kk > m ? kk : m;
            has = true;
          }
      if (__popcll(__ballot(has)) >= k) {
        const uint32_t seed = wave_kth32(m, has, k);
        L.thr_key = seed > L.thr_key ? seed : L.thr_key;
        publish_key(row_key, seed);
        seeded = true;
      }
    }
    L.thr_key = row_bound > L.thr_key ? row_bound : L.thr_key;
    row_bound = load_shared_key(row_key);  // used at the next block (in flight meanwhile)
    const uint32_t thr = L.thr_key;
    const int nb0 = blk.b1, nb1 = end - nb0 > kWaveSub ? nb0 + kWaveSub : end;
    bool slow = false;
#pragma unroll
    for (int v = 0; v < B::NV; ++v) {
      // four elements per lane (256 per wave) at a time, so that a group always fits when its check passes
#pragma unroll
      for (int g = 0; g < B::W; g += 4) {
        if (!slow) {
          if (L.count > kWaveCap - 4 * kWave) {
            // the group might not fit: admit the rest of the block from memory, pruning as it goes
            const ListState st = admit_range<T>(list, ListState{L.count, L.thr_key}, xr, blk.b0 + v * kWave * B::W,
                                                blk.b1, B::W, g, k);
            L.count = st.count;
            L.thr_key = st.thr_key;
            slow = true;
          } else {
            bool any = false;
#pragma unroll
            for (int j = g; j < g + 4; ++j) any |= blk.valid(v, j) && blk.key(v, j) >= thr;
            if (__ballot(any)) {
#pragma unroll
              for (int j = g; j < g + 4; ++j) {
                const uint32_t kk = blk.key(v, j);
                L.push(((u64)kk << 32) | (u64)(~(uint32_t)(blk.first(v) + j)), blk.valid(v, j) && kk >= thr);
              }
            }
          }
        }
      }
      blk.load_vec(xr, v, nb0, nb1);
    }
    if (L.count > kWavePruneAt) {
      L.prune(k);
      publish_key(row_key, L.thr_key);
    }
    if (nb0 >= end) break;
    blk.b0 = nb0;
    blk.b1 = nb1;
  }
  L.prune(k);
  if (nchunks == 1 && lane_id() == 0)  // the row's only wave: leave the counter zero
    __hip_atomic_store(row_key, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  L.finish<T>(values, indices, work + (row * nchunks + part) * (long long)k, row, k, nchunks == 1);
}

// k <= 64 merge: one wave per split row streams the row's nchunks lists (k composites each, smallest first) through
// its list from the largest list minimum, writes the sorted row and zeroes the row's shared word.
template <typename T>
__global__ void __launch_bounds__(kWave)
    topk_merge_wave(void* __restrict__ values, long long* __restrict__ indices, const u64* __restrict__ work,
                    unsigned* __restrict__ shared, int nchunks, int k) {
  __shared__ u64 list[kWaveCap];
  const long long row = blockIdx.x;
  const u64* wr = work + row * (long long)nchunks * k;
  u64 fl = 0;
  for (int c = lane_id(); c < nchunks; c += kWave) {
    const u64 v = wr[(long long)c * k];
    fl = v > fl ? v : fl;
  }
  fl = wave_ext64<true>(fl);
  const u64 floor = fl > 1 ? fl : 1;
  WaveList L;
  L.buf = list;
  L.count = 0;
  L.thr_key = shared[row];  // the row's bound: every top-k key is at least this
  const int total = nchunks * k;
  for (int base = 0; base < total; base += 4 * kWave) {
    u64 c[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = base + j * kWave + lane_id();
      c[j] = i < total ? wr[i] : 0ull;
    }
    if (L.count > kWaveCap - 4 * kWave) L.prune(k);
#pragma unroll
    for (int j = 0; j < 4; ++j) L.push(c[j], c[j] >= floor && (uint32_t)(c[j] >> 32) >= L.thr_key);
  }
  L.prune(k);
  __syncthreads();
  if (lane_id() == 0) shared[row] = 0u;
  L.finish<T>(values, indices, nullptr, row, k, true);
}

// ---- merge kernel ----------------------------------------------------------------------------------------------------

template <typename T>
__global__ void __launch_bounds__(kThreads)
    topk_merge(void* __restrict__ values, long long* __restrict__ indices, const u64* __restrict__ work, int nchunks,
               int k) {
  __shared__ Smem<kMergeBuf> s;
  const long long row = blockIdx.x;
  const u64* wr = work + row * (long long)nchunks * k;
  // floor: the largest chunk minimum (slot 0 of each list)
  u64 fl = 0;
  for (int c = threadIdx.x; c < nchunks; c += kThreads) {
    const u64 v = wr[(long long)c * k];
    fl = v > fl ? v : fl;
  }
  fl = block_ext64<true>(fl, s);
  if (threadIdx.x == 0) {
    s.count = 0;
    s.thr = fl > 1 ? fl : 1;
  }
  __syncthreads();
  const long long total = (long long)nchunks * k;
  for (long long t0 = 0; t0 < total; t0 += kMergeTile) {
    const u64 thr = s.thr;
    u64 c[kMergePer];
    bool keep[kMergePer];
    bool any = false;
#pragma unroll
    for (int j = 0; j < kMergePer; ++j) {
      const long long i = t0 + (long long)j * kThreads + (int)threadIdx.x;
      c[j] = i < total ? wr[i] : 0ull;
      keep[j] = c[j] >= thr;
      any |= keep[j];
    }
    int fill = 0;
    if (__ballot(any)) fill = append<kMergePer>(s, c, keep);
    // one block-wide decision per tile (every wave branches alike even if one has moved on to the next tile)
    if (__syncthreads_or(fill > kMergeBuf - kMergeTile)) prune(s, k);
  }
  prune(s, k);
  const int n = s.count;
  sort_desc(s, n);
  write_outputs<T>(values, indices, row, k, s.buf, n);
}

// ---- host side -------------------------------------------------------------------------------------------------------

// Tuning slots (0 = automatic): 0 resident workgroups per CU assumed by plan(), 1 elements per lane of a register
// block (16, 32 or 64).
enum { kTuneBlocksPerCu = 0, kTuneE = 1 };
constexpr int kDefaultE = 32;

int lane_elems() {
  const int e = rw_host::tune_get(kTuneE);
  return (e == 16 || e == 32 || e == 64) ? e : kDefaultE;
}

template <typename T, bool VEC>
int launch_chunks(const void* x, void* values, void* indices, void* work, void* counters, long long rows,
                  long long cols, long long chunk, int nchunks, int k, hipStream_t stream) {
  const dim3 grid((unsigned)nchunks, (unsigned)rows);
  const int e = VEC ? lane_elems() : 16;
  if (k <= kSeedMaxK)
    hipLaunchKernelGGL((topk_wave<T, VEC>), grid, dim3(kWave), 0, stream, (const T*)x, values, (long long*)indices,
                       (u64*)work, (unsigned*)counters, cols, chunk, nchunks, k);
  else if (e == 16)
    hipLaunchKernelGGL((topk_chunks<T, VEC, 16>), grid, dim3(kThreads), 0, stream, (const T*)x, values,
                       (long long*)indices, (u64*)work, cols, chunk, nchunks, k);
  else if (e == 64)
    hipLaunchKernelGGL((topk_chunks<T, VEC, 64>), grid, dim3(kThreads), 0, stream, (const T*)x, values,
                       (long long*)indices, (u64*)work, cols, chunk, nchunks, k);
  else
    hipLaunchKernelGGL((topk_chunks<T, VEC, 32>), grid, dim3(kThreads), 0, stream, (const T*)x, values,
                       (long long*)indices, (u64*)work, cols, chunk, nchunks, k);
  if (nchunks > 1) {
    if (k <= kSeedMaxK)
      hipLaunchKernelGGL((topk_merge_wave<T>), dim3((unsigned)rows), dim3(kWave), 0, stream, values,
                         (long long*)indices, (const u64*)work, (unsigned*)counters, nchunks, k);
    else
      hipLaunchKernelGGL((topk_merge<T>), dim3((unsigned)rows), dim3(kThreads), 0, stream, values,
                         (long long*)indices, (const u64*)work, nchunks, k);
  }
  return (int)hipGetLastError();
}

}  // namespace

// topk/kernel.cu:520 `plan`: the chunk length (columns per workgroup) for a rows x cols launch, chosen so the grid of
// chunks fills the GPU's resident slots once (CUs x resident one-wave workgroups of the k <= 64 kernel per CU), never
// shorter than max(min_chunk, 2048); a multiple of 8 when a row is split. The caller's min_chunk carries the k
// dependence (larger k, longer chunks: fewer lists of k to merge). `threads` and `depth` are the reference's CUDA
// tuning knobs, accepted and not used.
extern "C" long long plan(long long rows, long long cols, int dtype, int threads, int depth, int min_chunk) {
  (void)threads;
  (void)depth;
  if (rows <= 0 || cols <= 0) return cols > 0 ? cols : 1;
  static int occ[2] = {0, 0};
  const int d = dtype == 1 ? 1 : 0;
  int per_cu = rw_host::tune_get(kTuneBlocksPerCu);
  if (per_cu <= 0) {
    if (occ[d] <= 0) {
      int n = 0;
      const hipError_t e = d ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, topk_wave<uint16_t, true>, kWave, 0)
                             : hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, topk_wave<float, true>, kWave, 0);
      if (e != hipSuccess || n <= 0) {
        (void)hipGetLastError();
        n = 8;
      }
      occ[d] = n;
    }
    per_cu = occ[d];
  }
  long long len = min_chunk > kWaveSub ? min_chunk : kWaveSub;
  const long long slots = (long long)rw_host::device_cus() * per_cu;
  long long per_row = slots / rows;
  if (per_row < 1) per_row = 1;
  const long long fill = (cols + per_row - 1) / per_row;
  if (fill > len) len = fill;
  if (len >= cols) return cols;
  return (len + 7) / 8 * 8;
}

// topk/kernel.cu:549 `launch`: values [rows, k] in x's dtype and int64 indices [rows, k], sorted descending with ties
// by the lowest index. work: u64 [rows * nchunks * k] with nchunks = ceil(cols / chunk), used when nchunks > 1;
// counters: u32 [>= rows], zero on entry and left zero (the two-kernel hand-off does not touch them). Checks as the
// reference's, except that k may be up to 1024 (the reference stops at 512): rows <= 0 or k <= 0 is a no-op; -1 for
// k > cols, k > 1024, cols > INT_MAX / 2, rows > 65535, chunk <= 0, a split row with chunk % 4 or
// nchunks * k > INT_MAX / 2, threads not 128, 256 or 512, depth not 2, 4 or 8, or a dtype other than 0 and 1.
extern "C" int launch(const void* x, void* values, void* indices, void* work, void* counters, long long rows,
                      long long cols, int k, int dtype, int threads, int depth, long long chunk, hipStream_t stream) {
  if (rows <= 0 || k <= 0) return rw_host::kOk;
  if (k > cols || k > kMaxK || cols > INT_MAX / 2 || rows > 65535 || chunk <= 0) return rw_host::kInvalid;
  const long long nchunks = (cols + chunk - 1) / chunk;
  if (nchunks > 1 && (chunk % 4 || nchunks * k > INT_MAX / 2)) return rw_host::kInvalid;
  if ((threads != 128 && threads != 256 && threads != 512) || (depth != 2 && depth != 4 && depth != 8))
    return rw_host::kInvalid;
  if (dtype == 0) {
    if (cols % 4 == 0 && rw_host::aligned16(x))
      return launch_chunks<float, true>(x, values, indices, work, counters, rows, cols, chunk, (int)nchunks, k, stream);
    return launch_chunks<float, false>(x, values, indices, work, counters, rows, cols, chunk, (int)nchunks, k, stream);
  }
  if (dtype == 1) {
    if (cols % 8 == 0 && (chunk % 8 == 0 || nchunks == 1) && rw_host::aligned16(x))
      return launch_chunks<uint16_t, true>(x, values, indices, work, counters, rows, cols, chunk, (int)nchunks, k, stream);
    return launch_chunks<uint16_t, false>(x, values, indices, work, counters, rows, cols, chunk, (int)nchunks, k, stream);
  }
  return rw_host::kInvalid;
}

// No counterpart in the reference (whose counters self-reset only when a launch completes): zeroes counters[0, rows)
// on `stream`. This build leaves the counters untouched, so the call only restores a caller's invariant.
extern "C" int topk_reset(void* counters, long long rows, hipStream_t stream) {
  if (rows <= 0) return rw_host::kOk;
  if (!counters) return rw_host::kInvalid;
  return (int)hipMemsetAsync(counters, 0, (size_t)rows * sizeof(unsigned), stream);
}

extern "C" int topk_tune(int slot, int value) { return rw_host::tune_set(slot, value); }
