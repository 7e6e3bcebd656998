// Row-wise top-k (largest, sorted descending, ties broken by the lowest index) of x[rows, cols] in fp32 (dtype 0) or
// bf16 (dtype 1), behind the reference's C-ABI `plan` and `launch` (topk/kernel.cu:520-570), for 1 <= k <= 1024.
//
// Order (topk/kernel.cu:1-3, :56-60): every element is ranked by the 64-bit composite (key << 32) | ~index, key = ~u
// for a set sign bit and u | 0x80000000 otherwise (u the fp32 bits; a bf16 element is widened first). Composites are
// distinct, a larger one comes first, and composite 0 means "no element". Values are decoded from the composites bit
// for bit, so x is read once.
//
// k <= 64: topk_tile, one kernel (see its comment); the row's last workgroup merges the chunk lists, handed over
// through device-coherent stores and loads and a per-row arrival counter, as the reference's last-block merge. k = 1
// is a kernel of its own, topk_one: each lane's largest composite straight from the registers, 1024-thread workgroups
// over four chunks each, and the same hand-off of one composite per workgroup.
//
// 64 < k <= 1024: topk_wide, one kernel of the same shape (see its comment): a bound from group maxima admits about
// 1.4k elements per tile, the row's last workgroup merges the chunks' candidate lists from a floor made of their
// published bounds, and the output row is ordered by bucketing and ranking in LDS.
#include <climits>
#include <cstdint>
#include <mutex>
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
constexpr int kSeedMaxK = 64;  // the largest k of the tile kernel

template <int CAP>
struct Smem {
  u64 buf[CAP];
  unsigned hist[kBins];
  unsigned wsum[kWaves];
  u64 red[kWaves];
  u64 red2[kWaves];  // reductions of two values at one barrier (with red), and of a second pair (with wsum)
  u64 red3[kWaves];
  u64 red4[kWaves];
  u64 thr;       // admit composites >= thr (>= 1: composite 0 is never admitted)
  int count;     // composites in buf
  int bin;       // narrowing: the bin holding the wanted rank
  int above;     // narrowing: composites in the bins above it
  int last;      // the row's last arrival (split rows of the 64 < k kernel)
  int members;   // bucketed selection: the wanted bucket's members gathered so far
  u64 pick;      // bucketed selection: the k-th largest
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
  return pick64<MAX>(pick64<MAX>(readlane64(v, 0), readlane64(v, 16)),
                     pick64<MAX>(readlane64(v, 32), readlane64(v, 48)));
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

constexpr int kDppRowShr = 0x110;  // + n: row_shr:n, lane l reads lane l - n of its 16-lane row (0 below it)

// Inclusive prefix sum of a u32 over the wave's lanes (lane order): DPP row shifts inside each 16-lane row, then the
// sums of the rows below (lanes 15, 31 and 47) added.
__device__ __forceinline__ uint32_t wave_incl_u32(uint32_t v) {
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, kDppRowShr + 1, 0xF, 0xF, false);
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, kDppRowShr + 2, 0xF, 0xF, false);
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, kDppRowShr + 4, 0xF, 0xF, false);
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, kDppRowShr + 8, 0xF, 0xF, false);
  const uint32_t r0 = (uint32_t)__builtin_amdgcn_readlane((int)v, 15);
  const uint32_t r01 = r0 + (uint32_t)__builtin_amdgcn_readlane((int)v, 31);
  const uint32_t r012 = r01 + (uint32_t)__builtin_amdgcn_readlane((int)v, 47);
  const int wrow = lane_id() >> 4;
  return wrow == 0 ? v : v + (wrow == 1 ? r0 : wrow == 2 ? r01 : r012);
}

// The exclusive prefix over the wave's lanes of a count n in [0, 2^B), and the wave's total in `total`: a ballot per
// bit of n.
template <int B>
__device__ __forceinline__ int wave_excl_count(int n, int& total) {
  int excl = 0, tot = 0;
#pragma unroll
  for (int b = 0; b < B; ++b) {
    const u64 m = __ballot((n >> b) & 1);
    excl += lanes_below(m) << b;
    tot += __popcll(m) << b;
  }
  total = tot;
  return excl;
}

// Appends the lane's composites c with keep to buf, in lane order within each of the N rounds: one LDS atomic per wave
// reserves the positions of all of the wave's kept composites, and each kept lane writes at the reserved base plus
// the kept lanes below it. The buffer's count is s.count once every wave has appended.
template <int N, typename S>
__device__ __forceinline__ void append(S& s, const u64 (&c)[N], const bool (&keep)[N]) {
  u64 m[N];
  int total = 0;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    m[i] = __ballot(keep[i]);
    total += __popcll(m[i]);
  }
  if (total == 0) return;
  int base = 0;
  if (lane_id() == 0) base = atomicAdd(&s.count, total);
  base = __builtin_amdgcn_readfirstlane(base);
#pragma unroll
  for (int i = 0; i < N; ++i) {
    if (keep[i]) s.buf[base + lanes_below(m[i])] = c[i];
    base += __popcll(m[i]);
  }
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
  unsigned incl = wave_incl_u32(mine);
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

// Whether the buffer holds more than `limit` composites, uniform over the workgroup: every wave reads the count before
// any wave goes on (to append, in the loops that call this), so that no wave reads a count another wave has already
// raised and the waves cannot disagree on a prune (whose barriers they would then pair with different barriers).
template <typename S>
__device__ __forceinline__ bool prune_due(S& s, int limit) {
  const bool due = s.count > limit;
  __syncthreads();
  return due;
}

template <typename T> struct Fmt;
template <> struct Fmt<float> { static constexpr int W = 4; };      // elements per 16-byte vector
template <> struct Fmt<uint16_t> { static constexpr int W = 8; };

// ---- tile kernels (k <= 64) ---------------------------------------------------------------------------------------

constexpr int kTileE = 64;      // elements per lane of a register tile (16384 per workgroup)
constexpr int kTileSeg = 512;   // each wave's list segment (composites)
constexpr int kTileKeep = 256;  // a list holding more than this after a batch is pruned to its k largest
constexpr int kTileSort = 256;  // rank-sort capacity (one composite per thread)
static_assert(kTileKeep <= kTileSort && kTileKeep + 4 * kWave <= kTileSeg, "a kept list must fit the rank sort, and a "
              "wave's share of it a step of re-pushes");
static_assert(kTileSort == kThreads, "the rank sort and the merge heads use one composite per thread");

typedef unsigned long long u64x2 __attribute__((ext_vector_type(2)));

constexpr int kStageGroups = 64;  // each wave's staged 8-element groups in a filter pass (Tile::filter_groups)

struct TileSmem {
  u64 seg[kWaves][kTileSeg + 2];  // (+ a spare slot for a batch's writes past the end, padded to 16 bytes)
  u32x4 stage[kWaves][2 * kStageGroups + 2];  // filter_groups: each wave's staged groups, 8 fp32 elements each (+ a
                                              // spare group for the writes past the end)
  uint32_t stage_at[kWaves][kStageGroups + 1];  // and the index of each staged group's first element
  alignas(16) u64 sorted[kTileSort];
  u64 top[kSeedMaxK];  // an output row's composites in order (for the fused draw)
  uint32_t red[2][kWaves];
  int cnt[kWaves];
  alignas(16) uint32_t lm[kThreads];  // a tile's lane maxima (the threshold of a row taken whole)
  uint32_t thr;
  u64 pick;
  int last;
};

// Order-preserving 32-bit key of fp32 bits u (the upper half of a composite).
__device__ __forceinline__ uint32_t key_of(uint32_t u) { return u ^ ((uint32_t)((int32_t)u >> 31) | 0x80000000u); }
// Its inverse: the fp32 bits of key K.
__device__ __forceinline__ uint32_t bits_of(uint32_t K) { return (K & 0x80000000u) ? (K & 0x7fffffffu) : ~K; }

// Wave-wide maximum (MAX) or minimum of a u32; every lane returns it.
template <bool MAX>
__device__ __forceinline__ uint32_t wave_ext32(uint32_t v) {
  auto pick = [](uint32_t a, uint32_t b) { return MAX ? (a > b ? a : b) : (a < b ? a : b); };
  v = pick(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, kDppXor1, 0xF, 0xF, false));
  v = pick(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, kDppXor2, 0xF, 0xF, false));
  v = pick(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, kDppHalfMirror, 0xF, 0xF, false));
  v = pick(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, kDppMirror, 0xF, 0xF, false));
  const uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)v, 0);
  const uint32_t b = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
  const uint32_t c = (uint32_t)__builtin_amdgcn_readlane((int)v, 32);
  const uint32_t d = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
  return pick(pick(a, b), pick(c, d));
}

constexpr int kThrBits = 12;  // bits resolved by the threshold search below the highest differing one

// A lower bound of the k-th largest (1 <= k <= the number of lanes with ok) of the wave's 32-bit values v (one per
// lane) with at least k of them at or above it: a bitwise search from the highest bit where the valid minimum and
// maximum differ, keeping the largest prefix with at least k values at or above it (counted with ballots), stopped
// after kThrBits bits (the bound is then within 2^(top - kThrBits) of the k-th). Wave-uniform. The values are shifted
// so that the searched bits are always bits kThrBits - 1 .. 0 and the loop unrolls into four scalar instructions and
// one compare per bit (a search that also visits bits above the highest differing one leaves the prefix as it is):
// 128 x 128256 k = 50 19.36 -> 18.95 us against the loop over bit positions, whose scalar instructions the CU's one
// scalar unit issues for every wave of every workgroup in the same phase.
__device__ __forceinline__ uint32_t wave_kth32(uint32_t v, bool ok, int k) {
  v = ok ? v : 0u;
  const uint32_t mx = wave_ext32<true>(v);
  if (k == 1) return mx;
  const uint32_t mn = wave_ext32<false>(ok ? v : 0xffffffffu);
  if (mx == mn) return mx;
  const int top = 31 - __builtin_clz(mx ^ mn);
  const int sh = top >= kThrBits ? top - (kThrBits - 1) : 0;
  const uint32_t vs = v >> sh;
  uint32_t p = (mx & ~((2u << top) - 1u)) >> sh;
#pragma unroll
  for (int b = kThrBits - 1; b >= 0; --b) {
    const uint32_t cand = p | (1u << b);  // >= 1: the lanes without ok (0) never count
    if (__popcll(__ballot(vs >= cand)) >= k) p = cand;
  }
  return p << sh;
}

// wave_kth32 over four values per lane (a workgroup's 256 lane maxima, 0 for a lane without elements): a lower bound
// of the k-th largest with at least k values at or above it, within kThrBits bits below the highest differing one;
// 0 when fewer than k values are nonzero. Wave-uniform.
__device__ __forceinline__ uint32_t wave_kth32x4(const uint32_t (&v)[4], int k) {
  int n = 0;
  uint32_t hi = 0, lo = 0xffffffffu;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    n += __popcll(__ballot(v[j] != 0u));
    hi = v[j] > hi ? v[j] : hi;
    lo = v[j] != 0u && v[j] < lo ? v[j] : lo;
  }
  if (n < k) return 0u;
  const uint32_t mx = wave_ext32<true>(hi);
  if (k == 1) return mx;
  const uint32_t mn = wave_ext32<false>(lo);
  if (mx == mn) return mx;
  const int top = 31 - __builtin_clz(mx ^ mn);
  const int sh = top >= kThrBits ? top - (kThrBits - 1) : 0;
  uint32_t vs[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) vs[j] = v[j] >> sh;
  uint32_t p = (mx & ~((2u << top) - 1u)) >> sh;
#pragma unroll
  for (int b = kThrBits - 1; b >= 0; --b) {
    const uint32_t cand = p | (1u << b);
    int c = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) c += __popcll(__ballot(vs[j] >= cand));
    if (c >= k) p = cand;
  }
  return p << sh;
}

// Block-wide reductions of wave-uniform values through two alternating rows of LDS slots: one barrier each (a row is
// rewritten only after the barrier of the other row's use, which every reader of the first has passed). Every wave of
// the block makes the same sequence of calls.
struct BlockRed {
  uint32_t (*slot)[kWaves];
  int phase;

  template <typename Op>
  __device__ __forceinline__ uint32_t all(uint32_t v, Op op) {
    if (lane_id() == 0) slot[phase][wave_id()] = v;
    __syncthreads();
    uint32_t r = slot[phase][0];
#pragma unroll
    for (int i = 1; i < kWaves; ++i) r = op(r, slot[phase][i]);
    phase ^= 1;
    return r;
  }
  __device__ __forceinline__ uint32_t sum(uint32_t v) {
    return all(v, [](uint32_t a, uint32_t b) { return a + b; });
  }
  __device__ __forceinline__ uint32_t max(uint32_t v) {
    return all(v, [](uint32_t a, uint32_t b) { return a > b ? a : b; });
  }
  __device__ __forceinline__ uint32_t min(uint32_t v) {
    return all(v, [](uint32_t a, uint32_t b) { return a < b ? a : b; });
  }
};

// The exact k-th largest composite among the block's slots: slot(i, key, lo) for i < N fills in slot i of this lane
// and says whether it is occupied; at least k slots are. A bitwise search for the k-th key from the common prefix of
// the keys' range (a block count per candidate bit), then, among the composites with that key, for the lower word.
// Every thread returns it.
template <int N, typename F>
__device__ __forceinline__ u64 block_kth(const F& slot, int k, BlockRed& red) {
  uint32_t kmx = 0, kmn = 0xffffffffu;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    uint32_t kk, lw;
    if (slot(i, kk, lw)) {
      kmx = kk > kmx ? kk : kmx;
      kmn = kk < kmn ? kk : kmn;
    }
  }
  kmx = red.max(wave_ext32<true>(kmx));
  kmn = red.min(wave_ext32<false>(kmn));
  uint32_t K = kmx;
  if (kmx != kmn) {
    const int top = 31 - __builtin_clz(kmx ^ kmn);
    K = kmx & ~((2u << top) - 1u);
    for (int b = top; b >= 0; --b) {
      const uint32_t cand = K | (1u << b);
      int c = 0;
#pragma unroll
      for (int i = 0; i < N; ++i) {
        uint32_t kk, lw;
        const bool ok = slot(i, kk, lw);
        c += __popcll(__ballot(ok && kk >= cand));
      }
      if ((int)red.sum((uint32_t)c) >= k) K = cand;
    }
  }
  int gt = 0, eq = 0;
  uint32_t lmx = 0, lmn = 0xffffffffu;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    uint32_t kk, lw;
    const bool ok = slot(i, kk, lw);
    const bool e = ok && kk == K;
    gt += __popcll(__ballot(ok && kk > K));
    eq += __popcll(__ballot(e));
    lmx = e && lw > lmx ? lw : lmx;
    lmn = e && lw < lmn ? lw : lmn;
  }
  gt = (int)red.sum((uint32_t)gt);
  eq = (int)red.sum((uint32_t)eq);
  lmx = red.max(wave_ext32<true>(lmx));
  lmn = red.min(wave_ext32<false>(lmn));
  const int r = k - gt;  // 1 <= r <= eq
  uint32_t L = lmn;
  if (r < eq) {
    const int top = 31 - __builtin_clz(lmx ^ lmn);
    L = lmx & ~((2u << top) - 1u);
    for (int b = top; b >= 0; --b) {
      const uint32_t cand = L | (1u << b);
      int c = 0;
#pragma unroll
      for (int i = 0; i < N; ++i) {
        uint32_t kk, lw;
        const bool ok = slot(i, kk, lw);
        c += __popcll(__ballot(ok && kk == K && lw >= cand));
      }
      if ((int)red.sum((uint32_t)c) >= r) L = cand;
    }
  }
  return ((u64)K << 32) | L;
}

// A workgroup's candidate list: wave w appends to its own LDS segment (positions from a ballot, no atomics). cnt may
// pass kTileSeg within an overflowing batch, whose excess is not stored; the batch is then settled from registers.
struct TileList {
  u64* seg;
  int cnt;  // wave-uniform

  __device__ __forceinline__ void push(u64 c, bool keep) {
    const u64 m = __ballot(keep);
    if (m) {
      const int pos = cnt + lanes_below(m);
      if (keep && pos < kTileSeg) seg[pos] = c;
      cnt += __popcll(m);
    }
  }

  // push() for a batch whose ballot m is already known: keep is this lane's bit of m, comp() its composite. A batch
  // that passes the segment's end is counted, and its writes past the end land in the segment's spare slot (the list
  // then overflows and the batch is pushed again, see settle()): a clamp per lane instead of a scalar bound check.
  template <typename C>
  __device__ __forceinline__ void push_mask(u64 m, bool keep, const C& comp) {
    if (m) {
      if (keep) {
        const int pos = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                                        __builtin_amdgcn_mbcnt_lo((uint32_t)m, (uint32_t)cnt));
        seg[pos < kTileSeg ? pos : kTileSeg] = comp();
      }
      cnt += __popcll(m);
    }
  }

  // Keeps exactly the k largest of the list (which holds more, none dropped); returns the k-th.
  __device__ __forceinline__ u64 prune(BlockRed& red, int k) {
    constexpr int PER = kTileSeg / kWave;
    const int lane = lane_id();
    const int n = cnt;
    u64 c[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) c[i] = lane + i * kWave < n ? seg[lane + i * kWave] : 0ull;
    const u64 kth = block_kth<PER>(
        [&](int i, uint32_t& kk, uint32_t& lw) {
          kk = (uint32_t)(c[i] >> 32);
          lw = (uint32_t)c[i];
          return lane + i * kWave < n;
        },
        k, red);
    cnt = 0;
#pragma unroll
    for (int i = 0; i < PER; ++i) push(c[i], lane + i * kWave < n && c[i] >= kth);
    return kth;
  }

  // After a batch of pushes onto a list whose waves held cnt0 each: a list longer than kTileKeep is pruned to its k
  // largest. If a segment overflowed, the batch is dropped and pushed again in `steps` steps from `floor` (a lower
  // bound of the k-th): step(s, floor, check) pushes step s's composites >= floor, calling check() after each group of
  // at most 256 per wave, and check() prunes whenever the list passes kTileKeep, raising floor to the k-th. Returns
  // the new k-th, or 0, and sets `total` to the list's length when it is at most kTileKeep without a prune (else 0).
  template <typename S>
  __device__ __forceinline__ u64 settle(BlockRed& red, int k, int cnt0, int steps, u64 floor, const S& step,
                                        int& total) {
    const uint32_t v = red.sum((uint32_t)cnt + (cnt > kTileSeg ? (1u << 24) : 0u));
    total = 0;
    if (!(v >> 24)) {
      if ((int)(v & 0xffffffu) > kTileKeep) return prune(red, k);
      total = (int)(v & 0xffffffu);
      return 0ull;
    }
    cnt = cnt0;
    u64 kth = 0;
    auto check = [&] {
      if ((int)red.sum((uint32_t)cnt) > kTileKeep) {
        kth = prune(red, k);
        floor = kth > floor ? kth : floor;
      }
    };
    for (int st = 0; st < steps; ++st) step(st, floor, check);
    return kth;
  }
};

// The number of composites of list[0, n16) greater than c; n16 is a multiple of 16 and the list is zero-padded to it.
// Sixteen entries (eight 16-byte LDS reads, all broadcasts) per step keep the reads in flight together.
__device__ __forceinline__ int rank_in(const u64* list, int n16, u64 c) {
  int r = 0;
  for (int j = 0; j < n16; j += 16) {
    u64x2 p[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) p[i] = *reinterpret_cast<const u64x2*>(list + j + 2 * i);
#pragma unroll
    for (int i = 0; i < 8; ++i) r += (p[i].x > c) + (p[i].y > c);
  }
  return r;
}

// The rank sort of a short list split over the block: for n <= 64 every wave ranks all n entries against a quarter of
// the list, for n <= 128 each half of the block against a half, so that a thread reads a quarter or a half of the list
// instead of all of it (below 129 entries one thread per entry would leave two or three waves idle); the partial counts
// meet behind one barrier. (128 x 128256: about 75 candidates per chunk, 60 in the merge; a list of 16 or fewer loses a
// little to the barrier, but a separate path for it made the kernel's code larger and every k slower.) rank_pad(n) is
// the length the list must be zero-padded to (the zeros rank below every composite).
__device__ __forceinline__ int rank_groups(int n) { return n <= 64 ? 4 : n <= 128 ? 2 : 1; }
__device__ __forceinline__ int rank_pad(int n) {
  return rank_groups(n) == 4 ? 64 : rank_groups(n) == 2 ? ((n + 31) & ~31) : ((n + 15) & ~15);
}

// The number of entries of list[0, n) (distinct composites, n <= kThreads, zero-padded to rank_pad(n)) greater than
// list[t] for thread t < n; kTileSort for the others. The partial counts meet in part[0, kThreads) (LDS ints apart from
// the list) behind one barrier. Every thread of the block calls it.
__device__ __forceinline__ int split_rank(const u64* list, int n, int* part) {
  const int t = (int)threadIdx.x;
  const int groups = rank_groups(n);  // block-uniform
  const int per = kThreads / groups;                 // entries per group's pass: 64, 128 or 256 (>= n)
  const int len = rank_pad(n) / groups;              // a multiple of 16
  const int i = t & (per - 1), g = t / per;
  int r = i < n ? rank_in(list + g * len, len, list[i]) : 0;
  if (groups > 1) {
    part[t] = r;
    __syncthreads();
    for (int j = 1; j < groups; ++j) r += part[j * per + i];  // t < n: group 0, i == t
  }
  return t < n ? r : kTileSort;
}

// Keeps exactly the k largest of the block's list of n composites (k < n <= kTileSort) by ranking every entry against
// all of them (one per thread; cheaper than a bitwise search for short lists) and returns the k-th.
__device__ __forceinline__ u64 prune_ranked(TileSmem& s, TileList& L, int k) {
  const int wave = wave_id(), lane = lane_id(), t = threadIdx.x;
  if (lane == 0) s.cnt[wave] = L.cnt;
  __syncthreads();
  int pre = 0, n = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const int c = s.cnt[w];
    pre += w < wave ? c : 0;
    n += c;
  }
  for (int i = lane; i < L.cnt; i += kWave) s.sorted[pre + i] = L.seg[i];
  const int n16 = (n + 15) & ~15;
  if (t >= n && t < n16) s.sorted[t] = 0ull;
  __syncthreads();
  const u64 mine = t < n ? s.sorted[t] : 0ull;
  const int rank = t < n ? rank_in(s.sorted, n16, mine) : kTileSort;
  if (rank == k - 1) s.pick = mine;
  L.cnt = 0;
  L.push(mine, rank < k);
  __syncthreads();
  return s.pick;
}

// Ranks the block's list (at most kTileSort composites) and writes its k largest, in order, as the output row (a
// list holding at least k) or to the chunk list wr with device-coherent stores (0 past the end of a shorter list).
template <typename T>
__device__ __forceinline__ void finish_list(TileSmem& s, const TileList& L, void* values, long long* indices, u64* wr,
                                            long long row, int k, bool to_output) {
  const int wave = wave_id(), lane = lane_id(), t = threadIdx.x;
  if (lane == 0) s.cnt[wave] = L.cnt;
  __syncthreads();
  int pre = 0, n = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const int c = s.cnt[w];
    pre += w < wave ? c : 0;
    n += c;
  }
  for (int i = lane; i < L.cnt; i += kWave) s.sorted[pre + i] = L.seg[i];
  if (t >= n && t < rank_pad(n)) s.sorted[t] = 0ull;
  __syncthreads();
  // the partial ranks in the list segments, read above, behind the barrier
  const int rank = split_rank(s.sorted, n, reinterpret_cast<int*>(&s.seg[0][0]));
  if (t < n) {
    const u64 mine = s.sorted[t];
    if (rank < k) {
      if (to_output) {
        if constexpr (sizeof(T) == 4) static_cast<uint32_t*>(values)[row * k + rank] = composite_bits(mine);
        else static_cast<uint16_t*>(values)[row * k + rank] = (uint16_t)(composite_bits(mine) >> 16);
        indices[row * k + rank] = composite_index(mine);
        s.top[rank] = mine;
      } else {
        __hip_atomic_store(wr + rank, mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  if (!to_output)
    for (int j = n + t; j < k; j += kThreads)
      __hip_atomic_store(wr + j, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---- the chunk hand-off ----------------------------------------------------------------------------------------------

// A split row's chunks hand their results to the row's last arrival as the reference's topk_filter does
// (topk/kernel.cu:411-442): each chunk stores its result in its slots of the caller's work, then counts its arrival
// on the caller's counters[row]; the arrival that finds every other chunk counted merges, and zeroes the counter for
// the next launch. Results are written and read with agent-scope atomic (relaxed) stores and loads, which gfx950
// performs coherently across its XCDs (each XCD has its own L2), and the counter is an agent-scope atomic add. The
// order between them:
//  - writer: `s_waitcnt vmcnt(0)` after the result stores waits until the memory system has acknowledged every store
//    of the wave (on gfx9 that counter covers stores as well as loads), and the add is issued after it, so the results
//    are complete at agent scope before the add can be observed;
//  - reader: the last arrival branches on the value the add returned, so its loads issue after the add has completed,
//    and as agent-scope loads they take the coherent value, not a stale L1 or L2 copy.
// This is LLVM's agent-scope release and acquire for gfx942/gfx950 (the AMDGPU memory model) without the L2 write-back
// (buffer_wbl2) and invalidate (buffer_inv) that make non-atomic data visible: every location handed over here is
// accessed only through agent-scope atomics, so there is no such data, and per-workgroup whole-L2 maintenance measured
// about 100 us over a 1024-workgroup grid.

// One wave's arrival: waits for the wave's result stores, then lane 0 counts the arrival on *counter. Returns, uniform
// over the wave, whether it was the last of n.
__device__ __forceinline__ bool hand_off_arrive(unsigned* counter, int n) {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  unsigned old = 0;
  if (lane_id() == 0) old = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return (unsigned)__builtin_amdgcn_readfirstlane(old) == (unsigned)n - 1;
}

// A workgroup's arrival: each wave waits for its own result stores, the barrier gathers the waves, and thread 0 counts
// the arrival on *counter. Returns, uniform over the workgroup, whether it was the last of n.
template <typename S>
__device__ __forceinline__ bool block_hand_off(S& s, unsigned* counter, int n) {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0)
    s.last = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (unsigned)n - 1;
  __syncthreads();
  return s.last != 0;
}

typedef short s16x2 __attribute__((ext_vector_type(2)));

constexpr int kWideGroups = 8;  // groups per lane for the admission bound of the 64 < k <= 1024 kernel

// What a vector load past a tile's end reads instead (all ones: the sentinel below).
__device__ u32x4 g_sentinel_vec = {~0u, ~0u, ~0u, ~0u};

// Stage stamps, for a separate timing build only (bench.py --topk-stages compiles this file with ROWKERN_TOPK_STAGES
// into its own library; the op library is built without it, and there TOPK_STAGE and TOPK_WAVE_STAGE compile to
// nothing). Thread 0 of each workgroup records the 100 MHz s_memrealtime clock at stage i of its kernel in slot i of
// the workgroup's row of stamps, and lane 0 of each wave the moment its tile's loads have landed in slot 16 + wave.
// The clock is read by an asm statement after the LDS operations before it have completed; a stamp that follows
// register work (TOPK_STAGE_AT, TOPK_WAVE_STAGE_AT) first takes that work's result as an asm operand, so the compiler
// cannot read the clock before the work is done (it may move the clock builtin freely).
#ifdef ROWKERN_TOPK_STAGES
constexpr long long kStageWGs = 4096;  // workgroups with stamps (blockIdx.y * gridDim.x + blockIdx.x below this)
constexpr int kStageSlots = 32;
__device__ unsigned long long g_stage_stamps[kStageWGs * kStageSlots];
__device__ __forceinline__ void stage_stamp(int slot) {
  const long long wg = (long long)blockIdx.y * gridDim.x + blockIdx.x;
  unsigned long long t;
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_memrealtime %0\n\ts_waitcnt lgkmcnt(0)" : "=s"(t) : : "memory");
  if (wg < kStageWGs) g_stage_stamps[wg * kStageSlots + slot] = t;
}
#define TOPK_STAGE(i) \
  do {                              \
    if (threadIdx.x == 0) stage_stamp(i); \
  } while (0)
#define TOPK_STAGE_AT(i, v)                \
  do {                                     \
    asm volatile("" : : "v"(v) : "memory"); \
    TOPK_STAGE(i);                         \
  } while (0)
#define TOPK_WAVE_STAGE_AT(v)                                                                   \
  do {                                                                                          \
    asm volatile("" : : "v"(v) : "memory");                                                     \
    if ((threadIdx.x & 63) == 0 && (threadIdx.x >> 6) < 16) stage_stamp(16 + (int)(threadIdx.x >> 6)); \
  } while (0)
#else
#define TOPK_STAGE(i) \
  do {                \
  } while (0)
#define TOPK_STAGE_AT(i, v) \
  do {                      \
  } while (0)
#define TOPK_WAVE_STAGE_AT(v) \
  do {                        \
  } while (0)
#endif

// A register tile: thread t of the workgroup's NT holds vectors v * NT + t (v < NV = EPL / W) of elements [b0, b1) of a
// row, W each, as raw bits; an element outside [b0, b1) holds the sentinel (all ones: the -NaN whose key is the smallest of
// its format), read from g_sentinel_vec by a vector load past the end. load() only issues the loads.
//
// The raw bits are ordered without forming keys: over non-negative values key order is the signed order of the bits
// (as int32, or int16 for a bf16 half), over negative values it is the reverse. So the largest element of a set, in
// key order, is its signed maximum when that is non-negative and its signed minimum otherwise (the sentinel, -1 as an
// integer, is the largest negative one: it never moves the minimum of a set holding a real element); and for a
// threshold key K with bits t, key(u) >= K iff (int)u >= (int)t when K is a non-negative value, iff u <= t (unsigned)
// when K is negative.
// WL: a tile whose vectors are whole but for the last takes them without the per-vector select of the sentinel's
// address (the k = 1 kernel: 128 x 128256 13.43 -> 13.25 us, 512 x 32000 12.30 -> 12.11 us; the other kernels
// measured from 0.1 us faster to 0.3 us slower with it, interleaved on one MI355X).
template <typename T, bool VEC, int NT = kThreads, int EPL = kTileE, bool WL = false>
struct Tile {
  static constexpr int W = Fmt<T>::W;
  static constexpr int NV = EPL / W;
  static constexpr uint32_t kSentinelKey = sizeof(T) == 4 ? 0u : 0xffffu;  // key of the sentinel
  u32x4 r[NV];
  int b0, b1;
  int lane0;  // b0 + threadIdx.x * W, the first element of vector 0 (kept opaque with the registers)

  __device__ __forceinline__ int first(int v) const { return lane0 + v * NT * W; }
  __device__ __forceinline__ uint32_t bits(int v, int j) const {
    if constexpr (sizeof(T) == 4) {
      return r[v][j];
    } else {
      const uint32_t w = r[v][j >> 1];
      return (j & 1) ? (w & 0xffff0000u) : (w << 16);
    }
  }
  __device__ __forceinline__ u64 comp(int v, int j) const {
    return ((u64)key_of(bits(v, j)) << 32) | (u64)(~(uint32_t)(first(v) + j));
  }

  __device__ __forceinline__ void load(const T* row, int t0, int end) {
    b0 = t0;
    b1 = end - t0 > NT * EPL ? t0 + NT * EPL : end;
    lane0 = b0 + (int)threadIdx.x * W;
    if constexpr (VEC && WL) {
      if (b1 - b0 >= (NV - 1) * NT * W) {  // uniform: every vector but the last is whole
        const T* base = row + lane0;
#pragma unroll
        for (int v = 0; v < NV - 1; ++v)
          r[v] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(base + (uint32_t)(v * NT * W)));
        const int e0 = first(NV - 1);
        r[NV - 1] = load16<true>(e0 < b1 ? (const void*)(row + e0) : (const void*)&g_sentinel_vec, 0);
        asm volatile("" ::: "memory");
        return;
      }
    }
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const int e0 = first(v);
      if constexpr (VEC) {
        r[v] = load16<true>(e0 < b1 ? (const void*)(row + e0) : (const void*)&g_sentinel_vec, 0);
      } else {
        uint32_t u[W];
#pragma unroll
        for (int j = 0; j < W; ++j) {
          const int e = e0 + j;
          if constexpr (sizeof(T) == 4) u[j] = e < b1 ? reinterpret_cast<const uint32_t*>(row)[e] : 0xffffffffu;
          else u[j] = e < b1 ? (uint32_t)reinterpret_cast<const uint16_t*>(row)[e] : 0xffffu;
        }
        if constexpr (sizeof(T) == 4) r[v] = (u32x4){u[0], u[1], u[2], u[3]};
        else r[v] = (u32x4){u[0] | (u[1] << 16), u[2] | (u[3] << 16), u[4] | (u[5] << 16), u[6] | (u[7] << 16)};
      }
    }
    asm volatile("" ::: "memory");  // issue the loads here: the scheduler must not sink them past later work
  }

  // The lane's largest composite: its largest key and the lowest index holding it (raw bits equal the key's bits, the
  // key mapping being one to one). A sentinel element (past the chunk's end, key 0, after every real element of the
  // lane in index order) never wins over a real one.
  __device__ __forceinline__ u64 best_composite() {
    const uint32_t m = max_key();  // vector by vector as the loads complete
    const uint32_t t = bits_of(m);
    opaque();
    // the first match's vector and element, visited from the last element to the first; both are inline constants
    // (a select of each element's offset would hold 64 literal offsets in registers)
    int vb = 0, jb = 0;
#pragma unroll
    for (int v = NV - 1; v >= 0; --v) {
#pragma unroll
      for (int j = W - 1; j >= 0; --j) {
        bool eq;
        if constexpr (sizeof(T) == 4) {
          eq = r[v][j] == t;
        } else {
          const uint32_t w = r[v][j >> 1];
          eq = ((j & 1) ? (w & 0xffff0000u) : (w << 16)) == t;
        }
        vb = eq ? v : vb;
        jb = eq ? j : jb;
      }
    }
    const int off = vb * NT * W + jb;
    return ((u64)m << 32) | (u64)(~(uint32_t)(lane0 + off));
  }

  // The key of this lane's largest element (the sentinel's key for a lane holding none).
  __device__ __forceinline__ uint32_t max_key() const {
    if constexpr (sizeof(T) == 4) {
      int mx = INT_MIN, mn = INT_MAX;
#pragma unroll
      for (int v = 0; v < NV; ++v)
#pragma unroll
        for (int j = 0; j < W; ++j) {
          const int x = (int)r[v][j];
          mx = x > mx ? x : mx;
          mn = x < mn ? x : mn;
        }
      return key_of((uint32_t)(mx >= 0 ? mx : mn));
    } else {
      s16x2 mx = {(short)-32768, (short)-32768}, mn = {(short)32767, (short)32767};
#pragma unroll
      for (int v = 0; v < NV; ++v)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t w = r[v][j];  // (bit-casting the element expression itself reads element 0)
          const s16x2 x = __builtin_bit_cast(s16x2, w);
          mx = __builtin_elementwise_max(mx, x);
          mn = __builtin_elementwise_min(mn, x);
        }
      const uint32_t lo = (uint32_t)(uint16_t)(mx.x >= 0 ? mx.x : mn.x) << 16;
      const uint32_t hi = (uint32_t)(uint16_t)(mx.y >= 0 ? mx.y : mn.y) << 16;
      const uint32_t kl = key_of(lo), kh = key_of(hi);
      return kl > kh ? kl : kh;
    }
  }

  // Pushes every element with key >= K (K above the sentinel's key; NEG: K is a negative value): one compare per
  // element on the raw bits, the list's positions from the compare's ballot.
  template <bool NEG, typename Lst>
  __device__ __forceinline__ void filter(Lst& L, uint32_t K) {
    const uint32_t t = bits_of(K);
    // over a non-negative threshold every admitted element is non-negative, and its key is its bits with the top bit
    // set; ~(lane0 + off) = nl - off: one instruction each per push instead of two
    uint32_t nl = ~(uint32_t)lane0;
    asm volatile("" : "+v"(nl));
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      bool a[W];
      u64 m[W];
#pragma unroll
      for (int j = 0; j < W; ++j) {
        if constexpr (sizeof(T) == 4) {
          a[j] = NEG ? r[v][j] <= t : (int)r[v][j] >= (int)t;
        } else {
          const uint32_t w = r[v][j >> 1];
          if (j & 1) a[j] = NEG ? w <= (t | 0xffffu) : (int)w >= (int)t;  // the low half only breaks ties
          else a[j] = NEG ? (uint16_t)w <= (uint16_t)(t >> 16) : (int16_t)(uint16_t)w >= (int16_t)(uint16_t)(t >> 16);
        }
        m[j] = __ballot(a[j]);
      }
      // (no test of the vector as a whole first: most vectors of a wave admit an element, and the test cost more
      // scalar instructions than the per-element tests it skipped)
#pragma unroll
      for (int j = 0; j < W; ++j)
        L.push_mask(m[j], a[j], [&] {
          if constexpr (NEG) return comp(v, j);
          return ((u64)(bits(v, j) | 0x80000000u) << 32) | (u64)(nl - (uint32_t)(v * NT * W + j));
        });
    }
  }

  // filter() for a non-negative threshold key K over fp32 tiles, by groups of 8 elements (two vectors): a group whose
  // signed maximum of the raw bits is below K's bits holds no element with key >= K (over a non-negative threshold
  // the key order is the signed order of the bits, and a negative element's bits are negative), so only the groups
  // reaching it are staged, each by its lane, into the wave's LDS area (two 16-byte writes and the group's first index;
  // positions from a ballot per group), and the wave then tests the staged elements exactly, 64 at a time, pushing
  // the admitted ones. A group reaching K holds about one admitted element: per wave a compare per group and a push
  // per 64 staged elements, instead of a compare per element and a push per element position that any lane admits. A
  // wave with more than kStageGroups groups to stage (ties, adversarial orders) takes the per-element filter.
  template <typename Lst>
  __device__ __forceinline__ void filter_groups(Lst& L, uint32_t K, u32x4* stage, uint32_t* stage_at) {
    static_assert(sizeof(T) == 4, "fp32 tiles: two vectors per group");
    constexpr int NG = NV / 2;
    const int t = (int)bits_of(K);  // >= 0
    const int lane = lane_id();
    int n = 0;  // wave-uniform
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      int gm = INT_MIN;
#pragma unroll
      for (int v = 2 * g; v < 2 * g + 2; ++v)
#pragma unroll
        for (int j = 0; j < W; ++j) gm = (int)r[v][j] > gm ? (int)r[v][j] : gm;
      const bool c = gm >= t;
      const u64 m = __ballot(c);
      if (m) {
        if (c) {
          const int pos = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                                         __builtin_amdgcn_mbcnt_lo((uint32_t)m, (uint32_t)n));
          const int at = pos < kStageGroups ? pos : kStageGroups;  // past the end: the spare group
          stage[2 * at] = r[2 * g];
          stage[2 * at + 1] = r[2 * g + 1];
          stage_at[at] = (uint32_t)first(2 * g);
        }
        n += __popcll(m);
      }
    }
    if (n > kStageGroups) {
      filter<false>(L, K);
      return;
    }
    wave_lds_sync();  // the wave's staging writes before its reads of other lanes' entries
    const uint32_t* su = reinterpret_cast<const uint32_t*>(stage);
    for (int b = 0; b < 8 * n; b += kWave) {  // wave-uniform trip count
      const int i = b + lane, slot = i >> 3, e = i & 7;
      const bool ok = i < 8 * n;
      const uint32_t u = su[ok ? i : 0];
      const uint32_t at = stage_at[ok ? slot : 0] + (uint32_t)((e >> 2) * NT * W + (e & 3));
      // over a non-negative threshold the key of an admitted element is its bits with the top bit set
      const bool keep = ok && (int)u >= t;
      L.push_mask(__ballot(keep), keep, [&] { return ((u64)(u | 0x80000000u) << 32) | (u64)(~at); });
    }
  }

  // Keys of the lane's kWideGroups groups of 64 / kWideGroups elements (vectors g * VPG .. g * VPG + VPG - 1): each
  // group's largest element in key order, 0 (counted nowhere) for a group past the tile's end.
  __device__ __forceinline__ void group_keys(uint32_t (&g)[kWideGroups]) const {
    constexpr int VPG = NV / kWideGroups;
    static_assert(VPG * kWideGroups == NV, "groups must be whole vectors");
#pragma unroll
    for (int gi = 0; gi < kWideGroups; ++gi) {
      uint32_t key;
      if constexpr (sizeof(T) == 4) {
        int mx = INT_MIN, mn = INT_MAX;
#pragma unroll
        for (int v = gi * VPG; v < gi * VPG + VPG; ++v)
#pragma unroll
          for (int j = 0; j < W; ++j) {
            const int x = (int)r[v][j];
            mx = x > mx ? x : mx;
            mn = x < mn ? x : mn;
          }
        key = key_of((uint32_t)(mx >= 0 ? mx : mn));
      } else {
        s16x2 mx = {(short)-32768, (short)-32768}, mn = {(short)32767, (short)32767};
#pragma unroll
        for (int v = gi * VPG; v < gi * VPG + VPG; ++v)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const uint32_t w = r[v][j];  // (bit-casting the element expression itself reads element 0)
            const s16x2 x = __builtin_bit_cast(s16x2, w);
            mx = __builtin_elementwise_max(mx, x);
            mn = __builtin_elementwise_min(mn, x);
          }
        const uint32_t kl = key_of((uint32_t)(uint16_t)(mx.x >= 0 ? mx.x : mn.x) << 16);
        const uint32_t kh = key_of((uint32_t)(uint16_t)(mx.y >= 0 ? mx.y : mn.y) << 16);
        key = kl > kh ? kl : kh;
      }
      g[gi] = first(gi * VPG) < b1 ? key : 0u;
    }
  }

  // Whether element j of vector v has key >= K, where t = bits_of(K) (the compare of filter()).
  template <bool NEG>
  __device__ __forceinline__ bool admits(int v, int j, uint32_t t) const {
    if constexpr (sizeof(T) == 4) {
      return NEG ? r[v][j] <= t : (int)r[v][j] >= (int)t;
    } else {
      const uint32_t w = r[v][j >> 1];
      if (j & 1) return NEG ? w <= (t | 0xffffu) : (int)w >= (int)t;
      return NEG ? (uint16_t)w <= (uint16_t)(t >> 16) : (int16_t)(uint16_t)w >= (int16_t)(uint16_t)(t >> 16);
    }
  }

  // filter() into a shared buffer: appends every element with key >= K (K above the sentinel's key; NEG: K is a
  // negative value) to s.buf in two passes. Each lane counts its admitted elements. One exclusive prefix over the
  // wave (a ballot per bit of the counts) and one LDS atomic per wave reserve the wave's positions, and each lane
  // writes its elements in order. This needs no ballot per element, which at the wide kernel's admission rate (an
  // admitted lane in nearly every 64-lane column) cost as many scalar instructions as the compares. Appends past the
  // buffer's first `lim` entries are counted in s.count and not stored.
  template <bool NEG, typename S>
  __device__ __forceinline__ void filter_append(S& s, uint32_t K, int lim) {
    const uint32_t t = bits_of(K);
    int n = 0;
#pragma unroll
    for (int v = 0; v < NV; ++v)
#pragma unroll
      for (int j = 0; j < W; ++j) n += admits<NEG>(v, j, t) ? 1 : 0;
    int total = 0;
    const int excl = wave_excl_count<7>(n, total);  // n <= kTileE = 64
    if (total == 0) return;
    int base = 0;
    if (lane_id() == 0) base = atomicAdd(&s.count, total);
    base = __builtin_amdgcn_readfirstlane(base);
    if (base + total <= lim) {
      // every element of the wave fits: no bound check per element. Over a non-negative threshold every admitted
      // element is non-negative, and its key is its bits with the top bit set.
      u64* at = s.buf + base + excl;
      uint32_t nl = ~(uint32_t)lane0;  // ~(lane0 + off) = nl - off: one add per element
      asm volatile("" : "+v"(nl));
#pragma unroll
      for (int v = 0; v < NV; ++v)
#pragma unroll
        for (int j = 0; j < W; ++j)
          if (admits<NEG>(v, j, t)) {
            const uint32_t u = bits(v, j);
            const uint32_t key = NEG ? key_of(u) : (u | 0x80000000u);
            *at = ((u64)key << 32) | (u64)(nl - (uint32_t)(v * NT * W + j));
            ++at;
          }
      return;
    }
    int pos = base + excl;
#pragma unroll
    for (int v = 0; v < NV; ++v)
#pragma unroll
      for (int j = 0; j < W; ++j)
        if (admits<NEG>(v, j, t)) {
          if (pos < lim) s.buf[pos] = comp(v, j);
          ++pos;
        }
  }

  // filter_append<false> for fp32 tiles by way of the wave's LDS staging area (CAPW vectors, then their first indices):
  // a vector whose signed maximum of the raw bits is below t = bits_of(K) holds no element with key >= K (as in
  // filter_groups), so each lane stages only its vectors reaching t, and the wave then tests the staged elements 64 at
  // a time, appending the admitted ones (one LDS atomic per batch of 64; positions from the batch's ballot). At the
  // wide kernel's admission rate a staged vector holds about one admitted element, so this replaces a compare and a
  // masked write per element position with a compare per vector and a few instructions per 64 staged elements.
  // Appends at or past `lim` are counted in s.count and not stored. Returns false, having appended nothing, when the
  // wave has more than CAPW vectors to stage (ties, clustered values); its lanes then take filter_append.
  template <int CAPW, typename S>
  __device__ __forceinline__ bool stage_append(S& s, uint32_t K, u32x4* stage, uint32_t* stage_at, int lim) {
    static_assert(sizeof(T) == 4, "fp32 tiles");
    const int t = (int)bits_of(K);  // >= 0
    int n = 0;                      // wave-uniform
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const int a = (int)r[v][0], b = (int)r[v][1], c = (int)r[v][2], d = (int)r[v][3];
      const int ab = a > b ? a : b, cd = c > d ? c : d;
      const bool hit = (ab > cd ? ab : cd) >= t;
      const u64 m = __ballot(hit);
      int pos = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                               __builtin_amdgcn_mbcnt_lo((uint32_t)m, (uint32_t)n));
      pos = pos < CAPW - 1 ? pos : CAPW - 1;  // past the area: the last slot (the wave then returns false)
      if (hit) {
        stage[pos] = r[v];
        stage_at[pos] = (uint32_t)first(v);
      }
      n += __popcll(m);
    }
    if (n > CAPW) return false;
    wave_lds_sync();  // the wave's staging writes before its reads of other lanes' entries
    const int lane = lane_id();
    const uint32_t* su = reinterpret_cast<const uint32_t*>(stage);
    // two batches of 64 staged elements per step, all four reads issued together, one LDS atomic for both
    for (int b = 0; b < 4 * n; b += 2 * kWave) {  // wave-uniform trip count
      const int i0 = b + lane, i1 = i0 + kWave;
      const bool ok0 = i0 < 4 * n, ok1 = i1 < 4 * n;
      const int a0 = ok0 ? i0 : 0, a1 = ok1 ? i1 : 0;
      const uint32_t u0 = su[a0], u1 = su[a1];
      const uint32_t x0 = stage_at[a0 >> 2] + (uint32_t)(a0 & 3), x1 = stage_at[a1 >> 2] + (uint32_t)(a1 & 3);
      const bool k0 = ok0 && (int)u0 >= t, k1 = ok1 && (int)u1 >= t;
      const u64 m0 = __ballot(k0), m1 = __ballot(k1);
      const int c0 = __popcll(m0), c = c0 + __popcll(m1);
      if (c == 0) continue;
      int base = 0;
      if (lane == 0) base = atomicAdd(&s.count, c);
      base = __builtin_amdgcn_readfirstlane(base);
      const int p0 = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m0 >> 32),
                                                    __builtin_amdgcn_mbcnt_lo((uint32_t)m0, (uint32_t)base));
      const int p1 = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m1 >> 32),
                                                    __builtin_amdgcn_mbcnt_lo((uint32_t)m1, (uint32_t)(base + c0)));
      // over a non-negative threshold the key of an admitted element is its bits with the top bit set
      if (k0 && p0 < lim) s.buf[p0] = ((u64)(u0 | 0x80000000u) << 32) | (u64)(~x0);
      if (k1 && p1 < lim) s.buf[p1] = ((u64)(u1 | 0x80000000u) << 32) | (u64)(~x1);
    }
    return true;
  }

  // The lane's elements with composites in [lo, hi].
  __device__ __forceinline__ int count_range(u64 lo, u64 hi) const {
    int n = 0;
#pragma unroll
    for (int v = 0; v < NV; ++v)
#pragma unroll
      for (int j = 0; j < W; ++j) {
        const u64 c = comp(v, j);
        n += (VEC ? first(v) < b1 : first(v) + j < b1) && c >= lo && c <= hi ? 1 : 0;
      }
    return n;
  }

  // Appends the elements of vector v, held in r[0], with composites in [floor, top] to s.buf (exact validity; the
  // caller keeps room for them); then moves the later vectors down one place (as push_first).
  template <typename S>
  __device__ __forceinline__ void append_first(S& s, int v, u64 floor, u64 top = ~0ull) {
    const int e0 = first(v);
    u64 c[W];
    bool keep[W];
    bool any = false;
#pragma unroll
    for (int j = 0; j < W; ++j) {
      c[j] = ((u64)key_of(bits(0, j)) << 32) | (u64)(~(uint32_t)(e0 + j));
      keep[j] = (VEC ? e0 < b1 : e0 + j < b1) && c[j] >= floor && c[j] <= top;
      any |= keep[j];
    }
    if (__ballot(any)) append<W>(s, c, keep);
#pragma unroll
    for (int i = 0; i + 1 < NV; ++i) r[i] = r[i + 1];
  }

  // Pushes the elements of vector v, held in r[0], with composites >= floor, calling check() after every 4 per lane;
  // then moves the later vectors down one place (the overflow path walks the tile in order this way, so that the
  // registers are indexed statically).
  template <typename Lst, typename C>
  __device__ __forceinline__ void push_first(Lst& L, int v, u64 floor, const C& check) {
    const int e0 = first(v);
#pragma unroll
    for (int g = 0; g < W; g += 4) {
#pragma unroll
      for (int j = g; j < g + 4; ++j) {
        const u64 c = ((u64)key_of(bits(0, j)) << 32) | (u64)(~(uint32_t)(e0 + j));
        L.push(c, (VEC ? e0 < b1 : e0 + j < b1) && c >= floor);
      }
      check();
    }
#pragma unroll
    for (int i = 0; i + 1 < NV; ++i) r[i] = r[i + 1];
  }

  // Makes the registers opaque to the compiler, so that it keeps the tile as 16-byte register quads instead of
  // widening every key into the upper half of a 64-bit composite ahead of its use.
  __device__ __forceinline__ void opaque() {
#pragma unroll
    for (int v = 0; v < NV; ++v) asm volatile("" : "+v"(r[v]));
    asm volatile("" : "+v"(lane0));
  }
};

// k <= 64 merge of a split row (the row's last workgroup). Every chunk list holds its chunk's k largest, descending,
// so the first h = ceil(k / nchunks) entries of the lists give nchunks * h >= k distinct composites: the k-th largest
// of these heads bounds the row's k-th from below and, the row's top k being spread over the chunks, admits little
// beyond the answer. The lists (read with device-coherent loads: other workgroups wrote them) are then streamed
// through the list from that floor, settled as in a tile, rank-sorted and written out.
template <typename T>
__device__ __forceinline__ void merge_lists(TileSmem& s, BlockRed& red, TileList& L, void* values,
                                            long long* indices, const u64* wr, long long row, int nchunks, int k) {
  const int t = threadIdx.x;
  const int h = (k + nchunks - 1) / nchunks;
  const int nh = h * nchunks;
  constexpr int PER = 8;
  const int total = nchunks * k;
  auto ld = [&](int at) { return __hip_atomic_load(wr + at, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
  u64 c[PER];
  auto load = [&](int base) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int at = base + i * kThreads + t;
      c[i] = at < total ? ld(at) : 0ull;
    }
  };
  load(0);  // in flight together with the heads
  u64 floor = 1;
  if (nh <= kWave && total <= kThreads * PER) {
    // Every wave finds the floor itself from its own copy of the heads, one per lane. No barrier: the waves agree.
    // Up to 16 heads: the head ranked k-1 among them, ranked in the wave's list segment (unused until the streamed
    // merge below) in one step of reads. More: a key with at least k heads at or above it (the wave's bitwise search,
    // within 2^-kThrBits of the range below the k-th head's key), whose lowest composite is then at or below the
    // row's k-th; a dozen ballots cost less than ranking 32 or more heads.
    const int l = lane_id(), wave = wave_id();
    const u64 hv = l < nh ? ld((l / h) * k + l % h) : 0ull;
    if (__popcll(__ballot(hv != 0)) >= k) {
      if (nh <= 16) {
        u64* hs = s.seg[wave];
        if (l < 16) hs[l] = hv;  // zero past nh: the padding rank_in reads
        wave_lds_sync();
        const u64 at = __ballot(hv != 0 && rank_in(hs, 16, hv) == k - 1);  // one lane: composites are distinct
        floor = readlane64(hv, __builtin_ctzll(at));
      } else {
        const uint32_t p = wave_kth32((uint32_t)(hv >> 32), hv != 0, k);
        floor = p ? (u64)p << 32 : 1ull;
      }
    }
    // the entries at or above the floor, compacted into s.sorted by one exchange of the waves' counts
    u64 m[PER];
    int wn = 0;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      m[i] = __ballot(c[i] >= floor);  // (c[i] is 0 past the lists' ends and in a short list's padding)
      wn += __popcll(m[i]);
    }
    if (l == 0) s.cnt[wave] = wn;
    __syncthreads();
    TOPK_STAGE(6);
    int pre = 0, n = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const int cw = s.cnt[w];
      pre += w < wave ? cw : 0;
      n += cw;
    }
    if (n <= kTileSort) {  // uniform over the block
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        if (c[i] >= floor) {
          const int at = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m[i] >> 32),
                                                        __builtin_amdgcn_mbcnt_lo((uint32_t)m[i], (uint32_t)pre));
          s.sorted[at] = c[i];
        }
        pre += __popcll(m[i]);
      }
      if (t >= n && t < rank_pad(n)) s.sorted[t] = 0ull;
      __syncthreads();
      TOPK_STAGE(7);
      // the partial ranks in the list segments (the heads' copies there were read before the barrier)
      const int rank = split_rank(s.sorted, n, reinterpret_cast<int*>(&s.seg[0][0]));
      if (t < n) {
        const u64 mine = s.sorted[t];
        if (rank < k) {
          if constexpr (sizeof(T) == 4) static_cast<uint32_t*>(values)[row * k + rank] = composite_bits(mine);
          else static_cast<uint16_t*>(values)[row * k + rank] = (uint16_t)(composite_bits(mine) >> 16);
          indices[row * k + rank] = composite_index(mine);
          s.top[rank] = mine;
        }
      }
      return;
    }
    // more than a rank sort holds (ties, adversarial orders): the streamed merge below, from this floor
  } else if (nh <= kTileSort) {
    const u64 hv = t < nh ? ld((t / h) * k + t % h) : 0ull;
    s.sorted[t] = hv;  // zero past nh: the padding rank_in reads
    const int real = (int)red.sum((uint32_t)__popcll(__ballot(hv != 0)));
    if (real >= k) {
      if (hv != 0 && rank_in(s.sorted, (nh + 15) & ~15, hv) == k - 1) s.pick = hv;
      __syncthreads();
      floor = s.pick;
    }
  }
  TOPK_STAGE(6);
  for (int base = 0; base < total; base += kThreads * PER) {
    if (base > 0) load(base);
    const int cnt0 = L.cnt;
#pragma unroll
    for (int i = 0; i < PER; ++i) L.push(c[i], c[i] >= floor);
    int listed = 0;
    const u64 kth = L.settle(
        red, k, cnt0, PER, floor,
        [&](int, const u64& f, const auto& check) {
          L.push(c[0], c[0] >= f);
          check();
#pragma unroll
          for (int i = 0; i + 1 < PER; ++i) c[i] = c[i + 1];
        },
        listed);
    floor = kth > floor ? kth : floor;
  }
  TOPK_STAGE(7);
  finish_list<T>(s, L, values, indices, nullptr, row, k, true);
}

// ---- sampling from the top k ---------------------------------------------------------------------------------------

constexpr int kSamplePer = kMaxK / kWave;  // list entries per lane (k <= 1024)

__device__ __forceinline__ float readlane_f(float v, int lane) {
  return __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(v), lane));
}

// Inclusive prefix sum over the wave's lanes (lane order): a scan inside each 16-lane row by DPP row shifts, then the
// sums of the rows below (read from lanes 15, 31 and 47) added.
__device__ __forceinline__ float wave_prefix(float v) {
  v += dpp<kDppRowShr + 1>(v);
  v += dpp<kDppRowShr + 2>(v);
  v += dpp<kDppRowShr + 4>(v);
  v += dpp<kDppRowShr + 8>(v);
  const float r0 = readlane_f(v, 15), r01 = r0 + readlane_f(v, 31), r012 = r01 + readlane_f(v, 47);
  const int wrow = lane_id() >> 4;
  return wrow == 0 ? v : v + (wrow == 1 ? r0 : wrow == 2 ? r01 : r012);
}

// The draw from a row of a top-k list by one wave (every lane returns it): temperature, top-p and a draw with the
// caller's uniform u in [0, 1). With x = value / temperature, e_i = exp(x_i - max x) and S_i = e_0 + ... + e_i (list
// order), the draw keeps the entries i with S_(i-1) < top_p * S_(k-1) (always the first; every entry when top_p >= 1),
// and picks the first kept i with S_i > u * S_last_kept (the last kept if rounding leaves none). temperature <= 0 is
// greedy: position 0, the list's largest value (lowest index among ties). Values must be finite when temperature > 0.
// Lane l holds positions [l E, l E + E), E = ceil(k / 64) <= PER: the result does not depend on PER.
template <int PER, typename Value, typename Index>
__device__ __forceinline__ long long sample_row(const Value& value_at, const Index& index_at, int k, float u,
                                                float temperature, float top_p) {
  const int lane = lane_id();
  const int per = PER == 1 ? 1 : (k + kWave - 1) / kWave;
  const int base = lane * per;
  int chosen;
  if (temperature <= 0.0f) {
    chosen = 0;  // greedy: the list's first entry, its largest value (lowest position among ties)
  } else {
    float x[PER];
    float m = -INFINITY;
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      const int i = base + e;
      x[e] = e < per && i < k ? value_at(i) / temperature : -INFINITY;
      m = fmaxf(m, x[e]);
    }
    m = wave_max(m);
    float run = 0.0f;
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      const float ex = (e < per && base + e < k) ? expf(x[e] - m) : 0.0f;
      run += ex;
      x[e] = run;  // lane-local inclusive sums
    }
    const float incl = wave_prefix(run);
    const float lane_excl = incl - run;
    const float total = readlane_f(incl, kWave - 1);
    const float cut = top_p * total;
    // kept: positions whose exclusive sum is below the cut (a prefix of the list; at least position 0)
    int keep = 0;
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      const float excl = lane_excl + (e ? x[e - 1] : 0.0f);
      keep += (e < per && base + e < k && (base + e == 0 || top_p >= 1.0f || excl < cut)) ? 1 : 0;
    }
    const int kept = (int)wave_sum((float)keep);
    // the kept mass is the inclusive sum at position kept - 1
    float mass = 0.0f;
#pragma unroll
    for (int e = 0; e < PER; ++e)
      if (e < per && base + e == kept - 1) mass = lane_excl + x[e];
    mass = wave_max(mass);
    const float target = u * mass;
    int first = kept - 1;
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      const int i = base + e;
      if (e < per && i < kept && lane_excl + x[e] > target && i < first) first = i;
    }
    chosen = (int)wave_ext32<false>((uint32_t)first);
  }
  return index_at(chosen);
}

// Accessors of row `row` of a top-k list in memory (values in T, int64 indices), for sample_row.
template <typename T>
struct ListInMemory {
  const void* values;
  const long long* indices;
  long long row;
  int k;
  __device__ __forceinline__ float operator()(int i) const {
    if constexpr (sizeof(T) == 4) return static_cast<const float*>(values)[row * k + i];
    else return __uint_as_float((uint32_t) static_cast<const uint16_t*>(values)[row * k + i] << 16);
  }
  __device__ __forceinline__ long long index(int i) const { return indices[row * k + i]; }
};

// Sampling fused into the top-k launch (topk_launch_sample): when out is not null, the workgroup that writes a row's
// values and indices then draws out[row] from them as topk_sample does (k = 1: the one index).
struct SampleArgs {
  const float* u;
  long long* out;
  float temperature;
  float top_p;
  // the row's uniform, loaded by the workgroup that will draw well before its draw (0 without a draw)
  __device__ __forceinline__ float uniform(long long row) const { return out ? u[row] : 0.0f; }
};

// The fused draw of a row of k > 64 whose list this workgroup's waves have just written: every thread calls it (the
// barrier makes the list visible to the first wave, which draws). u is the row's uniform.
template <typename T>
__device__ __forceinline__ void sample_list(const SampleArgs& sa, float u, const void* values,
                                            const long long* indices, long long row, int k) {
  if (!sa.out) return;
  __syncthreads();
  if (wave_id() != 0) return;
  const ListInMemory<T> list{values, indices, row, k};
  const long long drawn =
      sample_row<kSamplePer>(list, [&](int i) { return list.index(i); }, k, u, sa.temperature, sa.top_p);
  if (lane_id() == 0) sa.out[row] = drawn;
}

// The fused draw of a row of k <= 64 whose composites finish_list also left in order in top[] (LDS): the values are
// decoded from the composites (the bits written to the output), so the draw equals the one from memory.
__device__ __forceinline__ void sample_top(const SampleArgs& sa, float u, const u64* top, long long row, int k) {
  if (!sa.out) return;
  __syncthreads();
  if (wave_id() != 0) return;
  const long long drawn = sample_row<1>([&](int i) { return __uint_as_float(composite_bits(top[i])); },
                                        [&](int i) { return composite_index(top[i]); }, k, u, sa.temperature,
                                        sa.top_p);
  if (lane_id() == 0) sa.out[row] = drawn;
}


// ---- the k = 1 kernel ----------------------------------------------------------------------------------------------

constexpr int kOneThreads = 1024;  // threads of a k = 1 workgroup
constexpr int kOneE = 32;          // elements per lane of its register tile (32768 per workgroup)
constexpr int kOneChunks = 2;      // consecutive chunks of the caller's chunking per k = 1 workgroup

// k = 1: one 1024-thread workgroup per kOneChunks consecutive chunks of a row (the result does not depend on the
// chunking), in register tiles of 32768 elements, all of a tile's loads in flight at once. Each lane's largest
// composite comes straight from its registers (no bound, list or block reduction per tile), then the wave's and,
// through LDS, the workgroup's. A row split over several workgroups hands over as topk_tile's chunks do: each stores
// its best in the work slot of its group (work[row * nchunks + group], inside the caller's [rows, nchunks] slots),
// waits for the store and counts its arrival on counters[row]; the row's last arrival takes the largest slot and
// zeroes the counter.
// The shape is measured (interleaved runs on one MI355X, 128 x 128256 fp32): eight 16-byte loads per lane in two
// resident workgroups of sixteen waves per CU, 13.49 us, against sixteen loads per lane in one (65536-element tiles
// over four chunks) 13.95 us, 512 threads over one chunk 13.82 us, 1024 threads with four loads per lane over one
// chunk 14.77 us.
template <typename T, bool VEC, bool DRAW>
__global__ void __launch_bounds__(kOneThreads)
    topk_one(const T* __restrict__ x, void* __restrict__ values, long long* __restrict__ indices,
             u64* __restrict__ work, unsigned* __restrict__ counters, long long cols, long long chunk, int nchunks,
             int groups, SampleArgs sa) {
  if constexpr (!DRAW) sa.out = nullptr;  // a launch without the draw: its code compiles away
  __shared__ u64 best_of[kOneThreads / kWave];
  const long long row = blockIdx.y;
  const int group = blockIdx.x;
  const int begin = (int)((long long)group * kOneChunks * chunk);
  const int end = (int)(group == groups - 1 ? cols : begin + kOneChunks * chunk);  // the last group ends the row
  const T* xr = x + row * cols;
  TOPK_STAGE(0);
  using TL = Tile<T, VEC, kOneThreads, kOneE, true>;
  constexpr int TE = kOneThreads * kOneE;
  u64 best = 0;
  for (int t0 = begin; t0 < end; t0 += TE) {
    TL tile;
    tile.load(xr, t0, end);
    const u64 c = tile.best_composite();
    best = c > best ? c : best;
  }
  TOPK_STAGE_AT(1, best);
  TOPK_WAVE_STAGE_AT(best);
  best = wave_ext64<true>(best);
  if (lane_id() == 0) best_of[wave_id()] = best;
  __syncthreads();
  TOPK_STAGE(2);
  if (wave_id() != 0) return;
  best = wave_ext64<true>(lane_id() < kOneThreads / kWave ? best_of[lane_id()] : 0ull);
  if (groups > 1) {
    u64* slots = work + row * (long long)nchunks;
    if (lane_id() == 0) __hip_atomic_store(slots + group, best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const bool last = hand_off_arrive(counters + row, groups);
    TOPK_STAGE(3);
    if (!last) return;
    u64 m = 0;
    for (int i = lane_id(); i < groups; i += kWave) {
      const u64 v = __hip_atomic_load(slots + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      m = v > m ? v : m;
    }
    best = wave_ext64<true>(m);
    if (lane_id() == 0) __hip_atomic_store(counters + row, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (lane_id() != 0) return;
  if constexpr (sizeof(T) == 4) static_cast<uint32_t*>(values)[row] = composite_bits(best);
  else static_cast<uint16_t*>(values)[row] = (uint16_t)(composite_bits(best) >> 16);
  indices[row] = composite_index(best);
  if (sa.out) sa.out[row] = composite_index(best);  // the draw from a one-entry list
  TOPK_STAGE(8);
}

// ---- the k <= 64 kernel --------------------------------------------------------------------------------------------

// k <= 64: one 256-thread workgroup per (chunk, row). The chunk is taken in register tiles of 16384 elements, all of a
// tile's loads in flight at once. Per tile: each wave takes (a lower bound of) the ceil(k / 4)-th largest of its 64
// lane maxima, which has that many distinct elements at or above it, and the smallest of the four waves' keys has at
// least k (a row taken whole, WHOLE: the k-th of the workgroup's 256 lane maxima); with the k-th of the earlier tiles
// it is the admission key. Admitted elements (about k * 1.5 per tile on continuous data) are appended to the waves'
// LDS segments; a list beyond kTileKeep is pruned to k, and an overflowing
// tile (ties, or adversarial orders) is pushed again in index order with a prune whenever the list passes kTileKeep.
// The list is then rank-sorted and written out for an unsplit row. A split row's chunk writes its k largest,
// descending, to its slots of the caller's work [rows, nchunks, k] with device-coherent stores, waits for them to
// complete and counts its arrival on the caller's counters[row]; the row's last arrival merges the lists (merge_lists)
// and zeroes the counter for the next launch -- no L2 write-back or invalidate, and no second kernel (the protocol of
// topk/kernel.cu:411-442, without its __threadfence: see hand_off_arrive).
template <typename T, bool VEC, bool DRAW, bool WHOLE>
__global__ void __launch_bounds__(kThreads)
    topk_tile(const T* __restrict__ x, void* __restrict__ values, long long* __restrict__ indices,
              u64* __restrict__ work, unsigned* __restrict__ counters, long long cols, long long chunk, int nchunks,
              int k, SampleArgs sa) {
  if constexpr (!DRAW) sa.out = nullptr;  // a launch without the draw: its code compiles away
  __shared__ TileSmem s;
  const long long row = blockIdx.y;
  const int part = blockIdx.x;
  const int begin = (int)((long long)part * chunk);
  const int end = (int)(part == nchunks - 1 ? cols : begin + chunk);  // the last chunk may hold a merged tail
  const T* xr = x + row * cols;
  BlockRed red;  // fields assigned at run time (an aggregate initializer of LDS addresses does not compile)
  red.slot = s.red;
  red.phase = 0;
  TileList L;
  L.seg = s.seg[wave_id()];
  L.cnt = 0;
  TOPK_STAGE(0);
  uint32_t thr = 0;
  const int kw = (k + kWaves - 1) / kWaves;
  using TL = Tile<T, VEC>;
  constexpr int TE = kThreads * kTileE;
  auto process = [&](TL& tile, bool more) __attribute__((always_inline)) {
    const bool has = tile.lane0 < tile.b1;
    const uint32_t m = tile.max_key();  // vector by vector as the loads complete
    TOPK_STAGE_AT(1, m);
    TOPK_WAVE_STAGE_AT(m);
    uint32_t tb;
    if constexpr (WHOLE) {
      // a row taken whole (no merge after it): the k-th of the workgroup's 256 lane maxima, found by wave 0, admits
      // about 56 elements of a randn tile at k = 50 against 76 (512 x 32000: 17.6 -> 16.5 us); for split rows the
      // per-wave bounds below measured faster
      s.lm[threadIdx.x] = has ? m : 0u;
      __syncthreads();
      if (wave_id() == 0) {
        const u32x4 q = reinterpret_cast<const u32x4*>(s.lm)[lane_id()];
        const uint32_t v4[4] = {q.x, q.y, q.z, q.w};
        const uint32_t tw = wave_kth32x4(v4, k);
        TOPK_STAGE_AT(11, tw);
        if (lane_id() == 0) s.thr = tw;
      }
      __syncthreads();
      tb = s.thr;
    } else {
      const uint32_t tw = __popcll(__ballot(has)) >= kw ? wave_kth32(m, has, kw) : 0u;
      TOPK_STAGE_AT(11, tw);
      tb = red.min(tw);
    }
    TOPK_STAGE(2);
    thr = tb > thr ? tb : thr;
    L.cnt = __builtin_amdgcn_readfirstlane(L.cnt);
    const int cnt0 = L.cnt;
    tile.opaque();
    if (thr > TL::kSentinelKey) {
      if (thr & 0x80000000u) {
        if constexpr (sizeof(T) == 4) tile.filter_groups(L, thr, s.stage[wave_id()], s.stage_at[wave_id()]);
        else tile.template filter<false>(L, thr);
      } else {
        tile.template filter<true>(L, thr);
      }
    } else {
      L.cnt = kTileSeg + 1;  // no usable bound: every element may pass, so the tile takes the exact re-push path
    }
    TOPK_STAGE_AT(9, L.cnt);
    int total = 0;
    u64 kth = L.settle(
        red, k, cnt0, TL::NV, (u64)thr << 32,
        [&](int v, const u64& floor, const auto& check) { tile.push_first(L, v, floor, check); }, total);
    TOPK_STAGE(10);
    // before another tile, keep the list near k so that it admits less: the list's k-th raises the admission key
    if (more && total > 2 * k) kth = prune_ranked(s, L, k);
    const uint32_t kk = (uint32_t)(kth >> 32);
    thr = kk > thr ? kk : thr;
  };
  // One register tile at a time, all of its loads in flight at once (the workgroups resident on a CU keep the memory
  // busy while one of them computes; a second register tile per workgroup halves the resident workgroups and was
  // slower).
  for (int t0 = begin; t0 < end; t0 += TE) {
    TL tile;
    tile.load(xr, t0, end);
    process(tile, end - t0 > TE);
  }
  TOPK_STAGE(3);
  if (nchunks == 1) {
    const float u = sa.uniform(row);
    finish_list<T>(s, L, values, indices, nullptr, row, k, true);
    sample_top(sa, u, s.top, row, k);
    return;
  }
  u64* wr = work + row * (long long)nchunks * k;
  finish_list<T>(s, L, values, indices, wr + (long long)part * k, row, k, false);
  TOPK_STAGE(4);
  // hand-off: the row's last arrival merges the lists and zeroes the row's counter for the next launch
  const bool last = block_hand_off(s, counters + row, nchunks);
  TOPK_STAGE(5);
  if (!last) return;
  const float u = sa.uniform(row);
  L.cnt = 0;
  merge_lists<T>(s, red, L, values, indices, wr, row, nchunks, k);
  TOPK_STAGE(8);
  if (threadIdx.x == 0) __hip_atomic_store(counters + row, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  sample_top(sa, u, s.top, row, k);
}

// ---- wide kernel (64 < k <= 1024) ----------------------------------------------------------------------------------

constexpr int kWideCap = 4096;    // the wide kernel's candidate buffer (composites)
constexpr int kWideList = 2048;   // the most candidates ranked at once (write_ranked)
constexpr int kWideMaxChunks = 256;
constexpr int kListSlack = 64;  // a split row's chunk publishes twice its share of k and kListSlack more (at most k)
constexpr int kAgainE = 32;     // elements per lane of the merger's tiles when it reads chunks again from x
constexpr int kStageVecs = 192;    // vectors one wave may stage for its appends (Tile::stage_append)
constexpr int kStageMaxKeep = 512;  // staged appends for buffer targets up to this (about 1.3 / 4 of it per wave)
static_assert(kStageVecs * 20 <= (kWideCap - kWideList) / kWaves * 8,
              "a wave's staged vectors and indices fit its area");

constexpr int kRankBuckets = 4096;  // buckets of write_ranked (16-bit counters and first positions)

// The ordering of write_ranked (below) over m candidates (k <= m <= kWideList) held in registers: cin[r] where in[r],
// NS slots per thread, every candidate in [mn, mx] (mx the largest, or mn a lower bound: a candidate below it lands
// in the last bucket and is still ordered exactly). `zeroed`: the caller has zeroed the counters (s.buf[kWideList,
// kWideList + kRankBuckets / 4)) behind a barrier. The scatter into s.buf[0, m) follows the barriers of the counts, so
// the caller's reads of it before the call need no barrier of their own. Every thread calls it.
template <typename T, int NS, typename S>
__device__ __forceinline__ void write_ranked_regs(S& s, const u64 (&cin)[NS], const bool (&in)[NS], int m, int k,
                                                  void* values, long long* indices, long long row, u64 mx, u64 mn,
                                                  bool zeroed) {
  constexpr int P = kWideList / kThreads;
  constexpr int BPT = kRankBuckets / kThreads;  // buckets per thread in the scan
  static_assert(kWideList * 2 <= kWideCap && kRankBuckets * 2 * sizeof(uint16_t) <= kWideList * sizeof(u64) &&
                    kWideList < 65536 && BPT % 2 == 0,
                "the bucketed copy, the counters and the first positions share the buffer; counts fit 16 bits");
  const int t = (int)threadIdx.x;
  const u64 range = mx - mn;
  const int bits = range ? 64 - __clzll(range) : 0;
  const int sh = bits > 12 ? bits - 12 : 0;  // (mx - mn) >> sh < 4096 = kRankBuckets
  u64* sorted = s.buf;
  unsigned* cnt2 = reinterpret_cast<unsigned*>(s.buf + kWideList);  // bucket b's count: half b & 1 of word b >> 1
  uint16_t* first = reinterpret_cast<uint16_t*>(cnt2 + kRankBuckets / 2);
  auto count_of = [&](int b) { return (int)((cnt2[b >> 1] >> (16 * (b & 1))) & 0xffffu); };
  if (!zeroed) {
    for (int w = t; w < kRankBuckets / 2; w += kThreads) cnt2[w] = 0;
    __syncthreads();
  }
  int bk[NS], slot[NS];
#pragma unroll
  for (int r = 0; r < NS; ++r) {
    const u64 d = (mx - cin[r]) >> sh;
    bk[r] = d < (u64)kRankBuckets ? (int)d : kRankBuckets - 1;
    const int half = 16 * (bk[r] & 1);
    slot[r] = in[r] ? (int)((atomicAdd(&cnt2[bk[r] >> 1], 1u << half) >> half) & 0xffffu) : 0;
  }
  __syncthreads();
  TOPK_STAGE(12);
  // exclusive scan of the counts, bucket 0 (the largest candidates) first
  unsigned own[BPT], sum = 0;
#pragma unroll
  for (int i = 0; i < BPT; i += 2) {
    const unsigned w = cnt2[(t * BPT + i) >> 1];
    own[i] = w & 0xffffu;
    own[i + 1] = w >> 16;
    sum += own[i] + own[i + 1];
  }
  const unsigned incl = wave_incl_u32(sum);
  if (lane_id() == kWave - 1) s.wsum[wave_id()] = incl;
  __syncthreads();
  unsigned run = incl - sum;
  for (int w = 0; w < wave_id(); ++w) run += s.wsum[w];
#pragma unroll
  for (int i = 0; i < BPT; ++i) {
    first[t * BPT + i] = (uint16_t)run;
    run += own[i];
  }
  __syncthreads();
  TOPK_STAGE(13);
#pragma unroll
  for (int r = 0; r < NS; ++r)
    if (in[r]) sorted[first[bk[r]] + slot[r]] = cin[r];
  __syncthreads();
  TOPK_STAGE(14);
  // Ranked in bucket order: lane i takes sorted[i], so neighbouring lanes read the same bucket's members (LDS
  // broadcasts rather than scattered reads) and write neighbouring output positions. Every position first, then the
  // stores. A thread's reads are issued together, stage by stage (its entries, their buckets' ranges, the buckets'
  // first four members), with no branch between them but the block-uniform one that skips the entry slots r with
  // r * kThreads >= m (128 x 128256 at k = 65 fills one of the eight): every index stays inside the buffer whether or
  // not the entry exists (i < kWideList; f + 3 <= m + 3 < kWideCap), and a missing entry's position is discarded.
  // Buckets of more than four members (rare) are finished after.
  u64 c[P];
  int pos[P], f[P], n[P];
#pragma unroll
  for (int r = 0; r < P; ++r) {
    if (r * kThreads >= m) break;
    c[r] = sorted[r * kThreads + t];
    const u64 d = (mx - c[r]) >> sh;
    const int b = d < (u64)kRankBuckets ? (int)d : kRankBuckets - 1;
    f[r] = (int)first[b];
    n[r] = count_of(b);
  }
#pragma unroll
  for (int r = 0; r < P; ++r) {
    if (r * kThreads >= m) break;
    const u64 a = sorted[f[r]], e1 = sorted[f[r] + 1], e2 = sorted[f[r] + 2], e3 = sorted[f[r] + 3];
    pos[r] = f[r] + (a > c[r]) + (1 < n[r] && e1 > c[r]) + (2 < n[r] && e2 > c[r]) + (3 < n[r] && e3 > c[r]);
  }
#pragma unroll
  for (int r = 0; r < P; ++r) {
    if (r * kThreads >= m) break;
    if (r * kThreads + t >= m) {
      pos[r] = k;
      continue;
    }
    for (int j = 4; j < n[r]; j += 4) {
      const int g = f[r] + j;
      const u64 a = sorted[g], e1 = sorted[g + 1], e2 = sorted[g + 2], e3 = sorted[g + 3];
      pos[r] += (a > c[r]) + (j + 1 < n[r] && e1 > c[r]) + (j + 2 < n[r] && e2 > c[r]) + (j + 3 < n[r] && e3 > c[r]);
    }
  }
  TOPK_STAGE_AT(15, pos[0]);
#pragma unroll
  for (int r = 0; r < P; ++r) {
    if (r * kThreads >= m) break;
    if (pos[r] < k) {
      if constexpr (sizeof(T) == 4) static_cast<uint32_t*>(values)[row * k + pos[r]] = composite_bits(c[r]);
      else static_cast<uint16_t*>(values)[row * k + pos[r]] = (uint16_t)(composite_bits(c[r]) >> 16);
      indices[row * k + pos[r]] = composite_index(c[r]);
    }
  }
}

// Writes the k largest of the m candidates s.buf[0, m) (k <= m <= kWideList), in order, as the output row, by
// write_ranked_regs: the candidates are bucketed by their distance below the largest, (max - c) >> sh with sh chosen
// so that the range fills kRankBuckets buckets, with 16-bit LDS counters (two to a word, so that counters and first
// positions fit beside the bucketed copy); an exclusive scan of the counts gives each bucket's first output position;
// the candidates are scattered by bucket into LDS, and each one's position is its bucket's first plus the number of
// its bucket's members above it. Nearly linear on spread-out values; a bucket holding many candidates (values
// clustered far below an outlier) costs its size per member. `lo`, when not 0, is a lower bound of the candidates known
// to the caller, used in place of their minimum (a candidate below it would still be ordered exactly: it lands in the
// last bucket, below every other bucket's members). `hi`, when not 0 (with lo not 0), is the largest candidate, known
// to the caller; the block is then not reduced here, and the caller's barrier after its writes of s.buf suffices.
// `zeroed`: the caller has zeroed the counters (s.buf[kWideList, kWideList + kRankBuckets / 4)) behind that barrier.
// Every thread calls it.
template <typename T, typename S>
__device__ __forceinline__ void write_ranked(S& s, int m, int k, void* values, long long* indices, long long row,
                                             u64 lo, u64 hi = 0, bool zeroed = false) {
  constexpr int P = kWideList / kThreads;
  const int t = (int)threadIdx.x;
  u64 c[P];
  bool in[P];
  u64 mx = 0, mn = ~0ull;
#pragma unroll
  for (int r = 0; r < P; ++r) {
    const int i = r * kThreads + t;
    in[r] = i < m;
    c[r] = in[r] ? s.buf[i] : 0ull;
    if (in[r]) {
      mx = c[r] > mx ? c[r] : mx;
      mn = c[r] < mn ? c[r] : mn;
    }
  }
  if (hi && lo) {  // the reads above need no barrier before the writes below: the counters lie past s.buf[0, m), and
    mx = hi;        // the scatter into s.buf[0, m) comes after the barriers of the counts
    mn = lo;
  } else {
    mx = block_ext64<true>(mx, s);  // also orders every read of s.buf above before the writes below
    mn = lo ? lo : block_ext64<false>(mn, s);
  }
  write_ranked_regs<T>(s, c, in, m, k, values, indices, row, mx, mn, zeroed);
}

// Writes the k largest of a chunk's m candidates s.buf[0, m) (k < m <= kWideList) to list[0, k) with device-coherent
// stores, in no particular order, and returns the k-th largest (the smallest written), block-uniform: the candidates
// stay in registers from one read. Their keys are counted in kRankBuckets 16-bit LDS counters, bucket (hi - key) >> sh,
// with [lo, hi] the caller's range of the keys (hi the chunk's largest, lo its admission key; a candidate below lo,
// kept from an earlier tile, counts in the last bucket) and sh set so that it fills them. A scan finds the bucket B
// holding the k-th. When B is kept whole (the usual case: about m / kRankBuckets members), everything in buckets up to
// B is kept and the k-th is the smallest of B, from a reduction over the kept candidates; otherwise B's members are
// gathered and ranked among themselves for the k-th. Each thread stores its kept candidates at positions from a block
// scan of the kept counts. A bucket of more than kThreads members (values clustered far below an outlier) takes the
// general prune (histogram narrowing) and stores the buffer. `zeroed`: the caller has zeroed the counters
// (s.buf[kWideList, kWideList + kRankBuckets / 4)) and s.members behind a barrier. Every thread calls it; the block is
// synchronized on entry (the caller's) and on return.
template <typename S>
__device__ __forceinline__ u64 cut_publish(S& s, int m, int k, u64* list, uint32_t lo, uint32_t hi, bool zeroed) {
  constexpr int P = kWideList / kThreads;
  constexpr int BPT = kRankBuckets / kThreads;  // buckets per thread in the scan (BPT / 4 u64 words of counters)
  static_assert(BPT % 4 == 0 && kWideList < 65536, "counts fit 16 bits");
  const int t = (int)threadIdx.x, lane = lane_id(), wave = wave_id();
  unsigned* cnt2 = reinterpret_cast<unsigned*>(s.buf + kWideList);  // bucket b: half b & 1 of word b >> 1
  u64* members = s.buf + kWideList + kRankBuckets / 4;                // after the counters (kRankBuckets * 2 bytes)
  u64* own = reinterpret_cast<u64*>(cnt2) + t * (BPT / 4);
  if (!zeroed) {
#pragma unroll
    for (int i = 0; i < BPT / 4; ++i) own[i] = 0ull;  // past the candidates (m <= kWideList)
    if (t == 0) s.members = 0;
    __syncthreads();
  }
  lo = lo < hi ? lo : hi;
  const uint32_t D = hi - lo;
  const int sh = (D >> 12) ? (32 - __builtin_clz(D)) - 12 : 0;  // D >> sh < kRankBuckets
  // the candidate slots in use (block-uniform): the rest are skipped as a block (128 x 128256 at k = 1024: 2 of 8)
  const int used = (m + kThreads - 1) / kThreads;
  u64 c[P];
  int bk[P];
#pragma unroll
  for (int r = 0; r < P; ++r) {
    c[r] = 0ull;
    bk[r] = kRankBuckets;
  }
#pragma unroll
  for (int r = 0; r < P; ++r) {
    if (r >= used) break;
    const int i = r * kThreads + t;
    c[r] = i < m ? s.buf[i] : 0ull;
    const uint32_t d = (hi - (uint32_t)(c[r] >> 32)) >> sh;
    bk[r] = i < m ? (d < (uint32_t)kRankBuckets ? (int)d : kRankBuckets - 1) : kRankBuckets;
    if (bk[r] < kRankBuckets) atomicAdd(&cnt2[bk[r] >> 1], 1u << (16 * (bk[r] & 1)));
  }
  __syncthreads();
  // the bucket holding position k - 1 (bucket 0 holds the largest candidates)
  unsigned cn[BPT], sum = 0;
#pragma unroll
  for (int i = 0; i < BPT / 4; ++i) {
    const u64 w = own[i];
    cn[4 * i] = (unsigned)w & 0xffffu;
    cn[4 * i + 1] = (unsigned)w >> 16;
    cn[4 * i + 2] = (unsigned)(w >> 32) & 0xffffu;
    cn[4 * i + 3] = (unsigned)(w >> 48);
  }
#pragma unroll
  for (int i = 0; i < BPT; ++i) sum += cn[i];
  const unsigned incl = wave_incl_u32(sum);
  if (lane == kWave - 1) s.wsum[wave] = incl;
  __syncthreads();
  unsigned run = incl - sum;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) run += w < wave ? s.wsum[w] : 0u;
  if (run < (unsigned)k && (unsigned)k <= run + sum) {
    // the last bucket whose count from the top before it is short of k (no register array indexed at run time)
    unsigned acc = run, before = run, here = 0;
    int at = 0;
#pragma unroll
    for (int i = 0; i < BPT; ++i) {
      const bool short_of_k = acc < (unsigned)k;
      at = short_of_k ? i : at;
      before = short_of_k ? acc : before;
      here = short_of_k ? cn[i] : here;
      acc += cn[i];
    }
    s.bin = t * BPT + at;
    s.above = (int)before;
    s.hist[0] = here;
  }
  __syncthreads();
  const int B = s.bin, rb = k - s.above, pop = (int)s.hist[0];  // the k-th is the rb-th largest of bucket B's pop
  u64 kth = 0, least = 0;  // the k-th (found below when B is kept whole); the smallest composite kept from bucket B
  const bool whole = rb == pop && B < kRankBuckets - 1;  // B kept whole: every member of B is at or above the k-th
  if (!whole) {
    if (pop > kThreads) {
      prune(s, k);
      for (int i = t; i < k; i += kThreads)
        __hip_atomic_store(list + i, s.buf[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return s.thr;
    }
#pragma unroll
    for (int i = 0; i < P; ++i) {
      if (i >= used) break;
      if (bk[i] == B) members[atomicAdd(&s.members, 1)] = c[i];
    }
    __syncthreads();
    if (t < pop) {
      const u64 mem = members[t];
      int above = 0;
      for (int j = 0; j < pop; ++j) above += members[j] > mem;
      if (above == rb - 1) s.pick = mem;
    }
    __syncthreads();
    kth = least = s.pick;
  }
  // positions (exactly k kept), slot-major: every thread's slot i before any slot i + 1, waves in order within a slot
  // and lanes in order within a wave, so that one store instruction writes a contiguous run (coherent stores of
  // scattered 8-byte entries each cost the memory a whole sector)
  bool keep[P];
  u64 km[P];
  unsigned* per = s.hist + 64;  // [P][kWaves] kept counts (s.hist[0] holds pop, read above without a barrier since)
  u64 mn = ~0ull;               // B kept whole: the smallest kept
#pragma unroll
  for (int i = 0; i < P; ++i) {
    keep[i] = false;
    km[i] = 0ull;
  }
#pragma unroll
  for (int i = 0; i < P; ++i) {
    if (i >= used) break;
    keep[i] = bk[i] < B || (bk[i] == B && c[i] >= least);
    km[i] = __ballot(keep[i]);
    if (lane == 0) per[i * kWaves + wave] = (unsigned)__popcll(km[i]);
    if (whole) mn = keep[i] && c[i] < mn ? c[i] : mn;
  }
  if (whole) {
    mn = wave_ext64<false>(mn);
    if (lane == 0) s.red2[wave] = mn;
  }
  __syncthreads();
  if (whole) {
#pragma unroll
    for (int w = 0; w < kWaves; ++w) mn = s.red2[w] < mn ? s.red2[w] : mn;
    kth = mn;
  }
  unsigned base = 0;
#pragma unroll
  for (int i = 0; i < P; ++i) {
    if (i >= used) break;
    unsigned before = 0, all = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const unsigned v = per[i * kWaves + w];
      before += w < wave ? v : 0u;
      all += v;
    }
    if (keep[i])
      __hip_atomic_store(list + base + before + lanes_below(km[i]), c[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    base += all;
  }
  return kth;
}

// A lower bound of the k-th largest of the wave's values v[i] (N per lane; 0 marks no value and is never counted) with
// at least k values at or above it; 0 when the wave holds fewer than k values. The bitwise search of wave_kth32 over N
// values per lane, over [max(lo, smallest value), largest value]: `lo` (wave-uniform) must not exceed the k-th largest,
// and a higher one resolves the same number of bits more finely. The range is first tried from two binades below the
// largest value (one more ballot per value), kept when k values lie at or above that end: the smallest value is often
// far below the k-th (group maxima of both signs), and 12 bits over the whole range resolve the bound to a quarter.
template <int N>
__device__ __forceinline__ uint32_t wave_kth_multi(const uint32_t (&v)[N], int k, uint32_t lo) {
  uint32_t mx = 0, mn = 0xffffffffu;
  int real = 0;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    mx = v[i] > mx ? v[i] : mx;
    mn = v[i] != 0 && v[i] < mn ? v[i] : mn;
    real += __popcll(__ballot(v[i] != 0));
  }
  if (real < k) return 0u;
  mx = wave_ext32<true>(mx);
  mn = wave_ext32<false>(mn);
  mn = lo > mn ? lo : mn;
  if (mx <= mn) return mx;
  constexpr uint32_t kTwoBinades = 2u << 23;
  if (mx - mn > kTwoBinades) {
    const uint32_t near = mx - kTwoBinades;
    int c = 0;
#pragma unroll
    for (int i = 0; i < N; ++i) c += __popcll(__ballot(v[i] >= near));
    if (c >= k) mn = near;
  }
  const int top = 31 - __builtin_clz(mx ^ mn);
  uint32_t p = mx & ~((2u << top) - 1u);
  for (int b = top; b >= 0 && b > top - kThrBits; --b) {
    const uint32_t cand = p | (1u << b);
    int c = 0;
#pragma unroll
    for (int i = 0; i < N; ++i) c += __popcll(__ballot(v[i] >= cand));
    if (c >= k) p = cand;
  }
  return p;
}

constexpr uint32_t kBoundWindow = (1u << 24) - 1u;  // two binades of fp32 keys below the largest, less one

// The block's k- and q-bounds of a tile from its group maxima g (0: no group): the k-th (q-th) largest of the block's
// group maxima has k (q) distinct elements at or above it. They are counted in kRankBuckets buckets (16-bit LDS
// counters, two to a word) over the window [M - kBoundWindow, M] below the largest, M: bucket (M - g) >> sh, sh set
// so that the window fits. Where the count from the top first reaches k (q), bucket b, the bound is that bucket's
// lower edge M - ((b + 1) << sh) + 1 (1 if that is not positive): every group maximum of buckets 0..b is at or above
// it, and it lies within 2^sh of the k-th (q-th) largest. One count per group instead of a ballot per group and
// candidate bit. Returns false, with no bounds, when fewer than k group maxima lie in the window (group maxima spread
// over more than two binades; the caller then searches each wave's whole range). q = 0 asks for no q-bound (bq = 0).
// A third count, k2 (0: none), gives bk2 the same way, or 0 when fewer than k2 group maxima lie in the window.
// Uses the last kRankBuckets / 4 entries of s.buf (the buffer holds at most kWideCap - kWideList candidates between
// tiles). M is set to the largest group maximum (the tile's largest key) in every case. Every thread calls it; the
// result is block-uniform.
template <typename S>
__device__ __forceinline__ bool hist_bounds(S& s, BlockRed& red, const uint32_t (&g)[kWideGroups], int k, int q,
                                            int k2, uint32_t& bk, uint32_t& bq, uint32_t& bk2, uint32_t& M) {
  constexpr int BPT = kRankBuckets / kThreads;  // buckets per thread in the scan (BPT / 4 u64 words of counters)
  static_assert(kRankBuckets / 4 <= kWideList && BPT % 4 == 0 && kThreads * kWideGroups < 65536,
                "the counters lie past the candidates kept between tiles; counts fit 16 bits");
  // bucket b: half b & 1 of word b >> 1
  unsigned* cnt2 = reinterpret_cast<unsigned*>(s.buf + kWideCap - kRankBuckets / 4);
  const int t = (int)threadIdx.x;
  u64* mine = reinterpret_cast<u64*>(cnt2) + t * (BPT / 4);
#pragma unroll
  for (int i = 0; i < BPT / 4; ++i) mine[i] = 0ull;
  uint32_t mx = 0;
#pragma unroll
  for (int i = 0; i < kWideGroups; ++i) mx = g[i] > mx ? g[i] : mx;
  M = red.max(wave_ext32<true>(mx));  // its barrier also orders the zeroing before the counts
  if (M == 0) return false;
  const uint32_t lo = M > kBoundWindow ? M - kBoundWindow : 1u;
  const uint32_t D = M - lo;
  const int sh = (D >> 12) ? (32 - __builtin_clz(D)) - 12 : 0;  // D >> sh < 4096 = kRankBuckets
#pragma unroll
  for (int i = 0; i < kWideGroups; ++i) {
    if (g[i] >= lo) {
      const uint32_t b = (M - g[i]) >> sh;
      atomicAdd(&cnt2[b >> 1], 1u << (16 * (b & 1)));
    }
  }
  __syncthreads();
  // (the tile's registers are live here: the counts stay packed, four to a u64, and are unpacked where used)
  u64 w4[BPT / 4];
  uint32_t sum = 0;
#pragma unroll
  for (int i = 0; i < BPT / 4; ++i) {
    w4[i] = mine[i];
    const uint32_t lo = (uint32_t)w4[i], hi = (uint32_t)(w4[i] >> 32);
    sum += (lo & 0xffffu) + (lo >> 16) + (hi & 0xffffu) + (hi >> 16);
  }
  const uint32_t incl = wave_incl_u32(sum);
  const int wv = __builtin_amdgcn_readfirstlane(wave_id());  // (a scalar: a vector copy was spilled to memory)
  if (lane_id() == kWave - 1) s.wsum[wv] = incl;
  __syncthreads();
  uint32_t run = incl - sum, total = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const uint32_t v = s.wsum[w];
    run += w < wv ? v : 0u;
    total += v;
  }
  if (total < (uint32_t)k) return false;
  // the thread whose buckets hold the k-th (q-th) from the top records the bucket: the last one whose count from the
  // top before it is short of k (q); only the waves holding such a thread walk their buckets
  const bool hk = run < (uint32_t)k && (uint32_t)k <= run + sum, hq = run < (uint32_t)q && (uint32_t)q <= run + sum;
  const bool hk2 = run < (uint32_t)k2 && (uint32_t)k2 <= run + sum;
  if (hk || hq || hk2) {
    uint32_t acc = run;
    int atk = 0, atq = 0, atk2 = 0;
#pragma unroll
    for (int i = 0; i < BPT; ++i) {
      atk = acc < (uint32_t)k ? i : atk;
      atq = acc < (uint32_t)q ? i : atq;
      atk2 = acc < (uint32_t)k2 ? i : atk2;
      acc += (uint32_t)(w4[i >> 2] >> (16 * (i & 3))) & 0xffffu;
    }
    if (hk) s.hist[0] = (unsigned)(t * BPT + atk);
    if (hq) s.hist[1] = (unsigned)(t * BPT + atq);
    if (hk2) s.hist[2] = (unsigned)(t * BPT + atk2);
  }
  __syncthreads();
  auto edge = [&](unsigned b) {
    const u64 below = (u64)(b + 1) << sh;
    return below >= (u64)M ? 1u : M - (uint32_t)below + 1u;
  };
  bk = edge(s.hist[0]);
  bq = q > 0 ? edge(s.hist[1]) : 0u;
  bk2 = k2 > 0 && (uint32_t)k2 <= total ? edge(s.hist[2]) : 0u;
  return true;
}

// 64 < k <= 1024: one 256-thread workgroup per (chunk, row), the chunk in register tiles as topk_tile. A split row's
// chunk admits its candidates at an m-bound, m = min(k, 2 ceil(k * chunk / cols) + kListSlack): twice a full chunk's
// share of the row's k and a margin (128 x 128256 at k = 1024: 326 of 16384), so that rows whose largest values cluster
// in one chunk at up to about twice the density elsewhere need no second look at x. Per tile: each lane's 64 elements
// form kWideGroups groups; a group's largest element has the group behind it, so the m-th largest of the block's group
// maxima has m distinct elements at or above it: with the m-th of the earlier tiles it is the admission key (about
// 1.1 m admitted per tile on continuous data). The q-th largest, q = ceil(k / nchunks), gives a q-bound the same way.
// Admitted elements are appended to an LDS buffer (fp32: through each wave's staging area; else one LDS atomic per wave
// and 16 elements per lane); a tile that overflows it (ties, adversarial orders) is appended again vector by vector
// from the buffer's m-th, pruning to m (histogram narrowing) whenever a vector might not fit. An unsplit row keeps k,
// ranks its candidates (write_ranked) and writes the first k.
//
// A split row's chunk writes its list to the caller's work: the row's [nchunks, k] slots hold the nchunks lists of ls
// entries (zero-padded), then, when m < k, each chunk's separator. When m < k the list is the chunk's candidates at or
// above the separator, the larger of the admission key and the prunes' floor, as they are (no cut) when they fit ls;
// else (and when m = k) its m largest, with the smallest of them as the separator (0: the list holds every element of
// the chunk). The header (k-bound key << 32 | q-bound key; when m < k the k-bound comes from a third count of the group
// maxima, or is 0) goes to indices[row * k + part] (the row's output, not yet written: nchunks <= k), all with
// device-coherent stores, and the chunk counts its arrival on counters[row] (block_hand_off). The row's last arrival
// merges. The smallest q-bound (nchunks * q >= k elements at or above it) and the largest k-bound bound the row's k-th
// largest T from below: the floor. Every element a chunk left out lies below its separator, and every list entry at
// or above it; so when at least k list entries lie at or above the largest separator S (then T >= S), every element at
// or above T is in the lists, and the lists' entries at or above the floor (about 1.4 k) are gathered, ranked and the
// first k written out. Otherwise (a chunk holding more than m of the row's k largest: sorted rows, ties, values
// clustered by index) the merger reads again from x the chunks that may have left out part of the row's k largest
// (below). The counter is zeroed for the next launch either way.
template <typename T, bool VEC, bool DRAW>
__global__ void __launch_bounds__(kThreads, 4)  // four waves per SIMD: 128 VGPRs, four workgroups per CU
    topk_wide(const T* __restrict__ x, void* __restrict__ values, long long* __restrict__ indices,
              u64* __restrict__ work, unsigned* __restrict__ counters, long long cols, long long chunk, int nchunks,
              int k, SampleArgs sa) {
  if constexpr (!DRAW) sa.out = nullptr;  // a launch without the draw: its code compiles away
  __shared__ Smem<kWideCap> s;
  __shared__ uint32_t redslots[2][kWaves];
  const long long row = blockIdx.y;
  const int part = blockIdx.x;
  const int begin = (int)((long long)part * chunk);
  const int end = (int)(begin + chunk < cols ? begin + chunk : cols);
  const T* xr = x + row * cols;
  BlockRed red;
  red.slot = redslots;
  red.phase = 0;
  const int q = (k + nchunks - 1) / nchunks;
  // entries each chunk publishes: twice a full chunk's share of the row's k (the last chunk may be shorter) and a
  // margin, at most k
  const long long share = ((long long)k * chunk + cols - 1) / cols;
  const int m = nchunks > 1 && 2 * share + kListSlack < k ? 2 * (int)share + kListSlack : k;
  // the lists' stride: when m < k, room for the candidates at or above the admission key, which has m distinct
  // elements at or above it (about 1.1 m on continuous data), and less than k, so that the separators fit after the
  // lists in the row's nchunks * k slots of work
  const int lsr = (m + m / 8 + 16 + 63) / 64 * 64;
  const int ls = m < k ? (lsr < k ? lsr : k - 1) : m;
  const bool split = nchunks > 1;
  const int kt = split ? m : k;  // the buffer's target: the chunk's m largest, or the row's k
  uint32_t thr = 0, thq = 0, cmax = 0;  // the admission key, the q-bound, the chunk's largest key
  uint32_t thk = 0;                     // m < k: a k-bound (k distinct elements of the chunk at or above it), or 0
  if (threadIdx.x == 0) {
    s.count = 0;
    s.thr = 1;
  }
  __syncthreads();
  TOPK_STAGE(0);
  const int kw = (kt + kWaves - 1) / kWaves, kwq = (q + kWaves - 1) / kWaves;
  using TL = Tile<T, VEC>;
  constexpr int TE = kThreads * kTileE;
  constexpr int kStep = kThreads * TL::W;  // what one vector of a tile may append
  for (int t0 = begin; t0 < end; t0 += TE) {
    TL tile;
    tile.load(xr, t0, end);
    const int cnt0 = s.count;  // block-uniform: the buffer is settled between tiles
    uint32_t g[kWideGroups];
    tile.group_keys(g);
    TOPK_STAGE_AT(1, g[0]);
    TOPK_WAVE_STAGE_AT(g[0]);
    uint32_t tb, qb, kb2 = 0, tm;
    if (!hist_bounds(s, red, g, kt, split ? q : 0, kt < k ? k : 0, tb, qb, kb2, tm)) {
      // the group maxima spread over more than the window: each wave's bound from a search over its whole range
      const uint32_t tw = wave_kth_multi<kWideGroups>(g, kw, 0u);
      tb = red.min(tw);
      // q <= kt, so the wave's q-th largest group maximum is at or above its kt-bound: the search starts there (the
      // groups' smallest maximum is often negative, and 12 bits over that range resolve the bound to about 0.5)
      qb = split ? red.min(wave_kth_multi<kWideGroups>(g, kwq, tw)) : 0u;
    }
    thr = tb > thr ? tb : thr;
    thq = qb > thq ? qb : thq;
    thk = __builtin_amdgcn_readfirstlane(kb2 > thk ? kb2 : thk);  // (block-uniform: kept in a scalar register)
    cmax = tm > cmax ? tm : cmax;
    TOPK_STAGE(2);
    tile.opaque();
    bool redo = true;
    if (thr > TL::kSentinelKey) {
      int lim = kWideCap;
      if (!(thr & 0x80000000u)) {
        tile.template filter_append<true>(s, thr, lim);
      } else if (sizeof(T) == 4 && cnt0 == 0 && kt <= kStageMaxKeep) {
        // fp32 over a non-negative bound, the tile's candidates into an empty buffer: each wave stages its vectors
        // reaching the bound in its quarter of s.buf[kWideList, kWideCap) (free after the bounds' last read), and
        // the appends stay below kWideList meanwhile
        lim = kWideList;
        u32x4* stage = reinterpret_cast<u32x4*>(s.buf + kWideList + wave_id() * ((kWideCap - kWideList) / kWaves));
        if constexpr (sizeof(T) == 4) {
          if (!tile.template stage_append<kStageVecs>(s, thr, stage, reinterpret_cast<uint32_t*>(stage + kStageVecs),
                                                      lim))
            tile.template filter_append<false>(s, thr, lim);
        }
      } else {
        tile.template filter_append<false>(s, thr, lim);
      }
      __syncthreads();
      redo = s.count > lim;
    }
    if (redo) {  // every element may pass, or the buffer overflowed: append again vector by vector, pruning to kt
      __syncthreads();
      if (threadIdx.x == 0) s.count = cnt0;
      __syncthreads();
      const u64 bound = thr > TL::kSentinelKey ? (u64)thr << 32 : 0ull;
      for (int v = 0; v < TL::NV; ++v) {
        if (prune_due(s, kWideCap - kStep)) prune(s, kt);
        const u64 floor = s.thr > bound ? s.thr : bound;
        tile.append_first(s, v, floor);
        __syncthreads();
      }
    }
    if (end - t0 > TE && s.count > kWideCap - kWideList) {  // before another tile: room for a tile's candidates
      prune(s, kt);
      const uint32_t kk = (uint32_t)(s.thr >> 32);
      thr = kk > thr ? kk : thr;
    }
  }
  if (!split) {
    const float u = sa.uniform(row);
    if (s.count > kWideList) prune(s, k);
    write_ranked<T>(s, s.count, k, values, indices, row, 0ull);
    sample_list<T>(sa, u, values, indices, row, k);
    return;
  }
  TOPK_STAGE(3);
  // publish: the list (zero-padded to ls), its separator (m < k) and the header (k-bound key << 32 | q-bound key) in
  // the row's output. When m < k the list holds the chunk's candidates as they are when they fit ls (128 x 128256 at
  // k = 1024: about 350 of at most 384), else their m largest (cut_publish).
  u64* wr = work + row * (long long)nchunks * k;
  u64* mine = wr + (long long)part * ls;
  if (s.count > kWideList) prune(s, m);
  const int n = s.count;
  u64 kth = 0;  // the separator (m < k): every element of the chunk not in its list lies below it (0: none is left out)
  if (n > ls) {
    kth = cut_publish(s, n, m, mine, thr, cmax, false);  // the m-th largest, the smallest entry of the list
    for (int i = m + (int)threadIdx.x; i < ls; i += kThreads)
      __hip_atomic_store(mine + i, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {
    if (m < k) {
      // Every element left out lies below the last admission key (those of earlier tiles were no higher) or below the
      // prunes' floor s.thr. Candidates below the separator (admitted by an earlier tile's lower key, or by a 16-bit
      // compare of the key's upper half) are left out too, so that every list entry lies at or above it (the second
      // look at x reads a chunk's elements below its separator only). The key has m distinct elements at or above it,
      // all kept: with fewer than m candidates (no usable bound: every element appended) none is left out.
      const u64 ak = (u64)thr << 32;
      kth = n < m ? 0ull : ak > s.thr ? ak : s.thr;
    } else if (n == m) {  // (block-uniform) the chunk's k largest: their smallest gives the header's k-bound
      u64 mn = ~0ull;
      for (int i = threadIdx.x; i < n; i += kThreads) mn = s.buf[i] < mn ? s.buf[i] : mn;
      kth = block_ext64<false>(mn, s);
    }
    for (int i = threadIdx.x; i < ls; i += kThreads) {
      const u64 e = i < n ? s.buf[i] : 0ull;
      __hip_atomic_store(mine + i, e >= kth ? e : 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  TOPK_STAGE(4);
  u64* heads = reinterpret_cast<u64*>(indices + row * k);
  u64* seps = wr + (long long)nchunks * ls;  // m < k: nchunks * (ls + 1) <= nchunks * k slots of the row
  if (threadIdx.x == 0) {
    const uint32_t kb = m < k ? thk : (uint32_t)(kth >> 32) > thr ? (uint32_t)(kth >> 32) : thr;
    __hip_atomic_store(heads + part, ((u64)kb << 32) | thq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (m < k) __hip_atomic_store(seps + part, kth, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  const bool last = block_hand_off(s, counters + row, nchunks);
  TOPK_STAGE(5);
  if (!last) return;
  const float u = sa.uniform(row);
  // merge (the row's last arrival): the floor from the headers, then every list's entries at or above it
  auto ld = [&](const u64* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
  const int t = (int)threadIdx.x, lane = lane_id(), wave = wave_id();
  // Rows whose lists fit the registers (128 x 128256: 8 x 384 entries) read them all at once, right after the headers:
  // the floor's reduction runs while the lists' loads are in flight (loads return in order), and one block scan places
  // the entries at or above it.
  constexpr int kGatherAll = 3072;  // list entries the merger reads in one batch
  constexpr int PB = kGatherAll / kThreads;
  const int entries = nchunks * ls;  // the row's lists, contiguous in wr
  u64 kmax = 0, qmn = ~0ull, smax = 0;
  const u64 h0 = t < nchunks ? ld(heads + t) : 0ull;
  const u64 s0 = m < k && t < nchunks ? ld(seps + t) : 0ull;
  u64 e[PB];
  if (entries <= kGatherAll) {
#pragma unroll
    for (int i = 0; i < PB; ++i) {
      const int at = i * kThreads + t;
      e[i] = at < entries ? ld(wr + at) : 0ull;
    }
  }
  for (int c = t; c < nchunks; c += kThreads) {
    const u64 h = c == t ? h0 : ld(heads + c);
    const u64 sp = m == k ? 0ull : c == t ? s0 : ld(seps + c);
    const u64 kb = h & 0xffffffff00000000ull, qb = h << 32;
    kmax = kb > kmax ? kb : kmax;
    qmn = qb < qmn ? qb : qmn;
    smax = sp > smax ? sp : smax;
  }
  kmax = wave_ext64<true>(kmax);
  qmn = wave_ext64<false>(qmn);
  smax = wave_ext64<true>(smax);
  if (lane == 0) {
    s.red[wave] = kmax;
    s.red2[wave] = qmn;
    s.red4[wave] = smax;
  }
  __syncthreads();
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    kmax = s.red[w] > kmax ? s.red[w] : kmax;
    qmn = s.red2[w] < qmn ? s.red2[w] : qmn;  // 0 when a chunk has no q-bound
    smax = s.red4[w] > smax ? s.red4[w] : smax;
  }
  u64 floor = kmax > qmn ? kmax : qmn;
  floor = floor > 1 ? floor : 1;
  TOPK_STAGE(6);
  bool whole = true;      // every element at or above T is in the lists
  bool gathered = false;  // the buffer holds the lists' entries at or above the floor
  if (entries <= kGatherAll) {
    unsigned n = 0, ns = 0;
    u64 mx = 0;
    bool keep[PB];
#pragma unroll
    for (int i = 0; i < PB; ++i) {
      keep[i] = e[i] >= floor;
      n += keep[i] ? 1u : 0u;
      ns += e[i] >= smax ? 1u : 0u;
      mx = keep[i] && e[i] > mx ? e[i] : mx;
    }
    const unsigned incl = wave_incl_u32(n);
    const unsigned wns = (unsigned)wave_sum((float)ns);  // exact: at most kGatherAll
    mx = wave_ext64<true>(mx);
    if (lane == kWave - 1) s.wsum[wave] = incl;
    if (lane == 0) {
      s.red3[wave] = mx;
      s.hist[wave] = wns;
    }
    // the ordering's counters, zeroed behind the barrier below (they stay zero unless more than kWideList are kept)
    u64* cz = s.buf + kWideList + t * (kRankBuckets / 4 / kThreads);
#pragma unroll
    for (int i = 0; i < kRankBuckets / 4 / kThreads; ++i) cz[i] = 0ull;
    __syncthreads();
    unsigned nm = 0, pos = incl - n, above = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      nm += s.wsum[w];
      pos += w < wave ? s.wsum[w] : 0u;
      mx = s.red3[w] > mx ? s.red3[w] : mx;
      above += s.hist[w];
    }
    whole = smax == 0 || above >= (unsigned)k;
    if (whole && nm <= (unsigned)kWideList) {
      // (block-uniform) ordered straight from the registers: the counters were zeroed behind the barrier above
      TOPK_STAGE(7);
      write_ranked_regs<T>(s, e, keep, (int)nm, k, values, indices, row, mx, floor, true);
      TOPK_STAGE(8);
      if (t == 0) __hip_atomic_store(counters + row, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      sample_list<T>(sa, u, values, indices, row, k);
      return;
    }
    if (nm <= (unsigned)kWideCap) {  // (block-uniform) all of them fit the buffer: one write
#pragma unroll
      for (int i = 0; i < PB; ++i)
        if (e[i] >= floor) s.buf[pos++] = e[i];
      if (t == 0) {
        s.count = (int)nm;
        s.thr = floor;
      }
      __syncthreads();
      if (whole) {
        TOPK_STAGE(7);
        if (nm > (unsigned)kWideList) prune(s, k);
        write_ranked<T>(s, s.count, k, values, indices, row, floor, mx, nm <= (unsigned)kWideList);
        TOPK_STAGE(8);
        if (t == 0) __hip_atomic_store(counters + row, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        sample_list<T>(sa, u, values, indices, row, k);
        return;
      }
      gathered = true;
    }
  }
  if (!gathered) {
    // longer rows (or more entries at the floor than the buffer holds): the lists in turn, pruning as they come
    if (t == 0) {
      s.count = 0;
      s.thr = floor;
    }
    __syncthreads();
    constexpr int PER = kMaxK / kThreads;  // list entries per thread (m <= kMaxK)
    constexpr int kInFlight = 2;           // lists whose loads are in flight while one is taken (4 measured no faster)
    static_assert(PER * kThreads <= kWideCap - kWideList, "room for a whole list above a buffer of kWideList");
    u64 cv[kInFlight][PER];
    unsigned ns = 0;  // entries at or above the largest separator
    auto load = [&](int c, u64 (&v)[PER]) {
      const u64* list = wr + (long long)c * ls;
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const int at = i * kThreads + (int)threadIdx.x;
        v[i] = at < ls ? ld(list + at) : 0ull;
      }
    };
    auto take = [&](const u64 (&v)[PER]) {  // appends the entries at or above the floor (room for a list is kept)
      if (prune_due(s, kWideCap - kWideList)) prune(s, k);
      const u64 f = s.thr;
      bool keep[PER];
      bool any = false;
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        keep[i] = v[i] >= f;
        any |= keep[i];
        ns += v[i] >= smax ? 1u : 0u;
      }
      if (__ballot(any)) append<PER>(s, v, keep);
      __syncthreads();
    };
#pragma unroll
    for (int j = 0; j < kInFlight; ++j)
      if (j < nchunks) load(j, cv[j]);
    for (int c = 0; c < nchunks; c += kInFlight) {
#pragma unroll
      for (int j = 0; j < kInFlight; ++j) {
        if (c + j < nchunks) {
          take(cv[j]);
          if (c + j + kInFlight < nchunks) load(c + j + kInFlight, cv[j]);
        }
      }
    }
    whole = smax == 0 || block_count((int)ns, s) >= k;
  }
  if (!whole) {
    // A chunk may hold more than m of the row's k largest. The buffer holds every list entry at or above the floor
    // (less entries pruned below its k-th), so its k-th largest L bounds T from below. The elements a chunk left out
    // lie below its separator: the chunks whose separator exceeds L are read again from x, and their elements in
    // [L, separator) appended, a tile at a time when the tile's count fits the buffer, else vector by vector, pruning
    // to k whenever a vector might not fit.
    const int n = s.count;
    u64 L = n >= k ? kth_largest(s, n, k) : floor;
    L = L > floor ? L : floor;
    TOPK_STAGE(9);
    const u64 again = __ballot(t < nchunks && s0 > L);  // (thread c holds chunk c's separator)
    if (lane == 0) s.red3[wave] = again;
    __syncthreads();
    using TR = Tile<T, VEC, kThreads, kAgainE>;
    for (int w = 0; w < kWaves; ++w) {
      u64 mask = s.red3[w];
      mask = (u64)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(mask >> 32)) << 32 |
             (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)mask);
      while (mask) {
        const int c = w * kWave + __builtin_ctzll(mask);
        mask &= mask - 1;
        const u64 sep = ld(seps + c);
        const u64 top = ((u64)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(sep >> 32)) << 32 |
                         (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)sep)) - 1u;  // (sep > L >= 1)
        const int c0 = (int)((long long)c * chunk), c1 = (int)(c0 + chunk < cols ? c0 + chunk : cols);
        for (int t0 = c0; t0 < c1; t0 += kThreads * kAgainE) {
          TR tile;
          tile.load(xr, t0, c1);
          // (s.thr and s.count are settled: the last step ended with a barrier; the count is read before the
          // barriers of block_count, so that no wave reads it after another wave's appends)
          const u64 f = s.thr > L ? s.thr : L;
          const int held = s.count;
          const int add = block_count(tile.count_range(f, top), s);
          tile.opaque();  // the composites are formed again below, not held from the count
          if (held + add <= kWideCap) {
            for (int v = 0; v < TR::NV; ++v) tile.append_first(s, v, f, top);
            __syncthreads();
          } else {
            for (int v = 0; v < TR::NV; ++v) {
              if (prune_due(s, kWideCap - kStep)) prune(s, k);
              tile.append_first(s, v, s.thr > L ? s.thr : L, top);
              __syncthreads();
            }
          }
        }
      }
    }
    TOPK_STAGE(10);
  }
  TOPK_STAGE(7);
  if (s.count > kWideList) prune(s, k);
  write_ranked<T>(s, s.count, k, values, indices, row, floor);  // every candidate kept is at or above the floor
  TOPK_STAGE(8);
  if (t == 0) __hip_atomic_store(counters + row, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  sample_list<T>(sa, u, values, indices, row, k);
}

// One wave per row of a top-k list (values [rows, k] in T, int64 indices, as topk writes them): out[row] drawn by
// sample_row.
template <typename T>
__global__ void __launch_bounds__(kWave)
    topk_sample(const void* __restrict__ values, const long long* __restrict__ indices, const float* __restrict__ u,
                long long* __restrict__ out, int k, float temperature, float top_p) {
  const long long row = blockIdx.x;
  const ListInMemory<T> list{values, indices, row, k};
  const auto index_at = [&](int i) { return list.index(i); };
  const long long drawn = k <= kWave ? sample_row<1>(list, index_at, k, u[row], temperature, top_p)
                                     : sample_row<kSamplePer>(list, index_at, k, u[row], temperature, top_p);
  if (lane_id() == 0) out[row] = drawn;
}

// ---- the naive tier ------------------------------------------------------------------------------------------------

// The naive tier (the harness's "seed" column; launch() takes it when tuning slot 1 is 1): one workgroup per row
// takes the row's k largest one at a time, each round a scan of the whole row, element by element, for the largest
// composite below the previous round's. Exact by construction (the composites are distinct) and k passes over the row.
template <typename T>
__global__ void __launch_bounds__(kThreads)
    topk_seed(const T* __restrict__ x, void* __restrict__ values, long long* __restrict__ indices, long long cols,
              int k) {
  __shared__ u64 part[kWaves];
  const long long row = blockIdx.x;
  const T* xr = x + row * cols;
  u64 prev = ~0ull;  // above every composite
  for (int r = 0; r < k; ++r) {
    u64 best = 0;  // below every composite of an element
    for (long long j = threadIdx.x; j < cols; j += kThreads) {
      uint32_t u;
      if constexpr (sizeof(T) == 4) u = reinterpret_cast<const uint32_t*>(xr)[j];
      else u = (uint32_t)reinterpret_cast<const uint16_t*>(xr)[j] << 16;
      const u64 c = composite(u, (uint32_t)j);
      best = c < prev && c > best ? c : best;
    }
    best = wave_ext64<true>(best);
    if (lane_id() == 0) part[wave_id()] = best;
    __syncthreads();
    u64 m = part[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) m = part[w] > m ? part[w] : m;
    __syncthreads();  // every wave has read part before the next round rewrites it
    if (threadIdx.x == 0) {
      if constexpr (sizeof(T) == 4) static_cast<uint32_t*>(values)[row * k + r] = composite_bits(m);
      else static_cast<uint16_t*>(values)[row * k + r] = (uint16_t)(composite_bits(m) >> 16);
      indices[row * k + r] = composite_index(m);
    }
    prev = m;
  }
}

// ---- host side ------------------------------------------------------------------------------------------------------

// Tuning slots (0 = automatic): 0 resident workgroups per CU assumed by plan(); 1 the naive tier for launch() (1).
enum { kTuneBlocksPerCu = 0, kTuneSeed = 1 };

// The chunking a launch of the caller's nchunks chunks of `chunk` columns actually runs, and the u64 slots of the
// caller's work it uses (0 for unsplit rows). The result does not depend on the chunking, so the launch may join
// chunks (fewer, longer ones), which keeps every slot it uses inside the caller's rows * nchunks * k:
//  - k <= 64: a last chunk too short to give each of the four waves a vector would leave a wave without a bound, and
//    the tile would take the exact re-push path; when the previous chunk can take it within one register tile, it
//    does. k = 1 uses one slot per chunk (its workgroups take four chunks each and use the first slots of the row).
//  - chunks shorter than kShortChunk are joined into chunks of one register tile (16384 elements), or of half of one
//    when that grid would have fewer than 64 workgroups (for k = 1 unless a row fits two tiles): a chunk's chain
//    after its loads costs about the same at any length up to a tile, and every chunk adds a list to its row's merge.
//    On MI355X, from the plan's chunks of 2048 or 4008 columns at k = 50: 1 x 128256 11.3 -> 9.4 us, 8 x 128256
//    16.8 -> 10.3 us, 32 x 128256 19.6 -> 12.2 us, 16 x 32000 11.5 -> 9.9 us; at k = 1: 32 x 128256 10.2 -> 6.9 us,
//    4 x 128256 6.3 -> 5.4 us, 16 x 32000 6.4 -> 4.8 us; at k = 300, from chunks of 16 k = 4800 columns: 8 x 128256
//    26.8 -> 13.1 us, 32 x 128256 33.6 -> 15.2 us.
//  - 1 < k <= 64: a row of two chunks within two register tiles is taken whole by one workgroup, tile after tile,
//    when there are at least as many rows as CUs (512 x 32000 fp32 at k = 50: 19.2 -> 17.6 us on MI355X; the chunks'
//    hand-off and merge cost more than the second tile's wait, while one workgroup per row still fills the GPU).
//  - k > 64: chunks long enough for a useful bound (16k elements: a tile holds the 4 * ceil(k / 4) group maxima the
//    bound needs), and at least as long as the joined chunks above (from the plan's 9496 columns at 64 x 151936:
//    k = 65 20.8 -> 19.1 us, k = 300 21.3 -> 19.7 us; 32 x 262144: k = 65 23.9 -> 18.3 us, k = 300 39.7 -> 19.4 us),
//    and few enough for the merge: at most kWideMaxChunks, and at most k, so that the chunks' bound headers fit the
//    row's output indices.
struct Chunking {
  long long chunk;
  int nchunks;
  long long slots;
};
constexpr long long kShortChunk = 8192;

Chunking chunking(long long rows, long long cols, long long chunk, int nchunks, int k, int width) {
  const long long tile = (long long)kThreads * kTileE;
  // the length short chunks are joined to (a multiple of 8); k = 1 takes a row of up to two tiles whole (its
  // workgroups take two chunks each)
  const bool whole_tiles = rows * ((cols + tile - 1) / tile) >= 64 || (k == 1 && cols <= 2 * tile);
  const long long joined = whole_tiles ? tile : tile / 2;
  if (k <= kSeedMaxK) {
    if (nchunks > 1 && chunk < kShortChunk) {
      const long long want = joined;
      if (want > chunk) {
        chunk = want < cols ? want : cols;
        nchunks = (int)((cols + chunk - 1) / chunk);  // fewer than the caller's: its work holds them
      }
    }
    const long long tail = cols - (long long)(nchunks - 1) * chunk;
    if (nchunks > 1 && tail < (long long)kThreads * width && chunk + tail <= (long long)kThreads * kTileE) --nchunks;
    if (k > 1 && nchunks == 2 && cols <= 2LL * kThreads * kTileE && rows >= rw_host::device_cus()) {
      chunk = cols;
      nchunks = 1;
    }
  } else {
    const long long most = k < kWideMaxChunks ? k : kWideMaxChunks;
    long long want = 16LL * k;
    if (want < joined) want = joined;
    if (want < (cols + most - 1) / most) want = (cols + most - 1) / most;
    if (chunk < want && nchunks > 1) {
      chunk = want < cols ? (want + 7) / 8 * 8 : cols;
      nchunks = (int)((cols + chunk - 1) / chunk);
    }
  }
  return Chunking{chunk, nchunks, nchunks > 1 ? rows * nchunks * (k == 1 ? 1LL : (long long)k) : 0LL};
}

// The kernels of a launch whose rows are split into nchunks chunks of `chunk` columns. work and counters are the
// caller's (work: u64 [rows * nchunks * k]; counters: u32 [rows], zero), rechunked by chunking().
template <typename T, bool VEC>
int launch_chunks(const void* x, void* values, void* indices, void* work, void* counters, long long rows,
                  long long cols, long long chunk0, int nchunks0, int k, const SampleArgs& sa, hipStream_t stream) {
  const Chunking c = chunking(rows, cols, chunk0, nchunks0, k, Tile<T, VEC>::W);
  const long long chunk = c.chunk;
  const int nchunks = c.nchunks;
  if (k <= kSeedMaxK) {
    if (k == 1) {
      const int groups = (nchunks + kOneChunks - 1) / kOneChunks;
      if (sa.out)
        hipLaunchKernelGGL((topk_one<T, VEC, true>), dim3((unsigned)groups, (unsigned)rows), dim3(kOneThreads), 0,
                           stream, (const T*)x, values, (long long*)indices, (u64*)work, (unsigned*)counters, cols,
                           chunk, nchunks, groups, sa);
      else
        hipLaunchKernelGGL((topk_one<T, VEC, false>), dim3((unsigned)groups, (unsigned)rows), dim3(kOneThreads), 0,
                           stream, (const T*)x, values, (long long*)indices, (u64*)work, (unsigned*)counters, cols,
                           chunk, nchunks, groups, sa);
      return (int)hipGetLastError();
    }
    if (sa.out)
      hipLaunchKernelGGL((topk_tile<T, VEC, true, false>), dim3((unsigned)nchunks, (unsigned)rows), dim3(kThreads), 0,
                         stream, (const T*)x, values, (long long*)indices, (u64*)work, (unsigned*)counters, cols,
                         chunk, nchunks, k, sa);
    else if (nchunks == 1)
      hipLaunchKernelGGL((topk_tile<T, VEC, false, true>), dim3(1u, (unsigned)rows), dim3(kThreads), 0, stream,
                         (const T*)x, values, (long long*)indices, (u64*)work, (unsigned*)counters, cols, chunk,
                         nchunks, k, sa);
    else
      hipLaunchKernelGGL((topk_tile<T, VEC, false, false>), dim3((unsigned)nchunks, (unsigned)rows), dim3(kThreads), 0,
                         stream, (const T*)x, values, (long long*)indices, (u64*)work, (unsigned*)counters, cols,
                         chunk, nchunks, k, sa);
    return (int)hipGetLastError();
  }
  const dim3 wgrid((unsigned)nchunks, (unsigned)rows);
  if (sa.out)
    hipLaunchKernelGGL((topk_wide<T, VEC, true>), wgrid, dim3(kThreads), 0, stream, (const T*)x, values,
                       (long long*)indices, (u64*)work, (unsigned*)counters, cols, chunk, nchunks, k, sa);
  else
    hipLaunchKernelGGL((topk_wide<T, VEC, false>), wgrid, dim3(kThreads), 0, stream, (const T*)x, values,
                       (long long*)indices, (u64*)work, (unsigned*)counters, cols, chunk, nchunks, k, sa);
  return (int)hipGetLastError();
}

// Zeroes counters[0, n).
__global__ void __launch_bounds__(kThreads) topk_zero(unsigned* __restrict__ counters, long long n) {
  for (long long i = (long long)blockIdx.x * kThreads + threadIdx.x; i < n; i += (long long)gridDim.x * kThreads)
    counters[i] = 0u;
}

}  // namespace

// topk/kernel.cu:520 `plan`: the chunk length (columns per workgroup) for a rows x cols launch. The grid of chunks
// fills the GPU's resident workgroup slots (CUs x resident workgroups of the k <= 64 kernel per CU) about once; a chunk
// longer than one register tile (16384 elements) is rounded up to whole tiles; never shorter than min_chunk, which
// carries the caller's k dependence; a multiple of 8 when a row is split. (launch lengthens the chunks of k > 64 to at
// least 16k elements.) `threads` and `depth` are the reference's CUDA tuning knobs, accepted and not used.
extern "C" long long plan(long long rows, long long cols, int dtype, int threads, int depth, int min_chunk) {
  (void)threads;
  (void)depth;
  (void)dtype;
  if (rows <= 0 || cols <= 0) return cols > 0 ? cols : 1;
  static int occ = 0;
  int per_cu = rw_host::tune_get(kTuneBlocksPerCu);
  if (per_cu <= 0) {
    if (occ <= 0) {
      int n = 0;
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, topk_tile<float, true, false, false>, kThreads, 0) !=
              hipSuccess ||
          n <= 0) {
        (void)hipGetLastError();
        n = 4;
      }
      occ = n;
    }
    per_cu = occ;
  }
  const long long tile = (long long)kThreads * kTileE;
  long long per_row = (long long)rw_host::device_cus() * per_cu / rows;
  if (per_row < 1) per_row = 1;
  long long len = (cols + per_row - 1) / per_row;
  if (len > tile) len = (len + tile - 1) / tile * tile;
  if (len < min_chunk) len = min_chunk;
  if (len >= cols) return cols;
  return (len + 7) / 8 * 8;
}

// topk/kernel.cu:549 `launch`: values [rows, k] in x's dtype and int64 indices [rows, k], sorted descending with ties
// by the lowest index. work: u64 [rows * nchunks * k] with nchunks = ceil(cols / chunk), the chunk lists of split rows;
// counters: u32 [>= rows], zero on entry and left zero (each split row's arrivals are counted on counters[row] and its
// last arrival zeroes it). Both belong to the caller, as in the reference (topk/candidate.py:38-63), and the library
// allocates nothing. Checks as the reference's, except that k may be up to 1024 (the reference stops at 512): rows <= 0
// or k <= 0 is a no-op; -1 for k > cols, k > 1024, cols > INT_MAX / 2, rows > 65535, chunk <= 0, a split row with
// chunk % 4 or nchunks * k > INT_MAX / 2, threads not 128, 256 or 512, depth not 2, 4 or 8, a dtype other than 0 and
// 1, or (this build's addition) a split row with a null work or counters.
namespace {
int launch_impl(const void* x, void* values, void* indices, void* work, void* counters, long long rows,
                long long cols, int k, int dtype, int threads, int depth, long long chunk, const SampleArgs& sa,
                hipStream_t stream) {
  if (rows <= 0 || k <= 0) return rw_host::kOk;
  if (k > cols || k > kMaxK || cols > INT_MAX / 2 || rows > 65535 || chunk <= 0) return rw_host::kInvalid;
  const long long nchunks = (cols + chunk - 1) / chunk;
  if (nchunks > 1 && (chunk % 4 || nchunks * k > INT_MAX / 2)) return rw_host::kInvalid;
  if ((threads != 128 && threads != 256 && threads != 512) || (depth != 2 && depth != 4 && depth != 8))
    return rw_host::kInvalid;
  if (nchunks > 1 && (!work || !counters)) return rw_host::kInvalid;
  if (dtype != 0 && dtype != 1) return rw_host::kInvalid;
  if (!sa.out && rw_host::tune_get(kTuneSeed) == 1) {
    if (dtype == 0)
      hipLaunchKernelGGL(topk_seed<float>, dim3((unsigned)rows), dim3(kThreads), 0, stream, (const float*)x, values,
                         (long long*)indices, cols, k);
    else
      hipLaunchKernelGGL(topk_seed<uint16_t>, dim3((unsigned)rows), dim3(kThreads), 0, stream, (const uint16_t*)x,
                         values, (long long*)indices, cols, k);
    return (int)hipGetLastError();
  }
  const int n = (int)nchunks;
  if (dtype == 0) {
    if (cols % 4 == 0 && rw_host::aligned16(x))
      return launch_chunks<float, true>(x, values, indices, work, counters, rows, cols, chunk, n, k, sa, stream);
    return launch_chunks<float, false>(x, values, indices, work, counters, rows, cols, chunk, n, k, sa, stream);
  }
  if (dtype == 1) {
    if (cols % 8 == 0 && (chunk % 8 == 0 || nchunks == 1) && rw_host::aligned16(x))
      return launch_chunks<uint16_t, true>(x, values, indices, work, counters, rows, cols, chunk, n, k, sa, stream);
    return launch_chunks<uint16_t, false>(x, values, indices, work, counters, rows, cols, chunk, n, k, sa, stream);
  }
  return rw_host::kInvalid;
}
}  // namespace

extern "C" int launch(const void* x, void* values, void* indices, void* work, void* counters, long long rows,
                      long long cols, int k, int dtype, int threads, int depth, long long chunk, hipStream_t stream) {
  return launch_impl(x, values, indices, work, counters, rows, cols, k, dtype, threads, depth, chunk,
                     SampleArgs{nullptr, nullptr, 0.0f, 0.0f}, stream);
}

// No counterpart in the reference (the top-k launch of a decoder's sampler with the draw fused in): launch(), and in
// the same kernel the draw of topk_sample_launch() from each row's list -- the workgroup that writes a row's values and
// indices draws out[row] from them, so out equals topk_sample_launch() on launch()'s output. Same arguments and checks
// as launch(), plus uniforms[rows] (fp32 in [0, 1)), out (int64 [rows]), temperature (<= 0: greedy) and top_p (>= 1:
// no nucleus cut); -1 also for a null uniforms or out when rows > 0.
extern "C" int topk_launch_sample(const void* x, void* values, void* indices, void* work, void* counters,
                                  long long rows, long long cols, int k, int dtype, int threads, int depth,
                                  long long chunk, const float* uniforms, void* out, float temperature, float top_p,
                                  hipStream_t stream) {
  if (rows > 0 && k > 0 && (!uniforms || !out)) return rw_host::kInvalid;
  return launch_impl(x, values, indices, work, counters, rows, cols, k, dtype, threads, depth, chunk,
                     SampleArgs{uniforms, (long long*)out, temperature, top_p}, stream);
}

// ---- the allocation-free entry point ---------------------------------------------------------------------------------

// Scratch of topk_launch_noalloc, one copy per GPU the library runs on, held until the process ends: the per-row
// arrival counters (kNoAllocRows u32) and then the chunk results (up to kNoAllocWork bytes of u64 slots). In host code
// `scratch` names a host-side stand-in, not device memory: the launcher asks for its device address once per device
// (hipGetSymbolAddress) and passes that address to the kernels.
constexpr size_t kNoAllocRows = 65536;                     // rows > 65535 are rejected by launch() anyway
constexpr size_t kNoAllocCounterBytes = kNoAllocRows * 4;  // 256 KiB
constexpr size_t kNoAllocWork = (size_t)16 << 20;          // 16 MiB of chunk results: rows * nchunks * k * 8 bytes
static __device__ __align__(256) unsigned char scratch[kNoAllocCounterBytes + kNoAllocWork];

namespace {
constexpr int kMaxDevices = 64;

// The device address of `scratch` on the current device, looked up once per device; nullptr with *err set on failure.
unsigned char* scratch_address(int* err) {
  static std::mutex mu;
  static unsigned char* addr[kMaxDevices];
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    *err = e != hipSuccess ? (int)e : rw_host::kInvalid;
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (!addr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      *err = e != hipSuccess ? (int)e : rw_host::kInvalid;
      return nullptr;
    }
    addr[dev] = static_cast<unsigned char*>(p);
  }
  *err = rw_host::kOk;
  return addr[dev];
}

}  // namespace

// No counterpart in the reference: launch() for callers that cannot allocate device memory (code under HIP graph
// capture, tight serving loops, harnesses that forbid hipMalloc). The same arguments without work and counters: the
// library's static per-GPU scratch holds them, and the call allocates nothing. Each call first zeroes the scratch's
// counters for its rows with a small kernel (no memset node, so the call may be captured into a graph), then runs
// launch()'s kernels. -1 as launch(), and also when a split row's results would not fit the scratch: more than 16 MiB
// of u64 slots in the chunking the launch runs (rows * nchunks * k for k > 1, rows * nchunks for k = 1, after k > 64
// lengthens short chunks and k <= 64 folds a short last one). Every call on one GPU uses that GPU's one scratch: calls that
// overlap on one GPU (two streams, or two host threads) race and must be ordered by the caller.
extern "C" int topk_launch_noalloc(const void* x, void* values, void* indices, long long rows, long long cols, int k,
                                   int dtype, int threads, int depth, long long chunk, hipStream_t stream) {
  if (rows <= 0 || k <= 0) return rw_host::kOk;
  if (k > cols || k > kMaxK || cols > INT_MAX / 2 || rows > 65535 || chunk <= 0) return rw_host::kInvalid;
  const long long nchunks = (cols + chunk - 1) / chunk;
  if (nchunks > 1 && (chunk % 4 || nchunks * k > INT_MAX / 2)) return rw_host::kInvalid;  // launch()'s own checks
  // the slots the launch will use, after its rechunking (the width only matters for short last tiles, and bf16's is
  // the wider: its fold takes no fewer chunks than fp32's)
  const Chunking c = chunking(rows, cols, chunk, (int)nchunks, k, dtype == 1 ? Fmt<uint16_t>::W : Fmt<float>::W);
  if ((unsigned long long)c.slots * 8ull > (unsigned long long)kNoAllocWork) return rw_host::kInvalid;
  int err = rw_host::kOk;
  unsigned char* base = scratch_address(&err);
  if (!base) return err;
  unsigned* counters = reinterpret_cast<unsigned*>(base);
  u64* work = reinterpret_cast<u64*>(base + kNoAllocCounterBytes);
  if (nchunks > 1) {
    long long grid = (rows + kThreads - 1) / kThreads;
    hipLaunchKernelGGL(topk_zero, dim3((unsigned)grid), dim3(kThreads), 0, stream, counters, rows);
    err = (int)hipGetLastError();
    if (err != rw_host::kOk) return err;
  }
  return launch_impl(x, values, indices, work, counters, rows, cols, k, dtype, threads, depth, chunk,
                     SampleArgs{nullptr, nullptr, 0.0f, 0.0f}, stream);
}

// No counterpart in the reference (whose counters self-reset only when a launch completes): zeroes counters[0, rows)
// on `stream` with a small kernel (no memset node, so the call may be captured into a graph), for a caller recovering
// from a launch that did not complete.
extern "C" int topk_reset(void* counters, long long rows, hipStream_t stream) {
  if (rows <= 0) return rw_host::kOk;
  if (!counters) return rw_host::kInvalid;
  long long grid = (rows + kThreads - 1) / kThreads;
  if (grid > 1024) grid = 1024;
  hipLaunchKernelGGL(topk_zero, dim3((unsigned)grid), dim3(kThreads), 0, stream, (unsigned*)counters, rows);
  return (int)hipGetLastError();
}

// Sampling from a top-k list (no counterpart in the reference: the step after top-k in a decoder's sampler; see
// topk_sample): out[row] = the int64 index drawn for each row from values/indices [rows, k] (k <= 1024, values in
// fp32 (dtype 0) or bf16 (1)), with the caller's uniforms u[rows] in [0, 1), temperature (<= 0: greedy) and top_p
// (>= 1: no nucleus cut). Returns 0 (rows <= 0 is a no-op), -1 for k outside [1, 1024], rows > 2^31 - 1, a null
// pointer or an unknown dtype, otherwise the hipError_t of the launch.
extern "C" int topk_sample_launch(const void* values, const void* indices, const float* uniforms, void* out,
                                  long long rows, int k, int dtype, float temperature, float top_p,
                                  hipStream_t stream) {
  if (rows <= 0) return rw_host::kOk;
  if (k < 1 || k > kMaxK || rows > 2147483647LL || !values || !indices || !uniforms || !out)
    return rw_host::kInvalid;
  if (dtype == 0)
    hipLaunchKernelGGL((topk_sample<float>), dim3((unsigned)rows), dim3(kWave), 0, stream, values,
                       (const long long*)indices, uniforms, (long long*)out, k, temperature, top_p);
  else if (dtype == 1)
    hipLaunchKernelGGL((topk_sample<uint16_t>), dim3((unsigned)rows), dim3(kWave), 0, stream, values,
                       (const long long*)indices, uniforms, (long long*)out, k, temperature, top_p);
  else
    return rw_host::kInvalid;
  return (int)hipGetLastError();
}

extern "C" int topk_tune(int slot, int value) { return rw_host::tune_set(slot, value); }

#ifdef ROWKERN_TOPK_STAGES
// The stage build's read-out: the stamps of the last launches (dst: host memory of `bytes`, at most the table) and
// their reset to zero.
extern "C" int topk_stages_read(void* dst, long long bytes) {
  if (!dst || bytes < 0 || bytes > (long long)sizeof(g_stage_stamps)) return rw_host::kInvalid;
  return (int)hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_stage_stamps), (size_t)bytes, 0, hipMemcpyDeviceToHost);
}
extern "C" int topk_stages_clear() {
  static unsigned long long zeros[kStageWGs * kStageSlots];
  return (int)hipMemcpyToSymbol(HIP_SYMBOL(g_stage_stamps), zeros, sizeof(zeros), 0, hipMemcpyHostToDevice);
}
#endif
