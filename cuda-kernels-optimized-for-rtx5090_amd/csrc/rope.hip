// Rotary position embedding (rotate-half / NeoX pairing, full rotary) of q[tokens, q_heads, D] and k[tokens, kv_heads,
// D] in bf16 (qk dtype 1) or fp16 (2), behind the reference's C-ABI `launch` (rope/kernel.cu:201-215), which reads
// cos/sin from a cache [P, D] (fp32 0, bf16 1, fp16 2) at the rows position_ids pick, plus `rope_launch_freq`, which
// computes cos/sin on the fly from the positions and an fp32 inverse-frequency table inv_freq[D/2].
//
// For h = D/2, element i < h of a head pairs with i + h (rope/kernel.cu:5-6):
//   out[i]     = x[i] * cos[i]         - x[i + h] * sin[i]
//   out[i + h] = x[i + h] * cos[i + h] + x[i] * sin[i + h]
// in fp32 with each product and the sum rounded (no contraction: this file is compiled with fp-contract off), then
// one round-to-nearest-even to the output dtype, as torch eager's x * cos + rotate_half(x) * sin. The on-the-fly entry
// uses cos[i] = cos[i + h] = fp32(cos(angle)), sin likewise, with angle = fp32(float(pos) * inv_freq[i]) (the fp32
// product of torch's outer product) and cos, sin evaluated in fp64 and rounded once to fp32.
//
// q_out may be q and k_out may be k (in place): every lane reads its elements before it writes the same elements and
// no other lane touches them, so the input and output pointers are not declared restrict.
//
// Vector path (D % 16 == 0, D <= 1024, all tensors 16-byte aligned): an item is 8 pairs of one head (two 16-byte
// vectors of x); a token has heads * D / 16 items and a block takes one token at a time, IPT items per lane, walking
// the tokens with the grid's stride and loading its next token's items while it rotates and stores the current one.
// A token's cos/sin are put into an LDS table once per block (double-buffered by token parity, one barrier per token)
// and read from there by every head: the on-the-fly entry computes its D/2 (cos, sin) pairs, the cache entry loads
// the token's cos and sin rows (as the reference loads them once per thread for all its heads, rope/kernel.cu:103-135),
// prefetched with the token's items. Other shapes run a scalar kernel (one pair per thread per head).
#include <climits>
#include <cmath>

#include "host.hpp"
#include "rowwise.hpp"

#pragma clang fp contract(off)

using namespace rw;

namespace {

constexpr int kMaxHalf = 512;  // vector path: D <= 1024

// The LDS tables of a token's cos/sin. Lane j's item covers pairs [8c, 8c + 8) with c = j % 8 (a block's threads are a
// multiple of 64 and a head has D / 16 items), so the 8 lanes of one read step read 8 different 8-entry groups at once.
// Each group is padded so that those 8 reads fall in distinct LDS banks (with 32 or 64 banks of 4 bytes) while every
// read stays a 16-byte one:
//  - on the fly: (cos, sin) of pair i as a float2 at float2 index i + 2 (i / 8): groups 80 bytes apart;
//  - cache: the token's cos row then its sin row, fp32, element e of a row at float index e + 4 (e / 32) of it (16
//    bytes after every 128), the sin row at kCacheRow floats after the cos row: groups 32 bytes apart, 48 across the
//    padding.
__device__ __forceinline__ int freq_slot(int i) { return i + 2 * (i >> 3); }
__device__ __forceinline__ int cache_slot(int e) { return e + 4 * (e >> 5); }
constexpr int kFreqTable = 2 * (kMaxHalf + kMaxHalf / 4);          // floats of one buffer: kMaxHalf padded float2
constexpr int kCacheRow = 2 * kMaxHalf + (2 * kMaxHalf) / 8;       // floats of one padded row of D <= 1024
constexpr int kCacheTable = 2 * kCacheRow;                          // cos row and sin row

struct Shape {
  long long tokens;
  int q_heads, kv_heads, head_dim;
  int v_heads;  // kv_heads when the cache write is fused (the V heads follow the K heads as copy-only items), else 0
};

// Fused KV-cache write: the rotated K heads go to k_out = the key cache and the V heads to v_cache, both laid out
// [slots, kv_heads, head_dim], at the token's slot slots[token] (a negative slot writes nothing). Unused otherwise.
struct Cache {
  const void* v;
  void* v_cache;
  const long long* slots;
};

// Source tensor and element offset of head h of a token: q heads, then k heads, then the fused write's v heads.
template <bool KV>
__device__ __forceinline__ const void* head_src(const void* q, const void* k, const Cache& kv, long long token, int h,
                                                const Shape& s, long long& o) {
  if (h < s.q_heads) {
    o = (token * s.q_heads + h) * (long long)s.head_dim;
    return q;
  }
  const int hk = h - s.q_heads;
  if (!KV || hk < s.kv_heads) {
    o = (token * s.kv_heads + hk) * (long long)s.head_dim;
    return k;
  }
  o = (token * s.kv_heads + (hk - s.kv_heads)) * (long long)s.head_dim;
  return kv.v;
}

// Destination of head h: q_out at the token for q heads; k_out and (fused write) v_cache at the token's slot row.
// Returns nullptr when the head is not written (a fused write's negative slot).
template <bool KV>
__device__ __forceinline__ void* head_dst(void* q_out, void* k_out, const Cache& kv, long long token, long long slot,
                                          int h, const Shape& s, long long& o) {
  if (h < s.q_heads) {
    o = (token * s.q_heads + h) * (long long)s.head_dim;
    return q_out;
  }
  const int hk = h - s.q_heads;
  if (KV && slot < 0) return nullptr;
  if (!KV || hk < s.kv_heads) {
    o = (slot * s.kv_heads + hk) * (long long)s.head_dim;
    return k_out;
  }
  o = (slot * s.kv_heads + (hk - s.kv_heads)) * (long long)s.head_dim;
  return kv.v_cache;
}

template <int IPT>
struct Items {
  u32x4 a[IPT], b[IPT];
  u32x4 trig;    // cache entry: this thread's 16-byte vector of the token's cos and sin rows (see load_trig)
  long long pos;  // on the fly: the token's position
};

// Loads the IPT items of lane j of nt for `token` (an out-of-range item is clamped to the token's last item, never
// stored).
template <bool KV, int IPT>
__device__ __forceinline__ void load_items(Items<IPT>& r, const void* q, const void* k, const Cache& kv,
                                           long long token, const Shape& s, int items, int lanes_per_head, int j,
                                           int nt) {
  const int half = s.head_dim >> 1;
#pragma unroll
  for (int u = 0; u < IPT; ++u) {
    int it = j + u * nt;
    it = it < items ? it : items - 1;
    const int h = it / lanes_per_head, c = it - h * lanes_per_head;
    long long o;
    const void* x = head_src<KV>(q, k, kv, token, h, s, o);
    o += 8 * c;
    r.a[u] = load16<true>(x, o / 8);
    r.b[u] = load16<true>(x, (o + half) / 8);
  }
}

// Cache entry: thread j < 2 D / W (W cache elements per 16-byte vector) loads vector j of the token's cos row followed
// by its sin row (row ids[token] of each), into r.trig.
template <typename C>
__device__ __forceinline__ void load_trig(u32x4& v, const void* cos_rows, const void* sin_rows, long long id,
                                          int head_dim, int j) {
  const int per_row = head_dim / C::V;  // vectors per row
  if (j < 2 * per_row) {
    const void* rows = j < per_row ? cos_rows : sin_rows;
    const int jv = j < per_row ? j : j - per_row;
    v = load16<false>(rows, id * per_row + jv);
  }
}

// Cache entry: the thread's vector of load_trig into the LDS table, as fp32 at its padded positions.
template <typename C>
__device__ __forceinline__ void store_trig(const u32x4& v, float* tab, int head_dim, int j) {
  const int per_row = head_dim / C::V;
  if (j < 2 * per_row) {
    float f[C::V];
    unpack<C>(v, f);
    const int row = j < per_row ? 0 : 1;
    const int e0 = (j - row * per_row) * C::V;
    float* dst = tab + row * kCacheRow;
#pragma unroll
    for (int e = 0; e < C::V; e += 4)  // 4 consecutive elements never straddle the padding (it falls every 32)
      *reinterpret_cast<float4*>(dst + cache_slot(e0 + e)) = make_float4(f[e], f[e + 1], f[e + 2], f[e + 3]);
  }
}

// Rotates the items into w and then stores them, every store after every rotation: a register that a store still
// reads is written again only later (with all of a step's stores issued together, no rotation waits for a store
// issued after the next token's loads). cs(i) gives (cos[i], sin[i], cos[i + h], sin[i + h]) for 8 consecutive i.
template <typename T, bool KV, int IPT, typename Trig>
__device__ __forceinline__ void rotate_items(const Items<IPT>& r, Items<IPT>& w, void* q_out, void* k_out,
                                             const Cache& kv, long long token, long long slot, const Shape& s,
                                             int items, int lanes_per_head, int j, int nt, bool active,
                                             const Trig& trig) {
  const int half = s.head_dim >> 1;
  void* dst[IPT];
  long long off[IPT];
#pragma unroll
  for (int u = 0; u < IPT; ++u) {
    dst[u] = nullptr;
    off[u] = 0;
    const int it = j + u * nt;
    if (!active || it >= items) continue;
    const int h = it / lanes_per_head, c = it - h * lanes_per_head;
    long long o;
    void* out = head_dst<KV>(q_out, k_out, kv, token, slot, h, s, o);
    if (KV && !out) continue;
    dst[u] = out;
    off[u] = o + 8 * c;
    if (KV && h >= s.q_heads + s.kv_heads) {  // a fused write's V head: copied as it is
      w.a[u] = r.a[u];
      w.b[u] = r.b[u];
      continue;
    }
    float c1[8], s1[8], c2[8], s2[8];
    trig(8 * c, c1, s1, c2, s2);
    float a[8], b[8], oa[8], ob[8];
    unpack<T>(r.a[u], a);
    unpack<T>(r.b[u], b);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      oa[e] = a[e] * c1[e] - b[e] * s1[e];
      ob[e] = b[e] * c2[e] + a[e] * s2[e];
    }
    w.a[u] = pack<T>(oa);
    w.b[u] = pack<T>(ob);
  }
#pragma unroll
  for (int u = 0; u < IPT; ++u) {
    if (!dst[u]) continue;
    store16<true>(dst[u], off[u] / 8, w.a[u]);
    store16<true>(dst[u], (off[u] + half) / 8, w.b[u]);
  }
}

// cos/sin from the block's LDS table of the token's cache rows (store_trig's layout).
struct LdsCacheTrig {
  const float* tab;
  int half;
  __device__ __forceinline__ void operator()(int i, float* c1, float* s1, float* c2, float* s2) const {
    auto row8 = [&](const float* row, int e, float* v) {
      const float4 a = *reinterpret_cast<const float4*>(row + cache_slot(e));
      const float4 b = *reinterpret_cast<const float4*>(row + cache_slot(e + 4));
      v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
    };
    row8(tab, i, c1);
    row8(tab + kCacheRow, i, s1);
    row8(tab, i + half, c2);
    row8(tab + kCacheRow, i + half, s2);
  }
};

// cos/sin from the block's LDS table of the token's (cos, sin) pairs (freq_slot's layout).
struct LdsTrig {
  const float2* cs;
  __device__ __forceinline__ void operator()(int i, float* c1, float* s1, float* c2, float* s2) const {
    const float4* p = reinterpret_cast<const float4*>(cs + freq_slot(i));  // 8 pairs, 16-byte aligned (i % 8 == 0)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float4 v = p[e];
      c1[2 * e] = c2[2 * e] = v.x;
      s1[2 * e] = s2[2 * e] = v.y;
      c1[2 * e + 1] = c2[2 * e + 1] = v.z;
      s1[2 * e + 1] = s2[2 * e + 1] = v.w;
    }
  }
};

// fp32(cos(angle)), fp32(sin(angle)) of angle = fp32(float(pos) * inv_freq[i]), evaluated in fp64.
__device__ __forceinline__ float2 freq_trig(long long pos, float inv_freq) {
  const float angle = (float)pos * inv_freq;
  double sn, cn;
  sincos((double)angle, &sn, &cn);
  return make_float2((float)cn, (float)sn);
}

// On the fly: the LDS table of a token at position pos, (cos, sin) of pair i at float2 freq_slot(i) (threads j, j + nt,
// ... each fill the pairs of the inv_freq entries they copied).
__device__ __forceinline__ void fill_table(float* tab, long long pos, const float* invf, int half, int j, int nt) {
  float2* cs = reinterpret_cast<float2*>(tab);
  for (int i = j; i < half; i += nt) cs[freq_slot(i)] = freq_trig(pos, invf[i]);
}

// One token: on the fly, the token's table (tab, filled during the step before) is complete after the barrier, and the
// next token's table is filled into `next` after the rotation (every thread is past the step before, which read that
// buffer, once it has passed the barrier); from the cache, the token's cos/sin vectors (loaded with its items) are
// stored into tab first.
template <typename T, typename C, bool FREQ, bool KV, int IPT>
__device__ __forceinline__ void token_step(const Items<IPT>& r, Items<IPT>& w, const float* invf, void* q_out,
                                           void* k_out, const Cache& kv, long long token, const Shape& s, int items,
                                           int lanes_per_head, int j, int nt, float* tab, float* next,
                                           long long next_pos) {
  const bool active = token < s.tokens;
  const long long tok = active ? token : s.tokens - 1;
  const long long slot = KV ? kv.slots[tok] : tok;  // the k output row: the token's cache slot when fused
  const int half = s.head_dim >> 1;
  if constexpr (FREQ) {
    __syncthreads();
    rotate_items<T, KV, IPT>(r, w, q_out, k_out, kv, tok, slot, s, items, lanes_per_head, j, nt, active,
                             LdsTrig{reinterpret_cast<const float2*>(tab)});
    fill_table(next, next_pos, invf, half, j, nt);
  } else {
    store_trig<C>(r.trig, tab, s.head_dim, j);
    __syncthreads();
    rotate_items<T, KV, IPT>(r, w, q_out, k_out, kv, tok, slot, s, items, lanes_per_head, j, nt, active,
                             LdsCacheTrig{tab, half});
  }
}

// Persistent vector kernel: block b takes tokens b, b + grid, ... with a uniform trip count (a block past the last
// token loads an in-bounds token and stores nothing), two register sets of items (and, for the cache entry, of the
// token's cos/sin vectors; on the fly, of its position) alternating between tokens. The LDS table is double-buffered
// by token parity: a buffer is written again two tokens later, after the barrier of the token in between, which every
// thread passes only once it has read the buffer.
//
// Inside the token loop no value is read from memory with a vector load that a step must wait for: the vector memory
// counter retires loads and stores in order, so such a wait also waits for the next token's items, issued just before,
// and the two register sets no longer overlap. So the block size is read once (blockDim.x is a 16-bit load from the
// dispatch's arguments, which the compiler repeats after stores), inv_freq is copied into LDS once (each thread keeps
// the entries it computes), positions are uniform loads through the scalar cache, a step issues its stores after all
// of its rotations, and those stores' registers stay untouched until the next token's loads are issued (keep below):
// a register written while a store still reads it waits for that store and so for every load issued before it.
// WIDE: blocks of more than 256 threads (at most 128 registers per thread); otherwise at most 256 threads, which
// leaves the compiler room for the register sets without spilling.
template <typename T, typename C, bool FREQ, bool KV, int IPT, bool WIDE>
__global__ void __launch_bounds__(WIDE ? 1024 : 256)
    rope_vec(const void* q, const void* k, const void* __restrict__ cos_rows, const void* __restrict__ sin_rows,
             const float* __restrict__ inv_freq, const long long* __restrict__ ids, void* q_out, void* k_out,
             Cache kv, Shape s) {
  constexpr int TABLE = FREQ ? kFreqTable : kCacheTable;
  __shared__ __align__(16) float tab[2][TABLE];
  __shared__ float invf[FREQ ? kMaxHalf : 1];
  const int lanes_per_head = s.head_dim >> 4;
  const int items = (s.q_heads + s.kv_heads + (KV ? s.v_heads : 0)) * lanes_per_head;
  const int j = threadIdx.x;
  const int nt = __builtin_amdgcn_readfirstlane((int)blockDim.x);
  long long t = blockIdx.x;
  if (t >= s.tokens) return;
  const long long last = s.tokens - 1;
  Items<IPT> a, b, w;  // w: the rotated items of the last step, which its stores read
#pragma unroll
  for (int u = 0; u < IPT; ++u) w.a[u] = w.b[u] = (u32x4){0u, 0u, 0u, 0u};
  auto load = [&](Items<IPT>& r, long long tok) __attribute__((always_inline)) {
    load_items<KV, IPT>(r, q, k, kv, tok, s, items, lanes_per_head, j, nt);
    if constexpr (FREQ) r.pos = ids[tok];
    else load_trig<C>(r.trig, cos_rows, sin_rows, ids[tok], s.head_dim, j);
  };
  auto keep = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < IPT; ++u) asm volatile("" ::"v"(w.a[u]), "v"(w.b[u]));
  };
  load(a, t);
  if constexpr (FREQ) {  // the entries i = j, j + nt, ...: those whose pairs this thread computes
    for (int i = j; i < (s.head_dim >> 1); i += nt) invf[i] = inv_freq[i];
    fill_table(tab[0], a.pos, invf, s.head_dim >> 1, j, nt);
  }
  while (true) {
    const long long tb = t + gridDim.x;
    load(b, tb < s.tokens ? tb : last);
    keep();
    token_step<T, C, FREQ, KV, IPT>(a, w, invf, q_out, k_out, kv, t, s, items, lanes_per_head, j, nt, tab[0], tab[1],
                                    b.pos);
    t = tb;
    if (t >= s.tokens) break;
    const long long tc = t + gridDim.x;
    load(a, tc < s.tokens ? tc : last);
    keep();
    token_step<T, C, FREQ, KV, IPT>(b, w, invf, q_out, k_out, kv, t, s, items, lanes_per_head, j, nt, tab[1], tab[0],
                                    a.pos);
    t = tc;
    if (t >= s.tokens) break;
  }
}

// Scalar kernel for any even head_dim and alignment: one pair per thread per head, a 256-thread block per token.
template <typename T, typename C, bool FREQ, bool KV>
__global__ void __launch_bounds__(256)
    rope_scalar(const void* q, const void* k, const void* __restrict__ cos_rows, const void* __restrict__ sin_rows,
                const float* __restrict__ inv_freq, const long long* __restrict__ ids, void* q_out, void* k_out,
                Cache kv, Shape s) {
  const int half = s.head_dim >> 1;
  const int heads = s.q_heads + s.kv_heads + (KV ? s.v_heads : 0);
  const long long pairs = (long long)heads * half;
  for (long long token = blockIdx.x; token < s.tokens; token += gridDim.x) {
    const long long pos = ids[token];
    const long long slot = KV ? kv.slots[token] : token;
    for (long long p = threadIdx.x; p < pairs; p += 256) {
      const int h = (int)(p / half), i = (int)(p - (long long)h * half);
      long long oi, oo;
      const void* x = head_src<KV>(q, k, kv, token, h, s, oi);
      void* out = head_dst<KV>(q_out, k_out, kv, token, slot, h, s, oo);
      if (KV && !out) continue;
      if (KV && h >= s.q_heads + s.kv_heads) {  // a fused write's V head: copied as it is
        store_elem<T>(out, oo + i, load_elem<T>(x, oi + i));
        store_elem<T>(out, oo + i + half, load_elem<T>(x, oi + i + half));
        continue;
      }
      float c1, s1, c2, s2;
      if constexpr (FREQ) {
        const float2 v = freq_trig(pos, inv_freq[i]);
        c1 = c2 = v.x;
        s1 = s2 = v.y;
      } else {
        const long long row = pos * (long long)s.head_dim;
        c1 = load_elem<C>(cos_rows, row + i);
        s1 = load_elem<C>(sin_rows, row + i);
        c2 = load_elem<C>(cos_rows, row + i + half);
        s2 = load_elem<C>(sin_rows, row + i + half);
      }
      const float a = load_elem<T>(x, oi + i), b = load_elem<T>(x, oi + i + half);
      store_elem<T>(out, oo + i, a * c1 - b * s1);
      store_elem<T>(out, oo + i + half, b * c2 + a * s2);
    }
  }
}

// ---- host side ------------------------------------------------------------------------------------------------------

// Tuning slots (0 = automatic): threads per block, resident blocks per CU, forced scalar kernel (1).
enum { kTuneThreads = 0, kTuneBlocksPerCu = 1, kTuneScalar = 2 };

template <typename Kernel>
int blocks_per_cu(Kernel k, int threads) {
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k, threads, 0) != hipSuccess || n <= 0) {
    (void)hipGetLastError();
    n = 1;
  }
  return n;
}

struct Ptrs {
  const void* q;
  const void* k;
  const void* cos_rows;
  const void* sin_rows;
  const float* inv_freq;
  const long long* ids;
  void* q_out;
  void* k_out;
  Cache kv;
};

template <typename T, typename C, bool FREQ, bool KV, int IPT>
int launch_vec_k(const Ptrs& p, const Shape& s, int threads, hipStream_t stream) {
  auto kern = threads > 256 ? rope_vec<T, C, FREQ, KV, IPT, true> : rope_vec<T, C, FREQ, KV, IPT, false>;
  int occ = blocks_per_cu(kern, threads);
  int per_cu = rw_host::tune_get(kTuneBlocksPerCu);
  if (per_cu <= 0) per_cu = 8;  // 8 resident token blocks per CU by default (measured on MI355X)
  if (per_cu > occ) per_cu = occ;
  long long grid = (long long)rw_host::device_cus() * per_cu;
  if (grid > s.tokens) grid = s.tokens;
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(threads), 0, stream, p.q, p.k, p.cos_rows, p.sin_rows,
                     p.inv_freq, p.ids, p.q_out, p.k_out, p.kv, s);
  return (int)hipGetLastError();
}

template <typename T, typename C, bool FREQ, bool KV = false>
int launch_shape(const Ptrs& p, const Shape& s, bool vec, hipStream_t stream) {
  const int heads = s.q_heads + s.kv_heads + s.v_heads;
  if (vec && rw_host::tune_get(kTuneScalar) != 1) {
    const long long items = (long long)heads * (s.head_dim >> 4);
    int threads = rw_host::tune_get(kTuneThreads);
    if (threads % kWave != 0 || threads > 1024) threads = 0;  // a tuned block the kernel cannot take: automatic
    if (threads <= 0) {
      // at most 256 threads per token block, the items spread evenly over them (e.g. 320 items: 192 threads, 2 each);
      // beyond 4 items per thread, up to 1024 threads
      long long per = (items + 255) / 256;
      if (per > 4) per = (items + 1023) / 1024;
      threads = (int)(((items + per - 1) / per + 63) / 64 * 64);
      if (threads > 1024) threads = 1024;
    }
    if (!FREQ) {
      // the cache entry: one thread per 16-byte vector of the token's cos and sin rows (at most 512: D <= 1024)
      const int trig = 2 * s.head_dim / C::V;
      if (threads < trig) threads = (trig + 63) / 64 * 64;
    }
    const long long ipt = (items + threads - 1) / threads;
    if (ipt <= 1) return launch_vec_k<T, C, FREQ, KV, 1>(p, s, threads, stream);
    if (ipt <= 2) return launch_vec_k<T, C, FREQ, KV, 2>(p, s, threads, stream);
    if (ipt <= 4) return launch_vec_k<T, C, FREQ, KV, 4>(p, s, threads, stream);
  }
  long long grid = (long long)rw_host::device_cus() * 8;
  if (grid > s.tokens) grid = s.tokens;
  hipLaunchKernelGGL((rope_scalar<T, C, FREQ, KV>), dim3((unsigned)grid), dim3(256), 0, stream, p.q, p.k, p.cos_rows,
                     p.sin_rows, p.inv_freq, p.ids, p.q_out, p.k_out, p.kv, s);
  return (int)hipGetLastError();
}

bool all_aligned(const Ptrs& p, bool freq) {
  using rw_host::aligned16;
  return aligned16(p.q) && aligned16(p.k) && aligned16(p.q_out) && aligned16(p.k_out) &&
         (freq || (aligned16(p.cos_rows) && aligned16(p.sin_rows))) &&
         (!p.kv.v || (aligned16(p.kv.v) && aligned16(p.kv.v_cache)));
}

template <typename T>
int launch_cache(int cache_dtype, const Ptrs& p, const Shape& s, hipStream_t stream) {
  const bool vec = s.head_dim % 16 == 0 && s.head_dim / 2 <= kMaxHalf && all_aligned(p, false);
  if (cache_dtype == 0) return launch_shape<T, F32, false>(p, s, vec, stream);
  if (cache_dtype == 1) return launch_shape<T, BF16, false>(p, s, vec, stream);
  if (cache_dtype == 2) return launch_shape<T, F16, false>(p, s, vec, stream);
  return rw_host::kInvalid;
}

// The reference's argument checks (rope/kernel.cu:204-207).
int validate(long long tokens, int q_heads, int kv_heads, int head_dim, int rows, int splits) {
  if (tokens > 2147483647LL || head_dim <= 0 || head_dim % 2 || q_heads <= 0 || kv_heads <= 0 || rows < 1 ||
      splits < 1 || splits > 65535)
    return rw_host::kInvalid;
  return rw_host::kOk;
}

}  // namespace

// rope/kernel.cu:201 `launch`: q_out/k_out = q/k rotated by the cache rows ids pick (int64 positions in [0, P));
// q_out == q and k_out == k rotate in place. `rows` and `splits` are the reference's CUDA block-shape hints: validated
// as there and otherwise unused. tokens <= 0 is a no-op.
extern "C" int launch(const void* q, const void* k, const void* cos_rows, const void* sin_rows, const void* ids,
                      void* q_out, void* k_out, long long tokens, int q_heads, int kv_heads, int head_dim,
                      int qk_dtype, int cache_dtype, int rows, int splits, hipStream_t stream) {
  if (tokens <= 0) return rw_host::kOk;
  if (validate(tokens, q_heads, kv_heads, head_dim, rows, splits)) return rw_host::kInvalid;
  const Ptrs p{q,     k,     cos_rows, sin_rows, nullptr, (const long long*)ids,
               q_out, k_out, Cache{nullptr, nullptr, nullptr}};
  const Shape s{tokens, q_heads, kv_heads, head_dim, 0};
  if (qk_dtype == 1) return launch_cache<BF16>(cache_dtype, p, s, stream);
  if (qk_dtype == 2) return launch_cache<F16>(cache_dtype, p, s, stream);
  return rw_host::kInvalid;
}

// On-the-fly RoPE (no counterpart in the reference, which reads a cache): cos/sin of fp32(float(pos) * inv_freq[i])
// for inv_freq[head_dim / 2] (fp32, device memory), evaluated in fp64 and rounded to fp32, the same pair for i and
// i + head_dim / 2. Same shapes, dtypes (qk_dtype 1 or 2), in-place rule and return codes as `launch`.
extern "C" int rope_launch_freq(const void* q, const void* k, const void* ids, const float* inv_freq, void* q_out,
                                void* k_out, long long tokens, int q_heads, int kv_heads, int head_dim, int qk_dtype,
                                hipStream_t stream) {
  if (tokens <= 0) return rw_host::kOk;
  if (validate(tokens, q_heads, kv_heads, head_dim, 1, 1) || !inv_freq) return rw_host::kInvalid;
  const Ptrs p{q, k, nullptr, nullptr, inv_freq, (const long long*)ids, q_out, k_out, Cache{nullptr, nullptr, nullptr}};
  const Shape s{tokens, q_heads, kv_heads, head_dim, 0};
  const bool vec = head_dim % 16 == 0 && head_dim / 2 <= kMaxHalf && all_aligned(p, true);
  if (qk_dtype == 1) return launch_shape<BF16, F32, true>(p, s, vec, stream);
  if (qk_dtype == 2) return launch_shape<F16, F32, true>(p, s, vec, stream);
  return rw_host::kInvalid;
}

// RoPE fused with the KV-cache write (no counterpart in the reference; the step after RoPE in a decoder layer, as
// vLLM's rotary embedding + reshape_and_cache for the flash layout): q_out = rope(q) (q_out may be q); the rotated k
// and the unrotated v of token t go to row slot_mapping[t] of k_cache and v_cache, each [slots, kv_heads, head_dim]
// (a paged [blocks, block_size, kv_heads, head_dim] cache with slot = block * block_size + offset); a negative slot
// writes nothing for its token. cos/sin on the fly from inv_freq as rope_launch_freq; k and v are only read. Same
// shapes, dtypes and return codes as rope_launch_freq; v, caches or slot_mapping null is -1.
extern "C" int rope_kv_launch(const void* q, const void* k, const void* v, const void* ids, const float* inv_freq,
                              void* q_out, void* k_cache, void* v_cache, const void* slot_mapping, long long tokens,
                              int q_heads, int kv_heads, int head_dim, int qk_dtype, hipStream_t stream) {
  if (tokens <= 0) return rw_host::kOk;
  if (validate(tokens, q_heads, kv_heads, head_dim, 1, 1) || !inv_freq || !v || !k_cache || !v_cache ||
      !slot_mapping)
    return rw_host::kInvalid;
  const Ptrs p{q, k, nullptr, nullptr, inv_freq, (const long long*)ids, q_out, k_cache,
               Cache{v, v_cache, (const long long*)slot_mapping}};
  const Shape s{tokens, q_heads, kv_heads, head_dim, kv_heads};
  const bool vec = head_dim % 16 == 0 && head_dim / 2 <= kMaxHalf && all_aligned(p, true);
  if (qk_dtype == 1) return launch_shape<BF16, F32, true, true>(p, s, vec, stream);
  if (qk_dtype == 2) return launch_shape<F16, F32, true, true>(p, s, vec, stream);
  return rw_host::kInvalid;
}

extern "C" int rope_tune(int slot, int value) { return rw_host::tune_set(slot, value); }
