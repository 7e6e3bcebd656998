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
// Vector path (D % 16 == 0, all tensors 16-byte aligned): an item is 8 pairs of one head (two 16-byte vectors of x);
// a token has heads * D / 16 items and a block takes one token at a time, IPT items per lane, walking the tokens with
// the grid's stride and loading its next token's items while it rotates and stores the current one. The on-the-fly
// entry computes a token's D/2 (cos, sin) pairs once per block into LDS (double-buffered by token parity, one barrier
// per token) instead of once per head. Other shapes run a scalar kernel (one pair per thread per head).
#include <climits>
#include <cmath>

#include "host.hpp"
#include "rowwise.hpp"

#pragma clang fp contract(off)

using namespace rw;

namespace {

constexpr int kMaxHalf = 512;  // on-the-fly vector path: D <= 1024

// Eight cache values [i, i + 8) of a cos or sin row as floats.
template <typename C> __device__ __forceinline__ void load8(const void* p, long long i, float* v);
template <> __device__ __forceinline__ void load8<F32>(const void* p, long long i, float* v) {
  const u32x4 a = load16<false>(p, i / 4), b = load16<false>(p, i / 4 + 1);
  unpack<F32>(a, v);
  unpack<F32>(b, v + 4);
}
template <> __device__ __forceinline__ void load8<BF16>(const void* p, long long i, float* v) {
  unpack<BF16>(load16<false>(p, i / 8), v);
}
template <> __device__ __forceinline__ void load8<F16>(const void* p, long long i, float* v) {
  unpack<F16>(load16<false>(p, i / 8), v);
}

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
};

// Loads the IPT items of lane j for `token` (an out-of-range item is clamped to the token's last item, never stored).
template <bool KV, int IPT>
__device__ __forceinline__ void load_items(Items<IPT>& r, const void* q, const void* k, const Cache& kv,
                                           long long token, const Shape& s, int items, int lanes_per_head, int j) {
  const int half = s.head_dim >> 1;
#pragma unroll
  for (int u = 0; u < IPT; ++u) {
    int it = j + u * (int)blockDim.x;
    it = it < items ? it : items - 1;
    const int h = it / lanes_per_head, c = it - h * lanes_per_head;
    long long o;
    const void* x = head_src<KV>(q, k, kv, token, h, s, o);
    o += 8 * c;
    r.a[u] = load16<true>(x, o / 8);
    r.b[u] = load16<true>(x, (o + half) / 8);
  }
}

// Rotates and stores the items; cs(i) gives (cos[i], sin[i], cos[i + h], sin[i + h]) for 8 consecutive i.
template <typename T, bool KV, int IPT, typename Trig>
__device__ __forceinline__ void rotate_items(const Items<IPT>& r, void* q_out, void* k_out, const Cache& kv,
                                             long long token, long long slot, const Shape& s, int items,
                                             int lanes_per_head, int j, bool active, const Trig& trig) {
  const int half = s.head_dim >> 1;
#pragma unroll
  for (int u = 0; u < IPT; ++u) {
    const int it = j + u * (int)blockDim.x;
    if (!active || it >= items) continue;
    const int h = it / lanes_per_head, c = it - h * lanes_per_head;
    long long o;
    void* out = head_dst<KV>(q_out, k_out, kv, token, slot, h, s, o);
    if (KV && !out) continue;
    o += 8 * c;
    if (KV && h >= s.q_heads + s.kv_heads) {  // a fused write's V head: copied as it is
      store16<true>(out, o / 8, r.a[u]);
      store16<true>(out, (o + half) / 8, r.b[u]);
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
    store16<true>(out, o / 8, pack<T>(oa));
    store16<true>(out, (o + half) / 8, pack<T>(ob));
  }
}

// cos/sin from the cache row of the token's position.
template <typename C>
struct CacheTrig {
  const void* cos_rows;
  const void* sin_rows;
  long long row;  // element offset of the row
  int half;
  __device__ __forceinline__ void operator()(int i, float* c1, float* s1, float* c2, float* s2) const {
    load8<C>(cos_rows, row + i, c1);
    load8<C>(sin_rows, row + i, s1);
    load8<C>(cos_rows, row + i + half, c2);
    load8<C>(sin_rows, row + i + half, s2);
  }
};

// cos/sin from the block's LDS table of the token.
struct LdsTrig {
  const float2* cs;
  __device__ __forceinline__ void operator()(int i, float* c1, float* s1, float* c2, float* s2) const {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float2 v = cs[i + e];
      c1[e] = c2[e] = v.x;
      s1[e] = s2[e] = v.y;
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

template <typename T, typename C, bool FREQ, bool KV, int IPT>
__device__ __forceinline__ void token_step(const Items<IPT>& r, const void* cos_rows, const void* sin_rows,
                                           const float* inv_freq, const long long* ids, void* q_out, void* k_out,
                                           const Cache& kv, long long token, const Shape& s, int items,
                                           int lanes_per_head, int j, float2* cs) {
  const bool active = token < s.tokens;
  const long long tok = active ? token : s.tokens - 1;
  const long long slot = KV ? kv.slots[tok] : tok;  // the k output row: the token's cache slot when fused
  const int half = s.head_dim >> 1;
  if constexpr (FREQ) {
    const long long pos = ids[tok];
    for (int i = j; i < half; i += blockDim.x) cs[i] = freq_trig(pos, inv_freq[i]);
    __syncthreads();
    rotate_items<T, KV, IPT>(r, q_out, k_out, kv, tok, slot, s, items, lanes_per_head, j, active, LdsTrig{cs});
  } else {
    const long long row = ids[tok] * (long long)s.head_dim;
    rotate_items<T, KV, IPT>(r, q_out, k_out, kv, tok, slot, s, items, lanes_per_head, j, active,
                             CacheTrig<C>{cos_rows, sin_rows, row, half});
  }
}

// Persistent vector kernel: block b takes tokens b, b + grid, ... with a uniform trip count (a block past the last
// token loads an in-bounds token and stores nothing), two register sets of items alternating between tokens.
template <typename T, typename C, bool FREQ, bool KV, int IPT>
__global__ void __launch_bounds__(1024)
    rope_vec(const void* q, const void* k, const void* __restrict__ cos_rows, const void* __restrict__ sin_rows,
             const float* __restrict__ inv_freq, const long long* __restrict__ ids, void* q_out, void* k_out,
             Cache kv, Shape s) {
  __shared__ float2 cs[2][FREQ ? kMaxHalf : 1];
  const int lanes_per_head = s.head_dim >> 4;
  const int items = (s.q_heads + s.kv_heads + (KV ? s.v_heads : 0)) * lanes_per_head;
  const int j = threadIdx.x;
  long long t = blockIdx.x;
  if (t >= s.tokens) return;
  const long long last = s.tokens - 1;
  Items<IPT> a, b;
  load_items<KV, IPT>(a, q, k, kv, t, s, items, lanes_per_head, j);
  while (true) {
    const long long tb = t + gridDim.x;
    load_items<KV, IPT>(b, q, k, kv, tb < s.tokens ? tb : last, s, items, lanes_per_head, j);
    token_step<T, C, FREQ, KV, IPT>(a, cos_rows, sin_rows, inv_freq, ids, q_out, k_out, kv, t, s, items, lanes_per_head,
                                j, cs[0]);
    t = tb;
    if (t >= s.tokens) break;
    const long long tc = t + gridDim.x;
    load_items<KV, IPT>(a, q, k, kv, tc < s.tokens ? tc : last, s, items, lanes_per_head, j);
    token_step<T, C, FREQ, KV, IPT>(b, cos_rows, sin_rows, inv_freq, ids, q_out, k_out, kv, t, s, items, lanes_per_head,
                                j, cs[1]);
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
  auto kern = rope_vec<T, C, FREQ, KV, IPT>;
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
  const bool vec = s.head_dim % 16 == 0 && all_aligned(p, false);
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
