/* CPU oracle for the four row-wise kernels: a restatement, in plain C, of the arithmetic the reference specifies for
 * softmax, RMSNorm, RoPE and top-k, used only as the checker of the HIP kernels.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg may load this
 * library, and only to check or time against it; the product path never calls it.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off, no fast-math: every fp32 operation below rounds once).
 * Formats: fp32 as float, bf16 and fp16 as their raw uint16 bits; dtype codes as the reference ABI (softmax 0 fp32,
 * 1 bf16; rmsnorm / rope 1 bf16, 2 fp16; rope cache 0 fp32, 1 bf16, 2 fp16; topk 0 fp32, 1 bf16).
 *
 * How each function is pinned (tests/test_oracle.py): softmax against torch.softmax in fp64 and fp32 (the reference's
 * own path, softmax/baseline.py:13) and its invariants; RMSNorm against the reference's torch expression and closed
 * forms; RoPE against torch eager's x * cos + rotate_half(x) * sin bit for bit, brute-force loops and rotation
 * identities; top-k against a stable descending torch.sort, torch.topk and argmax. */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ---- formats --- */

static float f_from_bits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t bits_from_f(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* Round to nearest even to bf16 (NaN -> quiet NaN 0x7fc0, as torch's c10::BFloat16). */
uint16_t oracle_f32_to_bf16(float f) {
  uint32_t u = bits_from_f(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}
float oracle_bf16_to_f32(uint16_t h) { return f_from_bits((uint32_t)h << 16); }

/* IEEE binary16 <-> fp32, round to nearest even (subnormals and overflow to inf handled). */
float oracle_f16_to_f32(uint16_t h) {
  uint32_t s = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  if (e == 0x1f) return f_from_bits(s | 0x7f800000u | (m << 13));
  if (e == 0) {
    float v = (float)m * 5.9604644775390625e-8f; /* m * 2^-24, exact */
    return s ? -v : v;
  }
  return f_from_bits(s | ((e + 112u) << 23) | (m << 13));
}
uint16_t oracle_f32_to_f16(float f) {
  uint32_t u = bits_from_f(f), s = (u >> 16) & 0x8000u;
  uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint16_t)(s | 0x7e00u);
  if (a >= 0x477ff000u) return (uint16_t)(s | 0x7c00u); /* >= 65520 rounds to inf */
  if (a < 0x38800000u) { /* below the smallest normal 2^-14: subnormal, m * 2^-24 rounded to nearest even */
    double v = (double)f_from_bits(a) * 16777216.0;
    double r = nearbyint(v); /* default rounding mode: to nearest even */
    return (uint16_t)(s | (uint32_t)r);
  }
  uint32_t e = (a >> 23) - 112u, m = a & 0x7fffffu;
  uint32_t h = (e << 10) | (m >> 13);
  uint32_t rest = m & 0x1fffu;
  if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h++;
  return (uint16_t)(s | h);
}

static float load_fmt(const void* p, long long i, int fmt) {
  if (fmt == 0) return ((const float*)p)[i];
  if (fmt == 1) return oracle_bf16_to_f32(((const uint16_t*)p)[i]);
  return oracle_f16_to_f32(((const uint16_t*)p)[i]);
}
static void store_fmt(void* p, long long i, float v, int fmt) {
  if (fmt == 0) ((float*)p)[i] = v;
  else if (fmt == 1) ((uint16_t*)p)[i] = oracle_f32_to_bf16(v);
  else ((uint16_t*)p)[i] = oracle_f32_to_f16(v);
}
static float round_fmt(float v, int fmt) {
  if (fmt == 1) return oracle_bf16_to_f32(oracle_f32_to_bf16(v));
  if (fmt == 2) return oracle_f16_to_f32(oracle_f32_to_f16(v));
  return v;
}

/* Correct rounding of a double to bf16 (one rounding, not through fp32). */
static uint16_t bf16_from_double(double v) {
  if (isnan(v)) return 0x7fc0u;
  float f = (float)v; /* nearest fp32 */
  uint32_t u = bits_from_f(f);
  uint32_t lo = u & 0xffffu;
  if (lo == 0x8000u && (double)f != v) {
    /* f sits exactly on a bf16 midpoint but v does not: the side of v decides */
    uint32_t up = (u & 0xffff0000u) + 0x10000u, dn = u & 0xffff0000u;
    double vu = (double)f_from_bits(up), vd = (double)f_from_bits(dn);
    return (uint16_t)((fabs(v - vu) < fabs(v - vd) ? up : dn) >> 16);
  }
  return oracle_f32_to_bf16(f);
}

/* ---- softmax (softmax/baseline.py:12-13, softmax/kernel.cu:1) -------------------------------------------------------
 * y = exp(x - max) / sum exp(x - max) over each row, evaluated in fp64 and rounded once to the row's format (fp32 or
 * bf16): the reference harness's fp64 oracle. */
void oracle_softmax(const void* x, void* y, long long rows, long long cols, int dtype) {
  const int fmt = dtype == 0 ? 0 : 1;
  for (long long r = 0; r < rows; ++r) {
    const long long o = r * cols;
    double m = -INFINITY; /* a NaN element is skipped here and makes the sum, hence the row, NaN */
    for (long long j = 0; j < cols; ++j) {
      const double v = load_fmt(x, o + j, fmt);
      if (v > m) m = v;
    }
    double s = 0.0;
    for (long long j = 0; j < cols; ++j) s += exp((double)load_fmt(x, o + j, fmt) - m);
    for (long long j = 0; j < cols; ++j) {
      double v = exp((double)load_fmt(x, o + j, fmt) - m) / s;
      if (fmt == 0) ((float*)y)[o + j] = (float)v;
      else ((uint16_t*)y)[o + j] = bf16_from_double(v);
    }
  }
}

/* ---- RMSNorm (rmsnorm/kernel.cu:1-8, :34-50, :64-97; rmsnorm/candidate.py:3-4) --------------------------------------
 * sum  = exact sum of x^2 (long double; every square of a 2-byte value is exact in fp32)
 * mean = fp32(sum) / cols in fp32;  v = mean + eps in fp32
 * inv  = T(fp32(1 / sqrt(v)))  -- rsqrt correctly rounded to fp32 (via fp64), then rounded to the dtype
 * y    = T(x * inv)            -- exact fp32 product, one rounding
 * y    = T(w * y)              -- only with a weight: torch's `w * y` on dtype tensors
 * `inv_out` (optional) receives each row's inv as fp32. */
void oracle_rmsnorm(const uint16_t* x, const uint16_t* w, uint16_t* y, long long rows, long long cols, int dtype,
                    float eps, float* inv_out) {
  const int fmt = dtype == 2 ? 2 : 1;
  for (long long r = 0; r < rows; ++r) {
    const long long o = r * cols;
    long double acc = 0.0L;
    for (long long j = 0; j < cols; ++j) {
      float f = load_fmt(x, o + j, fmt);
      acc += (long double)(f * f);
    }
    const float s32 = (float)acc;
    const float mean = s32 / (float)cols;
    const float v = mean + eps;
    const float inv = round_fmt((float)(1.0 / sqrt((double)v)), fmt);
    if (inv_out) inv_out[r] = inv;
    for (long long j = 0; j < cols; ++j) {
      float t = load_fmt(x, o + j, fmt) * inv;
      if (w) t = load_fmt(w, j, fmt) * round_fmt(t, fmt);
      store_fmt(y, o + j, t, fmt);
    }
  }
}

/* Fused residual add + RMSNorm (no counterpart in the reference; its torch statement on dtype tensors is
 * `h = x + residual; y = w * T(h * inv(h))`): h = T(fp32(x) + fp32(residual)) is written to h_out, then y is
 * oracle_rmsnorm of h. x, residual, h_out and y are [rows, cols] bits of the dtype. */
void oracle_rmsnorm_add(const uint16_t* x, const uint16_t* res, const uint16_t* w, uint16_t* y, uint16_t* h_out,
                        long long rows, long long cols, int dtype, float eps) {
  const int fmt = dtype == 2 ? 2 : 1;
  for (long long i = 0; i < rows * cols; ++i) store_fmt(h_out, i, load_fmt(x, i, fmt) + load_fmt(res, i, fmt), fmt);
  oracle_rmsnorm(h_out, w, y, rows, cols, dtype, eps, 0);
}

/* ---- RoPE (rope/kernel.cu:1-11, :73-79, :119-126; rope/candidate.py:3-5) --------------------------------------------
 * For each token, head and i < h = D/2, with a = x[i], b = x[i + h] of the head:
 *   out[i]     = T(fp32(fp32(a * c1) - fp32(b * s1)))
 *   out[i + h] = T(fp32(fp32(b * c2) + fp32(a * s2)))
 * cache form: c1 = cos[p][i], s1 = sin[p][i], c2 = cos[p][i + h], s2 = sin[p][i + h] with p = ids[token];
 * frequency form: c1 = c2 = fp32(cos(t)), s1 = s2 = fp32(sin(t)) with t = fp32(float(pos) * inv_freq[i]) and cos,
 * sin in fp64 (the correctly rounded fp32 values). q is [tokens, q_heads, D], k is [tokens, kv_heads, D]; outputs
 * may alias. */
static void rope_head(const void* x, void* out, long long o, int half, int fmt, const float* c1, const float* s1,
                      const float* c2, const float* s2) {
  for (int i = 0; i < half; ++i) {
    const float a = load_fmt(x, o + i, fmt), b = load_fmt(x, o + i + half, fmt);
    const float p1 = a * c1[i], p2 = b * s1[i], p3 = b * c2[i], p4 = a * s2[i];
    const float oa = p1 - p2, ob = p3 + p4;
    store_fmt(out, o + i, oa, fmt);
    store_fmt(out, o + i + half, ob, fmt);
  }
}

static void rope_token(const void* q, const void* k, void* q_out, void* k_out, long long t, int q_heads, int kv_heads,
                       int head_dim, int fmt, const float* c1, const float* s1, const float* c2, const float* s2) {
  const int half = head_dim / 2;
  for (int h = 0; h < q_heads; ++h) {
    const long long o = (t * q_heads + h) * (long long)head_dim;
    rope_head(q, q_out, o, half, fmt, c1, s1, c2, s2);
  }
  for (int h = 0; h < kv_heads; ++h) {
    const long long o = (t * kv_heads + h) * (long long)head_dim;
    rope_head(k, k_out, o, half, fmt, c1, s1, c2, s2);
  }
}

void oracle_rope_cache(const void* q, const void* k, const void* cos_rows, const void* sin_rows, const int64_t* ids,
                       void* q_out, void* k_out, long long tokens, int q_heads, int kv_heads, int head_dim,
                       int qk_dtype, int cache_dtype) {
  const int half = head_dim / 2, fmt = qk_dtype == 2 ? 2 : 1;
  float* buf = (float*)malloc(sizeof(float) * 4 * (size_t)half);
  float *c1 = buf, *s1 = buf + half, *c2 = buf + 2 * half, *s2 = buf + 3 * half;
  for (long long t = 0; t < tokens; ++t) {
    const long long row = ids[t] * (long long)head_dim;
    for (int i = 0; i < half; ++i) {
      c1[i] = load_fmt(cos_rows, row + i, cache_dtype);
      s1[i] = load_fmt(sin_rows, row + i, cache_dtype);
      c2[i] = load_fmt(cos_rows, row + i + half, cache_dtype);
      s2[i] = load_fmt(sin_rows, row + i + half, cache_dtype);
    }
    rope_token(q, k, q_out, k_out, t, q_heads, kv_heads, head_dim, fmt, c1, s1, c2, s2);
  }
  free(buf);
}

void oracle_rope_freq(const void* q, const void* k, const int64_t* ids, const float* inv_freq, void* q_out,
                      void* k_out, long long tokens, int q_heads, int kv_heads, int head_dim, int qk_dtype) {
  const int half = head_dim / 2, fmt = qk_dtype == 2 ? 2 : 1;
  float* buf = (float*)malloc(sizeof(float) * 2 * (size_t)half);
  float *c = buf, *s = buf + half;
  for (long long t = 0; t < tokens; ++t) {
    const float pos = (float)ids[t];
    for (int i = 0; i < half; ++i) {
      const float angle = pos * inv_freq[i];
      c[i] = (float)cos((double)angle);
      s[i] = (float)sin((double)angle);
    }
    rope_token(q, k, q_out, k_out, t, q_heads, kv_heads, head_dim, fmt, c, s, c, s);
  }
  free(buf);
}

/* cos/sin cache [positions, D] of the frequency form (fp32), the table oracle_rope_freq evaluates on the fly. */
void oracle_rope_table(const float* inv_freq, long long positions, int head_dim, float* cos_out, float* sin_out) {
  const int half = head_dim / 2;
  for (long long p = 0; p < positions; ++p) {
    for (int i = 0; i < half; ++i) {
      const float angle = (float)p * inv_freq[i];
      const float c = (float)cos((double)angle), s = (float)sin((double)angle);
      cos_out[p * head_dim + i] = cos_out[p * head_dim + i + half] = c;
      sin_out[p * head_dim + i] = sin_out[p * head_dim + i + half] = s;
    }
  }
}

/* ---- top-k (topk/kernel.cu:1-15, :56-81) ----------------------------------------------------------------------------
 * Each element is ranked by its composite (key << 32) | ~index with key = ~u for a set sign bit, else u | 0x80000000 (u
 * the fp32 bits; a bf16 element is widened to fp32 first): values descending, ties by the lowest index, +0 above -0,
 * +NaN above +inf and -NaN below -inf. The k largest composites, in descending order, give the values (the element
 * bits, unchanged) and int64 indices. k <= cols. */
static uint64_t composite(uint32_t u, uint32_t i) {
  const uint32_t key = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)key << 32) | (uint64_t)(~i);
}

static void heap_down(uint64_t* h, int n, int i) { /* min-heap */
  for (;;) {
    int l = 2 * i + 1, r = l + 1, m = i;
    if (l < n && h[l] < h[m]) m = l;
    if (r < n && h[r] < h[m]) m = r;
    if (m == i) return;
    uint64_t t = h[i]; h[i] = h[m]; h[m] = t;
    i = m;
  }
}

static int cmp_desc(const void* a, const void* b) {
  const uint64_t x = *(const uint64_t*)a, y = *(const uint64_t*)b;
  return x < y ? 1 : (x > y ? -1 : 0);
}

void oracle_topk(const void* x, void* values, int64_t* indices, long long rows, long long cols, int k, int dtype) {
  uint64_t* heap = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)(k > 0 ? k : 1));
  for (long long r = 0; r < rows; ++r) {
    int n = 0;
    for (long long j = 0; j < cols; ++j) {
      uint32_t u = dtype == 0 ? ((const uint32_t*)x)[r * cols + j] : (uint32_t)((const uint16_t*)x)[r * cols + j] << 16;
      uint64_t c = composite(u, (uint32_t)j);
      if (n < k) {
        heap[n++] = c;
        if (n == k)
          for (int i = k / 2 - 1; i >= 0; --i) heap_down(heap, k, i);
      } else if (c > heap[0]) {
        heap[0] = c;
        heap_down(heap, k, 0);
      }
    }
    qsort(heap, (size_t)n, sizeof(uint64_t), cmp_desc);
    for (int i = 0; i < n; ++i) {
      const uint64_t c = heap[i];
      const uint32_t key = (uint32_t)(c >> 32);
      const uint32_t u = (key & 0x80000000u) ? (key & 0x7fffffffu) : ~key;
      const uint32_t idx = ~(uint32_t)c;
      if (dtype == 0) ((uint32_t*)values)[r * k + i] = u;
      else ((uint16_t*)values)[r * k + i] = (uint16_t)(u >> 16);
      indices[r * k + i] = (int64_t)idx;
    }
  }
  free(heap);
}

/* ---- sampling from a top-k list (no counterpart in the reference; the step after top-k in a decoder's sampler) ------
 * The rule of the HIP kernel, restated in fp64 for each row of values/indices [rows, k] (the order top-k writes):
 * x_i = v_i / temperature, e_i = exp(x_i - max x), S_i = e_0 + ... + e_i; keep the positions i with i == 0 or
 * S_(i-1) < top_p * S_(k-1) (every position when top_p >= 1); draw the first kept i with S_i > u * S_(last kept), else
 * the last kept. temperature <= 0 takes position 0. ambiguous[row] = 1 when the draw's target lies within
 * 2e-5 * S_(k-1) of an interval edge (where the kernel's fp32 sums may decide it either way). */
void oracle_topk_sample(const void* values, const int64_t* indices, const float* u, int64_t* out, long long rows,
                        int k, int dtype, float temperature, float top_p, int* ambiguous) {
  double* S = (double*)malloc(sizeof(double) * (size_t)k);
  for (long long r = 0; r < rows; ++r) {
    ambiguous[r] = 0;
    if (temperature <= 0.0f) {
      out[r] = indices[r * k];
      continue;
    }
    double m = -INFINITY;
    for (int i = 0; i < k; ++i) {
      const double x = (double)load_fmt(values, r * k + i, dtype == 1 ? 1 : 0) / (double)temperature;
      if (x > m) m = x;
    }
    double run = 0.0;
    for (int i = 0; i < k; ++i) {
      const double x = (double)load_fmt(values, r * k + i, dtype == 1 ? 1 : 0) / (double)temperature;
      run += exp(x - m);
      S[i] = run;
    }
    /* a cut that rounding moves changes the kept mass by less than tol, which moves the target by less than tol:
     * the draw's tolerance band (2 tol) covers it */
    const double total = S[k - 1], tol = 1e-5 * total, cut = (double)top_p * total;
    int kept = top_p >= 1.0f ? k : 1;
    for (int i = 1; i < k && top_p < 1.0f; ++i)
      if (S[i - 1] < cut) kept = i + 1;
    const double target = (double)u[r] * S[kept - 1];
    int chosen = kept - 1;
    for (int i = 0; i < kept; ++i) {
      if (fabs(S[i] - target) < 2.0 * tol) ambiguous[r] = 1;
      if (S[i] > target && i < chosen) chosen = i;
    }
    out[r] = indices[r * k + chosen];
  }
  free(S);
}

/* The admissible draws of oracle_topk_sample for every row, as a range of list positions [lo[r], hi[r]]: the positions
 * that the draw rule picks when the prefix sums S_i, the cut top_p * S_(k-1) and the target u * S_(kept-1) each move by
 * up to tol = 1e-5 of the total (what fp32 evaluation of the same rule, in any order of summation over k <= 1024 terms,
 * stays within). A row whose u and cut lie away from every boundary gets lo = hi = the exact draw's position; a row near
 * one gets the two (rarely more) positions either side; the exact draw is always in the band. temperature <= 0:
 * [0, 0]. */
void oracle_topk_sample_band(const void* values, const float* u, int* lo, int* hi, long long rows, int k, int dtype,
                             float temperature, float top_p) {
  double* S = (double*)malloc(sizeof(double) * (size_t)k);
  for (long long r = 0; r < rows; ++r) {
    if (temperature <= 0.0f) {
      lo[r] = hi[r] = 0;
      continue;
    }
    double m = -INFINITY;
    for (int i = 0; i < k; ++i) {
      const double x = (double)load_fmt(values, r * k + i, dtype == 1 ? 1 : 0) / (double)temperature;
      if (x > m) m = x;
    }
    double run = 0.0;
    for (int i = 0; i < k; ++i) {
      const double x = (double)load_fmt(values, r * k + i, dtype == 1 ? 1 : 0) / (double)temperature;
      run += exp(x - m);
      S[i] = run;
    }
    const double total = S[k - 1], tol = 1e-5 * total, cut = (double)top_p * total;
    /* the kept counts the cut allows: 1 + the positions i >= 1 whose S_(i-1) is below the cut, +- the tolerance */
    int kmin = top_p >= 1.0f ? k : 1, kmax = kmin;
    for (int i = 1; i < k && top_p < 1.0f; ++i) {
      if (S[i - 1] < cut - 2.0 * tol) kmin = i + 1;
      if (S[i - 1] < cut + 2.0 * tol) kmax = i + 1;
    }
    /* the exact draw (oracle_topk_sample's rule) is always admissible; it is also the whole band of a row whose sums
     * are not finite, where no comparison holds (values must be finite when temperature > 0) */
    int kept0 = top_p >= 1.0f ? k : 1;
    for (int i = 1; i < k && top_p < 1.0f; ++i)
      if (S[i - 1] < cut) kept0 = i + 1;
    const double target0 = (double)u[r] * S[kept0 - 1];
    int l = kept0 - 1;
    for (int i = 0; i < kept0; ++i)
      if (S[i] > target0 && i < l) l = i;
    int h = l;
    for (int kept = kmin; kept <= kmax; ++kept) {
      const double target = (double)u[r] * S[kept - 1];
      /* position i can be the first kept one above the target; and the last kept one when none may be above it */
      for (int i = 0; i < kept; ++i) {
        const int above = S[i] > target - 2.0 * tol;
        const int first = i == 0 || S[i - 1] <= target + 2.0 * tol;
        const int last = i == kept - 1 && S[i] <= target + 2.0 * tol;
        if ((above && first) || last) {
          if (i < l) l = i;
          if (i > h) h = i;
        }
      }
    }
    lo[r] = l;
    hi[r] = h;
  }
  free(S);
}
