// RMSNorm of x[rows, cols] over cols for bf16 (dtype 1) and fp16 (dtype 2) rows, behind the reference's C-ABI `launch`
// (rmsnorm/kernel.cu:132-139) plus a weighted entry `rmsnorm_launch_weighted`.
//
// Per row (rmsnorm/kernel.cu:1-8, rmsnorm/candidate.py:3-4):
//   sum  = sum of x^2                                   (each square is exact in fp32 for a 2-byte format)
//   inv  = T(rsqrt(float(sum) / cols + eps))            (fp32 mean and eps, rsqrt rounded to x's dtype)
//   y    = T(x * inv)                                   (one round to nearest even; the product is exact in fp32)
//   y    = T(w * y)                                     (weighted entry only: torch's `w * y` on dtype tensors)
// The fused residual entry (`rmsnorm_add_launch`) first forms h = T(x + residual), writes it to residual_out and
// normalizes h as above: torch's `h = x + residual; y = rmsnorm(h)` on dtype tensors, one pass over memory.
// The squares are summed in fp64, which makes the sum exact to far below fp32 resolution, so float(sum) is the
// correctly rounded fp32 sum and does not depend on the summation order; rsqrt is evaluated in fp64 and rounded to
// fp32 (the correctly rounded fp32 rsqrt). The reference's fp32 sum and rsqrtf are within an fp32 ulp or two of these
// values; the result differs from it only where that ulp moves inv across a rounding boundary of the dtype. A NaN in a
// row makes the row NaN and a sum beyond the fp32 range makes inv 0, as in the reference.
//
// Rows whose length is a multiple of 8 with 16-byte aligned x, y (and w) run the row kernel: a group of WAVES waves
// holds one row in registers as NV 16-byte vectors per lane, reduces the sum over the group (DPP within a wave, LDS
// slots across waves) and writes y from the registers; each lane holds the weight vectors of its columns once for all
// rows. Workgroups are persistent and load their next row while they reduce and store the current one. Other rows use
// a generic kernel (one workgroup per row, scalar accesses, two passes).
#include <climits>
#include <cmath>

#include "host.hpp"
#include "rowwise.hpp"

using namespace rw;

namespace {

constexpr int kMaxNv = 8;
constexpr int kMaxWaves = 16;

template <int NV>
struct Regs {
  u32x4 v[NV];
};

template <int G, int NV, bool FULL, bool NTL>
__device__ __forceinline__ void load_vectors(Regs<NV>& r, const void* base, long long first, long long count, int t) {
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    long long i = (long long)k * G + t;
    if constexpr (!FULL) i = i < count ? i : count - 1;
    r.v[k] = load16<NTL>(base, first + i);
  }
}

// inv from the exact sum of squares: fp32 mean and eps as the reference, rsqrt correctly rounded to fp32, then to T.
template <typename T>
__device__ __forceinline__ float row_inv(double sum, int cols, float eps) {
  const float mean = (float)sum / (float)cols;
  const float v = mean + eps;
  const float inv32 = (float)(1.0 / sqrt((double)v));
  return round_to<T>(inv32);
}

template <typename T, int WAVES, int NV, bool FULL, bool HAS_W, bool NTS>
__device__ __forceinline__ void norm_row(const Regs<NV>& r, const Regs<NV>& w, void* y, long long row,
                                         long long nvec, int cols, float eps, int t, bool active, double* slots,
                                         int wave, int first) {
  constexpr int G = WAVES * kWave;
  double acc = 0.0;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    float f[T::V];
    unpack<T>(r.v[k], f);
    const bool ok = FULL || (long long)k * G + t < nvec;
#pragma unroll
    for (int i = 0; i < T::V; ++i) acc += ok ? (double)(f[i] * f[i]) : 0.0;
  }
  acc = group_reduce<WAVES>(acc, OpSum{}, slots, wave, first);
  const float inv = row_inv<T>(acc, cols, eps);
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const long long i = (long long)k * G + t;
    if (active && (FULL || i < nvec)) {
      float f[T::V];
      unpack<T>(r.v[k], f);
#pragma unroll
      for (int e = 0; e < T::V; ++e) f[e] = f[e] * inv;
      if constexpr (HAS_W) {
        float g[T::V];
        unpack<T>(w.v[k], g);
#pragma unroll
        for (int e = 0; e < T::V; ++e) f[e] = g[e] * round_to<T>(f[e]);
      }
      store16<NTS>(y, row * nvec + i, pack<T>(f));
    }
  }
}

// Fused residual: r becomes h = T(x + residual), which is written to res_out (the lane's own vectors: res_out may be
// residual, and y may be x).
template <typename T, int G, int NV, bool FULL, bool NTS>
__device__ __forceinline__ void add_residual(Regs<NV>& r, const Regs<NV>& res, void* res_out, long long row,
                                             long long nvec, int t, bool active) {
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    float a[T::V], b[T::V];
    unpack<T>(r.v[k], a);
    unpack<T>(res.v[k], b);
#pragma unroll
    for (int e = 0; e < T::V; ++e) a[e] = a[e] + b[e];
    r.v[k] = pack<T>(a);
    const long long i = (long long)k * G + t;
    if (active && (FULL || i < nvec)) store16<NTS>(res_out, row * nvec + i, r.v[k]);
  }
}

// Row kernel. A block is max(WAVES, 4) waves; GROUPS = block waves / WAVES groups walk their own rows with a uniform
// trip count (a group past the last row loads an in-bounds row and stores nothing). Two LDS slot arrays alternate
// between consecutive rows, so a slot is never rewritten before the barrier of the next reduction.
// With RES the group also loads the residual rows, forms h = T(x + residual) and writes it to res_out before the
// normalisation (x and y, and residual and res_out, may be the same buffers: a lane reads its vectors before it
// writes them).
template <typename T, int WAVES, int NV, bool FULL, bool HAS_W, bool RES, bool NTL, bool NTS>
__global__ void __launch_bounds__((WAVES < 4 ? 4 : WAVES) * 64)
    rmsnorm_rows(const void* x, const void* res, const void* __restrict__ w, void* y, void* res_out, long long rows,
                 long long nvec, int cols, float eps) {
  constexpr int BW = WAVES < 4 ? 4 : WAVES;
  constexpr int GROUPS = BW / WAVES;
  constexpr int G = WAVES * kWave;
  __shared__ double slots[2][BW];
  const int wave = wave_id();
  const int first = (wave / WAVES) * WAVES;
  const int t = (int)threadIdx.x - first * kWave;
  const long long step = (long long)gridDim.x * GROUPS;
  long long base = (long long)blockIdx.x * GROUPS;
  if (base >= rows) return;
  const long long last = rows - 1;
  Regs<NV> wr;
  if constexpr (HAS_W) load_vectors<G, NV, FULL, false>(wr, w, 0, nvec, t);
  long long ra = base + wave / WAVES;
  Regs<NV> a, b;
  Regs<RES ? NV : 1> ea, eb;  // residual rows
  load_vectors<G, NV, FULL, NTL>(a, x, (ra < rows ? ra : last) * nvec, nvec, t);
  if constexpr (RES) load_vectors<G, NV, FULL, NTL>(ea, res, (ra < rows ? ra : last) * nvec, nvec, t);
  while (true) {
    const long long rb = ra + step;
    load_vectors<G, NV, FULL, NTL>(b, x, (rb < rows ? rb : last) * nvec, nvec, t);
    if constexpr (RES) {
      load_vectors<G, NV, FULL, NTL>(eb, res, (rb < rows ? rb : last) * nvec, nvec, t);
      add_residual<T, G, NV, FULL, NTS>(a, ea, res_out, ra, nvec, t, ra < rows);
    }
    norm_row<T, WAVES, NV, FULL, HAS_W, NTS>(a, wr, y, ra, nvec, cols, eps, t, ra < rows, slots[0], wave, first);
    base += step;
    if (base >= rows) break;
    ra = rb;
    const long long rc = ra + step;
    load_vectors<G, NV, FULL, NTL>(a, x, (rc < rows ? rc : last) * nvec, nvec, t);
    if constexpr (RES) {
      load_vectors<G, NV, FULL, NTL>(ea, res, (rc < rows ? rc : last) * nvec, nvec, t);
      add_residual<T, G, NV, FULL, NTS>(b, eb, res_out, ra, nvec, t, ra < rows);
    }
    norm_row<T, WAVES, NV, FULL, HAS_W, NTS>(b, wr, y, ra, nvec, cols, eps, t, ra < rows, slots[1], wave, first);
    base += step;
    if (base >= rows) break;
    ra = rc;
  }
}

// Generic kernel: any row length and alignment, one 256-thread block per row (grid-strided), two scalar passes.
// With RES, pass 1 writes h = T(x + residual) to res_out and pass 2 reads h back (the thread's own elements).
template <typename T, bool HAS_W, bool RES>
__global__ void __launch_bounds__(256)
    rmsnorm_generic(const void* x, const void* res, const void* __restrict__ w, void* y, void* res_out,
                    long long rows, int cols, float eps) {
  __shared__ double slots[2][4];
  const int wave = wave_id();
  int parity = 0;
  const void* src = RES ? (const void*)res_out : x;
  for (long long row = blockIdx.x; row < rows; row += gridDim.x, parity ^= 1) {
    const long long o = row * (long long)cols;
    double acc = 0.0;
    for (int j = threadIdx.x; j < cols; j += 256) {
      float f = load_elem<T>(x, o + j);
      if constexpr (RES) {
        f = round_to<T>(f + load_elem<T>(res, o + j));
        store_elem<T>(res_out, o + j, f);
      }
      acc += (double)(f * f);
    }
    acc = group_reduce<4>(acc, OpSum{}, slots[parity], wave, 0);
    const float inv = row_inv<T>(acc, cols, eps);
    for (int j = threadIdx.x; j < cols; j += 256) {
      float v = load_elem<T>(src, o + j) * inv;
      if constexpr (HAS_W) v = load_elem<T>(w, j) * round_to<T>(v);
      store_elem<T>(y, o + j, v);
    }
  }
}

// ---- host side ------------------------------------------------------------------------------------------------------

// Tuning slots (0 = automatic): waves per row, vectors per lane, resident blocks per CU, forced generic kernel (1),
// non-temporal loads (1 on, 2 off).
enum { kTuneWaves = 0, kTuneNv = 1, kTuneBlocksPerCu = 2, kTuneGeneric = 3, kTuneNtLoads = 4 };

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

struct Args {
  const void* x;
  const void* w;
  void* y;
  const void* res;
  void* res_out;
  long long rows;
  long long nvec;
  int cols;
  float eps;
  hipStream_t stream;
};

template <typename T, int WAVES, int NV, bool FULL, bool HAS_W, bool RES, bool NTL>
int launch_k(const Args& a) {
  constexpr int BW = WAVES < 4 ? 4 : WAVES;
  constexpr int GROUPS = BW / WAVES;
  auto kern = rmsnorm_rows<T, WAVES, NV, FULL, HAS_W, RES, NTL, true>;
  static int occ = 0;
  if (occ <= 0) occ = blocks_per_cu(kern, BW * kWave);
  // about 8 resident waves per CU by default (more waves only contend for the memory queues; measured on MI355X)
  int per_cu = rw_host::tune_get(kTuneBlocksPerCu);
  if (per_cu <= 0) per_cu = 8 / BW > 1 ? 8 / BW : 1;
  if (per_cu > occ) per_cu = occ;
  const long long need = (a.rows + GROUPS - 1) / GROUPS;
  long long grid = (long long)rw_host::device_cus() * per_cu;
  if (grid > need) grid = need;
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(BW * kWave), 0, a.stream, a.x, a.res, a.w, a.y, a.res_out, a.rows,
                     a.nvec, a.cols, a.eps);
  return (int)hipGetLastError();
}

template <typename T, int WAVES, int NV, bool HAS_W, bool RES, bool NTL>
int launch_nv(const Args& a) {
  if (a.nvec == (long long)WAVES * kWave * NV) return launch_k<T, WAVES, NV, true, HAS_W, RES, NTL>(a);
  return launch_k<T, WAVES, NV, false, HAS_W, RES, NTL>(a);
}

template <typename T, int WAVES, bool HAS_W, bool RES, bool NTL>
int launch_w(int nv, const Args& a) {
  switch (nv) {
    case 1: return launch_nv<T, WAVES, 1, HAS_W, RES, NTL>(a);
    case 2: return launch_nv<T, WAVES, 2, HAS_W, RES, NTL>(a);
    case 4: return launch_nv<T, WAVES, 4, HAS_W, RES, NTL>(a);
    case 8: return launch_nv<T, WAVES, 8, HAS_W, RES, NTL>(a);
    default: return rw_host::kInvalid;
  }
}

template <typename T, bool HAS_W, bool RES, bool NTL>
int launch_rows(int waves, int nv, const Args& a) {
  switch (waves) {
    case 1: return launch_w<T, 1, HAS_W, RES, NTL>(nv, a);
    case 2: return launch_w<T, 2, HAS_W, RES, NTL>(nv, a);
    case 4: return launch_w<T, 4, HAS_W, RES, NTL>(nv, a);
    case 8: return launch_w<T, 8, HAS_W, RES, NTL>(nv, a);
    case 16: return launch_w<T, 16, HAS_W, RES, NTL>(nv, a);
    default: return rw_host::kInvalid;
  }
}

template <typename T, bool HAS_W, bool RES = false>
int launch_typed(const void* x, const void* w, void* y, long long rows, int cols, float eps, hipStream_t stream,
                 const void* res = nullptr, void* res_out = nullptr) {
  const bool vec = cols % T::V == 0 && rw_host::aligned16(x) && rw_host::aligned16(y) &&
                   (!HAS_W || rw_host::aligned16(w)) &&
                   (!RES || (rw_host::aligned16(res) && rw_host::aligned16(res_out)));
  const long long nvec = cols / T::V;
  if (vec && rw_host::tune_get(kTuneGeneric) != 1 && nvec <= (long long)kMaxWaves * kWave * kMaxNv) {
    // One wave per row up to 4 vectors per lane (2048 two-byte columns), then more waves at 4 vectors per lane (and 8
    // per lane once 16 waves are not enough).
    auto auto_waves = [&] {
      const int w = pow2_at_least((nvec + (long long)kWave * 4 - 1) / ((long long)kWave * 4));
      return w > kMaxWaves ? kMaxWaves : w;
    };
    auto auto_nv = [&](int w) { return pow2_at_least((nvec + (long long)w * kWave - 1) / ((long long)w * kWave)); };
    int waves = rw_host::tune_get(kTuneWaves), nv = rw_host::tune_get(kTuneNv);
    if (waves <= 0) waves = auto_waves();
    if (nv <= 0) nv = auto_nv(waves);
    // a tuned shape the row kernel does not have (launch_rows below) is ignored: the automatic choice runs
    const bool shape = (waves == 1 || waves == 2 || waves == 4 || waves == 8 || waves == 16) &&
                       (nv == 1 || nv == 2 || nv == 4 || nv == 8);
    if (!shape) {
      waves = auto_waves();
      nv = auto_nv(waves);
    }
    if ((long long)waves * kWave * nv >= nvec) {
      const Args a{x, w, y, res, res_out, rows, nvec, cols, eps, stream};
      // non-temporal loads unless switched off (2): x is read once
      return rw_host::tune_get(kTuneNtLoads) != 2 ? launch_rows<T, HAS_W, RES, true>(waves, nv, a)
                                                  : launch_rows<T, HAS_W, RES, false>(waves, nv, a);
    }
  }
  long long grid = (long long)rw_host::device_cus() * 8;
  if (grid > rows) grid = rows;
  hipLaunchKernelGGL((rmsnorm_generic<T, HAS_W, RES>), dim3((unsigned)grid), dim3(256), 0, stream, x, res, w, y,
                     res_out, rows, cols, eps);
  return (int)hipGetLastError();
}

// The reference's argument checks (rmsnorm/kernel.cu:134-135). `threads` is its CUDA block size: validated the same
// way and otherwise unused, since the row grouping is chosen from the row length.
int validate(long long rows, int cols, int threads) {
  if (rows > 2147483647LL || cols <= 0 || threads < 32 || threads > 1024 || threads % 32) return rw_host::kInvalid;
  return rw_host::kOk;
}

}  // namespace

// rmsnorm/kernel.cu:132 `launch`: dtype 1 = bf16, 2 = fp16; y = x * inv with no weight. rows <= 0 is a no-op.
extern "C" int launch(const void* x, void* y, long long rows, int cols, int dtype, float eps, int threads,
                      hipStream_t stream) {
  if (rows <= 0) return rw_host::kOk;
  if (validate(rows, cols, threads)) return rw_host::kInvalid;
  if (dtype == 1) return launch_typed<BF16, false>(x, nullptr, y, rows, cols, eps, stream);
  if (dtype == 2) return launch_typed<F16, false>(x, nullptr, y, rows, cols, eps, stream);
  return rw_host::kInvalid;
}

// Weighted RMSNorm (no counterpart in the reference, which has no weight): y = T(w * T(x * inv)) with w[cols] in x's
// dtype; w == nullptr gives `launch`'s result. Same argument checks and return codes as `launch`.
extern "C" int rmsnorm_launch_weighted(const void* x, const void* weight, void* y, long long rows, int cols, int dtype,
                                       float eps, int threads, hipStream_t stream) {
  if (!weight) return launch(x, y, rows, cols, dtype, eps, threads, stream);
  if (rows <= 0) return rw_host::kOk;
  if (validate(rows, cols, threads)) return rw_host::kInvalid;
  if (dtype == 1) return launch_typed<BF16, true>(x, weight, y, rows, cols, eps, stream);
  if (dtype == 2) return launch_typed<F16, true>(x, weight, y, rows, cols, eps, stream);
  return rw_host::kInvalid;
}

// Fused residual add + RMSNorm (no counterpart in the reference; the step before an inference layer's norm):
// h = T(x + residual) is written to residual_out, then y = RMSNorm(h) (times weight when weight != nullptr), in one
// pass: x and residual read once, residual_out and y written once. residual_out may be residual and y may be x (in
// place). Same argument checks and return codes as `launch`; residual and residual_out must not be null.
extern "C" int rmsnorm_add_launch(const void* x, const void* residual, const void* weight, void* y, void* residual_out,
                                  long long rows, int cols, int dtype, float eps, int threads, hipStream_t stream) {
  if (rows <= 0) return rw_host::kOk;
  if (validate(rows, cols, threads) || !residual || !residual_out) return rw_host::kInvalid;
  if (dtype == 1)
    return weight ? launch_typed<BF16, true, true>(x, weight, y, rows, cols, eps, stream, residual, residual_out)
                  : launch_typed<BF16, false, true>(x, nullptr, y, rows, cols, eps, stream, residual, residual_out);
  if (dtype == 2)
    return weight ? launch_typed<F16, true, true>(x, weight, y, rows, cols, eps, stream, residual, residual_out)
                  : launch_typed<F16, false, true>(x, nullptr, y, rows, cols, eps, stream, residual, residual_out);
  return rw_host::kInvalid;
}

extern "C" int rmsnorm_tune(int slot, int value) { return rw_host::tune_set(slot, value); }
