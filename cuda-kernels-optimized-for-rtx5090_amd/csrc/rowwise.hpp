// Device helpers shared by the row-wise kernels, written for gfx950 (CDNA4, wave64).
//
//  - element formats: fp32, bf16 and fp16 rows moved as raw 16-byte vectors (4 or 8 elements) and widened to fp32 in
//    registers; narrowing is round-to-nearest-even through the hardware packed converts (v_cvt_pk_bf16_f32 on
//    gfx950, which equals the software RNE bit for bit over all 2^32 inputs, NaN staying NaN);
//  - 16-byte global loads and stores, optionally non-temporal (streamed data that is touched once);
//  - wave64 reductions through DPP (quad_perm, row_half_mirror, row_mirror) inside each 16-lane row and v_readlane
//    across the four rows: the result is wave-uniform and its summation order is fixed, so a row's result does not
//    depend on which wave or workgroup computed it;
//  - block reductions through one LDS slot per wave.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rw {

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

// Element formats. `V` is the element count of one 16-byte vector.
struct F32 { static constexpr int V = 4; static constexpr int bytes = 4; };
struct BF16 { static constexpr int V = 8; static constexpr int bytes = 2; };
struct F16 { static constexpr int V = 8; static constexpr int bytes = 2; };

// ---- conversions -------------------------------------------------------------------------------------------------

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __builtin_bit_cast(float, w & 0xffff0000u); }

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, bf16x2));
}
__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, f16x2));
}
__device__ __forceinline__ f32x2 unpack_f16x2(uint32_t w) {
  return __builtin_convertvector(__builtin_bit_cast(f16x2, w), f32x2);
}

// One element rounded to the format and widened back (the value a stored element would read back as).
template <typename T> __device__ __forceinline__ float round_to(float v);
template <> __device__ __forceinline__ float round_to<F32>(float v) { return v; }
template <> __device__ __forceinline__ float round_to<BF16>(float v) { return bf16_lo(pack_bf16x2(v, 0.0f)); }
template <> __device__ __forceinline__ float round_to<F16>(float v) { return unpack_f16x2(pack_f16x2(v, 0.0f)).x; }

// A raw 16-byte vector widened to V floats / V floats narrowed into a raw 16-byte vector.
template <typename T> __device__ __forceinline__ void unpack(const u32x4& r, float* f);
// (A vector element is copied to a scalar before the bit cast: bit-casting the element lvalue itself reads the vector's
// first element.)
template <> __device__ __forceinline__ void unpack<F32>(const u32x4& r, float* f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t u = r[i];
    f[i] = __builtin_bit_cast(float, u);
  }
}
template <> __device__ __forceinline__ void unpack<BF16>(const u32x4& r, float* f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = bf16_lo(r[i]);
    f[2 * i + 1] = bf16_hi(r[i]);
  }
}
template <> __device__ __forceinline__ void unpack<F16>(const u32x4& r, float* f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const f32x2 v = unpack_f16x2(r[i]);
    f[2 * i] = v.x;
    f[2 * i + 1] = v.y;
  }
}

template <typename T> __device__ __forceinline__ u32x4 pack(const float* f);
template <> __device__ __forceinline__ u32x4 pack<F32>(const float* f) {
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = __builtin_bit_cast(uint32_t, f[i]);
  return r;
}
template <> __device__ __forceinline__ u32x4 pack<BF16>(const float* f) {
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = pack_bf16x2(f[2 * i], f[2 * i + 1]);
  return r;
}
template <> __device__ __forceinline__ u32x4 pack<F16>(const float* f) {
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = pack_f16x2(f[2 * i], f[2 * i + 1]);
  return r;
}

// e^d for a value that is rounded to bf16 or fp16 afterwards: 2^(d log2 e) by the hardware's exp2 (v_exp_f32),
// evaluated 64 binades up and scaled back, so that results below the fp32 normal range are not flushed to zero (the
// instruction flushes them). The relative error, about 1e-5 (the roundings of d log2 e + 64 and the instruction's own),
// is far below the 2^-9 half ulp of bf16; four instructions where the correctly rounded expf takes about fourteen, which
// keeps the 16-bit softmax paths (twice the elements per byte of fp32) memory-bound. d = -inf gives 0, NaN stays NaN.
__device__ __forceinline__ float exp_narrow(float d) {
  return __builtin_amdgcn_exp2f(d * 1.44269504088896341f + 64.0f) * 0x1p-64f;
}
// The exponential of a path whose outputs have format T: expf for fp32 (within the 1e-5 relative bar of its results),
// exp_narrow for the 16-bit formats.
template <typename T> __device__ __forceinline__ float exp_to(float d) { return exp_narrow(d); }
template <> __device__ __forceinline__ float exp_to<F32>(float d) { return expf(d); }

// Scalar element access (unaligned / ragged paths).
template <typename T> __device__ __forceinline__ float load_elem(const void* p, long long i);
template <> __device__ __forceinline__ float load_elem<F32>(const void* p, long long i) {
  return static_cast<const float*>(p)[i];
}
template <> __device__ __forceinline__ float load_elem<BF16>(const void* p, long long i) {
  return __builtin_bit_cast(float, (uint32_t) static_cast<const uint16_t*>(p)[i] << 16);
}
template <> __device__ __forceinline__ float load_elem<F16>(const void* p, long long i) {
  return (float)static_cast<const _Float16*>(p)[i];
}
template <typename T> __device__ __forceinline__ void store_elem(void* p, long long i, float v);
template <> __device__ __forceinline__ void store_elem<F32>(void* p, long long i, float v) {
  static_cast<float*>(p)[i] = v;
}
template <> __device__ __forceinline__ void store_elem<BF16>(void* p, long long i, float v) {
  static_cast<uint16_t*>(p)[i] = (uint16_t)(pack_bf16x2(v, 0.0f) & 0xffffu);
}
template <> __device__ __forceinline__ void store_elem<F16>(void* p, long long i, float v) {
  static_cast<uint16_t*>(p)[i] = (uint16_t)(pack_f16x2(v, 0.0f) & 0xffffu);
}

// ---- 16-byte global memory access ----------------------------------------------------------------------------------

// Vector `v` (16-byte units) of the region starting at `p`.
template <bool NT>
__device__ __forceinline__ u32x4 load16(const void* p, long long v) {
  const u32x4* q = static_cast<const u32x4*>(p) + v;
  if constexpr (NT) return __builtin_nontemporal_load(q);
  else return *q;
}
template <bool NT>
__device__ __forceinline__ void store16(void* p, long long v, const u32x4& r) {
  u32x4* q = static_cast<u32x4*>(p) + v;
  if constexpr (NT) __builtin_nontemporal_store(r, q);
  else *q = r;
}

// ---- wave64 reductions ----------------------------------------------------------------------------------------------

// DPP controls: quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror. Applied in this order with a
// commutative operator they leave each 16-lane row holding its row's reduction.
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140;

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ double dpp(double v) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const int lo = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL, 0xF, 0xF, false);
  const int hi = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL, 0xF, 0xF, false);
  return __builtin_bit_cast(double, ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}
__device__ __forceinline__ float readlane(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}
__device__ __forceinline__ double readlane(double v, int lane) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, lane);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), lane);
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

struct OpMax {
  __device__ __forceinline__ float operator()(float a, float b) const { return fmaxf(a, b); }
};
struct OpSum {
  __device__ __forceinline__ float operator()(float a, float b) const { return a + b; }
  __device__ __forceinline__ double operator()(double a, double b) const { return a + b; }
};

// Wave-uniform reduction of v over the 64 lanes (every lane must be active).
template <typename Op, typename F>
__device__ __forceinline__ F wave_reduce(F v, Op op) {
  v = op(v, dpp<kDppXor1>(v));
  v = op(v, dpp<kDppXor2>(v));
  v = op(v, dpp<kDppHalfMirror>(v));
  v = op(v, dpp<kDppMirror>(v));
  return op(op(readlane(v, 0), readlane(v, 16)), op(readlane(v, 32), readlane(v, 48)));
}
__device__ __forceinline__ float wave_max(float v) { return wave_reduce(v, OpMax{}); }
__device__ __forceinline__ float wave_sum(float v) { return wave_reduce(v, OpSum{}); }
__device__ __forceinline__ double wave_sum(double v) { return wave_reduce(v, OpSum{}); }

// Reduction over the WAVES waves [first, first + WAVES) of a block that cooperate on one row: each wave's lane 0
// writes slots[wave], the block synchronizes, and every lane combines the group's slots in wave order. The caller
// alternates between two slot arrays for consecutive reductions so that no slot is rewritten before every wave has
// read it (the barrier of the next reduction separates them).
template <int WAVES, typename Op, typename F>
__device__ __forceinline__ F group_reduce(F v, Op op, F* slots, int wave, int first) {
  v = wave_reduce(v, op);
  if constexpr (WAVES == 1) {
    return v;
  } else {
    if ((threadIdx.x & (kWave - 1)) == 0) slots[wave] = v;
    __syncthreads();
    F r = slots[first];
#pragma unroll
    for (int i = 1; i < WAVES; ++i) r = op(r, slots[first + i]);
    return r;
  }
}

__device__ __forceinline__ int wave_id() { return (int)(threadIdx.x >> 6); }
__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & (kWave - 1)); }

// Orders one wave's LDS writes before its later LDS reads of other lanes' entries (a wave's LDS operations execute in
// order; this keeps the compiler from moving them across).
__device__ __forceinline__ void wave_lds_sync() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_wave_barrier();
}

}  // namespace rw
