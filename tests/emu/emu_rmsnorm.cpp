// Runs csrc/rmsnorm.hip's entry points under the CPU emulation (hip/hip_runtime.h beside this file) and compares
// every output with the oracle (oracle/oracle.c: oracle_rmsnorm, oracle_rmsnorm_add) bit for bit. Every device buffer
// lies between guard pages.
//
// usage: emu_rmsnorm rows cols dtype(1 bf16, 2 fp16) mode seed [waves nv blocks_per_cu [offset]]
//   mode 0: launch (no weight); 1: rmsnorm_launch_weighted; 2: rmsnorm_add_launch with a weight, into new buffers;
//   3: rmsnorm_add_launch in place (residual_out = residual, y = x). waves / nv / blocks_per_cu force the row
//   kernel's shape through rmsnorm_tune (0: automatic); offset shifts x by that many elements from a 16-byte boundary.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <vector>

extern "C" int launch(const void* x, void* y, long long rows, int cols, int dtype, float eps, int threads,
                      hipStream_t stream);
extern "C" int rmsnorm_launch_weighted(const void* x, const void* weight, void* y, long long rows, int cols, int dtype,
                                       float eps, int threads, hipStream_t stream);
extern "C" int rmsnorm_add_launch(const void* x, const void* residual, const void* weight, void* y,
                                  void* residual_out, long long rows, int cols, int dtype, float eps, int threads,
                                  hipStream_t stream);
extern "C" int rmsnorm_tune(int slot, int value);
extern "C" void oracle_rmsnorm(const uint16_t* x, const uint16_t* w, uint16_t* y, long long rows, long long cols,
                               int dtype, float eps, float* inv_out);
extern "C" void oracle_rmsnorm_add(const uint16_t* x, const uint16_t* res, const uint16_t* w, uint16_t* y,
                                   uint16_t* h_out, long long rows, long long cols, int dtype, float eps);

static uint16_t to_bits(float f, int dtype) {
  if (dtype == 1) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
  }
  const _Float16 h = (_Float16)f;
  uint16_t b;
  std::memcpy(&b, &h, 2);
  return b;
}

int main(int argc, char** argv) {
  if (argc < 6) {
    std::fprintf(stderr, "usage: rows cols dtype mode seed [waves nv blocks_per_cu [offset]]\n");
    return 2;
  }
  const long long rows = atoll(argv[1]);
  const int cols = atoi(argv[2]), dtype = atoi(argv[3]), mode = atoi(argv[4]), seed = atoi(argv[5]);
  if (argc > 8) {
    rmsnorm_tune(0, atoi(argv[6]));
    rmsnorm_tune(1, atoi(argv[7]));
    rmsnorm_tune(2, atoi(argv[8]));
  }
  const int offset = argc > 9 ? atoi(argv[9]) : 0;
  const float eps = 1e-6f;
  const size_t n = (size_t)rows * cols;
  std::mt19937_64 g(seed);
  std::normal_distribution<float> nd(0.0f, 1.0f);
  std::uniform_real_distribution<float> ud(0.5f, 1.5f);
  std::vector<uint16_t> hx(n), hr(n), hw(cols);
  for (size_t i = 0; i < n; ++i) hx[i] = to_bits(nd(g), dtype);
  for (size_t i = 0; i < n; ++i) hr[i] = to_bits(nd(g), dtype);
  for (int i = 0; i < cols; ++i) hw[i] = to_bits(ud(g), dtype);
  // device buffers (x shifted by `offset` elements)
  uint16_t *xb, *rb, *w, *y, *ro;
  hipMalloc((void**)&xb, (n + offset) * 2);
  hipMalloc((void**)&rb, n * 2);
  hipMalloc((void**)&w, cols * 2);
  hipMalloc((void**)&y, n * 2);
  hipMalloc((void**)&ro, n * 2);
  uint16_t* x = xb + offset;
  std::memcpy(x, hx.data(), n * 2);
  std::memcpy(rb, hr.data(), n * 2);
  std::memcpy(w, hw.data(), cols * 2);
  std::vector<uint16_t> ry(n), rh(n);
  int err = 0;
  bool ok = true;
  if (mode == 0 || mode == 1) {
    oracle_rmsnorm(hx.data(), mode == 1 ? hw.data() : nullptr, ry.data(), rows, cols, dtype, eps, nullptr);
    err = mode == 0 ? launch(x, y, rows, cols, dtype, eps, 256, nullptr)
                    : rmsnorm_launch_weighted(x, w, y, rows, cols, dtype, eps, 256, nullptr);
    ok = !err && std::memcmp(y, ry.data(), n * 2) == 0;
  } else {
    oracle_rmsnorm_add(hx.data(), hr.data(), hw.data(), ry.data(), rh.data(), rows, cols, dtype, eps);
    if (mode == 2) {
      err = rmsnorm_add_launch(x, rb, w, y, ro, rows, cols, dtype, eps, 256, nullptr);
      ok = !err && std::memcmp(y, ry.data(), n * 2) == 0 && std::memcmp(ro, rh.data(), n * 2) == 0 &&
           std::memcmp(rb, hr.data(), n * 2) == 0;
    } else {
      err = rmsnorm_add_launch(x, rb, w, x, rb, rows, cols, dtype, eps, 256, nullptr);
      ok = !err && std::memcmp(x, ry.data(), n * 2) == 0 && std::memcmp(rb, rh.data(), n * 2) == 0;
    }
  }
  long long first = -1;
  if (!ok) {
    const uint16_t* got = mode == 3 ? x : y;
    for (size_t i = 0; i < n && first < 0; ++i)
      if (got[i] != ry[i]) first = (long long)i;
  }
  std::printf("rows %lld cols %d dtype %d mode %d: %s (err %d, first difference %lld)\n", rows, cols, dtype, mode,
              ok ? "ALL OK" : "FAILED", err, first);
  hipFree(xb);
  hipFree(rb);
  hipFree(w);
  hipFree(y);
  hipFree(ro);
  return ok ? 0 : 1;
}
