// Two copies of the top-k library in one process, each the kernels' source (csrc/topk.hip) built for the CPU under
// the HIP emulation as a shared object of its own and opened with dlopen (RTLD_LOCAL): launches alternate between the
// copies on the same caller buffers (one input, one work, one counters array) with k = 1, 50 and 1024 interleaved,
// and every launch is compared bit for bit with the oracle, with the counters left at zero and no allocation by
// either copy. This is the process layout of two GPU faults recorded in earlier timing runs (several top-k libraries
// loaded at once, k = 1 / 50 / 1024 back to back); the kernels keep no state of their own between launches.
//
// usage: emu_two_copies lib_a.so lib_b.so rows cols dtype rounds seed
#include <dlfcn.h>
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <vector>

typedef long long (*plan_fn)(long long, long long, int, int, int, int);
typedef int (*launch_fn)(const void*, void*, void*, void*, void*, long long, long long, int, int, int, int, long long,
                         hipStream_t);
extern "C" void oracle_topk(const void* x, void* values, int64_t* indices, long long rows, long long cols, int k,
                            int dtype);

struct Copy {
  void* handle;
  plan_fn plan;
  launch_fn launch;
};

static bool open_copy(const char* path, Copy& c) {
  c.handle = dlopen(path, RTLD_NOW | RTLD_LOCAL);
  if (!c.handle) {
    std::printf("dlopen %s: %s\n", path, dlerror());
    return false;
  }
  c.plan = (plan_fn)dlsym(c.handle, "plan");
  c.launch = (launch_fn)dlsym(c.handle, "launch");
  return c.plan && c.launch;
}

int main(int argc, char** argv) {
  if (argc < 8) {
    std::fprintf(stderr, "usage: lib_a lib_b rows cols dtype rounds seed\n");
    return 2;
  }
  Copy lib[2];
  if (!open_copy(argv[1], lib[0]) || !open_copy(argv[2], lib[1])) return 3;
  if (lib[0].launch == lib[1].launch) {
    std::printf("the two copies resolve to one launch()\n");
    return 3;
  }
  const long long rows = atoll(argv[3]), cols = atoll(argv[4]);
  const int dtype = atoi(argv[5]), rounds = atoi(argv[6]), seed = atoi(argv[7]);
  const size_t esz = dtype == 0 ? 4 : 2, n = (size_t)rows * cols;
  std::vector<char> host(n * esz);
  std::mt19937_64 g(seed);
  std::normal_distribution<float> nd(0.0f, 2.0f);
  for (size_t i = 0; i < n; ++i) {
    const float f = nd(g);
    uint32_t u;
    std::memcpy(&u, &f, 4);
    if (dtype == 0) std::memcpy(&host[i * 4], &u, 4);
    else {
      const uint16_t b = (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
      std::memcpy(&host[i * 2], &b, 2);
    }
  }
  void *x, *vals, *idx, *work, *cnt;
  const int ks[3] = {1, 50, 1024};
  long long most = 1;  // the largest work any launch below needs (a shared caller workspace)
  long long chunks[3];
  for (int j = 0; j < 3; ++j) {
    const int k = ks[j];
    chunks[j] = lib[0].plan(rows, cols, dtype, 256, 4, k > 64 ? 16 * k : 2048);
    const long long nch = (cols + chunks[j] - 1) / chunks[j];
    if (nch > 1 && rows * nch * k > most) most = rows * nch * k;
  }
  hipMalloc(&x, n * esz);
  std::memcpy(x, host.data(), n * esz);
  hipMalloc(&vals, rows * 1024 * esz);
  hipMalloc(&idx, rows * 1024 * 8);
  hipMalloc(&work, most * 8);
  hipMalloc(&cnt, rows * 4);
  std::memset(cnt, 0, rows * 4);
  std::vector<std::vector<char>> rv(3);
  std::vector<std::vector<int64_t>> ri(3);
  for (int j = 0; j < 3; ++j) {
    rv[j].resize(rows * ks[j] * esz);
    ri[j].resize(rows * ks[j]);
    oracle_topk(host.data(), rv[j].data(), ri[j].data(), rows, cols, ks[j], dtype);
  }
  int bad = 0;
  for (int r = 0; r < rounds; ++r) {
    for (int j = 0; j < 3; ++j) {
      const Copy& c = lib[(r + j) % 2];
      const int k = ks[j];
      std::memset(vals, 0xA5, rows * k * esz);
      std::memset(idx, 0xA5, rows * k * 8);
      const long long m0 = emu::mallocs();
      const int err = c.launch(x, vals, idx, work, cnt, rows, cols, k, dtype, 256, 4, chunks[j], nullptr);
      bool zero = true;
      for (long long i = 0; i < rows; ++i) zero &= ((unsigned*)cnt)[i] == 0;
      const bool ok = !err && emu::mallocs() == m0 && zero && std::memcmp(idx, ri[j].data(), rows * k * 8) == 0 &&
                      std::memcmp(vals, rv[j].data(), rows * k * esz) == 0;
      if (!ok) {
        ++bad;
        std::printf("round %d copy %d k=%d: err %d, counters zero %d, allocations %lld, outputs %s\n", r, (r + j) % 2,
                    k, err, zero, emu::mallocs() - m0, ok ? "equal" : "differ");
      }
    }
    std::printf("round %d done\n", r);
    std::fflush(stdout);
  }
  std::printf(bad ? "FAILED %d\n" : "ALL OK\n", bad);
  return bad ? 1 : 0;
}
