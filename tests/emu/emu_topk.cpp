// Runs csrc/topk.hip's plan() and launch() under the CPU emulation (hip/hip_runtime.h beside this file) and compares
// every launch with the oracle (oracle/oracle.c: oracle_topk), bit for bit: values, int64 indices, and the caller's
// counters left at zero; a launch must not allocate (the caller's work and counters carry the hand-off). Each launch
// is followed by topk_launch_sample(), whose values, indices and draws must equal launch()'s and
// topk_sample_launch()'s on them, with every draw one of the oracle's admissible draws (oracle_topk_sample_band: the
// exact draw's position, and its neighbour where the uniform or the nucleus cut lies within rounding of a boundary).
// Every buffer the kernels touch (input, outputs, work and counters) lies between guard pages.
//
// usage: emu_topk rows cols dtype ks chunk min_chunk reps seed [shuffle_seed [pattern]]
//   dtype 0 fp32, 1 bf16; ks comma-separated; chunk 0 takes plan()'s (min_chunk max 16k for k > 64, as the
//   wrapper); reps launches per k on the same buffers; shuffle_seed >= 0 shuffles the workgroup order and each
//   round of the lane schedule; pattern: randn (N(0, 2)), ints (0..5: ties), ascending, descending, negative (all
//   values below -1), allones (rows of the all-ones NaN with a few real values), outlier (randn and one value of 1e30
//   per row), binades (randn scaled over 24 binades), clustered (randn raised inside one eighth of each row, by 4 on
//   even rows and by 0.6 on odd rows, so that one or two chunks hold most of the row's largest values).
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

extern "C" long long plan(long long rows, long long cols, int dtype, int threads, int depth, int min_chunk);
extern "C" int launch(const void* x, void* values, void* indices, void* work, void* counters, long long rows,
                      long long cols, int k, int dtype, int threads, int depth, long long chunk, hipStream_t stream);
extern "C" int topk_launch_sample(const void* x, void* values, void* indices, void* work, void* counters,
                                  long long rows, long long cols, int k, int dtype, int threads, int depth,
                                  long long chunk, const float* uniforms, void* out, float temperature, float top_p,
                                  hipStream_t stream);
extern "C" int topk_sample_launch(const void* values, const void* indices, const float* uniforms, void* out,
                                  long long rows, int k, int dtype, float temperature, float top_p,
                                  hipStream_t stream);
extern "C" int topk_tune(int slot, int value);
extern "C" void oracle_topk(const void* x, void* values, int64_t* indices, long long rows, long long cols, int k,
                            int dtype);
extern "C" void oracle_topk_sample_band(const void* values, const float* u, int* lo, int* hi, long long rows, int k,
                                        int dtype, float temperature, float top_p);
extern "C" void oracle_topk_sample(const void* values, const int64_t* indices, const float* u, int64_t* out,
                                   long long rows, int k, int dtype, float temperature, float top_p, int* ambiguous);

static uint16_t bf16_rne(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

int main(int argc, char** argv) {
  if (argc < 9) {
    std::fprintf(stderr, "usage: rows cols dtype ks chunk min_chunk reps seed [shuffle_seed [pattern]]\n");
    return 2;
  }
  const long long rows = atoll(argv[1]), cols = atoll(argv[2]);
  const int dtype = atoi(argv[3]);
  std::vector<int> ks;
  for (char* p = argv[4]; *p;) {
    ks.push_back((int)strtol(p, &p, 10));
    if (*p == ',') ++p;
  }
  const long long chunk_arg = atoll(argv[5]);
  const int min_chunk = atoi(argv[6]), reps = atoi(argv[7]), seed = atoi(argv[8]);
  emu::S().shuffle_seed = argc > 9 ? atoi(argv[9]) : -1;
  if (emu::S().shuffle_seed >= 0) emu::S().rng.seed(emu::S().shuffle_seed);
  const std::string pattern = argc > 10 ? argv[10] : "randn";
  if (std::getenv("EMU_TOPK_NAIVE") && topk_tune(1, 1) != 0) return 2;  // launch() takes the naive tier
  const size_t esz = dtype == 0 ? 4 : 2;
  const size_t n = (size_t)rows * cols;
  std::vector<char> host(n * esz);
  std::mt19937_64 g(seed);
  std::normal_distribution<float> nd(0.0f, 2.0f);
  for (size_t i = 0; i < n; ++i) {
    const long long r = (long long)(i / cols), c = (long long)(i % cols);
    float f = nd(g);
    bool ones = false;
    if (pattern == "ints") f = (float)(g() % 6);
    else if (pattern == "ascending") f = (float)c;
    else if (pattern == "descending") f = (float)(cols - c);
    else if (pattern == "negative") f = -1.0f - std::fabs(f);
    else if (pattern == "allones") ones = r % 3 == 0 ? c % 7 == 0 : r % 3 == 1 ? c != 5 : c < cols - 10;
    else if (pattern == "outlier") f = c == (r * 7919) % cols ? 1e30f : f;  // one value far above the rest
    else if (pattern == "binades") f = std::ldexp(f, (int)(c % 24) - 12);  // magnitudes over 24 binades
    else if (pattern == "clustered") {
      const long long w = cols / 8, at = (r * 3 % 8) * w + (r * 101) % (w + 1);
      f += c >= at && c < at + w ? (r % 2 ? 0.6f : 4.0f) : 0.0f;
    }
    else if (pattern != "randn") {
      std::fprintf(stderr, "unknown pattern %s\n", pattern.c_str());
      return 2;
    }
    if (dtype == 0) {
      uint32_t u;
      std::memcpy(&u, &f, 4);
      if (ones) u = 0xffffffffu;
      std::memcpy(&host[i * 4], &u, 4);
    } else {
      const uint16_t b = ones ? (uint16_t)0xffff : bf16_rne(f);
      std::memcpy(&host[i * 2], &b, 2);
    }
  }
  void* x = nullptr;
  if (hipMalloc(&x, n * esz) != hipSuccess) return 3;
  std::memcpy(x, host.data(), n * esz);
  float* uni = nullptr;
  hipMalloc((void**)&uni, rows * 4);
  for (long long r = 0; r < rows; ++r) uni[r] = (float)((r * 37 + 11) % 100) / 100.0f;
  int bad = 0;
  for (int k : ks) {
    if (k > cols) continue;
    const int mc = k > 64 && 16 * k > min_chunk ? 16 * k : min_chunk;
    const long long chunk = chunk_arg > 0 ? chunk_arg : plan(rows, cols, dtype, 256, 4, mc);
    const long long nch = (cols + chunk - 1) / chunk;
    void *vals, *idx, *work, *cnt;
    hipMalloc(&vals, rows * k * esz);
    hipMalloc(&idx, rows * k * 8);
    hipMalloc(&work, (nch > 1 ? rows * nch * k : 1) * 8);
    hipMalloc(&cnt, rows * 4);
    std::memset(cnt, 0, rows * 4);
    std::vector<char> rv(rows * k * esz);
    std::vector<int64_t> ri(rows * k);
    oracle_topk(host.data(), rv.data(), ri.data(), rows, cols, k, dtype);
    for (int rep = 0; rep < reps; ++rep) {
      std::memset(vals, 0xA5, rows * k * esz);
      std::memset(idx, 0xA5, rows * k * 8);
      const long long m0 = emu::mallocs();
      const int err = launch(x, vals, idx, work, cnt, rows, cols, k, dtype, 256, 4, chunk, nullptr);
      if (emu::mallocs() != m0) {
        std::printf("k=%d chunk=%lld: launch allocated device memory\n", k, chunk);
        ++bad;
      }
      if (err) {
        std::printf("k=%d chunk=%lld: launch returned %d\n", k, chunk, err);
        ++bad;
        break;
      }
      const bool ok_i = std::memcmp(idx, ri.data(), rows * k * 8) == 0;
      const bool ok_v = std::memcmp(vals, rv.data(), rows * k * esz) == 0;
      bool zero = true;
      for (long long i = 0; i < rows; ++i) zero &= ((unsigned*)cnt)[i] == 0;
      // the fused draw: the same list, and the draw of topk_sample_launch() on it
      void *vals2, *idx2, *drawn1, *drawn2;
      hipMalloc(&vals2, rows * k * esz);
      hipMalloc(&idx2, rows * k * 8);
      hipMalloc(&drawn1, rows * 8);
      hipMalloc(&drawn2, rows * 8);
      const float temperature = rep % 2 ? 0.0f : 0.8f, top_p = 0.9f;
      const int err2 = topk_launch_sample(x, vals2, idx2, work, cnt, rows, cols, k, dtype, 256, 4, chunk, uni,
                                          drawn2, temperature, top_p, nullptr);
      const int err3 = topk_sample_launch(vals, idx, uni, drawn1, rows, k, dtype, temperature, top_p, nullptr);
      bool fused_ok = !err2 && !err3 && std::memcmp(vals2, vals, rows * k * esz) == 0 &&
                      std::memcmp(idx2, idx, rows * k * 8) == 0 && std::memcmp(drawn1, drawn2, rows * 8) == 0;
      // and the oracle's admissible draws, every row
      std::vector<int> lo(rows), hi(rows);
      oracle_topk_sample_band(rv.data(), uni, lo.data(), hi.data(), rows, k, dtype, temperature, top_p);
      for (long long r = 0; r < rows; ++r) {
        bool in = false;
        for (int p = lo[r]; p <= hi[r] && p < k; ++p) in |= ((int64_t*)drawn2)[r] == ri[r * k + p];
        fused_ok &= in;
      }
      hipFree(vals2);
      hipFree(idx2);
      hipFree(drawn1);
      hipFree(drawn2);
      if (!fused_ok) {
        ++bad;
        std::printf("k=%d chunk=%lld rep %d: fused draw differs (errors %d %d)\n", k, chunk, rep, err2, err3);
      }
      if (!ok_i || !ok_v || !zero) {
        ++bad;
        long long first = -1;
        for (long long i = 0; i < rows * k && first < 0; ++i)
          if (((int64_t*)idx)[i] != ri[i]) first = i;
        std::printf("k=%d chunk=%lld rep %d: MISMATCH indices %d values %d counters zero %d, first bad index %lld\n",
                    k, chunk, rep, ok_i, ok_v, zero, first);
      }
    }
    std::printf("k=%d chunk=%lld nchunks=%lld reps=%d done\n", k, chunk, nch, reps);
    std::fflush(stdout);
    hipFree(vals);
    hipFree(idx);
    hipFree(work);
    hipFree(cnt);
  }
  hipFree(x);
  hipFree(uni);
  std::printf(bad ? "FAILED %d\n" : "ALL OK\n", bad);
  return bad ? 1 : 0;
}
