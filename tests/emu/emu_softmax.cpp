// Runs csrc/softmax.hip's launch() under the CPU emulation (hip/hip_runtime.h beside this file) and compares the
// output with the oracle (oracle/oracle.c: oracle_softmax, the fp64 softmax rounded once) within the softmax
// tolerance: fp32 |y - oracle| <= 1e-5 |oracle| (one ulp for subnormal results), bf16 within 1 ulp (NaN must meet
// NaN). Every device buffer lies between guard pages. The co-resident tier (4) needs EMU_CONCURRENT: its workgroups
// wait for one another.
//
// usage: emu_softmax rows cols dtype(0 fp32, 1 bf16) tier seed [waves nv [offset [pattern [reps [wait_ticks]]]]]
//   tier: 1 row, 2 stream, 3 generic, 4 co-resident (preferred through softmax_tune); waves / nv: the row tier's
//   shape (tier 1), the stream tier's waves (tier 2), the co-resident tier's row groups in nv (tier 4; fewer groups
//   than rows make each workgroup walk several rows), 0 automatic; offset shifts x and y by that many elements from a
//   16-byte boundary (a misaligned row takes the generic tier); pattern: randn (N(0, 4)) or special (-inf elements,
//   an all -inf row, a row of one huge value); reps: launches on the same buffers, each checked (the co-resident
//   tier's pair table is reused by the next launch, under fresh tags); wait_ticks bounds the co-resident tier's wait
//   (1 makes its workgroups stop waiting and take the row's statistics from x).
// EMU_GRAPH set: after an eager launch, the launch is recorded as a graph (the emulation's capture) and every rep
// replays it, each with new values in x (seed + rep); odd reps first run an eager launch of the same shape on other
// values and buffers, which leaves its own pairs in the table. Every replay is checked against the oracle of its x.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

extern "C" int launch(const void* x, void* y, long long rows, long long cols, int dtype, int threads, int aux,
                      hipStream_t stream);
extern "C" int softmax_tune(int slot, int value);
extern "C" void oracle_softmax(const void* x, void* y, long long rows, long long cols, int dtype);

static uint16_t bf16_rne(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

static int ordered(uint16_t b) { return b & 0x8000 ? 0x8000 - (int)b : (int)b; }
static bool nan16(uint16_t b) { return (b & 0x7f80) == 0x7f80 && (b & 0x7f); }

int main(int argc, char** argv) {
  if (argc < 6) {
    std::fprintf(stderr, "usage: rows cols dtype tier seed [waves nv [offset [pattern]]]\n");
    return 2;
  }
  const long long rows = atoll(argv[1]), cols = atoll(argv[2]);
  const int dtype = atoi(argv[3]), tier = atoi(argv[4]), seed = atoi(argv[5]);
  const int waves = argc > 6 ? atoi(argv[6]) : 0, nv = argc > 7 ? atoi(argv[7]) : 0;
  const int offset = argc > 8 ? atoi(argv[8]) : 0;
  const std::string pattern = argc > 9 ? argv[9] : "randn";
  const int reps = argc > 10 ? atoi(argv[10]) : 1;
  if (argc > 11) softmax_tune(7, atoi(argv[11]));
  softmax_tune(5, tier);
  if (tier == 2) {
    softmax_tune(3, waves);
  } else if (tier == 4) {
    softmax_tune(4, nv);
  } else {
    softmax_tune(0, waves);
    softmax_tune(1, nv);
  }
  const size_t esz = dtype == 0 ? 4 : 2, n = (size_t)rows * cols;
  const bool graph = std::getenv("EMU_GRAPH") != nullptr;
  if (pattern != "randn" && pattern != "special") {
    std::fprintf(stderr, "unknown pattern %s\n", pattern.c_str());
    return 2;
  }
  // the input of rep r: seed + r (rep 0 only, without EMU_GRAPH)
  auto make_input = [&](int s, std::vector<char>& host) {
    std::mt19937_64 g(s);
    std::normal_distribution<float> nd(0.0f, 4.0f);
    host.assign(n * esz, 0);
    for (size_t i = 0; i < n; ++i) {
      const long long r = (long long)(i / cols), c = (long long)(i % cols);
      float v = nd(g);
      if (pattern == "special") {
        if (r % 4 == 0 && c % 5 == 1) v = -INFINITY;
        if (r % 4 == 1) v = -INFINITY;
        if (r % 4 == 2 && c == cols / 2) v = 80.0f;
      }
      if (dtype == 0) std::memcpy(&host[i * 4], &v, 4);
      else {
        const uint16_t b = bf16_rne(v);
        std::memcpy(&host[i * 2], &b, 2);
      }
    }
  };
  std::vector<char> host;
  make_input(seed, host);
  char *xb, *yb, *x2, *y2;
  hipMalloc((void**)&xb, (n + offset) * esz);
  hipMalloc((void**)&yb, (n + offset) * esz);
  hipMalloc((void**)&x2, n * esz);
  hipMalloc((void**)&y2, n * esz);
  char* x = xb + offset * esz;
  char* y = yb + offset * esz;
  std::memcpy(x, host.data(), n * esz);
  std::vector<char> ref(n * esz);
  oracle_softmax(host.data(), ref.data(), rows, cols, dtype);
  int err = 0;
  long long bad = 0, first = -1;
  emu::Graph recorded;
  if (graph) {
    // an eager launch first (a warm-up, as a graph capture usually follows one), then the capture
    std::memcpy(x2, host.data(), n * esz);
    err = launch(x2, y2, rows, cols, dtype, 256, 0, nullptr);
    emu::capture_begin(recorded);
    err = launch(x, y, rows, cols, dtype, 256, 0, nullptr);
    emu::capture_end();
  }
  for (int rep = 0; rep < reps && !err && !bad; ++rep) {
    if (graph && rep > 0) {
      make_input(seed + rep, host);
      std::memcpy(x, host.data(), n * esz);
      oracle_softmax(host.data(), ref.data(), rows, cols, dtype);
    }
    std::memset(y, 0xA5, n * esz);
    if (graph) {
      if (rep % 2) {
        // an eager launch of the same shape on other values in between: its pairs sit in the same table slots
        std::vector<char> other;
        make_input(seed + 1000 + rep, other);
        std::memcpy(x2, other.data(), n * esz);
        err = launch(x2, y2, rows, cols, dtype, 256, 0, nullptr);
      }
      emu::replay(recorded);
    } else {
      err = launch(x, y, rows, cols, dtype, 256, 0, nullptr);
    }
    for (size_t i = 0; i < n && !err; ++i) {
      bool ok;
      if (dtype == 0) {
        float a, b;
        std::memcpy(&a, y + i * 4, 4);
        std::memcpy(&b, &ref[i * 4], 4);
        // below the normal range one ulp (2^-149) is more than 1e-5 of the value: one ulp is allowed there
        const double tol = std::fmax(1e-5 * std::fabs((double)b), 0x1p-149);
        ok = std::isnan(b) ? std::isnan(a) : std::fabs((double)a - b) <= tol;
      } else {
        uint16_t a, b;
        std::memcpy(&a, y + i * 2, 2);
        std::memcpy(&b, &ref[i * 2], 2);
        ok = nan16(b) ? nan16(a) : !nan16(a) && std::abs(ordered(a) - ordered(b)) <= 1;
      }
      if (!ok && first < 0) first = (long long)i;
      bad += !ok;
    }
  }
  const bool input_kept = std::memcmp(x, host.data(), n * esz) == 0;
  const bool ok = !err && !bad && input_kept;
  std::printf("rows %lld cols %lld dtype %d tier %d: %s (err %d, %lld outside tolerance, first %lld, input kept %d)\n",
              rows, cols, dtype, tier, ok ? "ALL OK" : "FAILED", err, bad, first, input_kept);
  hipFree(xb);
  hipFree(yb);
  hipFree(x2);
  hipFree(y2);
  return ok ? 0 : 1;
}
