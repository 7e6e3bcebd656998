// Runs csrc/rope.hip's entry points under the CPU emulation (hip/hip_runtime.h beside this file) and compares every
// output with the oracle (oracle/oracle.c: oracle_rope_cache, oracle_rope_freq, oracle_rope_table) bit for bit. Every
// device buffer lies between guard pages.
//
// usage: emu_rope tokens q_heads kv_heads head_dim dtype(1 bf16, 2 fp16) form inplace seed
//   form 0/1/2: launch with an fp32 / bf16 / fp16 cos-sin cache (the on-the-fly table, in that dtype); 3:
//   rope_launch_freq; 4: rope_kv_launch (a 3*tokens-slot cache, every fourth token's slot -1). inplace: q_out = q
//   and k_out = k (forms 0-3; form 4 rotates q in place).
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <vector>

extern "C" int launch(const void* q, const void* k, const void* cos_rows, const void* sin_rows, const void* ids,
                      void* q_out, void* k_out, long long tokens, int q_heads, int kv_heads, int head_dim,
                      int qk_dtype, int cache_dtype, int rows, int splits, hipStream_t stream);
extern "C" int rope_launch_freq(const void* q, const void* k, const void* ids, const float* inv_freq, void* q_out,
                                void* k_out, long long tokens, int q_heads, int kv_heads, int head_dim, int qk_dtype,
                                hipStream_t stream);
extern "C" int rope_kv_launch(const void* q, const void* k, const void* v, const void* ids, const float* inv_freq,
                              void* q_out, void* k_cache, void* v_cache, const void* slot_mapping, long long tokens,
                              int q_heads, int kv_heads, int head_dim, int qk_dtype, hipStream_t stream);
extern "C" void oracle_rope_cache(const void* q, const void* k, const void* cos_rows, const void* sin_rows,
                                  const int64_t* ids, void* q_out, void* k_out, long long tokens, int q_heads,
                                  int kv_heads, int head_dim, int qk_dtype, int cache_dtype);
extern "C" void oracle_rope_freq(const void* q, const void* k, const int64_t* ids, const float* inv_freq, void* q_out,
                                 void* k_out, long long tokens, int q_heads, int kv_heads, int head_dim, int qk_dtype);
extern "C" void oracle_rope_table(const float* inv_freq, long long positions, int head_dim, float* cos_out,
                                  float* sin_out);

static uint16_t to_bits(float f, int dtype) {
  if (dtype == 1) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
  }
  const _Float16 h = (_Float16)f;
  uint16_t b;
  std::memcpy(&b, &h, 2);
  return b;
}

template <typename T>
static T* dev_copy(const std::vector<T>& h) {
  T* d = nullptr;
  hipMalloc((void**)&d, h.size() * sizeof(T) + 16);
  std::memcpy(d, h.data(), h.size() * sizeof(T));
  return d;
}

int main(int argc, char** argv) {
  if (argc < 9) {
    std::fprintf(stderr, "usage: tokens q_heads kv_heads head_dim dtype form inplace seed\n");
    return 2;
  }
  const long long tokens = atoll(argv[1]);
  const int qh = atoi(argv[2]), kh = atoi(argv[3]), D = atoi(argv[4]), dtype = atoi(argv[5]), form = atoi(argv[6]),
            inplace = atoi(argv[7]), seed = atoi(argv[8]);
  const int P = 4096, half = D / 2;
  std::mt19937_64 g(seed);
  std::normal_distribution<float> nd(0.0f, 1.0f);
  const size_t nq = (size_t)tokens * qh * D, nk = (size_t)tokens * kh * D;
  std::vector<uint16_t> hq(nq), hk(nk), hv(nk);
  for (auto& b : hq) b = to_bits(nd(g), dtype);
  for (auto& b : hk) b = to_bits(nd(g), dtype);
  for (auto& b : hv) b = to_bits(nd(g), dtype);
  std::vector<int64_t> ids(tokens);
  for (auto& p : ids) p = (int64_t)(g() % P);
  std::vector<float> inv(half);
  for (int i = 0; i < half; ++i) inv[i] = (float)(1.0 / std::pow(10000.0, (2.0 * i) / D));
  std::vector<uint16_t> rq(nq), rk(nk);
  uint16_t* q = dev_copy(hq);
  uint16_t* k = dev_copy(hk);
  int64_t* dids = dev_copy(ids);
  float* dinv = dev_copy(inv);
  uint16_t *qo = q, *ko = k;
  if (!inplace) {
    hipMalloc((void**)&qo, nq * 2);
    hipMalloc((void**)&ko, nk * 2);
  }
  int err = 0;
  bool ok = true;
  if (form <= 2) {
    std::vector<float> cs((size_t)P * D), sn((size_t)P * D);
    oracle_rope_table(inv.data(), P, D, cs.data(), sn.data());
    void *dc, *ds;
    std::vector<uint16_t> c16(cs.size()), s16(sn.size());
    if (form == 0) {
      dc = dev_copy(cs);
      ds = dev_copy(sn);
    } else {
      for (size_t i = 0; i < cs.size(); ++i) {
        c16[i] = to_bits(cs[i], form);
        s16[i] = to_bits(sn[i], form);
      }
      dc = dev_copy(c16);
      ds = dev_copy(s16);
    }
    oracle_rope_cache(hq.data(), hk.data(), form == 0 ? (const void*)cs.data() : c16.data(),
                      form == 0 ? (const void*)sn.data() : s16.data(), ids.data(), rq.data(), rk.data(), tokens, qh, kh,
                      D, dtype, form);
    err = launch(q, k, dc, ds, dids, qo, ko, tokens, qh, kh, D, dtype, form, 8, 1, nullptr);
    ok = !err && std::memcmp(qo, rq.data(), nq * 2) == 0 && std::memcmp(ko, rk.data(), nk * 2) == 0;
    hipFree(dc);
    hipFree(ds);
  } else if (form == 3) {
    oracle_rope_freq(hq.data(), hk.data(), ids.data(), inv.data(), rq.data(), rk.data(), tokens, qh, kh, D, dtype);
    err = rope_launch_freq(q, k, dids, dinv, qo, ko, tokens, qh, kh, D, dtype, nullptr);
    ok = !err && std::memcmp(qo, rq.data(), nq * 2) == 0 && std::memcmp(ko, rk.data(), nk * 2) == 0;
  } else {
    const long long S = 3 * tokens;
    const size_t row = (size_t)kh * D;
    std::vector<int64_t> slots(tokens);
    for (long long t = 0; t < tokens; ++t) slots[t] = t % 4 == 3 ? -1 : S - 1 - 3 * t;  // distinct, in [0, S)
    std::vector<uint16_t> kc0((size_t)S * row), vc0((size_t)S * row);
    for (size_t i = 0; i < kc0.size(); ++i) {
      kc0[i] = (uint16_t)(0x1234 + i);
      vc0[i] = (uint16_t)(0x4321 + i);
    }
    uint16_t* v = dev_copy(hv);
    uint16_t* kc = dev_copy(kc0);
    uint16_t* vc = dev_copy(vc0);
    int64_t* ds = dev_copy(slots);
    oracle_rope_freq(hq.data(), hk.data(), ids.data(), inv.data(), rq.data(), rk.data(), tokens, qh, kh, D, dtype);
    std::vector<uint16_t> ekc = kc0, evc = vc0;
    for (long long t = 0; t < tokens; ++t)
      if (slots[t] >= 0) {
        std::memcpy(&ekc[(size_t)slots[t] * row], &rk[(size_t)t * row], row * 2);
        std::memcpy(&evc[(size_t)slots[t] * row], &hv[(size_t)t * row], row * 2);
      }
    err = rope_kv_launch(q, k, v, dids, dinv, qo, kc, vc, ds, tokens, qh, kh, D, dtype, nullptr);
    ok = !err && std::memcmp(qo, rq.data(), nq * 2) == 0 && std::memcmp(kc, ekc.data(), ekc.size() * 2) == 0 &&
         std::memcmp(vc, evc.data(), evc.size() * 2) == 0 && std::memcmp(k, hk.data(), nk * 2) == 0 &&
         std::memcmp(v, hv.data(), nk * 2) == 0;
    hipFree(v);
    hipFree(kc);
    hipFree(vc);
    hipFree(ds);
  }
  std::printf("tokens %lld heads %d/%d D %d dtype %d form %d inplace %d: %s (err %d)\n", tokens, qh, kh, D, dtype,
              form, inplace, ok ? "ALL OK" : "FAILED", err);
  return ok ? 0 : 1;
}
