// A CPU emulation of the HIP surface that csrc/topk.hip uses, for running the kernels' own source on the host (test
// infrastructure, never linked into the libraries):
//  - every thread of a workgroup is a cooperative fiber (makecontext for its entry, _setjmp/_longjmp to switch);
//  - every cross-lane operation (ballot, DPP, readlane, readfirstlane, shfl_up) is an exchange between two barriers of
//    the wave's live lanes, and __syncthreads a barrier of the block's live threads; lanes that have returned take no
//    part, as on the hardware. Lanes of one wave reaching a barrier from different source lines, or a schedule in
//    which no fiber can run, abort with a report;
//  - within a workgroup, every lane runs to its next exchange point in turn, or, with EMU_WAVE_AHEAD set, each wave
//    runs on until all of its lanes wait at a block barrier (waves ahead of one another between barriers);
//  - workgroups run one after another (shuffled on request), or, with EMU_CONCURRENT set, each on an OS thread of its
//    own, all at once (as co-resident workgroups that wait for one another need); __shared__ is a function-local
//    thread_local static, so each workgroup's thread has its own;
//  - device buffers lie between PROT_NONE pages (flush against the upper one, or against the lower one with
//    EMU_ALIGN_START set) and start filled with 0xA5, so an access outside a buffer faults at once;
//  - the atomics are sequentially consistent operations (fibers of one workgroup switch only at barriers), except
//    in the weak mode (EMU_WEAK set): there an agent-scope store (__hip_atomic_store) is held in its lane's queue of
//    pending stores and becomes visible to other workgroups late and out of order -- a pending store drains at random
//    at the lane's later atomic operations, ballots, sleeps and barriers (so a lane that keeps running sees its
//    stores complete in the end, as the hardware's do), all of the lane's drain at `s_waitcnt vmcnt(0)` (the wait
//    that orders them before a later arrival count), and what a lane left pending when it ended drains one store at a
//    time, now and then, while other lanes run, and wholly when the launch completes. A lane reads its own pending
//    stores (same-address order is kept); atomic read-modify-writes act on memory at once. With EMU_DROP_VMCNT set as
//    well, `s_waitcnt vmcnt(0)` drains nothing: the planted mistake that the weak mode must expose.
//  - hipMalloc calls are counted (emu::mallocs()), so a driver can show that a launch allocates nothing.
#pragma once
#include <sched.h>
#include <setjmp.h>
#include <sys/mman.h>
#include <ucontext.h>
#include <unistd.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <atomic>
#include <chrono>
#include <functional>
#include <map>
#include <mutex>
#include <random>
#include <thread>
#include <vector>

#define __global__
#define __device__
#define __host__
#define __forceinline__ inline
#define __launch_bounds__(...)
#define __shared__ static thread_local
#define __align__(n) __attribute__((aligned(n)))
#define EMU_ASM(...) emu::asm_hook(#__VA_ARGS__)

typedef int hipError_t;
enum { hipSuccess = 0, hipErrorInvalidValue = 1 };
typedef struct ihipStream_t* hipStream_t;
enum hipDeviceAttribute_t { hipDeviceAttributeMultiprocessorCount = 1 };

struct float2 {
  float x, y;
};
inline float2 make_float2(float a, float b) { return float2{a, b}; }
// Raw buffer resources: a base and a byte extent; a load returns zeros for the dwords at or past the extent.
struct __amdgpu_buffer_rsrc_t {
  const char* base;
  long long bytes;
};
inline __amdgpu_buffer_rsrc_t emu_make_buffer_rsrc(void* base, short, int bytes, int) {
  return __amdgpu_buffer_rsrc_t{static_cast<const char*>(base), (long long)(unsigned)bytes};
}
#define __builtin_amdgcn_make_buffer_rsrc(b, s, n, f) emu_make_buffer_rsrc((b), (s), (n), (f))
typedef unsigned emu_u32x4 __attribute__((ext_vector_type(4)));
inline emu_u32x4 emu_raw_buffer_load_b128(const __amdgpu_buffer_rsrc_t& r, int voff, int soff, int) {
  const long long off = (long long)(unsigned)voff + (long long)(unsigned)soff;
  emu_u32x4 v = {0u, 0u, 0u, 0u};
  for (int i = 0; i < 4; ++i) {
    if (off + 4 * i + 4 <= r.bytes) {
      unsigned u;
      std::memcpy(&u, r.base + off + 4 * i, 4);
      v[i] = u;
    }
  }
  return v;
}
#define __builtin_amdgcn_raw_buffer_load_b128(r, vo, so, aux) emu_raw_buffer_load_b128((r), (vo), (so), (aux))
struct alignas(16) float4 {
  float x, y, z, w;
};
inline float4 make_float4(float a, float b, float c, float d) { return float4{a, b, c, d}; }

struct dim3 {
  unsigned x, y, z;
  dim3(unsigned a = 1, unsigned b = 1, unsigned c = 1) : x(a), y(b), z(c) {}
};

namespace emu {
constexpr int kW = 64;
constexpr int kMaxThreads = 1024;
constexpr size_t kStack = 256 * 1024;

struct Idx { unsigned x, y, z; };

struct Bar {
  int arrived = 0;
  unsigned gen = 0;
  int line = -1;
};

struct Pending {
  void* p;
  uint64_t v;
  int size;
};

struct Fiber {
  std::vector<Pending> pending;  // the weak mode's stores not yet visible
  jmp_buf jb;
  ucontext_t uc;
  char* stack = nullptr;
  Idx tid;
  bool done = false, started = false;
  Bar* wait = nullptr;
  unsigned wait_gen = 0;
};

struct State {
  Fiber fib[kMaxThreads];
  int n = 0;
  Fiber* cur = nullptr;
  jmp_buf sched;
  ucontext_t sched_uc;
  Idx block_idx{0, 0, 0};
  dim3 grid, block;
  Bar wbar[kMaxThreads / kW], bbar;
  int wactive[kMaxThreads / kW], bactive = 0;
  uint64_t slots[kMaxThreads / kW][kW];
  std::function<void()> body;
  unsigned long long switches = 0, inactive_reads = 0;
  int shuffle_seed = -1;
  std::mt19937 rng{1};
  char* stacks = nullptr;  // the fibers' stacks, kStack each
};
// The calling OS thread's state (a workgroup's thread in concurrent mode takes one from a pool).
inline State*& tls_state() {
  static thread_local State* p = nullptr;
  return p;
}
inline State& S() {
  State*& p = tls_state();
  if (!p) p = new State;
  return *p;
}

inline const Idx& tid() { return S().cur->tid; }
inline int flat() { return (int)S().cur->tid.x; }
inline int wid() { return flat() / kW; }
inline int lid() { return flat() % kW; }

[[noreturn]] inline void fail(const char* what, int line) {
  std::fprintf(stderr, "EMU FAIL: %s (line %d) block (%u,%u) thread %d\n", what, line, S().block_idx.x,
               S().block_idx.y, S().cur ? flat() : -1);
  std::fflush(stderr);
  std::abort();
}

// ---- the weak mode ------------------------------------------------------------------------------------------------
inline bool weak() {
  static const bool w = std::getenv("EMU_WEAK") != nullptr;
  return w;
}
inline bool drop_vmcnt() {
  static const bool d = std::getenv("EMU_DROP_VMCNT") != nullptr;
  return d;
}
inline std::mutex& inflight_mu() {
  static std::mutex m;
  return m;
}
inline std::vector<Pending>& inflight() {  // stores of ended lanes, not yet visible
  static std::vector<Pending> q;
  return q;
}
inline void apply(const Pending& e) {
  if (e.size == 8) __atomic_store_n((uint64_t*)e.p, e.v, __ATOMIC_SEQ_CST);
  else if (e.size == 4) __atomic_store_n((uint32_t*)e.p, (uint32_t)e.v, __ATOMIC_SEQ_CST);
  else if (e.size == 2) __atomic_store_n((uint16_t*)e.p, (uint16_t)e.v, __ATOMIC_SEQ_CST);
  else __atomic_store_n((uint8_t*)e.p, (uint8_t)e.v, __ATOMIC_SEQ_CST);
}
inline void drain_all(std::vector<Pending>& q) {
  for (const Pending& e : q) apply(e);
  q.clear();
}
// Lets some pending stores (the lane's own, and some of ended lanes') become visible, out of order.
inline void maybe_drain() {
  State& s = S();
  if (!s.cur) return;
  std::vector<Pending>& q = s.cur->pending;
  for (size_t i = 0; i < q.size();) {
    if (s.rng() % 8 == 0) {
      apply(q[i]);
      q[i] = q.back();  // out of order, except that a lane keeps one entry per address (see store)
      q.pop_back();
    } else {
      ++i;
    }
  }
  if (s.rng() % 64 == 0) {  // now and then one store of an ended lane, picked at random
    std::lock_guard<std::mutex> lock(inflight_mu());
    std::vector<Pending>& g = inflight();
    if (!g.empty()) {
      const size_t i = s.rng() % g.size();
      apply(g[i]);
      g[i] = g.back();
      g.pop_back();
    }
  }
}
inline void asm_hook(const char* text) {
  if (!weak() || !S().cur) return;
  if (std::strstr(text, "vmcnt(0)") && !drop_vmcnt()) drain_all(S().cur->pending);
}
template <typename T>
inline Pending* own_pending(const T* p) {
  State& s = S();
  if (!s.cur) return nullptr;
  for (Pending& e : s.cur->pending)
    if (e.p == (const void*)p) return &e;
  return nullptr;
}
inline std::atomic<long long>& malloc_count() {
  static std::atomic<long long> n{0};
  return n;
}
inline long long mallocs() { return malloc_count().load(); }

inline void yield() {
  State& s = S();
  ++s.switches;
  if (!_setjmp(s.cur->jb)) _longjmp(s.sched, 1);
}

inline void arrive(Bar& b, int active, int line) {
  if (b.arrived == 0) b.line = line;
  else if (b.line != line) {
    std::fprintf(stderr, "EMU: barrier mismatch: line %d vs line %d\n", b.line, line);
    fail("lanes of one barrier at different sites", line);
  }
  if (++b.arrived == active) {
    b.arrived = 0;
    ++b.gen;
    return;
  }
  S().cur->wait = &b;
  S().cur->wait_gen = b.gen;
  yield();
}
inline void wave_sync(int line) { arrive(S().wbar[wid()], S().wactive[wid()], line); }
inline void block_sync(int line) {
  if (weak()) maybe_drain();
  arrive(S().bbar, S().bactive, line);
}

inline bool lane_done(int w, int l) { return S().fib[w * kW + l].done; }

inline uint64_t ballot(bool p, int line) {
  if (weak()) maybe_drain();  // a lane's stores complete while it runs, whatever it runs
  State& s = S();
  const int w = wid();
  s.slots[w][lid()] = p;
  wave_sync(line);
  uint64_t m = 0;
  for (int i = 0; i < kW; ++i)
    if (w * kW + i < s.n && !lane_done(w, i) && s.slots[w][i]) m |= 1ull << i;
  wave_sync(line);
  return m;
}
inline uint64_t read_from(uint64_t mine, int src, int line) {
  State& s = S();
  const int w = wid();
  s.slots[w][lid()] = mine;
  wave_sync(line);
  uint64_t r = 0;
  if (src < 0 || src >= kW || lane_done(w, src)) ++s.inactive_reads;
  else r = s.slots[w][src];
  wave_sync(line);
  return r;
}
inline int first_active(int w) {
  for (int i = 0; i < kW; ++i)
    if (!lane_done(w, i)) return i;
  return 0;
}
inline int readlane(int v, int lane, int line) { return (int)(uint32_t)read_from((uint32_t)v, lane, line); }
inline int readfirstlane(int v, int line) {
  // the first lane that is not done (every live lane takes part)
  State& s = S();
  const int w = wid();
  s.slots[w][lid()] = (uint32_t)v;
  wave_sync(line);
  const int r = (int)(uint32_t)s.slots[w][first_active(w)];
  wave_sync(line);
  return r;
}
// the lane that lane l reads under DPP control ctrl, or -1 where the source is out of range
inline int dpp_src(int l, int ctrl, int line) {
  if (ctrl > 0x110 && ctrl < 0x120) return (l & 15) >= ctrl - 0x110 ? l - (ctrl - 0x110) : -1;  // row_shr:n
  switch (ctrl) {
    case 0xB1: return l ^ 1;
    case 0x4E: return l ^ 2;
    case 0x141: return (l & ~7) | (7 - (l & 7));
    case 0x140: return (l & ~15) | (15 - (l & 15));
    default: fail("unsupported dpp control", line);
  }
}
inline int update_dpp(int old, int src, int ctrl, int rm, int bm, bool bc, int line) {
  if (rm != 0xF || bm != 0xF) fail("dpp masks", line);
  const int from = dpp_src(lid(), ctrl, line);
  const int r = (int)(uint32_t)read_from((uint32_t)src, from < 0 ? lid() : from, line);
  return from < 0 ? (bc ? 0 : old) : r;  // an out-of-range source writes 0 (bound_ctrl) or keeps old
}
inline unsigned mbcnt_lo(unsigned m, unsigned c) {
  const int l = lid();
  const uint64_t below = l >= 32 ? 0xffffffffull : ((1ull << l) - 1);
  return c + (unsigned)__builtin_popcountll((uint64_t)m & below);
}
inline unsigned mbcnt_hi(unsigned m, unsigned c) {
  const int l = lid() - 32;
  const uint64_t below = l <= 0 ? 0ull : ((1ull << l) - 1);
  return c + (unsigned)__builtin_popcountll((uint64_t)m & below);
}
template <typename T>
inline T shfl_up(T v, unsigned d, int width, int line) {
  static_assert(sizeof(T) <= 8, "");
  uint64_t u = 0;
  std::memcpy(&u, &v, sizeof(T));
  const int l = lid();
  const int src = (l % width) >= (int)d ? l - (int)d : l;
  u = read_from(u, src, line);
  T r;
  std::memcpy(&r, &u, sizeof(T));
  return r;
}

inline void trampoline() {
  State& s = S();
  s.body();
  Fiber* f = s.cur;
  if (!f->pending.empty()) {  // a lane that ends leaves its stores in flight
    std::lock_guard<std::mutex> lock(inflight_mu());
    for (const Pending& e : f->pending) inflight().push_back(e);
    f->pending.clear();
  }
  f->done = true;
  const int w = (int)f->tid.x / kW;
  --s.wactive[w];
  --s.bactive;
  // a lane that ends releases barriers its peers wait at (ended lanes take no part, as on the hardware)
  Bar& wb = s.wbar[w];
  if (wb.arrived > 0 && wb.arrived == s.wactive[w]) {
    wb.arrived = 0;
    ++wb.gen;
  }
  if (s.bbar.arrived > 0 && s.bbar.arrived == s.bactive) {
    s.bbar.arrived = 0;
    ++s.bbar.gen;
  }
  _longjmp(s.sched, 1);
}

inline void run_block() {
  State& s = S();
  for (int i = 0; i < s.n; ++i) {
    Fiber& f = s.fib[i];
    if (!f.stack) {
      // the stacks of a workgroup's fibers in one mapping (one mapping each would pass the process's mapping limit
      // with a few dozen 1024-thread workgroups at once), a guard page below the lowest
      if (!s.stacks) {
        char* base = (char*)mmap(nullptr, kMaxThreads * kStack + 4096, PROT_READ | PROT_WRITE,
                                 MAP_PRIVATE | MAP_ANONYMOUS | MAP_NORESERVE, -1, 0);
        if (base == MAP_FAILED) fail("stack mmap", 0);
        mprotect(base, 4096, PROT_NONE);
        s.stacks = base + 4096;
      }
      f.stack = s.stacks + (size_t)i * kStack;
    }
    f.done = false;
    f.started = false;
    f.wait = nullptr;
    f.tid = Idx{(unsigned)i, 0, 0};
    getcontext(&f.uc);
    f.uc.uc_stack.ss_sp = f.stack;
    f.uc.uc_stack.ss_size = kStack;
    f.uc.uc_link = nullptr;
    makecontext(&f.uc, (void (*)())trampoline, 0);
  }
  for (int w = 0; w < (s.n + kW - 1) / kW; ++w) {
    s.wactive[w] = (s.n - w * kW) < kW ? s.n - w * kW : kW;
    s.wbar[w] = Bar{};
  }
  s.bactive = s.n;
  s.bbar = Bar{};
  std::vector<int> order(s.n);
  for (int i = 0; i < s.n; ++i) order[i] = i;
  int remaining = s.n;
  // EMU_WAVE_AHEAD: a wave runs on (through its own cross-lane exchanges) until every one of its lanes waits at a
  // block barrier or has ended, before the next wave starts: waves run ahead of one another between block barriers,
  // as they may on the hardware, so a value one wave writes to __shared__ without a barrier is seen by the waves
  // after it. Without it, every lane runs to its next exchange point in turn, and all waves read before any writes.
  static const bool ahead = std::getenv("EMU_WAVE_AHEAD") != nullptr;
  auto run_one = [&](Fiber& f) {
    if (f.done) return false;
    if (f.wait && f.wait->gen == f.wait_gen) return false;
    f.wait = nullptr;
    s.cur = &f;
    if (!_setjmp(s.sched)) {
      if (!f.started) {
        f.started = true;
        swapcontext(&s.sched_uc, &f.uc);
      } else {
        _longjmp(f.jb, 1);
      }
    }
    if (f.done) --remaining;
    return true;
  };
  const int waves = (s.n + kW - 1) / kW;
  std::vector<int> worder(waves);
  for (int w = 0; w < waves; ++w) worder[w] = w;
  while (remaining) {
    bool progress = false;
    if (s.shuffle_seed >= 0) std::shuffle(order.begin(), order.end(), s.rng);
    if (ahead) {
      if (s.shuffle_seed >= 0) std::shuffle(worder.begin(), worder.end(), s.rng);
      for (int w : worder) {
        for (bool again = true; again;) {
          again = false;
          for (int oi = 0; oi < s.n; ++oi)
            if (order[oi] / kW == w && run_one(s.fib[order[oi]])) again = progress = true;
        }
      }
    }
    for (int oi = 0; oi < s.n && !ahead; ++oi)
      if (run_one(s.fib[order[oi]])) progress = true;
    if (!progress) {
      std::fprintf(stderr, "EMU DEADLOCK in block (%u,%u): %d lanes left\n", s.block_idx.x, s.block_idx.y, remaining);
      for (int w = 0; w < (s.n + kW - 1) / kW; ++w)
        std::fprintf(stderr, "  wave %d: active %d, wave barrier arrived %d at line %d\n", w, s.wactive[w],
                     s.wbar[w].arrived, s.wbar[w].line);
      std::fprintf(stderr, "  block barrier arrived %d of %d at line %d\n", s.bbar.arrived, s.bactive, s.bbar.line);
      std::abort();
    }
  }
  s.cur = nullptr;
}

inline bool concurrent() { return std::getenv("EMU_CONCURRENT") != nullptr; }
inline void sleep_a_while() {
  if (weak()) maybe_drain();
  if (concurrent()) sched_yield();
}
inline unsigned long long realtime_ticks() {
  // EMU_CLOCK_STOPPED: time never advances, so a bounded wait can only end by what it waits for
  static const bool stopped = std::getenv("EMU_CLOCK_STOPPED") != nullptr;
  if (stopped) return 0;
  return (unsigned long long)std::chrono::duration_cast<std::chrono::microseconds>(
             std::chrono::steady_clock::now().time_since_epoch()).count() / 10;
}

inline void launch(dim3 grid, dim3 block, std::function<void()> body) {
  State& s = S();
  if (block.y != 1 || block.z != 1 || block.x > (unsigned)kMaxThreads) fail("block shape", 0);
  s.grid = grid;
  s.block = block;
  s.n = (int)block.x;
  s.body = std::move(body);
  std::vector<Idx> blocks;
  for (unsigned z = 0; z < grid.z; ++z)
    for (unsigned y = 0; y < grid.y; ++y)
      for (unsigned x = 0; x < grid.x; ++x) blocks.push_back(Idx{x, y, z});
  if (s.shuffle_seed >= 0) std::shuffle(blocks.begin(), blocks.end(), s.rng);
  if (!concurrent()) {
    for (const Idx& b : blocks) {
      s.block_idx = b;
      run_block();
    }
    drain_all(inflight());  // the launch completes: every store is visible
    return;
  }
  // every workgroup on its own thread, with a state from the pool (kept for the next launch)
  static std::vector<State*> pool;
  while (pool.size() < blocks.size()) pool.push_back(new State);
  std::vector<std::thread> threads;
  for (size_t j = 0; j < blocks.size(); ++j) {
    State* w = pool[j];
    w->grid = grid;
    w->block = block;
    w->n = s.n;
    w->body = s.body;
    w->block_idx = blocks[j];
    w->shuffle_seed = s.shuffle_seed;
    if (s.shuffle_seed >= 0) w->rng.seed((unsigned)(s.shuffle_seed * 7919 + j));
    // EMU_STAGGER: workgroups start up to 400 ms apart (a workgroup's work takes tens of ms here), so that early ones
    // reach their waits long before late ones have published anything
    static const bool stagger = std::getenv("EMU_STAGGER") != nullptr;
    const int delay_ms = stagger ? (int)(j % 3) * 200 : 0;
    threads.emplace_back([w, delay_ms] {
      if (delay_ms) std::this_thread::sleep_for(std::chrono::milliseconds(delay_ms));
      tls_state() = w;
      run_block();
    });
  }
  for (std::thread& t : threads) t.join();
  drain_all(inflight());
}

// Device buffers end at a PROT_NONE page (an access past the end faults at once) and start after one; contents start
// as a fill pattern, not zeros (device memory is not cleared by an allocation).
struct Mapping {
  char* base;
  size_t len;
};
inline std::map<void*, Mapping>& maps() {
  static std::map<void*, Mapping> m;
  return m;
}
inline void* guarded_alloc(size_t n) {
  const size_t pg = 4096;
  const size_t body = (n + pg - 1) / pg * pg + pg;
  char* base = (char*)mmap(nullptr, body + 2 * pg, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS, -1, 0);
  if (base == MAP_FAILED) return nullptr;
  mprotect(base, pg, PROT_NONE);
  mprotect(base + pg + body, pg, PROT_NONE);
  char* p = std::getenv("EMU_ALIGN_START") ? base + pg : base + pg + body - ((n + 15) & ~(size_t)15);
  std::memset(base + pg, 0xA5, body);
  maps()[p] = Mapping{base, body + 2 * pg};
  return p;
}
inline void guarded_free(void* p) {
  auto it = maps().find(p);
  if (it == maps().end()) {
    std::fprintf(stderr, "EMU: free of an unknown pointer %p\n", p);
    std::abort();
  }
  munmap(it->second.base, it->second.len);
  maps().erase(it);
}
}  // namespace emu

#define threadIdx (emu::tid())
#define blockIdx (emu::S().block_idx)
#define gridDim (emu::S().grid)
#define blockDim (emu::S().block)
#define __syncthreads() emu::block_sync(__LINE__)
#define __ballot(p) emu::ballot((p), __LINE__)
#define __builtin_amdgcn_readlane(v, l) emu::readlane((int)(v), (int)(l), __LINE__)
#define __builtin_amdgcn_readfirstlane(v) emu::readfirstlane((int)(v), __LINE__)
#define __builtin_amdgcn_update_dpp(o, s, c, r, b, bc) \
  emu::update_dpp((int)(o), (int)(s), (c), (r), (b), (bc), __LINE__)
#define __builtin_amdgcn_mbcnt_lo(m, c) emu::mbcnt_lo((unsigned)(m), (unsigned)(c))
#define __builtin_amdgcn_mbcnt_hi(m, c) emu::mbcnt_hi((unsigned)(m), (unsigned)(c))
#define __builtin_amdgcn_wave_barrier() emu::wave_sync(__LINE__)
#define __builtin_amdgcn_s_sleep(n) emu::sleep_a_while()
// the 100 MHz real-time counter, slowed 1000-fold: fibers and OS threads advance far more slowly than waves, so a
// wait budget in ticks keeps its proportion to the work around it
#define __builtin_amdgcn_s_memrealtime() emu::realtime_ticks()
#define __shfl_up(v, d, w) emu::shfl_up((v), (unsigned)(d), (int)(w), __LINE__)

#define __HIP_MEMORY_SCOPE_AGENT 0
template <typename T>
inline T emu_atomic_load(const T* p) {
  if (emu::weak()) {
    emu::maybe_drain();
    if (emu::Pending* e = emu::own_pending(p)) {
      T v;
      std::memcpy(&v, &e->v, sizeof(T));
      return v;
    }
  }
  return __atomic_load_n(p, __ATOMIC_SEQ_CST);
}
template <typename T, typename U>
inline void emu_atomic_store(T* p, U v) {
  static_assert(sizeof(T) <= 8, "");
  const T t = (T)v;
  if (!emu::weak() || !emu::S().cur) {
    __atomic_store_n(p, t, __ATOMIC_SEQ_CST);
    return;
  }
  emu::maybe_drain();
  uint64_t bits = 0;
  std::memcpy(&bits, &t, sizeof(T));
  if (emu::Pending* e = emu::own_pending(p)) e->v = bits;  // the later store to an address replaces the earlier
  else emu::S().cur->pending.push_back(emu::Pending{(void*)p, bits, (int)sizeof(T)});
}
// A read-modify-write acts on memory at once, after the lane's own pending store to the same address.
template <typename T>
inline void emu_rmw_prepare(T* p) {
  if (!emu::weak()) return;
  emu::maybe_drain();
  std::vector<emu::Pending>& q = emu::S().cur->pending;
  for (size_t i = 0; i < q.size(); ++i)
    if (q[i].p == (void*)p) {
      emu::apply(q[i]);
      q.erase(q.begin() + (long)i);
      break;
    }
}
#define __hip_atomic_load(p, o, sc) emu_atomic_load((p))
#define __hip_atomic_store(p, v, o, sc) emu_atomic_store((p), (v))
template <typename T, typename U>
inline T emu_fetch_add(T* p, U v) {
  if (emu::S().cur) emu_rmw_prepare(p);
  return __atomic_fetch_add(p, (T)v, __ATOMIC_SEQ_CST);
}
#define __hip_atomic_fetch_add(p, v, o, sc) emu_fetch_add((p), (v))
template <typename T, typename U>
inline T emu_fetch_max(T* p, U v) {
  if (emu::S().cur) emu_rmw_prepare(p);
  T old = __atomic_load_n(p, __ATOMIC_SEQ_CST);
  while ((T)v > old && !__atomic_compare_exchange_n(p, &old, (T)v, false, __ATOMIC_SEQ_CST, __ATOMIC_SEQ_CST)) {
  }
  return old;
}
#define __hip_atomic_fetch_max(p, v, o, sc) emu_fetch_max((p), (v))
template <typename T, typename U>
inline T atomicAdd(T* p, U v) {
  return __atomic_fetch_add(p, (T)v, __ATOMIC_SEQ_CST);  // LDS atomics (workgroup-local)
}

inline int __popcll(unsigned long long v) { return __builtin_popcountll(v); }
#define __builtin_amdgcn_exp2f(x) exp2f(x)
inline int __clzll(long long v) { return v ? __builtin_clzll((unsigned long long)v) : 64; }
inline int __clz(int v) { return v ? __builtin_clz((unsigned)v) : 32; }
inline float __uint_as_float(unsigned u) { return __builtin_bit_cast(float, u); }
inline unsigned __float_as_uint(float f) { return __builtin_bit_cast(unsigned, f); }

inline hipError_t hipGetDevice(int* d) {
  *d = 0;
  return hipSuccess;
}
inline hipError_t hipGetLastError() { return hipSuccess; }
// a device variable's address: on the host of this emulation the variable itself
#define HIP_SYMBOL(x) (&(x))
inline hipError_t hipGetSymbolAddress(void** p, const void* symbol) {
  *p = const_cast<void*>(symbol);
  return hipSuccess;
}
inline hipError_t hipDeviceGetAttribute(int* v, hipDeviceAttribute_t, int) {
  *v = 256;
  return hipSuccess;
}
template <typename F>
inline hipError_t hipOccupancyMaxActiveBlocksPerMultiprocessor(int* n, F, int, size_t) {
  *n = 4;
  return hipSuccess;
}
inline hipError_t hipMalloc(void** p, size_t n) {
  ++emu::malloc_count();
  *p = emu::guarded_alloc(n);
  return *p ? hipSuccess : hipErrorInvalidValue;
}
inline hipError_t hipFree(void* p) {
  if (p) emu::guarded_free(p);
  return hipSuccess;
}
inline hipError_t hipMemsetAsync(void* p, int v, size_t n, hipStream_t) {
  std::memset(p, v, n);
  return hipSuccess;
}
// Graph capture: between emu::capture_begin() and emu::capture_end() launches are recorded, not run, and
// hipStreamIsCapturing reports an active capture; emu::replay() runs a recorded sequence again (kernel arguments as
// they were captured, like a HIP graph's kernel nodes).
namespace emu {
typedef std::vector<std::function<void()>> Graph;
inline Graph*& recording() {
  static Graph* g = nullptr;
  return g;
}
inline void capture_begin(Graph& g) {
  g.clear();
  recording() = &g;
}
inline void capture_end() { recording() = nullptr; }
inline void replay(const Graph& g) {
  for (const auto& node : g) node();
}
inline void launch_or_record(dim3 grid, dim3 block, std::function<void()> body) {
  if (recording()) recording()->push_back([grid, block, body] { launch(grid, block, body); });
  else launch(grid, block, std::move(body));
}
}  // namespace emu
enum hipStreamCaptureStatus { hipStreamCaptureStatusNone = 0, hipStreamCaptureStatusActive = 1 };
inline hipError_t hipStreamIsCapturing(hipStream_t, hipStreamCaptureStatus* st) {
  *st = emu::recording() ? hipStreamCaptureStatusActive : hipStreamCaptureStatusNone;
  return hipSuccess;
}
// arguments are captured by value: a recorded launch runs after the launching function has returned
#define hipLaunchKernelGGL(K, G, B, SH, ST, ...) emu::launch_or_record(dim3(G), dim3(B), [=]() { K(__VA_ARGS__); })
