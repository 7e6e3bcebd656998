// PyTorch-ROCm operators over the four op libraries' C entry points: torch.ops.ckopt.*, for callers that hold torch
// tensors (eager code, torch.compile graphs through the Meta shape functions below). Each operator checks its tensors,
// allocates its outputs with torch on the input's device, and calls the same `launch` (or extension entry) that the
// reference's ctypes wrappers bind (softmax/kernel.cu:520, rmsnorm/kernel.cu:132 via rmsnorm/candidate.py:25-28,
// rope/kernel.cu:201 via rope/candidate.py:27-29, topk/kernel.cu:520-570 via topk/candidate.py:30-35) on torch's
// current HIP stream. The op libraries are opened with dlopen from build/<op>/libkernel.so beside this library's
// build/torch/ directory (each exports a C `launch`, so they cannot be linked into one object); a missing library is
// an error at the first call, never a fallback. The libraries' declarations are include/{softmax,rmsnorm,rope,topk}.h.
#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <dlfcn.h>
#include <hip/hip_runtime_api.h>
#include <torch/library.h>

#include <algorithm>
#include <cstdint>
#include <mutex>
#include <string>
#include <tuple>
#include <unordered_map>
#include <utility>

namespace {

// The build/ directory: this library is build/torch/libckopt_torch.so.
std::string build_dir() {
  Dl_info info;
  if (dladdr(reinterpret_cast<void*>(&build_dir), &info) && info.dli_fname) {
    std::string p(info.dli_fname);
    for (int up = 0; up < 2; ++up) {
      const auto slash = p.rfind('/');
      p = slash == std::string::npos ? std::string(".") : p.substr(0, slash);
    }
    return p;
  }
  return ".";
}

void* op_library(const std::string& op) {
  static std::mutex mu;
  static std::unordered_map<std::string, void*> open;
  std::lock_guard<std::mutex> lock(mu);
  auto it = open.find(op);
  if (it != open.end()) return it->second;
  const std::string path = build_dir() + "/" + op + "/libkernel.so";
  void* h = dlopen(path.c_str(), RTLD_NOW | RTLD_LOCAL);
  TORCH_CHECK(h != nullptr, "ckopt: cannot open ", path, " (build it with make_libs.py): ", dlerror());
  open[op] = h;
  return h;
}

template <typename F>
F entry(const char* op, const char* name) {
  void* f = dlsym(op_library(op), name);
  TORCH_CHECK(f != nullptr, "ckopt: build/", op, "/libkernel.so exports no ", name);
  return reinterpret_cast<F>(f);
}

// include/softmax.h, include/rmsnorm.h, include/rope.h, include/topk.h
using SoftmaxLaunch = int (*)(const void*, void*, long long, long long, int, int, int, hipStream_t);
using RmsLaunch = int (*)(const void*, void*, long long, int, int, float, int, hipStream_t);
using RmsWeighted = int (*)(const void*, const void*, void*, long long, int, int, float, int, hipStream_t);
using RmsAdd = int (*)(const void*, const void*, const void*, void*, void*, long long, int, int, float, int,
                       hipStream_t);
using RopeLaunch = int (*)(const void*, const void*, const void*, const void*, const void*, void*, void*, long long,
                           int, int, int, int, int, int, int, hipStream_t);
using RopeFreq = int (*)(const void*, const void*, const void*, const float*, void*, void*, long long, int, int, int,
                         int, hipStream_t);
using RopeKv = int (*)(const void*, const void*, const void*, const void*, const float*, void*, void*, void*,
                       const void*, long long, int, int, int, int, hipStream_t);
using TopkPlan = long long (*)(long long, long long, int, int, int, int);
using TopkLaunch = int (*)(const void*, void*, void*, void*, void*, long long, long long, int, int, int, int,
                           long long, hipStream_t);
using TopkLaunchSample = int (*)(const void*, void*, void*, void*, void*, long long, long long, int, int, int, int,
                                 long long, const float*, void*, float, float, hipStream_t);
using TopkSample = int (*)(const void*, const void*, const float*, void*, long long, int, int, float, float,
                           hipStream_t);

hipStream_t current_stream(const at::Tensor& t) { return c10::hip::getCurrentHIPStream(t.device().index()).stream(); }

void launched(int err, const char* what) {
  TORCH_CHECK(err != -1, "ckopt::", what, ": the kernel library rejected the arguments");
  TORCH_CHECK(err == 0, "ckopt::", what, ": kernel launch failed: HIP error ", err);
}

void on_gpu(const at::Tensor& t, const char* what) {
  TORCH_CHECK(t.is_cuda(), "ckopt::", what, ": tensors must be on the GPU, got ", t.device());
}

void same_device(const at::Tensor& a, const at::Tensor& b, const char* what) {
  TORCH_CHECK(a.device() == b.device(), "ckopt::", what, ": tensors on ", a.device(), " and ", b.device());
}

int norm_code(const at::Tensor& x, const char* what) {
  TORCH_CHECK(x.scalar_type() == at::kBFloat16 || x.scalar_type() == at::kHalf, "ckopt::", what,
              ": bf16 or fp16 tensors, got ", x.scalar_type());
  return x.scalar_type() == at::kBFloat16 ? 1 : 2;
}

// ---- softmax (softmax/kernel.cu:520) --------------------------------------------------------------------------------

at::Tensor softmax_gpu(const at::Tensor& x_in) {
  on_gpu(x_in, "softmax");
  TORCH_CHECK(x_in.scalar_type() == at::kFloat || x_in.scalar_type() == at::kBFloat16,
              "ckopt::softmax: fp32 or bf16, got ", x_in.scalar_type());
  TORCH_CHECK(x_in.dim() >= 1, "ckopt::softmax: at least one dimension");
  c10::DeviceGuard guard(x_in.device());
  const at::Tensor x = x_in.contiguous();
  at::Tensor y = at::empty_like(x);
  const long long cols = x.size(-1), rows = cols ? x.numel() / cols : 0;
  static const auto fn = entry<SoftmaxLaunch>("softmax", "launch");
  launched(fn(x.data_ptr(), y.data_ptr(), rows, cols, x.scalar_type() == at::kFloat ? 0 : 1, 256, 1024,
              current_stream(x)),
           "softmax");
  return y;
}

// ---- RMSNorm (rmsnorm/kernel.cu:132; the weighted and fused-residual extensions) -----------------------------------

void rms_checks(const at::Tensor& x, const c10::optional<at::Tensor>& w, const char* what) {
  on_gpu(x, what);
  norm_code(x, what);
  TORCH_CHECK(x.dim() == 2 && x.size(1) >= 1, "ckopt::", what, ": x is [rows, cols], got ", x.sizes());
  if (w) {
    TORCH_CHECK(w->scalar_type() == x.scalar_type() && w->dim() == 1 && w->size(0) == x.size(1), "ckopt::", what,
                ": weight is [cols] of x's dtype");
    same_device(x, *w, what);
  }
}

at::Tensor rmsnorm_gpu(const at::Tensor& x_in, const c10::optional<at::Tensor>& weight, double eps) {
  rms_checks(x_in, weight, "rmsnorm");
  c10::DeviceGuard guard(x_in.device());
  const at::Tensor x = x_in.contiguous();
  at::Tensor y = at::empty_like(x);
  const int code = norm_code(x, "rmsnorm");
  if (weight) {
    const at::Tensor w = weight->contiguous();
    static const auto fn = entry<RmsWeighted>("rmsnorm", "rmsnorm_launch_weighted");
    launched(fn(x.data_ptr(), w.data_ptr(), y.data_ptr(), x.size(0), (int)x.size(1), code, (float)eps, 256,
                current_stream(x)),
             "rmsnorm");
  } else {
    static const auto fn = entry<RmsLaunch>("rmsnorm", "launch");
    launched(fn(x.data_ptr(), y.data_ptr(), x.size(0), (int)x.size(1), code, (float)eps, 256, current_stream(x)),
             "rmsnorm");
  }
  return y;
}

// h = x + residual written to h_out, y = rmsnorm(h) [* weight]
void rmsnorm_add_into(const at::Tensor& x, const at::Tensor& r, const c10::optional<at::Tensor>& weight, double eps,
                      at::Tensor& y, at::Tensor& h_out) {
  const int code = norm_code(x, "rmsnorm_add");
  at::Tensor w;
  if (weight) w = weight->contiguous();
  static const auto fn = entry<RmsAdd>("rmsnorm", "rmsnorm_add_launch");
  launched(fn(x.data_ptr(), r.data_ptr(), weight ? w.data_ptr() : nullptr, y.data_ptr(), h_out.data_ptr(), x.size(0),
              (int)x.size(1), code, (float)eps, 256, current_stream(x)),
           "rmsnorm_add");
}

void residual_checks(const at::Tensor& x, const at::Tensor& r) {
  on_gpu(r, "rmsnorm_add");
  TORCH_CHECK(r.scalar_type() == x.scalar_type() && r.sizes() == x.sizes(), "ckopt::rmsnorm_add: residual is x's "
              "dtype and shape");
  same_device(x, r, "rmsnorm_add");
}

std::tuple<at::Tensor, at::Tensor> rmsnorm_add_gpu(const at::Tensor& x_in, const at::Tensor& r_in,
                                                   const c10::optional<at::Tensor>& weight, double eps) {
  rms_checks(x_in, weight, "rmsnorm_add");
  residual_checks(x_in, r_in);
  c10::DeviceGuard guard(x_in.device());
  const at::Tensor x = x_in.contiguous(), r = r_in.contiguous();
  at::Tensor y = at::empty_like(x), h = at::empty_like(x);
  rmsnorm_add_into(x, r, weight, eps, y, h);
  return {y, h};
}

at::Tensor rmsnorm_add_inplace_gpu(const at::Tensor& x_in, at::Tensor& residual,
                                   const c10::optional<at::Tensor>& weight, double eps) {
  rms_checks(x_in, weight, "rmsnorm_add_");
  residual_checks(x_in, residual);
  TORCH_CHECK(residual.is_contiguous(), "ckopt::rmsnorm_add_: the residual is overwritten in place and must be "
              "contiguous");
  c10::DeviceGuard guard(x_in.device());
  const at::Tensor x = x_in.contiguous();
  at::Tensor y = at::empty_like(x);
  rmsnorm_add_into(x, residual, weight, eps, y, residual);
  return y;
}

// ---- RoPE (rope/kernel.cu:201; the on-the-fly and KV-cache extensions) ---------------------------------------------

void rope_checks(const at::Tensor& q, const at::Tensor& k, const at::Tensor& ids, const char* what) {
  on_gpu(q, what);
  norm_code(q, what);
  TORCH_CHECK(k.scalar_type() == q.scalar_type(), "ckopt::", what, ": q and k of one dtype");
  TORCH_CHECK(q.dim() == 4 && k.dim() == 4 && ids.dim() == 2 && ids.scalar_type() == at::kLong, "ckopt::", what,
              ": q [B, S, Hq, D], k [B, S, Hk, D], position_ids int64 [B, S]");
  TORCH_CHECK(q.size(0) == ids.size(0) && q.size(1) == ids.size(1) && k.size(0) == ids.size(0) &&
                  k.size(1) == ids.size(1) && q.size(3) == k.size(3) && q.size(3) % 2 == 0,
              "ckopt::", what, ": shapes q ", q.sizes(), ", k ", k.sizes(), ", position_ids ", ids.sizes());
  same_device(q, k, what);
  same_device(q, ids, what);
}

void inv_freq_checks(const at::Tensor& q, const at::Tensor& inv_freq, const char* what) {
  TORCH_CHECK(inv_freq.scalar_type() == at::kFloat && inv_freq.dim() == 1 && inv_freq.size(0) == q.size(3) / 2,
              "ckopt::", what, ": inv_freq is fp32 [D / 2]");
  same_device(q, inv_freq, what);
}

std::tuple<at::Tensor, at::Tensor> rope_gpu(const at::Tensor& q_in, const at::Tensor& k_in, const at::Tensor& cos_in,
                                            const at::Tensor& sin_in, const at::Tensor& ids_in) {
  rope_checks(q_in, k_in, ids_in, "rope");
  TORCH_CHECK((cos_in.scalar_type() == at::kFloat || cos_in.scalar_type() == at::kBFloat16 ||
               cos_in.scalar_type() == at::kHalf) &&
                  sin_in.scalar_type() == cos_in.scalar_type() && cos_in.dim() == 2 &&
                  sin_in.sizes() == cos_in.sizes() && cos_in.size(1) == q_in.size(3),
              "ckopt::rope: cos and sin are [P, D] in fp32, bf16 or fp16");
  same_device(q_in, cos_in, "rope");
  same_device(q_in, sin_in, "rope");
  c10::DeviceGuard guard(q_in.device());
  const at::Tensor q = q_in.contiguous(), k = k_in.contiguous(), ids = ids_in.contiguous();
  const at::Tensor cs = cos_in.contiguous(), sn = sin_in.contiguous();
  at::Tensor qo = at::empty_like(q), ko = at::empty_like(k);
  const int cache = cs.scalar_type() == at::kFloat ? 0 : cs.scalar_type() == at::kBFloat16 ? 1 : 2;
  static const auto fn = entry<RopeLaunch>("rope", "launch");
  launched(fn(q.data_ptr(), k.data_ptr(), cs.data_ptr(), sn.data_ptr(), ids.data_ptr(), qo.data_ptr(), ko.data_ptr(),
              q.size(0) * q.size(1), (int)q.size(2), (int)k.size(2), (int)q.size(3), norm_code(q, "rope"), cache, 40,
              1, current_stream(q)),
           "rope");
  return {qo, ko};
}

void rope_inplace_gpu(at::Tensor& q, at::Tensor& k, const at::Tensor& ids_in, const at::Tensor& inv_freq_in) {
  rope_checks(q, k, ids_in, "rope_");
  inv_freq_checks(q, inv_freq_in, "rope_");
  TORCH_CHECK(q.is_contiguous() && k.is_contiguous(), "ckopt::rope_: q and k are rotated in place and must be "
              "contiguous");
  c10::DeviceGuard guard(q.device());
  const at::Tensor ids = ids_in.contiguous(), inv = inv_freq_in.contiguous();
  static const auto fn = entry<RopeFreq>("rope", "rope_launch_freq");
  launched(fn(q.data_ptr(), k.data_ptr(), ids.data_ptr(), inv.data_ptr<float>(), q.data_ptr(), k.data_ptr(),
              q.size(0) * q.size(1), (int)q.size(2), (int)k.size(2), (int)q.size(3), norm_code(q, "rope_"),
              current_stream(q)),
           "rope_");
}

void rope_kv_inplace_gpu(at::Tensor& q, const at::Tensor& k_in, const at::Tensor& v_in, const at::Tensor& ids_in,
                         const at::Tensor& inv_freq_in, at::Tensor& k_cache, at::Tensor& v_cache,
                         const at::Tensor& slots_in) {
  rope_checks(q, k_in, ids_in, "rope_kv_");
  inv_freq_checks(q, inv_freq_in, "rope_kv_");
  TORCH_CHECK(q.is_contiguous(), "ckopt::rope_kv_: q is rotated in place and must be contiguous");
  TORCH_CHECK(v_in.scalar_type() == q.scalar_type() && v_in.sizes() == k_in.sizes(), "ckopt::rope_kv_: v is k's "
              "dtype and shape");
  for (const at::Tensor* c : {&k_cache, &v_cache}) {
    TORCH_CHECK(c->scalar_type() == q.scalar_type() && c->dim() == 3 && c->size(1) == k_in.size(2) &&
                    c->size(2) == k_in.size(3) && c->is_contiguous() && c->sizes() == k_cache.sizes(),
                "ckopt::rope_kv_: caches are contiguous [slots, Hk, D] of q's dtype");
    same_device(q, *c, "rope_kv_");
  }
  TORCH_CHECK(slots_in.scalar_type() == at::kLong && slots_in.sizes() == ids_in.sizes(), "ckopt::rope_kv_: "
              "slot_mapping is int64 [B, S]");
  same_device(q, v_in, "rope_kv_");
  same_device(q, slots_in, "rope_kv_");
  c10::DeviceGuard guard(q.device());
  const at::Tensor k = k_in.contiguous(), v = v_in.contiguous(), ids = ids_in.contiguous();
  const at::Tensor inv = inv_freq_in.contiguous(), slots = slots_in.contiguous();
  static const auto fn = entry<RopeKv>("rope", "rope_kv_launch");
  launched(fn(q.data_ptr(), k.data_ptr(), v.data_ptr(), ids.data_ptr(), inv.data_ptr<float>(), q.data_ptr(),
              k_cache.data_ptr(), v_cache.data_ptr(), slots.data_ptr(), q.size(0) * q.size(1), (int)q.size(2),
              (int)k.size(2), (int)q.size(3), norm_code(q, "rope_kv_"), current_stream(q)),
           "rope_kv_");
}

// ---- top-k (topk/kernel.cu:520-570) and the sampling extensions -----------------------------------------------------

// The caller's side of the top-k launch protocol, kept per (device, stream): a zeroed int32 counter array (at least
// 4096, as the reference's wrapper sizes it) and the plan and workspace of the most recent shape. A split row's
// chunks count their arrivals on counters[row] and hand their lists over in work, so two launches in flight at once
// must not share them: launches on one stream are ordered, and each stream has its own pair. The buffers are
// allocated while their stream is current and used only on it, so the caching allocator's stream-ordered reuse covers
// them (a buffer replaced by a larger one is freed behind the launches already queued on that stream).
struct TopkState {
  at::Tensor counters;
  std::tuple<long long, long long, int, int> shape{-1, -1, -1, -1};
  long long chunk = 0;
  at::Tensor work;
};

struct TopkLaunchArgs {
  long long chunk;
  void* work;
  void* counters;
  hipStream_t stream;
};

struct TopkKeyHash {
  size_t operator()(const std::pair<int, uintptr_t>& k) const {
    return std::hash<uintptr_t>()(k.second) * 31u + (size_t)k.first;
  }
};

TopkLaunchArgs topk_plan(const at::Tensor& x, int k) {
  static std::mutex mu;
  static std::unordered_map<std::pair<int, uintptr_t>, TopkState, TopkKeyHash> per_stream;
  std::lock_guard<std::mutex> lock(mu);
  const long long rows = x.size(0), cols = x.size(1);
  const int dtype = x.scalar_type() == at::kFloat ? 0 : 1;
  const hipStream_t stream = current_stream(x);
  TopkState& st = per_stream[{(int)x.device().index(), reinterpret_cast<uintptr_t>(stream)}];
  if (!st.counters.defined() || st.counters.numel() < rows)
    st.counters = at::zeros({std::max<long long>(rows, 4096)}, x.options().dtype(at::kInt));
  const auto shape = std::make_tuple(rows, cols, dtype, k);
  if (st.shape != shape) {
    static const auto plan = entry<TopkPlan>("topk", "plan");
    // k > 64 asks for chunks of at least 16k columns (a useful bound per chunk, fewer lists to merge)
    st.chunk = plan(rows, cols, dtype, 256, 4, k > 64 ? std::max(2048, 16 * k) : 2048);
    const long long nchunks = (cols + st.chunk - 1) / st.chunk;
    st.work = at::empty({nchunks > 1 ? rows * nchunks * k : 1}, x.options().dtype(at::kLong));
    st.shape = shape;
  }
  return {st.chunk, st.work.data_ptr(), st.counters.data_ptr(), stream};
}

void topk_checks(const at::Tensor& x, int64_t k, const char* what) {
  on_gpu(x, what);
  TORCH_CHECK(x.scalar_type() == at::kFloat || x.scalar_type() == at::kBFloat16, "ckopt::", what,
              ": fp32 or bf16, got ", x.scalar_type());
  TORCH_CHECK(x.dim() == 2 && k >= 1 && k <= 1024 && x.size(1) >= k, "ckopt::", what,
              ": x is [rows, cols] with cols >= k and 1 <= k <= 1024, got ", x.sizes(), " and k = ", k);
}

std::tuple<at::Tensor, at::Tensor> topk_gpu(const at::Tensor& x_in, int64_t k) {
  topk_checks(x_in, k, "topk");
  c10::DeviceGuard guard(x_in.device());
  const at::Tensor x = x_in.contiguous();
  at::Tensor values = at::empty({x.size(0), k}, x.options());
  at::Tensor indices = at::empty({x.size(0), k}, x.options().dtype(at::kLong));
  const TopkLaunchArgs a = topk_plan(x, (int)k);
  static const auto fn = entry<TopkLaunch>("topk", "launch");
  launched(fn(x.data_ptr(), values.data_ptr(), indices.data_ptr(), a.work, a.counters, x.size(0), x.size(1), (int)k,
              x.scalar_type() == at::kFloat ? 0 : 1, 256, 4, a.chunk, a.stream),
           "topk");
  return {values, indices};
}

void uniform_checks(const at::Tensor& like, const at::Tensor& u, const char* what) {
  TORCH_CHECK(u.scalar_type() == at::kFloat && u.dim() == 1 && u.size(0) == like.size(0), "ckopt::", what,
              ": uniforms are fp32 [rows]");
  same_device(like, u, what);
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> topk_and_sample_gpu(const at::Tensor& x_in, int64_t k,
                                                                   const at::Tensor& u_in, double temperature,
                                                                   double top_p) {
  topk_checks(x_in, k, "topk_and_sample");
  uniform_checks(x_in, u_in, "topk_and_sample");
  c10::DeviceGuard guard(x_in.device());
  const at::Tensor x = x_in.contiguous(), u = u_in.contiguous();
  at::Tensor values = at::empty({x.size(0), k}, x.options());
  at::Tensor indices = at::empty({x.size(0), k}, x.options().dtype(at::kLong));
  at::Tensor drawn = at::empty({x.size(0)}, x.options().dtype(at::kLong));
  const TopkLaunchArgs a = topk_plan(x, (int)k);
  static const auto fn = entry<TopkLaunchSample>("topk", "topk_launch_sample");
  launched(fn(x.data_ptr(), values.data_ptr(), indices.data_ptr(), a.work, a.counters, x.size(0), x.size(1), (int)k,
              x.scalar_type() == at::kFloat ? 0 : 1, 256, 4, a.chunk, u.data_ptr<float>(), drawn.data_ptr(),
              (float)temperature, (float)top_p, a.stream),
           "topk_and_sample");
  return {values, indices, drawn};
}

at::Tensor topk_sample_gpu(const at::Tensor& values_in, const at::Tensor& indices_in, const at::Tensor& u_in,
                           double temperature, double top_p) {
  on_gpu(values_in, "topk_sample");
  TORCH_CHECK((values_in.scalar_type() == at::kFloat || values_in.scalar_type() == at::kBFloat16) &&
                  values_in.dim() == 2 && values_in.size(1) >= 1 && values_in.size(1) <= 1024 &&
                  indices_in.scalar_type() == at::kLong && indices_in.sizes() == values_in.sizes(),
              "ckopt::topk_sample: values [rows, k] (fp32/bf16, k <= 1024) and int64 indices of that shape");
  uniform_checks(values_in, u_in, "topk_sample");
  same_device(values_in, indices_in, "topk_sample");
  c10::DeviceGuard guard(values_in.device());
  const at::Tensor v = values_in.contiguous(), i = indices_in.contiguous(), u = u_in.contiguous();
  at::Tensor out = at::empty({v.size(0)}, v.options().dtype(at::kLong));
  static const auto fn = entry<TopkSample>("topk", "topk_sample_launch");
  launched(fn(v.data_ptr(), i.data_ptr(), u.data_ptr<float>(), out.data_ptr(), v.size(0), (int)v.size(1),
              v.scalar_type() == at::kFloat ? 0 : 1, (float)temperature, (float)top_p, current_stream(v)),
           "topk_sample");
  return out;
}

// ---- shapes without data (Meta), for tracing ------------------------------------------------------------------------

at::Tensor softmax_meta(const at::Tensor& x) { return at::empty_like(x); }
at::Tensor rmsnorm_meta(const at::Tensor& x, const c10::optional<at::Tensor>&, double) { return at::empty_like(x); }
std::tuple<at::Tensor, at::Tensor> rmsnorm_add_meta(const at::Tensor& x, const at::Tensor&,
                                                    const c10::optional<at::Tensor>&, double) {
  return {at::empty_like(x), at::empty_like(x)};
}
at::Tensor rmsnorm_add_inplace_meta(const at::Tensor& x, at::Tensor&, const c10::optional<at::Tensor>&, double) {
  return at::empty_like(x);
}
std::tuple<at::Tensor, at::Tensor> rope_meta(const at::Tensor& q, const at::Tensor& k, const at::Tensor&,
                                             const at::Tensor&, const at::Tensor&) {
  return {at::empty_like(q), at::empty_like(k)};
}
void rope_inplace_meta(at::Tensor&, at::Tensor&, const at::Tensor&, const at::Tensor&) {}
void rope_kv_inplace_meta(at::Tensor&, const at::Tensor&, const at::Tensor&, const at::Tensor&, const at::Tensor&,
                          at::Tensor&, at::Tensor&, const at::Tensor&) {}
std::tuple<at::Tensor, at::Tensor> topk_meta(const at::Tensor& x, int64_t k) {
  return {at::empty({x.size(0), k}, x.options()), at::empty({x.size(0), k}, x.options().dtype(at::kLong))};
}
std::tuple<at::Tensor, at::Tensor, at::Tensor> topk_and_sample_meta(const at::Tensor& x, int64_t k, const at::Tensor&,
                                                                    double, double) {
  return {at::empty({x.size(0), k}, x.options()), at::empty({x.size(0), k}, x.options().dtype(at::kLong)),
          at::empty({x.size(0)}, x.options().dtype(at::kLong))};
}
at::Tensor topk_sample_meta(const at::Tensor& v, const at::Tensor&, const at::Tensor&, double, double) {
  return at::empty({v.size(0)}, v.options().dtype(at::kLong));
}

}  // namespace

TORCH_LIBRARY(ckopt, m) {
  m.def("softmax(Tensor x) -> Tensor");
  m.def("rmsnorm(Tensor x, Tensor? weight=None, float eps=1e-06) -> Tensor");
  m.def("rmsnorm_add(Tensor x, Tensor residual, Tensor? weight=None, float eps=1e-06) -> (Tensor, Tensor)");
  m.def("rmsnorm_add_(Tensor x, Tensor(a!) residual, Tensor? weight=None, float eps=1e-06) -> Tensor");
  m.def("rope(Tensor q, Tensor k, Tensor cos, Tensor sin, Tensor position_ids) -> (Tensor, Tensor)");
  m.def("rope_(Tensor(a!) q, Tensor(b!) k, Tensor position_ids, Tensor inv_freq) -> ()");
  m.def("rope_kv_(Tensor(a!) q, Tensor k, Tensor v, Tensor position_ids, Tensor inv_freq, Tensor(b!) k_cache, "
        "Tensor(c!) v_cache, Tensor slot_mapping) -> ()");
  m.def("topk(Tensor x, int k=50) -> (Tensor, Tensor)");
  m.def("topk_and_sample(Tensor x, int k, Tensor uniforms, float temperature=1.0, float top_p=1.0) -> "
        "(Tensor, Tensor, Tensor)");
  m.def("topk_sample(Tensor values, Tensor indices, Tensor uniforms, float temperature=1.0, float top_p=1.0) -> "
        "Tensor");
}

TORCH_LIBRARY_IMPL(ckopt, CUDA, m) {
  m.impl("softmax", &softmax_gpu);
  m.impl("rmsnorm", &rmsnorm_gpu);
  m.impl("rmsnorm_add", &rmsnorm_add_gpu);
  m.impl("rmsnorm_add_", &rmsnorm_add_inplace_gpu);
  m.impl("rope", &rope_gpu);
  m.impl("rope_", &rope_inplace_gpu);
  m.impl("rope_kv_", &rope_kv_inplace_gpu);
  m.impl("topk", &topk_gpu);
  m.impl("topk_and_sample", &topk_and_sample_gpu);
  m.impl("topk_sample", &topk_sample_gpu);
}

TORCH_LIBRARY_IMPL(ckopt, Meta, m) {
  m.impl("softmax", &softmax_meta);
  m.impl("rmsnorm", &rmsnorm_meta);
  m.impl("rmsnorm_add", &rmsnorm_add_meta);
  m.impl("rmsnorm_add_", &rmsnorm_add_inplace_meta);
  m.impl("rope", &rope_meta);
  m.impl("rope_", &rope_inplace_meta);
  m.impl("rope_kv_", &rope_kv_inplace_meta);
  m.impl("topk", &topk_meta);
  m.impl("topk_and_sample", &topk_and_sample_meta);
  m.impl("topk_sample", &topk_sample_meta);
}
