"""Benchmark of the row-wise kernels on one MI355X: per-kernel us/call and achieved HBM GB/s against the 8 TB/s peak.

    python bench.py [--steps K] [--warmup W] [--workload NAME] [--no-cold] [--no-cpu]
    python bench.py --copy-calibration          # plain kernels of known traffic, for the counter scaling
    python bench.py --ceiling                   # the practical HBM ceiling at each workload's size (probe kernels)
    python bench.py --probes                    # every probe structure and cache policy at each workload's size
    python bench.py --build-probes              # compile the probes (bench_probes.hip) into _build/
    python bench.py --topk-stages               # where a top-k launch's time goes, stage by stage (stage build)
    python bench.py --build-topk-stages         # compile that build (csrc/topk.hip with its stamps) into _build/
    python bench.py --profile-summary DIR       # turn one profiling lease's outputs into profiles/
    python bench.py --traffic-from DIR          # turn FETCH_SIZE / WRITE_SIZE counter runs into profiles/traffic.json

A step is one launch of the op over its whole workload with the inputs already resident in HBM. Each workload is
instantiated R times (R copies of its inputs and outputs, more bytes in all than the 256 MB Infinity Cache and the L2s
hold), and the K timed launches cycle through the copies back to back, bracketed by one pair of HIP events recorded on
the stream the launches run on (torch's current stream, which the C-ABI is handed): a launch never finds its data in
a cache, and the per-launch mean is the kernels' own duration plus the gaps between dependent launches -- the figure
the rocprofv3 kernel trace of the same command reports. `value` = algorithmic bytes / that mean: every input element
read once and every output element written once (workloads.algorithmic_bytes).

--cold (the default; --no-cold skips it) also times single launches one at a time, each after reading a 1 GiB buffer
(which evicts the caches without leaving dirty lines) and between its own pair of events: that adds the dispatch
latency of an isolated launch (a few microseconds) to every figure.

The JSON line is printed for the headline workload (RMSNorm bf16 [16384, 4096] with weight); `per_workload` carries
every named workload measured the same way. Beside each GPU figure, "cpu" times the reference's PyTorch path for that
workload on this host's cores (oracle/torch_paths, test infrastructure used here only as the timed baseline) over the
whole workload (--cpu-seconds of host time shared by all); the headline's is also `cpu_baseline`.
"""

import argparse
import glob
import csv
import hashlib
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
PKG_DIR = os.path.join(ROOT, "cuda-kernels-optimized-for-rtx5090_amd")

METRIC = "per-kernel µs/call + achieved HBM GB/s (% of MI355X peak) at named shape, 1 GPU"
PEAK_GBS = 8000.0
HEADLINE = "rmsnorm_16384x4096"
FLUSH_BYTES = 1 << 30
ROTATE_BYTES = 1280 << 20  # the copies of one workload together (at least 4): five times the Infinity Cache
COPY_BYTES = 256 << 20     # the calibration kernels: 256 MiB read by one, 256 MiB written by the other
TRAFFIC_PATH = os.path.join(ROOT, "profiles", "traffic.json")
# the kernels whose counters give each workload's traffic: a name fragment; the dispatches of one launch that contain
# it are summed (the whole launch for the two-kernel paths)
KERNELS = {"rmsnorm_16384x4096": "rmsnorm_rows", "softmax_4096x4096": "softmax_rows",
           "softmax_64x262144": "softmax_coop", "rope_4x4096_32q_8kv_128": "rope_vec",
           "topk_128x128256_k1": "topk_one", "topk_128x128256_k50": "topk_tile",
           "topk_128x128256_k1024": "topk_wide", "rmsnorm_add_16384x4096": "rmsnorm_rows",
           "rope_kv_4x4096_32q_8kv_128": "rope_vec", "rope_cache_4x4096_32q_8kv_128": "rope_vec"}


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=100)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--workload", default=None, help="measure only this workload (default: all)")
    p.add_argument("--k", type=int, default=None, help="top-k: measure only this k (default: 1, 50 and 1024)")
    p.add_argument("--tune", action="append", default=[],
                   help="op:slot=value, set before measuring through the op library's tuning hook (e.g. topk:0=2 "
                        "for plan()'s resident workgroups per CU); may be repeated")
    p.add_argument("--no-cold", action="store_true", help="skip the flushed single-launch timing")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--cpu-seconds", type=float, default=20.0,
                   help="host time shared by the CPU legs of the measured workloads")
    p.add_argument("--copy-calibration", action="store_true",
                   help="only launch a 256 MiB read-only and a 256 MiB write-only kernel --steps times (for the "
                        "counter scaling)")
    p.add_argument("--ceiling", action="store_true",
                   help="only time the bandwidth probes (bench_probes.hip): the best of the copy structures moving "
                        "each workload's algorithmic bytes, and a read of the top-k input")
    p.add_argument("--probes", action="store_true",
                   help="only time every probe structure and cache-policy pair at each workload's size")
    p.add_argument("--probe-summary", default=None,
                   help="directory of one probe lease (sweep.json, ceiling.json, pmc_*/, occ/): writes profiles/")
    p.add_argument("--summary-bench", default=None, help="a bench line (JSON file) whose workloads --probe-summary "
                                                         "sets beside the probes")
    p.add_argument("--build-probes", action="store_true",
                   help="compile bench_probes.hip into _build/libbench_probes.so (on a host with hipcc)")
    p.add_argument("--topk-stages", action="store_true",
                   help="only the top-k stage timeline at 128 x 128256 fp32, k = 1, 50 and 1024 (the stage build)")
    p.add_argument("--build-topk-stages", action="store_true",
                   help="compile csrc/topk.hip with its stage stamps into _build/libtopk_stages.so")
    p.add_argument("--profile-summary", default=None,
                   help="directory of one profiling lease (bench.json, stats/, traffic/, occ/): writes profiles/")
    p.add_argument("--traffic-from", default=None,
                   help="directory with rocprofv3 counter CSVs (fetch/ and write/ runs of this script and of "
                        "--copy-calibration); writes profiles/traffic.json")
    return p.parse_args()


class Case:
    """One workload bound to R device copies: `launch(i)` runs the op once on copy i % R."""

    def __init__(self, pkg, name, dev, k=None):
        import torch
        self.name, self.k = name, k
        w = pkg.workloads
        self.bytes = w.algorithmic_bytes(name, k or 50)
        inp = w.WORKLOADS[name]()
        stream = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731
        if name.startswith("softmax"):
            lib = pkg.candidate("softmax")._lib
            rows, cols = inp["x"].shape
            self.dtype = "fp32"

            def make():
                x = inp["x"].to(dev)
                y = torch.empty_like(x)
                return lambda: lib.launch(x.data_ptr(), y.data_ptr(), rows, cols, 0, 256, 1024, stream())
            footprint = 2 * inp["x"].numel() * 4
        elif name.startswith("rmsnorm_add"):
            lib = pkg.candidate("rmsnorm")._lib
            rows, cols = inp["x"].shape
            eps = inp["eps"]
            wt = inp["weight"].to(dev)
            self.dtype = "bf16"

            def make():
                # in place, as a decoder layer does: the residual stream is overwritten with x + residual
                x, r = inp["x"].to(dev), inp["residual"].to(dev)
                y = torch.empty_like(x)
                return lambda: lib.rmsnorm_add_launch(x.data_ptr(), r.data_ptr(), wt.data_ptr(), y.data_ptr(),
                                                      r.data_ptr(), rows, cols, 1, eps, 256, stream())
            footprint = 3 * inp["x"].numel() * 2
        elif name.startswith("rmsnorm"):
            lib = pkg.candidate("rmsnorm")._lib
            rows, cols = inp["x"].shape
            eps = inp["eps"]
            wt = inp["weight"].to(dev)
            self.dtype = "bf16"

            def make():
                x = inp["x"].to(dev)
                y = torch.empty_like(x)
                return lambda: lib.rmsnorm_launch_weighted(x.data_ptr(), wt.data_ptr(), y.data_ptr(), rows, cols, 1,
                                                           eps, 256, stream())
            footprint = 2 * inp["x"].numel() * 2
        elif name.startswith("rope_kv"):
            lib = pkg.candidate("rope")._lib
            B, S, Hq, D = inp["q"].shape
            Hk = inp["k"].shape[2]
            pos, inv = inp["position_ids"].to(dev), inp["inv_freq"].to(dev)
            slots = inp["slot_mapping"].to(dev)
            self.dtype = "bf16"

            def make():
                # q rotated in place; k, v read; the cache rows written
                q, kk, v = inp["q"].to(dev), inp["k"].to(dev), inp["v"].to(dev)
                kc, vc = inp["k_cache"].to(dev), inp["v_cache"].to(dev)
                return lambda: lib.rope_kv_launch(q.data_ptr(), kk.data_ptr(), v.data_ptr(), pos.data_ptr(),
                                                  inv.data_ptr(), q.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                                                  slots.data_ptr(), B * S, Hq, Hk, D, 1, stream())
            footprint = (inp["q"].numel() + 4 * inp["k"].numel()) * 2
        elif name.startswith("rope_cache"):
            lib = pkg.candidate("rope")._lib
            B, S, Hq, D = inp["q"].shape
            Hk = inp["k"].shape[2]
            pos, cos, sin = inp["position_ids"].to(dev), inp["cos"].to(dev), inp["sin"].to(dev)
            self.dtype = "bf16"

            def make():
                # the reference's ABI: cos/sin read from the fp32 cache; in place
                q, kk = inp["q"].to(dev), inp["k"].to(dev)
                return lambda: lib.launch(q.data_ptr(), kk.data_ptr(), cos.data_ptr(), sin.data_ptr(), pos.data_ptr(),
                                          q.data_ptr(), kk.data_ptr(), B * S, Hq, Hk, D, 1, 0, 40, 1, stream())
            footprint = 2 * (inp["q"].numel() + inp["k"].numel()) * 2
        elif name.startswith("rope"):
            lib = pkg.candidate("rope")._lib
            B, S, Hq, D = inp["q"].shape
            Hk = inp["k"].shape[2]
            pos, inv = inp["position_ids"].to(dev), inp["inv_freq"].to(dev)
            self.dtype = "bf16"

            def make():
                # in place: every call rotates the same buffers again (the traffic is the same every time)
                q, kk = inp["q"].to(dev), inp["k"].to(dev)
                return lambda: lib.rope_launch_freq(q.data_ptr(), kk.data_ptr(), pos.data_ptr(), inv.data_ptr(),
                                                    q.data_ptr(), kk.data_ptr(), B * S, Hq, Hk, D, 1, stream())
            footprint = 2 * (inp["q"].numel() + inp["k"].numel()) * 2
        elif name.startswith("topk_sample"):
            cand = pkg.candidate("topk")
            lib = cand._lib
            rows, cols = inp["x"].shape
            k, temp, top_p = inp["k"], inp["temperature"], inp["top_p"]
            chunk = cand._plan(inp["x"].to(dev), rows, cols, 0, k)[0]
            nchunks = -(-cols // chunk)
            uni = inp["uniforms"].to(dev)
            self.dtype = "fp32"

            def make():
                x = inp["x"].to(dev)
                vals = torch.empty(rows, k, device=dev)
                idx = torch.empty(rows, k, dtype=torch.int64, device=dev)
                drawn = torch.empty(rows, dtype=torch.int64, device=dev)
                work = torch.empty(max(1, rows * nchunks * k), dtype=torch.int64, device=dev)
                counters = torch.zeros(rows, dtype=torch.int32, device=dev)
                keep = (x, vals, idx, drawn, work, counters)

                def run():  # top-k with the draw fused into its launch
                    return lib.topk_launch_sample(keep[0].data_ptr(), vals.data_ptr(), idx.data_ptr(),
                                                  work.data_ptr(), counters.data_ptr(), rows, cols, k, 0,
                                                  cand._THREADS, cand._DEPTH, chunk, uni.data_ptr(), drawn.data_ptr(),
                                                  temp, top_p, stream())
                return run
            footprint = inp["x"].numel() * 4
        elif name.startswith("topk"):
            cand = pkg.candidate("topk")
            lib = cand._lib
            rows, cols = inp["x"].shape
            chunk = cand._plan(inp["x"].to(dev), rows, cols, 0, k)[0]
            nchunks = -(-cols // chunk)
            self.dtype = "fp32"

            def make():
                x = inp["x"].to(dev)
                vals = torch.empty(rows, k, device=dev)
                idx = torch.empty(rows, k, dtype=torch.int64, device=dev)
                work = torch.empty(max(1, rows * nchunks * k), dtype=torch.int64, device=dev)
                counters = torch.zeros(rows, dtype=torch.int32, device=dev)
                keep = (x, vals, idx, work, counters)
                return lambda: lib.launch(keep[0].data_ptr(), vals.data_ptr(), idx.data_ptr(), work.data_ptr(),
                                          counters.data_ptr(), rows, cols, k, 0, cand._THREADS, cand._DEPTH, chunk,
                                          stream())
            footprint = inp["x"].numel() * 4
        else:
            raise KeyError(name)
        self.copies = max(4, -(-ROTATE_BYTES // footprint))
        self.launchers = [make() for _ in range(self.copies)]
        self.inputs = inp

    def launch(self, i=0):
        return self.launchers[i % self.copies]()

    @property
    def label(self):
        return self.name if self.k is None else f"{self.name}_k{self.k}"


def check(err, label):
    if err:
        raise RuntimeError(f"{label}: launch returned {err}")


def time_rotating(case, steps, warmup):
    """K launches back to back over the rotating copies between one pair of events: the mean per launch."""
    import torch
    for i in range(warmup):
        check(case.launch(i), case.label)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    a.record()
    for i in range(steps):
        check(case.launch(warmup + i), case.label)
    b.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    us = a.elapsed_time(b) * 1e3 / steps
    return {"us_mean": us, "bytes": case.bytes, "wall_s": wall, "copies": case.copies,
            "gbs": case.bytes / (us * 1e-6) / 1e9, "pct_peak": 100.0 * case.bytes / (us * 1e-6) / 1e9 / PEAK_GBS}


def time_cold(case, steps, flush):
    """Single launches, each after a cache-evicting read and between its own events: median and p10/p90."""
    import torch
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    torch.cuda.synchronize()
    for i in range(steps):
        flush()
        starts[i].record()
        err = case.launch(i)
        ends[i].record()
        check(err, case.label)
    torch.cuda.synchronize()
    us = sorted(s.elapsed_time(e) * 1e3 for s, e in zip(starts, ends))
    return {"cold_us_median": us[len(us) // 2], "cold_us_p10": us[len(us) // 10],
            "cold_us_p90": us[(9 * len(us)) // 10]}


def cpu_paths(pkg, name, k):
    """(description, a callable running the reference's torch path once over the whole workload) for the CPU leg of a
    workload. The paths (oracle/torch_paths, test infrastructure used here only as the timed baseline):
    softmax/baseline.py:13 for softmax, the rmsnorm/kernel.cu:1-8 expression (times the weight) for RMSNorm, HF-style
    cos/sin construction for the tokens' positions and the rope/kernel.cu:1-11 rotation for RoPE, torch.topk for
    top-k. Every call runs over the whole workload (each takes at most tens of milliseconds on a server's cores), so
    the figure is not one of a sample that the host's caches hold."""
    import torch
    from oracle import torch_paths
    inp = pkg.workloads.WORKLOADS[name]()
    if name.startswith("softmax"):
        x = inp["x"]
        return f"torch.softmax over x{list(x.shape)} fp32", lambda: torch_paths.softmax(x)
    if name == "rmsnorm_16384x4096":
        x, w, eps = inp["x"], inp["weight"], inp["eps"]
        return "rmsnorm expression over x[16384, 4096] bf16 + weight", lambda: torch_paths.rmsnorm(x, w, eps)
    if name == "rmsnorm_add_16384x4096":
        x, r, w, eps = inp["x"], inp["residual"], inp["weight"], inp["eps"]
        return "h = x + residual, rmsnorm(h) * weight over [16384, 4096] bf16", \
            lambda: torch_paths.rmsnorm_add(x, r, w, eps)
    if name.startswith("rope"):
        q, kk, pos, inv = inp["q"], inp["k"], inp["position_ids"], inp["inv_freq"]

        def rope():
            # HF-style cos/sin for the positions, then the rotation of q and k in fp32, one rounding
            freqs = torch.outer(pos[0].float(), inv)
            emb = torch.cat((freqs, freqs), dim=-1)
            cos, sin = emb.cos(), emb.sin()
            return torch_paths.rope(q, cos, sin, pos), torch_paths.rope(kk, cos, sin, pos)
        if name.startswith("rope_kv"):
            v, slots = inp["v"], inp["slot_mapping"].reshape(-1)
            kc, vc = inp["k_cache"], inp["v_cache"]
            tokens = slots.numel()

            def rope_kv():
                qo, ko = rope()
                kc.index_copy_(0, slots, ko.reshape(tokens, 8, 128))
                vc.index_copy_(0, slots, v.reshape(tokens, 8, 128))
                return qo
            return "cos/sin, rotation of q and k, cache scatter of k and v over 16384 tokens", rope_kv
        if name.startswith("rope_cache"):
            cos, sin = inp["cos"], inp["sin"]
            return "the rotation of q[4, 4096, 32, 128] and k[4, 4096, 8, 128] bf16 with cos/sin gathered from the " \
                   "fp32 cache [4096, 128]", lambda: (torch_paths.rope(q, cos, sin, pos),
                                                      torch_paths.rope(kk, cos, sin, pos))
        return "cos/sin and the rotation of q[4, 4096, 32, 128] and k[4, 4096, 8, 128] bf16", rope
    if name == "topk_sample_128x128256":
        x, u = inp["x"], inp["uniforms"]
        kk, temp, top_p = inp["k"], inp["temperature"], inp["top_p"]

        def topk_sample():
            v, i = torch.topk(x, kk, dim=-1, sorted=True)
            p = torch.softmax(v / temp, dim=-1)
            c = torch.cumsum(p, dim=-1)
            keep = (c - p) < top_p * c[:, -1:]
            p = p * keep
            c = torch.cumsum(p, dim=-1)
            pick = torch.searchsorted(c, (u * c[:, -1]).unsqueeze(-1)).clamp_(max=kk - 1)
            return i.gather(-1, pick)
        return "torch.topk (k = 50) over x[128, 128256] fp32, softmax, nucleus cut, draw", topk_sample
    if name == "topk_128x128256":
        x = inp["x"]
        return f"torch.topk k = {k} over x[128, 128256] fp32", lambda: torch.topk(x, k, dim=-1, sorted=True)
    raise KeyError(name)


def cpu_leg(pkg, name, k, seconds):
    """The reference's CPU path for one workload on this host's cores (cpu_paths), in the metric's unit: the workload's
    algorithmic bytes / the median time of a call, over `seconds` of calls (at least 10, after 2 warm-ups)."""
    import torch
    torch.set_num_threads(os.cpu_count() or 1)
    what, fn = cpu_paths(pkg, name, k)
    nbytes = pkg.workloads.algorithmic_bytes(name, k or 50)
    for _ in range(2):
        fn()
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < 10:
        t = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t)
    times.sort()
    med = times[len(times) // 2]
    return {"value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "cores": torch.get_num_threads(), "kind": "port",
            "us_per_call": round(med * 1e6, 1),
            "sample": f"the whole workload: {what}; median of {len(times)} calls after 2 warm-ups, "
                      f"{med * 1e3:.3f} ms/call; cpu_count={os.cpu_count()}, cpu={cpu_model()}"}


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def sources_sha16():
    """A digest of the op libraries' kernel sources (csrc/), naming the code a measurement was made on."""
    h = hashlib.sha256()
    csrc = os.path.join(PKG_DIR, "csrc")
    for name in sorted(os.listdir(csrc)):
        if name.endswith((".hip", ".hpp")):
            with open(os.path.join(csrc, name), "rb") as f:
                h.update(name.encode() + b"\0" + f.read())
    return h.hexdigest()[:16]


def roofline_entry(res, label):
    """The roofline object of the bench line. `traffic` is not measured by this run: it is read from the committed
    profiles/traffic.json (FETCH_SIZE and WRITE_SIZE counter runs of a separate profiling lease), and
    `traffic_source` says so, with whether those runs counted the kernel sources this run uses."""
    traffic, source = None, None
    if os.path.exists(TRAFFIC_PATH):
        with open(TRAFFIC_PATH) as f:
            table = json.load(f)
        traffic = table.get(label, {}).get("bytes_per_launch")
        counted = table.get("sources_sha16")
        source = {"file": "profiles/traffic.json",
                  "how": "rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE runs of a separate profiling lease, not this run",
                  "sources_sha16": counted, "same_sources_as_this_run": counted == sources_sha16()}
    return {"bound": "hbm", "achieved": round(res["gbs"], 1), "peak": PEAK_GBS, "unit": "GB/s",
            "frac": round(res["gbs"] / PEAK_GBS, 4), "traffic": traffic, "traffic_source": source}


def copy_calibration(steps):
    """Plain streaming kernels of known traffic, each launched `steps` times over 4 rotating buffers of COPY_BYTES:
    torch's sum of an fp32 buffer (reads COPY_BYTES; its counter FETCH_SIZE scales the reads) and torch's fill_ of one
    (writes COPY_BYTES; its WRITE_SIZE scales the writes)."""
    import torch
    dev = torch.device("cuda:0")
    n = COPY_BYTES // 4
    bufs = [torch.ones(n, device=dev) for _ in range(4)]
    sink = torch.empty((), device=dev)
    for i in range(steps):
        torch.sum(bufs[i % 4], dim=0, out=sink)
        bufs[(i + 2) % 4].fill_(1.0)
    torch.cuda.synchronize()
    print(json.dumps({"calibration_bytes": COPY_BYTES, "launches": steps}))


PROBES_SRC = os.path.join(ROOT, "bench_probes.hip")
PROBES_LIB = os.path.join(ROOT, "_build", "libbench_probes.so")
PROBE_FAMILIES = {"stride": 0, "xcd": 1, "oneshot": 2, "slab": 3, "lds": 4, "row": 5, "read": 6, "write": 7}
POLICIES = {"none": 0, "nt": 2, "sc0sc1": 17, "ntsc1": 18, "ntsc0sc1": 19}
# The probes --ceiling takes the best of at each size: one of each structure, with the row kernels' cache policy.
CEILING_PROBES = ("stride_u4_b8_nt_nt", "stride_u16_b8_nt_nt", "xcd_u4_b8_nt_nt", "oneshot_u8_b8_nt_nt",
                  "slab_u4_b8_nt_nt", "lds_u4_b8_nt_nt", "row_u4_b8_nt_nt")


def build_probes():
    """Compiles bench_probes.hip for gfx950 with the op libraries' hipcc flags into _build/libbench_probes.so."""
    import subprocess
    from __graft_entry__ import load_package
    load_package()
    from ck5090_amd import make_libs
    os.makedirs(os.path.dirname(PROBES_LIB), exist_ok=True)
    tmp = PROBES_LIB + ".tmp"
    proc = subprocess.run([make_libs.hipcc(), *make_libs.HIPCC_FLAGS, PROBES_SRC, "-o", tmp], capture_output=True,
                          text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for bench_probes.hip ({proc.returncode}):\n" + proc.stderr[-6000:])
    os.replace(tmp, PROBES_LIB)
    return PROBES_LIB


def probe_lib():
    import ctypes
    if not os.path.exists(PROBES_LIB):
        raise RuntimeError(f"no probe library at {PROBES_LIB}: build it first (python bench.py --build-probes)")
    lib = ctypes.CDLL(PROBES_LIB)
    lib.probe_run.argtypes = [ctypes.c_int] * 5 + [ctypes.c_void_p] * 3 + [ctypes.c_longlong, ctypes.c_void_p]
    lib.probe_run.restype = ctypes.c_int
    return lib


STAGES_LIB = os.path.join(ROOT, "_build", "libtopk_stages.so")


def build_topk_stages():
    """Compiles csrc/topk.hip with ROWKERN_TOPK_STAGES (per-workgroup stage stamps, see the file) into
    _build/libtopk_stages.so: a timing build beside the op library, which is built without the stamps."""
    import subprocess
    from __graft_entry__ import load_package
    load_package()
    from ck5090_amd import make_libs
    os.makedirs(os.path.dirname(STAGES_LIB), exist_ok=True)
    tmp = STAGES_LIB + ".tmp"
    src = os.path.join(make_libs.CSRC, "topk.hip")
    proc = subprocess.run([make_libs.hipcc(), *make_libs.HIPCC_FLAGS, *make_libs.OP_FLAGS["topk"],
                           "-DROWKERN_TOPK_STAGES", "-I", make_libs.CSRC, src, "-o", tmp], capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for the top-k stage build ({proc.returncode}):\n" + proc.stderr[-6000:])
    os.replace(tmp, STAGES_LIB)
    return STAGES_LIB


# The stamped stages of each top-k kernel (slot: name); slots 16 + w hold wave w's loads-landed moment.
TOPK_STAGES = {
    "topk_one": [(0, "start"), (1, "loads landed (wave 0)"), (2, "workgroup's best"), (3, "arrival counted"),
                 (8, "row written")],
    "topk_tile": [(0, "start"), (1, "loads landed (wave 0)"), (11, "wave 0's bound"), (2, "threshold"),
                  (9, "tile filtered"),
                  (10, "list settled"), (3, "chunk's tiles done"),
                  (4, "chunk list published"), (5, "arrival counted"), (6, "merge: floor, candidates counted"),
                  (7, "merge: candidates compacted"), (8, "row written")],
    "topk_wide": [(0, "start"), (1, "loads landed (wave 0)"), (2, "bounds"), (3, "tile appended"), (4, "list published"),
                  (5, "arrival counted"), (6, "merge: floor from the headers"), (7, "merge: lists gathered"),
                  (12, "ordering: bucket counts"), (13, "ordering: bucket scan"), (14, "ordering: scatter"),
                  (15, "ordering: positions"), (8, "row written")],
}
STAGE_SLOTS, STAGE_WGS = 32, 4096
STAGE_TICK_US = 0.01  # s_memrealtime runs at 100 MHz


def topk_stages(launches=3, copies=5):
    """The stage timeline of one top-k launch per k (1, 50, 1024) at 128 x 128256 fp32, from the stage build: per
    stage, when the workgroups reach it (from the launch's first stamp) and how long each workgroup spends from the
    stage before (the per-workgroup delta). Each timed launch reads a copy of x last read `copies` - 1 launches
    earlier (more bytes than the caches hold), after warm-up launches. Returns the text lines."""
    import ctypes
    import numpy as np
    import torch
    if not os.path.exists(STAGES_LIB):
        raise RuntimeError(f"no stage build at {STAGES_LIB}: build it first (python bench.py --build-topk-stages)")
    lib = ctypes.CDLL(STAGES_LIB)
    lib.plan.argtypes = [ctypes.c_longlong, ctypes.c_longlong, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int]
    lib.plan.restype = ctypes.c_longlong
    lib.launch.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_longlong, ctypes.c_longlong] + [ctypes.c_int] * 4 + \
                          [ctypes.c_longlong, ctypes.c_void_p]
    lib.topk_stages_read.argtypes = [ctypes.c_void_p, ctypes.c_longlong]
    rows, cols = 128, 128256
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)
    xs = [torch.randn(rows, cols, device=dev, generator=g) * 2 for _ in range(copies)]
    stream = torch.cuda.current_stream(dev).cuda_stream
    out = []
    for k, kernel in ((1, "topk_one"), (50, "topk_tile"), (1024, "topk_wide")):
        chunk = lib.plan(rows, cols, 0, 256, 4, max(2048, 16 * k) if k > 64 else 2048)
        nch = -(-cols // chunk)
        vals = torch.empty(rows, k, device=dev)
        idx = torch.empty(rows, k, dtype=torch.int64, device=dev)
        work = torch.empty(rows * nch * k, dtype=torch.int64, device=dev)
        counters = torch.zeros(rows, dtype=torch.int32, device=dev)

        def go(i):
            x = xs[i % copies]
            rc = lib.launch(x.data_ptr(), vals.data_ptr(), idx.data_ptr(), work.data_ptr(), counters.data_ptr(), rows,
                            cols, k, 0, 256, 4, chunk, stream)
            if rc != 0:
                raise RuntimeError(f"top-k stage build: launch returned {rc}")
        for i in range(2 * copies + 1):  # the last warm-up launch reads copy 0
            go(i)
        torch.cuda.synchronize()
        ref = torch.topk(xs[0], k, dim=1)
        if not (torch.equal(vals, ref.values) and torch.equal(idx, ref.indices)):
            raise RuntimeError(f"top-k stage build differs from torch.topk at k = {k}")
        per = {i: ([], []) for i, _ in TOPK_STAGES[kernel]}
        spans, wave_skew, wgs = [], [], 0
        for rep in range(launches):
            for i in range(1, copies):  # the other copies, then copy 0 again
                go(i)
            if lib.topk_stages_clear() != 0:
                raise RuntimeError("topk_stages_clear failed")
            go(0)
            torch.cuda.synchronize()
            buf = np.zeros(STAGE_WGS * STAGE_SLOTS, dtype=np.uint64)
            if lib.topk_stages_read(buf.ctypes.data, buf.nbytes) != 0:
                raise RuntimeError("topk_stages_read failed")
            t = buf.reshape(STAGE_WGS, STAGE_SLOTS).astype(np.int64)
            t = t[t[:, 0] > 0]
            wgs = len(t)
            t0 = t[:, 0].min()
            spans.append((t[:, :16].max() - t0) * STAGE_TICK_US)
            waves = t[:, 16:]
            seen = waves > 0
            lo = np.where(seen, waves, np.iinfo(np.int64).max).min(axis=1)
            hi = np.where(seen, waves, 0).max(axis=1)
            wave_skew += list((hi - lo)[seen.any(axis=1)] * STAGE_TICK_US)
            prev = None
            for i, _ in TOPK_STAGES[kernel]:
                col = t[:, i]
                per[i][0].extend(((col[col > 0] - t0) * STAGE_TICK_US).tolist())
                if prev is not None:
                    ok = (col > 0) & (t[:, prev] > 0)
                    per[i][1].extend(((col[ok] - t[ok, prev]) * STAGE_TICK_US).tolist())
                prev = i
        out.append(f"k = {k}: {kernel}, {wgs} workgroups (chunk {chunk}), {launches} launches; launch span (first stamp "
                   f"to last) median {np.median(spans):.2f} us; loads landed across one workgroup's waves: median "
                   f"{np.median(wave_skew):.2f}, p90 {np.percentile(wave_skew, 90):.2f} us")
        out.append(f"  {'stage':36s} {'workgroups':>10s} {'reached: median':>16s} {'p90':>7s} {'max':>7s}   "
                   f"{'from the stage before: median':>29s} {'p90':>7s}")
        for i, name in TOPK_STAGES[kernel]:
            at, d = (np.array(v) for v in per[i])
            if len(at) == 0:
                continue
            dd = f"{np.median(d):29.2f} {np.percentile(d, 90):7.2f}" if len(d) else f"{'':29s} {'':7s}"
            out.append(f"  {name:36s} {len(at) // launches:10d} {np.median(at):16.2f} {np.percentile(at, 90):7.2f} "
                       f"{at.max():7.2f}   {dd}")
        out.append("")
    return out


def parse_probe(spec):
    """'family_u<unroll>_b<blocks per CU>_<load policy>_<store policy>' -> the arguments of probe_run."""
    fam, u, b, lp, sp = spec.split("_")
    return PROBE_FAMILIES[fam], int(u[1:]), int(b[1:]), POLICIES[lp], POLICIES[sp]


class ProbeCase:
    """A bandwidth probe (bench_probes.hip) bound to R device copies, timed as the workloads are. `nbytes` is the total
    HBM traffic of one launch: a copy reads nbytes / 2 and writes as many, a read or a write moves nbytes."""

    def __init__(self, lib, spec, nbytes, dev):
        import torch
        family, unroll, bpc, lp, sp = parse_probe(spec)
        copy = family not in (PROBE_FAMILIES["read"], PROBE_FAMILIES["write"])
        self.label, self.k = spec, None
        moved = (nbytes // 2 if copy else nbytes) // 16 * 16
        stream = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731
        sink = torch.zeros(1, dtype=torch.int32, device=dev)

        self.buffers = []  # the copies' tensors, held for as long as their pointers are launched on

        def make():
            reads, writes = family != PROBE_FAMILIES["write"], family != PROBE_FAMILIES["read"]
            x = torch.ones(moved // 4, dtype=torch.float32, device=dev) if reads else None
            y = torch.empty(moved // 4, dtype=torch.float32, device=dev) if writes else None
            self.buffers.append((x, y, sink))
            xp, yp = x.data_ptr() if reads else None, y.data_ptr() if writes else None
            return lambda: lib.probe_run(family, unroll, bpc, lp, sp, xp, yp, sink.data_ptr(), moved, stream())
        footprint = 2 * moved if copy else moved
        self.copies = max(4, -(-ROTATE_BYTES // footprint))
        self.launchers = [make() for _ in range(self.copies)]
        self.bytes = 2 * moved if copy else moved

    def launch(self, i=0):
        return self.launchers[i % self.copies]()


def time_probes(specs, sizes, steps, warmup):
    """{(spec, size label): timing} for every probe at every (label, total bytes) size."""
    import torch
    dev = torch.device("cuda:0")
    lib = probe_lib()
    out = {}
    for label, nbytes in sizes:
        for spec in specs:
            case = ProbeCase(lib, spec, nbytes, dev)
            res = time_rotating(case, steps, warmup)
            print(f"[probe] {label} {spec}: {res['us_mean']:.2f} us/call  {res['gbs']:.0f} GB/s  "
                  f"{res['pct_peak']:.1f}% of peak", file=sys.stderr, flush=True)
            out[(spec, label)] = {key: round(res[key], 3) for key in ("us_mean", "bytes", "gbs", "pct_peak")}
            del case
            torch.cuda.empty_cache()
    return out


def ceiling_sizes(pkg):
    w = pkg.workloads
    return [(n, w.algorithmic_bytes(n)) for n in ("softmax_4096x4096", "rmsnorm_16384x4096", "rope_4x4096_32q_8kv_128",
                                                  "rmsnorm_add_16384x4096", "rope_kv_4x4096_32q_8kv_128")]


def ceiling(pkg, steps, warmup):
    """The practical HBM ceiling at each workload's size: the best of the copy probes (one of each structure) moving
    the workload's algorithmic bytes, half read and half written (the 1R + 1W pattern of the row kernels), and the read
    probe over the top-k input. One JSON line {workload: {best, us_mean, gbs, pct_peak, probes: {spec: us_mean}}}."""
    res = time_probes(CEILING_PROBES, ceiling_sizes(pkg), steps, warmup)
    res.update(time_probes(("read_u8_b8_nt_nt",), [("topk_128x128256", 128 * 128256 * 4)], steps, warmup))
    out = {}
    for (spec, label), r in res.items():
        e = out.setdefault(label, {"probes": {}})
        e["probes"][spec] = r["us_mean"]
        if "us_mean" not in e or r["us_mean"] < e["us_mean"]:
            e.update({"best": spec, **{k: r[k] for k in ("us_mean", "bytes", "gbs", "pct_peak")}})
    print(json.dumps(out))


def probe_sweep(pkg, steps, warmup):
    """Every probe structure and every cache-policy pair of the stride probe at each workload's size, plus the read and
    the write probes at the same sizes. One JSON line {size: {spec: us_mean}}."""
    specs = [f"stride_u{u}_b{b}_nt_nt" for u in (2, 4, 8, 16) for b in (4, 8, 16)]
    specs += [f"stride_u4_b8_{lp}_{sp}" for lp in POLICIES for sp in POLICIES if (lp, sp) != ("nt", "nt")]
    specs += [f"{f}_u{u}_b8_nt_nt" for f, us in (("xcd", (4, 8)), ("oneshot", (4, 8, 16)), ("slab", (4, 8)),
                                                  ("lds", (2, 4, 8)), ("row", (4, 8))) for u in us]
    sizes = ceiling_sizes(pkg)
    res = time_probes(specs, sizes, steps, warmup)
    half = [(f"{label}_each_way", nbytes // 2) for label, nbytes in sizes]
    res.update(time_probes(("read_u8_b8_nt_nt", "read_u4_b8_nt_nt", "write_u4_b8_nt_nt", "write_u8_b8_nt_nt"), half,
                           steps, warmup))
    out = {}
    for (spec, label), r in res.items():
        out.setdefault(label, {})[spec] = [r["us_mean"], r["pct_peak"]]
    print(json.dumps(out))


def counter_means(run_dir, counter):
    """Mean per dispatch of `counter` for each kernel name in the rocprofv3 counter CSVs under run_dir."""
    sums, counts = {}, {}
    for path in glob.glob(os.path.join(run_dir, "**", "*counter_collection.csv"), recursive=True):
        with open(path) as f:
            for r in csv.DictReader(f):
                if r["Counter_Name"] != counter:
                    continue
                key = (r["Kernel_Name"], r.get("Dispatch_Id") or r.get("Correlation_Id"))
                sums[key] = sums.get(key, 0.0) + float(r["Counter_Value"])
    per_kernel = {}
    for (name, _), v in sums.items():
        per_kernel.setdefault(name, []).append(v)
    return {name: sum(v) / len(v) for name, v in per_kernel.items()}


def traffic_from(run_dir):
    """FETCH_SIZE and WRITE_SIZE (KiB per dispatch) of each workload's dominant kernel, scaled by the ratio of the
    calibration copy's known bytes to its counted bytes, into profiles/traffic.json."""
    fetch = {}
    write = {}
    for sub in sorted(os.listdir(run_dir)):
        d = os.path.join(run_dir, sub)
        if os.path.isdir(d):
            fetch.update({(sub, n): v for n, v in counter_means(d, "FETCH_SIZE").items()})
            write.update({(sub, n): v for n, v in counter_means(d, "WRITE_SIZE").items()})

    def pick(table, sub, pattern):
        hits = [v for (s, n), v in table.items() if s == sub and pattern in n]
        return sum(hits) if hits else None

    cf, cw = pick(fetch, "copy_fetch", "reduce_kernel"), pick(write, "copy_write", "FillFunctor")
    f_scale = COPY_BYTES / (cf * 1024) if cf else 1.0
    w_scale = COPY_BYTES / (cw * 1024) if cw else 1.0
    out = {"_method": "rocprofv3 --pmc FETCH_SIZE, then --pmc WRITE_SIZE, in separate runs of bench.py --workload W "
                      "(KiB per dispatch, mean over dispatches of the named kernels, summed over the kernels of one "
                      "launch), each scaled by the known bytes of the matching kernel of bench.py --copy-calibration "
                      "(a 256 MiB sum for FETCH_SIZE, a 256 MiB fill for WRITE_SIZE) over its counted bytes",
           "calibration_fetch_kib": cf and round(cf, 1), "calibration_write_kib": cw and round(cw, 1),
           "fetch_scale": round(f_scale, 4), "write_scale": round(w_scale, 4),
           "sources_sha16": sources_sha16()}
    for label, kernel in KERNELS.items():
        f = pick(fetch, f"{label}_fetch", kernel)
        w = pick(write, f"{label}_write", kernel)
        if f is None or w is None:
            continue
        out[label] = {"kernel": kernel, "fetch_kib": round(f, 1), "write_kib": round(w, 1),
                      "bytes_per_launch": int(round(f * 1024 * f_scale + w * 1024 * w_scale))}
    os.makedirs(os.path.dirname(TRAFFIC_PATH), exist_ok=True)
    with open(TRAFFIC_PATH, "w") as f:
        json.dump(out, f, indent=1)
    print(json.dumps(out))


def kernel_stats(db_path):
    """Per-kernel call count and average duration (us) from a rocprofv3 --kernel-trace --stats database."""
    import sqlite3
    con = sqlite3.connect(db_path)
    rows = con.execute("select name, total_calls, average from top_kernels").fetchall()
    con.close()
    return [(name, int(calls), float(avg)) for name, calls, avg in rows]


def short_kernel(name):
    """A kernel's symbol without the return type, namespaces and argument list, template arguments kept."""
    return name.replace("void ", "").replace("(anonymous namespace)::", "").replace("at::native::", "").split("(")[0]


def occupancy(run_dir, cus=256, xcds=8):
    """Per-kernel means per dispatch of the occupancy and instruction counters in run_dir's counter CSVs: resident
    waves per CU (4 * SQ_WAVE_CYCLES, which counts in units of four cycles, over the busy cycles of one XCD,
    GRBM_GUI_ACTIVE / xcds as read summed over the XCDs, over the CUs), the occupancy as a % of the 32 waves a CU holds
    (rocprofv3's OccupancyPercent formula for gfx950), and the instructions issued per wave."""
    out = {}
    for name in ("SQ_WAVES", "SQ_WAVE_CYCLES", "GRBM_GUI_ACTIVE", "SQ_INSTS_VALU", "SQ_INSTS_SALU", "SQ_INSTS_LDS"):
        for kernel, v in counter_means(run_dir, name).items():
            out.setdefault(kernel, {})[name] = v
    res = {}
    for kernel, c in out.items():
        if len(c) < 6 or c["SQ_WAVES"] <= 64:
            continue
        busy = c["GRBM_GUI_ACTIVE"] / xcds
        waves = 4 * c["SQ_WAVE_CYCLES"] / busy / cus
        res[kernel] = {"waves": int(c["SQ_WAVES"]), "resident_waves_per_cu": round(waves, 2),
                       "occupancy_pct": round(100 * waves / 32, 1),
                       "valu_per_wave": round(c["SQ_INSTS_VALU"] / c["SQ_WAVES"]),
                       "salu_per_wave": round(c["SQ_INSTS_SALU"] / c["SQ_WAVES"]),
                       "lds_per_wave": round(c["SQ_INSTS_LDS"] / c["SQ_WAVES"])}
    return res


WAVE_PASSES = (("SQ_WAVES", "SQ_WAVE_CYCLES", "SQ_BUSY_CYCLES", "SQ_WAIT_ANY", "SQ_WAIT_INST_ANY", "SQ_ACTIVE_INST_ANY",
                "SQ_ACTIVE_INST_VALU", "SQ_ACTIVE_INST_SCA", "GRBM_GUI_ACTIVE"),
               ("SQ_ACTIVE_INST_LDS", "SQ_ACTIVE_INST_VMEM", "SQ_ACTIVE_INST_MISC", "SQ_WAIT_INST_LDS",
                "SQ_LDS_BANK_CONFLICT", "SQ_INSTS_VMEM_RD", "SQ_INSTS_VMEM_WR", "SQ_INSTS_LDS"))


def wave_breakdown(run_dir):
    """Where each kernel's wave time goes, from the two counter passes of WAVE_PASSES (run_dir/a, run_dir/b): per
    dispatch, the share of wave-cycles (SQ_WAVE_CYCLES, like the others in units of four cycles) spent waiting for
    anything, waiting for an instruction's dependency, and issuing VALU, scalar, LDS and memory instructions; LDS bank
    conflict cycles and memory instructions per wave."""
    out = {}
    for sub, names in zip(("a", "b"), WAVE_PASSES):
        for name in names:
            for kernel, v in counter_means(os.path.join(run_dir, sub), name).items():
                out.setdefault(kernel, {})[name] = v
    res = {}
    for kernel, c in out.items():
        if c.get("SQ_WAVES", 0) <= 64 or not c.get("SQ_WAVE_CYCLES"):
            continue
        wc = c["SQ_WAVE_CYCLES"]
        pct = lambda n: round(100 * c.get(n, 0) / wc, 1)  # noqa: E731
        res[kernel] = {"waves": int(c["SQ_WAVES"]), "wait_any_pct": pct("SQ_WAIT_ANY"),
                       "wait_inst_pct": pct("SQ_WAIT_INST_ANY"), "active_any_pct": pct("SQ_ACTIVE_INST_ANY"),
                       "valu_pct": pct("SQ_ACTIVE_INST_VALU"), "scalar_pct": pct("SQ_ACTIVE_INST_SCA"),
                       "lds_pct": pct("SQ_ACTIVE_INST_LDS"), "vmem_pct": pct("SQ_ACTIVE_INST_VMEM"),
                       "wait_lds_pct": pct("SQ_WAIT_INST_LDS"),
                       "lds_conflict_per_wave": round(c.get("SQ_LDS_BANK_CONFLICT", 0) / c["SQ_WAVES"], 1),
                       "vmem_rd_per_wave": round(c.get("SQ_INSTS_VMEM_RD", 0) / c["SQ_WAVES"], 1),
                       "vmem_wr_per_wave": round(c.get("SQ_INSTS_VMEM_WR", 0) / c["SQ_WAVES"], 1)}
    return res


def profile_summary(run_dir):
    """Writes profiles/ from one profiling lease (run_dir as the profiling script leaves it: bench.json and
    bench.err of the bench line, stats/ of the kernel trace, traffic/ of the FETCH_SIZE / WRITE_SIZE runs, occ/ of the
    occupancy runs): kernel_trace_bench_workloads.txt, traffic.json and traffic_counters.txt, and
    occupancy_bench_workloads.txt."""
    prof = os.path.join(ROOT, "profiles")
    with open(os.path.join(run_dir, "bench.json")) as f:
        line = json.loads(f.read().strip().splitlines()[-1])
    dbs = glob.glob(os.path.join(run_dir, "stats", "**", "*results.db"), recursive=True)
    stats = kernel_stats(dbs[0]) if dbs else []
    lines = ["# Kernel durations on MI355X: rocprofv3 kernel trace of bench.py, with bench.py's own figures from the same",
             "# lease (one fresh box, the same binaries)", "",
             "Commands (from /tmp, TMPDIR=/tmp):",
             "    python3 bench.py                                                        -> the bench line",
             "    rocprofv3 --kernel-trace --stats -d <dir>/stats -o s -- python3 bench.py --no-cold --no-cpu",
             "    python3 bench.py --profile-summary <dir>                                -> this file", "",
             f"{'kernel':<76} {'calls':>6} {'avg us':>9}"]
    for name, calls, avg in sorted(stats, key=lambda r: -r[1] * r[2]):
        lines.append(f"{short_kernel(name)[:76]:<76} {calls:>6} {avg:>9.2f}")
    lines += ["", "bench.py (back-to-back launches over rotating copies; single flushed launch median):",
              f"{'workload':<34} {'us/launch':>10} {'GB/s':>8} {'% of 8 TB/s':>12} {'flushed us':>11}"]
    for lab, r in line["per_workload"].items():
        lines.append(f"{lab:<34} {r['us_mean']:>10.2f} {r['gbs']:>8.0f} {r['pct_peak']:>12.1f} "
                     f"{r.get('cold_us_median', float('nan')):>11.2f}")
    with open(os.path.join(prof, "kernel_trace_bench_workloads.txt"), "w") as f:
        f.write("\n".join(lines) + "\n")
    traffic_from(os.path.join(run_dir, "traffic"))
    with open(TRAFFIC_PATH) as f:
        tr = json.load(f)
    from __graft_entry__ import load_package
    pkg = load_package()
    t_lines = ["# HBM traffic per launch from rocprofv3 counters", "",
               "Commands (from /tmp, TMPDIR=/tmp, one counter per run; W in the workloads below):",
               "    rocprofv3 --pmc FETCH_SIZE --output-format csv -d <dir>/traffic/W_fetch -o p -- python3 bench.py "
               "--workload W --steps 5 --warmup 1 --no-cold --no-cpu",
               "    rocprofv3 --pmc WRITE_SIZE --output-format csv -d <dir>/traffic/W_write -o p -- python3 bench.py "
               "--workload W --steps 5 --warmup 1 --no-cold --no-cpu",
               "    (top-k: --workload topk_128x128256 --k 50, and --k 1024)",
               "    rocprofv3 --pmc FETCH_SIZE --output-format csv -d <dir>/traffic/copy_fetch -o p -- python3 bench.py "
               "--copy-calibration --steps 5   (and WRITE_SIZE into copy_write)",
               "    python3 bench.py --profile-summary <dir>   -> profiles/traffic.json and this file", "",
               f"Calibration: a 256 MiB torch sum counts FETCH_SIZE {tr['calibration_fetch_kib']} KiB -> fetch scale "
               f"{tr['fetch_scale']};",
               f"             a 256 MiB torch fill counts WRITE_SIZE {tr['calibration_write_kib']} KiB -> write scale "
               f"{tr['write_scale']}.", "",
               f"{'workload':<28} {'kernels':<14} {'FETCH KiB':>10} {'WRITE KiB':>10} {'bytes/launch':>13} "
               f"{'algorithmic':>12} {'ratio':>6}"]
    for label, r in tr.items():
        if label.startswith("_") or not isinstance(r, dict):
            continue
        name, _, kk = label.partition("_k")
        k = int(kk) if kk.isdigit() else None
        if k is None:
            name = label
        algo = pkg.workloads.algorithmic_bytes(name, k or 50)
        t_lines.append(f"{label:<28} {r['kernel']:<14} {r['fetch_kib']:>10.1f} {r['write_kib']:>10.1f} "
                       f"{r['bytes_per_launch']:>13} {algo:>12} {r['bytes_per_launch'] / algo:>6.3f}")
    with open(os.path.join(prof, "traffic_counters.txt"), "w") as f:
        f.write("\n".join(t_lines) + "\n")
    occ_lines = ["# Occupancy and instructions per wave on MI355X (rocprofv3 counters, per dispatch, mean over the "
                 "dispatches of each kernel)", "",
                 "Command (from /tmp, TMPDIR=/tmp, one run per workload W):",
                 "    rocprofv3 --pmc SQ_WAVES SQ_WAVE_CYCLES SQ_BUSY_CYCLES SQ_INSTS_VALU SQ_INSTS_SALU SQ_INSTS_LDS "
                 "GRBM_GUI_ACTIVE --output-format csv -d <dir>/occ/W -o p -- python3 bench.py --workload W --steps 5 "
                 "--warmup 1 --no-cold --no-cpu",
                 "resident waves per CU = 4 * SQ_WAVE_CYCLES / (GRBM_GUI_ACTIVE / 8 XCDs) / 256 CUs; occupancy = that "
                 "/ 32 waves per CU (rocprofv3's OccupancyPercent for gfx950); over the whole dispatch, ramp and tail "
                 "included", "",
                 f"{'workload':<26} {'kernel':<52} {'waves':>6} {'waves/CU':>9} {'occ %':>6} {'VALU/w':>7} "
                 f"{'SALU/w':>7} {'LDS/w':>6}"]
    for w in sorted(os.listdir(os.path.join(run_dir, "occ"))):
        for kernel, r in occupancy(os.path.join(run_dir, "occ", w)).items():
            occ_lines.append(f"{w:<26} {short_kernel(kernel)[:52]:<52} {r['waves']:>6} {r['resident_waves_per_cu']:>9} "
                             f"{r['occupancy_pct']:>6} {r['valu_per_wave']:>7} {r['salu_per_wave']:>7} "
                             f"{r['lds_per_wave']:>6}")
    with open(os.path.join(prof, "occupancy_bench_workloads.txt"), "w") as f:
        f.write("\n".join(occ_lines) + "\n")
    w_lines = []
    wdir = os.path.join(run_dir, "waves")
    if os.path.isdir(wdir):
        w_lines = ["# Where the wave time goes on MI355X (rocprofv3 SQ counters, per dispatch, mean over the dispatches of each "
                   "kernel)", "",
                   "Commands (from /tmp, TMPDIR=/tmp, two runs per workload W, one per counter set):",
                   "    rocprofv3 --pmc " + " ".join(WAVE_PASSES[0]) + " --output-format csv -d <dir>/waves/W/a -o p -- "
                   "python3 bench.py --workload W --steps 5 --warmup 1 --no-cold --no-cpu",
                   "    rocprofv3 --pmc " + " ".join(WAVE_PASSES[1]) + " --output-format csv -d <dir>/waves/W/b -o p -- "
                   "python3 bench.py --workload W --steps 5 --warmup 1 --no-cold --no-cpu",
                   "Shares of SQ_WAVE_CYCLES (the time waves are resident): waiting for anything (memory, barriers, "
                   "dependencies), waiting for an",
                   "instruction's dependency, and issuing VALU, scalar, LDS and memory instructions (issue shares overlap "
                   "the waits of other waves", "of the same SIMD); LDS bank-conflict cycles and memory instructions per "
                   "wave.", "",
                   f"{'workload':<24} {'kernel':<46} {'wait%':>6} {'dep%':>5} {'issue%':>7} {'VALU%':>6} {'SCA%':>5} "
                   f"{'LDS%':>5} {'VMEM%':>6} {'LDSwait%':>8} {'conf/w':>7} {'rd/w':>6} {'wr/w':>6}"]
        for w in sorted(os.listdir(wdir)):
            for kernel, r in wave_breakdown(os.path.join(wdir, w)).items():
                w_lines.append(f"{w:<24} {short_kernel(kernel)[:46]:<46} {r['wait_any_pct']:>6} {r['wait_inst_pct']:>5} "
                               f"{r['active_any_pct']:>7} {r['valu_pct']:>6} {r['scalar_pct']:>5} {r['lds_pct']:>5} "
                               f"{r['vmem_pct']:>6} {r['wait_lds_pct']:>8} {r['lds_conflict_per_wave']:>7} "
                               f"{r['vmem_rd_per_wave']:>6} {r['vmem_wr_per_wave']:>6}")
        with open(os.path.join(prof, "wave_cycles_bench_workloads.txt"), "w") as f:
            f.write("\n".join(w_lines) + "\n")
    print("\n".join(lines + [""] + t_lines + [""] + occ_lines + [""] + w_lines))


def probe_summary(run_dir, bench_json=None):
    """Writes profiles/probe_ceiling_and_structures.txt from one probe lease (run_dir as the probe script leaves it:
    sweep.json of --probes, ceiling.json of --ceiling, pmc_FETCH_SIZE/ and pmc_WRITE_SIZE/ of the counter runs of
    --ceiling --steps 5 --warmup 1, occ_probes/ (or occ/) of its occupancy run), set beside the workloads of a bench
    line (bench_json, from the same lease when it has one)."""
    def last_json(path):
        with open(path) as f:
            return json.loads(f.read().strip().splitlines()[-1])
    sweep = last_json(os.path.join(run_dir, "sweep.json"))
    ceil = last_json(os.path.join(run_dir, "ceiling.json"))
    work = last_json(bench_json)["per_workload"] if bench_json else {}
    sizes = [s for s in sweep if not s.endswith("_each_way")]
    lines = ["# Bandwidth probes: what a plain copy, read or write reaches on MI355X at each workload's size", "",
             "Commands (one MI355X; the rocprofv3 runs from /tmp, TMPDIR=/tmp):",
             "    python3 bench.py --probes          -> every structure and cache-policy pair below",
             "    python3 bench.py --ceiling         -> the best structure at each size (the ceiling table)",
             "    rocprofv3 --pmc FETCH_SIZE --output-format csv -d <dir>/pmc_FETCH_SIZE -o p -- python3 bench.py "
             "--ceiling --steps 5 --warmup 1   (and WRITE_SIZE; and SQ_WAVES SQ_WAVE_CYCLES SQ_BUSY_CYCLES "
             "SQ_INSTS_VALU SQ_INSTS_SALU SQ_INSTS_LDS GRBM_GUI_ACTIVE into <dir>/occ)",
             "    python3 bench.py --probe-summary <dir> [--summary-bench <bench line>]   -> this file", "",
             "Probes (bench_probes.hip): stride = persistent grid-stride copy, u = 16-byte vectors per lane in flight, "
             "b = workgroups",
             "of 256 threads per CU; xcd = stride with each XCD walking one contiguous eighth; oneshot = one workgroup "
             "per tile, no loop;",
             "slab = one contiguous slab per workgroup, register double-buffered; lds = loads straight to LDS "
             "(global_load_lds_dwordx4);",
             "row = the row kernels' structure (a row per workgroup, next row loaded during a barrier exchange); "
             "read / write = one",
             "direction only. Cache policies (load_store): none, nt, sc0sc1, ntsc1, ntsc0sc1. Sizes are the workloads' "
             "algorithmic bytes,",
             "half read and half written; each probe timed as the workloads are (20 warm-up + 100 launches over "
             "rotating copies, >= 1.25 GiB).", "",
             "## us per launch (% of 8 TB/s)", "",
             "| probe | " + " | ".join(sizes) + " |", "|---|" + "---|" * len(sizes)]
    for spec in sweep[sizes[0]]:
        lines.append(f"| {spec} | " + " | ".join(f"{sweep[s][spec][0]:.2f} ({sweep[s][spec][1]:.1f})"
                                                   for s in sizes) + " |")
    each = [s for s in sweep if s.endswith("_each_way")]
    lines += ["", "## One direction only, at half of each size (the bytes one direction of the copy moves)", "",
              "| probe | " + " | ".join(each) + " |", "|---|" + "---|" * len(each)]
    for spec in sweep[each[0]]:
        lines.append(f"| {spec} | " + " | ".join(f"{sweep[s][spec][0]:.2f} ({sweep[s][spec][1]:.1f})"
                                                   for s in each) + " |")
    lines += ["", "## Ceiling (bench.py --ceiling: the best of one probe per structure, nt loads and stores) and the "
              "workloads", "",
              "| size | best probe | us | % of 8 TB/s | best of the sweep (any policy) | workload us | workload % of "
              "8 TB/s | workload / best probe |", "|---|---|---|---|---|---|---|---|"]
    for label, e in ceil.items():
        best_any = min(sweep.get(label, {}).items(), key=lambda kv: kv[1][0], default=(None, [float("nan")]))
        wl = work.get(label) or work.get(f"{label}_k1")
        wl_us = wl["us_mean"] if wl else None
        lines.append(f"| {label} | {e['best']} | {e['us_mean']:.2f} | {e['pct_peak']:.1f} | "
                     f"{best_any[0]} {best_any[1][0]:.2f} | " +
                     (f"{wl_us:.2f} | {wl['pct_peak']:.1f} | {100 * min(e['us_mean'], best_any[1][0]) / wl_us:.1f}%"
                      if wl else "- | - | -") + " |")
    # counters: every probe ran the same sizes the same number of times, so the means per dispatch compare directly
    fetch = counter_means(os.path.join(run_dir, "pmc_FETCH_SIZE"), "FETCH_SIZE")
    write = counter_means(os.path.join(run_dir, "pmc_WRITE_SIZE"), "WRITE_SIZE")
    occ_dir = os.path.join(run_dir, "occ_probes")
    occ = occupancy(occ_dir if os.path.isdir(occ_dir) else os.path.join(run_dir, "occ"))
    with open(TRAFFIC_PATH) as f:
        tr = json.load(f)
    sizes_b = [e["bytes"] for lab, e in ceil.items() if lab != "topk_128x128256"]
    copy_half = sum(sizes_b) / len(sizes_b) / 2 / 1024
    lines += ["", "## Counters of the ceiling probes (means per dispatch over the five copy sizes; the read probe over "
              "the top-k input)", "",
              f"FETCH_SIZE scaled by {tr['fetch_scale']} and WRITE_SIZE by {tr['write_scale']} (profiles/traffic.json"
              f" calibration); the copy probes' mean algorithmic bytes each way: {copy_half:.0f} KiB.", "",
              "| kernel | FETCH KiB (scaled) | WRITE KiB | read / algorithmic | resident waves per CU | occupancy % | "
              "VALU per wave | SALU per wave |", "|---|---|---|---|---|---|---|---|"]
    for kernel, f_kib in fetch.items():
        if "probe" in kernel or not any(t in kernel for t in ("copy_", "read_", "write_")):
            continue
        sk = short_kernel(kernel)
        f_scaled = f_kib * tr["fetch_scale"]
        algo = copy_half if sk.startswith("copy_") else 128 * 128256 * 4 / 1024
        o = occ.get(kernel, {})
        lines.append(f"| {sk} | {f_scaled:.0f} | {write.get(kernel, 0):.0f} | {f_scaled / algo:.3f} | "
                     f"{o.get('resident_waves_per_cu', '-')} | {o.get('occupancy_pct', '-')} | "
                     f"{o.get('valu_per_wave', '-')} | {o.get('salu_per_wave', '-')} |")
    path = os.path.join(ROOT, "profiles", "probe_ceiling_and_structures.txt")
    with open(path, "w") as f:
        f.write("\n".join(lines) + "\n")
    print("\n".join(lines))


def main():
    args = parse()
    if args.traffic_from:
        traffic_from(args.traffic_from)
        return
    if args.profile_summary:
        profile_summary(args.profile_summary)
        return
    if args.build_probes:
        print(build_probes())
        return
    if args.build_topk_stages:
        print(build_topk_stages())
        return
    if args.probe_summary:
        probe_summary(args.probe_summary, args.summary_bench)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}); "
              "run it with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if args.copy_calibration:
        copy_calibration(args.steps)
        return
    import torch
    from __graft_entry__ import load_package
    pkg = load_package()
    for spec in args.tune:  # op:slot=value, through the op library's tuning hook (sweeps and A/B runs)
        op, _, rest = spec.partition(":")
        slot, _, value = rest.partition("=")
        rc = getattr(pkg.candidate(op)._lib, f"{op}_tune")(int(slot), int(value))
        if rc != 0:
            raise SystemExit(f"--tune {spec}: the {op} library refused slot {slot}")
        print(f"[tune] {op} slot {slot} = {value}", file=sys.stderr, flush=True)
    if args.ceiling:
        ceiling(pkg, args.steps, args.warmup)
        return
    if args.topk_stages:
        print("\n".join(topk_stages()), flush=True)
        return
    if args.probes:
        probe_sweep(pkg, args.steps, args.warmup)
        return
    dev = torch.device("cuda:0")
    flush_buf = None if args.no_cold else torch.empty(FLUSH_BYTES // 4, dtype=torch.float32, device=dev).fill_(1.0)
    sink = torch.empty((), device=dev)

    def flush():
        torch.sum(flush_buf, dim=0, out=sink)

    names = [args.workload] if args.workload else list(pkg.workloads.WORKLOADS)
    cases = []
    for name in names:
        if name.startswith("topk") and not name.startswith("topk_sample"):
            cases += [(name, k) for k in ([args.k] if args.k else (1, 50, 1024))]
        else:
            cases.append((name, None))
    results = {}
    for name, k in cases:
        case = Case(pkg, name, dev, k)
        print(f"[bench] {case.label}: {args.warmup} warm-up + {args.steps} timed launches over {case.copies} copies",
              file=sys.stderr, flush=True)
        res = time_rotating(case, args.steps, args.warmup)
        if not args.no_cold:
            res.update(time_cold(case, args.steps, flush))
        results[case.label] = res
        print(f"[bench] {case.label}: {res['us_mean']:.2f} us/call  {res['gbs']:.0f} GB/s  "
              f"{res['pct_peak']:.1f}% of peak" +
              (f"  (single flushed launch: median {res['cold_us_median']:.2f} us)" if not args.no_cold else ""),
              file=sys.stderr, flush=True)
        del case
        torch.cuda.empty_cache()

    head = HEADLINE if HEADLINE in results else next(iter(results))
    hr = results[head]
    line = {
        "metric": METRIC, "value": round(hr["gbs"], 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(hr["us_mean"] / 1e3, 6), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16" if head.startswith(("rmsnorm", "rope")) else "fp32",
        "data": "synthetic: seeded torch.Generator inputs of the named shapes (workloads.py), resident in HBM; "
                "timed launches rotate over copies larger than the caches",
        "config": {"workload": head, "us_per_call": round(hr["us_mean"], 3), "pct_of_peak": round(hr["pct_peak"], 2),
                   "algorithmic_bytes": hr["bytes"], "copies": hr["copies"]},
        "roofline": roofline_entry(hr, head),
        "cpu_baseline": None,
        "per_workload": {lab: {key: (round(v, 3) if isinstance(v, float) else v) for key, v in r.items()
                               if key not in ("wall_s", "bytes")}
                         for lab, r in results.items()},
    }
    if not args.no_cpu:
        # the reference's CPU path beside every GPU figure, sharing one bounded budget of host time
        each = args.cpu_seconds / max(1, len(cases))
        for name, k in cases:
            label = name if k is None else f"{name}_k{k}"
            print(f"[bench] CPU baseline {label} (torch path on the host cores)", file=sys.stderr, flush=True)
            cpu = cpu_leg(pkg, name, k, each)
            line["per_workload"][label]["cpu"] = cpu
            if label == head:
                line["cpu_baseline"] = {key: cpu[key] for key in ("value", "unit", "cores", "kind", "sample")}
    print(json.dumps(line))


if __name__ == "__main__":
    main()
