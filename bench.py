"""Benchmark of the row-wise kernels on one MI355X: per-kernel us/call and achieved HBM GB/s against the 8 TB/s peak.

    python bench.py [--steps K] [--warmup W] [--workload NAME] [--all] [--warm] [--no-cpu]

A step is one launch of the op over its whole workload with the inputs already resident in HBM. Before every timed
step the 256 MB Infinity Cache and the L2s are flushed by reading a 1 GiB buffer (reads leave no dirty lines, so the
timed launch pays for no write-back of the flush), then the launch is bracketed by HIP events recorded on the stream it
runs on (torch's current stream, which the C-ABI is handed). The K durations give the mean (reported as ms_per_step
and used for `value`), median, p10 and p90. `value` = algorithmic bytes / mean duration: every input element read once
and every output element written once (workloads.algorithmic_bytes).

The JSON line is printed for the headline workload (RMSNorm bf16 [16384, 4096] with weight); `per_workload` carries
the other named workloads measured the same way (--all, the default, or just the headline with --workload). The CPU
baseline times the reference's PyTorch path for the headline on this host's cores (oracle/torch_paths, test
infrastructure used here only as the timed baseline) on a bounded sample of rows.
"""

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "per-kernel µs/call + achieved HBM GB/s (% of MI355X peak) at named shape, 1 GPU"
PEAK_GBS = 8000.0
HEADLINE = "rmsnorm_16384x4096"
FLUSH_BYTES = 1 << 30


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=100)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--workload", default=None, help="measure only this workload (default: all)")
    p.add_argument("--all", action="store_true", help="measure every named workload (the default)")
    p.add_argument("--warm", action="store_true", help="also time back-to-back launches without flushing")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    return p.parse_args()


class Case:
    """One workload bound to device tensors: `launch()` runs the op once; `kernel` names the dominant kernel."""

    def __init__(self, pkg, name, dev, k=None):
        import torch
        self.name, self.k = name, k
        w = pkg.workloads
        self.bytes = w.algorithmic_bytes(name, k or 50)
        inp = w.WORKLOADS[name]()
        if name.startswith("softmax"):
            x = inp["x"].to(dev)
            y = torch.empty_like(x)
            lib = pkg.candidate("softmax")._lib
            rows, cols = x.shape
            self.launch = lambda: lib.launch(x.data_ptr(), y.data_ptr(), rows, cols, 0, 256, 1024,
                                             torch.cuda.current_stream().cuda_stream)
            self.dtype = "fp32"
        elif name.startswith("rmsnorm"):
            x, wt = inp["x"].to(dev), inp["weight"].to(dev)
            y = torch.empty_like(x)
            lib = pkg.candidate("rmsnorm")._lib
            rows, cols = x.shape
            eps = inp["eps"]
            self.launch = lambda: lib.rmsnorm_launch_weighted(x.data_ptr(), wt.data_ptr(), y.data_ptr(), rows, cols, 1,
                                                              eps, 256, torch.cuda.current_stream().cuda_stream)
            self.dtype = "bf16"
        elif name.startswith("rope"):
            q, kk = inp["q"].to(dev), inp["k"].to(dev)
            pos, inv = inp["position_ids"].to(dev), inp["inv_freq"].to(dev)
            lib = pkg.candidate("rope")._lib
            B, S, Hq, D = q.shape
            # in place: every call rotates the same buffers again (the traffic is the same every time)
            self.launch = lambda: lib.rope_launch_freq(q.data_ptr(), kk.data_ptr(), pos.data_ptr(), inv.data_ptr(),
                                                       q.data_ptr(), kk.data_ptr(), B * S, Hq, kk.shape[2], D, 1,
                                                       torch.cuda.current_stream().cuda_stream)
            self.dtype = "bf16"
        elif name.startswith("topk"):
            cand = pkg.candidate("topk")
            x = inp["x"].to(dev)
            rows, cols = x.shape
            _, chunk, work_ptr, counters_ptr, _, _ = cand._plan(x, rows, cols, 0, k)
            vals = torch.empty(rows, k, device=dev)
            idx = torch.empty(rows, k, dtype=torch.int64, device=dev)
            lib = cand._lib
            self.launch = lambda: lib.launch(x.data_ptr(), vals.data_ptr(), idx.data_ptr(), work_ptr, counters_ptr,
                                             rows, cols, k, 0, cand._THREADS, cand._DEPTH, chunk,
                                             torch.cuda.current_stream().cuda_stream)
            self.dtype = "fp32"
        else:
            raise KeyError(name)
        self.inputs = inp

    @property
    def label(self):
        return self.name if self.k is None else f"{self.name}_k{self.k}"


def time_case(case, steps, warmup, flush, warm):
    import torch
    for _ in range(warmup):
        assert case.launch() == 0
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        flush()
        starts[i].record()
        err = case.launch()
        ends[i].record()
        if err:
            raise RuntimeError(f"{case.label}: launch returned {err}")
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    us = sorted(s.elapsed_time(e) * 1e3 for s, e in zip(starts, ends))
    mean = sum(us) / len(us)
    out = {"us_mean": mean, "us_median": us[len(us) // 2], "us_p10": us[len(us) // 10],
           "us_p90": us[(9 * len(us)) // 10], "bytes": case.bytes, "wall_s": wall}
    out["gbs"] = case.bytes / (mean * 1e-6) / 1e9
    out["pct_peak"] = 100.0 * out["gbs"] / PEAK_GBS
    if warm:
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(steps):
            case.launch()
        b.record()
        torch.cuda.synchronize()
        wus = a.elapsed_time(b) * 1e3 / steps
        out["warm_us"] = wus
        out["warm_gbs"] = case.bytes / (wus * 1e-6) / 1e9
    return out


def cpu_baseline(pkg, seconds):
    """The reference's PyTorch path for the headline (x * rsqrt(mean(x^2) + eps).to(bf16), then weight *) on this
    host's cores, on a bounded sample of rows, reported in the metric's unit."""
    import torch
    from oracle import torch_paths
    torch.set_num_threads(os.cpu_count() or 1)
    inp = pkg.workloads.rmsnorm_16384x4096()
    rows = 2048
    x, w, eps = inp["x"][:rows].contiguous(), inp["weight"], inp["eps"]
    nbytes = 2 * x.numel() * 2 + w.numel() * 2
    for _ in range(2):
        torch_paths.rmsnorm(x, w, eps)
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < 10:
        t = time.perf_counter()
        torch_paths.rmsnorm(x, w, eps)
        times.append(time.perf_counter() - t)
    times.sort()
    med = times[len(times) // 2]
    return {"value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"{rows} of 16384 rows (x[{rows}, 4096] bf16 + weight), median of {len(times)} calls of the "
                      f"torch path after 2 warm-ups, {med * 1e3:.2f} ms/call; cpu_count={os.cpu_count()}"}


def roofline_entry(res, label):
    traffic = None
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(path):
        with open(path) as f:
            traffic = json.load(f).get(label, {}).get("bytes_per_launch")
    return {"bound": "hbm", "achieved": round(res["gbs"], 1), "peak": PEAK_GBS, "unit": "GB/s",
            "frac": round(res["gbs"] / PEAK_GBS, 4), "traffic": traffic}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}); "
              "run it with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch
    from __graft_entry__ import load_package
    pkg = load_package()
    dev = torch.device("cuda:0")
    flush_buf = torch.empty(FLUSH_BYTES // 4, dtype=torch.float32, device=dev).fill_(1.0)
    sink = torch.empty((), device=dev)

    def flush():
        torch.sum(flush_buf, dim=0, out=sink)

    names = [args.workload] if args.workload else list(pkg.workloads.WORKLOADS)
    cases = []
    for name in names:
        if name.startswith("topk"):
            if not os.path.exists(pkg.lib_path("topk")):
                continue
            cases += [(name, k) for k in (1, 50, 1024)]
        else:
            cases.append((name, None))
    results = {}
    for name, k in cases:
        case = Case(pkg, name, dev, k)
        print(f"[bench] {case.label}: {args.warmup} warm-up + {args.steps} timed launches", file=sys.stderr, flush=True)
        res = time_case(case, args.steps, args.warmup, flush, args.warm)
        results[case.label] = res
        print(f"[bench] {case.label}: {res['us_mean']:.2f} us/call  {res['gbs']:.0f} GB/s  "
              f"{res['pct_peak']:.1f}% of peak" + (f"  (warm {res['warm_us']:.2f} us)" if args.warm else ""),
              file=sys.stderr, flush=True)
        del case
        torch.cuda.empty_cache()

    head = HEADLINE if HEADLINE in results else next(iter(results))
    hr = results[head]
    line = {
        "metric": METRIC, "value": round(hr["gbs"], 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(hr["us_mean"] / 1e3, 6), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16" if head.startswith(("rmsnorm", "rope")) else "fp32",
        "data": "synthetic: seeded torch.Generator inputs of the named shapes (workloads.py), resident in HBM; "
                "L2 and Infinity Cache flushed before every timed launch",
        "config": {"workload": head, "us_per_call": round(hr["us_mean"], 3), "us_median": round(hr["us_median"], 3),
                   "pct_of_peak": round(hr["pct_peak"], 2), "algorithmic_bytes": hr["bytes"]},
        "roofline": roofline_entry(hr, head),
        "cpu_baseline": None,
        "per_workload": {k: {"us_mean": round(v["us_mean"], 3), "us_median": round(v["us_median"], 3),
                             "us_p10": round(v["us_p10"], 3), "us_p90": round(v["us_p90"], 3),
                             "gbs": round(v["gbs"], 1), "pct_peak": round(v["pct_peak"], 2),
                             **({"warm_us": round(v["warm_us"], 3), "warm_gbs": round(v["warm_gbs"], 1)}
                                if "warm_us" in v else {})}
                         for k, v in results.items()},
    }
    if not args.no_cpu and head == HEADLINE:
        print("[bench] CPU baseline (torch path on the host cores)", file=sys.stderr, flush=True)
        line["cpu_baseline"] = cpu_baseline(pkg, args.cpu_seconds)
    print(json.dumps(line))


if __name__ == "__main__":
    main()
