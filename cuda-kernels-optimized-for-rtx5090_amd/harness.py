"""Harness for the four ops, in the shape of the reference's optimization reports (softmax/README.md:1-12 and the
other ops' READMEs): each workload is run through the op's candidate wrapper (`run(inputs)`, with the op's
params.json), the PyTorch GPU path the reference calls its baseline, and the op's naive kernel (the "seed": this
build's scalar tier, forced through the tuning hook); correctness is checked against an fp64 (or exact) reference
computed here, for the seed's output too, and a Markdown table is printed:

    | workload | correctness | timing | candidate ms | baseline ms | seed ms | vs baseline | vs seed | dtype |

    python cuda-kernels-optimized-for-rtx5090_amd/harness.py [--op softmax|rmsnorm|rope|topk|all] [--quick] [--json]

Timing: the median of `--reps` launches, each after a 1 GiB read that evicts the caches, between HIP events on the
current stream (an isolated launch: it includes the dispatch latency, for all three columns alike). "timing" is PASS
when the candidate is not slower than the baseline. The workloads are the reference READMEs' (hidden size 4096 for
RMSNorm and Llama-style 32 q / 8 kv heads of 128 for RoPE, which those READMEs do not state), or with --quick one
small workload per op and dtype.

Correctness (the reference ships no harness; these are this build's bars): softmax within 1e-5 relative of the fp64
softmax (fp32) or 1 ulp of it (bf16); RMSNorm within 2 ulp of torch's expression x * rsqrt(mean(x^2) + eps) on the
dtype (inv may round one ulp apart); RoPE within 1 ulp of torch eager's x * cos + rotate_half(x) * sin over the same
cache; top-k values equal to torch.topk's and indices equal wherever the value is unique in its row.
"""

import argparse
import importlib.util
import json
import os
import sys

import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def _package():
    name = "ck5090_amd"
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(name, os.path.join(HERE, "__init__.py"),
                                                  submodule_search_locations=[HERE])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


DT = {"fp32": torch.float32, "bf16": torch.bfloat16, "fp16": torch.float16}


def _ordered(t):
    """16-bit float bits mapped to integers in value order (adjacent values differ by 1)."""
    a = t.contiguous().view(torch.int16).to(torch.int32)
    return torch.where(a < 0, -32768 - a, a)


def _ulps(a, b):
    return (_ordered(a) - _ordered(b)).abs()


# ---- workloads ----------------------------------------------------------------------------------------------------


def softmax_workloads(quick):
    shapes = [(256, 1024)] if quick else [(4096, 1024), (4096, 8192), (256, 262144)]
    for dt in ("fp32", "bf16"):
        for rows, cols in shapes:
            yield f"s{rows}x{cols}_{dt}", dt, (rows, cols)


def rmsnorm_workloads(quick):
    rows_list = [64] if quick else [1, 1024, 32768]
    for dt in ("bf16", "fp16"):
        for rows in rows_list:
            yield f"s{rows}_{dt}", dt, (rows, 4096)


def rope_workloads(quick):
    shapes = [("decode_b4", 4, 1)] if quick else [("decode_b1", 1, 1), ("decode_b16", 16, 1), ("decode_b64", 64, 1),
                                                  ("prefill_s512", 1, 512), ("prefill_s2048", 1, 2048),
                                                  ("prefill_s8192", 1, 8192)]
    for dt in ("bf16", "fp16"):
        for name, b, s in shapes:
            yield f"{name}_{dt}", dt, (b, s)


def topk_workloads(quick):
    shapes = [(8, 32000)] if quick else [(1, 128256), (64, 151936), (512, 32000)]
    for dt in ("fp32", "bf16"):
        for rows, cols in shapes:
            yield f"s{rows}x{cols}_{dt}", dt, (rows, cols)


# ---- per-op cases: inputs, candidate, baseline, seed, check ----------------------------------------------------------


class Case:
    def __init__(self, pkg, op, dt, shape, dev):
        self.pkg, self.op, self.dt, self.dev = pkg, op, DT[dt], dev
        g = torch.Generator().manual_seed(hash((op, dt, shape)) & 0xFFFF)
        if op == "softmax":
            self.inputs = {"x": (torch.randn(*shape, generator=g) * 3).to(self.dt).to(dev)}
        elif op == "rmsnorm":
            self.inputs = {"x": torch.randn(*shape, generator=g).to(self.dt).to(dev), "eps": 1e-6}
        elif op == "rope":
            b, s = shape
            self.inputs = {"q": torch.randn(b, s, 32, 128, generator=g).to(self.dt).to(dev),
                           "k": torch.randn(b, s, 8, 128, generator=g).to(self.dt).to(dev),
                           "position_ids": (torch.randint(0, 8192, (b, s), generator=g) if s == 1 else
                                            torch.arange(s).view(1, s).expand(b, s).contiguous()).to(dev)}
            inv = 1.0 / (10000.0 ** (torch.arange(0, 128, 2, dtype=torch.int64).float() / 128))
            emb = torch.cat([torch.outer(torch.arange(8192).float(), inv)] * 2, -1)
            self.inputs["cos"], self.inputs["sin"] = emb.cos().to(dev), emb.sin().to(dev)
        elif op == "topk":
            self.inputs = {"x": (torch.randn(*shape, generator=g) * 2).to(self.dt).to(dev), "k": 50}
        self.cand = pkg.candidate(op)

    def candidate(self):
        return self.cand.run(self.inputs)

    def baseline(self):
        i = self.inputs
        if self.op == "softmax":
            return {"y": torch.softmax(i["x"], dim=-1)}
        if self.op == "rmsnorm":
            x = i["x"]
            return {"y": x * torch.rsqrt(x.float().pow(2).mean(-1, keepdim=True) + i["eps"]).to(x.dtype)}
        if self.op == "rope":
            cos, sin = i["cos"][i["position_ids"]].unsqueeze(2), i["sin"][i["position_ids"]].unsqueeze(2)

            def rot(x):
                xf = x.float()
                half = torch.cat((-xf[..., 64:], xf[..., :64]), -1)
                return (xf * cos + half * sin).to(x.dtype)
            return {"q_out": rot(i["q"]), "k_out": rot(i["k"])}
        v, ix = torch.topk(i["x"], i["k"], dim=-1)
        return {"values": v, "indices": ix}

    def seed(self):
        """The naive scalar tier of this build (None when the op has none)."""
        slot = {"softmax": (5, 3), "rmsnorm": (3, 1), "rope": (2, 1), "topk": (1, 1)}.get(self.op)
        if slot is None:
            return None
        tune = getattr(self.cand._lib, f"{self.op}_tune")
        tune(*slot)
        try:
            return self.cand.run(self.inputs)
        finally:
            tune(slot[0], 0)

    def check(self, out):
        i = self.inputs
        if self.op == "softmax":
            ref = torch.softmax(i["x"].double(), dim=-1)
            y = out["y"]
            if y.dtype == torch.float32:
                return bool(((y.double() - ref).abs() <= 1e-5 * ref.abs()).all())
            return bool((_ulps(y, ref.to(y.dtype)) <= 1).all())
        if self.op == "rmsnorm":
            return bool((_ulps(out["y"], self.baseline()["y"]) <= 2).all())
        if self.op == "rope":
            base = self.baseline()
            return bool((_ulps(out["q_out"], base["q_out"]) <= 1).all() and
                        (_ulps(out["k_out"], base["k_out"]) <= 1).all())
        base = self.baseline()
        if not torch.equal(out["values"], base["values"]):
            return False
        vals = out["values"]
        unique = torch.ones_like(vals, dtype=torch.bool)
        unique[:, 1:] &= vals[:, 1:] != vals[:, :-1]
        unique[:, :-1] &= vals[:, :-1] != vals[:, 1:]
        return bool(torch.equal(out["indices"][unique], base["indices"][unique]))


def time_ms(fn, reps, flush):
    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    times = []
    for _ in range(reps):
        flush()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        fn()
        b.record()
        torch.cuda.synchronize()
        times.append(a.elapsed_time(b))
    times.sort()
    return times[len(times) // 2]


WORKLOADS = {"softmax": softmax_workloads, "rmsnorm": rmsnorm_workloads, "rope": rope_workloads,
             "topk": topk_workloads}


def run(ops=("softmax", "rmsnorm", "rope", "topk"), quick=False, reps=20):
    """Runs the workloads of `ops`; returns one dict per row of the report."""
    pkg = _package()
    dev = torch.device("cuda:0")
    flush_buf = torch.ones(1 << 28, device=dev)
    sink = torch.empty((), device=dev)

    def flush():
        torch.sum(flush_buf, dim=0, out=sink)

    rows = []
    for op in ops:
        for name, dt, shape in WORKLOADS[op](quick):
            case = Case(pkg, op, dt, shape, dev)
            ok = case.check(case.candidate())
            seed_out = case.seed()
            seed_ok = seed_out is None or case.check(seed_out)
            cand = time_ms(case.candidate, reps, flush)
            base = time_ms(case.baseline, reps, flush)
            seed = time_ms(case.seed, reps, flush) if seed_out is not None else None
            correct = ("PASS" if seed_ok else "FAIL (seed)") if ok else "FAIL"
            rows.append({"op": op, "workload": name, "correctness": correct,
                         "timing": "PASS" if cand <= base else "FAIL", "candidate_ms": cand, "baseline_ms": base,
                         "seed_ms": seed, "dtype": dt})
            del case
            torch.cuda.empty_cache()
    return rows


def _fmt(v):
    return "n/a" if v is None else f"{v:.4g}"


def table(rows):
    lines = []
    for op in dict.fromkeys(r["op"] for r in rows):
        lines += [f"## {op}", "", "Speedup = reference time / incumbent time; below 1.0 is a slowdown.", "",
                  "| workload | correctness | timing | candidate ms | baseline ms | seed ms | vs baseline | vs seed | "
                  "dtype |", "|---|---|---|---|---|---|---|---|---|"]
        for r in (r for r in rows if r["op"] == op):
            vb = r["baseline_ms"] / r["candidate_ms"]
            vs = None if r["seed_ms"] is None else r["seed_ms"] / r["candidate_ms"]
            mark = lambda s: "n/a" if s is None else (f"{s:.4g}" + (" (slowdown)" if s < 1 else ""))  # noqa: E731
            lines.append(f"| {r['workload']} | {r['correctness']} | {r['timing']} | {_fmt(r['candidate_ms'])} | "
                         f"{_fmt(r['baseline_ms'])} | {_fmt(r['seed_ms'])} | {mark(vb)} | {mark(vs)} | {r['dtype']} |")
        lines.append("")
    return "\n".join(lines)


def main(argv=None):
    p = argparse.ArgumentParser()
    p.add_argument("--op", default="all", choices=["all", "softmax", "rmsnorm", "rope", "topk"])
    p.add_argument("--quick", action="store_true", help="one small workload per op and dtype")
    p.add_argument("--reps", type=int, default=20)
    p.add_argument("--json", action="store_true", help="print the rows as JSON instead of the Markdown table")
    a = p.parse_args(argv)
    ops = ("softmax", "rmsnorm", "rope", "topk") if a.op == "all" else (a.op,)
    rows = run(ops, a.quick, a.reps)
    print(json.dumps(rows) if a.json else table(rows))
    return 0 if all(r["correctness"] == "PASS" for r in rows) else 1


if __name__ == "__main__":
    sys.exit(main())
