"""Builds one `libkernel.so` per op from csrc/<op>.hip for gfx950 with hipcc, into build/<op>/.

Each library exports the reference's C-ABI for its op (`launch`, and `plan` for top-k) plus the extensions declared in
include/<op>.h, so a harness that loads `$CKOPT_BUILD_DIR/libkernel.so` can point CKOPT_BUILD_DIR at build/<op>.

    python make_libs.py            # build every op
    python make_libs.py softmax    # build some
"""

import concurrent.futures
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIBS = ("softmax", "rmsnorm", "rope", "topk", "probe")  # the four ops and the bandwidth probes of bench.py --ceiling
ARCH = os.environ.get("ROWKERN_ARCH", "gfx950")

# -packed-fp32-ops: no v_pk_{add,mul,fma}_f32 (some of their forms are unreliable on this part); hipcc's host pass
# warns that it does not know the feature, which is harmless.
HIPCC_FLAGS = [
    "--offload-arch=" + ARCH, "-O3", "-std=c++17", "-fPIC", "-shared",
    "-ffp-contract=off", "-fno-gpu-rdc",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]

# Per-op additions. topk: no wave-level atomic optimizer, which turns the start-order count (an atomic by one lane,
# issued first thing in the k <= 64 kernel) into a broadcast of its result that waits for the atomic before the tile's
# loads are issued.
OP_FLAGS = {"topk": ["-mllvm", "-amdgpu-atomic-optimizer-strategy=None"]}


def hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if cand and (os.path.sep not in cand or os.path.exists(cand)):
            return cand
    raise RuntimeError("hipcc not found")


def lib_path(op):
    return os.path.join(HERE, "build", op, "libkernel.so")


def build_one(op):
    src = os.path.join(CSRC, op + ".hip")
    out = lib_path(op)
    os.makedirs(os.path.dirname(out), exist_ok=True)
    tmp = out + ".tmp"
    cmd = [hipcc(), *HIPCC_FLAGS, *OP_FLAGS.get(op, []), "-I", CSRC, src, "-o", tmp]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    lines = [l for l in (proc.stdout + proc.stderr).splitlines() if "not a recognized feature" not in l]
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {op} ({proc.returncode}):\n" + "\n".join(lines))
    os.replace(tmp, out)
    return op, out, "\n".join(lines)


def build(ops=LIBS, jobs=4):
    """Compiles the given ops; returns {op: path}. Raises RuntimeError on a compiler error."""
    results = {}
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        for op, out, log in pool.map(build_one, ops):
            results[op] = out
            if log.strip():
                print(f"[build {op}] {log}", file=sys.stderr)
    return results


if __name__ == "__main__":
    ops = sys.argv[1:] or LIBS
    for op, path in build(ops).items():
        print(op, path)
