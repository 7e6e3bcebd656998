"""Builds one `libkernel.so` per op from csrc/<op>.hip for gfx950 with hipcc, into build/<op>/, and the PyTorch-ROCm
operators over them (csrc/torch_ops.cpp, torch.ops.ckopt.*) into build/torch/libckopt_torch.so.

Each op library exports the reference's C-ABI for its op (`launch`, and `plan` for top-k) plus the extensions declared
in include/<op>.h, so a harness that loads `$CKOPT_BUILD_DIR/libkernel.so` can point CKOPT_BUILD_DIR at build/<op>.

    python make_libs.py            # build every op and the torch operators
    python make_libs.py softmax    # build some (torch: the operators)
"""

import concurrent.futures
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIBS = ("softmax", "rmsnorm", "rope", "topk")
TORCH = "torch"  # the torch operators over the op libraries
ARCH = os.environ.get("ROWKERN_ARCH", "gfx950")

# -packed-fp32-ops: no v_pk_{add,mul,fma}_f32 (some of their forms are unreliable on this part); hipcc's host pass
# warns that it does not know the feature, which is harmless.
HIPCC_FLAGS = [
    "--offload-arch=" + ARCH, "-O3", "-std=c++17", "-fPIC", "-shared",
    "-ffp-contract=off", "-fno-gpu-rdc",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]

# Per-op additions. topk: no wave-level atomic optimizer: every atomic of the top-k kernels (the arrival counts, the
# LDS list reservations) is issued by one lane already, and the optimizer's scan and broadcast around it would only
# add instructions and waits.
OP_FLAGS = {"topk": ["-mllvm", "-amdgpu-atomic-optimizer-strategy=None"]}


def hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if cand and (os.path.sep not in cand or os.path.exists(cand)):
            return cand
    raise RuntimeError("hipcc not found")


def lib_path(op):
    return os.path.join(HERE, "build", op, "libkernel.so")


def torch_lib_path():
    return os.path.join(HERE, "build", TORCH, "libckopt_torch.so")


def build_torch_ops():
    """csrc/torch_ops.cpp against the installed PyTorch-ROCm (its headers and libraries), with the host compiler: the
    operators hold no device code of their own, they call the op libraries."""
    import torch
    from torch.utils import cpp_extension
    out = torch_lib_path()
    os.makedirs(os.path.dirname(out), exist_ok=True)
    tmp = out + ".tmp"
    torch_lib = os.path.join(os.path.dirname(torch.__file__), "lib")
    cmd = [os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-fPIC", "-shared", "-D__HIP_PLATFORM_AMD__=1",
           "-DUSE_ROCM=1", f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}",
           *[f"-I{p}" for p in cpp_extension.include_paths(device_type="cuda")], "-I", os.path.join(HERE, "..", "include"),
           os.path.join(CSRC, "torch_ops.cpp"), f"-L{torch_lib}", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu",
           "-ltorch_hip", f"-Wl,-rpath,{torch_lib}", "-ldl", "-o", tmp]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"the torch operators failed to build ({proc.returncode}):\n" + proc.stderr[-6000:])
    os.replace(tmp, out)
    return TORCH, out, ""


def build_one(op):
    if op == TORCH:
        return build_torch_ops()
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


def build(ops=LIBS + (TORCH,), jobs=4):
    """Compiles the given ops; returns {op: path}. Raises RuntimeError on a compiler error."""
    results = {}
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        for op, out, log in pool.map(build_one, ops):
            results[op] = out
            if log.strip():
                print(f"[build {op}] {log}", file=sys.stderr)
    return results


if __name__ == "__main__":
    ops = sys.argv[1:] or LIBS + (TORCH,)
    for op, path in build(ops).items():
        print(op, path)
