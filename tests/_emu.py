"""Builds a kernel source file from the package's csrc/ as a CPU program under the HIP emulation in tests/emu/.

The source is compiled as the library builds it, except that its inline asm statements (scheduling fences and waits
for the memory counters, which have no meaning on the CPU) become no-ops. It is linked with a driver from tests/emu/
and the oracle's C restatement, which the driver compares the kernels' outputs with.
"""

import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(ROOT, "cuda-kernels-optimized-for-rtx5090_amd", "csrc")
EMU = os.path.join(HERE, "emu")


def _clang():
    for cand in ("/opt/rocm/llvm/bin/clang++", shutil.which("clang++")):
        if cand and os.path.exists(cand):
            return cand
    return None


def build(tmpdir, source, driver):
    """Compiles csrc/<source> with tests/emu/<driver> and oracle/oracle.c into an executable; returns its path."""
    clang = _clang()
    if clang is None or shutil.which("gcc") is None:
        pytest.skip("clang++ (for the kernels' vector extensions on the host) or gcc is missing")
    stem = os.path.splitext(source)[0]
    with open(os.path.join(CSRC, source)) as f:
        src = f.read().replace("asm volatile(", "EMU_ASM(")
    kern = os.path.join(str(tmpdir), stem + "_emu.cpp")
    with open(kern, "w") as f:
        f.write(src)
    obj = os.path.join(str(tmpdir), "oracle.o")
    if not os.path.exists(obj):
        subprocess.run(["gcc", "-O2", "-c", os.path.join(ROOT, "oracle", "oracle.c"), "-o", obj], check=True)
    exe = os.path.join(str(tmpdir), "emu_" + stem)
    proc = subprocess.run([clang, "-std=c++17", "-O1", "-U_FORTIFY_SOURCE", "-D_FORTIFY_SOURCE=0",
                           "-fno-strict-aliasing", "-w", "-pthread", "-I", EMU, "-I", CSRC, kern,
                           os.path.join(EMU, driver), obj, "-o", exe, "-lm"], capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr[-4000:]
    return exe


def run(exe, args, env=None, timeout=600, concurrent=False):
    """Runs the emulation with the given arguments and asserts that it reports ALL OK. concurrent: every workgroup on an
    OS thread of its own, all at once (EMU_CONCURRENT)."""
    env = dict(os.environ if env is None else env)
    env.pop("EMU_CONCURRENT", None)
    if concurrent:
        env["EMU_CONCURRENT"] = "1"
    proc = subprocess.run([exe, *[str(a) for a in args]], capture_output=True, text=True, timeout=timeout, env=env)
    out = proc.stdout + proc.stderr
    assert proc.returncode == 0 and "ALL OK" in proc.stdout, f"{args}: rc {proc.returncode}\n{out[-3000:]}"
