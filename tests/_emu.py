"""Builds a kernel source file from the package's csrc/ as a CPU program under the HIP emulation in tests/emu/.

The source is compiled as the library builds it, except that its inline asm statements (scheduling fences and waits
for the memory counters) go to the emulation's hook, where `s_waitcnt vmcnt(0)` makes the lane's pending stores
visible in the weak mode and everything else is a no-op. It is linked with a driver from tests/emu/
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
    kern = kernel_source(tmpdir, source)
    obj = os.path.join(str(tmpdir), "oracle.o")
    src = os.path.join(ROOT, "oracle", "oracle.c")
    if not os.path.exists(obj) or os.path.getmtime(obj) < os.path.getmtime(src):
        subprocess.run(["gcc", "-O2", "-c", src, "-o", obj], check=True)
    exe = os.path.join(str(tmpdir), "emu_" + stem)
    proc = subprocess.run([clang, "-std=c++17", "-O1", "-U_FORTIFY_SOURCE", "-D_FORTIFY_SOURCE=0",
                           "-fno-strict-aliasing", "-w", "-pthread", "-I", EMU, "-I", str(tmpdir), "-I", CSRC, kern,
                           os.path.join(EMU, driver), obj, "-o", exe, "-lm"], capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr[-4000:]
    return exe


def kernel_source(tmpdir, source):
    """csrc/<source> with its inline asm statements routed to the emulation's hook; returns the path of the copy. The
    csrc headers are copied beside it the same way (the copy's directory comes first on the include path)."""
    stem = os.path.splitext(source)[0]
    for name in os.listdir(CSRC):
        if name.endswith(".hpp"):
            with open(os.path.join(CSRC, name)) as f:
                text = f.read().replace("asm volatile(", "EMU_ASM(")
            with open(os.path.join(str(tmpdir), name), "w") as f:
                f.write(text)
    with open(os.path.join(CSRC, source)) as f:
        src = f.read().replace("asm volatile(", "EMU_ASM(")
    kern = os.path.join(str(tmpdir), stem + "_emu.cpp")
    with open(kern, "w") as f:
        f.write(src)
    return kern


def build_shared(tmpdir, source, name):
    """Compiles csrc/<source> alone into a shared object tmpdir/name (the emulation's runtime inside it)."""
    clang = _clang()
    if clang is None:
        pytest.skip("clang++ (for the kernels' vector extensions on the host) is missing")
    out = os.path.join(str(tmpdir), name)
    proc = subprocess.run([clang, "-std=c++17", "-O1", "-fPIC", "-shared", "-U_FORTIFY_SOURCE", "-D_FORTIFY_SOURCE=0",
                           "-fno-strict-aliasing", "-w", "-pthread", "-I", EMU, "-I", str(tmpdir), "-I", CSRC,
                           kernel_source(tmpdir, source), "-o", out], capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr[-4000:]
    return out


def build_driver(tmpdir, driver, libs=("-ldl",)):
    """Compiles tests/emu/<driver> with the oracle's C restatement (no kernel source) into an executable."""
    clang = _clang()
    if clang is None or shutil.which("gcc") is None:
        pytest.skip("clang++ or gcc is missing")
    obj = os.path.join(str(tmpdir), "oracle_pic.o")
    src = os.path.join(ROOT, "oracle", "oracle.c")
    if not os.path.exists(obj) or os.path.getmtime(obj) < os.path.getmtime(src):
        subprocess.run(["gcc", "-O2", "-fPIC", "-c", src, "-o", obj], check=True)
    exe = os.path.join(str(tmpdir), os.path.splitext(driver)[0])
    # -rdynamic: the emulation runtime's state (allocation count, schedules) is the driver's, shared by every library
    # the driver opens; each library keeps its own kernels and statics
    proc = subprocess.run([clang, "-std=c++17", "-O1", "-w", "-pthread", "-rdynamic", "-I", EMU,
                           os.path.join(EMU, driver), obj, "-o", exe, "-lm", *libs], capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr[-4000:]
    return exe


def run(exe, args, env=None, timeout=600, concurrent=False, weak=False, expect_ok=True):
    """Runs the emulation with the given arguments and asserts that it reports ALL OK (or, with expect_ok False, that
    it reports a failure). concurrent: every workgroup on an OS thread of its own, all at once (EMU_CONCURRENT). weak:
    agent-scope stores become visible late and out of order (EMU_WEAK)."""
    env = dict(os.environ if env is None else env)
    for var in ("EMU_CONCURRENT", "EMU_WEAK"):
        env.pop(var, None)
    if concurrent:
        env["EMU_CONCURRENT"] = "1"
    if weak:
        env["EMU_WEAK"] = "1"
    proc = subprocess.run([exe, *[str(a) for a in args]], capture_output=True, text=True, timeout=timeout, env=env)
    out = proc.stdout + proc.stderr
    if expect_ok:
        assert proc.returncode == 0 and "ALL OK" in proc.stdout, f"{args}: rc {proc.returncode}\n{out[-3000:]}"
    else:
        assert proc.returncode != 0 and "FAILED" in proc.stdout, f"{args}: expected a failure\n{out[-3000:]}"
    return out
