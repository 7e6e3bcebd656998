"""CPU checks of the drop-in boundary: every library loads and exports exactly the entry points include/<op>.h
declares, the argument checks return the reference's codes without touching a GPU, and the wrappers reject what the
reference's wrappers reject (with ValueError) before any launch.
"""

import ctypes
import os
import re
import subprocess

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
OPS = ("softmax", "rmsnorm", "rope", "topk")


def declared(op):
    text = open(os.path.join(ROOT, "include", op + ".h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"^\s*(?:int|long long)\s+(\w+)\s*\(", text, flags=re.M)


def exported(path):
    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if " T " in line}


@pytest.mark.parametrize("op", OPS)
def test_library_exports_the_header(pkg, op):
    path = pkg.lib_path(op)
    assert os.path.exists(path), f"{path} not built"
    lib = ctypes.CDLL(path)
    names = declared(op)
    assert "launch" in names
    for name in names:
        assert hasattr(lib, name), f"{op}: {name} declared in include/{op}.h but not exported"
    # nothing beyond the header is exported with C linkage
    c_symbols = {s for s in exported(path) if not s.startswith("_Z") and not s.startswith("_")}
    assert c_symbols == set(names), f"{op}: exported {sorted(c_symbols)} vs declared {sorted(names)}"


def test_probe_library_exports_and_codes_without_gpu():
    # the measurement's bandwidth probes (bench_probes.hip, bench.py --ceiling / --probes): a library of their own,
    # outside the package and the op boundary; argument checks answer before any launch
    import bench
    path = bench.PROBES_LIB
    assert os.path.exists(path), f"{path} not built"
    c_symbols = {s for s in exported(path) if not s.startswith("_Z") and not s.startswith("_")}
    assert c_symbols == {"probe_run"}
    lib = bench.probe_lib()
    stride, read, write = (bench.PROBE_FAMILIES[f] for f in ("stride", "read", "write"))
    assert lib.probe_run(stride, 4, 8, 2, 2, None, None, None, 0, None) == 0  # nothing to move
    assert lib.probe_run(stride, 4, 8, 2, 2, 16, 16, None, 24, None) == -1  # not whole 16-byte vectors
    assert lib.probe_run(stride, 4, 8, 2, 2, 16, 16, None, (1 << 30) + 16, None) == -1  # beyond 1 GiB
    assert lib.probe_run(stride, 3, 8, 2, 2, 16, 16, None, 32, None) == -1  # no such unroll
    assert lib.probe_run(stride, 4, 8, 1, 2, 16, 16, None, 32, None) == -1  # no such policy pair
    assert lib.probe_run(stride, 4, 0, 2, 2, 16, 16, None, 32, None) == -1  # blocks per CU out of range
    assert lib.probe_run(bench.PROBE_FAMILIES["row"], 4, 8, 0, 2, 16, 16, None, 32, None) == -1  # nt only
    assert lib.probe_run(read, 8, 8, 2, 2, 16, None, None, 32, None) == -1  # no sink
    assert lib.probe_run(write, 4, 8, 2, 2, None, None, None, 32, None) == -1  # nothing to write to
    assert lib.probe_run(99, 4, 8, 2, 2, 16, 16, 16, 32, None) == -1
    for spec in bench.CEILING_PROBES:
        bench.parse_probe(spec)


def test_topk_stage_build_is_separate(pkg):
    # the top-k stage stamps (bench.py --topk-stages) live in a build of their own: the op library exports none of
    # the read-out, the stage build exports the op library's entry points plus the read-out, and its read-out checks
    # its arguments before any copy
    import bench
    assert os.path.exists(bench.STAGES_LIB), f"{bench.STAGES_LIB} not built"
    op = {s for s in exported(pkg.lib_path("topk")) if not s.startswith("_")}
    staged = {s for s in exported(bench.STAGES_LIB) if not s.startswith("_")}
    assert not any(s.startswith("topk_stages") for s in op)
    assert staged == op | {"topk_stages_read", "topk_stages_clear"}
    lib = ctypes.CDLL(bench.STAGES_LIB)
    lib.topk_stages_read.argtypes = [ctypes.c_void_p, ctypes.c_longlong]
    assert lib.topk_stages_read(None, 8) == -1
    assert lib.topk_stages_read(ctypes.c_void_p(16), (bench.STAGE_WGS * bench.STAGE_SLOTS + 1) * 8) == -1


def test_softmax_codes_without_gpu(pkg):
    lib = ctypes.CDLL(pkg.lib_path("softmax"))
    assert lib.launch(None, None, ctypes.c_longlong(0), ctypes.c_longlong(5), 0, 256, 1024, None) == 0
    assert lib.launch(None, None, ctypes.c_longlong(5), ctypes.c_longlong(0), 0, 256, 1024, None) == 0
    assert lib.launch(None, None, ctypes.c_longlong(5), ctypes.c_longlong(5), 2, 256, 1024, None) == -1
    assert lib.softmax_tune(99, 1) == -1 and lib.softmax_tune(0, 0) == 0


def test_rmsnorm_codes_without_gpu(pkg):
    lib = ctypes.CDLL(pkg.lib_path("rmsnorm"))
    lib.launch.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_longlong, ctypes.c_int, ctypes.c_int,
                           ctypes.c_float, ctypes.c_int, ctypes.c_void_p]
    assert lib.launch(None, None, 0, 8, 1, 1e-6, 256, None) == 0          # no rows: no-op
    assert lib.launch(None, None, 1 << 31, 8, 1, 1e-6, 256, None) == -1   # rows beyond int32
    assert lib.launch(None, None, 4, 0, 1, 1e-6, 256, None) == -1         # cols
    assert lib.launch(None, None, 4, 8, 1, 1e-6, 48, None) == -1          # threads not a multiple of 32
    assert lib.launch(None, None, 4, 8, 1, 1e-6, 2048, None) == -1        # threads > 1024
    assert lib.launch(None, None, 4, 8, 0, 1e-6, 256, None) == -1         # fp32 is not served
    lib.rmsnorm_launch_weighted.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_longlong, ctypes.c_int, ctypes.c_int,
                                                                     ctypes.c_float, ctypes.c_int, ctypes.c_void_p]
    assert lib.rmsnorm_launch_weighted(None, 1, None, 4, 8, 3, 1e-6, 256, None) == -1
    assert lib.rmsnorm_launch_weighted(None, 1, None, 0, 8, 1, 1e-6, 256, None) == 0


def test_rope_codes_without_gpu(pkg):
    lib = ctypes.CDLL(pkg.lib_path("rope"))
    lib.launch.argtypes = [ctypes.c_void_p] * 7 + [ctypes.c_longlong] + [ctypes.c_int] * 7 + [ctypes.c_void_p]
    n = [None] * 7
    assert lib.launch(*n, 0, 1, 1, 128, 1, 0, 40, 1, None) == 0
    assert lib.launch(*n, 1 << 31, 1, 1, 128, 1, 0, 40, 1, None) == -1
    assert lib.launch(*n, 4, 1, 1, 127, 1, 0, 40, 1, None) == -1
    assert lib.launch(*n, 4, 1, 0, 128, 1, 0, 40, 1, None) == -1
    assert lib.launch(*n, 4, 1, 1, 128, 0, 0, 40, 1, None) == -1
    assert lib.launch(*n, 4, 1, 1, 128, 1, 3, 40, 1, None) == -1
    assert lib.launch(*n, 4, 1, 1, 128, 1, 0, 40, 0, None) == -1


def test_wrappers_reject_bad_inputs_before_launch(pkg):
    with pytest.raises(ValueError):
        pkg.softmax(torch.zeros(4, 4, dtype=torch.float64))
    with pytest.raises(ValueError):
        pkg.softmax(torch.zeros(4, 4))  # a CPU tensor: no CPU path
    with pytest.raises(ValueError):
        pkg.rmsnorm(torch.zeros(4, 8))  # fp32 is not an RMSNorm dtype of the reference
    with pytest.raises(ValueError):
        pkg.rmsnorm(torch.zeros(4, 8, dtype=torch.bfloat16))
    q = torch.zeros(1, 2, 2, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        pkg.rope(q, q, torch.zeros(1, 2, dtype=torch.int32), cos=torch.zeros(4, 64), sin=torch.zeros(4, 64))
    with pytest.raises(ValueError):
        pkg.rope(q, q, torch.zeros(1, 2, dtype=torch.int64), cos=torch.zeros(4, 64), sin=torch.zeros(4, 64))


def test_topk_codes_without_gpu(pkg):
    # the argument checks run before any HIP call; the caller's work and counters are required for split rows
    lib = ctypes.CDLL(pkg.lib_path("topk"))
    lib.launch.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_longlong, ctypes.c_longlong] + [ctypes.c_int] * 4 + \
        [ctypes.c_longlong, ctypes.c_void_p]
    p = 256  # never dereferenced: every call below returns before a launch
    assert lib.launch(p, p, p, p, p, 0, 100, 5, 0, 256, 4, 100, None) == 0       # no rows
    assert lib.launch(p, p, p, p, p, 2, 100, 0, 0, 256, 4, 100, None) == 0       # k = 0
    assert lib.launch(p, p, p, p, p, 2, 100, 101, 0, 256, 4, 100, None) == -1    # k > cols
    assert lib.launch(p, p, p, p, p, 2, 5000, 1025, 0, 256, 4, 5000, None) == -1  # k > 1024
    assert lib.launch(p, p, p, p, p, 70000, 100, 5, 0, 256, 4, 100, None) == -1  # rows > 65535
    assert lib.launch(p, p, p, p, p, 2, 100, 5, 0, 256, 4, 50, None) == -1       # split with chunk % 4
    assert lib.launch(p, p, p, p, p, 2, 100, 5, 0, 100, 4, 100, None) == -1      # threads
    assert lib.launch(p, p, p, p, p, 2, 100, 5, 0, 256, 3, 100, None) == -1      # depth
    assert lib.launch(p, p, p, p, p, 2, 100, 5, 2, 256, 4, 100, None) == -1      # dtype
    assert lib.launch(p, p, p, None, p, 2, 100, 5, 0, 256, 4, 52, None) == -1    # split row without work
    assert lib.launch(p, p, p, p, None, 2, 100, 5, 0, 256, 4, 52, None) == -1    # split row without counters
    lib.topk_reset.argtypes = [ctypes.c_void_p, ctypes.c_longlong, ctypes.c_void_p]
    assert lib.topk_reset(None, 0, None) == 0 and lib.topk_reset(None, 4, None) == -1
