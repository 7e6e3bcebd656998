"""GPU parity of RMSNorm (build/rmsnorm/libkernel.so: `launch` and `rmsnorm_launch_weighted`) against the oracle.

The kernel sums the squares in fp64 (exact far below fp32 resolution) and rounds rsqrt correctly, so it must equal the
oracle bit for bit. Against the reference's own torch expression it must be within 1 ulp wherever the rounded inv
agrees, with inv itself one ulp apart on the rare rows where torch's fp32 sum lands across a rounding boundary.
"""

import numpy as np
import pytest
import torch

from _util import bits16, same_bits16, ulp16

pytestmark = pytest.mark.gpu

DT = {torch.bfloat16: "bf16", torch.float16: "fp16"}


def check(pkg, oracle, dev, x, w, eps=1e-6, what=""):
    print(f"[rmsnorm] {what} {tuple(x.shape)} {x.dtype} weight={w is not None}", flush=True)
    y = pkg.rmsnorm(x.to(dev), None if w is None else w.to(dev), eps)
    ref = oracle.rmsnorm(bits16(x), None if w is None else bits16(w), eps, DT[x.dtype])
    got = bits16(y)
    if not same_bits16(got, ref, x.dtype == torch.float16):
        d = ulp16(got, ref)
        bad = np.argwhere(got != ref)
        raise AssertionError(f"{what}: {len(bad)} elements differ from the oracle (max {d.max()} ulp), first {bad[0]}")
    return y


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,cols", [(1, 8), (3, 512), (5, 1000), (17, 4096), (4, 4104), (3, 8192),
                                       (2, 32768), (2, 65536), (3, 1001), (2, 70000), (1, 3)])
def test_shapes(pkg, oracle, dev, dtype, rows, cols):
    g = torch.Generator().manual_seed(rows * 1009 + cols)
    x = torch.randn(rows, cols, generator=g).to(dtype)
    w = (torch.rand(cols, generator=g) + 0.5).to(dtype)
    check(pkg, oracle, dev, x, None, what=f"{rows}x{cols}")
    check(pkg, oracle, dev, x, w, what=f"{rows}x{cols} weighted")


def test_random_shapes(pkg, oracle, dev):
    # seeded random shapes (odd lengths included), both dtypes, with and without the weight, several eps
    rng = np.random.default_rng(78)
    g = torch.Generator().manual_seed(78)
    for case in range(60):
        cols = int(np.exp(rng.uniform(0, np.log(100000))))
        rows = int(rng.integers(1, max(2, min(300, 2_000_000 // cols))))
        dtype = torch.bfloat16 if case % 2 else torch.float16
        x = (torch.randn(rows, cols, generator=g) * float(rng.choice([0.01, 1.0, 20.0]))).to(dtype)
        w = (torch.rand(cols, generator=g) + 0.5).to(dtype) if case % 3 else None
        eps = float(rng.choice([1e-6, 1e-5, 1e-3]))
        check(pkg, oracle, dev, x, w, eps, what=f"random case {case}")


def test_many_rows_and_eps(pkg, oracle, dev):
    g = torch.Generator().manual_seed(3)
    x = torch.randn(10000, 1024, generator=g).bfloat16()
    check(pkg, oracle, dev, x, None, 1e-6, "10000x1024")
    check(pkg, oracle, dev, x * 1e-3, None, 1e-2, "eps dominates")


def test_special_values(pkg, oracle, dev):
    g = torch.Generator().manual_seed(4)
    x = torch.randn(6, 4096, generator=g).bfloat16()
    x[1, 9] = float("nan")
    x[2, :] = 1e20  # squares overflow fp32: inv = 0, the reference's rule
    x[3, :] = 0.0   # inv = rsqrt(eps)
    x[4, 5] = float("inf")
    y = check(pkg, oracle, dev, x, None, what="special").cpu()
    assert y[1].isnan().all() and (y[2] == 0).all() and (y[3] == 0).all()
    assert not y[[0, 5]].isnan().any()


def test_misaligned_pointer_uses_generic(pkg, oracle, dev):
    g = torch.Generator().manual_seed(5)
    base = torch.randn(3 * 4096 + 1, generator=g).bfloat16().to(dev)
    x = base[1:].view(3, 4096)
    y = torch.empty_like(x)
    lib = pkg.candidate("rmsnorm")._lib
    assert lib.launch(x.data_ptr(), y.data_ptr(), 3, 4096, 1, 1e-6, 256, torch.cuda.current_stream().cuda_stream) == 0
    assert np.array_equal(bits16(y), oracle.rmsnorm(bits16(x.cpu()), None, 1e-6, "bf16"))


def test_config_rmsnorm_16384x4096(pkg, oracle, dev):
    inp = pkg.workloads.rmsnorm_16384x4096()
    x, w = inp["x"], inp["weight"]
    y = check(pkg, oracle, dev, x, w, inp["eps"], "rmsnorm_16384x4096")
    # against the reference's torch expression (rmsnorm/candidate.py:3-4, weighted as w * y) on the CPU: bit for bit
    # over all 67M outputs (the oracle equals it there, tests/test_oracle.py)
    from oracle import torch_paths
    ref = bits16(torch_paths.rmsnorm(x, w, inp["eps"]))
    assert np.array_equal(bits16(y), ref)


def test_tuning_overrides_keep_results(pkg, oracle, dev):
    lib = pkg.candidate("rmsnorm")._lib
    g = torch.Generator().manual_seed(6)
    x = torch.randn(777, 4096, generator=g).bfloat16()
    w = (torch.rand(4096, generator=g) + 0.5).bfloat16()
    try:
        for waves, nv in [(1, 8), (2, 4), (4, 2), (8, 1)]:
            for per_cu in (1, 3):
                lib.rmsnorm_tune(0, waves)
                lib.rmsnorm_tune(1, nv)
                lib.rmsnorm_tune(2, per_cu)
                check(pkg, oracle, dev, x, w, what=f"waves={waves} nv={nv} per_cu={per_cu}")
        for slot in range(5):
            lib.rmsnorm_tune(slot, 0)
        lib.rmsnorm_tune(3, 1)
        check(pkg, oracle, dev, x, w, what="generic")
    finally:
        for slot in range(5):
            lib.rmsnorm_tune(slot, 0)


def check_add(pkg, oracle, dev, x, r, w, eps=1e-6, what="", inplace=False):
    print(f"[rmsnorm_add] {what} {tuple(x.shape)} {x.dtype} weight={w is not None} inplace={inplace}", flush=True)
    rd = r.to(dev)
    y, h = pkg.rmsnorm_add(x.to(dev), rd, None if w is None else w.to(dev), eps, inplace=inplace)
    ry, rh = oracle.rmsnorm_add(bits16(x), bits16(r), None if w is None else bits16(w), eps, DT[x.dtype])
    assert np.array_equal(bits16(h), rh), f"{what}: h differs"
    assert same_bits16(bits16(y), ry, x.dtype == torch.float16), f"{what}: y differs (max {ulp16(bits16(y), ry).max()})"
    if inplace:
        assert h.data_ptr() == rd.data_ptr() and np.array_equal(bits16(rd), rh)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,cols", [(1, 8), (5, 1000), (17, 4096), (4, 4104), (2, 32768), (3, 1001), (1000, 2048)])
def test_fused_residual_shapes(pkg, oracle, dev, dtype, rows, cols):
    g = torch.Generator().manual_seed(rows * 7919 + cols)
    x = torch.randn(rows, cols, generator=g).to(dtype)
    r = (torch.randn(rows, cols, generator=g) * 2).to(dtype)
    w = (torch.rand(cols, generator=g) + 0.5).to(dtype)
    check_add(pkg, oracle, dev, x, r, None, what=f"{rows}x{cols}")
    check_add(pkg, oracle, dev, x, r, w, what=f"{rows}x{cols} weighted", inplace=True)


def test_fused_residual_generic_and_special(pkg, oracle, dev):
    g = torch.Generator().manual_seed(12)
    x = torch.randn(6, 4096, generator=g).bfloat16()
    r = torch.randn(6, 4096, generator=g).bfloat16()
    r[1, 3] = float("nan")
    r[2, :] = -x[2, :]  # h = 0: inv = rsqrt(eps), y = 0
    check_add(pkg, oracle, dev, x, r, None, what="special")
    lib = pkg.candidate("rmsnorm")._lib
    try:
        lib.rmsnorm_tune(3, 1)  # the generic two-pass kernel, in place
        check_add(pkg, oracle, dev, x, r, None, what="generic", inplace=True)
    finally:
        lib.rmsnorm_tune(3, 0)


def test_config_rmsnorm_add_16384x4096(pkg, oracle, dev):
    inp = pkg.workloads.rmsnorm_add_16384x4096()
    check_add(pkg, oracle, dev, inp["x"], inp["residual"], inp["weight"], inp["eps"], "rmsnorm_add_16384x4096",
              inplace=True)
