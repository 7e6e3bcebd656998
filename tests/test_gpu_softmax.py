"""GPU parity of softmax (build/softmax/libkernel.so through the reference ABI `launch`) against the oracle.

fp32: |y - oracle| <= 1e-5 |oracle| + 2^-147 elementwise (the oracle is the fp64 softmax rounded once); bf16: within
1 ulp. The absolute term is four ulps of the fp32 subnormal range (2^-149 each), where a relative bound cannot hold for
any computation that rounds more than once: exp(x - max) rounded to a subnormal, then scaled by the row's 1 / sum, is
off by up to about 1.5 ulps there, and the reference's own PyTorch path (torch.softmax, fp32 on the CPU) is off by up
to 33 ulps from the oracle on rows whose outputs reach that range (checked in tests/test_oracle.py). Outputs of
normal magnitude keep the relative bound alone.
Shapes cover every tier: wave-per-row and workgroup-per-row rows (full and ragged), the single-pass co-resident tier
for long rows (one row per workgroup, and row groups walking several rows when the rows' chunks do not all fit at
once), the two-pass stream tier for rows beyond it, and the generic tier for lengths that are not a multiple of the
vector width and for misaligned pointers.
"""

import ctypes
import time

import numpy as np
import pytest
import torch

from _util import assert_rel, assert_ulp, bits16

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-5
FP32_SUBNORMAL_ATOL = 2.0 ** -147


def run_fp32(pkg, oracle, dev, x, what):
    print(f"[softmax fp32] {what} shape={tuple(x.shape)}", flush=True)
    y = pkg.softmax(x.to(dev)).cpu()
    assert_rel(y.numpy(), oracle.softmax(x.numpy(), "fp32"), FP32_TOL, what, FP32_SUBNORMAL_ATOL)
    return y


@pytest.mark.parametrize("rows,cols", [(1, 4), (3, 256), (5, 1000), (64, 1024), (9, 2048), (7, 4096),
                                       (33, 8192), (3, 12288), (2, 32768), (2, 32772), (3, 65536),
                                       (2, 131072 + 4), (5, 1), (4, 7), (6, 1001), (2, 40001)])
def test_fp32_shapes(pkg, oracle, dev, rows, cols):
    g = torch.Generator().manual_seed(rows * 100003 + cols)
    run_fp32(pkg, oracle, dev, torch.randn(rows, cols, generator=g) * 3, f"{rows}x{cols}")


@pytest.mark.parametrize("rows,cols", [(3, 512), (64, 2048), (7, 8192), (2, 65536), (2, 131072), (4, 1003)])
def test_bf16_shapes(pkg, oracle, dev, rows, cols):
    g = torch.Generator().manual_seed(rows * 7 + cols)
    x = (torch.randn(rows, cols, generator=g) * 3).bfloat16()
    print(f"[softmax bf16] {rows}x{cols}", flush=True)
    y = pkg.softmax(x.to(dev))
    assert_ulp(bits16(y), oracle.softmax(bits16(x), "bf16"), 1, f"bf16 {rows}x{cols}")


def test_random_shapes(pkg, oracle, dev):
    # seeded random shapes across every tier (short rows to rows of 2^18 and beyond), fp32 and bf16, with spreads from
    # flat to peaked rows
    rng = np.random.default_rng(77)
    g = torch.Generator().manual_seed(77)
    for case in range(60):
        cols = int(np.exp(rng.uniform(0, np.log(300000))))
        rows = int(rng.integers(1, max(2, min(300, 2_000_000 // cols))))
        scale = float(rng.choice([0.1, 1.0, 3.0, 30.0]))
        x = torch.randn(rows, cols, generator=g) * scale
        if case % 2:
            run_fp32(pkg, oracle, dev, x, f"random case {case}")
        else:
            xb = x.bfloat16()
            print(f"[softmax bf16] random case {case} {rows}x{cols}", flush=True)
            y = pkg.softmax(xb.to(dev))
            assert_ulp(bits16(y), oracle.softmax(bits16(xb), "bf16"), 1, f"bf16 random case {case} {rows}x{cols}")


def test_many_rows_persistent(pkg, oracle, dev):
    # more rows than resident workgroups: every workgroup walks several rows
    g = torch.Generator().manual_seed(5)
    run_fp32(pkg, oracle, dev, torch.randn(20000, 256, generator=g), "20000x256")
    run_fp32(pkg, oracle, dev, torch.randn(5000, 1024, generator=g), "5000x1024")


def test_misaligned_and_special_values(pkg, oracle, dev):
    g = torch.Generator().manual_seed(6)
    base = torch.randn(4 * 1024 + 1, generator=g).to(dev)
    x = base[1:].view(4, 1024)  # data pointer 4 bytes past a 16-byte boundary: the generic tier
    y = torch.empty_like(x)
    lib = pkg.candidate("softmax")._lib
    assert lib.launch(x.data_ptr(), y.data_ptr(), 4, 1024, 0, 256, 1024, torch.cuda.current_stream().cuda_stream) == 0
    assert_rel(y.cpu().numpy(), oracle.softmax(x.cpu().numpy(), "fp32"), FP32_TOL, "misaligned",
               FP32_SUBNORMAL_ATOL)
    s = torch.randn(4, 1024, generator=g)
    s[0, 10] = float("-inf")
    s[1, :] = float("-inf")
    s[2, 5] = float("nan")
    s[3, ::3] = float("-inf")
    y = pkg.softmax(s.to(dev)).cpu()
    assert y[0, 10] == 0 and torch.isnan(y[1]).all() and torch.isnan(y[2]).all() and (y[3, ::3] == 0).all()
    ref = oracle.softmax(s.numpy(), "fp32")
    assert_rel(y[[0, 3]].numpy(), ref[[0, 3]], FP32_TOL, "special values", FP32_SUBNORMAL_ATOL)


def test_long_rows_with_infinite_chunks(pkg, oracle, dev):
    g = torch.Generator().manual_seed(7)
    x = torch.randn(3, 70000, generator=g)
    x[0, :40000] = float("-inf")  # whole chunks of -inf must not poison the merge
    x[1, :] = float("-inf")
    y = pkg.softmax(x.to(dev)).cpu()
    assert torch.isnan(y[1]).all()
    ref = oracle.softmax(x.numpy(), "fp32")
    assert_rel(y[[0, 2]].numpy(), ref[[0, 2]], FP32_TOL, "long rows", FP32_SUBNORMAL_ATOL)


@pytest.mark.parametrize("rows,cols,dtype", [(64, 262144, "fp32"), (3, 70000, "fp32"), (1, 1 << 20, "fp32"),
                                             (100, 40000, "fp32"), (8, 131072, "bf16"), (2, 300000, "bf16")])
def test_long_rows_single_pass_and_stream(pkg, oracle, dev, rows, cols, dtype):
    """Long rows through the co-resident single-pass tier (4) and the two-pass stream tier (2), preferred in turn."""
    lib = pkg.candidate("softmax")._lib
    g = torch.Generator().manual_seed(rows + cols)
    x = torch.randn(rows, cols, generator=g) * 4
    x[0, : cols // 3] = float("-inf")  # whole chunks of -inf in the first row
    if dtype == "bf16":
        x = x.bfloat16()
        ref = oracle.softmax(bits16(x), "bf16")
    else:
        ref = oracle.softmax(x.numpy(), "fp32")
    xd = x.to(dev)
    try:
        for tier in (4, 2):
            lib.softmax_tune(5, tier)
            print(f"[softmax long] {rows}x{cols} {dtype} tier={tier}", flush=True)
            y = pkg.softmax(xd)
            if dtype == "bf16":
                assert_ulp(bits16(y), ref, 1, f"tier {tier}")
            else:
                assert_rel(y.cpu().numpy(), ref, FP32_TOL, f"tier {tier}", FP32_SUBNORMAL_ATOL)
    finally:
        lib.softmax_tune(5, 0)


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
def test_coresident_graph_replay(pkg, oracle, dev, dtype):
    """A 64 x 262144 launch (the co-resident tier) recorded into a HIP graph with torch.cuda.graph and
    replayed on new values of x, with eager launches of other values on the same pair-table slots between some
    replays. Each replay must take fresh tags on the device: with the tags of the capture it would accept the pairs
    the replay before it left. The wait budget is raised to 2^30 ticks (about 10 s), so a replay can only finish
    quickly by finding its own pairs, not by the fallback; each replay is checked against the oracle of its x."""
    lib = pkg.candidate("softmax")._lib
    rows, cols = 64, 262144
    g = torch.Generator().manual_seed(31)
    xs = []
    for i in range(4):
        x = torch.randn(rows, cols, generator=g) * (5 if i % 2 == 0 else 2)
        x.view(-1)[torch.randperm(rows * cols, generator=g)[: rows * cols // 100]] = 20.0 - 3 * i
        xs.append(x.bfloat16() if dtype == "bf16" else x)
    code = 1 if dtype == "bf16" else 0

    def ref(x):
        return oracle.softmax(bits16(x), "bf16") if dtype == "bf16" else oracle.softmax(x.numpy(), "fp32")

    def check(y, x, what):
        if dtype == "bf16":
            assert_ulp(bits16(y), ref(x), 1, what)
        else:
            assert_rel(y.cpu().numpy(), ref(x), FP32_TOL, what, FP32_SUBNORMAL_ATOL)

    xd, yd = xs[0].to(dev), torch.empty(rows, cols, dtype=xs[0].dtype, device=dev)
    x2, y2 = torch.empty_like(xd), torch.empty_like(yd)
    try:
        lib.softmax_tune(5, 4)
        lib.softmax_tune(7, 1 << 30)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):  # the eager warm-up launch, on a side stream as torch's capture recipe has it
            assert lib.launch(xd.data_ptr(), yd.data_ptr(), rows, cols, code, 256, 1024, side.cuda_stream) == 0
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        check(yd, xs[0], "eager warm-up")
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            rc = lib.launch(xd.data_ptr(), yd.data_ptr(), rows, cols, code, 256, 1024,
                            torch.cuda.current_stream().cuda_stream)
        assert rc == 0
        for rep in range(6):
            x = xs[rep % 4]
            print(f"[softmax graph] {dtype} replay {rep}", flush=True)
            xd.copy_(x.to(dev))
            yd.fill_(float("nan"))
            if rep % 3 == 2:  # an eager launch of other values first: its pairs sit in the same table slots
                x2.copy_(xs[(rep + 1) % 4].to(dev))
                s = torch.cuda.current_stream().cuda_stream
                assert lib.launch(x2.data_ptr(), y2.data_ptr(), rows, cols, code, 256, 1024, s) == 0
            torch.cuda.synchronize()
            t0 = time.monotonic()
            graph.replay()
            torch.cuda.synchronize()
            took = time.monotonic() - t0
            assert took < 1.0, f"replay {rep} took {took:.2f} s: its waits ended by the time budget, not by its pairs"
            check(yd, x, f"replay {rep}")
    finally:
        lib.softmax_tune(7, 0)
        lib.softmax_tune(5, 0)


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
def test_single_pass_fallback_when_the_wait_ends(pkg, oracle, dev, dtype):
    """The co-resident tier with its wait bounded to one tick of its clock (forced from the host): workgroups that find
    their row's pairs incomplete take the row's statistics from x, the rest merge the pairs; every output stays within
    the tolerance, over repeated launches, with one row per workgroup and with row groups walking several rows."""
    lib = pkg.candidate("softmax")._lib
    g = torch.Generator().manual_seed(21)
    x = torch.randn(6, 262144 + 4096, generator=g) * 4
    x[1, ::7] = float("-inf")
    x[2, 5000] = 30.0  # an outlier that keeps every output in the normal range (a subnormal one has no 1e-5 ulp)
    if dtype == "bf16":
        x = x.bfloat16()
        ref = oracle.softmax(bits16(x), "bf16")
    else:
        ref = oracle.softmax(x.numpy(), "fp32")
    xd = x.to(dev)
    try:
        lib.softmax_tune(5, 4)
        lib.softmax_tune(7, 1)
        for rep, groups in enumerate((0, 0, 2, 4)):
            lib.softmax_tune(4, groups)
            print(f"[softmax fallback] {dtype} launch {rep} groups={groups}", flush=True)
            y = pkg.softmax(xd)
            if dtype == "bf16":
                assert_ulp(bits16(y), ref, 1, f"launch {rep}")
            else:
                assert_rel(y.cpu().numpy(), ref, FP32_TOL, f"launch {rep}", FP32_SUBNORMAL_ATOL)
    finally:
        lib.softmax_tune(7, 0)
        lib.softmax_tune(5, 0)
        lib.softmax_tune(4, 0)
    y = pkg.softmax(xd)  # the default wait again, on the slots the fallback launches left
    if dtype == "bf16":
        assert_ulp(bits16(y), ref, 1, "after")
    else:
        assert_rel(y.cpu().numpy(), ref, FP32_TOL, "after", FP32_SUBNORMAL_ATOL)


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
def test_single_pass_rows_beyond_one_wave(pkg, oracle, dev, dtype):
    """More long rows than the GPU holds chunks of at once (the reference's 256 x 262144 README shape): row groups walk
    several rows each, still one read of x; and row groups forced down to 1, 3 and 5 (many rows per workgroup, the
    pair table's two parities in turn, the last iteration of some groups shorter)."""
    lib = pkg.candidate("softmax")._lib
    g = torch.Generator().manual_seed(22)
    x = torch.randn(256, 262144, generator=g) * 5
    x[3, :100000] = float("-inf")
    if dtype == "bf16":
        x = x.bfloat16()
        ref = oracle.softmax(bits16(x), "bf16")
    else:
        ref = oracle.softmax(x.numpy(), "fp32")
    print(f"[softmax groups] 256x262144 {dtype}", flush=True)
    y = pkg.softmax(x.to(dev))
    if dtype == "bf16":
        assert_ulp(bits16(y), ref, 1, "256x262144")
    else:
        assert_rel(y.cpu().numpy(), ref, FP32_TOL, "256x262144", FP32_SUBNORMAL_ATOL)
    xs = x[:13, :70000].contiguous()
    refs = oracle.softmax(bits16(xs), "bf16") if dtype == "bf16" else oracle.softmax(xs.numpy(), "fp32")
    xd = xs.to(dev)
    try:
        lib.softmax_tune(5, 4)
        for groups in (1, 3, 5):
            lib.softmax_tune(4, groups)
            print(f"[softmax groups] 13x70000 {dtype} groups={groups}", flush=True)
            for _ in range(2):
                y = pkg.softmax(xd)
                if dtype == "bf16":
                    assert_ulp(bits16(y), refs, 1, f"groups {groups}")
                else:
                    assert_rel(y.cpu().numpy(), refs, FP32_TOL, f"groups {groups}", FP32_SUBNORMAL_ATOL)
    finally:
        lib.softmax_tune(4, 0)
        lib.softmax_tune(5, 0)


def test_rows_beyond_the_single_pass_tier(pkg, oracle, dev):
    """A row of more than 64 chunks (16384 fp32 each) takes the two-pass stream tier."""
    g = torch.Generator().manual_seed(23)
    run_fp32(pkg, oracle, dev, torch.randn(2, (1 << 20) + 4096, generator=g) * 3, "2x(2^20+4096)")


def test_single_pass_back_to_back_shapes(pkg, oracle, dev):
    """Consecutive single-pass launches of different shapes on one stream: each takes fresh tags in the pair table."""
    g = torch.Generator().manual_seed(9)
    xs = [torch.randn(64, 262144, generator=g), torch.randn(5, 50000, generator=g),
          torch.randn(16, 1 << 18, generator=g), torch.randn(5, 50000, generator=g)]
    ds = [x.to(dev) for x in xs]
    ys = [pkg.softmax(d) for d in ds + ds]  # queued back to back, then checked
    for i, y in enumerate(ys):
        print(f"[softmax back-to-back] launch {i} shape={tuple(xs[i % 4].shape)}", flush=True)
        assert_rel(y.cpu().numpy(), oracle.softmax(xs[i % 4].numpy(), "fp32"), FP32_TOL, f"launch {i}",
                   FP32_SUBNORMAL_ATOL)


def test_empty_is_noop(pkg, dev):
    lib = pkg.candidate("softmax")._lib
    s = torch.cuda.current_stream().cuda_stream
    assert lib.launch(None, None, 0, 10, 0, 256, 1024, s) == 0
    assert lib.launch(None, None, 10, 0, 1, 256, 1024, s) == 0
    x = torch.empty(0, 5, device=dev)
    assert pkg.softmax(x).shape == (0, 5)


def test_config_softmax_4096x4096(pkg, oracle, dev):
    x = pkg.workloads.softmax_4096x4096()["x"]
    y = run_fp32(pkg, oracle, dev, x, "softmax_4096x4096")
    s = y.double().sum(-1)
    assert torch.allclose(s, torch.ones_like(s), atol=1e-5)


def test_config_softmax_64x262144(pkg, oracle, dev):
    x = pkg.workloads.softmax_64x262144()["x"]
    y = run_fp32(pkg, oracle, dev, x, "softmax_64x262144")
    # the reference's own path (torch fp32) agrees within the same tolerance
    assert_rel(y.numpy(), torch.softmax(x, -1).numpy(), 2 * FP32_TOL, "vs torch fp32", FP32_SUBNORMAL_ATOL)


def test_tuning_overrides_keep_results(pkg, oracle, dev):
    """Every row-tier shape the tuning slots can force computes the same row."""
    lib = pkg.candidate("softmax")._lib
    g = torch.Generator().manual_seed(8)
    x = torch.randn(300, 4096, generator=g)
    ref = oracle.softmax(x.numpy(), "fp32")
    xd = x.to(dev)
    try:
        for waves, nv in [(2, 8), (4, 4), (8, 2), (16, 1)]:
            lib.softmax_tune(0, waves)
            lib.softmax_tune(1, nv)
            for per_cu in (1, 2):
                lib.softmax_tune(2, per_cu)
                print(f"[softmax tune] waves={waves} nv={nv} per_cu={per_cu}", flush=True)
                assert_rel(pkg.softmax(xd).cpu().numpy(), ref, FP32_TOL, f"w{waves} nv{nv}", FP32_SUBNORMAL_ATOL)
        lib.softmax_tune(0, 0), lib.softmax_tune(1, 0), lib.softmax_tune(2, 0)
        for tier in (2, 3):
            lib.softmax_tune(5, tier)
            print(f"[softmax tune] tier={tier}", flush=True)
            assert_rel(pkg.softmax(xd).cpu().numpy(), ref, FP32_TOL, f"tier {tier}", FP32_SUBNORMAL_ATOL)
    finally:
        for slot in range(8):
            lib.softmax_tune(slot, 0)
