"""The allocation-free top-k entry point (topk_launch_noalloc: launch() with the library's static per-GPU scratch in
place of the caller's work and counters) against the existing entry point, through the C-ABI: bit-for-bit equal
values and indices on two calls in a row, the second with a smaller input (the scratch keeps the first call's
contents), for every k class and both dtypes; and the rejection of a request whose chunk results exceed the scratch."""

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


def noalloc(lib):
    f = lib.topk_launch_noalloc
    f.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_longlong, ctypes.c_longlong, ctypes.c_int, ctypes.c_int,
                                          ctypes.c_int, ctypes.c_int, ctypes.c_longlong, ctypes.c_void_p]
    f.restype = ctypes.c_int
    return f


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("k", [1, 50, 1024])
def test_noalloc_equals_launch_on_two_calls(pkg, dev, dt, k):
    cand = pkg.candidate("topk")
    lib = cand._lib
    fn = noalloc(lib)
    g = torch.Generator().manual_seed(70 + k)
    code = 0 if dt == torch.float32 else 1
    for rows, cols in [(128, 128256), (7, 50000)]:  # the second call smaller than the first
        x = (torch.randn(rows, cols, generator=g) * 2).to(dt).to(dev)
        print(f"[noalloc] {rows}x{cols} {dt} k={k}", flush=True)
        ref = cand.run({"x": x, "k": k})
        chunk = lib.plan(rows, cols, code, 256, 4, max(2048, 16 * k) if k > 64 else 2048)
        vals = torch.full((rows, k), -7, dtype=dt, device=dev)
        idx = torch.full((rows, k), -7, dtype=torch.int64, device=dev)
        err = fn(x.data_ptr(), vals.data_ptr(), idx.data_ptr(), rows, cols, k, code, 256, 4, chunk,
                 torch.cuda.current_stream().cuda_stream)
        assert err == 0
        torch.cuda.synchronize()
        assert torch.equal(idx, ref["indices"]), f"indices differ ({rows}x{cols} k={k})"
        assert torch.equal(vals.view(torch.int16) if dt == torch.bfloat16 else vals.view(torch.int32),
                           ref["values"].view(torch.int16) if dt == torch.bfloat16 else
                           ref["values"].view(torch.int32)), f"values differ ({rows}x{cols} k={k})"


def test_noalloc_rejects_beyond_its_scratch(pkg, dev):
    fn = noalloc(pkg.candidate("topk")._lib)
    x = torch.zeros(128, 128256, device=dev)
    out = torch.empty(128, 1024, device=dev)
    idx = torch.empty(128, 1024, dtype=torch.int64, device=dev)
    s = torch.cuda.current_stream().cuda_stream
    # k > 64 lengthens the caller's 4096-column chunks to 16384 (16k): 8 chunks per row. 128 rows need 128 * 8 * 1024
    # u64 slots = 8 MiB, within the 16 MiB scratch; 512 rows need 32 MiB, beyond it
    xl = torch.zeros(512, 128256, device=dev)
    outl = torch.empty(512, 1024, device=dev)
    idxl = torch.empty(512, 1024, dtype=torch.int64, device=dev)
    assert fn(xl.data_ptr(), outl.data_ptr(), idxl.data_ptr(), 512, 128256, 1024, 0, 256, 4, 4096, s) == -1
    assert fn(x.data_ptr(), out.data_ptr(), idx.data_ptr(), 128, 128256, 1024, 0, 256, 4, 4096, s) == 0
    torch.cuda.synchronize()
    assert (idx == torch.arange(1024, device=dev)).all(), "all-zero rows: indices 0..k-1"
    assert fn(x.data_ptr(), out.data_ptr(), idx.data_ptr(), 0, 128256, 1024, 0, 256, 4, 4096, s) == 0
