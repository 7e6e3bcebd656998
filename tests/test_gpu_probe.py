"""The measurement's bandwidth probes (csrc/probe.hip, bench.py --ceiling) on the GPU: the copy probe copies exactly,
for sizes that do and do not fill its persistent grid, and the read probe reads without writing its sink (the data
never produces the marker value). The rates they measure are only meaningful if they move what they claim to move.
"""

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def probe(pkg):
    lib = ctypes.CDLL(pkg.lib_path("probe"))
    lib.probe_copy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_longlong, ctypes.c_void_p]
    lib.probe_read.argtypes = [ctypes.c_void_p, ctypes.c_longlong, ctypes.c_void_p, ctypes.c_void_p]
    return lib


@pytest.mark.parametrize("nbytes", [16, 4096 + 48, 1 << 20, (64 << 20) + 16 * 37])
def test_copy_probe_copies_exactly(probe, dev, nbytes):
    g = torch.Generator().manual_seed(nbytes % 1000)
    x = torch.randint(-2**31, 2**31 - 1, (nbytes // 4,), generator=g, dtype=torch.int32).to(dev)
    y = torch.zeros_like(x)
    guard = torch.full((64,), 7, dtype=torch.int32, device=dev)  # a separate allocation the probe must not touch
    stream = torch.cuda.current_stream().cuda_stream
    assert probe.probe_copy(x.data_ptr(), y.data_ptr(), nbytes, stream) == 0
    torch.cuda.synchronize()
    assert torch.equal(x, y)
    assert bool((guard == 7).all())


def test_read_probe_leaves_its_sink(probe, dev):
    x = torch.ones((32 << 20) // 4, dtype=torch.float32, device=dev)
    sink = torch.full((1,), 5, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    assert probe.probe_read(x.data_ptr(), x.numel() * 4, sink.data_ptr(), stream) == 0
    torch.cuda.synchronize()
    assert int(sink.item()) == 5
