"""The measurement's bandwidth probes (bench_probes.hip, bench.py --ceiling and --probes) on the GPU: every copy
structure and every cache-policy pair of the stride probe copies exactly, for sizes that do and do not fill the
persistent grids; the read probe reads without writing its sink (the data never produces the marker value); the write
probe fills exactly its buffer. The rates they measure are only meaningful if they move what they claim to move.
"""

import ctypes

import pytest
import torch

import bench

pytestmark = pytest.mark.gpu

COPY_SPECS = sorted(set(bench.CEILING_PROBES) | {
    f"stride_u{u}_b8_nt_nt" for u in (2, 8)} | {
    f"stride_u4_b8_{lp}_{sp}" for lp in bench.POLICIES for sp in bench.POLICIES} | {
    "xcd_u8_b8_nt_nt", "oneshot_u4_b8_nt_nt", "oneshot_u16_b8_nt_nt", "slab_u8_b8_nt_nt", "lds_u2_b8_nt_nt",
    "lds_u8_b8_nt_nt", "row_u8_b8_nt_nt", "stride_u4_b16_nt_nt"})


@pytest.fixture(scope="module")
def lib():
    return bench.probe_lib()


def _run(lib, spec, x, y, sink, nbytes):
    family, unroll, bpc, lp, sp = bench.parse_probe(spec)
    return lib.probe_run(family, unroll, bpc, lp, sp, x, y, sink, nbytes, torch.cuda.current_stream().cuda_stream)


@pytest.mark.parametrize("spec", COPY_SPECS)
@pytest.mark.parametrize("nbytes", [16, 4096 + 48, (8 << 20) + 16 * 37])
def test_copy_probes_copy_exactly(lib, dev, spec, nbytes):
    print(f"probe {spec} bytes {nbytes}", flush=True)
    g = torch.Generator().manual_seed(nbytes % 1000)
    x = torch.randint(-2**31, 2**31 - 1, (nbytes // 4,), generator=g, dtype=torch.int32).to(dev)
    y = torch.zeros(nbytes // 4 + 64, dtype=torch.int32, device=dev)  # 256 bytes past the end must stay 0
    assert _run(lib, spec, x.data_ptr(), y.data_ptr(), None, nbytes) == 0
    torch.cuda.synchronize()
    assert torch.equal(x, y[: nbytes // 4])
    assert bool((y[nbytes // 4:] == 0).all())


def test_read_probe_leaves_its_sink(lib, dev):
    x = torch.ones((32 << 20) // 4, dtype=torch.float32, device=dev)
    sink = torch.full((1,), 5, dtype=torch.int32, device=dev)
    for spec in ("read_u4_b8_nt_nt", "read_u8_b8_nt_nt"):
        assert _run(lib, spec, x.data_ptr(), None, sink.data_ptr(), x.numel() * 4) == 0
    torch.cuda.synchronize()
    assert int(sink.item()) == 5


@pytest.mark.parametrize("spec", ["write_u4_b8_nt_nt", "write_u8_b8_nt_nt"])
def test_write_probe_fills_its_buffer(lib, dev, spec):
    nbytes = (4 << 20) + 16 * 5
    y = torch.zeros(nbytes // 4 + 64, dtype=torch.int32, device=dev)
    assert _run(lib, spec, None, y.data_ptr(), None, nbytes) == 0
    torch.cuda.synchronize()
    v = y[: nbytes // 4].view(-1, 4)
    assert bool((v[:, 0] == 1).all()) and bool((v[:, 1] == 2).all()) and bool((v[:, 2] == 3).all())
    assert bool((y[nbytes // 4:] == 0).all())
