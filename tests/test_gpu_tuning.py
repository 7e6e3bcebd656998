"""The tuning hooks (`softmax_tune`, `rmsnorm_tune`, `rope_tune`) cannot break the reference entry points: a tuned
launch shape that the kernels do not have is ignored and the automatic choice runs, so `launch` still succeeds and
its output equals the untuned launch's bit for bit. (RMSNorm's one-wave case with an automatic vector count is a
shape the kernel has at the shorter rows; its output does not depend on the shape, so it is equal there too.)
"""

import pytest
import torch

pytestmark = pytest.mark.gpu


def tuned(pkg, op, settings, fn):
    """fn() with the op library's tuning slots set (slot, value), restored to automatic after."""
    tune = getattr(pkg.candidate(op)._lib, f"{op}_tune")
    for slot, value in settings:
        assert tune(slot, value) == 0
    try:
        out = fn()
        torch.cuda.synchronize()
        return out
    finally:
        for slot, _ in settings:
            assert tune(slot, 0) == 0


@pytest.mark.parametrize("settings", [[(0, 3)], [(1, 5)], [(1, 32)], [(0, 16), (1, 16)], [(0, 32)]],
                         ids=["waves3", "nv5", "nv32", "nv16_with_16_waves", "waves32"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_softmax_ignores_shapes_it_has_not(pkg, dev, settings, dtype):
    g = torch.Generator().manual_seed(5)
    for cols in (1024, 4096, 32768):
        x = (torch.randn(6, cols, generator=g) * 3).to(dtype).to(dev)
        print(f"[tuning] softmax {settings} {cols} {dtype}", flush=True)
        want = pkg.softmax(x)
        got = tuned(pkg, "softmax", settings, lambda: pkg.softmax(x))
        assert torch.equal(got.view(torch.int16 if dtype != torch.float32 else torch.int32),
                           want.view(torch.int16 if dtype != torch.float32 else torch.int32))


@pytest.mark.parametrize("settings", [[(0, 3)], [(1, 16)], [(0, 1), (1, 0)], [(0, 32)]],
                         ids=["waves3", "nv16", "one_wave_auto_nv", "waves32"])
def test_rmsnorm_ignores_shapes_it_has_not(pkg, dev, settings):
    g = torch.Generator().manual_seed(6)
    for cols in (512, 4096, 32768):
        x = torch.randn(5, cols, generator=g).bfloat16().to(dev)
        w = (torch.rand(cols, generator=g) + 0.5).bfloat16().to(dev)
        print(f"[tuning] rmsnorm {settings} {cols}", flush=True)
        want = pkg.rmsnorm(x, w)
        got = tuned(pkg, "rmsnorm", settings, lambda: pkg.rmsnorm(x, w))
        assert torch.equal(got.view(torch.int16), want.view(torch.int16))


@pytest.mark.parametrize("threads", [100, 2048, -64])
def test_rope_ignores_blocks_it_cannot_take(pkg, dev, threads):
    g = torch.Generator().manual_seed(7)
    q = torch.randn(2, 33, 32, 128, generator=g).bfloat16().to(dev)
    k = torch.randn(2, 33, 8, 128, generator=g).bfloat16().to(dev)
    pos = torch.randint(0, 4096, (2, 33), generator=g).to(dev)
    inv = (1.0 / (10000.0 ** (torch.arange(0, 128, 2).float() / 128))).to(dev)
    print(f"[tuning] rope threads={threads}", flush=True)
    wq, wk = pkg.rope(q, k, pos, inv_freq=inv)
    gq, gk = tuned(pkg, "rope", [(0, threads)], lambda: pkg.rope(q, k, pos, inv_freq=inv))
    assert torch.equal(gq.view(torch.int16), wq.view(torch.int16))
    assert torch.equal(gk.view(torch.int16), wk.view(torch.int16))
