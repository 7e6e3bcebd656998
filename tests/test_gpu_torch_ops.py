"""GPU parity of the PyTorch-ROCm operators (torch.ops.ckopt.*, build/torch/libckopt_torch.so) against the oracle: the
same bars as the C-ABI tests (softmax fp32 within 1e-5 relative, bf16 within 1 ulp; RMSNorm, RoPE and top-k bit for
bit), each operator on small seeded inputs, with the in-place forms checked on the tensors they write."""

import numpy as np
import pytest
import torch

from _util import assert_rel, bits16, ulp16

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ckopt(pkg):
    return pkg.ops()


def test_softmax(ckopt, oracle, dev):
    g = torch.Generator().manual_seed(50)
    x = torch.randn(33, 5000, generator=g) * 3
    y = ckopt.softmax(x.to(dev))
    assert_rel(y.cpu().numpy(), oracle.softmax(x.numpy(), "fp32"), 1e-5, "ckopt.softmax fp32")
    xb = (torch.randn(2, 3, 70000, generator=g) * 3).bfloat16()  # leading dims become rows; long rows
    yb = ckopt.softmax(xb.to(dev))
    assert ulp16(bits16(yb).reshape(6, 70000), oracle.softmax(bits16(xb).reshape(6, 70000), "bf16")).max() <= 1


def test_rmsnorm_and_fused_residual(ckopt, oracle, dev):
    g = torch.Generator().manual_seed(51)
    x = torch.randn(40, 4096, generator=g).bfloat16()
    w = (torch.rand(4096, generator=g) + 0.5).bfloat16()
    assert np.array_equal(bits16(ckopt.rmsnorm(x.to(dev))), oracle.rmsnorm(bits16(x)))
    assert np.array_equal(bits16(ckopt.rmsnorm(x.to(dev), w.to(dev), 1e-6)), oracle.rmsnorm(bits16(x), bits16(w)))
    xh = torch.randn(40, 1000, generator=g).half()
    assert np.array_equal(bits16(ckopt.rmsnorm(xh.to(dev), None, 1e-5)),
                          oracle.rmsnorm(bits16(xh), None, 1e-5, "fp16"))
    r = torch.randn(40, 4096, generator=g).bfloat16()
    ry, rh = oracle.rmsnorm_add(bits16(x), bits16(r), bits16(w))
    y, h = ckopt.rmsnorm_add(x.to(dev), r.to(dev), w.to(dev), 1e-6)
    assert np.array_equal(bits16(y), ry) and np.array_equal(bits16(h), rh)
    rd = r.to(dev)
    y2 = ckopt.rmsnorm_add_(x.to(dev), rd, w.to(dev), 1e-6)
    assert np.array_equal(bits16(y2), ry) and np.array_equal(bits16(rd), rh), "in place: h over the residual"


def test_rope_forms(ckopt, oracle, pkg, dev):
    g = torch.Generator().manual_seed(52)
    q = torch.randn(2, 16, 8, 128, generator=g).bfloat16()
    k = torch.randn(2, 16, 2, 128, generator=g).bfloat16()
    pos = torch.randint(0, 4096, (2, 16), generator=g)
    inv = pkg.workloads.rope_inv_freq(128)
    cos = torch.randn(4096, 128, generator=g)
    sin = torch.randn(4096, 128, generator=g)
    qo, ko = ckopt.rope(q.to(dev), k.to(dev), cos.to(dev), sin.to(dev), pos.to(dev))
    rq, rk = oracle.rope_cache(bits16(q).reshape(32, 8, 128), bits16(k).reshape(32, 2, 128), cos.numpy(),
                               sin.numpy(), pos.view(-1).numpy())
    assert np.array_equal(bits16(qo).reshape(32, 8, 128), rq) and np.array_equal(bits16(ko).reshape(32, 2, 128), rk)
    qd, kd = q.to(dev), k.to(dev)
    ckopt.rope_(qd, kd, pos.to(dev), inv.to(dev))
    rq, rk = oracle.rope_freq(bits16(q).reshape(32, 8, 128), bits16(k).reshape(32, 2, 128), pos.view(-1).numpy(),
                              inv.numpy())
    assert np.array_equal(bits16(qd).reshape(32, 8, 128), rq) and np.array_equal(bits16(kd).reshape(32, 2, 128), rk)
    v = torch.randn(2, 16, 2, 128, generator=g).bfloat16()
    slots = torch.randperm(40, generator=g)[:32].view(2, 16)
    slots[0, 3] = -1
    kc, vc = torch.zeros(40, 2, 128, dtype=torch.bfloat16), torch.zeros(40, 2, 128, dtype=torch.bfloat16)
    qd, kcd, vcd = q.to(dev), kc.to(dev), vc.to(dev)
    ckopt.rope_kv_(qd, k.to(dev), v.to(dev), pos.to(dev), inv.to(dev), kcd, vcd, slots.to(dev))
    rq, rkc, rvc = oracle.rope_kv(bits16(q).reshape(32, 8, 128), bits16(k).reshape(32, 2, 128),
                                  bits16(v).reshape(32, 2, 128), pos.view(-1).numpy(), inv.numpy(),
                                  slots.view(-1).numpy(), bits16(kc), bits16(vc))
    assert np.array_equal(bits16(qd).reshape(32, 8, 128), rq)
    assert np.array_equal(bits16(kcd), rkc) and np.array_equal(bits16(vcd), rvc)


@pytest.mark.parametrize("k", [1, 50, 1024])
def test_topk_and_sampling(ckopt, oracle, dev, k):
    g = torch.Generator().manual_seed(53 + k)
    x = torch.randn(24, 60000, generator=g) * 2
    for _ in range(2):  # the second call reuses the operator's workspace and counters
        v, i = ckopt.topk(x.to(dev), k)
        rv, ri = oracle.topk(x.numpy(), k)
        assert np.array_equal(i.cpu().numpy(), ri) and np.array_equal(v.cpu().numpy(), rv)
    xb = x.bfloat16()
    vb, ib = ckopt.topk(xb.to(dev), k)
    rvb, rib = oracle.topk(bits16(xb), k, "bf16")
    assert np.array_equal(ib.cpu().numpy(), rib) and np.array_equal(bits16(vb), rvb)
    u = torch.rand(24, generator=g)
    drawn = ckopt.topk_sample(v, i, u.to(dev), 0.8, 0.9)
    v2, i2, drawn2 = ckopt.topk_and_sample(x.to(dev), k, u.to(dev), 0.8, 0.9)
    assert torch.equal(v2, v) and torch.equal(i2, i) and torch.equal(drawn2, drawn), "fused draw = two steps"
    lo, hi = oracle.topk_sample_band(rv, ri, u.numpy(), 0.8, 0.9)
    assert oracle.draw_admissible(drawn.cpu().numpy(), ri, lo, hi).all()


@pytest.mark.parametrize("k", [1, 50, 1024])
def test_topk_on_two_streams(ckopt, oracle, dev, k):
    """ckopt.topk issued on two streams at once, rows split over several chunks: the operator keeps its arrival
    counters and list workspace per (device, stream), so the two launches in flight never count arrivals on the same
    counters or write the same list slots. Four rounds, every result bit-exact against the oracle, and the counters
    left zero (a later launch on each stream is exact too)."""
    g = torch.Generator().manual_seed(60 + k)
    xa = torch.randn(64, 128256, generator=g) * 2
    xb = torch.randn(64, 128256, generator=g) * 3
    ra, rb = oracle.topk(xa.numpy(), k), oracle.topk(xb.numpy(), k)
    xad, xbd = xa.to(dev), xb.to(dev)
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    outs = []
    for rep in range(4):
        print(f"[ckopt.topk two streams] k={k} round {rep}", flush=True)
        with torch.cuda.stream(sa):
            oa = ckopt.topk(xad, k)
        with torch.cuda.stream(sb):
            ob = ckopt.topk(xbd, k)
        outs.append((oa, ob))
    torch.cuda.synchronize()
    for rep, ((va, ia), (vb, ib)) in enumerate(outs):
        assert np.array_equal(ia.cpu().numpy(), ra[1]) and np.array_equal(va.cpu().numpy(), ra[0]), f"a, round {rep}"
        assert np.array_equal(ib.cpu().numpy(), rb[1]) and np.array_equal(vb.cpu().numpy(), rb[0]), f"b, round {rep}"
    for s, x, r in ((sa, xad, ra), (sb, xbd, rb)):
        with torch.cuda.stream(s):
            v, i = ckopt.topk(x, k)
        torch.cuda.synchronize()
        assert np.array_equal(i.cpu().numpy(), r[1]) and np.array_equal(v.cpu().numpy(), r[0])


def test_errors_name_the_problem(ckopt, dev):
    with pytest.raises(RuntimeError, match="fp32 or bf16"):
        ckopt.softmax(torch.zeros(4, 4, dtype=torch.float64, device=dev))
    with pytest.raises(RuntimeError, match="k <= 1024"):
        ckopt.topk(torch.zeros(4, 2000, device=dev), 1025)
    with pytest.raises(RuntimeError, match="contiguous"):
        q = torch.zeros(1, 4, 2, 128, dtype=torch.bfloat16, device=dev).transpose(1, 2)
        ckopt.rope_(q, q, torch.zeros(1, 2, dtype=torch.long, device=dev),
                    torch.zeros(64, device=dev))
