"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the checker of the HIP kernels.

Each function of the oracle is checked against (a) the reference's own PyTorch path for the op (softmax/baseline.py:13,
the torch expressions of rmsnorm/candidate.py:3-4 and rope/candidate.py:3-5, a stable descending sort for
topk/kernel.cu:1-3) evaluated by the installed torch, (b) the committed golden fixtures made from those paths
(tests/golden/make_golden.py), and (c) what the mathematics fixes: closed forms, invariants and brute force on tiny
inputs. The last tests plant mistakes in oracle outputs and show these checks catch them.
"""

import os

import numpy as np
import pytest
import torch

from _util import assert_rel, assert_ulp, bits16, from_bits16, ulp16

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def golden(name):
    return np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False)


# ---- softmax -------------------------------------------------------------------------------------------------------


def test_softmax_fp32_matches_torch_fp64_and_fp32(oracle):
    g = torch.Generator().manual_seed(11)
    x = torch.randn(37, 1531, generator=g) * 4
    y = oracle.softmax(x.numpy(), "fp32")
    # torch's fp64 softmax rounded to fp32: at most one rounding apart
    ref64 = torch.softmax(x.double(), -1).float().numpy()
    d = np.abs(y.view(np.int32).astype(np.int64) - ref64.view(np.int32).astype(np.int64))
    assert d.max() <= 1
    # the reference's own fp32 path is within the fp32 tolerance of the fp64 oracle
    assert_rel(torch.softmax(x, -1).numpy(), y, 1e-5, "torch fp32 softmax vs oracle")


def test_softmax_subnormal_outputs_of_the_reference_path(oracle):
    # rows whose outputs reach the fp32 subnormal range (x ~ N(0, 30^2)): there the reference's own PyTorch path
    # (torch.softmax in fp32) differs from the oracle by more than 1e-5 relative on many elements, by up to 33
    # subnormal ulps (2^-149 each; the GPU tests allow the kernels 4, 2^-147); normal outputs stay within 1e-5
    g = torch.Generator().manual_seed(0)
    x = torch.randn(15, 58817, generator=g) * 30
    ref = oracle.softmax(x.numpy(), "fp32").astype(np.float64)
    t = torch.softmax(x, dim=-1).numpy().astype(np.float64)
    err = np.abs(t - ref)
    sub = np.abs(ref) < 2.0 ** -126
    assert ((err > 1e-5 * np.abs(ref)) & sub).sum() > 1000  # the relative bound alone fails the reference path
    assert 4 * 2.0 ** -149 < err[sub].max() <= 64 * 2.0 ** -149
    assert (err[~sub] <= 1e-5 * np.abs(ref[~sub])).all()


def test_softmax_invariants(oracle):
    g = torch.Generator().manual_seed(12)
    x = torch.randint(-40, 40, (9, 300), generator=g).float()
    y = oracle.softmax(x.numpy(), "fp32")
    assert np.allclose(y.astype(np.float64).sum(1), 1.0, rtol=0, atol=300 * 2 ** -24)
    # shift invariance: integer shifts keep every difference exact, so the result is bit-identical
    y2 = oracle.softmax((x + 1000).numpy(), "fp32")
    assert np.array_equal(y, y2)
    # constant row -> 1/n; a dominant entry -> one-hot; -inf -> 0
    c = oracle.softmax(np.full((2, 7), 3.25, np.float32), "fp32")
    assert np.all(c == np.float32(1.0 / 7.0))
    s = np.zeros((1, 5), np.float32)
    s[0, 2] = 1000.0
    assert np.array_equal(oracle.softmax(s, "fp32"), np.eye(5, dtype=np.float32)[2:3])
    m = np.array([[0.0, -np.inf, 0.0, -np.inf]], np.float32)
    assert np.array_equal(oracle.softmax(m, "fp32"), np.array([[0.5, 0.0, 0.5, 0.0]], np.float32))
    # a NaN anywhere makes the row NaN (torch.softmax does the same)
    n = np.array([[1.0, np.nan, 2.0]], np.float32)
    assert np.isnan(oracle.softmax(n, "fp32")).all() and torch.softmax(torch.from_numpy(n), -1).isnan().all()


def test_softmax_bf16_matches_torch(oracle):
    g = torch.Generator().manual_seed(13)
    x = (torch.randn(21, 999, generator=g) * 3).bfloat16()
    y = oracle.softmax(bits16(x), "bf16")
    ref = bits16(torch.softmax(x.double(), -1).bfloat16())  # through fp32: may round twice
    d = ulp16(y, ref)
    assert d.max() <= 1 and (d == 0).mean() > 0.999
    assert_ulp(bits16(torch.softmax(x, -1)), y, 1, "torch bf16 softmax vs oracle")


def test_softmax_golden(oracle):
    f = golden("softmax")
    y = oracle.softmax(f["x"], "fp32")
    assert_rel(y, f["y64"], 1e-7, "oracle vs torch fp64 fixture")
    assert_rel(f["y32"], y, 1e-5, "torch fp32 fixture vs oracle")
    yb = oracle.softmax(f["xb"], "bf16")
    assert_ulp(yb, f["yb"], 1, "oracle bf16 vs torch fixture")


# ---- RMSNorm -------------------------------------------------------------------------------------------------------


def _rms_torch(x, w=None, eps=1e-6):
    from oracle import torch_paths
    return torch_paths.rmsnorm(x, w, eps)


def _check_rms_against_torch(oracle, x, w, dtype_name, eps=1e-6):
    """Rows whose rounded inv agrees with torch's are bit-identical; the others differ in inv by exactly one ulp of the
    dtype (torch's fp32 sum and rsqrt sit within an fp32 ulp or two of the exact values) and must be rare."""
    y, inv = oracle.rmsnorm(bits16(x), bits16(w) if w is not None else None, eps, dtype_name, return_inv=True)
    ref = bits16(_rms_torch(x, w, eps))
    tinv = torch.rsqrt(x.float().pow(2).mean(-1) + eps).to(x.dtype)
    inv_bits = bits16(torch.from_numpy(inv).to(x.dtype))
    same = inv_bits == bits16(tinv)
    assert np.array_equal(y[same], ref[same])
    assert np.all(ulp16(inv_bits[~same], bits16(tinv)[~same]) == 1)
    assert (~same).mean() < 0.02
    return y


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_rmsnorm_matches_torch_path(oracle, dtype):
    g = torch.Generator().manual_seed(21)
    x = torch.randn(300, 512, generator=g).to(dtype)
    w = (torch.rand(512, generator=g) + 0.5).to(dtype)
    name = "bf16" if dtype == torch.bfloat16 else "fp16"
    _check_rms_against_torch(oracle, x, None, name)
    _check_rms_against_torch(oracle, x, w, name)


def test_rmsnorm_16384x4096_whole_workload_equals_torch(oracle, pkg):
    """The whole weighted RMSNorm workload (x [16384, 4096] bf16, w [4096], eps 1e-6): the oracle equals the
    reference's torch expression (rmsnorm/candidate.py:3-4, weighted as torch's w * y) bit for bit on all 67,108,864
    outputs, weighted and plain."""
    from oracle import torch_paths
    inp = pkg.workloads.rmsnorm_16384x4096()
    x, w, eps = inp["x"], inp["weight"], inp["eps"]
    assert np.array_equal(oracle.rmsnorm(bits16(x), bits16(w), eps, "bf16"), bits16(torch_paths.rmsnorm(x, w, eps)))
    assert np.array_equal(oracle.rmsnorm(bits16(x), None, eps, "bf16"), bits16(torch_paths.rmsnorm(x, None, eps)))


def test_rmsnorm_closed_forms(oracle):
    # constant row a: sum = n a^2 exactly, so every step is one fp32 rounding of a known value
    n, eps = 64, np.float32(1e-6)
    for a in (0.75, 3.0, -1.5, 1e-3):
        ab = from_bits16(oracle.f32_to_bf16_bits(np.full((1, n), a, np.float32)), torch.bfloat16)
        af = np.float32(ab[0, 0].float().item())
        mean = np.float32(np.float32(n * af * af) / np.float32(n))
        inv32 = np.float32(1.0 / np.sqrt(np.float64(np.float32(mean + eps))))
        inv = oracle.bf16_bits_to_f32(oracle.f32_to_bf16_bits(np.array([inv32])))[0]
        expect = oracle.f32_to_bf16_bits(np.full(n, af * inv, np.float32))
        assert np.array_equal(oracle.rmsnorm(bits16(ab))[0], expect)
    # scaling x by 2 halves inv exactly: the output is unchanged
    g = torch.Generator().manual_seed(22)
    x = torch.randn(50, 256, generator=g).bfloat16()
    assert np.array_equal(oracle.rmsnorm(bits16(x)), oracle.rmsnorm(bits16(x * 2)))
    # a NaN poisons its row only; a sum beyond fp32 makes inv 0 (the reference's rule)
    xn = x.clone()
    xn[3, 7] = float("nan")
    y = from_bits16(oracle.rmsnorm(bits16(xn)), torch.bfloat16)
    assert y[3].isnan().all() and not y[[0, 1, 2, 4]].isnan().any()
    big = torch.full((1, 64), 1e20).bfloat16()
    assert (from_bits16(oracle.rmsnorm(bits16(big)), torch.bfloat16) == 0).all()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_rmsnorm_add_matches_torch_path(oracle, dtype):
    """Fused residual add: h is torch's dtype sum bit for bit; y is RMSNorm of h under the same rule as above."""
    from oracle import torch_paths
    g = torch.Generator().manual_seed(23)
    x = torch.randn(300, 512, generator=g).to(dtype)
    r = (torch.randn(300, 512, generator=g) * 4).to(dtype)
    w = (torch.rand(512, generator=g) + 0.5).to(dtype)
    name = "bf16" if dtype == torch.bfloat16 else "fp16"
    for weight in (None, w):
        y, h = oracle.rmsnorm_add(bits16(x), bits16(r), None if weight is None else bits16(weight), 1e-6, name)
        ty, th = torch_paths.rmsnorm_add(x, r, weight)
        assert np.array_equal(h, bits16(th))
        assert np.array_equal(y, _check_rms_against_torch(oracle, th, weight, name))
    # a zero residual is plain RMSNorm; x + (-x) is a zero row (inv = rsqrt(eps), y = 0)
    y, h = oracle.rmsnorm_add(bits16(x), bits16(torch.zeros_like(x)), bits16(w), 1e-6, name)
    assert np.array_equal(y, oracle.rmsnorm(bits16(x), bits16(w), 1e-6, name)) and np.array_equal(h, bits16(x))
    y, h = oracle.rmsnorm_add(bits16(x), bits16(-x), None, 1e-6, name)
    assert not from_bits16(h, dtype).float().abs().any() and not from_bits16(y, dtype).float().abs().any()


def test_rmsnorm_golden(oracle):
    f = golden("rmsnorm")
    y = oracle.rmsnorm(f["x"], f["w"], 1e-6, "bf16")
    same = f["inv_torch"] == oracle.f32_to_bf16_bits(oracle.rmsnorm(f["x"], None, 1e-6, "bf16", True)[1])
    assert same.mean() > 0.98
    assert np.array_equal(y[same], f["y"][same])


# ---- RoPE ----------------------------------------------------------------------------------------------------------


def _rope_torch(q, k, cos, sin, ids):
    from oracle import torch_paths
    return torch_paths.rope(q, cos, sin, ids), torch_paths.rope(k, cos, sin, ids)


@pytest.mark.parametrize("qdt,cdt", [(torch.bfloat16, torch.float32), (torch.float16, torch.float32),
                                     (torch.bfloat16, torch.bfloat16), (torch.float16, torch.float16)])
def test_rope_cache_matches_torch_bitwise(oracle, qdt, cdt):
    from oracle import torch_paths
    g = torch.Generator().manual_seed(31)
    T, Hq, Hk, D, P = 40, 4, 2, 64, 4096
    q = torch.randn(T, Hq, D, generator=g).to(qdt)
    k = torch.randn(T, Hk, D, generator=g).to(qdt)
    ids = torch.randint(0, P, (T,), generator=g)
    cos, sin = torch_paths.rope_cache(P, D, dtype=cdt)
    rq, rk = _rope_torch(q, k, cos, sin, ids)
    name = "bf16" if qdt == torch.bfloat16 else "fp16"
    cname = {torch.float32: "fp32", torch.bfloat16: "bf16", torch.float16: "fp16"}[cdt]
    cnp = (lambda t: t.numpy()) if cdt == torch.float32 else bits16
    oq, ok = oracle.rope_cache(bits16(q), bits16(k), cnp(cos), cnp(sin), ids.numpy(), name, cname)
    assert np.array_equal(oq, bits16(rq)) and np.array_equal(ok, bits16(rk))


def test_rope_brute_force_and_identities(oracle):
    g = torch.Generator().manual_seed(32)
    T, H, D = 3, 2, 8
    q = torch.randn(T, H, D, generator=g).bfloat16()
    k = torch.randn(T, 1, D, generator=g).bfloat16()
    inv_freq = torch.tensor([1.0, 0.1, 0.01, 0.001])
    ids = np.array([0, 7, 4095], np.int64)
    oq, ok = oracle.rope_freq(bits16(q), bits16(k), ids, inv_freq.numpy())
    qf = q.float().numpy()
    f32 = np.float32
    for t in range(T):
        for h in range(H):
            for i in range(D // 2):
                ang = f32(f32(ids[t]) * f32(inv_freq[i].item()))
                c, s = f32(np.cos(np.float64(ang))), f32(np.sin(np.float64(ang)))
                a, b = qf[t, h, i], qf[t, h, i + D // 2]
                ea = f32(f32(a * c) - f32(b * s))
                eb = f32(f32(b * c) + f32(a * s))
                assert oq[t, h, i] == oracle.f32_to_bf16_bits(np.array([ea]))[0]
                assert oq[t, h, i + D // 2] == oracle.f32_to_bf16_bits(np.array([eb]))[0]
    # position 0 is the identity
    assert np.array_equal(oq[0], bits16(q)[0]) and np.array_equal(ok[0], bits16(k)[0])
    # the on-the-fly form equals the cache form over the table it evaluates
    cos, sin = oracle.rope_table(inv_freq.numpy(), 4096, D)
    cq, ck = oracle.rope_cache(bits16(q), bits16(k), cos, sin, ids)
    assert np.array_equal(cq, oq) and np.array_equal(ck, ok)
    # each pair's norm is preserved up to the two roundings
    g2 = torch.Generator().manual_seed(33)
    x = torch.randn(64, 8, 128, generator=g2).bfloat16()
    pos = np.arange(64, dtype=np.int64) * 61
    from oracle import torch_paths
    xo, _ = oracle.rope_freq(bits16(x), bits16(x[:, :1]), pos, torch_paths.inv_freq(128).numpy())
    a, b = x.float()[..., :64], x.float()[..., 64:]
    yo = from_bits16(xo, torch.bfloat16).float()
    ya, yb = yo[..., :64], yo[..., 64:]
    assert torch.allclose(ya * ya + yb * yb, a * a + b * b, rtol=2 ** -6, atol=1e-3)


def test_rope_freq_vs_torch_cache(oracle):
    """Against a cache built by torch (whose cos/sin may differ from the correctly rounded values by an fp32 ulp):
    within 1 bf16 ulp, and identical almost everywhere."""
    from oracle import torch_paths
    g = torch.Generator().manual_seed(34)
    T, D = 4096, 128
    q = torch.randn(T, 2, D, generator=g).bfloat16()
    k = torch.randn(T, 1, D, generator=g).bfloat16()
    ids = torch.arange(T)
    cos, sin = torch_paths.rope_cache(T, D)
    rq, rk = _rope_torch(q, k, cos, sin, ids)
    oq, ok = oracle.rope_freq(bits16(q), bits16(k), ids.numpy(), torch_paths.inv_freq(D).numpy())
    d = ulp16(oq, bits16(rq))
    assert (d == 0).mean() > 0.99
    # where a * cos and b * sin nearly cancel, an fp32 ulp of torch's cos/sin can move the result by a few bf16 ulps
    of = torch.from_numpy(oq.view(np.int16)).view(torch.bfloat16).float()
    tf = rq.float()
    xa = q.float().abs()
    pair = xa + torch.cat((xa[..., 64:], xa[..., :64]), -1)
    assert ((of - tf).abs() <= tf.abs() * 2 ** -7 + pair * 2 ** -22).all()


def test_rope_4x4096_on_the_fly_vs_torch_cache_whole_workload(oracle, pkg):
    """The whole RoPE workload (q [4, 4096, 32, 128] and k [4, 4096, 8, 128] bf16, positions 0..4095, theta 1e4): the
    on-the-fly form (cos/sin of the fp32 angle, correctly rounded from fp64) against the reference's PyTorch path with
    a cos/sin cache built by torch, over all 83,886,080 outputs. torch's cos/sin differ from the correctly rounded
    values by one fp32 ulp in about 5% of the cache's entries. That moves 349 outputs (274 of q, 75 of k) by at least
    one bf16 ulp. 21 move by more than one ulp (15 of q, at most 32 ulp; 6 of k, at most 26,112 ulp), each where
    a * cos and b * sin nearly cancel, so the difference is tiny in absolute terms: the bound below is the error an
    fp32 ulp of cos or sin can cause, plus the output's own rounding."""
    from oracle import torch_paths
    inp = pkg.workloads.rope_4x4096_32q_8kv_128()
    q, k, pos, inv = inp["q"], inp["k"], inp["position_ids"], inp["inv_freq"]
    assert torch.equal(inv, torch_paths.inv_freq(128))
    oq, ok = oracle.rope_freq(bits16(q).reshape(-1, 32, 128), bits16(k).reshape(-1, 8, 128), pos.view(-1).numpy(),
                              inv.numpy())
    cos, sin = torch_paths.rope_cache(4096, 128)
    ct, st = oracle.rope_table(inv.numpy(), 4096, 128)
    off = (ct != cos.numpy()).mean(), (st != sin.numpy()).mean()
    assert 0.03 < off[0] < 0.08 and 0.03 < off[1] < 0.08, off
    total_beyond = 0
    for x, o, name, n1, nmax in ((q, oq, "q", 274, 32), (k, ok, "k", 75, 26112)):
        t = torch_paths.rope(x, cos, sin, pos)
        d = ulp16(o.reshape(-1), bits16(t).reshape(-1))
        assert (d > 0).sum() == n1, (name, int((d > 0).sum()))
        assert d.max() == nmax, (name, int(d.max()))
        total_beyond += int((d > 1).sum())
        of = torch.from_numpy(o.reshape(t.shape).view(np.int16)).view(torch.bfloat16).float()
        tf = t.float()
        xa = x.float().abs()
        pair = xa + torch.cat((xa[..., 64:], xa[..., :64]), -1)
        assert ((of - tf).abs() <= tf.abs() * 2 ** -7 + pair * 2 ** -22).all(), name
    assert total_beyond == 21


def test_rope_kv_scatter_semantics(oracle):
    """The fused cache write: q and the scattered k rows are the frequency form's rotation, v rows are copied, a
    negative slot writes nothing and untouched rows keep their contents (checked element by element)."""
    g = torch.Generator().manual_seed(34)
    T_, H, Hk, D, S = 9, 4, 2, 64, 16
    q, k, v = (torch.randn(T_, H, D, generator=g).bfloat16(), torch.randn(T_, Hk, D, generator=g).bfloat16(),
               torch.randn(T_, Hk, D, generator=g).bfloat16())
    ids = torch.randint(0, 100, (T_,), generator=g)
    slots = torch.tensor([3, 0, -1, 15, 7, -1, 8, 1, 12])
    inv = torch.rand(D // 2, generator=g)
    kc0 = bits16(torch.randn(S, Hk, D, generator=g).bfloat16())
    vc0 = bits16(torch.randn(S, Hk, D, generator=g).bfloat16())
    qo, kc, vc = oracle.rope_kv(bits16(q), bits16(k), bits16(v), ids.numpy(), inv.numpy(), slots.numpy(), kc0, vc0)
    rq, rk = oracle.rope_freq(bits16(q), bits16(k), ids.numpy(), inv.numpy())
    assert np.array_equal(qo, rq)
    written = {int(s_): t for t, s_ in enumerate(slots.tolist()) if s_ >= 0}
    for slot in range(S):
        if slot in written:
            assert np.array_equal(kc[slot], rk[written[slot]]) and np.array_equal(vc[slot], bits16(v)[written[slot]])
        else:
            assert np.array_equal(kc[slot], kc0[slot]) and np.array_equal(vc[slot], vc0[slot])


def test_rope_golden(oracle):
    f = golden("rope")
    oq, ok = oracle.rope_cache(f["q"], f["k"], f["cos"], f["sin"], f["ids"])
    assert np.array_equal(oq, f["q_out"]) and np.array_equal(ok, f["k_out"])


# ---- top-k ---------------------------------------------------------------------------------------------------------


def test_topk_matches_stable_sort_and_topk(oracle):
    g = torch.Generator().manual_seed(41)
    x = torch.randn(16, 3000, generator=g) * 2
    for k in (1, 7, 50, 1024):
        v, i = oracle.topk(x.numpy(), k)
        sv, si = torch.sort(x, dim=-1, descending=True, stable=True)
        assert np.array_equal(i, si[:, :k].numpy()) and np.array_equal(v, sv[:, :k].numpy())
        # torch.topk leaves the order of equal values open (random fp32 rows do hold a few ties): values must agree,
        # indices wherever the value is unique in the row
        tv, ti = torch.topk(x, k, -1, sorted=True)
        assert np.array_equal(v, tv.numpy())
        xs = x.numpy()
        unique = np.array([[np.count_nonzero(xs[r] == val) == 1 for val in v[r]] for r in range(x.shape[0])])
        assert np.array_equal(i[unique], ti.numpy()[unique]) and unique.mean() > 0.99


def test_topk_ties_and_special_values(oracle):
    # ties: lowest index first, like a stable descending sort
    g = torch.Generator().manual_seed(42)
    x = torch.randint(0, 5, (8, 500), generator=g).float()
    v, i = oracle.topk(x.numpy(), 60)
    sv, si = torch.sort(x, dim=-1, descending=True, stable=True)
    assert np.array_equal(i, si[:, :60].numpy())
    # all equal -> indices 0..k-1; k = 1 is the first argmax
    v, i = oracle.topk(np.full((3, 100), 2.5, np.float32), 10)
    assert np.array_equal(i, np.tile(np.arange(10), (3, 1)))
    y = torch.randn(5, 777, generator=g)
    y[:, 100] = y[:, 300] = 9.0
    _, i1 = oracle.topk(y.numpy(), 1)
    assert np.array_equal(i1[:, 0], np.argmax(y.numpy(), 1)) and (i1[:, 0] == 100).all()
    # the composite order of topk/kernel.cu:56-60: +0 above -0, +NaN above +inf, -inf above -NaN
    z = np.array([[-0.0, 0.0, -np.inf, np.inf, np.float32("nan"), -np.float32("nan"), 1.0]], np.float32)
    _, iz = oracle.topk(z, 7)
    assert list(iz[0]) == [4, 3, 6, 1, 0, 2, 5]


def test_topk_bf16_and_brute_force(oracle):
    g = torch.Generator().manual_seed(43)
    x = (torch.randn(6, 211, generator=g)).bfloat16()
    v, i = oracle.topk(bits16(x), 13, "bf16")
    xb = bits16(x)
    for r in range(6):
        def comp(j):
            u = int(xb[r, j]) << 16
            key = (~u & 0xFFFFFFFF) if u & 0x80000000 else (u | 0x80000000)
            return (key << 32) | (~j & 0xFFFFFFFF)
        order = sorted(range(211), key=comp, reverse=True)[:13]
        assert list(i[r]) == order and list(v[r]) == [xb[r, j] for j in order]


def test_topk_golden(oracle):
    f = golden("topk")
    for k in (1, 50, 1024):
        v, i = oracle.topk(f["x"], k)
        assert np.array_equal(v, f[f"v{k}"]) and np.array_equal(i, f[f"i{k}"])


# ---- the checks catch planted mistakes -------------------------------------------------------------------------------


def test_planted_mistakes_are_caught(oracle):
    g = torch.Generator().manual_seed(51)
    # softmax: a sum over the wrong row, or a missing division, leaves the tolerance
    x = torch.randn(4, 200, generator=g)
    y = oracle.softmax(x.numpy(), "fp32")
    with pytest.raises(AssertionError):
        assert_rel(y[[1, 0, 2, 3]], torch.softmax(x.double(), -1).numpy(), 1e-5)
    with pytest.raises(AssertionError):
        assert_rel(y * np.float32(1 + 3e-5), torch.softmax(x.double(), -1).numpy(), 1e-5)
    # rmsnorm: inv not rounded to bf16 before the product changes most rows
    xb = torch.randn(64, 256, generator=g).bfloat16()
    inv32 = torch.rsqrt(xb.float().pow(2).mean(-1, keepdim=True) + 1e-6)
    wrong = bits16((xb.float() * inv32).bfloat16())
    assert (oracle.rmsnorm(bits16(xb)) != wrong).any(axis=1).mean() > 0.5
    # rope: a sign flip of the sin term or swapped halves is visible everywhere but position 0
    from oracle import torch_paths
    q = torch.randn(8, 1, 32, generator=g).bfloat16()
    cos, sin = torch_paths.rope_cache(8, 32)
    good = oracle.rope_cache(bits16(q), bits16(q), cos.numpy(), sin.numpy(), np.arange(8))[0]
    bad = bits16(torch_paths.rope(q, cos, -sin, torch.arange(8)))
    assert (good[1:] != bad[1:]).mean() > 0.5
    # top-k: an index off by one or a reversed tie order fails the stable-sort check
    t = torch.randint(0, 3, (2, 100), generator=g).float()
    _, i = oracle.topk(t.numpy(), 20)
    si = torch.sort(t, dim=-1, descending=True, stable=True)[1][:, :20].numpy()
    assert np.array_equal(i, si) and not np.array_equal(i + 1, si)
    assert not np.array_equal(i, torch.sort(t.flip(-1), dim=-1, descending=True, stable=True)[1][:, :20].numpy())


# ---- sampling from a top-k list --------------------------------------------------------------------------------------


def _sorted_list(rows, k, seed, scale=2.0):
    g = torch.Generator().manual_seed(seed)
    v, i = torch.sort(torch.randn(rows, 4 * k, generator=g) * scale, dim=-1, descending=True, stable=True)
    return v[:, :k].contiguous().numpy(), i[:, :k].contiguous().numpy()


def test_topk_sample_inverse_cdf(oracle):
    """temperature and no nucleus cut: the draw is the inverse CDF of softmax(v / T) at u, computed independently."""
    v, i = _sorted_list(200, 50, 41)
    u = np.random.default_rng(1).random(200, dtype=np.float32)
    for T in (0.5, 1.0, 2.0):
        got, amb = oracle.topk_sample(v, i, u, T, 1.0)
        p = np.exp((v.astype(np.float64) - v[:, :1]) / T)
        c = np.cumsum(p, axis=1)
        pos = np.array([np.searchsorted(c[r], u[r] * c[r, -1], side="right") for r in range(200)])
        expect = i[np.arange(200), np.minimum(pos, 49)]
        # ambiguous: u lands within fp32 rounding of an interval edge (common only among a peaked list's tail entries,
        # whose intervals are narrower than that)
        assert np.array_equal(got[~amb], expect[~amb]) and amb.mean() < 0.1


def test_topk_sample_nucleus_and_greedy(oracle):
    v, i = _sorted_list(100, 64, 42)
    p = np.exp(v.astype(np.float64) - v[:, :1])
    c = np.cumsum(p, axis=1)
    for top_p in (0.2, 0.6, 0.95):
        kept = 1 + np.sum(c[:, :-1] < top_p * c[:, -1:], axis=1)
        # u just below 1 draws the last kept position; u = 0 draws the first
        hi, amb = oracle.topk_sample(v, i, np.full(100, 1 - 2 ** -24, np.float32), 1.0, top_p)
        ok = ~amb
        assert np.array_equal(hi[ok], i[np.arange(100), kept - 1][ok])
        lo, _ = oracle.topk_sample(v, i, np.zeros(100, np.float32), 1.0, top_p)
        assert np.array_equal(lo, i[:, 0])
    g0, _ = oracle.topk_sample(v, i, np.full(100, 0.7, np.float32), 0.0, 0.5)
    assert np.array_equal(g0, i[:, 0])


def test_topk_sample_frequencies(oracle):
    """A regular grid of u draws each kept position in proportion to its renormalised probability."""
    v, i = _sorted_list(1, 8, 43)
    n = 4096
    u = ((np.arange(n) + 0.5) / n).astype(np.float32)
    got, _ = oracle.topk_sample(np.repeat(v, n, 0), np.repeat(i, n, 0), u, 0.8, 0.9)
    p = np.exp((v[0].astype(np.float64) - v[0, 0]) / 0.8)
    c = np.cumsum(p)
    kept = 1 + int(np.sum(c[:-1] < 0.9 * c[-1]))
    q = p[:kept] / c[kept - 1]
    freq = np.array([(got == i[0, j]).mean() for j in range(kept)])
    assert np.abs(freq - q).max() < 2.0 / n and set(got) <= set(i[0, :kept])


def _fp32_draws(v, i, u, T, top_p, order):
    """The draw rule evaluated in fp32 with a given association of the prefix sums: 'seq' (left to right), 'blocks'
    (sums inside blocks of 16, then across blocks, as a wave of lanes holding 16 each would), 'rev' (each prefix sum
    accumulated from its last term back to its first)."""
    x = (v.astype(np.float32) / np.float32(T)).astype(np.float32)
    e = np.exp((x - x.max(axis=1, keepdims=True)).astype(np.float32)).astype(np.float32)
    rows, k = e.shape
    S = np.empty_like(e)
    for r in range(rows):
        if order == "seq":
            S[r] = np.cumsum(e[r], dtype=np.float32)
        elif order == "blocks":
            acc = np.float32(0)
            for b in range(0, k, 16):
                part = np.cumsum(e[r, b:b + 16], dtype=np.float32)
                S[r, b:b + 16] = (part + acc).astype(np.float32)
                acc = np.float32(acc + part[-1])
        else:
            S[r] = [np.sum(e[r, :j + 1][::-1], dtype=np.float32) for j in range(k)]
    out = np.empty(rows, dtype=np.int64)
    for r in range(rows):
        tot = S[r, -1]
        kept = k if top_p >= 1 else 1 + int(np.sum(S[r, :-1] < np.float32(top_p) * tot))
        target = np.float32(u[r]) * S[r, kept - 1]
        above = np.nonzero(S[r, :kept] > target)[0]
        out[r] = i[r, above[0] if len(above) else kept - 1]
    return out


def test_topk_sample_band_holds_every_fp32_evaluation(oracle):
    """The admissible band contains the exact (fp64) draw and the draws of the rule evaluated in fp32 under three
    associations of the prefix sums; it is one position wide on most rows (wider only where u or the nucleus cut lies
    within rounding of a boundary), and never more than three."""
    for k, seed in ((50, 51), (300, 52), (1024, 53)):
        v, i = _sorted_list(48, k, seed)
        u = np.random.default_rng(seed).random(48, dtype=np.float32)
        for T, top_p in ((0.8, 0.9), (1.0, 1.0), (0.5, 0.3)):
            exact, amb = oracle.topk_sample(v, i, u, T, top_p)
            lo, hi = oracle.topk_sample_band(v, i, u, T, top_p)
            assert oracle.draw_admissible(exact, i, lo, hi).all()
            assert (hi - lo).max() <= 2 and (hi > lo).mean() <= max(0.1, amb.mean())
            for order in ("seq", "blocks", "rev"):
                d = _fp32_draws(v, i, u, T, top_p, order)
                assert oracle.draw_admissible(d, i, lo, hi).all(), (k, T, top_p, order)


def test_topk_sample_band_rejects_a_wrong_draw(oracle):
    # a draw one position off (the planted mistake of an off-by-one search) falls outside the band on most rows
    v, i = _sorted_list(200, 64, 54)
    u = np.random.default_rng(3).random(200, dtype=np.float32)
    exact, _ = oracle.topk_sample(v, i, u, 1.0, 1.0)
    lo, hi = oracle.topk_sample_band(v, i, u, 1.0, 1.0)
    pos = np.argmax(i == exact[:, None], axis=1)
    shifted = i[np.arange(200), np.minimum(pos + 1, 63)]
    assert oracle.draw_admissible(shifted, i, lo, hi).mean() < 0.1
