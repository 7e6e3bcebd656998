"""GPU parity of RoPE (build/rope/libkernel.so: the reference ABI `launch` with a cos/sin cache, and the on-the-fly
`rope_launch_freq`) against the oracle, bit for bit: the kernel evaluates exactly the oracle's fp32 operations (no
contraction) and, on the fly, the same correctly rounded cos/sin. Against a cache built by torch (whose cos/sin may be
an fp32 ulp off) the on-the-fly result is identical almost everywhere and within the error such an ulp explains.
"""

import numpy as np
import pytest
import torch

from _util import bits16, ulp16

pytestmark = pytest.mark.gpu

DT = {torch.bfloat16: "bf16", torch.float16: "fp16"}
CDT = {torch.float32: "fp32", torch.bfloat16: "bf16", torch.float16: "fp16"}


def inputs(B, S, Hq, Hk, D, dtype, seed, max_pos=8192):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, S, Hq, D, generator=g).to(dtype)
    k = torch.randn(B, S, Hk, D, generator=g).to(dtype)
    pos = torch.randint(0, max_pos, (B, S), generator=g)
    return q, k, pos


def flat(t):
    return bits16(t).reshape(-1, t.shape[2], t.shape[3])


def cache_np(t):
    return t.numpy() if t.dtype == torch.float32 else bits16(t)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("cdtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(1, 5, 4, 2, 64), (2, 33, 32, 8, 128), (1, 7, 3, 1, 256), (1, 9, 2, 2, 40)])
def test_cache_path(pkg, oracle, dev, dtype, cdtype, shape):
    from oracle import torch_paths
    B, S, Hq, Hk, D = shape
    q, k, pos = inputs(B, S, Hq, Hk, D, dtype, sum(shape))
    cos, sin = torch_paths.rope_cache(8192, D, dtype=cdtype)
    print(f"[rope cache] {shape} {dtype} cache {cdtype}", flush=True)
    qo, ko = pkg.rope(q.to(dev), k.to(dev), pos.to(dev), cos=cos.to(dev), sin=sin.to(dev))
    rq, rk = oracle.rope_cache(flat(q), flat(k), cache_np(cos), cache_np(sin), pos.view(-1).numpy(), DT[dtype],
                               CDT[cdtype])
    assert np.array_equal(flat(qo), rq) and np.array_equal(flat(ko), rk)
    # out of place: the inputs are untouched
    assert np.array_equal(bits16(q), bits16(q)) and qo.data_ptr() != q.data_ptr()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(1, 5, 4, 2, 64), (2, 33, 32, 8, 128), (1, 3, 64, 64, 128), (1, 9, 2, 2, 40),
                                   (1, 4, 1, 1, 1024)])
def test_freq_path_inplace(pkg, oracle, dev, dtype, shape):
    B, S, Hq, Hk, D = shape
    q, k, pos = inputs(B, S, Hq, Hk, D, dtype, 7 * sum(shape))
    inv_freq = pkg.workloads.rope_inv_freq(D)
    print(f"[rope freq] {shape} {dtype}", flush=True)
    qd, kd = q.to(dev), k.to(dev)
    qo, ko = pkg.rope(qd, kd, pos.to(dev), inv_freq=inv_freq.to(dev), inplace=True)
    assert qo.data_ptr() == qd.data_ptr() and ko.data_ptr() == kd.data_ptr()
    rq, rk = oracle.rope_freq(flat(q), flat(k), pos.view(-1).numpy(), inv_freq.numpy(), DT[dtype])
    assert np.array_equal(flat(qd), rq) and np.array_equal(flat(kd), rk)


def test_random_shapes(pkg, oracle, dev):
    # seeded random token counts, head counts and head sizes (the vector path for D % 16 == 0, the scalar path else),
    # positions up to 2^20, both 16-bit dtypes, the cache path (three cache dtypes) and the on-the-fly path, bit for bit
    from oracle import torch_paths
    rng = np.random.default_rng(79)
    for case in range(40):
        D = int(rng.choice([16, 32, 48, 64, 80, 96, 128, 160, 256, 512, 2, 6, 40, 72, 200]))
        B, S = int(rng.integers(1, 3)), int(rng.integers(1, 300))
        Hq, Hk = int(rng.integers(1, 40)), int(rng.integers(1, 9))
        dtype = torch.bfloat16 if case % 2 else torch.float16
        far = case % 4 < 2 and case % 3 == 0  # on the fly only: a cache of 2^20 rows would not be small
        q, k, pos = inputs(B, S, Hq, Hk, D, dtype, 1000 + case, max_pos=1 << 20 if far else 8192)
        print(f"[rope random] case {case} {(B, S, Hq, Hk, D)} {dtype}", flush=True)
        if case % 4 < 2:
            inv_freq = pkg.workloads.rope_inv_freq(D)
            qo, ko = pkg.rope(q.to(dev), k.to(dev), pos.to(dev), inv_freq=inv_freq.to(dev))
            rq, rk = oracle.rope_freq(flat(q), flat(k), pos.view(-1).numpy(), inv_freq.numpy(), DT[dtype])
        else:
            cdtype = [torch.float32, torch.bfloat16, torch.float16][case % 3]
            P = int(pos.max()) + 1
            cos, sin = torch_paths.rope_cache(P, D, dtype=cdtype)
            qo, ko = pkg.rope(q.to(dev), k.to(dev), pos.to(dev), cos=cos.to(dev), sin=sin.to(dev))
            rq, rk = oracle.rope_cache(flat(q), flat(k), cache_np(cos), cache_np(sin), pos.view(-1).numpy(),
                                       DT[dtype], CDT[cdtype])
        assert np.array_equal(flat(qo), rq) and np.array_equal(flat(ko), rk), f"random case {case}"


def test_cache_path_inplace_through_abi(pkg, oracle, dev):
    from oracle import torch_paths
    q, k, pos = inputs(2, 17, 8, 2, 128, torch.bfloat16, 99)
    cos, sin = torch_paths.rope_cache(8192, 128)
    qd, kd = q.to(dev), k.to(dev)
    qo, ko = pkg.rope(qd, kd, pos.to(dev), cos=cos.to(dev), sin=sin.to(dev), inplace=True)
    rq, rk = oracle.rope_cache(flat(q), flat(k), cos.numpy(), sin.numpy(), pos.view(-1).numpy())
    assert np.array_equal(flat(qd), rq) and np.array_equal(flat(kd), rk)


def test_position_zero_is_identity_and_large_positions(pkg, oracle, dev):
    q, k, _ = inputs(1, 6, 4, 2, 128, torch.bfloat16, 5)
    pos = torch.tensor([[0, 0, 1, 65535, 1 << 20, (1 << 24) + 1]])
    inv_freq = pkg.workloads.rope_inv_freq(128)
    qo, ko = pkg.rope(q.to(dev), k.to(dev), pos.to(dev), inv_freq=inv_freq.to(dev))
    assert np.array_equal(flat(qo)[:2], flat(q)[:2])
    rq, rk = oracle.rope_freq(flat(q), flat(k), pos.view(-1).numpy(), inv_freq.numpy())
    assert np.array_equal(flat(qo), rq) and np.array_equal(flat(ko), rk)


def test_invalid_arguments(pkg, dev):
    lib = pkg.candidate("rope")._lib
    s = torch.cuda.current_stream().cuda_stream
    x = torch.zeros(4, 128, dtype=torch.bfloat16, device=dev)
    p = x.data_ptr()
    assert lib.launch(p, p, p, p, p, p, p, 0, 1, 1, 128, 1, 0, 40, 1, s) == 0       # no tokens: no-op
    assert lib.launch(p, p, p, p, p, p, p, 1, 1, 1, 127, 1, 0, 40, 1, s) == -1      # odd head_dim
    assert lib.launch(p, p, p, p, p, p, p, 1, 0, 1, 128, 1, 0, 40, 1, s) == -1      # no q heads
    assert lib.launch(p, p, p, p, p, p, p, 1, 1, 1, 128, 3, 0, 40, 1, s) == -1      # qk dtype
    assert lib.launch(p, p, p, p, p, p, p, 1, 1, 1, 128, 1, 5, 40, 1, s) == -1      # cache dtype
    assert lib.launch(p, p, p, p, p, p, p, 1, 1, 1, 128, 1, 0, 0, 1, s) == -1       # rows < 1
    assert lib.launch(p, p, p, p, p, p, p, 1, 1, 1, 128, 1, 0, 40, 70000, s) == -1  # splits
    assert lib.rope_launch_freq(p, p, p, None, p, p, 1, 1, 1, 128, 1, s) == -1      # no inv_freq


def test_config_rope_4x4096_32q_8kv_128(pkg, oracle, dev):
    inp = pkg.workloads.rope_4x4096_32q_8kv_128()
    q, k, pos, inv_freq = inp["q"], inp["k"], inp["position_ids"], inp["inv_freq"]
    qd, kd = q.to(dev), k.to(dev)
    print("[rope] config in place, on the fly", flush=True)
    pkg.rope(qd, kd, pos.to(dev), inv_freq=inv_freq.to(dev), inplace=True)
    rq, rk = oracle.rope_freq(flat(q), flat(k), pos.view(-1).numpy(), inv_freq.numpy())
    assert np.array_equal(flat(qd), rq) and np.array_equal(flat(kd), rk)
    # The reference's own path: its ABI `launch` with a cos/sin cache built by torch (HF's formula, fp32), against
    # torch eager's rotation with that cache (rope/candidate.py:3-5) on the CPU, over all 84M outputs of q and k: bit
    # for bit. (The on-the-fly form above uses correctly rounded cos/sin, which torch's are not everywhere; it differs
    # from this path in 349 outputs, 21 of them by more than one bf16 ulp, all on near-cancellations:
    # tests/test_oracle.py pins those counts on the CPU.)
    from oracle import torch_paths
    cos, sin = torch_paths.rope_cache(4096, 128)
    print("[rope] config, reference ABI with torch's fp32 cache, against torch eager", flush=True)
    qo, ko = pkg.rope(q.to(dev), k.to(dev), pos.to(dev), cos=cos.to(dev), sin=sin.to(dev))
    assert np.array_equal(bits16(qo), bits16(torch_paths.rope(q, cos, sin, pos)))
    assert np.array_equal(bits16(ko), bits16(torch_paths.rope(k, cos, sin, pos)))
    # the cache form of the same call agrees with the on-the-fly form over the oracle's table
    ct, st = oracle.rope_table(inv_freq.numpy(), 4096, 128)
    qo, ko = pkg.rope(q.to(dev), k.to(dev), pos.to(dev), cos=torch.from_numpy(ct).to(dev),
                      sin=torch.from_numpy(st).to(dev))
    assert np.array_equal(flat(qo), rq) and np.array_equal(flat(ko), rk)


def kv_case(B, S, Hq, Hk, D, dtype, seed, slots_total=None, drop=0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, S, Hq, D, generator=g).to(dtype)
    k = torch.randn(B, S, Hk, D, generator=g).to(dtype)
    v = torch.randn(B, S, Hk, D, generator=g).to(dtype)
    pos = torch.randint(0, 8192, (B, S), generator=g)
    n = slots_total or 2 * B * S
    slots = torch.randperm(n, generator=g)[: B * S].view(B, S).clone()
    if drop:
        slots.view(-1)[torch.randperm(B * S, generator=g)[:drop]] = -1  # padding tokens: no cache write
    kc = torch.randn(n, Hk, D, generator=g).to(dtype)
    vc = torch.randn(n, Hk, D, generator=g).to(dtype)
    return q, k, v, pos, slots, kc, vc


def check_kv(pkg, oracle, dev, case, inv_freq, inplace, what):
    q, k, v, pos, slots, kc, vc = case
    print(f"[rope kv] {what} q={tuple(q.shape)} k={tuple(k.shape)} {q.dtype} slots={kc.shape[0]} inplace={inplace}",
          flush=True)
    qd, kcd, vcd = q.to(dev), kc.to(dev), vc.to(dev)
    kd = k.to(dev)
    qo = pkg.rope_kv(qd, kd, v.to(dev), pos.to(dev), inv_freq.to(dev), kcd, vcd, slots.to(dev), inplace=inplace)
    rq, rkc, rvc = oracle.rope_kv(flat(q), flat(k), flat(v), pos.view(-1).numpy(), inv_freq.numpy(),
                                  slots.view(-1).numpy(), bits16(kc), bits16(vc), DT[q.dtype])
    assert np.array_equal(flat(qo), rq), f"{what}: q differs"
    assert np.array_equal(bits16(kcd), rkc), f"{what}: k cache differs"
    assert np.array_equal(bits16(vcd), rvc), f"{what}: v cache differs"
    assert np.array_equal(bits16(kd), bits16(k)), f"{what}: k was modified"
    if inplace:
        assert qo.data_ptr() == qd.data_ptr()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(1, 5, 4, 2, 64), (2, 33, 32, 8, 128), (1, 9, 2, 2, 40), (1, 4, 1, 1, 256)])
def test_rope_kv_cache_write(pkg, oracle, dev, dtype, shape):
    B, S, Hq, Hk, D = shape
    inv_freq = pkg.workloads.rope_inv_freq(D)
    case = kv_case(B, S, Hq, Hk, D, dtype, 11 * sum(shape), drop=min(3, B * S - 1))
    check_kv(pkg, oracle, dev, case, inv_freq, True, f"{shape}")
    check_kv(pkg, oracle, dev, kv_case(B, S, Hq, Hk, D, dtype, 13 * sum(shape)), inv_freq, False, f"{shape} out")


def test_config_rope_kv_4x4096_32q_8kv_128(pkg, oracle, dev):
    inp = pkg.workloads.rope_kv_4x4096_32q_8kv_128()
    case = (inp["q"], inp["k"], inp["v"], inp["position_ids"], inp["slot_mapping"], inp["k_cache"], inp["v_cache"])
    check_kv(pkg, oracle, dev, case, inp["inv_freq"], True, "rope_kv_4x4096_32q_8kv_128")
