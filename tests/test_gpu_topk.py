"""GPU parity of top-k (build/topk/libkernel.so: `plan`, `launch`, `topk_reset`) against the oracle, bit for bit:
values (the element bits) and int64 indices, sorted descending with ties by the lowest index.

Covers single- and multi-chunk rows (the merge by the row's last workgroup to arrive, counted on the caller's
counters and handed over in the caller's work), every k class (1, the lane-maxima bound up to 64, the general path up
to 1024), ties and special values, negative rows and the all-ones NaN (the value the k <= 64 kernel pads tiles with),
bf16, unaligned and ragged rows, short last tiles, workspace reuse across shapes, work and outputs holding stale
bytes on entry, the counters' reset and self-reset, adversarial orders that force many prunes, the top-k workload at
k = 1, 50 and 1024, and the draw fused into the launch.
"""

import numpy as np
import pytest
import torch

from _util import bits16

pytestmark = pytest.mark.gpu


def lib(pkg):
    return pkg.candidate("topk")._lib


def run_abi(pkg, x, k, chunk=None, poison=False):
    """Launch through the C-ABI with an explicit chunk (None: plan's). poison: work, values and indices start as all
    ones (the kernels must not depend on what the caller's buffers held)."""
    cand = pkg.candidate("topk")
    L = lib(pkg)
    rows, cols = x.shape
    dtype = 0 if x.dtype == torch.float32 else 1
    if chunk is None:
        chunk = L.plan(rows, cols, dtype, 256, 4, max(4096, 16 * k))
    nchunks = -(-cols // chunk)
    work = torch.empty(max(1, rows * nchunks * k), dtype=torch.int64, device=x.device)
    counters = torch.zeros(max(rows, 1), dtype=torch.int32, device=x.device)
    vals = torch.empty(rows, k, dtype=x.dtype, device=x.device)
    idx = torch.empty(rows, k, dtype=torch.int64, device=x.device)
    if poison:
        for t in (work, vals, idx):
            t.view(torch.uint8).fill_(0xFF)
    err = L.launch(x.data_ptr(), vals.data_ptr(), idx.data_ptr(), work.data_ptr(), counters.data_ptr(), rows, cols, k,
                   dtype, 256, 4, chunk, torch.cuda.current_stream().cuda_stream)
    assert err == 0
    torch.cuda.synchronize()
    assert (counters == 0).all(), "the row counters must be left at zero"
    return vals, idx, nchunks


def expect(oracle, x, k):
    if x.dtype == torch.float32:
        return oracle.topk(x.cpu().numpy(), k, "fp32")
    return oracle.topk(bits16(x), k, "bf16")


def check(pkg, oracle, x_cpu, k, dev, chunk=None, what="", poison=False):
    print(f"[topk] {what} {tuple(x_cpu.shape)} {x_cpu.dtype} k={k} chunk={chunk}", flush=True)
    vals, idx, nchunks = run_abi(pkg, x_cpu.to(dev), k, chunk, poison)
    rv, ri = expect(oracle, x_cpu, k)
    got_i = idx.cpu().numpy()
    got_v = vals.cpu().numpy() if x_cpu.dtype == torch.float32 else bits16(vals)
    if not np.array_equal(got_i, ri):
        bad = np.argwhere(got_i != ri)
        r, j = bad[0]
        raise AssertionError(f"{what}: indices differ at {len(bad)} places (nchunks={nchunks}); first row {r} "
                             f"pos {j}: got {got_i[r, max(0, j - 2):j + 3]} ref {ri[r, max(0, j - 2):j + 3]}")
    assert np.array_equal(got_v.view(np.uint32) if got_v.dtype == np.float32 else got_v,
                          rv.view(np.uint32) if rv.dtype == np.float32 else rv), f"{what}: values differ"
    return nchunks


@pytest.mark.parametrize("k", [1, 2, 7, 50, 64, 65, 128, 300, 1024])
def test_k_classes_single_and_split(pkg, oracle, dev, k):
    g = torch.Generator().manual_seed(k)
    x = torch.randn(6, 20000, generator=g) * 2
    check(pkg, oracle, x, k, dev, chunk=None, what="planned")
    check(pkg, oracle, x, k, dev, chunk=20000, what="one chunk")
    assert check(pkg, oracle, x, k, dev, chunk=4096, what="five chunks") == 5
    check(pkg, oracle, x, k, dev, chunk=2052, what="ten chunks")


@pytest.mark.parametrize("rows,cols,k", [(1, 128256, 50), (64, 151936, 50), (512, 32000, 50), (3, 1000, 50),
                                         (2, 50, 50), (4, 1024, 1024), (1, 4097, 1024), (7, 10001, 13)])
def test_shapes(pkg, oracle, dev, rows, cols, k):
    g = torch.Generator().manual_seed(rows * 31 + cols + k)
    check(pkg, oracle, torch.randn(rows, cols, generator=g) * 2, k, dev, what="shape")


def test_ties_and_special_values(pkg, oracle, dev):
    g = torch.Generator().manual_seed(3)
    x = torch.randint(0, 6, (5, 30000), generator=g).float()  # massive ties: lowest indices win
    for k in (1, 50, 1024):
        check(pkg, oracle, x, k, dev, chunk=4096, what="ties")
    e = torch.full((3, 9000), 1.25)  # all equal
    check(pkg, oracle, e, 1024, dev, chunk=4096, what="all equal")
    check(pkg, oracle, e, 40, dev, what="all equal")
    s = torch.randn(2, 5000, generator=g)
    s[0, 10], s[0, 20], s[0, 30], s[0, 40] = 0.0, -0.0, float("inf"), float("-inf")
    s[1, 11], s[1, 12] = float("nan"), -float("nan")
    s[1, 100:200] = float("inf")
    check(pkg, oracle, s, 150, dev, what="special")
    check(pkg, oracle, s, 7, dev, chunk=1000, what="special split")


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_wide_merge_six_lists(pkg, oracle, dev, dt):
    # six lists of 1024 in the k > 64 merge; with ties every list entry reaches the floor, and the merge prunes to k
    # while it gathers
    g = torch.Generator().manual_seed(21)
    x = (torch.randn(3, 6 * 16384, generator=g) * 2).to(dt)
    assert check(pkg, oracle, x, 1024, dev, chunk=16384, what="six lists") == 6
    t = torch.randint(0, 6, (3, 6 * 16384), generator=g).float().to(dt)
    check(pkg, oracle, t, 1024, dev, chunk=16384, what="six lists, ties")
    check(pkg, oracle, t, 700, dev, chunk=16384, what="six lists, ties")


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_naive_tier(pkg, oracle, dev, dt):
    # the naive tier (tuning slot 1: the harness's seed column), one scan of the row per output position, against the
    # oracle: ties, every k class, unaligned lengths
    L = lib(pkg)
    g = torch.Generator().manual_seed(31)
    cases = [(torch.randn(3, 5000, generator=g) * 2, 50), (torch.randint(0, 6, (2, 3001), generator=g).float(), 64),
             (torch.randn(2, 1001, generator=g), 1), (torch.randn(2, 2003, generator=g), 300)]
    assert L.topk_tune(1, 1) == 0
    try:
        for x, k in cases:
            check(pkg, oracle, x.to(dt), k, dev, what="naive tier")
    finally:
        assert L.topk_tune(1, 0) == 0


def test_adversarial_orders(pkg, oracle, dev):
    # ascending rows: every tile beats the threshold so far (many prunes); descending: the first tile is the answer
    a = torch.arange(40000, dtype=torch.float32).view(1, -1).repeat(2, 1)
    a[1] = a[1].flip(0)
    for k in (1, 50, 1024):
        check(pkg, oracle, a, k, dev, chunk=8192, what="monotone")
        check(pkg, oracle, a, k, dev, chunk=40000, what="monotone one chunk")
    # a cluster of near-equal large values that a coarse histogram cannot split
    g = torch.Generator().manual_seed(4)
    c = torch.randn(2, 30000, generator=g)
    c[:, ::3] = 5.0 + torch.arange(10000).float() * 1e-7
    check(pkg, oracle, c, 1024, dev, what="cluster")


def test_negative_rows_and_all_ones_nan(pkg, oracle, dev):
    # log-probabilities: every value negative, so the bound and the admission compare work on reversed bit orders
    g = torch.Generator().manual_seed(6)
    lp = torch.log_softmax(torch.randn(4, 40000, generator=g) * 3, dim=-1)
    for k in (1, 50):
        check(pkg, oracle, lp, k, dev, what="log-probs")
        check(pkg, oracle, lp, k, dev, chunk=8192, what="log-probs split")
    # the all-ones NaN (bits 0xffffffff, the lowest key) among values, as the whole row but one, and as the k-th
    x = torch.randn(3, 20000, generator=g)
    xi = x.view(torch.int32)
    xi[0, ::7] = -1
    xi[1] = -1
    x[1, 5] = 1.0
    xi[2, :19990] = -1
    for k in (1, 13, 50):
        check(pkg, oracle, x, k, dev, what="all-ones nan")
        check(pkg, oracle, x, k, dev, chunk=4096, what="all-ones nan split")
    xb = torch.randn(3, 20000, generator=g).bfloat16()
    xbi = xb.view(torch.int16)
    xbi[0, ::7] = -1
    xbi[1] = -1
    xb[1, 5] = 1.0
    xbi[2, :19990] = -1
    for k in (1, 50):
        check(pkg, oracle, xb, k, dev, what="bf16 all-ones nan")
        check(pkg, oracle, xb, k, dev, chunk=4096, what="bf16 all-ones nan split")


def test_handoff_workspace_across_shapes(pkg, oracle, dev):
    # back-to-back split launches of growing and shrinking shapes on one stream, each with fresh caller buffers: every
    # launch must leave the counters all zeros; topk_reset clears them as well
    g = torch.Generator().manual_seed(7)
    shapes = [(2, 9000, 7, 2048), (512, 32000, 64, 1024), (3, 20000, 64, 1024), (64, 40000, 50, 4096),
              (2, 9000, 7, 2048)]
    for rows, cols, k, chunk in shapes:
        check(pkg, oracle, torch.randn(rows, cols, generator=g), k, dev, chunk=chunk, what="hand-off reuse")
    counters = torch.zeros(8, dtype=torch.int32, device=dev)
    assert lib(pkg).topk_reset(counters.data_ptr(), 8, torch.cuda.current_stream().cuda_stream) == 0
    check(pkg, oracle, torch.randn(5, 30000, generator=g), 50, dev, chunk=4096, what="after reset")


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("k", [1, 13, 50, 64, 100, 1024])
def test_short_last_tiles(pkg, oracle, dev, dt, k):
    # chunks whose last register tile leaves whole waves without data, or holds fewer lanes or groups than k: such a
    # tile has no admission bound and is pushed again, exactly, over its vectors (the re-push path). For k <= 64 the
    # launch folds a last chunk shorter than one vector per lane into the previous one when both fit one tile, so the
    # 2048-column cases reach that path only inside the fold; a multi-tile chunk plus a short tail (2 x 16384 + 640:
    # 160 fp32 or 80 bf16 vectors, so waves 2 and 3 hold none) still reaches it for both dtypes. The k > 64 kernel
    # picks its own chunk, so its tails come from the column counts.
    g = torch.Generator().manual_seed(900 + k)
    for cols, chunk in [(62 * 2048 + 1280, 2048), (3 * 2048 + 40, 2048), (2 * 17664, 17664), (2 * 16384 + 1280, 16384),
                        (2 * 16384 + 640, 16384), (16384 + 136, None), (1000, None)]:
        if k <= cols:
            x = (torch.randn(3, cols, generator=g) * 2).to(dt)
            check(pkg, oracle, x, k, dev, chunk=chunk, what="short last tile")


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_folded_last_chunk_bounds(pkg, oracle, dev, dt):
    # a last chunk shorter than one vector per lane is folded into the previous chunk when both fit one register tile:
    # tails on either side of that length, and previous chunks on either side of the tile's end
    w = 4 if dt == torch.float32 else 8
    short = 256 * w  # the length at which each of the four waves holds a vector
    g = torch.Generator().manual_seed(77)
    cases = [(2048, short - w), (2048, short), (2048, w), (16384 - (short - w), short - w),
             (16384 - (short - w) + 8, short - w)]
    for chunk, tail in cases:
        cols = 3 * chunk + tail
        x = (torch.randn(2, cols, generator=g) * 2).to(dt)
        for k in (1, 13, 64):
            check(pkg, oracle, x, k, dev, chunk=chunk, what=f"fold chunk={chunk} tail={tail}")


def test_bf16_and_unaligned(pkg, oracle, dev):
    g = torch.Generator().manual_seed(5)
    xb = torch.randn(8, 50000, generator=g).bfloat16()
    for k in (1, 50, 1024):
        check(pkg, oracle, xb, k, dev, what="bf16")
    check(pkg, oracle, xb[:, :49999].contiguous(), 50, dev, what="bf16 ragged")
    base = torch.randn(3 * 20000 + 1, generator=g).to(dev)
    x = base[1:].view(3, 20000)  # 4 bytes past a 16-byte boundary: scalar loads
    vals, idx, _ = run_abi(pkg, x, 50, 4096)
    rv, ri = oracle.topk(x.cpu().numpy(), 50)
    assert np.array_equal(idx.cpu().numpy(), ri) and np.array_equal(vals.cpu().numpy(), rv)


def test_workspace_reuse_and_wrapper(pkg, oracle, dev):
    g = torch.Generator().manual_seed(6)
    for i in range(3):  # the wrapper caches plan, workspace and counters across calls of one shape
        x = torch.randn(16, 60000, generator=g)
        v, ix = pkg.topk(x.to(dev), 50)
        rv, ri = oracle.topk(x.numpy(), 50)
        assert np.array_equal(ix.cpu().numpy(), ri) and np.array_equal(v.cpu().numpy(), rv)
    counters = pkg.candidate("topk")._buffers.counters[(dev, torch.cuda.current_stream(dev).cuda_stream)]
    assert (counters == 0).all()
    assert lib(pkg).topk_reset(counters.data_ptr(), counters.numel(), torch.cuda.current_stream().cuda_stream) == 0


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_stale_caller_buffers(pkg, oracle, dev, dt):
    # the caller's work, values and indices hold all-ones bytes on entry (stale composites, a stale header in the row's
    # indices): every k class, split and unsplit, must still be exact
    g = torch.Generator().manual_seed(41)
    x = (torch.randn(6, 40000, generator=g) * 2).to(dt)
    for k in (1, 13, 64, 65, 300, 1024):
        for chunk in (None, 4096, 40000):
            check(pkg, oracle, x, k, dev, chunk=chunk, what="stale buffers", poison=True)


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_wide_lists_uncut_cut_and_second_look(pkg, oracle, dev, dt):
    # k > 64 over 8 chunks of 16384, the caller's buffers stale: random rows publish their candidates uncut (lists
    # zero-padded past them); values from a few dozen integers tie at the admission key, so that a chunk's candidates
    # overflow its list and are cut to m (the slots past m zeroed); rows whose largest values sit in one chunk take
    # the second look at x
    g = torch.Generator().manual_seed(43)
    x = (torch.randn(4, 8 * 16384, generator=g) * 2).to(dt)
    ties = torch.randint(0, 50, (4, 8 * 16384), generator=g).float().to(dt)
    hot = torch.randn(4, 8 * 16384, generator=g) * 2
    for r in range(4):
        hot[r, r * 16384:(r + 1) * 16384] += 4.0 if r % 2 == 0 else 0.6
    hot = hot.to(dt)
    for k in (300, 1024):
        for what, t in (("uncut lists", x), ("cut lists", ties), ("one hot chunk", hot)):
            check(pkg, oracle, t, k, dev, chunk=16384, what=f"wide, {what}", poison=True)


def test_random_shapes_and_chunkings(pkg, oracle, dev):
    # seeded random shapes, k (every class up to 1024) and chunkings (the plan's and explicit ones, split and unsplit),
    # fp32 and bf16, stale caller buffers: each against the oracle
    rng = np.random.default_rng(2024)
    g = torch.Generator().manual_seed(2024)
    for case in range(160):
        rows = int(rng.integers(1, 9))
        cols = int(rng.integers(70, 140000))
        k = int(min(cols, rng.choice([1, 2, 13, 50, 64, 65, 100, 150, 257, 300, 600, 1000, 1024])))
        dt = torch.float32 if case % 3 else torch.bfloat16
        pattern = case % 4
        if pattern == 0:
            x = torch.randn(rows, cols, generator=g) * 3
        elif pattern == 1:  # few distinct values: ties everywhere
            x = torch.randint(0, 40, (rows, cols), generator=g).float()
        elif pattern == 2:  # negative rows (log-probabilities)
            x = -torch.rand(rows, cols, generator=g) * 20
        else:  # one hot region per row
            x = torch.randn(rows, cols, generator=g)
            at = int(rng.integers(0, cols))
            x[:, at:at + 3000] += 3.0
        chunk = None if case % 2 else int(rng.choice([2048, 4096, 16384, 32768])) // 8 * 8
        if chunk is not None and chunk >= cols:
            chunk = None
        check(pkg, oracle, x.to(dt), k, dev, chunk=chunk, what=f"random case {case}", poison=bool(case % 2))


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_many_short_rows_taken_whole(pkg, oracle, dev, dt):
    # as many rows as CUs or more, two chunks of a row within two register tiles: one workgroup takes the row whole
    # (the plan's chunking at 512 x 32000 and 400 x 30000), next to k = 1 and k > 64 on the same shapes
    g = torch.Generator().manual_seed(45)
    for rows, cols in ((512, 32000), (400, 30000)):
        x = (torch.randn(rows, cols, generator=g) * 2).to(dt)
        for k in (1, 2, 50, 64, 65):
            check(pkg, oracle, x, k, dev, what=f"short rows {rows}x{cols}", poison=True)


def test_joined_short_chunks(pkg, oracle, dev):
    # the caller's short chunks joined to 16384 or 8192 columns: 40 chunks per row (at k = 50 and 64, 80 heads, more
    # than a wave holds, and at k = 64 2560 list entries, more than one batch: the merge's block floor and streamed
    # lists), 8 rows of 8 chunks, one row of 16
    g = torch.Generator().manual_seed(46)
    for rows, cols in ((2, 40 * 16384), (8, 128256), (1, 128256)):
        x = torch.randn(rows, cols, generator=g) * 2
        for k in (7, 13, 50, 64):
            check(pkg, oracle, x, k, dev, chunk=2048, what=f"joined chunks {rows}x{cols}", poison=True)


def test_invalid_arguments(pkg, dev):
    L = lib(pkg)
    s = torch.cuda.current_stream().cuda_stream
    p = torch.zeros(16, device=dev).data_ptr()
    assert L.launch(p, p, p, p, p, 0, 100, 5, 0, 256, 4, 100, s) == 0      # no rows
    assert L.launch(p, p, p, p, p, 2, 100, 0, 0, 256, 4, 100, s) == 0      # k = 0
    assert L.launch(p, p, p, p, p, 2, 100, 101, 0, 256, 4, 100, s) == -1   # k > cols
    assert L.launch(p, p, p, p, p, 2, 5000, 1025, 0, 256, 4, 5000, s) == -1
    assert L.launch(p, p, p, p, p, 70000, 100, 5, 0, 256, 4, 100, s) == -1
    assert L.launch(p, p, p, p, p, 2, 100, 5, 0, 256, 4, 0, s) == -1      # chunk
    assert L.launch(p, p, p, p, p, 2, 100, 5, 0, 256, 4, 50, s) == -1     # split with chunk % 4
    assert L.launch(p, p, p, p, p, 2, 100, 5, 0, 100, 4, 100, s) == -1    # threads
    assert L.launch(p, p, p, p, p, 2, 100, 5, 0, 256, 3, 100, s) == -1    # depth
    assert L.launch(p, p, p, p, p, 2, 100, 5, 2, 256, 4, 100, s) == -1    # dtype
    assert L.launch(p, p, p, None, p, 2, 100, 5, 0, 256, 4, 52, s) == -1   # a split row without work
    assert L.launch(p, p, p, p, None, 2, 100, 5, 0, 256, 4, 52, s) == -1   # a split row without counters


@pytest.mark.parametrize("k", [1, 50, 1024])
def test_config_topk_128x128256(pkg, oracle, dev, k):
    x = pkg.workloads.topk_128x128256()["x"]
    nchunks = check(pkg, oracle, x, k, dev, what="topk_128x128256")
    print(f"[topk] chunks per row: {nchunks}", flush=True)
    # the reference's own path: a stable descending sort
    from oracle import torch_paths
    v, i = pkg.topk(x.to(dev), k)
    sv, si = torch_paths.topk(x, k)
    assert torch.equal(i.cpu(), si) and torch.equal(v.cpu(), sv)


def sample_case(rows, k, seed, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    v, i = torch.sort(torch.randn(rows, 3 * k, generator=g) * 2, dim=-1, descending=True, stable=True)
    v, i = v[:, :k].contiguous().to(dtype), i[:, :k].contiguous()
    return v, i, torch.rand(rows, generator=g)


@pytest.mark.parametrize("k", [1, 2, 50, 64, 65, 300, 1024])
def test_sample_matches_oracle(pkg, oracle, dev, k):
    for dtype in (torch.float32, torch.bfloat16):
        v, i, u = sample_case(256, k, 7 * k, dtype)
        vn = v.numpy() if dtype == torch.float32 else bits16(v)
        name = "fp32" if dtype == torch.float32 else "bf16"
        for temp, top_p in [(1.0, 1.0), (0.7, 0.9), (2.0, 0.3), (0.0, 0.5), (0.5, 1.0)]:
            print(f"[topk sample] k={k} {dtype} T={temp} top_p={top_p}", flush=True)
            got = pkg.topk_sample(v.to(dev), i.to(dev), u.to(dev), temp, top_p).cpu().numpy()
            # every row: the draw is one of the oracle's admissible positions (the exact draw's, or where u or the
            # nucleus cut lies within rounding of a boundary, its neighbour: the kernel's fp32 sums sit about 1e-6 of
            # the total from the oracle's fp64 ones)
            lo, hi = oracle.topk_sample_band(vn, i.numpy(), u.numpy(), temp, top_p, name)
            ok = oracle.draw_admissible(got, i.numpy(), lo, hi)
            assert ok.all(), f"k={k} T={temp} p={top_p}: {(~ok).sum()} rows outside the admissible draws"


def test_sample_after_topk_config(pkg, oracle, dev):
    """The pipeline: top-k of the config's logits, then one draw per row, against the oracle's top-k and draw."""
    inp = pkg.workloads.topk_sample_128x128256()
    x, k = inp["x"], inp["k"]
    v, i = pkg.topk(x.to(dev), k)
    got = pkg.topk_sample(v, i, inp["uniforms"].to(dev), inp["temperature"], inp["top_p"]).cpu().numpy()
    rv, ri = oracle.topk(x.numpy(), k)
    lo, hi = oracle.topk_sample_band(rv, ri, inp["uniforms"].numpy(), inp["temperature"], inp["top_p"])
    assert oracle.draw_admissible(got, ri, lo, hi).all()


@pytest.mark.parametrize("k", [1, 2, 50, 64, 65, 300, 1024])
def test_launch_sample_equals_two_steps(pkg, oracle, dev, k):
    """topk_launch_sample (the draw fused into the top-k launch) against launch() then topk_sample_launch(): values,
    indices and the drawn indices bit for bit, for split and unsplit rows, both dtypes, and greedy, nucleus and full
    draws; and the fused draws against the oracle's admissible draws on its own top-k list, every row."""
    cand = pkg.candidate("topk")
    g = torch.Generator().manual_seed(1000 + k)
    for rows, cols in [(5, 30000), (3, 1500)]:
        if k > cols:
            continue
        for dt in (torch.float32, torch.bfloat16):
            x = (torch.randn(rows, cols, generator=g) * 2).to(dt).to(dev)
            u = torch.rand(rows, generator=g).to(dev)
            for temperature, top_p in [(0.8, 0.9), (0.0, 1.0), (1.3, 1.0)]:
                print(f"[topk] fused draw {rows}x{cols} {dt} k={k} T={temperature} p={top_p}", flush=True)
                v2, i2, d2 = cand.run_and_sample({"x": x, "k": k}, u, temperature, top_p)
                out = cand.run({"x": x, "k": k})
                d1 = cand.sample(out["values"], out["indices"], u, temperature, top_p)
                torch.cuda.synchronize()
                assert torch.equal(i2, out["indices"]) and torch.equal(v2.view(-1), out["values"].view(-1))
                assert torch.equal(d2, d1), (d2.tolist(), d1.tolist())
                name = "fp32" if dt == torch.float32 else "bf16"
                rv, ri = oracle.topk(x.cpu().numpy() if dt == torch.float32 else bits16(x), k, name)
                lo, hi = oracle.topk_sample_band(rv, ri, u.cpu().numpy(), temperature, top_p, name)
                assert oracle.draw_admissible(d2.cpu().numpy(), ri, lo, hi).all()


def test_launch_sample_rejects_missing_buffers(pkg, dev):
    L = lib(pkg)
    x = torch.randn(2, 1000, device=dev)
    vals = torch.empty(2, 5, device=dev)
    idx = torch.empty(2, 5, dtype=torch.int64, device=dev)
    u = torch.rand(2, device=dev)
    s = torch.cuda.current_stream().cuda_stream
    work = torch.empty(1, dtype=torch.int64, device=dev)
    cnt = torch.zeros(2, dtype=torch.int32, device=dev)
    assert L.topk_launch_sample(x.data_ptr(), vals.data_ptr(), idx.data_ptr(), work.data_ptr(), cnt.data_ptr(), 2,
                                1000, 5, 0, 256, 4, 1000, None, idx.data_ptr(), 1.0, 1.0, s) == -1
    assert L.topk_launch_sample(x.data_ptr(), vals.data_ptr(), idx.data_ptr(), work.data_ptr(), cnt.data_ptr(), 2,
                                1000, 5, 0, 256, 4, 1000, u.data_ptr(), None, 1.0, 1.0, s) == -1
