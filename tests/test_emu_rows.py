"""The softmax, RMSNorm and RoPE kernels' own source (csrc/softmax.hip, rmsnorm.hip, rope.hip) run on the CPU under
the emulation of the HIP surface they use (tests/emu/hip/hip_runtime.h), each launch checked against the oracle:
RMSNorm and RoPE bit for bit, softmax within its tolerance (fp32 rtol 1e-5, one ulp for subnormal results; bf16
1 ulp), since its exp is the host's here.

Every device buffer lies between guard pages, so a read or write past either end of an input, output or cache ends
the run with a fault. The cases force each tier and register shape through the libraries' tuning slots, and cover
ragged rows and tails, misaligned buffers (the scalar paths), in-place forms, -inf and all -inf rows, RoPE's head
sizes down to 24 and its fused KV-cache write with skipped (-1) slots. The softmax co-resident tier, whose
workgroups wait for one another, runs with every workgroup on an OS thread of its own, over repeated launches (the
pair table is reused under fresh tags), with one row per workgroup and with row groups walking several rows; also
under the weak mode (its pairs become visible late and out of order) with the wait's clock stopped, so that every wait
must end by its pairs, never by its time budget; and recorded once as a graph (the emulation's capture) and replayed
on new values, with eager launches in between. Some cases also run with each wave running ahead to the next block
barrier before the next wave starts.
"""

import os

import pytest

from _emu import build, run


@pytest.fixture(scope="module")
def emu_dir(tmp_path_factory):
    return tmp_path_factory.mktemp("emu_rows")


@pytest.fixture(scope="module")
def emu_softmax(emu_dir):
    return build(emu_dir, "softmax.hip", "emu_softmax.cpp")


@pytest.fixture(scope="module")
def emu_rmsnorm(emu_dir):
    return build(emu_dir, "rmsnorm.hip", "emu_rmsnorm.cpp")


@pytest.fixture(scope="module")
def emu_rope(emu_dir):
    return build(emu_dir, "rope.hip", "emu_rope.cpp")


# rows, cols, dtype (0 fp32, 1 bf16), tier (1 row, 2 stream, 3 generic), seed, waves, nv, offset, pattern
SOFTMAX = [
    ("row_fp32", 37, 4096, 0, 1, 1, 0, 0, 0, "randn"),
    ("row_bf16", 37, 4096, 1, 1, 2, 0, 0, 0, "randn"),
    ("row_ragged_fp32", 19, 1000, 0, 1, 3, 0, 0, 0, "randn"),
    ("row_ragged_bf16", 19, 1000, 1, 1, 4, 0, 0, 0, "randn"),
    ("row_one_wave", 40, 256, 0, 1, 13, 1, 1, 0, "randn"),
    ("row_long_bf16", 3, 65536, 1, 1, 15, 0, 0, 0, "randn"),
    ("row_special_bf16", 8, 4096, 1, 1, 10, 0, 0, 0, "special"),
    ("stream_fp32", 5, 20000, 0, 2, 5, 4, 0, 0, "randn"),
    ("stream_bf16", 5, 20000, 1, 2, 6, 16, 0, 0, "randn"),
    ("stream_special", 8, 5000, 0, 2, 11, 8, 0, 0, "special"),
    ("generic_fp32", 7, 3000, 0, 3, 7, 0, 0, 0, "randn"),
    ("generic_odd_bf16", 7, 3001, 1, 3, 8, 0, 0, 0, "randn"),
    ("misaligned_fp32", 8, 4096, 0, 1, 9, 0, 0, 1, "randn"),
    ("generic_special", 8, 999, 1, 3, 12, 0, 0, 0, "special"),
]

# the co-resident tier (its workgroups wait for one another: run concurrently), with repeated launches on the same
# buffers: rows, cols, dtype, seed, pattern, reps, row groups (0: one row per workgroup)
COOP = [
    ("coop_fp32", 2, 70000, 0, 3, "randn", 3, 0),
    ("coop_bf16", 3, 100000, 1, 4, "randn", 2, 0),
    ("coop_special", 4, 40000, 0, 5, "special", 2, 0),
    ("coop_one_chunk_bf16", 2, 16384, 1, 6, "randn", 2, 0),
    ("coop_groups_fp32", 7, 70000, 0, 7, "randn", 3, 2),
    ("coop_groups_special_bf16", 5, 40000, 1, 8, "special", 2, 3),
]

# rows, cols, dtype (1 bf16, 2 fp16), mode (0 launch, 1 weighted, 2 add, 3 add in place), seed, waves, nv,
# blocks per CU, offset
RMSNORM = [
    ("weighted_bf16", 37, 4096, 1, 1, 1, 0, 0, 0, 0),
    ("plain_bf16", 37, 4096, 1, 0, 2, 0, 0, 0, 0),
    ("add_fp16", 37, 4096, 2, 2, 3, 0, 0, 0, 0),
    ("add_in_place_bf16", 37, 4096, 1, 3, 4, 0, 0, 0, 0),
    ("ragged", 19, 1000, 1, 1, 5, 0, 0, 0, 0),
    ("tiny_row", 19, 13, 1, 1, 6, 0, 0, 0, 0),
    ("misaligned", 5, 4096, 1, 1, 7, 0, 0, 0, 1),
    ("one_wave_8v", 40, 4096, 1, 1, 8, 1, 8, 2, 0),
    ("four_waves_2v_fp16", 40, 4096, 2, 1, 9, 4, 2, 1, 0),
    ("sixteen_waves_add", 40, 2048, 1, 2, 10, 16, 1, 1, 0),
    ("long_row", 3, 65536, 1, 1, 11, 0, 0, 0, 0),
    ("short_rows_in_place_fp16", 300, 128, 2, 3, 12, 0, 0, 0, 0),
]

# tokens, q_heads, kv_heads, head_dim, dtype (1 bf16, 2 fp16), form (0/1/2 fp32/bf16/fp16 cache, 3 frequencies,
# 4 fused KV-cache write), in place, seed
ROPE = [
    ("freq_bf16_in_place", 37, 32, 8, 128, 1, 3, 1, 1),
    ("freq_fp16", 37, 32, 8, 128, 2, 3, 0, 2),
    ("cache_fp32", 21, 8, 2, 128, 1, 0, 0, 3),
    ("cache_bf16_in_place", 21, 8, 2, 128, 1, 1, 1, 4),
    ("cache_fp16", 21, 8, 2, 128, 2, 2, 0, 5),
    ("kv_bf16", 33, 4, 4, 64, 1, 4, 0, 6),
    ("kv_fp16", 33, 4, 4, 64, 2, 4, 1, 7),
    ("freq_d24", 9, 3, 1, 24, 1, 3, 0, 8),
    ("cache_d24_in_place", 9, 3, 1, 24, 1, 0, 1, 9),
    ("kv_d256", 5, 2, 2, 256, 1, 4, 0, 10),
    ("cache_d256_few_heads", 7, 2, 1, 256, 1, 0, 0, 11),     # 128 cache vectors per token over 48 items
    ("cache_d1024_bf16_cache", 5, 2, 1, 1024, 2, 1, 1, 12),  # the largest vector-path head, a 16-bit cache
    ("cache_d1040_scalar", 3, 1, 1, 1040, 1, 0, 0, 13),      # beyond it: the scalar kernel
]


@pytest.mark.parametrize("case", SOFTMAX, ids=[c[0] for c in SOFTMAX])
def test_emulated_softmax_matches_oracle(emu_softmax, case):
    run(emu_softmax, case[1:])


@pytest.mark.parametrize("case", COOP, ids=[c[0] for c in COOP])
def test_emulated_softmax_coresident_tier(emu_softmax, case):
    rows, cols, dtype, seed, pattern, reps, groups = case[1:]
    run(emu_softmax, [rows, cols, dtype, 4, seed, 0, groups, 0, pattern, reps], concurrent=True)


@pytest.mark.parametrize("case", COOP, ids=[c[0] for c in COOP])
def test_emulated_softmax_coresident_weak_stopped_clock(emu_softmax, case):
    # pairs visible late and out of order, and a wait that cannot end by its time budget: every wait ends by its pairs
    rows, cols, dtype, seed, pattern, reps, groups = case[1:]
    env = dict(os.environ, EMU_CLOCK_STOPPED="1")
    run(emu_softmax, [rows, cols, dtype, 4, seed, 0, groups, 0, pattern, reps], env=env, concurrent=True, weak=True,
        timeout=300)


@pytest.mark.parametrize("case", COOP, ids=[c[0] for c in COOP])
def test_emulated_softmax_coresident_graph_replay(emu_softmax, case):
    # after an eager launch, the launch recorded once and replayed four times, each replay on new values of x, with
    # eager launches of other values on the same table slots between some replays; workgroups starting up to 400 ms
    # apart, pairs visible late and out of order and the clock stopped,
    # so a wait can only end by pairs carrying its own tags: a replay that accepted a pair left by the replay before it
    # (the same captured arguments) or by the eager launch would normalise with the wrong statistics
    rows, cols, dtype, seed, pattern, _, groups = case[1:]
    env = dict(os.environ, EMU_CLOCK_STOPPED="1", EMU_GRAPH="1", EMU_STAGGER="1")
    run(emu_softmax, [rows, cols, dtype, 4, seed, 0, groups, 0, pattern, 4], env=env, concurrent=True, weak=True,
        timeout=300)


@pytest.mark.parametrize("concurrent", [False, True], ids=["one_after_another", "concurrent"])
@pytest.mark.parametrize("case", COOP, ids=[c[0] for c in COOP])
def test_emulated_softmax_coresident_fallback(emu_softmax, case, concurrent):
    # the wait bounded to one tick: workgroups that find their row incomplete (all but the row's last when they run one
    # after another) take the row's statistics from x
    rows, cols, dtype, seed, pattern, reps, groups = case[1:]
    run(emu_softmax, [rows, cols, dtype, 4, seed, 0, groups, 0, pattern, reps, 1], concurrent=concurrent)


@pytest.mark.parametrize("case", RMSNORM, ids=[c[0] for c in RMSNORM])
def test_emulated_rmsnorm_matches_oracle(emu_rmsnorm, case):
    run(emu_rmsnorm, case[1:])


@pytest.mark.parametrize("case", ROPE, ids=[c[0] for c in ROPE])
def test_emulated_rope_matches_oracle(emu_rope, case):
    run(emu_rope, case[1:])


# Waves running ahead of one another between block barriers (EMU_WAVE_AHEAD: each wave runs on until it waits at a
# block barrier before the next wave starts): the cross-wave reductions' LDS slots must not be rewritten before every
# wave has read them.
@pytest.mark.parametrize("op, case", [("softmax", c) for c in SOFTMAX[:6] + SOFTMAX[7:9]] +
                         [("rmsnorm", c) for c in RMSNORM[7:10]] + [("rope", c) for c in ROPE[:1] + ROPE[5:6]],
                         ids=lambda v: v if isinstance(v, str) else v[0])
def test_emulated_rows_waves_ahead(emu_softmax, emu_rmsnorm, emu_rope, op, case):
    exe = {"softmax": emu_softmax, "rmsnorm": emu_rmsnorm, "rope": emu_rope}[op]
    run(exe, case[1:], env=dict(os.environ, EMU_WAVE_AHEAD="1"))

