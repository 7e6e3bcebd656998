"""The top-k kernels' own source (csrc/topk.hip) run on the CPU under an emulation of the HIP surface it uses
(tests/emu/hip/hip_runtime.h), every launch checked bit for bit against the oracle.

Each workgroup thread is a cooperative fiber and each cross-lane operation an exchange between barriers of the wave's
live lanes. Every buffer the kernels touch (input, outputs, work, counters and the library's own hand-off
workspaces) lies between guard pages, so an out-of-bounds access ends the run with a fault. The cases cover
single- and split-chunk rows, every k class (1, the lane-maxima bound up to 64, the wide path up to 1024), short last
tiles, ties, monotone and all-negative rows, the all-ones NaN, repeated launches on the same buffers (the arrival
counters' self-reset), and shuffled workgroup and lane schedules. The concurrent cases run every workgroup of a launch
on an OS thread of its own, so chunks publish and count their arrivals while the row's other chunks and merger run.
What the emulation does not model is the hardware's memory ordering between workgroups (the host's is stronger) and
the compiler's gfx950 code.
"""

import os

import pytest

from _emu import build, run


@pytest.fixture(scope="module")
def emu_topk(tmp_path_factory):
    return build(tmp_path_factory.mktemp("emu_topk"), "topk.hip", "emu_topk.cpp")


ALL_K = "1,7,50,64,65,300,1024"
# rows, cols, dtype (0 fp32, 1 bf16), ks, chunk (0: plan's), min_chunk, reps, seed, shuffle seed, pattern
CASES = [
    ("split_fp32", 2, 20000, 0, ALL_K, 4096, 2048, 2, 1, -1, "randn"),
    ("split_bf16", 2, 20000, 1, ALL_K, 4096, 2048, 2, 2, -1, "randn"),
    ("one_chunk", 3, 20000, 0, ALL_K, 20000, 2048, 1, 3, -1, "randn"),
    ("planned", 4, 30000, 1, "1,50,1024", 0, 2048, 2, 4, -1, "randn"),
    ("short_tail_bf16", 2, 62 * 2048 + 1280, 1, "1,13,50,64,100,1024", 2048, 2048, 1, 5, -1, "randn"),
    ("short_tail_fp32", 2, 3 * 2048 + 40, 0, "1,13,50,64,100,1024", 2048, 2048, 1, 6, -1, "randn"),
    ("tile_plus_tail", 2, 2 * 16384 + 1280, 1, "1,50,100,1024", 16384, 2048, 1, 7, -1, "randn"),
    ("ties", 3, 30000, 0, "1,50,1024", 4096, 2048, 1, 8, -1, "ints"),
    ("ascending", 2, 40000, 0, "1,50,1024", 8192, 2048, 1, 9, -1, "ascending"),
    ("descending", 2, 40000, 1, "1,50,1024", 8192, 2048, 1, 10, -1, "descending"),
    ("negative", 2, 40000, 0, "1,50,300", 8192, 2048, 1, 11, -1, "negative"),
    ("all_ones_nan", 3, 20000, 0, "1,13,50,300", 4096, 2048, 1, 12, -1, "allones"),
    ("all_ones_nan_bf16", 3, 20000, 1, "1,13,50,300", 4096, 2048, 1, 13, -1, "allones"),
    ("k_equals_cols", 2, 1024, 0, "1024", 0, 2048, 1, 14, -1, "randn"),
    ("shuffled", 2, 20000, 0, ALL_K, 4096, 2048, 2, 15, 99, "randn"),
    ("shuffled_bf16", 2, 20000, 1, "1,50,1024", 2052, 2048, 2, 16, 7, "ints"),
    ("many_chunks_wide", 2, 100000, 0, "65", 1024, 2048, 1, 17, -1, "randn"),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_emulated_topk_matches_oracle(emu_topk, case):
    run(emu_topk, case[1:])


# rows, cols, dtype, ks, chunk, min_chunk, reps, seed, shuffle seed, pattern: split rows whose chunks hand their lists
# to the row's last arrival while the other workgroups run
CONCURRENT = [
    ("c5_rows_fp32", 8, 128256, 0, "1,50,1024", 0, 16384, 3, 31, 5, "randn"),
    ("split_bf16_ties", 4, 40000, 1, "1,13,64,65,300", 4096, 2048, 3, 32, 6, "ints"),
    # 59 workgroups (their fiber stacks stay within the host's limit on memory mappings)
    ("many_chunks", 1, 60000, 0, "7,65", 1024, 2048, 2, 33, -1, "randn"),
]


@pytest.mark.parametrize("case", CONCURRENT, ids=[c[0] for c in CONCURRENT])
def test_emulated_topk_concurrent_workgroups(emu_topk, case):
    run(emu_topk, case[1:], concurrent=True)


def test_emulated_topk_guard_below_start(emu_topk):
    # the same buffers placed flush against their lower guard page
    env = dict(os.environ, EMU_ALIGN_START="1")
    for case in (CASES[0], CASES[4], CASES[6]):
        run(emu_topk, case[1:], env=env)
