"""The harness counterpart (cuda-kernels-optimized-for-rtx5090_amd/harness.py): every op's quick workloads pass its
correctness bars through the candidate wrappers, and the report has the reference README's columns."""

import importlib.util
import os

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def load_harness():
    spec = importlib.util.spec_from_file_location(
        "ck5090_harness", os.path.join(ROOT, "cuda-kernels-optimized-for-rtx5090_amd", "harness.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_quick_report_passes():
    h = load_harness()
    print("[harness] quick workloads of every op", flush=True)
    rows = h.run(quick=True, reps=3)
    assert {r["op"] for r in rows} == {"softmax", "rmsnorm", "rope", "topk"}
    assert all(r["correctness"] == "PASS" for r in rows), [r for r in rows if r["correctness"] != "PASS"]
    text = h.table(rows)
    header = ("| workload | correctness | timing | candidate ms | baseline ms | seed ms | vs baseline | vs seed "
              "| dtype |")
    assert header in text
