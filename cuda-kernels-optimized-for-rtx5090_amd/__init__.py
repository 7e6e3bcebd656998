"""MI355X-native row-wise LLM-inference kernels: softmax, RMSNorm, RoPE and top-k, hand-written in HIP for gfx950.

The product is one C-ABI library per op, build/<op>/libkernel.so (make_libs.py), exporting the reference's entry
points (`launch`, and `plan` for top-k; declared in include/<op>.h) plus a few extensions. Two bindings sit above
them: <op>/candidate.py mirrors the reference harness's `run(inputs)` wrapper for the op and loads that library with
ctypes (the functions below are conveniences over those wrappers), and torch_ops.py registers the PyTorch-ROCm
operators torch.ops.ckopt.* (build/torch/libckopt_torch.so) over the same entry points. Inputs must be GPU tensors;
there is no CPU fallback.
"""

import importlib.util
import os
import sys

from . import workloads  # noqa: F401  (named workloads: shapes, seeds, byte counts)

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
OPS = ("softmax", "rmsnorm", "rope", "topk")
TORCH = ("torch",)   # the torch operators over the op libraries


def lib_path(op):
    """The in-tree library of an op (what a harness's CKOPT_BUILD_DIR would point at)."""
    return os.path.join(PKG_DIR, "build", op, "libkernel.so")


def build(ops=OPS + TORCH):
    """Compiles the libraries of the given ops (and the torch operators); returns {op: path}."""
    from . import make_libs
    return make_libs.build(ops)


def candidate(op):
    """The op's reference-style wrapper module, <op>/candidate.py, loaded by file path as the reference harness loads
    its candidates (it loads the op's library on first use)."""
    name = f"{__name__}_{op}_candidate"
    mod = sys.modules.get(name)
    if mod is None:
        spec = importlib.util.spec_from_file_location(name, os.path.join(PKG_DIR, op, "candidate.py"))
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        sys.modules[name] = mod
    return mod


def ops():
    """torch.ops.ckopt, with the operators registered (torch_ops.py)."""
    from . import torch_ops
    return torch_ops.load()


def softmax(x):
    """softmax(x) over the last dim; fp32 or bf16."""
    return candidate("softmax").run({"x": x})["y"]


def rmsnorm(x, weight=None, eps=1e-6):
    """RMSNorm over the last dim of a 2-D bf16/fp16 x, optionally times weight."""
    inputs = {"x": x, "eps": eps}
    if weight is not None:
        inputs["weight"] = weight
    return candidate("rmsnorm").run(inputs)["y"]


def rmsnorm_add(x, residual, weight=None, eps=1e-6, inplace=False):
    """Fused residual add + RMSNorm: returns (y, h) with h = x + residual (written over residual when inplace) and
    y = rmsnorm(h), times weight when given."""
    inputs = {"x": x, "residual": residual, "eps": eps, "inplace": inplace}
    if weight is not None:
        inputs["weight"] = weight
    out = candidate("rmsnorm").run(inputs)
    return out["y"], out["residual"]


def rope(q, k, position_ids, cos=None, sin=None, inv_freq=None, inplace=False):
    """RoPE of q [B, S, Hq, D] and k [B, S, Hk, D]: from a cos/sin cache, or on the fly from inv_freq."""
    inputs = {"q": q, "k": k, "position_ids": position_ids, "inplace": inplace}
    if inv_freq is not None:
        inputs["inv_freq"] = inv_freq
    else:
        inputs["cos"], inputs["sin"] = cos, sin
    out = candidate("rope").run(inputs)
    return out["q_out"], out["k_out"]


def rope_kv(q, k, v, position_ids, inv_freq, k_cache, v_cache, slot_mapping, inplace=False):
    """RoPE fused with the KV-cache write: returns q_out; the rotated k and v land in the cache rows slot_mapping
    picks ([slots, Hk, D] caches, updated in place; a negative slot writes nothing)."""
    out = candidate("rope").run({"q": q, "k": k, "v": v, "position_ids": position_ids, "inv_freq": inv_freq,
                                 "k_cache": k_cache, "v_cache": v_cache, "slot_mapping": slot_mapping,
                                 "inplace": inplace})
    return out["q_out"]


def topk(x, k=50):
    """The k largest entries of each row of a 2-D fp32/bf16 x, sorted descending, ties by lowest index."""
    out = candidate("topk").run({"x": x, "k": k})
    return out["values"], out["indices"]


def topk_sample(values, indices, uniforms, temperature=1.0, top_p=1.0):
    """Draws one index per row from a top-k list with temperature, nucleus cut and the caller's uniforms."""
    return candidate("topk").sample(values, indices, uniforms, temperature, top_p)
