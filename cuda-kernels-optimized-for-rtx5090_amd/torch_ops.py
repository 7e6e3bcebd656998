"""The PyTorch-ROCm operators over the op libraries: torch.ops.ckopt.*.

build/torch/libckopt_torch.so (csrc/torch_ops.cpp, built by make_libs.py) registers, for GPU tensors and with shape
functions for meta/fake tensors (tracing):

    ckopt.softmax(x) -> y                                        softmax/kernel.cu:520 `launch`
    ckopt.rmsnorm(x, weight=None, eps=1e-6) -> y                 rmsnorm/kernel.cu:132 `launch`, rmsnorm_launch_weighted
    ckopt.rmsnorm_add(x, residual, weight=None, eps=1e-6) -> (y, h)   rmsnorm_add_launch
    ckopt.rmsnorm_add_(x, residual, weight=None, eps=1e-6) -> y  the same, h written over residual
    ckopt.rope(q, k, cos, sin, position_ids) -> (q_out, k_out)   rope/kernel.cu:201 `launch`
    ckopt.rope_(q, k, position_ids, inv_freq)                    rope_launch_freq, q and k rotated in place
    ckopt.rope_kv_(q, k, v, position_ids, inv_freq, k_cache, v_cache, slot_mapping)   rope_kv_launch
    ckopt.topk(x, k=50) -> (values, indices)                     topk/kernel.cu:520-570 `plan` + `launch`
    ckopt.topk_and_sample(x, k, uniforms, temperature=1.0, top_p=1.0) -> (values, indices, drawn)
    ckopt.topk_sample(values, indices, uniforms, temperature=1.0, top_p=1.0) -> drawn

Each call checks its tensors (a RuntimeError names what is wrong), allocates its outputs with torch on the input's
device and launches on torch's current stream; the top-k operators keep the caller-side workspace and counters of the
reference's launch protocol per device. There is no CPU path: a CPU tensor is an error.
"""

import os

import torch

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "build", "torch", "libckopt_torch.so")


def load():
    """Registers the operators (once per process) and returns the torch.ops.ckopt namespace."""
    if not hasattr(torch.ops.ckopt, "softmax"):
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"torch operators: no library at {LIB_PATH}; run make_libs.py first")
        torch.ops.load_library(LIB_PATH)
    return torch.ops.ckopt
