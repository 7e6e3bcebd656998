"""Rotary position embedding of q and k, served by this package's MI355X library through the reference's C entry
point.

Contract (the reference's rope/candidate.py:27-55 and its entry point rope/kernel.cu:201): run(inputs) with q
[B, S, Hq, D] and k [B, S, Hk, D] in bf16 (dtype code 1) or fp16 (code 2), position_ids int64 [B, S] and a cos/sin
table pair [P, D] in fp32 (cache code 0), bf16 (1) or fp16 (2) returns {"q_out", "k_out"}. Element i of a head pairs
with element i + D/2 (rotate-half); each head is rotated in fp32 by the table row its token's position selects, every
product and sum rounded on its own, and the result rounded once to q's dtype.

Additions of this build (no counterpart in the reference):
  - inputs["inv_freq"] (fp32 [D/2]) instead of cos/sin: the angles pos * inv_freq[i] are formed in fp32 and their
    cosine and sine evaluated inside the kernel (entry point rope_launch_freq); the result equals the table path fed
    a table built from the same fp32 angles;
  - inputs["inplace"] = True: q and k themselves are rotated and returned as q_out and k_out;
  - inputs "v", "k_cache", "v_cache" and "slot_mapping" (together with inv_freq): the rotation fused with the paged
    KV-cache write (entry point rope_kv_launch). q is rotated, and the rotated k and the untouched v land in the
    cache rows [slots, Hk, D] that slot_mapping (int64 [B, S], -1 = skip) names.

Inputs are made contiguous before the launch; an in-place call needs q and k contiguous to begin with.

Library: libkernel.so from the directory named by CKOPT_BUILD_DIR, or this package's build/rope/ when that variable is
unset. A missing library is an ImportError; there is no CPU path.

Tuning file: an optional params.json beside this file may hold "rows" and "splits". The C entry point validates them
as the reference does; the MI355X kernels choose their own launch shape.

Errors: ValueError before any launch for an input the kernels do not take, RuntimeError carrying the HIP error code
when the launch reports one.
"""

import ctypes
import json
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))


def _tuning():
    path = os.path.join(_HERE, "params.json")
    if not os.path.exists(path):
        return {}
    with open(path) as f:
        return json.load(f)


_TUNING = _tuning()
_ROWS = int(_TUNING.get("rows", 40))
_SPLITS = int(_TUNING.get("splits", 1))
_QK = {torch.bfloat16: 1, torch.float16: 2}
_CACHE = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}

LIB_PATH = os.path.join(os.environ.get("CKOPT_BUILD_DIR") or os.path.join(_HERE, "..", "build", "rope"),
                        "libkernel.so")
if not os.path.exists(LIB_PATH):
    raise ImportError(f"rope: no library at {LIB_PATH}; run make_libs.py first")
_lib = ctypes.CDLL(LIB_PATH)
_lib.launch.argtypes = [ctypes.c_void_p] * 7 + [ctypes.c_longlong] + [ctypes.c_int] * 7 + [ctypes.c_void_p]
_lib.launch.restype = ctypes.c_int
_lib.rope_launch_freq.argtypes = [ctypes.c_void_p] * 6 + [ctypes.c_longlong] + [ctypes.c_int] * 4 + [ctypes.c_void_p]
_lib.rope_launch_freq.restype = ctypes.c_int
_lib.rope_kv_launch.argtypes = [ctypes.c_void_p] * 9 + [ctypes.c_longlong] + [ctypes.c_int] * 4 + [ctypes.c_void_p]
_lib.rope_kv_launch.restype = ctypes.c_int


def _reject(q, k, cos, sin, ids, inv_freq, inplace):
    """A short reason when these tensors cannot go to the kernels, else None."""
    if q.dtype not in _QK or k.dtype != q.dtype:
        return f"dtypes q {q.dtype}, k {k.dtype}"
    if ids.dtype != torch.int64 or q.dim() != 4 or k.dim() != 4 or ids.dim() != 2:
        return f"position_ids {ids.dtype} {tuple(ids.shape)}, q {tuple(q.shape)}, k {tuple(k.shape)}"
    if tuple(q.shape[:2]) != tuple(ids.shape) or tuple(k.shape[:2]) != tuple(ids.shape) or q.shape[3] != k.shape[3] \
            or q.shape[3] % 2:
        return f"shapes q {tuple(q.shape)}, k {tuple(k.shape)}, position_ids {tuple(ids.shape)}"
    if inv_freq is None:
        if cos is None or sin is None or cos.dtype not in _CACHE or sin.dtype != cos.dtype or cos.dim() != 2 \
                or tuple(sin.shape) != tuple(cos.shape) or cos.shape[1] != q.shape[3]:
            return "cos/sin " + ("missing" if cos is None or sin is None else f"{cos.dtype} {tuple(cos.shape)}")
    elif inv_freq.dtype != torch.float32 or tuple(inv_freq.shape) != (q.shape[3] // 2,):
        return f"inv_freq {inv_freq.dtype} {tuple(inv_freq.shape)}"
    tensors = [q, k, ids] + ([cos, sin] if inv_freq is None else [inv_freq])
    if any(t.device != q.device for t in tensors) or q.device.type != "cuda":
        return "devices " + ", ".join(str(t.device) for t in tensors)
    if inplace and not (q.is_contiguous() and k.is_contiguous()):
        return "in-place rotation needs contiguous q and k"
    return None


def _run_kv(inputs):
    """The rotation fused with the cache write: returns q_out (q itself with inputs["inplace"]) and the two caches,
    whose rows named by slot_mapping now hold the rotated k and the given v."""
    q, k, v, ids = inputs["q"], inputs["k"], inputs["v"], inputs["position_ids"]
    kc, vc, slots, inv_freq = inputs["k_cache"], inputs["v_cache"], inputs["slot_mapping"], inputs.get("inv_freq")
    inplace = bool(inputs.get("inplace", False))
    reason = _reject(q, k, None, None, ids, inv_freq, inplace) if inv_freq is not None else "inv_freq missing"
    if reason is None:
        Hk, D = k.shape[2], k.shape[3]
        if v.dtype != q.dtype or tuple(v.shape) != tuple(k.shape):
            reason = f"v {v.dtype} {tuple(v.shape)}"
        elif any(c.dtype != q.dtype or c.dim() != 3 or tuple(c.shape[1:]) != (Hk, D) or not c.is_contiguous()
                 or c.device != q.device for c in (kc, vc)) or kc.shape != vc.shape:
            reason = f"caches {tuple(kc.shape)} {tuple(vc.shape)} (contiguous [slots, {Hk}, {D}] of q's dtype)"
        elif slots.dtype != torch.int64 or tuple(slots.shape) != tuple(ids.shape) or slots.device != q.device:
            reason = f"slot_mapping {slots.dtype} {tuple(slots.shape)}"
    if reason:
        raise ValueError(f"rope candidate: {reason}")
    q, k, v, ids, slots = q.contiguous(), k.contiguous(), v.contiguous(), ids.contiguous(), slots.contiguous()
    q_out = q if inplace else torch.empty_like(q)
    batch, seq, q_heads, head_dim = q.shape
    inv_freq = inv_freq.contiguous()
    err = _lib.rope_kv_launch(q.data_ptr(), k.data_ptr(), v.data_ptr(), ids.data_ptr(), inv_freq.data_ptr(),
                              q_out.data_ptr(), kc.data_ptr(), vc.data_ptr(), slots.data_ptr(), batch * seq, q_heads,
                              k.shape[2], head_dim, _QK[q.dtype], torch.cuda.current_stream(q.device).cuda_stream)
    if err:
        raise RuntimeError(f"kernel launch failed: HIP error {err}")
    return {"q_out": q_out, "k_cache": kc, "v_cache": vc}


def run(inputs):
    if "k_cache" in inputs:
        return _run_kv(inputs)
    q, k, ids = inputs["q"], inputs["k"], inputs["position_ids"]
    cos, sin, inv_freq = inputs.get("cos"), inputs.get("sin"), inputs.get("inv_freq")
    inplace = bool(inputs.get("inplace", False))
    reason = _reject(q, k, cos, sin, ids, inv_freq, inplace)
    if reason:
        raise ValueError(f"rope candidate: {reason}")
    q, k, ids = q.contiguous(), k.contiguous(), ids.contiguous()
    q_out, k_out = (q, k) if inplace else (torch.empty_like(q), torch.empty_like(k))
    batch, seq, q_heads, head_dim = q.shape
    stream = torch.cuda.current_stream(q.device).cuda_stream
    if inv_freq is None:
        cos, sin = cos.contiguous(), sin.contiguous()
        err = _lib.launch(q.data_ptr(), k.data_ptr(), cos.data_ptr(), sin.data_ptr(), ids.data_ptr(),
                          q_out.data_ptr(), k_out.data_ptr(), batch * seq, q_heads, k.shape[2], head_dim, _QK[q.dtype],
                          _CACHE[cos.dtype], _ROWS, _SPLITS, stream)
    else:
        inv_freq = inv_freq.contiguous()
        err = _lib.rope_launch_freq(q.data_ptr(), k.data_ptr(), ids.data_ptr(), inv_freq.data_ptr(), q_out.data_ptr(),
                                    k_out.data_ptr(), batch * seq, q_heads, k.shape[2], head_dim, _QK[q.dtype], stream)
    if err:
        raise RuntimeError(f"kernel launch failed: HIP error {err}")
    return {"q_out": q_out, "k_out": k_out}
