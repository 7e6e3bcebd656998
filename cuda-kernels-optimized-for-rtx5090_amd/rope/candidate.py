"""RoPE candidate wrapper: loads its kernel build, allocates q_out and k_out (or rotates in place) and launches.

q_out, k_out = q, k rotated by the cos/sin cache rows that position_ids pick (half-split pairing, full rotary, fp32
math, one rounding to the output dtype), as the reference's rope/candidate.py:3-5: q [B, S, Hq, D], k [B, S, Hk, D] in
bf16 (1) or fp16 (2), position_ids int64 [B, S], cos/sin [P, D] in fp32 (0), bf16 (1) or fp16 (2), through the
reference ABI's `launch`. Two extensions:
  - inputs["inv_freq"] (fp32 [D/2]) in place of cos/sin: cos/sin are computed on the fly from the positions
    (`rope_launch_freq`), equal to a cache built from inv_freq with fp32 angles;
  - inputs["inplace"] = True: q and k are rotated in place and returned as q_out and k_out;
  - inputs "v", "k_cache", "v_cache", "slot_mapping" (with inv_freq): RoPE fused with the KV-cache write
    (`rope_kv_launch`): q rotated, the rotated k and v written to the cache rows [slots, Hk, D] the slots pick.
Tensors are passed contiguous (an in-place call needs q and k contiguous already). params.json (optional) may set
"rows" and "splits", the reference ABI's block-shape hints, validated as the reference does. The library is
$CKOPT_BUILD_DIR/libkernel.so when CKOPT_BUILD_DIR is set, else this package's build/rope/libkernel.so.
"""

import ctypes
import json
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
_PARAMS_PATH = os.path.join(_HERE, "params.json")
_params = {}
if os.path.exists(_PARAMS_PATH):
    with open(_PARAMS_PATH) as _handle:
        _params = json.load(_handle)
_ROWS = int(_params.get("rows", 40))
_SPLITS = int(_params.get("splits", 1))
_QK = {torch.bfloat16: 1, torch.float16: 2}
_CACHE = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}

LIB_PATH = os.path.join(os.environ.get("CKOPT_BUILD_DIR") or os.path.join(_HERE, "..", "build", "rope"),
                        "libkernel.so")
if not os.path.exists(LIB_PATH):
    raise ImportError(f"rope: {LIB_PATH} is missing (build it with make_libs.py)")
_lib = ctypes.CDLL(LIB_PATH)
_lib.launch.argtypes = [ctypes.c_void_p] * 7 + [ctypes.c_longlong] + [ctypes.c_int] * 7 + [ctypes.c_void_p]
_lib.launch.restype = ctypes.c_int
_lib.rope_launch_freq.argtypes = [ctypes.c_void_p] * 6 + [ctypes.c_longlong] + [ctypes.c_int] * 4 + [ctypes.c_void_p]
_lib.rope_launch_freq.restype = ctypes.c_int
_lib.rope_kv_launch.argtypes = [ctypes.c_void_p] * 9 + [ctypes.c_longlong] + [ctypes.c_int] * 4 + [ctypes.c_void_p]
_lib.rope_kv_launch.restype = ctypes.c_int


def _problem(q, k, cos, sin, ids, inv_freq, inplace):
    """Why these inputs are not a rope call this kernel serves, or None."""
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
    """RoPE fused with the KV-cache write: q rotated (in place with inputs["inplace"]), rotated k and v written to the
    k_cache / v_cache rows [slots, Hk, D] that slot_mapping (int64 [B, S], -1 = no write) picks."""
    q, k, v, ids = inputs["q"], inputs["k"], inputs["v"], inputs["position_ids"]
    kc, vc, slots, inv_freq = inputs["k_cache"], inputs["v_cache"], inputs["slot_mapping"], inputs.get("inv_freq")
    inplace = bool(inputs.get("inplace", False))
    problem = _problem(q, k, None, None, ids, inv_freq, inplace) if inv_freq is not None else "inv_freq missing"
    if problem is None:
        Hk, D = k.shape[2], k.shape[3]
        if v.dtype != q.dtype or tuple(v.shape) != tuple(k.shape):
            problem = f"v {v.dtype} {tuple(v.shape)}"
        elif any(c.dtype != q.dtype or c.dim() != 3 or tuple(c.shape[1:]) != (Hk, D) or not c.is_contiguous()
                 or c.device != q.device for c in (kc, vc)) or kc.shape != vc.shape:
            problem = f"caches {tuple(kc.shape)} {tuple(vc.shape)} (contiguous [slots, {Hk}, {D}] of q's dtype)"
        elif slots.dtype != torch.int64 or tuple(slots.shape) != tuple(ids.shape) or slots.device != q.device:
            problem = f"slot_mapping {slots.dtype} {tuple(slots.shape)}"
    if problem:
        raise ValueError(f"rope candidate: {problem}")
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
    problem = _problem(q, k, cos, sin, ids, inv_freq, inplace)
    if problem:
        raise ValueError(f"rope candidate: {problem}")
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
