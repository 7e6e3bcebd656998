"""RMSNorm candidate wrapper: loads its kernel build, allocates y and launches the kernel.

y = x times rsqrt(the mean of x^2 over the last dim + eps) for x[rows, cols] in bf16 (1) or fp16 (2), with that rsqrt
rounded to x's dtype before the product (the reference's rmsnorm/candidate.py:3-4 and kernel.cu:1-8); eps is 1e-6
unless inputs["eps"] is given. With inputs["weight"] (a [cols] tensor of x's dtype) the result is weight * y, rounded
once more to the dtype, through the library's `rmsnorm_launch_weighted`; without it, through the reference ABI's
`launch`. x is passed contiguous. params.json (optional) may set "threads" (a multiple of 32 from 32 to 1024, default
256), validated as the reference does. The library is $CKOPT_BUILD_DIR/libkernel.so when CKOPT_BUILD_DIR is set, else
this package's build/rmsnorm/libkernel.so. With inputs["residual"] (x's dtype and shape) the call is the fused residual
add (no counterpart in the reference): h = x + residual is returned as "residual" (written over the given tensor when
inputs["inplace"] is true) and y = rmsnorm(h), times weight when given, through `rmsnorm_add_launch`.
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
_THREADS = int(_params.get("threads", 256))
_EPS = 1e-6
_DTYPES = {torch.bfloat16: 1, torch.float16: 2}

LIB_PATH = os.path.join(os.environ.get("CKOPT_BUILD_DIR") or os.path.join(_HERE, "..", "build", "rmsnorm"),
                        "libkernel.so")
if not os.path.exists(LIB_PATH):
    raise ImportError(f"rmsnorm: {LIB_PATH} is missing (build it with make_libs.py)")
_lib = ctypes.CDLL(LIB_PATH)
_lib.launch.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_longlong, ctypes.c_int, ctypes.c_int,
                        ctypes.c_float, ctypes.c_int, ctypes.c_void_p]
_lib.launch.restype = ctypes.c_int
_lib.rmsnorm_launch_weighted.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_longlong,
                                         ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_int, ctypes.c_void_p]
_lib.rmsnorm_launch_weighted.restype = ctypes.c_int
_lib.rmsnorm_add_launch.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_longlong, ctypes.c_int, ctypes.c_int,
                                                             ctypes.c_float, ctypes.c_int, ctypes.c_void_p]
_lib.rmsnorm_add_launch.restype = ctypes.c_int


def _problem(x, w):
    """Why x (and w) are not inputs this kernel serves, or None."""
    if x.dtype not in _DTYPES:
        return f"dtype {x.dtype}"
    if x.dim() != 2 or x.shape[1] < 1:
        return f"shape {tuple(x.shape)}"
    if x.device.type != "cuda":
        return f"device {x.device}"
    if w is not None and (w.dtype != x.dtype or tuple(w.shape) != (x.shape[1],) or w.device != x.device):
        return f"weight {w.dtype} {tuple(w.shape)} on {w.device}"
    return None


def run(inputs):
    x = inputs["x"]
    w = inputs.get("weight")
    r = inputs.get("residual")
    eps = float(inputs.get("eps", _EPS))
    problem = _problem(x, w)
    if problem is None and r is not None and (r.dtype != x.dtype or r.shape != x.shape or r.device != x.device):
        problem = f"residual {r.dtype} {tuple(r.shape)} on {r.device}"
    if problem:
        raise ValueError(f"rmsnorm candidate: {problem}")
    x = x.contiguous()
    y = torch.empty_like(x)
    rows, cols = x.shape
    stream = torch.cuda.current_stream(x.device).cuda_stream
    if r is not None:
        # fused residual add: h = x + residual goes to "residual" (in place when inputs["inplace"] and the given
        # residual is contiguous), y = rmsnorm(h) [* weight]
        r_in = r.contiguous()
        h = r_in if inputs.get("inplace") and r_in.data_ptr() == r.data_ptr() else torch.empty_like(x)
        wp = w.contiguous().data_ptr() if w is not None else None
        err = _lib.rmsnorm_add_launch(x.data_ptr(), r_in.data_ptr(), wp, y.data_ptr(), h.data_ptr(), rows, cols,
                                      _DTYPES[x.dtype], eps, _THREADS, stream)
        if err:
            raise RuntimeError(f"kernel launch failed: HIP error {err}")
        return {"y": y, "residual": h}
    if w is None:
        err = _lib.launch(x.data_ptr(), y.data_ptr(), rows, cols, _DTYPES[x.dtype], eps, _THREADS, stream)
    else:
        w = w.contiguous()
        err = _lib.rmsnorm_launch_weighted(x.data_ptr(), w.data_ptr(), y.data_ptr(), rows, cols, _DTYPES[x.dtype], eps,
                                           _THREADS, stream)
    if err:
        raise RuntimeError(f"kernel launch failed: HIP error {err}")
    return {"y": y}
