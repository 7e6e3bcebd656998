"""RMSNorm over the last dimension, served by this package's MI355X library through the reference's C entry point.

Contract (the reference's rmsnorm/candidate.py:25-50 and its entry point rmsnorm/kernel.cu:132): run({"x": x}) with
x a 2-D bf16 (dtype code 1) or fp16 (code 2) GPU tensor returns {"y": y}, y = x * inv for each row, where inv is
1 / sqrt(mean(x^2) + eps) rounded to x's dtype before the product (rmsnorm/kernel.cu:1-8). eps defaults to 1e-6;
inputs["eps"] overrides it.

Additions of this build (no counterpart in the reference):
  - inputs["weight"], a [cols] tensor of x's dtype: y = weight * (x * inv), the product rounded to the dtype again
    (entry point rmsnorm_launch_weighted);
  - inputs["residual"], x's dtype and shape: the residual add fused in front of the norm. h = x + residual comes back
    as "residual" (it overwrites the given tensor when inputs["inplace"] is true) and y = rmsnorm(h), weighted when a
    weight is given (entry point rmsnorm_add_launch).

Library: libkernel.so from the directory named by CKOPT_BUILD_DIR, or this package's build/rmsnorm/ when that variable
is unset. A missing library is an ImportError; there is no CPU path.

Tuning file: an optional params.json beside this file may hold "threads" (default 256). The C entry point validates it
as the reference does (a multiple of 32 in [32, 1024]); the MI355X kernels choose their own launch shape.

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
_THREADS = int(_TUNING.get("threads", 256))
_DEFAULT_EPS = 1e-6
_CODE = {torch.bfloat16: 1, torch.float16: 2}

LIB_PATH = os.path.join(os.environ.get("CKOPT_BUILD_DIR") or os.path.join(_HERE, "..", "build", "rmsnorm"),
                        "libkernel.so")
if not os.path.exists(LIB_PATH):
    raise ImportError(f"rmsnorm: no library at {LIB_PATH}; run make_libs.py first")
_lib = ctypes.CDLL(LIB_PATH)
# int launch(const void* x, void* y, long long rows, int cols, int dtype, float eps, int threads, hipStream_t)
_lib.launch.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_longlong, ctypes.c_int, ctypes.c_int,
                        ctypes.c_float, ctypes.c_int, ctypes.c_void_p]
_lib.launch.restype = ctypes.c_int
# int rmsnorm_launch_weighted(x, weight, y, rows, cols, dtype, eps, threads, stream)
_lib.rmsnorm_launch_weighted.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_longlong,
                                         ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_int, ctypes.c_void_p]
_lib.rmsnorm_launch_weighted.restype = ctypes.c_int
# int rmsnorm_add_launch(x, residual, weight, y, residual_out, rows, cols, dtype, eps, threads, stream)
_lib.rmsnorm_add_launch.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_longlong, ctypes.c_int, ctypes.c_int,
                                                             ctypes.c_float, ctypes.c_int, ctypes.c_void_p]
_lib.rmsnorm_add_launch.restype = ctypes.c_int


def _reject(x, w, r):
    """A short reason when x (with its optional weight w and residual r) cannot go to the kernels, else None."""
    if x.dtype not in _CODE:
        return f"dtype {x.dtype}"
    if x.dim() != 2 or x.shape[1] < 1:
        return f"shape {tuple(x.shape)}"
    if x.device.type != "cuda":
        return f"device {x.device}"
    if w is not None and (w.dtype != x.dtype or tuple(w.shape) != (x.shape[1],) or w.device != x.device):
        return f"weight {w.dtype} {tuple(w.shape)} on {w.device}"
    if r is not None and (r.dtype != x.dtype or r.shape != x.shape or r.device != x.device):
        return f"residual {r.dtype} {tuple(r.shape)} on {r.device}"
    return None


def _checked(err):
    if err:
        raise RuntimeError(f"kernel launch failed: HIP error {err}")


def run(inputs):
    x, w, r = inputs["x"], inputs.get("weight"), inputs.get("residual")
    eps = float(inputs.get("eps", _DEFAULT_EPS))
    reason = _reject(x, w, r)
    if reason:
        raise ValueError(f"rmsnorm candidate: {reason}")
    x = x.contiguous()
    y = torch.empty_like(x)
    rows, cols = x.shape
    code = _CODE[x.dtype]
    stream = torch.cuda.current_stream(x.device).cuda_stream
    w = w.contiguous() if w is not None else None  # held until the launch is queued
    wp = w.data_ptr() if w is not None else None
    if r is not None:
        r_in = r.contiguous()
        # h goes over the caller's residual only when asked to and when that tensor is the one the kernel reads
        h = r_in if inputs.get("inplace") and r_in.data_ptr() == r.data_ptr() else torch.empty_like(x)
        _checked(_lib.rmsnorm_add_launch(x.data_ptr(), r_in.data_ptr(), wp, y.data_ptr(), h.data_ptr(), rows, cols,
                                         code, eps, _THREADS, stream))
        return {"y": y, "residual": h}
    if wp is None:
        _checked(_lib.launch(x.data_ptr(), y.data_ptr(), rows, cols, code, eps, _THREADS, stream))
    else:
        _checked(_lib.rmsnorm_launch_weighted(x.data_ptr(), wp, y.data_ptr(), rows, cols, code, eps, _THREADS, stream))
    return {"y": y}
