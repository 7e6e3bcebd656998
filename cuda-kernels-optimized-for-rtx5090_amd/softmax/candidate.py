"""Softmax over the last dimension, served by this package's MI355X library through the reference's C entry point.

Contract (the same shape as the reference's softmax/baseline.py:12-13, whose entry point is softmax/kernel.cu:520):
run({"x": x}) returns {"y": y}, y holding softmax(x) along x's last dimension. x may be fp32 (dtype code 0) or bf16
(code 1) and have any number of leading dimensions, which become rows. Sums and exponentials are taken in fp32 and
each output element is rounded once.

Library: libkernel.so from the directory named by CKOPT_BUILD_DIR, or this package's build/softmax/ when that variable
is unset. A missing library is an ImportError; there is no CPU path.

Tuning file: an optional params.json beside this file may hold "threads" and "aux". The C entry point checks nothing
about them and the MI355X kernels pick their own launch shape, so they only travel through.

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
_AUX = int(_TUNING.get("aux", 1024))
_CODE = {torch.float32: 0, torch.bfloat16: 1}

LIB_PATH = os.path.join(os.environ.get("CKOPT_BUILD_DIR") or os.path.join(_HERE, "..", "build", "softmax"),
                        "libkernel.so")
if not os.path.exists(LIB_PATH):
    raise ImportError(f"softmax: no library at {LIB_PATH}; run make_libs.py first")
_lib = ctypes.CDLL(LIB_PATH)
# int launch(const void* x, void* y, long long rows, long long cols, int dtype, int threads, int aux, hipStream_t)
_lib.launch.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_longlong, ctypes.c_longlong, ctypes.c_int,
                        ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
_lib.launch.restype = ctypes.c_int


def _reject(x):
    """A short reason when x cannot go to the kernels, else None."""
    if x.dtype not in _CODE:
        return f"dtype {x.dtype}"
    if x.dim() < 1:
        return f"shape {tuple(x.shape)}"
    if x.device.type != "cuda":
        return f"device {x.device}"
    return None


def run(inputs):
    x = inputs["x"]
    reason = _reject(x)
    if reason:
        raise ValueError(f"softmax candidate: {reason}")
    x = x.contiguous()
    y = torch.empty_like(x)
    cols = x.shape[-1]
    rows = x.numel() // cols if cols else 0
    err = _lib.launch(x.data_ptr(), y.data_ptr(), rows, cols, _CODE[x.dtype], _THREADS, _AUX,
                      torch.cuda.current_stream(x.device).cuda_stream)
    if err:
        raise RuntimeError(f"kernel launch failed: HIP error {err}")
    return {"y": y}
