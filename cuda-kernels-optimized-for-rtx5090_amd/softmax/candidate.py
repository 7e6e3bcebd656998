"""Softmax candidate wrapper: loads its kernel build, allocates y and launches the kernel.

y = softmax(x) over the last dim of x in fp32 (dtype 0) or bf16 (1), every value accumulated in fp32 and rounded once,
with the run(inputs) -> {"y": y} contract of the reference's softmax/baseline.py:12-13 (the reference ships no softmax
candidate; its ABI is softmax/kernel.cu:520). The one `launch` entry of libkernel.so serves both dtypes; x is passed
contiguous and its leading dims are flattened into rows. params.json (optional) may set "threads" and "aux", the
reference ABI's block-size hints, which this build accepts and does not need. The library is
$CKOPT_BUILD_DIR/libkernel.so when CKOPT_BUILD_DIR is set, else this package's build/softmax/libkernel.so.
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
_AUX = int(_params.get("aux", 1024))
_DTYPES = {torch.float32: 0, torch.bfloat16: 1}

LIB_PATH = os.path.join(os.environ.get("CKOPT_BUILD_DIR") or os.path.join(_HERE, "..", "build", "softmax"),
                        "libkernel.so")
if not os.path.exists(LIB_PATH):
    raise ImportError(f"softmax: {LIB_PATH} is missing (build it with make_libs.py)")
_lib = ctypes.CDLL(LIB_PATH)
_lib.launch.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_longlong, ctypes.c_longlong, ctypes.c_int,
                        ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
_lib.launch.restype = ctypes.c_int


def _problem(x):
    """Why x is not an input this kernel serves, or None."""
    if x.dtype not in _DTYPES:
        return f"dtype {x.dtype}"
    if x.dim() < 1:
        return f"shape {tuple(x.shape)}"
    if x.device.type != "cuda":
        return f"device {x.device}"
    return None


def run(inputs):
    x = inputs["x"]
    problem = _problem(x)
    if problem:
        raise ValueError(f"softmax candidate: {problem}")
    x = x.contiguous()
    y = torch.empty_like(x)
    cols = x.shape[-1]
    rows = x.numel() // cols if cols else 0
    err = _lib.launch(x.data_ptr(), y.data_ptr(), rows, cols, _DTYPES[x.dtype], _THREADS, _AUX,
                      torch.cuda.current_stream(x.device).cuda_stream)
    if err:
        raise RuntimeError(f"kernel launch failed: HIP error {err}")
    return {"y": y}
