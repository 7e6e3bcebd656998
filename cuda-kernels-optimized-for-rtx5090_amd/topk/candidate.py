"""Top-k candidate wrapper: loads its kernel build, allocates the outputs and launches the kernel.

values, indices = the k largest entries of each row of x[m, n] in descending order and their positions, ties broken by
the lowest index (the reference's topk/candidate.py:1-10 with K = 50). k is inputs["k"] when given (1..1024; the
reference fixes 50). The one `launch` entry of libkernel.so serves both dtypes: fp32 (0) and bf16 (1), row-major x;
values keep x's dtype and indices are int64. `plan` picks the columns per workgroup so the grid is one resident wave;
rows split into several chunks merge in the kernel (the library keeps its hand-off workspaces; the reference's int64
workspace and per-row int32 counters are still allocated and passed, zeroed once). The plan and workspace of the last
shape are cached, so a repeated call allocates only its outputs.
params.json (optional) may set "log2_threads" (7..9), "log2_depth" (1..3) -- the reference's knobs, validated and not
needed by this build -- and "min_chunk". The library is $CKOPT_BUILD_DIR/libkernel.so when CKOPT_BUILD_DIR is set,
else this package's build/topk/libkernel.so.
"""

import ctypes
import json
import os

import torch

K = 50
K_MAX = 1024
_HERE = os.path.dirname(os.path.abspath(__file__))
_PARAMS_PATH = os.path.join(_HERE, "params.json")
_params = {}
if os.path.exists(_PARAMS_PATH):
    with open(_PARAMS_PATH) as _handle:
        _params = json.load(_handle)
_THREADS = 1 << int(_params.get("log2_threads", 8))
_DEPTH = 1 << int(_params.get("log2_depth", 2))
_MIN_CHUNK = int(_params.get("min_chunk", 2048))
_DTYPES = {torch.float32: 0, torch.bfloat16: 1}

LIB_PATH = os.path.join(os.environ.get("CKOPT_BUILD_DIR") or os.path.join(_HERE, "..", "build", "topk"),
                        "libkernel.so")
if not os.path.exists(LIB_PATH):
    raise ImportError(f"topk: {LIB_PATH} is missing (build it with make_libs.py)")
_lib = ctypes.CDLL(LIB_PATH)
_lib.plan.argtypes = [ctypes.c_longlong, ctypes.c_longlong, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int]
_lib.plan.restype = ctypes.c_longlong
_lib.launch.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                        ctypes.c_longlong, ctypes.c_longlong, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                        ctypes.c_longlong, ctypes.c_void_p]
_lib.launch.restype = ctypes.c_int
_lib.topk_reset.argtypes = [ctypes.c_void_p, ctypes.c_longlong, ctypes.c_void_p]
_lib.topk_reset.restype = ctypes.c_int
_lib.topk_sample_launch.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_longlong, ctypes.c_int, ctypes.c_int,
                                                             ctypes.c_float, ctypes.c_float, ctypes.c_void_p]
_lib.topk_sample_launch.restype = ctypes.c_int
_lib.topk_launch_sample.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_longlong, ctypes.c_longlong] + [ctypes.c_int] * 4 + \
                                   [ctypes.c_longlong, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_float, ctypes.c_float,
                                    ctypes.c_void_p]
_lib.topk_launch_sample.restype = ctypes.c_int

_counters = {}
_last = None  # (key, chunk, work pointer, counters pointer, work, counters) of the last shape


def _row_counters(device, rows):
    counters = _counters.get(device)
    if counters is None or counters.numel() < rows:
        counters = torch.zeros(rows if rows > 4096 else 4096, dtype=torch.int32, device=device)
        _counters[device] = counters
    return counters


def _plan(x, rows, cols, dtype, k=K):
    # Launches of one shape on the stream are serialized and every chunk rewrites its workspace slots before the row's
    # last workgroup reads them, so the workspace is reused; a new shape frees the old one before allocating.
    global _last
    key = (x.get_device(), rows, cols, dtype, k)
    if _last is not None and _last[0] == key:
        return _last
    _last = None
    # larger k: larger chunks (fewer lists of k to merge per row)
    chunk = _lib.plan(rows, cols, dtype, _THREADS, _DEPTH, max(_MIN_CHUNK, 16 * k) if k > 64 else _MIN_CHUNK)
    nchunks = -(-cols // chunk)
    work = torch.empty(rows * nchunks * k if nchunks > 1 else 1, dtype=torch.int64, device=x.device)
    counters = _row_counters(x.device, rows)
    _last = (key, chunk, work.data_ptr(), counters.data_ptr(), work, counters)
    return _last


def run(inputs):
    x = inputs["x"]
    k = int(inputs.get("k", K))
    dtype = _DTYPES.get(x.dtype)
    if dtype is None or x.dim() != 2 or not 1 <= k <= K_MAX or x.shape[1] < k or x.device.type != "cuda":
        raise ValueError(f"topk candidate takes a 2-D fp32 or bf16 GPU tensor with at least k columns and "
                         f"1 <= k <= {K_MAX}, got {x.dtype} with shape {tuple(x.shape)} on {x.device}, k = {k}")
    x = x.contiguous()
    rows, cols = x.shape
    _, chunk, work_ptr, counters_ptr, _, _ = _plan(x, rows, cols, dtype, k)
    values = torch.empty((rows, k), dtype=x.dtype, device=x.device)
    indices = torch.empty((rows, k), dtype=torch.int64, device=x.device)
    err = _lib.launch(x.data_ptr(), values.data_ptr(), indices.data_ptr(), work_ptr, counters_ptr,
                      rows, cols, k, dtype, _THREADS, _DEPTH, chunk, torch.cuda.current_stream(x.device).cuda_stream)
    if err:
        raise RuntimeError(f"kernel launch failed: HIP error {err}")
    return {"values": values, "indices": indices}


def sample(values, indices, uniforms, temperature=1.0, top_p=1.0):
    """One index per row drawn from a top-k list (run()'s values and indices): softmax(values / temperature), the
    nucleus cut top_p, and the caller's uniforms [rows] (fp32 in [0, 1)) as the draw; temperature <= 0 is greedy.
    No counterpart in the reference (the step after top-k in a decoder's sampler). Returns int64 [rows]."""
    dtype = _DTYPES.get(values.dtype)
    if dtype is None or values.dim() != 2 or indices.shape != values.shape or indices.dtype != torch.int64 \
            or uniforms.dtype != torch.float32 or tuple(uniforms.shape) != (values.shape[0],) \
            or not 1 <= values.shape[1] <= K_MAX or values.device.type != "cuda" \
            or indices.device != values.device or uniforms.device != values.device:
        raise ValueError(f"topk sample takes values [rows, k] (fp32/bf16, k <= {K_MAX}), int64 indices of that shape "
                         f"and fp32 uniforms [rows] on one GPU, got {values.dtype} {tuple(values.shape)}, "
                         f"{indices.dtype} {tuple(indices.shape)}, {uniforms.dtype} {tuple(uniforms.shape)}")
    values, indices, uniforms = values.contiguous(), indices.contiguous(), uniforms.contiguous()
    out = torch.empty(values.shape[0], dtype=torch.int64, device=values.device)
    err = _lib.topk_sample_launch(values.data_ptr(), indices.data_ptr(), uniforms.data_ptr(), out.data_ptr(),
                                  values.shape[0], values.shape[1], dtype, float(temperature), float(top_p),
                                  torch.cuda.current_stream(values.device).cuda_stream)
    if err:
        raise RuntimeError(f"kernel launch failed: HIP error {err}")
    return out


def run_and_sample(inputs, uniforms, temperature=1.0, top_p=1.0):
    """run() and sample() in one launch: the workgroup that writes a row's values and indices also draws the row's
    index (topk_launch_sample). Returns (values, indices, drawn int64 [rows]), equal to run() followed by sample()."""
    x = inputs["x"]
    k = int(inputs.get("k", K))
    dtype = _DTYPES.get(x.dtype)
    if dtype is None or x.dim() != 2 or not 1 <= k <= K_MAX or x.shape[1] < k or x.device.type != "cuda":
        raise ValueError(f"topk candidate takes a 2-D fp32 or bf16 GPU tensor with at least k columns and "
                         f"1 <= k <= {K_MAX}, got {x.dtype} with shape {tuple(x.shape)} on {x.device}, k = {k}")
    if uniforms.dtype != torch.float32 or tuple(uniforms.shape) != (x.shape[0],) or uniforms.device != x.device:
        raise ValueError(f"topk sample takes fp32 uniforms [rows] on x's device, got {uniforms.dtype} "
                         f"{tuple(uniforms.shape)} on {uniforms.device}")
    x, uniforms = x.contiguous(), uniforms.contiguous()
    rows, cols = x.shape
    _, chunk, work_ptr, counters_ptr, _, _ = _plan(x, rows, cols, dtype, k)
    values = torch.empty((rows, k), dtype=x.dtype, device=x.device)
    indices = torch.empty((rows, k), dtype=torch.int64, device=x.device)
    drawn = torch.empty(rows, dtype=torch.int64, device=x.device)
    err = _lib.topk_launch_sample(x.data_ptr(), values.data_ptr(), indices.data_ptr(), work_ptr, counters_ptr, rows,
                                  cols, k, dtype, _THREADS, _DEPTH, chunk, uniforms.data_ptr(), drawn.data_ptr(),
                                  float(temperature), float(top_p), torch.cuda.current_stream(x.device).cuda_stream)
    if err:
        raise RuntimeError(f"kernel launch failed: HIP error {err}")
    return values, indices, drawn
