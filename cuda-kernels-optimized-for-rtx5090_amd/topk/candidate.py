"""Top-k of each row, served by this package's MI355X library through the reference's C entry points.

Contract (the reference's topk/candidate.py and its entry points topk/kernel.cu:520-570): run({"x": x}) with x a
2-D fp32 (dtype code 0) or bf16 (code 1) GPU tensor returns {"values", "indices"}: per row the k largest entries in
descending order (values keep x's dtype) and their int64 column positions, ties going to the lower position. k is 50,
as in the reference, unless inputs["k"] says otherwise (this build takes 1 <= k <= 1024; the reference stops at 512).

Launch protocol, as the reference's: `plan` gives the columns each workgroup scans; when a row spans several chunks,
the chunks hand their results over through a caller-owned int64 workspace of rows * nchunks * k entries and a
caller-owned array of int32 per-row counters that starts at zero and that the kernel leaves at zero. This wrapper
owns both, per (device, stream): the workspace of the most recent shape is kept for the next call of that shape, and
the counters are one zeroed array of at least 4096 entries, grown when a call has more rows.

Additions of this build (no counterpart in the reference): sample() draws one index per row from a top-k list, and
run_and_sample() does the top-k and that draw in one launch.

Library: libkernel.so from the directory named by CKOPT_BUILD_DIR, or this package's build/topk/ when that variable is
unset. A missing library is an ImportError; there is no CPU path.

Tuning file: an optional params.json beside this file may hold "log2_threads" (7..9), "log2_depth" (1..3) and
"min_chunk". The first two are the reference's CUDA knobs, validated by `launch` and not needed by the MI355X kernels;
min_chunk is handed to `plan`.

Errors: ValueError before any launch for an input the kernels do not take, RuntimeError carrying the HIP error code
when the launch reports one.
"""

import ctypes
import json
import os

import torch

K = 50
K_MAX = 1024
_HERE = os.path.dirname(os.path.abspath(__file__))


def _tuning():
    path = os.path.join(_HERE, "params.json")
    if not os.path.exists(path):
        return {}
    with open(path) as f:
        return json.load(f)


_TUNING = _tuning()
_THREADS = 1 << int(_TUNING.get("log2_threads", 8))
_DEPTH = 1 << int(_TUNING.get("log2_depth", 2))
_MIN_CHUNK = int(_TUNING.get("min_chunk", 2048))
_CODE = {torch.float32: 0, torch.bfloat16: 1}

LIB_PATH = os.path.join(os.environ.get("CKOPT_BUILD_DIR") or os.path.join(_HERE, "..", "build", "topk"),
                        "libkernel.so")
if not os.path.exists(LIB_PATH):
    raise ImportError(f"topk: no library at {LIB_PATH}; run make_libs.py first")
_lib = ctypes.CDLL(LIB_PATH)
# long long plan(long long rows, long long cols, int dtype, int threads, int depth, int min_chunk)
_lib.plan.argtypes = [ctypes.c_longlong, ctypes.c_longlong, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int]
_lib.plan.restype = ctypes.c_longlong
# int launch(x, values, indices, work, counters, long long rows, long long cols, int k, int dtype, int threads,
#            int depth, long long chunk, hipStream_t)
_lib.launch.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                        ctypes.c_longlong, ctypes.c_longlong, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                        ctypes.c_longlong, ctypes.c_void_p]
_lib.launch.restype = ctypes.c_int
# int topk_reset(void* counters, long long rows, hipStream_t)
_lib.topk_reset.argtypes = [ctypes.c_void_p, ctypes.c_longlong, ctypes.c_void_p]
_lib.topk_reset.restype = ctypes.c_int
# int topk_sample_launch(values, indices, uniforms, out, long long rows, int k, int dtype, float temperature,
#                        float top_p, hipStream_t)
_lib.topk_sample_launch.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_longlong, ctypes.c_int, ctypes.c_int,
                                                             ctypes.c_float, ctypes.c_float, ctypes.c_void_p]
_lib.topk_sample_launch.restype = ctypes.c_int
# int topk_launch_sample(launch()'s arguments up to chunk, uniforms, out, float temperature, float top_p, hipStream_t)
_lib.topk_launch_sample.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_longlong, ctypes.c_longlong] + [ctypes.c_int] * 4 + \
                                   [ctypes.c_longlong, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_float, ctypes.c_float,
                                    ctypes.c_void_p]
_lib.topk_launch_sample.restype = ctypes.c_int


class _Buffers:
    """The caller-side state of the launch protocol, kept per (device, stream): one zeroed counter array, and the plan
    and workspace of the most recent shape. Calls on one stream are ordered, and each split chunk rewrites its
    workspace slots before its row's merge reads them, so one workspace serves a stream's calls; two streams with calls
    in flight at once must not count arrivals on the same counters, so each stream has its own."""

    def __init__(self):
        self.counters = {}   # (device, stream) -> int32 zeros
        self.recent = {}     # (device, stream) -> (key, chunk, work)

    def counters_for(self, where, device, rows):
        c = self.counters.get(where)
        if c is None or c.numel() < rows:
            c = torch.zeros(max(rows, 4096), dtype=torch.int32, device=device)
            self.counters[where] = c
        return c

    def plan(self, x, rows, cols, dtype, k):
        where = (x.device, torch.cuda.current_stream(x.device).cuda_stream)
        key = (rows, cols, dtype, k)
        recent = self.recent.get(where)
        if recent is None or recent[0] != key:
            self.recent.pop(where, None)  # drop the old workspace before making the new one
            # k > 64 asks for chunks of at least 16k columns (a useful bound per chunk, fewer lists to merge)
            chunk = _lib.plan(rows, cols, dtype, _THREADS, _DEPTH, max(_MIN_CHUNK, 16 * k) if k > 64 else _MIN_CHUNK)
            nchunks = -(-cols // chunk)
            work = torch.empty(rows * nchunks * k if nchunks > 1 else 1, dtype=torch.int64, device=x.device)
            recent = (key, chunk, work)
            self.recent[where] = recent
        return recent[1], recent[2], self.counters_for(where, x.device, rows)


_buffers = _Buffers()


def _plan(x, rows, cols, dtype, k=K):
    """(chunk, work, counters) for a launch of this shape."""
    return _buffers.plan(x, rows, cols, dtype, k)


def _check_x(x, k):
    if _CODE.get(x.dtype) is None or x.dim() != 2 or not 1 <= k <= K_MAX or x.shape[1] < k or x.device.type != "cuda":
        raise ValueError(f"topk candidate takes a 2-D fp32 or bf16 GPU tensor with at least k columns and "
                         f"1 <= k <= {K_MAX}, got {x.dtype} with shape {tuple(x.shape)} on {x.device}, k = {k}")


def _checked(err):
    if err:
        raise RuntimeError(f"kernel launch failed: HIP error {err}")


def run(inputs):
    x = inputs["x"]
    k = int(inputs.get("k", K))
    _check_x(x, k)
    x = x.contiguous()
    rows, cols = x.shape
    dtype = _CODE[x.dtype]
    chunk, work, counters = _plan(x, rows, cols, dtype, k)
    values = torch.empty((rows, k), dtype=x.dtype, device=x.device)
    indices = torch.empty((rows, k), dtype=torch.int64, device=x.device)
    _checked(_lib.launch(x.data_ptr(), values.data_ptr(), indices.data_ptr(), work.data_ptr(), counters.data_ptr(),
                         rows, cols, k, dtype, _THREADS, _DEPTH, chunk, torch.cuda.current_stream(x.device).cuda_stream))
    return {"values": values, "indices": indices}


def sample(values, indices, uniforms, temperature=1.0, top_p=1.0):
    """One index per row drawn from a top-k list (run()'s values and indices): softmax(values / temperature), the
    nucleus cut top_p, and the caller's uniforms [rows] (fp32 in [0, 1)) as the draw; temperature <= 0 is greedy.
    No counterpart in the reference (the step after top-k in a decoder's sampler). Returns int64 [rows]."""
    dtype = _CODE.get(values.dtype)
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
    _checked(err)
    return out


def run_and_sample(inputs, uniforms, temperature=1.0, top_p=1.0):
    """run() and sample() in one launch: the workgroup that writes a row's values and indices also draws the row's
    index (topk_launch_sample). Returns (values, indices, drawn int64 [rows]), equal to run() followed by sample()."""
    x = inputs["x"]
    k = int(inputs.get("k", K))
    _check_x(x, k)
    if uniforms.dtype != torch.float32 or tuple(uniforms.shape) != (x.shape[0],) or uniforms.device != x.device:
        raise ValueError(f"topk sample takes fp32 uniforms [rows] on x's device, got {uniforms.dtype} "
                         f"{tuple(uniforms.shape)} on {uniforms.device}")
    x, uniforms = x.contiguous(), uniforms.contiguous()
    rows, cols = x.shape
    dtype = _CODE[x.dtype]
    chunk, work, counters = _plan(x, rows, cols, dtype, k)
    values = torch.empty((rows, k), dtype=x.dtype, device=x.device)
    indices = torch.empty((rows, k), dtype=torch.int64, device=x.device)
    drawn = torch.empty(rows, dtype=torch.int64, device=x.device)
    _checked(_lib.topk_launch_sample(x.data_ptr(), values.data_ptr(), indices.data_ptr(), work.data_ptr(),
                                     counters.data_ptr(), rows, cols, k, dtype, _THREADS, _DEPTH, chunk,
                                     uniforms.data_ptr(), drawn.data_ptr(), float(temperature), float(top_p),
                                     torch.cuda.current_stream(x.device).cuda_stream))
    return values, indices, drawn
