"""CPU oracle of the four row-wise kernels (softmax, RMSNorm, RoPE, top-k).

TEST INFRASTRUCTURE ONLY: tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg are the only callers, and
only as the checker (or the timed CPU baseline). The product path never imports this package.

Two layers:
  - `liboracle.so` (oracle.c, built by oracle/Makefile): the C restatement of the reference's arithmetic, wrapped here
    with numpy in / numpy out (bf16 and fp16 carried as raw uint16 bits);
  - `torch_paths`: the reference's own PyTorch paths (softmax/baseline.py:13 and the torch expressions the other
    wrappers' docstrings name), used to pin the C restatement in tests.
"""

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

_lib = None


def build():
    """Compiles liboracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        src = os.path.join(HERE, "oracle.c")
        if not os.path.exists(LIB_PATH) or os.path.getmtime(LIB_PATH) < os.path.getmtime(src):
            build()
        L = ctypes.CDLL(LIB_PATH)
        vp, ll, i, f = ctypes.c_void_p, ctypes.c_longlong, ctypes.c_int, ctypes.c_float
        L.oracle_softmax.argtypes = [vp, vp, ll, ll, i]
        L.oracle_rmsnorm.argtypes = [vp, vp, vp, ll, ll, i, f, vp]
        L.oracle_rmsnorm_add.argtypes = [vp, vp, vp, vp, vp, ll, ll, i, f]
        L.oracle_topk_sample.argtypes = [vp, vp, vp, vp, ll, i, i, f, f, vp]
        L.oracle_topk_sample_band.argtypes = [vp, vp, vp, vp, ll, i, i, f, f]
        L.oracle_rope_cache.argtypes = [vp, vp, vp, vp, vp, vp, vp, ll, i, i, i, i, i]
        L.oracle_rope_freq.argtypes = [vp, vp, vp, vp, vp, vp, ll, i, i, i, i]
        L.oracle_rope_table.argtypes = [vp, ll, i, vp, vp]
        L.oracle_topk.argtypes = [vp, vp, vp, ll, ll, i, i]
        L.oracle_f32_to_bf16.argtypes = [f]
        L.oracle_f32_to_bf16.restype = ctypes.c_uint16
        L.oracle_f32_to_f16.argtypes = [f]
        L.oracle_f32_to_f16.restype = ctypes.c_uint16
        for fn in ("oracle_softmax", "oracle_rmsnorm", "oracle_rope_cache", "oracle_rope_freq", "oracle_rope_table",
                   "oracle_topk", "oracle_topk_sample", "oracle_topk_sample_band"):
            getattr(L, fn).restype = None
        _lib = L
    return _lib


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# dtype codes of the reference ABIs
SOFTMAX_DTYPES = {"fp32": 0, "bf16": 1}
NORM_DTYPES = {"bf16": 1, "fp16": 2}
CACHE_DTYPES = {"fp32": 0, "bf16": 1, "fp16": 2}


def softmax(x, dtype="fp32"):
    """x: float32 array (fp32) or uint16 bf16 bits, shape [rows, cols]. Returns the same kind."""
    if dtype == "fp32":
        x = _c(x, np.float32)
        y = np.empty_like(x)
    else:
        x = _c(x, np.uint16)
        y = np.empty_like(x)
    rows, cols = x.shape
    lib().oracle_softmax(_ptr(x), _ptr(y), rows, cols, SOFTMAX_DTYPES[dtype])
    return y


def rmsnorm(x, weight=None, eps=1e-6, dtype="bf16", return_inv=False):
    """x: uint16 bits [rows, cols]; weight: uint16 bits [cols] or None. Returns y bits (and fp32 inv per row)."""
    x = _c(x, np.uint16)
    w = _c(weight, np.uint16) if weight is not None else None
    y = np.empty_like(x)
    rows, cols = x.shape
    inv = np.empty(rows, dtype=np.float32)
    lib().oracle_rmsnorm(_ptr(x), _ptr(w), _ptr(y), rows, cols, NORM_DTYPES[dtype], ctypes.c_float(eps), _ptr(inv))
    return (y, inv) if return_inv else y


def rmsnorm_add(x, residual, weight=None, eps=1e-6, dtype="bf16"):
    """Fused residual add + RMSNorm on uint16 bits: returns (y, h) with h = T(x + residual) and y = rmsnorm(h)."""
    x, r = _c(x, np.uint16), _c(residual, np.uint16)
    w = _c(weight, np.uint16) if weight is not None else None
    y, h = np.empty_like(x), np.empty_like(x)
    rows, cols = x.shape
    lib().oracle_rmsnorm_add(_ptr(x), _ptr(r), _ptr(w), _ptr(y), _ptr(h), rows, cols, NORM_DTYPES[dtype],
                             ctypes.c_float(eps))
    return y, h


def rope_cache(q, k, cos, sin, ids, dtype="bf16", cache_dtype="fp32"):
    """q [tokens, qh, D], k [tokens, kh, D] uint16 bits; cos/sin [P, D]; ids int64 [tokens]. Returns (q_out, k_out)."""
    q, k = _c(q, np.uint16), _c(k, np.uint16)
    cdt = np.float32 if cache_dtype == "fp32" else np.uint16
    cos, sin, ids = _c(cos, cdt), _c(sin, cdt), _c(ids, np.int64)
    qo, ko = np.empty_like(q), np.empty_like(k)
    tokens, qh, D = q.shape
    lib().oracle_rope_cache(_ptr(q), _ptr(k), _ptr(cos), _ptr(sin), _ptr(ids), _ptr(qo), _ptr(ko), tokens, qh,
                            k.shape[1], D, NORM_DTYPES[dtype], CACHE_DTYPES[cache_dtype])
    return qo, ko


def rope_freq(q, k, ids, inv_freq, dtype="bf16"):
    """On-the-fly form: cos/sin of fp32(float(pos) * inv_freq[i]) in fp64, rounded to fp32."""
    q, k = _c(q, np.uint16), _c(k, np.uint16)
    ids, inv_freq = _c(ids, np.int64), _c(inv_freq, np.float32)
    qo, ko = np.empty_like(q), np.empty_like(k)
    tokens, qh, D = q.shape
    lib().oracle_rope_freq(_ptr(q), _ptr(k), _ptr(ids), _ptr(inv_freq), _ptr(qo), _ptr(ko), tokens, qh, k.shape[1],
                           D, NORM_DTYPES[dtype])
    return qo, ko


def rope_kv(q, k, v, ids, inv_freq, slots, k_cache, v_cache, dtype="bf16"):
    """RoPE fused with the KV-cache write (flash layout [slots, kv_heads, D]): returns (q_out, k_cache', v_cache')
    with q_out = rope_freq(q), and for every token t with slots[t] >= 0, k_cache'[slots[t]] = rope_freq(k)[t] and
    v_cache'[slots[t]] = v[t]; other cache rows keep their contents. All tensors as uint16 bits."""
    qo, ko = rope_freq(q, k, ids, inv_freq, dtype)
    kc, vc = np.array(k_cache, dtype=np.uint16, copy=True), np.array(v_cache, dtype=np.uint16, copy=True)
    for t, slot in enumerate(np.asarray(slots, dtype=np.int64)):
        if slot >= 0:
            kc[slot] = ko[t]
            vc[slot] = np.asarray(v, dtype=np.uint16)[t]
    return qo, kc, vc


def rope_table(inv_freq, positions, head_dim):
    """The fp32 cos/sin cache [positions, head_dim] that the on-the-fly form evaluates."""
    inv_freq = _c(inv_freq, np.float32)
    cos = np.empty((positions, head_dim), dtype=np.float32)
    sin = np.empty_like(cos)
    lib().oracle_rope_table(_ptr(inv_freq), positions, head_dim, _ptr(cos), _ptr(sin))
    return cos, sin


def topk(x, k, dtype="fp32"):
    """x: float32 [rows, cols] or uint16 bf16 bits. Returns (values in x's kind, int64 indices), each [rows, k]."""
    x = _c(x, np.float32 if dtype == "fp32" else np.uint16)
    rows, cols = x.shape
    assert 0 < k <= cols
    vals = np.empty((rows, k), dtype=x.dtype)
    idx = np.empty((rows, k), dtype=np.int64)
    lib().oracle_topk(_ptr(x), _ptr(vals), _ptr(idx), rows, cols, k, 0 if dtype == "fp32" else 1)
    return vals, idx


def f32_to_bf16_bits(a):
    """Round-to-nearest-even fp32 -> bf16 bits (numpy), NaN -> 0x7fc0."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    r = ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    r[nan] = np.uint16(0x7FC0)
    return r


def bf16_bits_to_f32(b):
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def topk_sample(values, indices, u, temperature=1.0, top_p=1.0, dtype="fp32"):
    """Draws one index per row of a top-k list (values fp32 or bf16 bits [rows, k], int64 indices) with uniforms u.
    Returns (drawn int64 [rows], ambiguous bool [rows]: the draw or the cut lies within fp32 rounding of a boundary)."""
    vals = _c(values, np.float32 if dtype == "fp32" else np.uint16)
    idx, uu = _c(indices, np.int64), _c(u, np.float32)
    rows, k = idx.shape
    out = np.empty(rows, dtype=np.int64)
    amb = np.empty(rows, dtype=np.int32)
    lib().oracle_topk_sample(_ptr(vals), _ptr(idx), _ptr(uu), _ptr(out), rows, k, 0 if dtype == "fp32" else 1,
                             ctypes.c_float(temperature), ctypes.c_float(top_p), _ptr(amb))
    return out, amb.astype(bool)


def topk_sample_band(values, indices, u, temperature=1.0, top_p=1.0, dtype="fp32"):
    """The admissible draws of topk_sample for every row: (lo, hi) int arrays of list positions, the draws that the
    rule gives when its sums, cut and target each move by up to 1e-5 of the row's total (fp32 evaluation in any order).
    A draw is correct when it is one of indices[r, lo[r]..hi[r]]."""
    vals = _c(values, np.float32 if dtype == "fp32" else np.uint16)
    uu = _c(u, np.float32)
    rows, k = np.asarray(indices).shape
    lo = np.empty(rows, dtype=np.int32)
    hi = np.empty(rows, dtype=np.int32)
    lib().oracle_topk_sample_band(_ptr(vals), _ptr(uu), _ptr(lo), _ptr(hi), rows, k, 0 if dtype == "fp32" else 1,
                                  ctypes.c_float(temperature), ctypes.c_float(top_p))
    return lo, hi


def draw_admissible(drawn, indices, lo, hi):
    """Whether each row's drawn index is one of indices[r, lo[r]..hi[r]]."""
    idx = np.asarray(indices)
    pos = np.arange(idx.shape[1])[None, :]
    window = (pos >= np.asarray(lo)[:, None]) & (pos <= np.asarray(hi)[:, None])
    return ((idx == np.asarray(drawn)[:, None]) & window).any(axis=1)