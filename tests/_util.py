"""Comparison helpers shared by the tests (bit views, ULP distances, tolerances)."""

import numpy as np
import torch


def bits16(t):
    """Raw uint16 bits of a bf16/fp16 tensor (any device) as a numpy array."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def from_bits16(a, dtype):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint16).view(np.int16)).view(dtype)


def ordered16(a):
    """Maps 16-bit float bits to integers ordered like the values (adjacent values differ by 1)."""
    a = a.astype(np.int32)
    return np.where(a & 0x8000, 0x8000 - a, a)


def ulp16(a, b):
    """Per-element distance in units of the last place between two 16-bit float bit arrays (NaN vs NaN -> 0)."""
    na, nb = is_nan16(a), is_nan16(b)
    d = np.abs(ordered16(a) - ordered16(b))
    d = np.where(na & nb, 0, d)
    d = np.where(na ^ nb, 1 << 20, d)
    return d


def is_nan16(a, fp16=False):
    a = a.astype(np.uint32)
    if fp16:
        return ((a & 0x7C00) == 0x7C00) & ((a & 0x03FF) != 0)
    return ((a & 0x7F80) == 0x7F80) & ((a & 0x007F) != 0)


def assert_rel(got, ref, rtol=1e-5, what="", atol=0.0):
    """|got - ref| <= rtol * |ref| + atol elementwise (NaN must match NaN)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    nan_g, nan_r = np.isnan(got), np.isnan(ref)
    assert np.array_equal(nan_g, nan_r), f"{what}: NaN positions differ"
    ok = nan_r | (np.abs(got - ref) <= rtol * np.abs(ref) + atol)
    if not ok.all():
        i = np.argwhere(~ok)[0]
        raise AssertionError(f"{what}: {int((~ok).sum())} elements beyond rtol {rtol} + atol {atol}; first at "
                             f"{tuple(i)}: got {got[tuple(i)]!r} ref {ref[tuple(i)]!r}")


def assert_ulp(got_bits, ref_bits, max_ulp=1, what=""):
    d = ulp16(got_bits, ref_bits)
    if d.max(initial=0) > max_ulp:
        i = np.unravel_index(int(np.argmax(d)), d.shape)
        raise AssertionError(f"{what}: {int((d > max_ulp).sum())} elements beyond {max_ulp} ulp; worst {int(d[i])} at "
                             f"{i}: got {got_bits[i]:#06x} ref {ref_bits[i]:#06x}")


def same_bits16(a, b, fp16=False):
    """Bitwise equality of 16-bit float arrays, with any NaN equal to any NaN (payload and sign of a NaN are not
    values: x86 and the GPU produce different default NaNs for inf * 0)."""
    na, nb = is_nan16(a, fp16), is_nan16(b, fp16)
    return np.array_equal(na, nb) and np.array_equal(np.where(na, 0, a), np.where(nb, 0, b))
