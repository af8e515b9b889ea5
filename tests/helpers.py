"""Shared helpers for the parity tests (device buffers via torch, tolerances)."""
import ctypes as C
import math

import numpy as np

from emberlm_amd import capi


def assert_close(got, ref, rtol=1e-4, name="", atol=0.0):
    """|a-b| <= rtol*|b| + rtol*max|b| + atol elementwise, and relative L2 <= rtol
    (the L2 check is skipped when the reference is all zero)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (name, got.shape, ref.shape)
    scale = float(np.max(np.abs(ref))) if ref.size else 0.0
    err = np.abs(got - ref)
    bound = rtol * np.abs(ref) + rtol * scale + atol
    bad = err > bound
    assert not bad.any(), (f"{name}: {int(bad.sum())} of {ref.size} outside tolerance; "
                           f"max err {err.max():.3e} at {np.unravel_index(err.argmax(), err.shape)}, "
                           f"scale {scale:.3e}")
    if scale > 0:
        l2 = np.linalg.norm(got - ref) / np.linalg.norm(ref)
        assert l2 <= rtol, f"{name}: relative L2 {l2:.3e} > {rtol}"


def dev(a, dtype=None):
    import torch
    a = np.ascontiguousarray(a)
    if dtype is None:
        dtype = np.float32 if a.dtype.kind == "f" else a.dtype
    return torch.from_numpy(np.ascontiguousarray(a.astype(dtype))).cuda()


def empty(shape, dtype=None):
    import torch
    return torch.empty(shape, dtype=dtype or torch.float32, device="cuda")


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def p(t):
    return C.c_void_p(t.data_ptr()) if t is not None else None


def call(name, *args):
    """C-ABI call on its own stream argument, ordered after and before torch's
    work: torch fills the inputs on its current stream, which need not be the
    stream the call runs on, so the device is synchronised on both sides."""
    import torch
    sync = torch.cuda.is_available()
    if sync:
        torch.cuda.synchronize()
    capi.call(name, *args)
    if sync:
        torch.cuda.synchronize()


def f32ptr(arr):
    arr = np.ascontiguousarray(arr, dtype=np.float32)
    return arr, arr.ctypes.data_as(C.POINTER(C.c_float))


def assert_matches_golden(golden, prefix, got, rtol=1e-4, rows=False):
    """Checks `got` against the summaries tests/golden/make_golden.py stored for
    it: every sampled value within rtol*|b| + rtol*max|b|, the L2 norm (from the
    sum of squares) and the maximum magnitude within rtol, the total sum within
    rtol of the norm times sqrt(n), and (rows=True) every row's sum and L2 norm."""
    got = np.asarray(got, dtype=np.float64)
    flat = got.reshape(-1)
    maxabs = float(golden[prefix + ".maxabs"])
    idx = golden[prefix + ".idx"]
    ref = golden[prefix + ".val"]
    err = np.abs(flat[idx] - ref)
    bound = rtol * np.abs(ref) + rtol * maxabs
    assert (err <= bound).all(), (prefix, "samples", float(err.max()), float(bound[err.argmax()]))
    norm_ref = math.sqrt(float(golden[prefix + ".sumsq"]))
    norm = math.sqrt(float((flat * flat).sum()))
    assert abs(norm - norm_ref) <= rtol * norm_ref, (prefix, "L2", norm, norm_ref)
    assert abs(float(np.abs(flat).max()) - maxabs) <= rtol * maxabs, (prefix, "max")
    assert abs(float(flat.sum()) - float(golden[prefix + ".sum"])) <= rtol * norm_ref * math.sqrt(
        flat.size), (prefix, "sum")
    if rows:
        r2 = got.reshape(-1, got.shape[-1])
        rs, rq = golden[prefix + ".row_sum"], golden[prefix + ".row_sumsq"]
        rn = np.sqrt(rq)
        assert (np.abs(r2.sum(1) - rs) <= rtol * rn * math.sqrt(r2.shape[1])).all(), (prefix, "row sums")
        assert (np.abs(np.sqrt((r2 * r2).sum(1)) - rn) <= rtol * rn).all(), (prefix, "row norms")


def fma_f32(a, b, c):
    """float32(a * b + c) rounded once, for float32 arrays.  a * b is exact in
    float64; TwoSum recovers the float64 sum's rounding error, whose sign
    decides the float32 rounding where the float64 sum lies exactly on a
    float32 midpoint (the only case where rounding twice can differ)."""
    x = np.asarray(a, np.float64) * np.asarray(b, np.float64)
    y = np.asarray(c, np.float64)
    s = x + y
    bb = s - x
    err = (x - (s - bb)) + (y - bb)
    f = s.astype(np.float32)
    lo = np.nextafter(f, np.float32(-np.inf))
    hi = np.nextafter(f, np.float32(np.inf))
    up_mid = (f.astype(np.float64) + hi.astype(np.float64)) / 2 == s
    dn_mid = (f.astype(np.float64) + lo.astype(np.float64)) / 2 == s
    f = np.where(up_mid & (err > 0), hi, f)
    f = np.where(dn_mid & (err < 0), lo, f)
    return f
