"""Shared helpers for the parity tests (device buffers via torch, tolerances)."""
import ctypes as C

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
