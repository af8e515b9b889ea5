"""numpy front end of oracle/ref_f32.c, the reference's scalar fp32 CPU test
ops (TEST INFRASTRUCTURE ONLY: bench.py's CPU baseline and its check in
tests/test_ref_f32.py; the product path never loads it).

Weights use the reference's layouts and the oracle's key names
(``oracle.BLOCK_KEYS``); every array is float32 and C-contiguous.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libref_f32.so")
_lib = None
_fp = C.POINTER(C.c_float)

_KEYS = ["input_layernorm", "q_proj", "k_proj", "v_proj", "o_proj", "q_norm", "k_norm",
         "post_attention_layernorm", "gate_proj", "up_proj", "down_proj"]


class BlockCfg(C.Structure):
    _fields_ = [("d", C.c_int), ("H", C.c_int), ("Hk", C.c_int), ("Dh", C.c_int), ("I", C.c_int),
                ("eps", C.c_float), ("theta", C.c_float)]


class BlockPtrs(C.Structure):
    _fields_ = [(k, _fp) for k in ("ln1", "wq", "wk", "wv", "wo", "qn", "kn", "ln2", "wg", "wu",
                                   "wd")]


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            subprocess.run(["make", "-s", "-C", _HERE], check=True)
        _lib = C.CDLL(_LIB_PATH)
        _lib.rf_lm_head_ce.restype = C.c_float
    return _lib


def f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _p(a):
    return None if a is None else a.ctypes.data_as(_fp)


def _ptrs(w: dict):
    return BlockPtrs(*[_p(w.get(k)) for k in _KEYS])


def block_fwd_bwd(cfg: BlockCfg, w: dict, x, dy, checkpoint=False):
    """One block over T tokens (batch 1): y, dx and the weight gradients
    (dict), with the reference's checkpointing (forward, then forward again
    before the backward) when `checkpoint`."""
    w = {k: f32(v) for k, v in w.items()}
    x, dy = f32(x), f32(dy)
    T = x.shape[0]
    y, dx = np.empty_like(x), np.empty_like(x)
    g = {k: np.zeros_like(v) for k, v in w.items()}
    gp = _ptrs(g)
    lib().rf_block_fwd_bwd(C.byref(cfg), C.byref(_ptrs(w)), _p(x), _p(dy), _p(y), _p(dx),
                           C.byref(gp), T, int(checkpoint))
    return y, dx, g


def attention_head(q, k, v, dout=None):
    """One causal attention head over [T, D] arrays: o, or (o, dq, dk, dv)."""
    q, k, v = f32(q), f32(k), f32(v)
    T, D = q.shape
    o = np.empty_like(q)
    if dout is None:
        lib().rf_attention_head(_p(q), _p(k), _p(v), None, _p(o), None, None, None, T, D)
        return o
    dq, dk, dv = np.empty_like(q), np.empty_like(q), np.empty_like(q)
    lib().rf_attention_head(_p(q), _p(k), _p(v), _p(f32(dout)), _p(o), _p(dq), _p(dk), _p(dv),
                            T, D)
    return o, dq, dk, dv


def lm_head_ce(h, E, tgt, mask):
    """Tied LM head + masked mean CE: (loss, dh, dE)."""
    h, E, mask = f32(h), f32(E), f32(mask)
    tgt = np.ascontiguousarray(tgt, dtype=np.int64)
    n, d = h.shape
    dh, dE = np.empty_like(h), np.zeros_like(E)
    loss = lib().rf_lm_head_ce(_p(h), _p(E), tgt.ctypes.data_as(C.POINTER(C.c_int64)), _p(mask),
                               _p(dh), _p(dE), n, d, E.shape[0])
    return float(loss), dh, dE


def adamw(p, g, m, v, lr, b1, b2, eps, wd, step):
    """In place on float32 p, m, v."""
    lib().rf_adamw(_p(p), _p(f32(g)), _p(m), _p(v), C.c_int64(p.size), C.c_float(lr),
                   C.c_float(b1), C.c_float(b2), C.c_float(eps), C.c_float(wd), step)
