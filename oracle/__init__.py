"""CPU oracle for the emberlm training hot path -- TEST INFRASTRUCTURE ONLY.

numpy front end (ctypes) over ``oracle/ember_oracle.c``, the double-precision
restatement of the reference's math.  Only ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` may import this package; the
product path (``emberlm_amd``) never does.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libember_oracle.so")
_lib = None

_d = C.POINTER(C.c_double)
_i64 = C.POINTER(C.c_int64)
I64 = C.c_int64


class OrcCfg(C.Structure):
    _fields_ = [
        ("vocab", C.c_int64), ("hidden", C.c_int64), ("inter", C.c_int64),
        ("layers", C.c_int64), ("heads", C.c_int64), ("kv_heads", C.c_int64),
        ("head_dim", C.c_int64), ("eps", C.c_double), ("theta", C.c_float),
        ("rope_factor", C.c_float), ("rope_low_freq", C.c_float),
        ("rope_high_freq", C.c_float), ("rope_orig_max_pos", C.c_int),
        ("qk_norm", C.c_int),
    ]


def build() -> None:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = C.CDLL(_LIB_PATH)
        _lib.orc_ce_masked_fwd.restype = C.c_double
        _lib.orc_model_loss.restype = C.c_double
        _lib.orc_model_num_params.restype = C.c_int64
        _lib.orc_rope_freq.restype = C.c_float
        _lib.orc_rope_freq.argtypes = [C.c_int, C.c_int, C.c_float, C.c_float, C.c_float,
                                       C.c_float, C.c_int]
    return _lib


def _f64(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float64)


def _p(a: np.ndarray):
    if a.dtype == np.int64:
        return a.ctypes.data_as(_i64)
    return a.ctypes.data_as(_d)


# ----------------------------------------------------------------- GEMM
def matmul(a, b, transa=False, transb=False):
    a, b = _f64(a), _f64(b)
    M, K = (a.shape[1], a.shape[0]) if transa else a.shape
    N = b.shape[0] if transb else b.shape[1]
    Kb = b.shape[1] if transb else b.shape[0]
    assert K == Kb
    c = np.zeros((M, N))
    lib().orc_matmul(_p(a), _p(b), _p(c), I64(M), I64(N), I64(K), int(transa), int(transb),
                     C.c_double(0.0))
    return c


def bmm(a, b, transa=False, transb=False):
    a, b = _f64(a), _f64(b)
    S = a.shape[0]
    M, K = (a.shape[2], a.shape[1]) if transa else a.shape[1:]
    N = b.shape[1] if transb else b.shape[2]
    c = np.zeros((S, M, N))
    lib().orc_bmm(_p(a), _p(b), _p(c), I64(S), I64(M), I64(N), I64(K), int(transa), int(transb))
    return c


# -------------------------------------------------------------- RMSNorm
def rmsnorm_fwd(x, w, eps):
    x, w = _f64(x), _f64(w)
    H = x.shape[-1]
    y = np.zeros_like(x)
    lib().orc_rmsnorm_fwd(_p(x), _p(w), _p(y), I64(x.size // H), I64(H), C.c_double(eps))
    return y


def rmsnorm_bwd(dy, x, w, eps):
    dy, x, w = _f64(dy), _f64(x), _f64(w)
    H = x.shape[-1]
    dx = np.zeros_like(x)
    dw = np.zeros(H)
    lib().orc_rmsnorm_bwd(_p(dy), _p(x), _p(w), _p(dx), _p(dw), I64(x.size // H), I64(H),
                          C.c_double(eps))
    return dx, dw


# ----------------------------------------------------------------- RoPE
def rope_freq(i, D, theta, factor=0.0, low=1.0, high=4.0, orig=8192):
    return lib().orc_rope_freq(i, D, theta, factor, low, high, orig)


def rope(x, theta, pos0=0, sign=1.0, factor=0.0, low=1.0, high=4.0, orig=8192):
    x = _f64(x)
    B, T, H, D = x.shape
    y = np.zeros_like(x)
    lib().orc_rope(_p(x), _p(y), I64(B), I64(T), I64(H), I64(D), I64(pos0), C.c_float(theta),
                   C.c_double(sign), C.c_float(factor), C.c_float(low), C.c_float(high),
                   C.c_int(orig))
    return y


# -------------------------------------------------------------- Softmax
def softmax_fwd(x):
    x = _f64(x)
    N = x.shape[-1]
    y = np.zeros_like(x)
    lib().orc_softmax_fwd(_p(x), _p(y), I64(x.size // N), I64(N))
    return y


def softmax_bwd(y, g):
    y, g = _f64(y), _f64(g)
    N = y.shape[-1]
    dx = np.zeros_like(y)
    lib().orc_softmax_bwd(_p(y), _p(g), _p(dx), I64(y.size // N), I64(N))
    return dx


def causal_mask(x, q0=0, fill=-3.4028234663852886e38):
    x = _f64(x)
    Tq, Tk = x.shape[-2], x.shape[-1]
    y = np.zeros_like(x)
    lib().orc_causal_mask(_p(x), _p(y), I64(x.size // Tk), I64(Tq), I64(Tk), I64(q0),
                          C.c_double(fill))
    return y


def repeat_kv(x, group):
    x = _f64(x)
    B, T, Hk, D = x.shape
    y = np.zeros((B, T, Hk * group, D))
    lib().orc_repeat_kv(_p(x), _p(y), I64(B * T), I64(Hk), I64(group), I64(D))
    return y


def repeat_kv_sum(y, group):
    y = _f64(y)
    B, T, H, D = y.shape
    x = np.zeros((B, T, H // group, D))
    lib().orc_repeat_kv_sum(_p(y), _p(x), I64(B * T), I64(H // group), I64(group), I64(D))
    return x


def permute(x, perm):
    x = _f64(x)
    shape = np.array(x.shape, dtype=np.int64)
    pa = (C.c_int * len(perm))(*perm)
    y = np.zeros(tuple(x.shape[p] for p in perm))
    lib().orc_permute(_p(x), _p(y), C.c_int(x.ndim), _p(shape), pa)
    return y


# -------------------------------------------------------------- SwiGLU
def silu(x):
    x = _f64(x)
    y = np.zeros_like(x)
    lib().orc_silu(_p(x), _p(y), I64(x.size))
    return y


def silu_bwd(x, g):
    x, g = _f64(x), _f64(g)
    dx = np.zeros_like(x)
    lib().orc_silu_bwd(_p(x), _p(g), _p(dx), I64(x.size))
    return dx


# ------------------------------------------------------------ Masked CE
def ce_masked_fwd(logits, tgt, mask):
    logits, mask = _f64(logits), _f64(mask)
    tgt = np.ascontiguousarray(tgt, dtype=np.int64)
    N, V = logits.shape
    lse = np.zeros(N)
    ms = C.c_double(0.0)
    loss = lib().orc_ce_masked_fwd(_p(logits), _p(tgt), _p(mask), I64(N), I64(V), _p(lse),
                                   C.byref(ms))
    return loss, lse, ms.value


def ce_masked_bwd(logits, tgt, mask, dy=1.0):
    logits, mask = _f64(logits), _f64(mask)
    tgt = np.ascontiguousarray(tgt, dtype=np.int64)
    N, V = logits.shape
    d = np.zeros_like(logits)
    lib().orc_ce_masked_bwd(_p(logits), _p(tgt), _p(mask), I64(N), I64(V), C.c_double(dy), _p(d))
    return d


# ------------------------------------------------------------ Embedding
def embedding_fwd(ids, w):
    ids = np.ascontiguousarray(ids, dtype=np.int64)
    w = _f64(w)
    out = np.zeros(ids.shape + (w.shape[1],))
    lib().orc_embedding_fwd(_p(ids), _p(w), _p(out), I64(ids.size), I64(w.shape[1]))
    return out


def embedding_bwd(ids, dy, V):
    ids = np.ascontiguousarray(ids, dtype=np.int64)
    dy = _f64(dy)
    H = dy.shape[-1]
    dw = np.zeros((V, H))
    lib().orc_embedding_bwd(_p(ids), _p(dy), _p(dw), I64(ids.size), I64(H), I64(V))
    return dw


# ---------------------------------------------------------------- AdamW
def adamw(p, g, m, v, lr, beta1, beta2, eps, wd, bc1, bc2):
    p, g, m, v = _f64(p).copy(), _f64(g), _f64(m).copy(), _f64(v).copy()
    lib().orc_adamw(_p(p), _p(g), _p(m), _p(v), I64(p.size), C.c_double(lr), C.c_double(beta1),
                    C.c_double(beta2), C.c_double(eps), C.c_double(wd), C.c_double(bc1),
                    C.c_double(bc2))
    return p, m, v


# ------------------------------------------------------------ Attention
def attention_fwd(q, k, v, scale=None):
    q, k, v = _f64(q), _f64(k), _f64(v)
    B, T, H, D = q.shape
    Hk = k.shape[2]
    scale = 1.0 / np.sqrt(D) if scale is None else scale
    o = np.zeros_like(q)
    lse = np.zeros((B, H, T))
    lib().orc_attention_fwd(_p(q), _p(k), _p(v), _p(o), _p(lse), I64(B), I64(T), I64(H),
                            I64(Hk), I64(D), C.c_double(scale))
    return o, lse


def attention_bwd(q, k, v, do, scale=None):
    q, k, v, do = _f64(q), _f64(k), _f64(v), _f64(do)
    B, T, H, D = q.shape
    Hk = k.shape[2]
    scale = 1.0 / np.sqrt(D) if scale is None else scale
    dq, dk, dv = np.zeros_like(q), np.zeros_like(k), np.zeros_like(v)
    lib().orc_attention_bwd(_p(q), _p(k), _p(v), _p(do), _p(dq), _p(dk), _p(dv), I64(B),
                            I64(T), I64(H), I64(Hk), I64(D), C.c_double(scale))
    return dq, dk, dv


def attention_offset(q, k, v, pos, scale=None):
    """Inference attention with a position offset: q [B,T,H,D] over key rows k,v
    [B,L,Hk,D]; query t sees keys j <= pos + t."""
    q, k, v = _f64(q), _f64(k), _f64(v)
    B, T, H, D = q.shape
    L, Hk = k.shape[1], k.shape[2]
    scale = 1.0 / np.sqrt(D) if scale is None else scale
    o = np.zeros_like(q)
    lib().orc_attention_offset(_p(q), _p(k), _p(v), _p(o), I64(B), I64(T), I64(L), I64(H),
                               I64(Hk), I64(D), I64(pos), C.c_double(scale))
    return o


# ---------------------------------------------------------- Block / Model
BLOCK_KEYS = ["input_layernorm", "q_proj", "k_proj", "v_proj", "o_proj", "q_norm", "k_norm",
              "post_attention_layernorm", "gate_proj", "up_proj", "down_proj"]


def make_cfg(**kw) -> OrcCfg:
    c = OrcCfg()
    defaults = dict(vocab=0, hidden=0, inter=0, layers=1, heads=1, kv_heads=1, head_dim=1,
                    eps=1e-5, theta=1e4, rope_factor=0.0, rope_low_freq=1.0,
                    rope_high_freq=4.0, rope_orig_max_pos=8192, qk_norm=0)
    defaults.update(kw)
    for k_, v_ in defaults.items():
        setattr(c, k_, v_)
    return c


def _block_ptrs(cfg, w: dict):
    arrs = []
    ptrs = (_d * 11)()
    for i, key in enumerate(BLOCK_KEYS):
        if key in w and w[key] is not None:
            a = _f64(w[key])
            arrs.append(a)
            ptrs[i] = _p(a)
        else:
            ptrs[i] = None
    return ptrs, arrs


def block_fwd(cfg, w: dict, x):
    x = _f64(x)
    B, T, _ = x.shape
    y = np.zeros_like(x)
    ptrs, keep = _block_ptrs(cfg, w)
    lib().orc_block_fwd(C.byref(cfg), ptrs, _p(x), _p(y), I64(B), I64(T))
    return y


def block_bwd(cfg, w: dict, x, dy):
    x, dy = _f64(x), _f64(dy)
    B, T, _ = x.shape
    dx = np.zeros_like(x)
    ptrs, keep = _block_ptrs(cfg, w)
    grads = {}
    gptrs = (_d * 11)()
    for i, key in enumerate(BLOCK_KEYS):
        shape = np.shape(w[key]) if (key in w and w[key] is not None) else (cfg.head_dim,)
        grads[key] = np.zeros(shape)
        gptrs[i] = _p(grads[key])
    lib().orc_block_bwd(C.byref(cfg), ptrs, _p(x), _p(dy), _p(dx), gptrs, I64(B), I64(T))
    return dx, {k_: v_ for k_, v_ in grads.items() if k_ in w and w[k_] is not None}


def model_loss(cfg, params: list, ids, targets, mask, want_grads=True):
    """params: list of arrays in collect_parameters order (src/nn/model.cpp:63-100)."""
    arrs = [_f64(p) for p in params]
    n = len(arrs)
    assert n == lib().orc_model_num_params(C.byref(cfg))
    pp = (_d * n)(*[_p(a) for a in arrs])
    grads = [np.zeros_like(a) for a in arrs] if want_grads else None
    gp = (_d * n)(*[_p(g) for g in grads]) if want_grads else None
    ids = np.ascontiguousarray(ids, dtype=np.int64)
    tg = np.ascontiguousarray(targets, dtype=np.int64)
    mk = _f64(mask)
    B, T = ids.shape
    loss = lib().orc_model_loss(C.byref(cfg), pp, gp, _p(ids), _p(tg), _p(mk), I64(B), I64(T))
    return loss, grads


def model_logits(cfg, params: list, ids):
    """Logits [B,T,V] of Model::forward without a cache."""
    arrs = [_f64(p) for p in params]
    n = len(arrs)
    assert n == lib().orc_model_num_params(C.byref(cfg))
    pp = (_d * n)(*[_p(a) for a in arrs])
    ids = np.ascontiguousarray(ids, dtype=np.int64)
    B, T = ids.shape
    out = np.zeros((B, T, cfg.vocab))
    lib().orc_model_logits(C.byref(cfg), pp, _p(ids), _p(out), I64(B), I64(T))
    return out
