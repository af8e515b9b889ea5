"""GPU parity of the inference path (reference include/ctd/nn/attention.h:43-97,
src/ops/kv_cache.cu, include/ctd/nn/model.h:152-163, src/core/sampling.cpp,
tools/ctd_generate/main.cpp) against the CPU oracle.

- KV cache kernels: write_kv / read_kv_expanded against numpy index arithmetic
  (bitwise: they only move floats).
- Decode attention (ember_attn_decode) against oracle.attention_offset, over the
  cache layout and the projection layout, one to five query heads per KV head,
  D 64/128, short and split key ranges (up to 8192 keys), T > 1 with an offset;
  bitwise run-to-run.
- QK-Norm + RoPE + cache write folded into the decode attention
  (ember_attn_decode_qkv) against the oracle and against the two launches it
  replaces, new rows inside one split and across a split boundary; the value
  rows and the untouched cache rows bitwise.
- Skinny GEMM (M <= 8 rows, the decode Linear) against the oracle.
- Device argmax against the host scan (ties, NaN, -inf), bitwise.
- Model::forward with a cache, as the reference's KVCachePrefillEquivalence
  (prefill with cache vs without: max |diff| < 5e-5) and
  KVCachePrefillThenDecode (decode after a prefix vs the full forward's last
  row: < 5e-4), plus many decode steps and chunked prefill against the
  oracle's full-sequence logits (causality makes every cached step a row of
  it).
- ctd_generate end to end against oracle/generate.py on the oracle's logits.
Tolerance for float results: |a-b| <= 1e-4|b| + 1e-4 max|b| and relative
L2 <= 1e-4 (fp32 against the fp64 oracle).
"""
import ctypes as C
import json
import os
import subprocess

import numpy as np
import pytest

import oracle as O
from oracle import generate as OG
from oracle import sampling as OS
from tests.helpers import assert_close, call, dev, empty, host, p

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

from emberlm_amd import capi  # noqa: E402
from emberlm_amd import trainer as TR  # noqa: E402
from tests.test_gpu_model import oracle_cfg, shapes  # noqa: E402


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.cuda.init()


def rng(s=0):
    return np.random.default_rng(s)


# ------------------------------------------------------------ KV cache ops
@pytest.mark.parametrize("B,T,Hk,D,S,pos", [(1, 1, 8, 128, 64, 17), (2, 5, 3, 64, 16, 11),
                                             (2, 3, 2, 6, 9, 0)])
def test_kv_write_and_read_expanded(B, T, Hk, D, S, pos):
    r = rng(B * T + D)
    src = r.standard_normal((B, T, Hk, D)).astype(np.float32)
    cache0 = r.standard_normal((B, Hk, S, D)).astype(np.float32)
    cache, srcd = dev(cache0), dev(src)
    call("ember_kv_write", p(srcd), p(cache), B, T, Hk, D, S, pos, None)
    ref = cache0.copy()
    ref[:, :, pos:pos + T, :] = src.transpose(0, 2, 1, 3)
    got = host(cache)
    assert np.array_equal(got, ref)
    group, L = 3, pos + T
    out = empty((B, Hk * group, L, D))
    call("ember_kv_read_expanded", p(cache), p(out), B, Hk, group, L, D, S, None)
    assert np.array_equal(host(out), np.repeat(ref[:, :, :L], group, axis=1))


# ------------------------------------------------------- decode attention
def decode(q, k, v, L, pos, layout, scale):
    """ember_attn_decode over a [B,Hk,S,D] cache ("cache") or [B,T,Hk,D] rows ("proj")."""
    B, T, H, D = q.shape
    if layout == "cache":
        _, Hk, S, _ = k.shape
        strides = (Hk * S * D, S * D, D)
    else:
        _, Tk, Hk, _ = k.shape
        strides = (Tk * Hk * D, D, Hk * D)
    qd, kd, vd = dev(q), dev(k), dev(v)
    o = empty((B, T, H, D))
    wsb = capi.lib().ember_attn_decode_workspace_bytes(B, T, H, Hk, D, L)
    ws = empty((max(1, wsb // 4),))
    call("ember_attn_decode", p(qd), p(kd), p(vd), p(o), B, T, H, Hk, D, L, pos, *strides,
         scale, p(ws) if wsb else None, wsb, None)
    return host(o)


CASES = [  # B, T, H, Hk, D, L, pos, S
    (1, 1, 16, 8, 128, 1, 0, 8),          # first decode position
    (1, 1, 16, 8, 128, 300, 299, 512),    # qwen3-1.7b heads, 5 splits
    (1, 1, 16, 8, 128, 4096, 4095, 4096), # full context: 64 splits of 64 keys
    (2, 1, 32, 8, 64, 1000, 999, 1024),   # llama3.2-1b heads (group 4)
    (1, 1, 15, 3, 64, 257, 256, 300),     # group 5: two row tiles
    (1, 1, 9, 3, 64, 77, 76, 80),         # smollm2-135m heads (group 3)
    (2, 7, 4, 2, 64, 40, 33, 48),         # chunked prefill: T 7 after 33 cached
    (1, 3, 4, 4, 128, 8192, 8189, 8192),  # long context, MHA
]


@pytest.mark.parametrize("B,T,H,Hk,D,L,pos,S", CASES)
def test_decode_attention_over_cache_vs_oracle(B, T, H, Hk, D, L, pos, S):
    r = rng(L + H)
    q = r.standard_normal((B, T, H, D)).astype(np.float32)
    k = r.standard_normal((B, Hk, S, D)).astype(np.float32)
    v = r.standard_normal((B, Hk, S, D)).astype(np.float32)
    scale = 1.0 / np.sqrt(D)
    got = decode(q, k, v, L, pos, "cache", scale)
    ref = O.attention_offset(q, k[:, :, :L].transpose(0, 2, 1, 3), v[:, :, :L].transpose(0, 2, 1, 3),
                             pos, scale)
    assert_close(got, ref, name="decode")
    assert np.array_equal(got, decode(q, k, v, L, pos, "cache", scale))  # reproducible


@pytest.mark.parametrize("T,pos", [(6, 3), (9, 20), (1, 5)])
def test_offset_attention_over_projections_vs_oracle(T, pos):
    r = rng(T + pos)
    B, H, Hk, D = 2, 6, 2, 64
    q = r.standard_normal((B, T, H, D)).astype(np.float32)
    k = r.standard_normal((B, T, Hk, D)).astype(np.float32)
    v = r.standard_normal((B, T, Hk, D)).astype(np.float32)
    got = decode(q, k, v, T, pos, "proj", 0.125)
    assert_close(got, O.attention_offset(q, k, v, pos, 0.125), name="offset")


# ------------------------------------------------------------- skinny GEMM
@pytest.mark.parametrize("M,N,K", [(1, 2048, 2048), (1, 151936, 64), (2, 1024, 2048),
                                   (3, 6144, 2048), (4, 2048, 6144), (7, 1001, 36), (8, 130, 1024),
                                   (5, 3, 4)])
def test_skinny_gemm_vs_oracle(M, N, K):
    r = rng(M * N + K)
    a = r.standard_normal((M, K)).astype(np.float32)
    b = r.standard_normal((N, K)).astype(np.float32)
    c0 = r.standard_normal((M, N)).astype(np.float32)
    A, Bm, Cm = dev(a), dev(b), dev(c0)
    call("ember_gemm_f32", 0, 1, M, N, K, 0.5, p(A), K, 0, p(Bm), K, 0, 2.0, p(Cm), N, 0, 1, None)
    ref = 0.5 * O.matmul(a, b, transb=True) + 2.0 * c0
    assert_close(host(Cm), ref, name="skinny")
    call("ember_gemm_f32", 0, 1, M, N, K, 1.0, p(A), K, 0, p(Bm), K, 0, 0.0, p(Cm), N, 0, 1, None)
    assert_close(host(Cm), O.matmul(a, b, transb=True), name="skinny beta0")


# ------------------------------------------------------ fused decode kernels
def ptr_array(ts):
    return (C.c_void_p * 3)(*[t.data_ptr() if t is not None else None for t in ts])


@pytest.mark.parametrize("M,K,Ns,norm,resid", [
    (1, 2048, (2048, 1024, 1024), True, False),   # qwen3-1.7b RMSNorm + Q/K/V
    (2, 2048, (2048,), False, True),              # O projection + residual
    (1, 6144, (2048,), False, True),              # down projection + residual
    (8, 576, (576, 192, 192), True, False),       # smollm2-135m, 8 rows
    (3, 64, (5, 7, 9), True, True),               # ragged rows
])
def test_decode_gemv_vs_oracle(M, K, Ns, norm, resid):
    r = rng(M * K)
    x = r.standard_normal((M, K)).astype(np.float32)
    nw = (1 + 0.1 * r.standard_normal(K)).astype(np.float32)
    Ws = [(0.05 * r.standard_normal((n, K))).astype(np.float32) for n in Ns]
    Rs = [r.standard_normal((M, n)).astype(np.float32) for n in Ns]
    xd, nwd = dev(x), dev(nw)
    Wd = [dev(w) for w in Ws]
    Yd = [empty((M, n)) for n in Ns]
    Rd = [dev(a) for a in Rs]
    Nn = (C.c_int64 * 3)(*Ns)
    call("ember_decode_gemv", p(xd), M, K, p(nwd) if norm else None, 1e-6, len(Ns),
         C.cast(ptr_array(Wd), C.POINTER(C.c_void_p)), Nn,
         C.cast(ptr_array(Yd), C.POINTER(C.c_void_p)),
         C.cast(ptr_array(Rd), C.POINTER(C.c_void_p)) if resid else None, None)
    xn = O.rmsnorm_fwd(x, nw, 1e-6) if norm else x
    for w, y, res in zip(Ws, Yd, Rs):
        ref = O.matmul(xn, w, transb=True) + (res if resid else 0.0)
        assert_close(host(y), ref, name="decode_gemv")


@pytest.mark.parametrize("M,K,I", [(1, 2048, 6144), (4, 576, 1536), (8, 128, 258)])
def test_decode_gateup_vs_oracle(M, K, I):
    r = rng(K + I)
    x = r.standard_normal((M, K)).astype(np.float32)
    nw = (1 + 0.1 * r.standard_normal(K)).astype(np.float32)
    wg, wu = ((0.05 * r.standard_normal((I, K))).astype(np.float32) for _ in range(2))
    out = empty((M, I))
    xd, nwd, wgd, wud = dev(x), dev(nw), dev(wg), dev(wu)  # held until the call has run
    call("ember_decode_gateup", p(xd), M, K, p(nwd), 1e-5, p(wgd), p(wud), I, p(out), None)
    xn = O.rmsnorm_fwd(x, nw, 1e-5)
    ref = O.silu(O.matmul(xn, wg, transb=True)) * O.matmul(xn, wu, transb=True)
    assert_close(host(out), ref, name="decode_gateup")


@pytest.mark.parametrize("B,T,H,Hk,D,pos,qk,factor", [(1, 1, 16, 8, 128, 300, True, 0.0),
                                                      (2, 3, 8, 2, 64, 17, False, 32.0),
                                                      (1, 2, 9, 3, 64, 0, False, 0.0)])
def test_decode_qkv_post_vs_oracle(B, T, H, Hk, D, pos, qk, factor):
    r = rng(H * D + pos)
    S, theta, eps = pos + T + 5, 5e5, 1e-6
    q = r.standard_normal((B, T, H, D)).astype(np.float32)
    k = r.standard_normal((B, T, Hk, D)).astype(np.float32)
    v = r.standard_normal((B, T, Hk, D)).astype(np.float32)
    qn, kn = ((1 + 0.1 * r.standard_normal(D)).astype(np.float32) for _ in range(2))
    ck0 = r.standard_normal((B, Hk, S, D)).astype(np.float32)
    cv0 = r.standard_normal((B, Hk, S, D)).astype(np.float32)
    ck, cv, qo = dev(ck0), dev(cv0), empty((B, T, H, D))
    freqs = (C.c_float * (D // 2))()
    capi.check(capi.lib().ember_rope_freqs_host(freqs, D, theta, factor, 1.0, 4.0, 64))
    qd, kd, vd, qnd, knd = dev(q), dev(k), dev(v), dev(qn), dev(kn)
    call("ember_decode_qkv_post", p(qd), p(kd), p(vd), B, T, H, Hk, D, p(qnd) if qk else None,
         p(knd) if qk else None, eps, freqs, pos, p(qo), p(ck), p(cv), S, None)
    rope = dict(theta=theta, pos0=pos, factor=factor, low=1.0, high=4.0, orig=64)
    qr = O.rope(O.rmsnorm_fwd(q, qn, eps) if qk else q, **rope)
    kr = O.rope(O.rmsnorm_fwd(k, kn, eps) if qk else k, **rope)
    assert_close(host(qo), qr, name="q")
    got_k, got_v = host(ck), host(cv)
    assert_close(got_k[:, :, pos:pos + T], kr.transpose(0, 2, 1, 3), name="k cache")
    assert np.array_equal(got_v[:, :, pos:pos + T], v.transpose(0, 2, 1, 3))
    keep = np.ones(S, bool)
    keep[pos:pos + T] = False                       # other cache rows untouched
    assert np.array_equal(got_k[:, :, keep], ck0[:, :, keep])
    assert np.array_equal(got_v[:, :, keep], cv0[:, :, keep])


@pytest.mark.parametrize("B,T,H,Hk,D,pos,S,qk,factor", [
    (1, 1, 16, 8, 128, 4095, 4096, True, 0.0),   # qwen3-1.7b heads, full context, 64 splits
    (1, 1, 16, 8, 128, 300, 512, True, 0.0),     # 5 splits
    (2, 3, 8, 2, 64, 17, 24, False, 32.0),       # llama3 frequencies, one split
    (1, 2, 9, 3, 64, 0, 4, False, 0.0),          # the cache's first rows
    (1, 7, 4, 2, 128, 1018, 1030, True, 0.0),    # new rows 1018..1024 across splits 31 | 32
])
def test_decode_attention_qkv_fold(B, T, H, Hk, D, pos, S, qk, factor):
    r = rng(H * D + pos + T)
    theta, eps, scale, L = 5e5, 1e-6, 1.0 / np.sqrt(D), pos + T
    q = r.standard_normal((B, T, H, D)).astype(np.float32)
    k = r.standard_normal((B, T, Hk, D)).astype(np.float32)
    v = r.standard_normal((B, T, Hk, D)).astype(np.float32)
    qn, kn = ((1 + 0.1 * r.standard_normal(D)).astype(np.float32) for _ in range(2))
    ck0 = r.standard_normal((B, Hk, S, D)).astype(np.float32)
    cv0 = r.standard_normal((B, Hk, S, D)).astype(np.float32)
    freqs = (C.c_float * (D // 2))()
    capi.check(capi.lib().ember_rope_freqs_host(freqs, D, theta, factor, 1.0, 4.0, 64))
    qd, kd, vd, qnd, knd = dev(q), dev(k), dev(v), dev(qn), dev(kn)
    wsb = capi.lib().ember_attn_decode_workspace_bytes(B, T, H, Hk, D, L)
    ws = empty((max(1, wsb // 4),))

    def fused():
        ck, cv, o = dev(ck0), dev(cv0), empty((B, T, H, D))
        call("ember_attn_decode_qkv", p(qd), p(kd), p(vd), B, T, H, Hk, D,
             p(qnd) if qk else None, p(knd) if qk else None, eps, freqs, pos, p(ck), p(cv), S,
             scale, p(o), p(ws) if wsb else None, wsb, None)
        return host(o), host(ck), host(cv)

    o, got_k, got_v = fused()
    rope = dict(theta=theta, pos0=pos, factor=factor, low=1.0, high=4.0, orig=64)
    qr = O.rope(O.rmsnorm_fwd(q, qn, eps) if qk else q, **rope)
    kr = O.rope(O.rmsnorm_fwd(k, kn, eps) if qk else k, **rope)
    assert_close(got_k[:, :, pos:L], kr.transpose(0, 2, 1, 3), name="k cache")
    assert np.array_equal(got_v[:, :, pos:L], v.transpose(0, 2, 1, 3))
    keep = np.ones(S, bool)
    keep[pos:L] = False                             # other cache rows untouched
    assert np.array_equal(got_k[:, :, keep], ck0[:, :, keep])
    assert np.array_equal(got_v[:, :, keep], cv0[:, :, keep])
    kf, vf = ck0[:, :, :L].astype(np.float64), cv0[:, :, :L].astype(np.float64)
    kf[:, :, pos:L] = kr.transpose(0, 2, 1, 3)
    vf[:, :, pos:L] = v.transpose(0, 2, 1, 3)
    ref = O.attention_offset(qr, kf.transpose(0, 2, 1, 3), vf.transpose(0, 2, 1, 3), pos, scale)
    assert_close(o, ref, name="o")
    # the two launches it replaces, on the same inputs
    ck, cv, qo = dev(ck0), dev(cv0), empty((B, T, H, D))
    call("ember_decode_qkv_post", p(qd), p(kd), p(vd), B, T, H, Hk, D, p(qnd) if qk else None,
         p(knd) if qk else None, eps, freqs, pos, p(qo), p(ck), p(cv), S, None)
    assert_close(o, decode(host(qo), host(ck), host(cv), L, pos, "cache", scale), rtol=1e-5,
                 name="o vs qkv_post + attn_decode")
    again = fused()
    assert all(np.array_equal(a, b) for a, b in zip(again, (o, got_k, got_v)))  # reproducible


# ------------------------------------------------------------------ argmax
def test_device_argmax_equals_host_scan():
    nan, inf = np.nan, np.inf
    r = rng(5)
    rows = [r.standard_normal(151936).astype(np.float32) for _ in range(3)]
    rows[1][[7, 90000, 151935]] = 50.0                  # ties: the first index wins
    special = np.array([[1.0, 3.0, 3.0, 2.0], [nan, 5.0, 7.0, 1.0], [1.0, nan, 0.5, 0.0],
                        [-inf, -inf, -inf, -inf], [-inf, 2.0, inf, inf], [nan, nan, nan, nan]],
                       np.float32)
    rows[2][:] = -1.0
    rows[2][[5, 100000]] = [-0.0, 0.0]                  # +0 and -0 tie: the first wins
    nan_first = r.standard_normal(151936).astype(np.float32)
    nan_first[0] = nan                                  # NaN at 0 wins by default
    for x in (np.stack(rows + [nan_first]), special):
        want = [OS.argmax(row) for row in x]
        xd = dev(x)
        out = torch.zeros(x.shape[0], dtype=torch.int64, device="cuda")
        call("ember_argmax_rows", p(xd), x.shape[0], x.shape[1], p(out), None)
        assert list(host(out)) == want
        wsb = capi.lib().ember_argmax_rows_workspace_bytes(x.shape[0], x.shape[1])
        ws = empty((max(1, wsb // 4),))
        out.zero_()
        call("ember_argmax_rows_ws", p(xd), x.shape[0], x.shape[1], p(out), p(ws), wsb, None)
        assert list(host(out)) == want
    assert want == [1, 0, 0, 0, 2, 0]
    # through ctd::sample: greedy on the device, the same tokens as the host path
    z = r.standard_normal((4, 5000)).astype(np.float32)
    assert np.array_equal(TR.sample(z, 0.0, on_device=True), TR.sample(z, 0.0))
    assert np.array_equal(TR.sample(z, 0.8, 50, 0.9, seed=3, draws=3, on_device=True),
                          TR.sample(z, 0.8, 50, 0.9, seed=3, draws=3))


# ------------------------------------------------- model with a KV cache
def infer_cfg(variant):
    base = dict(vocab_size=512, hidden_size=128, intermediate_size=256, num_layers=2,
                num_heads=4, num_kv_heads=2, head_dim=64, rms_norm_eps=1e-5, rope_theta=1e4)
    if variant == "qwen3":
        base.update(head_dim=128, qk_norm=1, rms_norm_eps=1e-6, rope_theta=1e6)
    elif variant == "llama3":
        base.update(num_heads=8, rope_theta=5e5, rope_factor=32.0, rope_original_max_pos=16)
    elif variant == "d32":  # head size outside the fused kernels: the reference op chain
        base.update(head_dim=32, qk_norm=1, rms_norm_eps=1e-6)
    return TR.make_config(**base)


def host_params(c, seed, std=0.2):
    """Weights drawn on the host in collect_parameters order: (names -> arrays)."""
    r = rng(seed)
    sh = shapes(c)
    tr = TR.Trainer(c, seed=0)
    params = []
    for i, name in enumerate(tr.names):
        if name == "model.embed_tokens.weight":
            a = std * r.standard_normal((c.vocab_size, c.hidden_size))
        elif name.endswith("norm.weight"):
            n = tr.numels[i]
            a = 1.0 + 0.1 * r.standard_normal(n)
        else:
            a = std * r.standard_normal(sh[name.split(".")[-2]])
        a = a.astype(np.float32)
        tr.set_param(i, a)
        params.append(a)
    return tr, params


@pytest.mark.parametrize("variant", ["smollm2", "qwen3", "llama3", "d32"])
def test_prefill_with_cache_equals_no_cache(variant):
    c = infer_cfg(variant)
    tr, params = host_params(c, 1)
    ids = rng(2).integers(0, c.vocab_size, (2, 37))
    full = tr.forward(ids)
    cache = tr.kv_cache(2, 64)
    cached = tr.forward(ids, cache, 0)
    assert np.abs(full - cached).max() < 5e-5          # reference KVCachePrefillEquivalence
    assert cache.current_len == 37
    assert_close(full, O.model_logits(oracle_cfg(c), params, ids), name="prefill logits")
    tr.close()


@pytest.mark.parametrize("variant", ["smollm2", "qwen3", "llama3", "d32"])
def test_prefill_then_decode_steps_equal_full_forward(variant):
    c = infer_cfg(variant)
    tr, params = host_params(c, 3)
    B, T, P = 2, 40, 25
    ids = rng(4).integers(0, c.vocab_size, (B, T))
    ref = O.model_logits(oracle_cfg(c), params, ids)
    full = tr.forward(ids)
    cache = tr.kv_cache(B, T + 4)
    tr.forward(ids[:, :P], cache, 0)
    assert cache.current_len == P
    for t in range(P, T):                           # one token per step
        step = tr.forward(ids[:, t:t + 1], cache, t)
        assert cache.current_len == t + 1
        assert np.abs(step[:, 0] - full[:, t]).max() < 5e-4  # KVCachePrefillThenDecode
        assert_close(step[:, 0], ref[:, t], name=f"decode step {t}")
    tr.close()


def test_chunked_prefill_and_last_only_logits():
    c = infer_cfg("qwen3")
    tr, params = host_params(c, 5)
    B, T = 2, 30
    ids = rng(6).integers(0, c.vocab_size, (B, T))
    ref = O.model_logits(oracle_cfg(c), params, ids)
    cache = tr.kv_cache(B, T)
    pos = 0
    for n in (11, 7, 1, 11):                        # T > 1 chunks after a cached prefix
        out = tr.forward(ids[:, pos:pos + n], cache, pos)
        assert_close(out, ref[:, pos:pos + n], name=f"chunk at {pos}")
        pos += n
    cache2 = tr.kv_cache(B, T)
    last = tr.forward(ids[:, :20], cache2, 0, last_only=True)
    assert last.shape == (B, 1, c.vocab_size)
    assert_close(last[:, 0], ref[:, 19], name="last-only prefill")
    last = tr.forward(ids[:, 20:23], cache2, 20, last_only=True)
    assert_close(last[:, 0], ref[:, 22], name="last-only chunk")
    tr.close()


def test_cache_bounds_are_checked():
    c = infer_cfg("smollm2")
    tr, _ = host_params(c, 7)
    cache = tr.kv_cache(1, 8)
    with pytest.raises(TR.CtdError, match="out of cache bounds"):
        tr.forward(np.zeros((1, 9), np.int64), cache, 0)
    with pytest.raises(TR.CtdError, match="batch"):
        tr.forward(np.zeros((2, 3), np.int64), cache, 0)
    tr.close()


# ------------------------------------------------------------ ctd_generate
GEN_EXE = os.path.join(os.path.dirname(TR.LIB_PATH), "ctd_generate")


@pytest.fixture(scope="module")
def gen_model(tmp_path_factory):
    c = infer_cfg("qwen3")
    tr, params = host_params(c, 11, std=0.3)
    d = tmp_path_factory.mktemp("gen")
    tr.save(d / "model.safetensors")
    tr.close()
    (d / "model.json").write_text(json.dumps(dict(
        vocab_size=c.vocab_size, hidden_size=c.hidden_size, intermediate_size=c.intermediate_size,
        num_hidden_layers=c.num_layers, num_attention_heads=c.num_heads,
        num_key_value_heads=c.num_kv_heads, head_dim=c.head_dim, qk_norm=True,
        rms_norm_eps=float(np.float32(c.rms_norm_eps)), rope_theta=c.rope_theta)))
    oc = oracle_cfg(c)
    return d, lambda toks: O.model_logits(oc, params, np.array([toks]))[0, -1]


def run_generate(d, req):
    r = subprocess.run([GEN_EXE, "--model", str(d / "model.safetensors"), "--config",
                        str(d / "model.json")], input=json.dumps(req), capture_output=True,
                       text=True, timeout=120)
    return r.returncode, r.stdout.splitlines(), r.stderr


def greedy_margins(last_logits, prompt, n):
    toks, gaps = list(prompt), []
    for _ in range(n):
        z = last_logits(toks)
        top2 = np.sort(z)[-2:]
        gaps.append(top2[1] - top2[0])
        toks.append(int(np.argmax(z)))
    return gaps


def test_generate_greedy_matches_oracle(gen_model):
    d, last_logits = gen_model
    req = {"input_ids": [5, 17, 300, 42, 7, 99], "max_new_tokens": 12, "temperature": 0.0}
    assert min(greedy_margins(last_logits, req["input_ids"], 12)) > 1e-3  # no near-ties
    rc, lines, err = run_generate(d, req)
    assert rc == 0, err
    assert lines == OG.generate(last_logits, req)
    assert json.loads(lines[-1]) == {"done": True, "generated_tokens": 12, "reason": "max_tokens"}
    assert "ctd_generate: prompt of 6 tokens" in err


def test_generate_sampled_matches_oracle(gen_model):
    d, last_logits = gen_model
    for extra in ({"temperature": 0.9, "seed": 7}, {"temperature": 0.7, "top_k": 20, "seed": 123},
                  {"temperature": 1.1, "top_p": 0.9, "seed": 2**40 + 3}):
        req = {"input_ids": [1, 2, 3, 4], "max_new_tokens": 10, **extra}
        rc, lines, err = run_generate(d, req)
        assert rc == 0, err
        assert lines == OG.generate(last_logits, req), extra


def test_generate_stop_reasons_and_budget_forcing(gen_model):
    d, last_logits = gen_model
    prompt = [9, 8, 7]
    first = OG.generate(last_logits, {"input_ids": prompt, "max_new_tokens": 3,
                                      "temperature": 0.0})
    t0 = json.loads(first[0])["token"]
    cases = [
        {"input_ids": prompt, "temperature": 0.0, "eos_ids": [t0]},          # eos at once
        {"input_ids": prompt, "temperature": 0.0, "max_seq_len": 8},          # cache full
        {"input_ids": [], "temperature": 0.0},                                # empty prompt
        {"input_ids": list(range(8)), "max_seq_len": 8},                      # prompt too long
        {"input_ids": prompt, "temperature": 0.0, "max_new_tokens": 9,        # budget forcing
         "thinking_token_budget": 2, "think_open_ids": [t0], "think_close_ids": [500, 501]},
    ]
    expect_reason = ["eos", "max_seq_len", "empty_prompt", "max_seq_len", "max_tokens"]
    for req, why in zip(cases, expect_reason):
        rc, lines, err = run_generate(d, req)
        assert rc == 0, err
        ref = OG.generate(last_logits, req)
        assert lines == ref, req
        assert json.loads(lines[-1])["reason"] == why
    forced = [json.loads(l)["token"] for l in OG.generate(last_logits, cases[-1])[:-1]]
    assert forced[0] == t0 and forced[3:5] == [500, 501]   # two thinking tokens, then close


def test_trainer_generate_greedy_matches_oracle():
    """The shared generation loop (greedy: token kept on the device, next step
    queued before the host reads it) through the C API."""
    c = infer_cfg("qwen3")
    tr, params = host_params(c, 11, std=0.3)
    oc = oracle_cfg(c)
    last_logits = lambda toks: O.model_logits(oc, params, np.array([toks]))[0, -1]  # noqa: E731
    prompt = [5, 17, 300, 42, 7, 99]
    ref = [json.loads(l)["token"] for l in
           OG.generate(last_logits, {"input_ids": prompt, "max_new_tokens": 12,
                                     "temperature": 0.0})[:-1]]
    toks, pf, dc = tr.generate(prompt, 12, max_seq=40)
    assert list(toks) == ref and pf > 0 and dc > 0
    toks, _, _ = tr.generate(prompt, 12, max_seq=40)      # repeatable
    assert list(toks) == ref
    tr.close()
