"""Pins the CPU oracle (oracle/ember_oracle.c) before it is trusted as the checker.

Each check comes from outside the oracle's own formula: the reference's
known-answer tests (literal values from /root/reference/tests/*.cpp), library
routines (numpy, scipy, torch on the CPU in float64), closed forms and
invariants, and central finite differences for every backward.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle as O



@pytest.fixture(autouse=True)
def _float64_default():
    # float64 torch defaults for this module only: a process-wide change made
    # at import would leak into the GPU tests collected with it.
    old = torch.get_default_dtype()
    torch.set_default_dtype(torch.float64)
    yield
    torch.set_default_dtype(old)


def rng(seed=0):
    return np.random.default_rng(seed)


def t64(a, grad=False):
    return torch.tensor(np.asarray(a, dtype=np.float64), requires_grad=grad)


def fd_grad(f, x, eps=1e-6, idx=None):
    """Central differences of scalar f at x (float64) for the flat indices idx."""
    x = np.array(x, dtype=np.float64)
    flat = x.reshape(-1)
    idx = range(flat.size) if idx is None else idx
    out = {}
    for i in idx:
        old = flat[i]
        flat[i] = old + eps
        fp = f(x)
        flat[i] = old - eps
        fm = f(x)
        flat[i] = old
        out[i] = (fp - fm) / (2 * eps)
    return out


# ---------------------------------------------------------------- GEMM
def test_matmul_nonsquare_kat():
    # tests/test_matmul.cpp:48-67
    a = np.array([[1, 2, 3], [4, 5, 6]], dtype=np.float64)
    b = np.arange(1, 13, dtype=np.float64).reshape(3, 4)
    np.testing.assert_array_equal(O.matmul(a, b), [[38, 44, 50, 56], [83, 98, 113, 128]])


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_matmul_transposes_vs_numpy(ta, tb):
    r = rng(1)
    M, N, K = 7, 5, 9
    a = r.standard_normal((K, M) if ta else (M, K))
    b = r.standard_normal((N, K) if tb else (K, N))
    ref = (a.T if ta else a) @ (b.T if tb else b)
    np.testing.assert_allclose(O.matmul(a, b, ta, tb), ref, rtol=1e-12, atol=1e-12)


def test_bmm_vs_numpy():
    r = rng(2)
    a, b = r.standard_normal((3, 4, 6)), r.standard_normal((3, 5, 6))
    np.testing.assert_allclose(O.bmm(a, b, False, True), a @ b.transpose(0, 2, 1), rtol=1e-12)


# ------------------------------------------------------------- RMSNorm
def test_rmsnorm_fwd_vs_torch():
    r = rng(3)
    x, w = r.standard_normal((5, 576)), r.standard_normal(576)
    ref = F.rms_norm(t64(x), (576,), t64(w), eps=1e-5).numpy()
    np.testing.assert_allclose(O.rmsnorm_fwd(x, w, 1e-5), ref, rtol=1e-12)


def test_rmsnorm_bwd_vs_torch_autograd():
    r = rng(4)
    x, w, dy = r.standard_normal((6, 32)), r.standard_normal(32), r.standard_normal((6, 32))
    tx, tw = t64(x, True), t64(w, True)
    (F.rms_norm(tx, (32,), tw, eps=1e-6) * t64(dy)).sum().backward()
    dx, dw = O.rmsnorm_bwd(dy, x, w, 1e-6)
    np.testing.assert_allclose(dx, tx.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dw, tw.grad.numpy(), rtol=1e-10, atol=1e-12)


def test_rmsnorm_bwd_finite_difference():
    r = rng(5)
    x, w, dy = r.standard_normal((3, 8)), r.standard_normal(8), r.standard_normal((3, 8))
    dx, dw = O.rmsnorm_bwd(dy, x, w, 1e-5)
    fx = fd_grad(lambda xx: float((O.rmsnorm_fwd(xx, w, 1e-5) * dy).sum()), x)
    fw = fd_grad(lambda ww: float((O.rmsnorm_fwd(x, ww, 1e-5) * dy).sum()), w)
    np.testing.assert_allclose(dx.reshape(-1), [fx[i] for i in range(24)], rtol=1e-6, atol=1e-8)
    np.testing.assert_allclose(dw, [fw[i] for i in range(8)], rtol=1e-6, atol=1e-8)


# ---------------------------------------------------------------- RoPE
def _rope_complex(x, theta, pos0, freqs):
    # Independent statement: rotate (a + i b) by exp(i * angle) per pair.
    B, T, H, D = x.shape
    z = x[..., : D // 2] + 1j * x[..., D // 2:]
    ang = np.array([[np.float32(np.float32(pos0 + t) * f) for f in freqs] for t in range(T)],
                   dtype=np.float64)
    z = z * np.exp(1j * ang)[None, :, None, :]
    return np.concatenate([z.real, z.imag], axis=-1)


def test_rope_position_offset_kat():
    # tests/test_rope.cpp:57-72: x = 1..8, pos 7, theta 1e4, D 8.
    x = np.arange(1, 9, dtype=np.float64).reshape(1, 1, 1, 8)
    freqs = [np.float32(np.float32(1e4) ** np.float32(-(2.0 * i) / 8)) for i in range(4)]
    ref = _rope_complex(x, 1e4, 7, freqs)
    got = O.rope(x, 1e4, pos0=7)
    np.testing.assert_allclose(got, ref, rtol=1e-6, atol=1e-6)
    # the reference test's tolerance against its float CPU oracle
    assert np.max(np.abs(got - ref)) < 1e-4


def test_rope_identity_and_norm_and_transpose():
    r = rng(6)
    x = r.standard_normal((2, 9, 3, 16))
    y0 = O.rope(x[:, :1], 1e5)  # position 0 is the identity rotation
    np.testing.assert_allclose(y0, x[:, :1], atol=0)
    y = O.rope(x, 1e5)
    pn = lambda a: a[..., :8] ** 2 + a[..., 8:] ** 2  # noqa: E731
    np.testing.assert_allclose(pn(y), pn(x), rtol=1e-12)
    back = O.rope(y, 1e5, sign=-1.0)
    np.testing.assert_allclose(back, x, atol=1e-12)


def test_rope_matches_complex_rotation_llama3():
    # Frequencies from the per-band statement (pinned to literals below), not
    # from the oracle.
    from tests.golden.make_golden import rope_freqs
    r = rng(7)
    D, theta = 64, 5e5
    x = r.standard_normal((1, 40, 2, D))
    freqs = rope_freqs(D, theta, 32.0, 1.0, 4.0, 8192)
    ref = _rope_complex(x, theta, 3, freqs)
    # the oracle's float arithmetic may land one ulp of a mid-band frequency
    # away (about 1e-7 rad at these positions)
    np.testing.assert_allclose(O.rope(x, theta, pos0=3, factor=32.0), ref, rtol=1e-7,
                               atol=1e-8)


# LLaMA-3.2 llama3 settings: D 64, theta 5e5, factor 32,
# low_freq 1, high_freq 4, original context L 8192.  The mid band
# (L/4 = 2048 < 2*pi/f <= 8192) holds i = 15, 16, 17.  Expected values worked
# out by hand from rope.cu:41-45 with f = 5e5^(-i/32):
#   i  f              2*pi/f       s = (wl-2048)/6144   (1-s) f + s f/32
#   15 2.13111954e-3  2948.30262   0.146533629          1.8285976285e-3
#   16 1.41421356e-3  4442.88294   0.389792145          8.8019076638e-4
#   17 9.38473870e-4  6695.10948   0.756365475          2.5082679882e-4
LLAMA3_MID = {15: 1.8285976285e-3, 16: 8.8019076638e-4, 17: 2.5082679882e-4}


def _llama3_alternatives(i, D=64, theta=5e5, fac=32.0, lf=1.0, hf=4.0, L=8192):
    """What two plausible mistakes give: HF's weighting and the reference's
    weights swapped."""
    base = theta ** (-2.0 * i / D)
    wl = 2 * math.pi / base
    s_hf = (L / wl - lf) / (hf - lf)
    s = (wl - L / hf) / (L / lf - L / hf)
    return (1 - s_hf) * base / fac + s_hf * base, s * base + (1 - s) * base / fac


def test_rope_llama3_mid_band_literals():
    for i, want in LLAMA3_MID.items():
        got = O.rope_freq(i, 64, 5e5, 32.0, 1.0, 4.0, 8192)
        assert got == pytest.approx(want, rel=1e-6), (i, got, want)
        hf_value, swapped = _llama3_alternatives(i)
        # a mistaken oracle would be at least 20% away from the literal
        assert abs(hf_value - want) > 0.2 * want and abs(swapped - want) > 0.2 * want


def test_rope_llama3_one_third_weight():
    # Constructed case: D 4, i 1 gives f = theta^(-1/2); theta = (4096/(2*pi))^2
    # puts the wavelength at 4096 exactly, so s = (4096-2048)/(8192-2048) = 1/3
    # and the reference's f' = (2/3) f + (1/3) f/32 = (65/96) f, where HF's
    # weighting (s' = (8192/4096 - 1)/3 = 1/3 on f, 2/3 on f/32) gives (34/96) f.
    theta = (4096 / (2 * math.pi)) ** 2
    base = float(np.float32(theta) ** np.float32(-0.5))
    got = O.rope_freq(1, 4, theta, 32.0, 1.0, 4.0, 8192)
    assert got / base == pytest.approx(65 / 96, rel=1e-6)
    assert abs(got / base - 34 / 96) > 0.3


def test_rope_llama3_bands():
    from tests.golden.make_golden import rope_freqs
    D, theta = 64, 5e5
    L, lf, hf, fac = 8192, 1.0, 4.0, 32.0
    closed = rope_freqs(D, theta, fac, lf, hf, L)
    for i, want in LLAMA3_MID.items():   # the per-band statement is pinned too
        assert float(closed[i]) == pytest.approx(want, rel=1e-6)
    for i in range(D // 2):
        base = float(np.float32(theta) ** np.float32(-(2.0 * i) / D))
        f = O.rope_freq(i, D, theta, fac, lf, hf, L)
        wl = 2 * math.pi / base
        if wl <= L / hf:
            assert f == base                                   # high-frequency band unchanged
        elif wl > L / lf:
            assert f == pytest.approx(base / fac, rel=1e-7)    # low-frequency band divided
        # every band within one float32 ulp of the per-band statement
        assert abs(np.float32(f) - closed[i]) <= np.spacing(closed[i]), i
    freqs = [O.rope_freq(i, D, theta, fac, lf, hf, L) for i in range(D // 2)]
    assert all(a >= b for a, b in zip(freqs, freqs[1:]))       # monotone in i
    assert O.rope_freq(0, D, theta, fac, lf, hf, L) == 1.0
    # below factor 1 the scaling is off: every frequency is the plain one
    plain = rope_freqs(D, theta)
    assert [O.rope_freq(i, D, theta, 0.0, lf, hf, L) for i in range(D // 2)] == list(plain)


# ------------------------------------------------------------- Softmax
def test_softmax_vs_scipy_and_extremes():
    from scipy.special import softmax as sp_softmax
    r = rng(8)
    x = r.standard_normal((4, 33)) * 5
    np.testing.assert_allclose(O.softmax_fwd(x), sp_softmax(x, axis=-1), rtol=1e-12)
    # tests/test_softmax.cpp:54-65
    y = O.softmax_fwd(np.array([[1000.0, 1001.0, 999.0]]))[0]
    assert abs(y.sum() - 1.0) < 1e-12 and y[1] > y[0] > y[2]


def test_softmax_bwd_vs_torch():
    r = rng(9)
    x, g = r.standard_normal((3, 11)), r.standard_normal((3, 11))
    tx = t64(x, True)
    (torch.softmax(tx, -1) * t64(g)).sum().backward()
    np.testing.assert_allclose(O.softmax_bwd(O.softmax_fwd(x), g), tx.grad.numpy(), rtol=1e-10,
                               atol=1e-13)


def test_causal_mask_kat():
    # tests/test_mask.cpp:10-30 and 32-41
    s = np.ones((1, 2, 4, 4))
    got = O.causal_mask(s)
    for i in range(4):
        for j in range(4):
            assert (got[0, :, i, j] <= -1e30).all() if j > i else (got[0, :, i, j] == 1).all()
    np.testing.assert_array_equal(O.causal_mask(np.ones((1, 5)), q0=4), np.ones((1, 5)))


# --------------------------------------------------------- GQA / permute
def test_repeat_kv_and_sum_vs_numpy():
    r = rng(10)
    x = r.standard_normal((2, 3, 2, 4))
    np.testing.assert_array_equal(O.repeat_kv(x, 3), np.repeat(x, 3, axis=2))
    y = r.standard_normal((2, 3, 6, 4))
    np.testing.assert_allclose(O.repeat_kv_sum(y, 3), y.reshape(2, 3, 2, 3, 4).sum(3), rtol=1e-14)


def test_permute_kats():
    # tests/test_permute.cpp:10-32 and 34-47
    x = np.arange(2 * 3 * 4 * 2, dtype=np.float64).reshape(2, 3, 4, 2)
    np.testing.assert_array_equal(O.permute(x, [0, 2, 1, 3]), x.transpose(0, 2, 1, 3))
    z = np.arange(60, dtype=np.float64).reshape(3, 4, 5) * 0.5
    np.testing.assert_array_equal(O.permute(O.permute(z, [2, 0, 1]), [1, 2, 0]), z)


# -------------------------------------------------------------- SwiGLU
def test_silu_and_bwd_vs_torch():
    r = rng(11)
    x, g = r.standard_normal(50) * 4, r.standard_normal(50)
    tx = t64(x, True)
    y = F.silu(tx)
    (y * t64(g)).sum().backward()
    np.testing.assert_allclose(O.silu(x), y.detach().numpy(), rtol=1e-13)
    np.testing.assert_allclose(O.silu_bwd(x, g), tx.grad.numpy(), rtol=1e-11, atol=1e-14)


# ------------------------------------------------------------ Masked CE
def test_ce_masked_vs_torch():
    r = rng(12)
    N, V = 9, 37
    logits, tgt = r.standard_normal((N, V)) * 3, r.integers(0, V, N)
    mask = (r.random(N) > 0.4).astype(np.float64)
    mask[0] = 1
    tl = t64(logits, True)
    per = F.cross_entropy(tl, torch.tensor(tgt), reduction="none")
    ref = (per * t64(mask)).sum() / mask.sum()
    ref.backward()
    loss, lse, ms = O.ce_masked_fwd(logits, tgt, mask)
    assert loss == pytest.approx(ref.item(), rel=1e-12)
    assert ms == mask.sum()
    np.testing.assert_allclose(lse, torch.logsumexp(t64(logits), -1).numpy(), rtol=1e-13)
    np.testing.assert_allclose(O.ce_masked_bwd(logits, tgt, mask), tl.grad.numpy(), rtol=1e-10,
                               atol=1e-14)


def test_ce_masked_invariants():
    # test_autograd.cpp:397-498: all-ones == plain CE; half mask == subset;
    # masked rows have zero grad; zero mask gives loss 0 in forward.
    r = rng(13)
    logits, tgt = r.standard_normal((5, 7)), r.integers(0, 7, 5)
    ones = np.ones(5)
    plain = F.cross_entropy(t64(logits), torch.tensor(tgt)).item()
    assert O.ce_masked_fwd(logits, tgt, ones)[0] == pytest.approx(plain, rel=1e-13)
    half = np.array([1, 0, 1, 0, 1.0])
    sub = F.cross_entropy(t64(logits[::2]), torch.tensor(tgt[::2])).item()
    assert O.ce_masked_fwd(logits, tgt, half)[0] == pytest.approx(sub, rel=1e-13)
    d = O.ce_masked_bwd(logits, tgt, half)
    assert (d[1] == 0).all() and (d[3] == 0).all()
    assert O.ce_masked_fwd(logits, tgt, np.zeros(5))[0] == 0.0


# ------------------------------------------------------------ Embedding
def test_embedding_kat_and_bwd():
    # tests/test_embedding.cpp:11-31
    w = np.array([[v * 10 + h for h in range(5)] for v in range(7)], dtype=np.float64)
    ids = np.array([[3, 0], [6, 3]])
    got = O.embedding_fwd(ids, w)
    np.testing.assert_array_equal(got.reshape(4, 5), [[i * 10 + h for h in range(5)] for i in [3, 0, 6, 3]])
    dy = rng(14).standard_normal((4, 5))
    ref = np.zeros((7, 5))
    np.add.at(ref, ids.reshape(-1), dy)
    np.testing.assert_allclose(O.embedding_bwd(ids, dy, 7), ref, rtol=1e-14)


# ---------------------------------------------------------------- AdamW
def test_adamw_single_element_kat():
    # tests/test_autograd.cpp:530-573 (two steps, b2 0.999, lr 0.01)
    p0, g, lr, b1, b2, eps = 1.0, 0.1, 0.01, 0.9, 0.999, 1e-8
    p, m, v = np.array([p0]), np.zeros(1), np.zeros(1)
    p, m, v = O.adamw(p, [g], m, v, lr, b1, b2, eps, 0.0, 1 - b1, 1 - b2)
    m1, v1 = (1 - b1) * g, (1 - b2) * g * g
    e1 = p0 - lr * ((m1 / (1 - b1)) / (math.sqrt(v1 / (1 - b2)) + eps))
    assert p[0] == pytest.approx(e1, abs=1e-12)
    p, m, v = O.adamw(p, [g], m, v, lr, b1, b2, eps, 0.0, 1 - b1 ** 2, 1 - b2 ** 2)
    m2, v2 = b1 * m1 + (1 - b1) * g, b2 * v1 + (1 - b2) * g * g
    e2 = e1 - lr * ((m2 / (1 - b1 ** 2)) / (math.sqrt(v2 / (1 - b2 ** 2)) + eps))
    assert p[0] == pytest.approx(e2, abs=1e-12)


def test_adamw_decoupled_decay_kat():
    # tests/test_autograd.cpp:579-597
    p, _, _ = O.adamw([1.0], [0.0], [0.0], [0.0], 0.01, 0.9, 0.999, 1e-8, 0.1, 0.1, 0.001)
    assert p[0] == pytest.approx(1.0 - 0.01 * 0.1, abs=1e-15)


def test_adamw_vs_torch_optim():
    r = rng(15)
    p0, lr, wd = r.standard_normal(20), 1e-3, 0.1
    tp = t64(p0, True)
    opt = torch.optim.AdamW([tp], lr=lr, betas=(0.9, 0.95), eps=1e-8, weight_decay=wd)
    p, m, v = p0.copy(), np.zeros(20), np.zeros(20)
    for step in range(1, 4):
        g = r.standard_normal(20)
        tp.grad = t64(g)
        opt.step()
        p, m, v = O.adamw(p, g, m, v, lr, 0.9, 0.95, 1e-8, wd, 1 - 0.9 ** step, 1 - 0.95 ** step)
    np.testing.assert_allclose(p, tp.detach().numpy(), rtol=1e-12)
    np.testing.assert_allclose(m, opt.state[tp]["exp_avg"].numpy(), rtol=1e-12)
    np.testing.assert_allclose(v, opt.state[tp]["exp_avg_sq"].numpy(), rtol=1e-12)


# ------------------------------------------------------------ Attention
@pytest.mark.parametrize("H,Hk", [(4, 4), (6, 2)])
def test_attention_vs_torch_sdpa(H, Hk):
    r = rng(16)
    B, T, D = 2, 13, 8
    q, k, v = (r.standard_normal((B, T, h, D)) for h in (H, Hk, Hk))
    do = r.standard_normal((B, T, H, D))
    tq, tk, tv = (t64(a.transpose(0, 2, 1, 3), True) for a in (q, k, v))
    g = H // Hk
    ref = F.scaled_dot_product_attention(tq, tk.repeat_interleave(g, 1), tv.repeat_interleave(g, 1),
                                         is_causal=True)
    (ref * t64(do.transpose(0, 2, 1, 3))).sum().backward()
    o, lse = O.attention_fwd(q, k, v)
    np.testing.assert_allclose(o, ref.detach().numpy().transpose(0, 2, 1, 3), rtol=1e-10, atol=1e-12)
    s = (tq @ tk.repeat_interleave(g, 1).transpose(-1, -2)).detach() / math.sqrt(D)
    s = s.masked_fill(torch.triu(torch.ones(T, T, dtype=torch.bool), 1), -math.inf)
    np.testing.assert_allclose(lse, torch.logsumexp(s, -1).numpy(), rtol=1e-12)
    dq, dk, dv = O.attention_bwd(q, k, v, do)
    np.testing.assert_allclose(dq, tq.grad.numpy().transpose(0, 2, 1, 3), rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(dk, tk.grad.numpy().transpose(0, 2, 1, 3), rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(dv, tv.grad.numpy().transpose(0, 2, 1, 3), rtol=1e-9, atol=1e-12)


# ------------------------------------------------------ Block / Model
def tiny_cfg(qk_norm, llama3=False):
    return O.make_cfg(vocab=23, hidden=16, inter=24, layers=2, heads=4, kv_heads=2, head_dim=4,
                      eps=1e-5, theta=1e4, qk_norm=int(qk_norm),
                      rope_factor=32.0 if llama3 else 0.0, rope_orig_max_pos=16)


def block_weights(cfg, r, norm_std=0.3):
    d, I, H, Hk, D = cfg.hidden, cfg.inter, cfg.heads, cfg.kv_heads, cfg.head_dim
    w = {
        "input_layernorm": 1 + norm_std * r.standard_normal(d),
        "q_proj": 0.3 * r.standard_normal((H * D, d)),
        "k_proj": 0.3 * r.standard_normal((Hk * D, d)),
        "v_proj": 0.3 * r.standard_normal((Hk * D, d)),
        "o_proj": 0.3 * r.standard_normal((d, H * D)),
        "post_attention_layernorm": 1 + norm_std * r.standard_normal(d),
        "gate_proj": 0.3 * r.standard_normal((I, d)),
        "up_proj": 0.3 * r.standard_normal((I, d)),
        "down_proj": 0.3 * r.standard_normal((d, I)),
    }
    if cfg.qk_norm:
        w["q_norm"] = 1 + norm_std * r.standard_normal(D)
        w["k_norm"] = 1 + norm_std * r.standard_normal(D)
    return w


def _torch_block(cfg, w, x):
    """Independent composition in torch (float64) of transformer_block.h:28-35."""
    B, T, d = x.shape
    H, Hk, D = cfg.heads, cfg.kv_heads, cfg.head_dim
    h1 = F.rms_norm(x, (d,), w["input_layernorm"], eps=cfg.eps)
    q = (h1 @ w["q_proj"].T).view(B, T, H, D)
    k = (h1 @ w["k_proj"].T).view(B, T, Hk, D)
    v = (h1 @ w["v_proj"].T).view(B, T, Hk, D)
    if cfg.qk_norm:
        q = F.rms_norm(q, (D,), w["q_norm"], eps=cfg.eps)
        k = F.rms_norm(k, (D,), w["k_norm"], eps=cfg.eps)
    from tests.golden.make_golden import rope_freqs
    freqs = torch.from_numpy(rope_freqs(D, cfg.theta, cfg.rope_factor, cfg.rope_low_freq,
                                        cfg.rope_high_freq, cfg.rope_orig_max_pos))
    ang = (torch.arange(T, dtype=torch.float32)[:, None] * freqs[None, :]).double()
    cos, sin = torch.cos(ang)[None, :, None, :], torch.sin(ang)[None, :, None, :]

    def rot(z):
        a, b = z[..., : D // 2], z[..., D // 2:]
        return torch.cat([a * cos - b * sin, a * sin + b * cos], -1)
    q, k = rot(q), rot(k)
    g = H // Hk
    o = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2).repeat_interleave(g, 1),
                                       v.transpose(1, 2).repeat_interleave(g, 1), is_causal=True)
    h = x + o.transpose(1, 2).reshape(B, T, H * D) @ w["o_proj"].T
    h2 = F.rms_norm(h, (d,), w["post_attention_layernorm"], eps=cfg.eps)
    return h + (F.silu(h2 @ w["gate_proj"].T) * (h2 @ w["up_proj"].T)) @ w["down_proj"].T


@pytest.mark.parametrize("qk_norm,llama3", [(False, False), (True, False), (False, True)])
def test_block_vs_torch_and_autograd(qk_norm, llama3):
    cfg = tiny_cfg(qk_norm, llama3)
    r = rng(17)
    w = block_weights(cfg, r)
    x = r.standard_normal((2, 6, cfg.hidden))
    dy = r.standard_normal((2, 6, cfg.hidden))
    tw = {k_: t64(v_, True) for k_, v_ in w.items()}
    tx = t64(x, True)
    ty = _torch_block(cfg, tw, tx)
    (ty * t64(dy)).sum().backward()
    np.testing.assert_allclose(O.block_fwd(cfg, w, x), ty.detach().numpy(), rtol=1e-10, atol=1e-12)
    dx, dw = O.block_bwd(cfg, w, x, dy)
    np.testing.assert_allclose(dx, tx.grad.numpy(), rtol=1e-8, atol=1e-11)
    for k_ in w:
        np.testing.assert_allclose(dw[k_], tw[k_].grad.numpy(), rtol=1e-8, atol=1e-11, err_msg=k_)


def test_block_bwd_finite_difference():
    cfg = tiny_cfg(True)
    r = rng(18)
    w = block_weights(cfg, r)
    x = r.standard_normal((1, 5, cfg.hidden))
    dy = r.standard_normal((1, 5, cfg.hidden))
    dx, dw = O.block_bwd(cfg, w, x, dy)
    f = lambda xx: float((O.block_fwd(cfg, w, xx) * dy).sum())  # noqa: E731
    idx = list(range(0, x.size, 7))
    fd = fd_grad(f, x, idx=idx)
    np.testing.assert_allclose([dx.reshape(-1)[i] for i in idx], [fd[i] for i in idx], rtol=1e-5, atol=1e-8)
    for key in ["q_norm", "k_proj", "down_proj"]:
        def fw(a, key=key):
            ww = dict(w)
            ww[key] = a
            return float((O.block_fwd(cfg, ww, x) * dy).sum())
        idx = list(range(0, w[key].size, max(1, w[key].size // 9)))
        fd = fd_grad(fw, w[key], idx=idx)
        np.testing.assert_allclose([dw[key].reshape(-1)[i] for i in idx], [fd[i] for i in idx],
                                   rtol=1e-5, atol=1e-8, err_msg=key)


def model_params(cfg, r):
    ps = [0.5 * r.standard_normal((cfg.vocab, cfg.hidden))]
    for _ in range(cfg.layers):
        w = block_weights(cfg, r)
        for key in O.BLOCK_KEYS:
            if key in w:
                ps.append(w[key])
    ps.append(1 + 0.3 * r.standard_normal(cfg.hidden))
    return ps


def test_model_loss_finite_difference_and_tied_head():
    cfg = tiny_cfg(True)
    r = rng(19)
    ps = model_params(cfg, r)
    B, T = 2, 5
    ids = r.integers(0, cfg.vocab, (B, T))
    tg = r.integers(0, cfg.vocab, (B, T))
    mask = np.array([[0, 0, 1, 1, 1], [0, 1, 1, 1, 1]], dtype=np.float64)
    loss, grads = O.model_loss(cfg, ps, ids, tg, mask)
    assert np.isfinite(loss)
    for pi in [0, 1, 6, 7, len(ps) - 1]:
        def f(a, pi=pi):
            qq = list(ps)
            qq[pi] = a
            return O.model_loss(cfg, qq, ids, tg, mask, want_grads=False)[0]
        idx = list(range(0, ps[pi].size, max(1, ps[pi].size // 11)))
        fd = fd_grad(f, ps[pi], idx=idx)
        np.testing.assert_allclose([grads[pi].reshape(-1)[i] for i in idx], [fd[i] for i in idx],
                                   rtol=1e-5, atol=1e-9, err_msg=f"param {pi}")


# ------------------------------------------------ Inference (KV cache) oracle
@pytest.mark.parametrize("H,Hk,T,L,pos", [(4, 4, 3, 12, 9), (6, 2, 5, 12, 7), (6, 3, 1, 9, 8),
                                          (4, 2, 4, 4, 0), (2, 1, 3, 6, 40)])
def test_attention_offset_vs_torch_sdpa_masked(H, Hk, T, L, pos):
    """Query t sees keys j <= pos + t: torch SDPA with that explicit boolean mask."""
    r = rng(31)
    B, D = 2, 8
    q = r.standard_normal((B, T, H, D))
    k, v = (r.standard_normal((B, L, Hk, D)) for _ in range(2))
    g = H // Hk
    allow = torch.tensor([[j <= pos + t for j in range(L)] for t in range(T)])
    ref = F.scaled_dot_product_attention(t64(q.transpose(0, 2, 1, 3)),
                                         t64(k.transpose(0, 2, 1, 3)).repeat_interleave(g, 1),
                                         t64(v.transpose(0, 2, 1, 3)).repeat_interleave(g, 1),
                                         attn_mask=allow)
    o = O.attention_offset(q, k, v, pos)
    np.testing.assert_allclose(o, ref.numpy().transpose(0, 2, 1, 3), rtol=1e-10, atol=1e-12)
    if pos == 0 and L == T:  # plain causal attention: the training oracle
        np.testing.assert_allclose(o, O.attention_fwd(q, k, v)[0], rtol=1e-12, atol=1e-14)


def test_model_logits_composition_and_loss():
    """Logits = embedding -> blocks -> final RMSNorm -> h E^T (each piece pinned above),
    and their masked CE is the model loss."""
    cfg = tiny_cfg(True, llama3=True)
    r = rng(32)
    ps = model_params(cfg, r)
    B, T = 2, 6
    ids = r.integers(0, cfg.vocab, (B, T))
    logits = O.model_logits(cfg, ps, ids)
    h = O.embedding_fwd(ids.reshape(-1), ps[0]).reshape(B, T, -1)
    keys = [k_ for k_ in O.BLOCK_KEYS if cfg.qk_norm or k_ not in ("q_norm", "k_norm")]
    for l in range(cfg.layers):
        w = dict(zip(keys, ps[1 + l * len(keys): 1 + (l + 1) * len(keys)]))
        h = O.block_fwd(cfg, w, h)
    hn = O.rmsnorm_fwd(h.reshape(B * T, -1), ps[-1], cfg.eps)
    np.testing.assert_allclose(logits.reshape(B * T, -1), hn @ ps[0].T, rtol=1e-12, atol=1e-12)
    tg = r.integers(0, cfg.vocab, (B, T))
    mask = np.ones((B, T))
    lse = np.log(np.exp(logits).sum(-1))
    ce = float(np.mean(lse - np.take_along_axis(logits, tg[..., None], -1)[..., 0]))
    assert math.isclose(ce, O.model_loss(cfg, ps, ids, tg, mask, want_grads=False)[0],
                        rel_tol=1e-12)
