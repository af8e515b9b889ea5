"""The scalar fp32 restatement of the reference's CPU test ops
(oracle/ref_f32.c), which bench.py times as the CPU baseline, computes the same
block, LM head and AdamW as the float64 oracle (pinned in test_oracle.py):
fp32 against fp64 within 1e-4 relative, checkpointing on equal to off bit for
bit, and its unit-test ops against the reference tests' known answers."""
import numpy as np
import pytest

import oracle as O
from oracle import ref_f32 as RF
from tests.helpers import assert_close


def cfgs(qk_norm):
    rc = RF.BlockCfg(d=48, H=4, Hk=2, Dh=16, I=64, eps=1e-5, theta=1e4)
    oc = O.make_cfg(vocab=32, hidden=48, inter=64, layers=1, heads=4, kv_heads=2, head_dim=16,
                    eps=float(np.float32(1e-5)), theta=1e4, qk_norm=int(qk_norm))
    return rc, oc


def weights(r, qk_norm):
    d, I, H, Hk, D = 48, 64, 4, 2, 16
    w = {"input_layernorm": 1 + 0.1 * r.standard_normal(d),
         "q_proj": 0.2 * r.standard_normal((H * D, d)), "k_proj": 0.2 * r.standard_normal((Hk * D, d)),
         "v_proj": 0.2 * r.standard_normal((Hk * D, d)), "o_proj": 0.2 * r.standard_normal((d, H * D)),
         "post_attention_layernorm": 1 + 0.1 * r.standard_normal(d),
         "gate_proj": 0.2 * r.standard_normal((I, d)), "up_proj": 0.2 * r.standard_normal((I, d)),
         "down_proj": 0.2 * r.standard_normal((d, I))}
    if qk_norm:
        w["q_norm"] = 1 + 0.1 * r.standard_normal(D)
        w["k_norm"] = 1 + 0.1 * r.standard_normal(D)
    return {k: v.astype(np.float32) for k, v in w.items()}


@pytest.mark.parametrize("qk_norm", [False, True])
def test_block_matches_oracle_and_checkpoint_is_bitwise(qk_norm):
    r = np.random.default_rng(3)
    rc, oc = cfgs(qk_norm)
    w = weights(r, qk_norm)
    T = 40
    x = r.standard_normal((T, 48)).astype(np.float32)
    dy = r.standard_normal((T, 48)).astype(np.float32)
    y, dx, g = RF.block_fwd_bwd(rc, w, x, dy, checkpoint=False)
    y2, dx2, g2 = RF.block_fwd_bwd(rc, w, x, dy, checkpoint=True)
    assert np.array_equal(y, y2) and np.array_equal(dx, dx2)
    assert all(np.array_equal(g[k], g2[k]) for k in g)
    wd = {k: v.astype(np.float64) for k, v in w.items()}
    x3, dy3 = x[None].astype(np.float64), dy[None].astype(np.float64)
    assert_close(y, O.block_fwd(oc, wd, x3)[0], name="y")
    dx_ref, dw_ref = O.block_bwd(oc, wd, x3, dy3)
    assert_close(dx, dx_ref[0], name="dx")
    for k in w:
        assert_close(g[k], dw_ref[k], name=k)


def test_attention_head_matches_oracle():
    r = np.random.default_rng(5)
    T, D = 33, 16
    q, k, v, do = (r.standard_normal((T, D)).astype(np.float32) for _ in range(4))
    o, dq, dk, dv = RF.attention_head(q, k, v, do)
    sh = lambda a: a.astype(np.float64).reshape(1, T, 1, D)  # noqa: E731
    o_ref, _ = O.attention_fwd(sh(q), sh(k), sh(v))
    dq_ref, dk_ref, dv_ref = O.attention_bwd(sh(q), sh(k), sh(v), sh(do))
    for got, ref, name in ((o, o_ref, "o"), (dq, dq_ref, "dq"), (dk, dk_ref, "dk"),
                           (dv, dv_ref, "dv")):
        assert_close(got, ref.reshape(T, D), name=name)


def test_lm_head_ce_and_adamw_match_oracle():
    r = np.random.default_rng(4)
    n, d, V = 12, 32, 50
    h = r.standard_normal((n, d)).astype(np.float32)
    E = (0.3 * r.standard_normal((V, d))).astype(np.float32)
    tgt = r.integers(0, V, n)
    mask = (r.random(n) > 0.3).astype(np.float32)
    loss, dh, dE = RF.lm_head_ce(h, E, tgt, mask)
    logits = h.astype(np.float64) @ E.T.astype(np.float64)
    assert loss == pytest.approx(O.ce_masked_fwd(logits, tgt, mask)[0], rel=1e-5)
    dl = O.ce_masked_bwd(logits, tgt, mask)
    assert_close(dh, dl @ E.astype(np.float64), name="dh")
    assert_close(dE, dl.T @ h.astype(np.float64), name="dE")
    # AdamW, two steps against the oracle's element formula (bias corrections in float)
    p = r.standard_normal(1000).astype(np.float32)
    g1, g2 = r.standard_normal(1000).astype(np.float32), r.standard_normal(1000).astype(np.float32)
    m, v = np.zeros(1000, np.float32), np.zeros(1000, np.float32)
    rp, rm, rv = p.astype(np.float64), np.zeros(1000), np.zeros(1000)
    for step, g in ((1, g1), (2, g2)):
        RF.adamw(p, g, m, v, 1e-3, 0.9, 0.95, 1e-8, 0.1, step)
        bc1 = np.float32(1 - np.float32(0.9) ** step)
        bc2 = np.float32(1 - np.float32(0.95) ** step)
        rp, rm, rv = O.adamw(rp, g, rm, rv, np.float32(1e-3), np.float32(0.9), np.float32(0.95),
                             np.float32(1e-8), np.float32(0.1), bc1, bc2)
    for got, ref in ((p, rp), (m, rm), (v, rv)):
        assert np.all(np.abs(got - ref) <= 1e-5 * np.abs(ref) + 1e-6 * np.abs(ref).max())


def test_unit_ops_known_answers():
    # Matmul.NonSquare (reference tests/test_matmul.cpp:48-67)
    a = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    b = np.arange(1, 13, dtype=np.float32).reshape(3, 4)
    c = np.empty((2, 4), np.float32)
    RF.lib().rf_mm(RF._p(a), RF._p(b), RF._p(c), 2, 3, 4, 0, 0)
    assert c.tolist() == [[38, 44, 50, 56], [83, 98, 113, 128]]
    # Rope.RespectsPositionOffset: x = 1..8, pos 7, theta 1e4 (tests/test_rope.cpp:57-72)
    x = np.arange(1, 9, dtype=np.float32)
    RF.lib().rf_rope(RF._p(x), 1, 1, 1, 8, 7, RF.C.c_float(1e4))
    np.testing.assert_allclose(x, O.rope(np.arange(1, 9, dtype=np.float64).reshape(1, 1, 1, 8),
                                         1e4, pos0=7).reshape(-1), atol=1e-4)
    # Softmax.ExtremeValuesStable (tests/test_softmax.cpp:54-65)
    s = np.array([1000, 1001, 999], np.float32)
    y = np.empty(3, np.float32)
    RF.lib().rf_softmax(RF._p(s), RF._p(y), 1, 3)
    assert abs(y.sum() - 1) < 1e-6 and y[1] > y[0] > y[2]
