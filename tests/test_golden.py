"""The CPU oracle against the golden fixtures in tests/golden: expected outputs
of an independent float64 torch composition of the reference's block
(tests/golden/make_golden.py), frozen in files, at BASELINE config 0's full
size (one SmolLM2-135M-shaped block, B=1, T=256).  The fixture files are also
checked against what the generator writes for them.  Nothing here touches the
GPU; the GPU tests compare the HIP path with the same fixtures.
"""
import os

import numpy as np

import oracle as O
from tests.golden import make_golden as MG
from tests.helpers import assert_matches_golden

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


def c1_cfg():
    c = MG.C1
    return O.make_cfg(vocab=256, hidden=c["hidden"], inter=c["inter"], layers=1, heads=c["heads"],
                      kv_heads=c["kv_heads"], head_dim=c["head_dim"], eps=c["eps"],
                      theta=c["theta"])


def test_oracle_c1_block_vs_golden():
    g = load("c1_block.npz")
    w, x, dy = MG.c1_inputs()
    cfg = c1_cfg()
    y = O.block_fwd(cfg, w, x)
    dx, dw = O.block_bwd(cfg, w, x, dy)
    # Both sides are float64; they differ only where float32 RoPE angles may round
    # apart by an ulp, so the bound is far below the HIP path's 1e-4.
    assert_matches_golden(g, "y", y, rtol=1e-6, rows=True)
    assert_matches_golden(g, "dx", dx, rtol=1e-6, rows=True)
    for k in MG.BLOCK_KEYS:
        assert_matches_golden(g, "d_" + k, dw[k], rtol=1e-6)


def test_golden_inputs_are_stable():
    # The legacy RandomState stream the fixtures' inputs come from: its first
    # draws for seed 0 are fixed (numpy keeps that generator frozen).
    r = np.random.RandomState(0)
    np.testing.assert_allclose(r.standard_normal(3), [1.764052345967664, 0.4001572083672233,
                                                      0.9787379841057392], rtol=0, atol=0)
    w, x, _ = MG.c1_inputs()
    assert w["input_layernorm"][0] == 0.02 * 1.764052345967664
    assert x.shape == (1, 256, 576)
