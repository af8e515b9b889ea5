"""Known answers for the test helpers that GPU tests compare against."""
import numpy as np

from tests.helpers import fma_f32

F = np.float32


def test_fma_f32_rounds_once_above_a_midpoint():
    # a*b = -2^-24 + 2^-70, c = 1 + 2^-23: the exact sum 1 + 2^-24 + 2^-70 lies
    # just above the midpoint between 1 and 1 + 2^-23, so one rounding gives
    # 1 + 2^-23; float64 first rounds it onto the midpoint, and ties-to-even
    # would then give 1.
    a = np.array([2.0 ** -12 * (1 + 2.0 ** -23)], F)
    b = np.array([-(2.0 ** -12) * (1 - 2.0 ** -23)], F)
    c = np.array([1 + 2.0 ** -23], F)
    assert (a.astype(np.float64) * b + c).astype(F)[0] == F(1.0)   # rounded twice
    assert fma_f32(a, b, c)[0] == F(1 + 2.0 ** -23)


def test_fma_f32_rounds_once_below_a_midpoint():
    # a*b = 2^-24 - 2^-70, c = 1 + 2^-23: the exact sum lies just below the
    # midpoint between 1 + 2^-23 and 1 + 2^-22; rounding twice would reach the
    # even neighbour 1 + 2^-22.
    a = np.array([2.0 ** -12 * (1 + 2.0 ** -23)], F)
    b = np.array([2.0 ** -12 * (1 - 2.0 ** -23)], F)
    c = np.array([1 + 2.0 ** -23], F)
    assert (a.astype(np.float64) * b + c).astype(F)[0] == F(1 + 2.0 ** -22)
    assert fma_f32(a, b, c)[0] == F(1 + 2.0 ** -23)


def test_fma_f32_ordinary_values():
    r = np.random.default_rng(0)
    a, b, c = (r.standard_normal(10000).astype(F) for _ in range(3))
    want = np.array([F(np.float64(x) * np.float64(y) + np.float64(z))
                     for x, y, z in zip(a, b, c)], F)
    got = fma_f32(a, b, c)
    # equal except where float64 rounding landed on a float32 midpoint
    assert (got == want).mean() > 0.999
    assert np.all(np.abs(got.astype(np.float64) - want) <= np.spacing(np.abs(want)))
