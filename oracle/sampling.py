"""CPU restatement of token sampling -- TEST INFRASTRUCTURE ONLY.

Follows the reference's src/core/sampling.cpp:10-113 (argmax_cpu, softmax_inplace,
sample_one_row) and the random stream it draws from: std::mt19937_64 (the C++
standard's 64-bit Mersenne Twister, [rand.predef]) seeded with the request seed,
and std::uniform_real_distribution<double>(0, 1), which in libstdc++ is
generate_canonical<double, 53>: one 64-bit engine output x, u = double(x) / 2^64,
clamped below 1.  Only tests import this module.
"""
from __future__ import annotations

import numpy as np

F32 = np.float32
_MASK64 = (1 << 64) - 1


class MT19937_64:
    """std::mt19937_64: w=64, n=312, m=156, r=31, a=0xB5026F5AA96619E9,
    u=29 d=0x5555555555555555, s=17 b=0x71D67FFFEDA60000, t=37
    c=0xFFF7EEE000000000, l=43, f=6364136223846793005."""

    N, M = 312, 156

    def __init__(self, seed=5489):
        mt = [0] * self.N
        mt[0] = seed & _MASK64
        for i in range(1, self.N):
            mt[i] = (6364136223846793005 * (mt[i - 1] ^ (mt[i - 1] >> 62)) + i) & _MASK64
        self.mt, self.i = mt, self.N

    def _twist(self):
        mt, N, M = self.mt, self.N, self.M
        upper, lower = 0xFFFFFFFF80000000, 0x7FFFFFFF
        for k in range(N):
            y = (mt[k] & upper) | (mt[(k + 1) % N] & lower)
            mt[k] = mt[(k + M) % N] ^ (y >> 1) ^ (0xB5026F5AA96619E9 if y & 1 else 0)
        self.i = 0

    def __call__(self):
        if self.i >= self.N:
            self._twist()
        y = self.mt[self.i]
        self.i += 1
        y ^= (y >> 29) & 0x5555555555555555
        y ^= (y << 17) & 0x71D67FFFEDA60000
        y ^= (y << 37) & 0xFFF7EEE000000000
        y ^= y >> 43
        return y & _MASK64


def uniform01(rng: MT19937_64) -> float:
    """uniform_real_distribution<double>(0, 1)(rng) as libstdc++ computes it."""
    u = float(rng()) / 18446744073709551616.0
    return np.nextafter(1.0, 0.0) if u >= 1.0 else u


def argmax(row) -> int:
    """argmax_cpu (sampling.cpp:12-19): first index whose value exceeds every earlier one."""
    best = 0
    for i in range(1, len(row)):
        if row[i] > row[best]:
            best = i
    return best


def _exp32(x):
    """float exp(x), correctly rounded (through double)."""
    return np.exp(np.asarray(x, np.float64)).astype(F32)


def probabilities(row, temperature, top_k=0, top_p=0.0):
    """The distribution sample_one_row draws from (sampling.cpp:31-85), float32."""
    z = np.asarray(row, F32) * (F32(1.0) / F32(temperature))
    V = z.size
    if 0 < top_k < V:
        thresh = np.sort(z)[::-1][top_k - 1]           # the k-th largest value
        z = np.where(z < thresh, F32(-np.inf), z).astype(F32)
    z = _exp32(z - z.max())
    total = 0.0
    for x in z:                                         # double sum in index order
        total += float(x)
    z = (z * F32(1.0 / total)).astype(F32)
    top_p = float(F32(top_p))                           # the request's float, widened
    if 0.0 < top_p < 1.0:
        # Descending probability; ties keep index order here, while the reference's
        # std::sort leaves their order unspecified (a tie straddling the cut-off is
        # the one case this restatement does not fix).
        order = sorted(range(V), key=lambda i: -float(z[i]))
        keep = np.zeros(V, bool)
        cum = 0.0
        for i in order:
            cum += float(z[i])
            keep[i] = True
            if cum >= top_p:
                break
        z = np.where(keep, z, F32(0.0)).astype(F32)
        total = 0.0
        for x in z:
            total += float(x)
        if total > 0.0:
            z = (z * F32(1.0 / total)).astype(F32)
    return z


def sample_row(row, rng: MT19937_64, temperature=1.0, top_k=0, top_p=0.0) -> int:
    """One token from one row: argmax when temperature <= 0, else one uniform draw
    walking the double CDF in index order (sampling.cpp:31-99)."""
    if temperature <= 0.0:
        return argmax(row)
    p = probabilities(row, temperature, top_k, top_p)
    u = uniform01(rng)
    c = 0.0
    for i, x in enumerate(p):
        c += float(x)
        if u < c:
            return i
    return len(p) - 1
