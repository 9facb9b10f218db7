"""std::mt19937_64 and libstdc++'s uniform_real_distribution<double>(0, 1)
first draw, written from the published MT19937-64 parameters (Matsumoto &
Nishimura) for the sampling tests.  Pinned by the C++ standard's required
10000th output of a default-seeded engine (tests/test_mt64.py)."""
from __future__ import annotations

_M = (1 << 64) - 1


class MT64:
    N, MM = 312, 156
    A = 0xB5026F5AA96619E9
    UPPER, LOWER = 0xFFFFFFFF80000000, 0x7FFFFFFF

    def __init__(self, seed: int = 5489):
        self.mt = [seed & _M]
        for i in range(1, self.N):
            p = self.mt[-1]
            self.mt.append((6364136223846793005 * (p ^ (p >> 62)) + i) & _M)
        self.i = self.N

    def _twist(self):
        mt = self.mt
        for k in range(self.N):
            y = (mt[k] & self.UPPER) | (mt[(k + 1) % self.N] & self.LOWER)
            mt[k] = mt[(k + self.MM) % self.N] ^ (y >> 1) ^ (self.A if y & 1 else 0)
        self.i = 0

    def __call__(self) -> int:
        if self.i >= self.N:
            self._twist()
        y = self.mt[self.i]
        self.i += 1
        y ^= (y >> 29) & 0x5555555555555555
        y ^= (y << 17) & 0x71D67FFFEDA60000
        y ^= (y << 37) & 0xFFF7EEE000000000
        y ^= y >> 43
        return y & _M


def first_uniform(seed: int) -> float:
    """generate_canonical<double, 53> over a 64-bit engine: one draw / 2^64."""
    u = float(MT64(seed)()) / 18446744073709551616.0
    return u if u < 1.0 else 0.9999999999999999
