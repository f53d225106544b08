"""The kernels divide by launch-time constants with the round-up multiply
method (na_common.h make_fastdiv / fdiv): q = (mulhi(n, mul) + n) >> shift.
This checks that formula against exact division for every divisor the
kernels can see up to 5000 and large ones, on boundary and random n < 2^31."""

import random


def make_fastdiv(d):
    l = 0
    while (1 << l) < d:
        l += 1
    mul = ((1 << 32) * ((1 << l) - d)) // d + 1
    assert 0 <= mul < (1 << 32)
    return mul, l


def fdiv(n, mul, shift):
    t = (n * mul) >> 32
    s = t + n
    assert s < (1 << 32)
    return s >> shift


def test_fastdiv_exact():
    rng = random.Random(0)
    divisors = list(range(1, 5001)) + [rng.randrange(1, 1 << 31) for _ in range(2000)] + \
        [(1 << 31) - 1, 1 << 30, (1 << 30) + 1]
    for d in divisors:
        mul, sh = make_fastdiv(d)
        ns = [0, 1, d - 1, d, d + 1, 2 * d - 1, 2 * d, (1 << 31) - 1, (1 << 31) - d]
        ns += [rng.randrange(0, 1 << 31) for _ in range(40)]
        ns += [k * d + r for k in (3, 1000, (1 << 31) // d - 1) for r in (0, d - 1) if k * d + r < (1 << 31)]
        for n in ns:
            if 0 <= n < (1 << 31):
                assert fdiv(n, mul, sh) == n // d, (n, d)
