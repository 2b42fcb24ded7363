"""The training quotas divide by a per-side constant (the weight sum, the
spare count) through its rounded reciprocal: q0 = RN(x * yr), r = x - q0 * y
(exact with an FMA), q = RN(q0 + r * yr) with yr = RN(1 / y) (Markstein's
theorem).  The GPU path relies on q being the correctly rounded x / y --
the reference's division -- in the ranges the quotas use; this checks that
identity on the CPU with exact rational arithmetic, on random operands of
both divisions and on quotients placed at and around halfway points."""
import math
import random
import struct
from fractions import Fraction as F


def _fma(a, b, c):
    return float(F(a) * F(b) + F(c))


def _div_r(x, y):
    yr = 1.0 / y
    q0 = x * yr
    r = _fma(-q0, y, x)
    return _fma(r, yr, q0)


def _f32(v):
    return struct.unpack("f", struct.pack("f", v))[0]


def test_quota_base_division():
    rng = random.Random(11)
    for it in range(20000):
        target = rng.choice([1, 2, 3, 200, 400, rng.randint(1, 2 ** 31 - 1)])
        w = _f32(rng.random() ** rng.choice([1, 3, 8]))
        if w == 0.0:
            continue
        x = float(target) * w
        y = rng.uniform(1e-3, 2000.0) if it % 3 else sum(_f32(rng.random()) for _ in range(rng.randint(1, 40)))
        assert _div_r(x, y) == x / y, (x, y)


def test_quota_cum_division():
    rng = random.Random(12)
    for it in range(20000):
        res = rng.randint(0, 2 ** 31 - 1) if it % 2 else rng.randint(0, 500)
        spare = rng.randint(1, 2 ** 31 - 1) if it % 3 else rng.randint(1, 5000)
        p = rng.randint(0, spare)
        x, y = float(res) * float(p), float(spare)
        assert _div_r(x, y) == x / y, (x, y)


def test_halfway_quotients():
    rng = random.Random(13)
    for _ in range(20000):
        y = rng.uniform(1.0, 2.0) * 2.0 ** rng.randint(-20, 12)
        q = rng.uniform(1.0, 2.0) * 2.0 ** rng.randint(-30, 31)
        ulp = math.ulp(q)
        near = F(q) + F(ulp) / 2 * rng.choice([1, 0, -1]) + F(rng.randint(-3, 3)) * F(ulp) / 1024
        x = float(near * F(y))
        assert _div_r(x, y) == x / y, (x, y)


def test_plain_product_is_not_enough():
    """The correction step matters: RN(x * yr) alone misses the correctly
    rounded quotient on some of these operands."""
    rng = random.Random(14)
    misses = 0
    for _ in range(20000):
        y = rng.uniform(1.0, 2.0) * 2.0 ** rng.randint(-20, 12)
        x = rng.uniform(1.0, 2.0) * 2.0 ** rng.randint(-30, 31)
        misses += (x * (1.0 / y)) != x / y
    assert misses > 0
