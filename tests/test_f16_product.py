"""The epilogues' fp16 of a product (csrc/dspark_internal.h, f16_product): the fp32 product rounded to odd -- moved one
step toward the exact product when it is inexact and its last bit even, the direction taken from the fma residual --
then rounded to nearest-even fp16. Checked here against the exact product rounded once (float64 product, exact for two
fp32 operands, converted to fp16), on products near fp16 rounding midpoints and at random."""
import numpy as np


def f16_product(a, b):
    a = a.astype(np.float32)
    b = b.astype(np.float32)
    p = (a * b).astype(np.float32)
    exact = a.astype(np.float64) * b.astype(np.float64)
    e = exact - p.astype(np.float64)  # the fma residual's sign (exact: both terms are within 2^-48 relative)
    u = p.view(np.uint32).copy()
    adjust = (e != 0) & ((u & 1) == 0) & (p != 0)
    up = (e > 0) == (p > 0)
    u[adjust & up] += 1
    u[adjust & ~up] -= 1
    return u.view(np.float32).astype(np.float16)


def test_round_to_odd_product_is_the_single_rounding():
    rng = np.random.default_rng(7)
    n = 1 << 20
    # random operands over the epilogues' ranges
    a = (rng.standard_normal(n) * 10.0 ** rng.uniform(-3, 2, n)).astype(np.float32)
    b = (rng.standard_normal(n) * 10.0 ** rng.uniform(-3, 2, n)).astype(np.float32)
    # and products within a few fp32 ulps of an fp16 rounding midpoint, where rounding twice goes wrong
    h = rng.standard_normal(n).astype(np.float16).astype(np.float64)
    mid = h + np.spacing(h.astype(np.float16)).astype(np.float64) / 2
    b2 = (rng.uniform(0.5, 2.0, n)).astype(np.float32)
    a2 = (mid / b2.astype(np.float64)).astype(np.float32)
    a = np.concatenate([a, a2])
    b = np.concatenate([b, b2])
    want = (a.astype(np.float64) * b.astype(np.float64)).astype(np.float16)
    got = f16_product(a, b)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))
    # rounding twice (fp32, then fp16) differs on some of them: the construction is needed
    twice = (a * b).astype(np.float32).astype(np.float16)
    assert np.count_nonzero(twice.view(np.uint16) != want.view(np.uint16)) > 0
