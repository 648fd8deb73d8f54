"""The softmax of the HIP router sums the fp32 exponentials with a wave tree
instead of one lane in expert order when every term is 0 or in [2^-22, 1]
(and E <= 256): then every partial sum is exact in binary64, so the two orders
give the same value.  These tests pin that fact, and that the bound matters."""
import math

import numpy as np
import pytest


def _sequential(terms):
    s = 0.0
    for t in terms:
        s = s + float(t)
    return s


def _tree(terms):
    # pairwise, the shape of a wave reduction
    v = [float(t) for t in terms]
    while len(v) > 1:
        if len(v) % 2:
            v.append(0.0)
        v = [v[i] + v[i + 1] for i in range(0, len(v), 2)]
    return v[0]


@pytest.mark.parametrize("E", [8, 65, 128, 200, 256])
def test_terms_in_range_sum_exactly_in_any_order(E):
    rng = np.random.default_rng(E)
    for trial in range(40):
        # exponents from 2^-22 up to 1, mantissas random, some exact zeros
        terms = (rng.uniform(1.0, 2.0, E) * np.exp2(rng.integers(-22, 0, E))).astype(np.float32)
        terms = np.minimum(terms, np.float32(1.0))
        terms[rng.random(E) < 0.1] = 0.0
        assert ((terms == 0) | ((terms >= 2.0 ** -22) & (terms <= 1))).all()
        exact = math.fsum(float(t) for t in terms)
        assert _sequential(terms) == exact
        assert _tree(terms) == exact
        for _ in range(3):
            assert _sequential(rng.permutation(terms)) == exact


def test_extremes_of_the_range():
    ones = np.ones(256, np.float32)
    assert _sequential(ones) == _tree(ones) == 256.0
    mixed = np.array([1.0] * 255 + [2.0 ** -22], np.float32)
    assert _sequential(mixed) == _tree(mixed) == math.fsum(mixed.astype(np.float64))


def test_terms_below_the_bound_can_depend_on_order():
    # 1 + 128 * 2^-54: one lane in order rounds every small term away, a tree
    # adds them first (2^-47) and keeps them
    terms = np.array([1.0] + [2.0 ** -54] * 128, np.float32)
    assert _sequential(terms) == 1.0
    assert _tree(terms[::-1]) == 1.0 + 2.0 ** -47
