"""The parity comparison itself (CPU): NaN-strict, infinity-aware."""

import numpy as np

from tests import _helpers as H


def test_max_abs_catches_a_planted_nan():
    exp = np.linspace(-1, 1, 64, dtype=np.float32).reshape(8, 8)
    got = exp.copy()
    assert H.max_abs(got, exp) == 0.0
    got[3, 5] = np.nan  # one GPU row partly NaN where the oracle is finite
    assert H.max_abs(got, exp) == float("inf")
    assert not H.max_abs(got, exp) <= 2e-2
    # and the other way round: the oracle NaN, the GPU finite
    assert H.max_abs(exp, got) == float("inf")


def test_max_abs_matching_nan_and_inf():
    exp = np.array([[np.nan, 1.0], [np.inf, -np.inf]])
    got = np.array([[np.nan, 1.0 + 1e-3], [np.inf, -np.inf]])
    assert abs(H.max_abs(got, exp) - 1e-3) < 1e-12
    got[1, 0] = 1e30  # finite where an infinity is expected
    assert H.max_abs(got, exp) == float("inf")
    assert H.max_abs(np.full(4, np.nan), np.full(4, np.nan)) == 0.0
    assert H.max_abs(np.empty((0, 3)), np.empty((0, 3))) == 0.0


def test_max_abs_broadcasts_like_subtraction():
    assert H.max_abs(np.zeros((2, 3)), np.array([0.0, 0.5, 0.0])) == 0.5
