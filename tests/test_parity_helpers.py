# SPDX-License-Identifier: Apache-2.0
"""The comparison rules of tests/parity.py, checked on the CPU: results equal to
the oracle's pass; a near-tie swap passes and is counted; a swap far from the
cut, a distance off by more than the tolerance, or a floor taken from another
row's norm fails."""
import numpy as np
import pytest

import oracle
import parity


def _case():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((500, 16)).astype(np.float32)
    q = rng.standard_normal((6, 16)).astype(np.float32)
    oi, od = oracle.flat_search(x, q, 10)
    return x, q, oi, od


def test_identical_results_pass_with_no_swaps():
    x, q, oi, od = _case()
    assert parity.tolerant(oi.copy(), od.copy(), oi, od, x, q, 0) == 0


def test_near_tie_swap_is_accepted_and_counted():
    x, q, oi, od = _case()
    # a row at exactly the k-th row's distance (a duplicate of it) replaces it
    x2 = np.vstack([x, x[oi[0, 9]][None]])
    dup = x2.shape[0] - 1
    gi, gd = oi.copy(), od.copy()
    gi[0, 9] = dup
    assert parity.tolerant(gi, gd, oi, od, x2, q, 0) == 1


def test_far_swap_is_rejected():
    x, q, oi, od = _case()
    far = int(np.argmax(np.sum((x - q[0]) ** 2, axis=1)))
    gi = oi.copy()
    gi[0, 9] = far
    with pytest.raises(AssertionError):
        parity.tolerant(gi, od.copy(), oi, od, x, q, 0)


def test_distance_error_is_rejected():
    x, q, oi, od = _case()
    gd = od.copy()
    gd[2, 3] *= 1.0 + 1e-3
    with pytest.raises(AssertionError):
        parity.tolerant(oi.copy(), gd, oi, od, x, q, 0)


def test_l2_floor_uses_the_pairs_own_norm():
    """One far row of huge norm must not loosen the floor of every other pair:
    an error of 2^-20 * ||x_far||^2 on a small distance is caught."""
    rng = np.random.default_rng(8)
    x = rng.standard_normal((200, 8)).astype(np.float32)
    x[150] = 1e4   # ||x||^2 = 8e8, never among the results
    q = rng.standard_normal((3, 8)).astype(np.float32)
    oi, od = oracle.flat_search(x, q, 5)
    assert not np.any(oi == 150)
    gd = od.copy()
    gd[1, 0] += np.float32(2.0 ** -20 * 8e8 * 0.5)   # within a database-wide floor, far outside the pair's
    with pytest.raises(AssertionError):
        parity.tolerant(oi.copy(), gd, oi, od, x, q, 0)
