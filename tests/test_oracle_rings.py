"""Pins of the oracle's closed-ring -> Hermite conversion
(ops/cubic_splatting.py:81-543) by mathematics: continuity and closure of
the ring, exact reproduction of Bezier branches of degree <= 3, end points
and end tangents for higher degrees (evaluated by de Casteljau, independent
of the basis tables), and the adjoint identity of forward and backward."""
import numpy as np
import pytest

from oracle import oracle as O


def _bezier(pts, t):
    """Point and derivative of the Bezier curve `pts` [kb, 2] at t by de
    Casteljau (no basis table)."""
    p = np.array(pts, np.float64)
    n = len(p) - 1
    while len(p) > 2:
        p = (1 - t) * p[:-1] + t * p[1:]
    pt = (1 - t) * p[0] + t * p[1]
    return pt, n * (p[1] - p[0])


def _branches(cp):
    K = cp.shape[0]
    kb = (K + 2) // 2
    return [cp[(b * (kb - 1) + np.arange(kb)) % K] for b in range(2)]


@pytest.mark.parametrize("K,sub", [(4, 4), (6, 3), (10, 4), (12, 2)])
def test_ring_is_continuous_and_closed(K, sub):
    rng = np.random.default_rng(K)
    cp = rng.normal(size=(3, K, 2)) * 50
    seg = O.closed_ring_segments(cp, sub).reshape(3, 2 * sub, 4, 2)
    np.testing.assert_allclose(seg[:, 1:, 0], seg[:, :-1, 3], atol=1e-9)  # within and across branches
    np.testing.assert_allclose(seg[:, 0, 0], seg[:, -1, 3], atol=1e-9)   # ring closes
    np.testing.assert_allclose(seg[:, 0, 0], cp[:, 0], atol=1e-9)


@pytest.mark.parametrize("K", [4, 6])
def test_low_degree_branches_are_reproduced_exactly(K):
    """A cubic Hermite piece with the curve's end points and end derivatives
    is the curve itself when the curve has degree <= 3."""
    rng = np.random.default_rng(7)
    sub = 5
    cp = rng.normal(size=(1, K, 2)) * 20
    seg = O.closed_ring_segments(cp, sub).reshape(2, sub, 4, 2)
    t = np.linspace(0.0, 1.0, sub + 1)
    for b, pts in enumerate(_branches(cp[0])):
        for s in range(sub):
            P = seg[b, s]
            for u in rng.random(5):
                herm = ((1 - u) ** 3 * P[0] + 3 * (1 - u) ** 2 * u * P[1]
                        + 3 * (1 - u) * u ** 2 * P[2] + u ** 3 * P[3])
                curve, _ = _bezier(pts, t[s] + u * (t[s + 1] - t[s]))
                np.testing.assert_allclose(herm, curve, atol=1e-9)


@pytest.mark.parametrize("K", [8, 10, 14])
def test_end_points_and_tangents_follow_the_bezier_branch(K):
    rng = np.random.default_rng(K)
    sub = 4
    cp = rng.normal(size=(1, K, 2)) * 30
    seg = O.closed_ring_segments(cp, sub).reshape(2, sub, 4, 2)
    t = np.linspace(0.0, 1.0, sub + 1)
    dt = t[1] - t[0]
    for b, pts in enumerate(_branches(cp[0])):
        for s in range(sub):
            p0, d0 = _bezier(pts, t[s])
            p3, d1 = _bezier(pts, t[s + 1])
            P = seg[b, s]
            np.testing.assert_allclose(P[0], p0, atol=1e-9)
            np.testing.assert_allclose(P[3], p3, atol=1e-9)
            np.testing.assert_allclose(3 * (P[1] - P[0]) / dt, d0, atol=1e-8)
            np.testing.assert_allclose(3 * (P[3] - P[2]) / dt, d1, atol=1e-8)


def test_basis_tables():
    for kb, sub in ((3, 4), (6, 4), (7, 9)):
        basis, deriv, dt = O.closed_ring_basis(kb, sub)
        np.testing.assert_allclose(basis.sum(1), 1.0, atol=1e-14)
        np.testing.assert_allclose(deriv.sum(1), 1.0, atol=1e-14)
        np.testing.assert_array_equal(basis[0], np.eye(kb)[0])
        np.testing.assert_array_equal(basis[-1], np.eye(kb)[-1])
        np.testing.assert_allclose(dt, 1.0 / sub)


@pytest.mark.parametrize("K,sub", [(4, 4), (10, 4), (12, 3)])
def test_backward_is_the_adjoint_of_the_forward(K, sub):
    rng = np.random.default_rng(11 * K + sub)
    N = 5
    x = rng.normal(size=(N, K, 2))
    y = rng.normal(size=(N * 2 * sub, 4, 2))
    lhs = float((O.closed_ring_segments(x, sub) * y).sum())
    rhs = float((x * O.closed_ring_segments_backward(y, N, K, sub)).sum())
    assert abs(lhs - rhs) <= 1e-10 * max(abs(lhs), 1.0)
