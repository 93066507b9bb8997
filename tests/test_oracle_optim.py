"""Pins of the oracle's Adan step (oracle.adan_step64, restating
ops/optim.py:78-110) by closed forms that do not share its code."""
import numpy as np

from oracle import oracle as O


def _run(gs, **kw):
    p = np.zeros_like(gs[0])
    m = n = d = npg = np.zeros_like(gs[0])
    for t, g in enumerate(gs, 1):
        p, m, n, d, npg = O.adan_step64(p, g, m, n, d, npg, step=t, **kw)
    return p, m, n, d, npg


def test_first_step_is_a_normalized_gradient_step():
    """Step 1: m = (1 - b1) g and n = (1 - b3) g^2 are undone by the bias
    corrections and the difference terms vanish, so p -= lr g / (|g| + eps)
    (a dropped bias correction or a nonzero first difference breaks this)."""
    g = np.array([0.3, -2.0, 1e-3, 5.0])
    p, m, n, d, npg = _run([g], lr=0.01, eps=1e-8)
    np.testing.assert_allclose(p, -0.01 * g / (np.abs(g) + 1e-8), rtol=1e-12)
    np.testing.assert_array_equal(d, 0.0)
    np.testing.assert_array_equal(npg, -g)


def test_constant_gradient_keeps_the_normalized_step():
    """With g constant the gradient difference is 0 after step 1, so d stays 0
    and every step moves p by lr g / (|g| + eps): after T steps
    p = -T lr g / (|g| + eps) for every beta (bias corrections exact)."""
    g = np.array([1.5, -0.25, 4.0])
    for betas in ((0.98, 0.92, 0.99), (0.5, 0.3, 0.9), (0.0, 0.0, 0.0)):
        p, m, n, d, _ = _run([g] * 7, lr=0.02, betas=betas, eps=0.0)
        np.testing.assert_allclose(p, -7 * 0.02 * np.sign(g), rtol=1e-12)
        np.testing.assert_allclose(d, 0.0, atol=1e-15)


def test_weight_decay_placement():
    """no_prox decays before the update, p (1 - lr wd) - lr g/(|g|+eps); the
    default divides after it, (p - lr g/(|g|+eps)) / (1 + lr wd)."""
    g = np.array([0.5, -1.0])
    p0 = np.array([2.0, -3.0])
    z = np.zeros(2)
    step = 0.1 * g / (np.abs(g) + 1e-8)
    p, *_ = O.adan_step64(p0, g, z, z, z, z, step=1, lr=0.1, weight_decay=0.5, no_prox=True)
    np.testing.assert_allclose(p, p0 * (1 - 0.05) - step, rtol=1e-12)
    p, *_ = O.adan_step64(p0, g, z, z, z, z, step=1, lr=0.1, weight_decay=0.5)
    np.testing.assert_allclose(p, (p0 - step) / (1 + 0.05), rtol=1e-12)


def test_second_step_by_hand():
    """Two steps with g1 = 1, g2 = -1 (betas 0.5, 0.5, 0.5, lr 1, eps 0)
    worked out from the update rule: the difference g2 - g1 = -2 enters d and
    the second-moment argument; a sign slip in the difference or a swapped
    beta changes the result."""
    p, m, n, d, npg = _run([np.array([1.0]), np.array([-1.0])], lr=1.0,
                           betas=(0.5, 0.5, 0.5), eps=0.0)
    # step 1: m = .5, n = .5, d = 0, p = -1
    # step 2: ngod = -2; m = .25 - .5 = -.25; d = -1; ngod2 = -1 - 1 = -2;
    #         n = .25 + 4 * .5 = 2.25; bc1 = bc2 = bc3 = .75;
    #         denom = 1.5 / sqrt(.75); p = -1 + (.25 / .75 + .5 / .75) / denom
    denom = 1.5 / np.sqrt(0.75)
    np.testing.assert_allclose(m, [-0.25])
    np.testing.assert_allclose(d, [-1.0])
    np.testing.assert_allclose(n, [2.25])
    np.testing.assert_allclose(p, [-1.0 + (0.25 / 0.75 + 0.5 / 0.75) / denom], rtol=1e-12)


def test_clip_scales_the_gradient():
    """The clip factor multiplies the gradient before every use: with a clip
    c the states are those of the gradient c g."""
    g = np.array([0.7, -0.2])
    a = _run([g, 2 * g], clip=0.25)
    b = _run([0.25 * g, 0.5 * g])
    for x, y in zip(a, b):
        np.testing.assert_allclose(x, y, rtol=1e-12)
