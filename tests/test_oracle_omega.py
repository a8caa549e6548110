"""Pins of the oracle's omega EMA (spherical_kv_pipeline.py:952-987) by
closed forms: the restatement is checked against what the mathematics fixes,
not against a retyped formula."""
import numpy as np

import oracle


def test_uniform_pages_share_the_mass_equally():
    nkv, g, P = 2, 4, 10
    m = np.full((nkv * g, P), 3.0)
    l = np.full((nkv * g, P), 2.0)
    om = oracle.omega_ema(m, l, np.zeros((nkv, P)), nkv, g, 0.0)
    np.testing.assert_allclose(om, 1.0 / P, rtol=1e-15)


def test_invalid_pages_get_no_mass_and_a_single_page_gets_all():
    nkv, g, P = 1, 2, 5
    m = np.zeros((g, P))
    l = np.zeros((g, P))
    l[:, 3] = 7.0                      # one valid page per q head
    m[:, 0] = 1e3                      # an invalid page's m must not win the max
    om = oracle.omega_ema(m, l, np.ones((nkv, P)), nkv, g, 0.5)
    np.testing.assert_allclose(om[0], [0.5, 0.5, 0.5, 1.0, 0.5], rtol=1e-15)


def test_two_pages_softmax_and_the_minus_60_clamp():
    # masses l1 e^{m1} : l2 e^{m2}; a page 100 below the max is clamped to e^-60
    m = np.array([[0.0, np.log(3.0)], [0.0, -100.0]])
    l = np.array([[1.0, 1.0], [2.0, 5.0]])
    om = oracle.omega_ema(m, l, np.zeros((2, 2)), 2, 1, 0.0)
    np.testing.assert_allclose(om[0], [0.25, 0.75], rtol=1e-14)
    w2 = 5.0 * np.exp(-60.0)
    np.testing.assert_allclose(om[1], [2.0 / (2.0 + w2), w2 / (2.0 + w2)], rtol=1e-14)


def test_group_mean_and_ema_blend():
    # q head 0 puts all mass on page 0, q head 1 on page 1: the kv head gets 1/2 each
    m = np.zeros((2, 3))
    l = np.array([[1.0, 0.0, 0.0], [0.0, 1.0, 0.0]])
    prev = np.array([[0.2, 0.4, 0.8]])
    om = oracle.omega_ema(m, l, prev, 1, 2, 0.9)
    np.testing.assert_allclose(om[0], prev[0] * 0.9 + np.array([0.5, 0.5, 0.0]) * 0.1, rtol=1e-15)


def test_head_with_no_valid_page_gets_zero_mass():
    m = np.random.default_rng(0).standard_normal((3, 4))
    om = oracle.omega_ema(m, np.zeros((3, 4)), np.full((3, 4), 2.0), 3, 1, 0.9)
    np.testing.assert_allclose(om, 1.8, rtol=1e-15)
