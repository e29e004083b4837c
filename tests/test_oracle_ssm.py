"""Pins the selective-scan oracle (``oracle/ssm.py``) on the CPU, without
retyping its formulas: the reference's golden fixture, an independent
per-step loop, the reference's scan invariants, and float64 finite
differences of the VJP."""

from __future__ import annotations

import numpy as np
import pytest
from _golden import load_golden

from oracle import ssm as S

# tolerance.toml:25-27 (selective_scan float32)
_ATOL, _RTOL = 1e-5, 1e-4


def _inputs(b, length, d, n, seed, with_d=True):
    # The reference test inputs (tests/test_nn_ssm.py:44-57): softplus delta,
    # A = -exp(randn).
    rng = np.random.RandomState(seed)
    shp = (length, d) if b is None else (b, length, d)
    bshp = (length, n) if b is None else (b, length, n)
    x = rng.standard_normal(shp)
    delta = np.log1p(np.exp(rng.standard_normal(shp)))
    A = -np.exp(rng.standard_normal((d, n)))
    B = rng.standard_normal(bshp)
    C = rng.standard_normal(bshp)
    D = rng.standard_normal((d,)) if with_d else None
    return x, delta, A, B, C, D


def test_golden_fixture():
    g = load_golden('selective_scan_float32')
    out = S.selective_scan(g['x'], g['delta'], g['A'], g['B'], g['C'], g['D'])
    assert out.dtype == np.float32
    np.testing.assert_allclose(out, g['out'], atol=_ATOL, rtol=_RTOL)


def _naive(x, delta, A, B, C, D=None):
    # Per-channel, per-state scalar loops.
    length, d = x.shape
    n = A.shape[1]
    y = np.zeros((length, d))
    for j in range(d):
        h = np.zeros(n)
        for t in range(length):
            for k in range(n):
                h[k] = np.exp(delta[t, j] * A[j, k]) * h[k] + delta[t, j] * B[t, k] * x[t, j]
            y[t, j] = np.dot(C[t], h) + (0.0 if D is None else D[j] * x[t, j])
    return y


def test_matches_naive_loops():
    x, delta, A, B, C, D = _inputs(None, 7, 4, 3, seed=1)
    np.testing.assert_allclose(S.selective_scan(x, delta, A, B, C, D),
                               _naive(x, delta, A, B, C, D), atol=1e-12)


def test_d_skip_is_linear():
    x, delta, A, B, C, D = _inputs(2, 6, 4, 3, seed=4)
    np.testing.assert_allclose(S.selective_scan(x, delta, A, B, C, D),
                               S.selective_scan(x, delta, A, B, C) + D * x, atol=1e-12)


def test_zero_A_is_a_cumulative_sum():
    x, delta, _, B, C, _ = _inputs(2, 6, 4, 3, seed=5)
    H = np.cumsum(delta[..., None] * B[..., None, :] * x[..., None], axis=-3)
    np.testing.assert_allclose(S.selective_scan(x, delta, np.zeros((4, 3)), B, C),
                               np.sum(H * C[..., None, :], axis=-1), atol=1e-12)


@pytest.mark.parametrize('with_d', [False, True])
def test_vjp_matches_finite_differences(with_d):
    x, delta, A, B, C, D = _inputs(2, 5, 3, 2, seed=7, with_d=with_d)
    dy = np.random.RandomState(8).standard_normal(x.shape)
    grads = S.selective_scan_vjp(x, delta, A, B, C, D, dy)
    args = [x, delta, A, B, C, D]
    eps = 1e-6

    def loss(*a):
        return float(np.sum(S.selective_scan(*a, acc_dtype=np.float64) * dy))

    for w in range(6):
        if args[w] is None:
            assert grads[w] is None
            continue
        fd = np.zeros_like(args[w])
        for idx in np.ndindex(args[w].shape):
            ap = list(args)
            am = list(args)
            ap[w] = args[w].copy()
            am[w] = args[w].copy()
            ap[w][idx] += eps
            am[w][idx] -= eps
            fd[idx] = (loss(*ap) - loss(*am)) / (2 * eps)
        assert grads[w].shape == args[w].shape
        np.testing.assert_allclose(grads[w], fd, atol=1e-6, rtol=1e-5)


def test_planted_vjp_mistake_fails():
    # A state cotangent without the decay term (g_t = C_t dy_t only) gives a
    # dx that the finite differences reject, while the oracle's passes.
    x, delta, A, B, C, D = _inputs(1, 4, 2, 2, seed=9)
    dy = np.random.RandomState(10).standard_normal(x.shape)
    good = S.selective_scan_vjp(x, delta, A, B, C, D, dy)[0]
    g = C[..., :, None, :] * dy[..., None]
    mutant = np.sum(g * delta[..., None] * B[..., :, None, :], axis=-1) + D * dy
    eps = 1e-6
    fd = np.zeros_like(x)
    for idx in np.ndindex(x.shape):
        xp, xm = x.copy(), x.copy()
        xp[idx] += eps
        xm[idx] -= eps
        fd[idx] = (np.sum(S.selective_scan(xp, delta, A, B, C, D, acc_dtype=np.float64) * dy)
                   - np.sum(S.selective_scan(xm, delta, A, B, C, D, acc_dtype=np.float64) * dy)) / (2 * eps)
    np.testing.assert_allclose(good, fd, atol=1e-6, rtol=1e-5)
    assert np.max(np.abs(mutant - fd)) > 1e-2
