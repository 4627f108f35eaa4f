"""Pins of the oracle's fp64 Oja step (stacr/layers.py:346-348, stacr/oja.py:73-79).

The reference's own tests hold no vector for this step, so it is pinned by what the mathematics
fixes: data inside span(Q) and an eigenbasis of X^T X are fixed points (update 0); an orthogonal
component P gives exactly P^T C / N (fixes the sign and which operand is transposed); the update
is quadratic in X; lr = 0 and N = 0 leave Q unchanged.
"""
import numpy as np
import pytest

from oracle import oracle as orc


def _basis(d, r, seed):
    q, _ = np.linalg.qr(np.random.default_rng(seed).standard_normal((d, r)))
    return q


@pytest.mark.parametrize("n,d,r", [(64, 20, 3), (300, 96, 16), (7, 40, 5)])
def test_in_span_data_is_a_fixed_point(n, d, r):
    q = _basis(d, r, n)
    c = np.random.default_rng(1).standard_normal((n, r))
    update, stepped = orc.oja_step(c @ q.T, q, 0.3)
    assert np.abs(update).max() <= 1e-12 * max(1.0, np.abs(c).max() ** 2)
    np.testing.assert_allclose(stepped, q, atol=1e-12)


@pytest.mark.parametrize("n,d,r", [(64, 20, 3), (300, 96, 16)])
def test_orthogonal_component_gives_closed_form(n, d, r):
    rng = np.random.default_rng(2)
    q = _basis(d, r, 3)
    c = rng.standard_normal((n, r))
    p = rng.standard_normal((n, d))
    p -= (p @ q) @ q.T  # P Q = 0
    update, _ = orc.oja_step(c @ q.T + p, q, 0.1)
    np.testing.assert_allclose(update, p.T @ c / n, atol=1e-12)


def test_eigenbasis_is_a_fixed_point_and_update_is_quadratic():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((500, 30)) * np.linspace(3, 0.1, 30)
    w, v = np.linalg.eigh(x.T @ x)
    top = v[:, np.argsort(w)[::-1][:4]]
    update, _ = orc.oja_step(x, top, 1.0)
    assert np.abs(update).max() <= 1e-10
    q = _basis(30, 4, 5)
    u1, _ = orc.oja_step(x, q, 1.0)
    u3, _ = orc.oja_step(3.0 * x, q, 1.0)
    np.testing.assert_allclose(u3, 9.0 * u1, rtol=1e-12, atol=1e-12)


def test_zero_rate_and_empty_batch_leave_basis_unchanged():
    q = _basis(12, 3, 6)
    x = np.random.default_rng(7).standard_normal((20, 12))
    _, stepped = orc.oja_step(x, q, 0.0)
    assert np.array_equal(stepped, q)
    update, stepped = orc.oja_step(np.zeros((0, 12)), q, 0.5)
    assert np.all(update == 0) and np.array_equal(stepped, q)


def test_orthonormalize_spans_input_with_orthonormal_columns():
    m = np.random.default_rng(8).standard_normal((40, 6))
    q = orc.orthonormalize(m)
    np.testing.assert_allclose(q.T @ q, np.eye(6), atol=1e-12)
    np.testing.assert_allclose(q @ (q.T @ m), m, atol=1e-12)
