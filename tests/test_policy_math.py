"""CPU pins for the float64 restatements the GPU policy tests compare against.

The KL divergence of two Beta laws in closed form,
  KL(Beta(a1, b1) || Beta(a2, b2)) = ln B(a2, b2) - ln B(a1, b1) + (a1 - a2) psi(a1)
                                     + (b1 - b2) psi(b1) + (a2 - a1 + b2 - b1) psi(a1 + b1),
is checked against direct quadrature of p1 log(p1 / p2) (scipy.integrate.quad),
including shapes below 1, so a sign or argument slip in the closed form fails here.
"""
from __future__ import annotations

import numpy as np
import pytest
from scipy import integrate, special, stats


def beta_kl(a1, b1, a2, b2):
    lnb = lambda a, b: special.gammaln(a) + special.gammaln(b) - special.gammaln(a + b)
    return (lnb(a2, b2) - lnb(a1, b1) + (a1 - a2) * special.digamma(a1) + (b1 - b2) * special.digamma(b1)
            + (a2 - a1 + b2 - b1) * special.digamma(a1 + b1))


@pytest.mark.parametrize("a1,b1,a2,b2", [(2.0, 3.0, 2.5, 2.0), (1.0, 1.0, 4.0, 1.5), (7.0, 2.0, 6.5, 2.2),
                                         (0.6, 0.8, 1.3, 0.5), (1.5, 0.4, 0.9, 0.9), (30.0, 40.0, 31.0, 38.0)])
def test_beta_kl_closed_form_matches_quadrature(a1, b1, a2, b2):
    p, q = stats.beta(a1, b1), stats.beta(a2, b2)
    f = lambda x: p.pdf(x) * (p.logpdf(x) - q.logpdf(x))
    want, err = integrate.quad(f, 0.0, 1.0, limit=400, points=[1e-6, 0.5, 1 - 1e-6])
    assert abs(beta_kl(a1, b1, a2, b2) - want) <= 1e-6 + 1e-6 * abs(want) + 10 * err


def test_beta_kl_zero_on_equal_laws_and_positive():
    rng = np.random.default_rng(1)
    a, b = rng.uniform(0.2, 50.0, 100), rng.uniform(0.2, 50.0, 100)
    assert np.all(np.abs(beta_kl(a, b, a, b)) < 1e-9)
    assert np.all(beta_kl(a, b, a * 1.1, b * 0.9) > 0.0)
