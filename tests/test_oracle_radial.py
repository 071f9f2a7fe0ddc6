"""Closed-form checks of the radial basis (e3nn's soft_one_hot_linspace, restated).

No reference test holds values of this third-party function; these checks fix what the
mathematics fixes: the Bessel functions sqrt(2/rc) sin(k pi r/rc) are orthonormal on
(0, rc) after multiplying by r, vanish outside it and tend to sqrt(2/rc) k pi/rc at r->0;
the Gaussians peak at the interior linspace points with height 1/1.12 and fall by e^-1
one step away.  The device kernel (radial_mlp) is checked against this oracle in
tests/test_edge_radial_gpu.py.
"""

import math

import numpy as np
import torch

from oracle.radial import soft_one_hot_linspace


def test_bessel_orthonormal_and_cutoff():
    rc, nb = 5.0, 8
    r = torch.linspace(1e-6, rc - 1e-6, 200001, dtype=torch.float64)
    b = soft_one_hot_linspace(r, 0.0, rc, nb, "bessel", True)
    f = b * r[:, None]
    gram = torch.trapezoid(f[:, :, None] * f[:, None, :], r, dim=0)
    np.testing.assert_allclose(gram.numpy(), np.eye(nb), atol=1e-6)
    outside = soft_one_hot_linspace(torch.tensor([rc, rc + 0.5, -1.0], dtype=torch.float64),
                                    0.0, rc, nb, "bessel", True)
    assert float(outside.abs().max()) == 0.0
    small = soft_one_hot_linspace(torch.tensor([1e-7], dtype=torch.float64), 0.0, rc, nb, "bessel", True)[0]
    lim = math.sqrt(2 / rc) * torch.arange(1, nb + 1, dtype=torch.float64) * math.pi / rc
    np.testing.assert_allclose(small.numpy(), lim.numpy(), rtol=1e-6)


def test_gaussian_centres_and_width():
    rc, nb = 5.0, 8
    step = rc / (nb + 1)
    centres = torch.arange(1, nb + 1, dtype=torch.float64) * step
    b = soft_one_hot_linspace(centres, 0.0, rc, nb, "gaussian", True)
    np.testing.assert_allclose(torch.diagonal(b).numpy(), np.full(nb, 1 / 1.12), rtol=1e-12)
    b1 = soft_one_hot_linspace(centres + step, 0.0, rc, nb, "gaussian", True)
    np.testing.assert_allclose(torch.diagonal(b1).numpy(), np.full(nb, math.exp(-1) / 1.12), rtol=1e-12)


def test_cosine_partition_of_unity():
    """Adjacent cosine bumps cos(pi d/2) and cos(pi (1-d)/2) are cos and sin of one angle: between the
    first and last centre the squares sum to 1; each bump is 1 at its centre and 0 one step away."""
    rc, nb = 5.0, 8
    step = rc / (nb + 1)
    r = torch.linspace(step, nb * step, 10001, dtype=torch.float64)
    b = soft_one_hot_linspace(r, 0.0, rc, nb, "cosine", True)
    np.testing.assert_allclose((b * b).sum(-1).numpy(), np.ones(r.shape[0]), atol=1e-12)
    centres = torch.arange(1, nb + 1, dtype=torch.float64) * step
    np.testing.assert_allclose(torch.diagonal(soft_one_hot_linspace(centres, 0.0, rc, nb, "cosine", True)).numpy(),
                               np.ones(nb), atol=1e-15)
    far = soft_one_hot_linspace(centres + step, 0.0, rc, nb, "cosine", True)
    assert float(torch.diagonal(far).abs().max()) < 1e-12


def test_smooth_finite_bump():
    """1.14136 e^2 exp(-1/(1+d)) exp(-1/(1-d)): 1.14136 at each centre, exp(-2/(1-d^2)) shape in between,
    exactly zero at and beyond one step from the centre, symmetric about it."""
    rc, nb = 5.0, 8
    step = rc / (nb + 1)
    centres = torch.arange(1, nb + 1, dtype=torch.float64) * step
    b = soft_one_hot_linspace(centres, 0.0, rc, nb, "smooth_finite", True)
    np.testing.assert_allclose(torch.diagonal(b).numpy(), np.full(nb, 1.14136), rtol=1e-12)
    d = 0.37
    bp = torch.diagonal(soft_one_hot_linspace(centres + d * step, 0.0, rc, nb, "smooth_finite", True))
    bm = torch.diagonal(soft_one_hot_linspace(centres - d * step, 0.0, rc, nb, "smooth_finite", True))
    want = 1.14136 * math.exp(2.0) * math.exp(-2.0 / (1 - d * d))
    np.testing.assert_allclose(bp.numpy(), np.full(nb, want), rtol=1e-12)
    np.testing.assert_allclose(bm.numpy(), bp.numpy(), rtol=1e-12)
    edge = soft_one_hot_linspace(centres + step, 0.0, rc, nb, "smooth_finite", True)
    assert float(torch.diagonal(edge).abs().max()) == 0.0


def test_fourier_orthogonal_and_cutoff():
    """sin(k pi r/rc)/sqrt(0.25 + nb/2): mutually orthogonal on (0, rc) with squared norm
    (rc/2)/(0.25 + nb/2), zero outside (0, rc)."""
    rc, nb = 5.0, 8
    r = torch.linspace(0.0, rc, 200001, dtype=torch.float64)
    b = soft_one_hot_linspace(r, 0.0, rc, nb, "fourier", True)
    gram = torch.trapezoid(b[:, :, None] * b[:, None, :], r, dim=0)
    np.testing.assert_allclose(gram.numpy(), np.eye(nb) * (rc / 2) / (0.25 + nb / 2), atol=1e-8)
    outside = soft_one_hot_linspace(torch.tensor([rc, rc + 0.3, -0.2], dtype=torch.float64),
                                    0.0, rc, nb, "fourier", True)
    assert float(outside.abs().max()) == 0.0
