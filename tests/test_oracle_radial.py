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
