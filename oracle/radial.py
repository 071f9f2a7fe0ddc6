"""Radial basis restated from e3nn (third-party, not under the reference tree).

The reference calls ``e3nn.math.soft_one_hot_linspace(r, 0, rc, nb, basis=..., cutoff=True)``
and multiplies by ``sqrt(nb)`` (``models/pure_cartesian_sparse_layers.py:319-321,410-412``,
``models/pure_cartesian_ictd_layers_full.py:464-465,930-937``).  e3nn is pinned only as
``e3nn>=0.4.4,<0.6.0`` (``setup.py:81``, ``requirements.txt:5``) and is absent from this image.
This module restates e3nn's published definition (``e3nn/math/_soft_one_hot_linspace.py``,
versions 0.4.4-0.5.x) for the bases the reference's configurations use.

Parity note: no reference test holds values of this function, so beyond the closed
forms checked in ``tests/test_oracle_radial.py`` (orthogonality of the Bessel basis on
(0, rc), the Gaussian centres and widths) its values are "parity unpinned".
"""

from __future__ import annotations

import math

import torch


def soft_one_hot_linspace(x: torch.Tensor, start: float, end: float, number: int,
                          basis: str, cutoff: bool) -> torch.Tensor:
    """``(..., number)`` basis values of ``x``; e3nn semantics for gaussian/bessel/cosine/fourier/smooth_finite."""
    if cutoff:
        values = torch.linspace(start, end, number + 2, dtype=x.dtype, device=x.device)
        step = values[1] - values[0]
        values = values[1:-1]
    else:
        values = torch.linspace(start, end, number, dtype=x.dtype, device=x.device)
        step = values[1] - values[0]
    if basis == "gaussian":
        diff = (x[..., None] - values) / step
        return diff.pow(2).neg().exp().div(1.12)
    if basis == "cosine":
        diff = (x[..., None] - values) / step
        return torch.cos(math.pi / 2 * diff) * (diff < 1) * (-1 < diff)
    if basis == "smooth_finite":
        # soft_unit_step(x) = exp(-1/x) for x > 0, else 0
        diff = (x[..., None] - values) / step

        def sus(v):
            return torch.where(v > 0, torch.exp(-1.0 / torch.where(v > 0, v, torch.ones_like(v))),
                               torch.zeros_like(v))

        return 1.14136 * math.exp(2.0) * sus(diff + 1) * sus(1 - diff)
    if basis == "fourier":
        u = (x[..., None] - start) / (end - start)
        if not cutoff:
            i = torch.arange(0, number, dtype=x.dtype, device=x.device)
            return torch.cos(math.pi * i * u) / math.sqrt(0.25 + number / 2)
        i = torch.arange(1, number + 1, dtype=x.dtype, device=x.device)
        return torch.sin(math.pi * i * u) / math.sqrt(0.25 + number / 2) * (0 < u) * (u < 1)
    if basis == "bessel":
        u = x[..., None] - start
        c = end - start
        roots = torch.arange(1, number + 1, dtype=x.dtype, device=x.device) * math.pi
        out = math.sqrt(2 / c) * torch.sin(roots * u / c) / u
        if not cutoff:
            return out
        return out * ((u / c) < 1) * (0 < u)
    raise ValueError(f"unsupported basis {basis!r}")
