"""Radial basis on the device: ``soft_one_hot_linspace(r, 0, rc, nb, basis, cutoff=True) * sqrt(nb)``.

Same definition as e3nn's ``soft_one_hot_linspace`` (the function the reference calls at
``models/pure_cartesian_sparse_layers.py:319-321,410-412``), for the two bases the
benchmark configurations use.
"""

from __future__ import annotations

import math

import torch


def radial_basis(r: torch.Tensor, rc: float, nb: int, basis: str) -> torch.Tensor:
    if basis == "bessel":
        k = torch.arange(1, nb + 1, dtype=r.dtype, device=r.device) * (math.pi / rc)
        x = r.unsqueeze(-1)
        inside = ((x / rc) < 1) & (x > 0)
        out = math.sqrt(2.0 / rc) * torch.sin(k * x) / x
        return out * inside * math.sqrt(nb)
    if basis == "gaussian":
        step = rc / (nb + 1)
        centres = torch.arange(1, nb + 1, dtype=r.dtype, device=r.device) * step
        d = (r.unsqueeze(-1) - centres) / step
        return torch.exp(-d * d) / 1.12 * math.sqrt(nb)
    raise ValueError(f"radial basis {basis!r} is not supported by the HIP path")
