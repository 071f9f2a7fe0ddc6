"""Test-side helpers for the sparse path: layouts, seeded models, oracle adapters."""

from __future__ import annotations

import numpy as np
import torch

from fsctep_amd.synthetic import seeded_value
from oracle import sparse_ref as R


def internal_to_ref(x: torch.Tensor) -> torch.Tensor:
    """x[N][13][C] -> reference flat (N, 26C): true half [C | C x 3 | C x 3 x 3] then zeros."""
    N, _, C = x.shape
    true = torch.cat([x[:, 0, :], x[:, 1:4, :].transpose(1, 2).reshape(N, 3 * C),
                      x[:, 4:13, :].transpose(1, 2).reshape(N, 9 * C)], dim=1)
    return torch.cat([true, torch.zeros_like(true)], dim=1)


def ref_to_internal(y: torch.Tensor, C: int) -> torch.Tensor:
    N = y.shape[0]
    x0 = y[:, :C].reshape(N, 1, C)
    x1 = y[:, C:4 * C].reshape(N, C, 3).transpose(1, 2)
    x2 = y[:, 4 * C:13 * C].reshape(N, C, 9).transpose(1, 2)
    return torch.cat([x0, x1, x2], dim=1)


def oracle_conv2(x, h, n, L, b, src, dst, N, inv_norm):
    """Reference conv2..n chain on internal layouts, from the oracle's TP and scatter."""
    E, C = h.shape[0], x.shape[2]
    w = h @ L.t() + b
    one = torch.ones(E, 1, dtype=x.dtype)
    zero3 = torch.zeros(E, 3, dtype=x.dtype)
    zero9 = torch.zeros(E, 9, dtype=x.dtype)
    nn_ = (n.unsqueeze(-1) * n.unsqueeze(-2)).reshape(E, 9)
    e_flat = torch.cat([one, n, nn_, torch.zeros(E, 1, dtype=x.dtype), zero3, zero9], dim=1)
    msg = R.sparse_tp(internal_to_ref(x)[src], e_flat, w, C, 1, C, 2)
    out = R.scatter_sum(msg, dst, N) * inv_norm
    return ref_to_internal(out, C)


def seeded_hip_model(channels: int, layers: int, seed: int, basis: str = "bessel"):
    from fsctep_amd.sparse import PureCartesianSparseTransformerLayer
    m = PureCartesianSparseTransformerLayer(
        max_embed_radius=5.0, main_max_radius=5.0, main_number_of_basis=8, hidden_dim_conv=channels,
        hidden_dim_sh=channels, hidden_dim=64, channel_in2=32, embedding_dim=16, max_atomvalue=10,
        output_size=8, invariant_channels=32, embed_size=[128, 128, 128], num_interaction=layers,
        function_type_main=basis, lmax=2, max_rank_other=1, k_policy="k0")
    with torch.no_grad():
        for name, p in m.named_parameters():
            p.copy_(torch.from_numpy(seeded_value(name, tuple(p.shape), seed)).to(p.dtype))
    return m.eval().requires_grad_(False)


def oracle_params(channels: int, layers: int, seed: int, dtype, basis: str = "bessel"):
    cfg = R.SparseConfig(channels=channels, num_interaction=layers, function_type=basis)
    p = {k: torch.tensor(seeded_value(k, s, seed), dtype=dtype) for k, s in R.param_shapes(cfg)}
    return cfg, p


def rel_inf(a, b) -> float:
    a = np.asarray(a.detach().cpu() if torch.is_tensor(a) else a, np.float64)
    b = np.asarray(b.detach().cpu() if torch.is_tensor(b) else b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))
