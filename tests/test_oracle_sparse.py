"""Pins the sparse-trunk oracle against the reference's golden vectors and the mathematics.

* golden vectors written by running the reference trunk (tests/golden/make_sparse_golden.py);
* the sparse TP against brute-force loops on a tiny case (path order, index order);
* O(3) invariance of energies / covariance of forces under a random rotation+reflection
  (the pattern of the reference's test/test_equivariance.py:304-376);
* forces against central finite differences (test/self_test_lammps_potential.py:727-744);
* a planted mistake in the oracle (wrong conv2 normalisation) must fail the golden check.
"""

import math

import numpy as np
import pytest
import torch

from conftest import load_golden
from fsctep_amd.synthetic import seeded_value
from oracle import sparse_ref as R


def cfg_for(g):
    return R.SparseConfig(channels=int(g["channels"]), num_interaction=int(g["layers"]),
                          function_type=str(g["function_type"]))


def params_for(cfg, seed, dtype):
    return {k: torch.tensor(seeded_value(k, s, seed), dtype=dtype) for k, s in R.param_shapes(cfg)}


def inputs_for(g, dtype):
    n = g["pos"].shape[0]
    return (torch.tensor(g["pos"], dtype=dtype), torch.tensor(g["species"]), torch.zeros(n, dtype=torch.long),
            torch.tensor(g["edge_src"]), torch.tensor(g["edge_dst"]),
            torch.tensor(g["edge_shifts"], dtype=dtype), torch.tensor(g["cell"], dtype=dtype))


def rel_inf(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


@pytest.mark.parametrize("name", ["sparse_open32_c32_l2", "sparse_pbc100_c64_l3"])
@pytest.mark.parametrize("dtype,tol", [(torch.float64, 1e-10), (torch.float32, 1e-5)])
def test_oracle_matches_reference_golden(name, dtype, tol):
    g = load_golden(name)
    cfg = cfg_for(g)
    p = params_for(cfg, int(g["param_seed"]), dtype)
    e, f = R.energy_forces(*inputs_for(g, dtype), p, cfg)
    tag = "f64" if dtype == torch.float64 else "f32"
    assert rel_inf(e, g[f"energy_{tag}"]) < tol
    assert rel_inf(f, g[f"forces_{tag}"]) < tol
    # the fp32 reference itself sits within 1e-5 of the fp64 reference
    assert rel_inf(g["forces_f32"], g["forces_f64"]) < 1e-5


def test_planted_normalisation_mistake_fails_golden(monkeypatch):
    g = load_golden("sparse_pbc100_c64_l3")
    cfg = cfg_for(g)
    p = params_for(cfg, int(g["param_seed"]), torch.float64)
    orig = R.conv2

    def wrong(f, vec, src, dst, n, p_, layer, cfg_, avg_degree=None, edge_chunk=None):
        # per-receiver in-degree instead of the global E/N of the reference's conv2
        out = orig(f, vec, src, dst, n, p_, layer, cfg_, avg_degree, edge_chunk) * (vec.shape[0] / n)
        cnt = R.scatter_sum(torch.ones_like(dst), dst, n).clamp(min=1).to(out.dtype)
        return out / cnt.unsqueeze(-1)

    monkeypatch.setattr(R, "conv2", wrong)
    e, _ = R.energy_forces(*inputs_for(g, torch.float64), p, cfg)
    assert rel_inf(e, g["energy_f64"]) > 1e-3


def test_sparse_tp_bruteforce():
    torch.manual_seed(0)
    E, c1, c2, co, lmax = 3, 2, 3, 2, 2
    x1 = torch.randn(E, R.o3_dim(c1, lmax), dtype=torch.float64)
    x2 = torch.randn(E, R.o3_dim(c2, lmax), dtype=torch.float64)
    paths = R.sparse_paths(lmax)
    assert [(q.L1, q.L2, q.Lout) for q in paths] == [(0, 0, 0), (0, 1, 1), (0, 2, 2), (1, 0, 1), (1, 1, 2), (2, 0, 2)]
    w = torch.randn(E, len(paths) * co * c1 * c2, dtype=torch.float64)
    out = R.split_o3(R.sparse_tp(x1, x2, w, c1, c2, co, lmax), co, lmax)
    A = R.split_o3(x1, c1, lmax)
    B = R.split_o3(x2, c2, lmax)
    W = w.view(E, len(paths), co, c1, c2)
    ref = {L: np.zeros((E, co) + (3,) * L) for L in range(3)}
    for e in range(E):
        for k, q in enumerate(paths):
            for c in range(co):
                for a in range(c1):
                    for b in range(c2):
                        t1 = A[(0, q.L1)][e, a].numpy()
                        t2 = B[(0, q.L2)][e, b].numpy()
                        ref[q.Lout][e, c] += float(W[e, k, c, a, b]) * np.multiply.outer(t1, t2)
    for L in range(3):
        np.testing.assert_allclose(out[(0, L)].numpy(), ref[L], rtol=1e-12, atol=1e-12)
        assert float(out[(1, L)].abs().max()) == 0.0


def _random_o3(seed):
    rng = np.random.default_rng(seed)
    q, r = np.linalg.qr(rng.standard_normal((3, 3)))
    q = q * np.sign(np.diag(r))
    if np.linalg.det(q) > 0:
        q = -q  # include a reflection
    return torch.tensor(q)


def test_oracle_o3_invariance():
    g = load_golden("sparse_open32_c32_l2")
    cfg = cfg_for(g)
    p = params_for(cfg, 7, torch.float64)
    pos, A, batch, src, dst, sh, cell = inputs_for(g, torch.float64)
    Q = _random_o3(3)
    e0, f0 = R.energy_forces(pos, A, batch, src, dst, sh, cell, p, cfg)
    e1, f1 = R.energy_forces(pos @ Q.T, A, batch, src, dst, sh, cell @ Q.T, p, cfg)
    assert rel_inf(e1, e0) < 1e-10
    assert rel_inf(f1, f0 @ Q.T) < 1e-10


def test_oracle_forces_finite_difference():
    g = load_golden("sparse_open32_c32_l2")
    cfg = cfg_for(g)
    p = params_for(cfg, int(g["param_seed"]), torch.float64)
    pos, A, batch, src, dst, sh, cell = inputs_for(g, torch.float64)
    _, f = R.energy_forces(pos, A, batch, src, dst, sh, cell, p, cfg)
    h = 1e-5
    for atom, ax in [(0, 0), (5, 1), (17, 2), (31, 0)]:
        pp = pos.clone()
        pp[atom, ax] += h
        ep = R.atom_energies(pp, A, batch, src, dst, sh, cell, p, cfg).sum()
        pp[atom, ax] -= 2 * h
        em = R.atom_energies(pp, A, batch, src, dst, sh, cell, p, cfg).sum()
        fd = -(ep - em) / (2 * h)
        assert abs(float(fd) - float(f[atom, ax])) < 1e-6 * max(1.0, abs(float(fd)))
