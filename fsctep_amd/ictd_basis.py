"""ICTD constants and path tables for the HIP kernels (host side, float64).

The harmonic basis of degree l is the null space of the Laplacian on Sym^l, symmetrically
orthonormalised under the isotropic-Gaussian Gram matrix (models/ictd_irreps.py:144-185).  The
null space is taken from the same LAPACK call the reference makes (``torch.linalg.svd`` of the
float64 Laplacian on the CPU): the reference's readout re-splits features across l-blocks
(models/pure_cartesian_ictd_layers_full.py:977-979), so energies depend on the l>=2 basis itself,
not only on its span.  Everything downstream of the null space (orthonormalisation, trace-chain
projectors, coupling tensors, their "component" normalisation) is uniquely determined.

Irreps are keys (l, parity); a configuration is the ordered list of active keys.  Node features
are stored component-major, x[N][M][C] with M = sum(2l+1) over keys; edge harmonics Y[E][(lmax+1)^2]
with block l at offset l^2.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from functools import lru_cache

import numpy as np


def monomials(L: int):
    return [(a, b, L - a - b) for a in range(L + 1) for b in range(L - a + 1)]


def _moment(n: int) -> float:
    return 0.0 if n % 2 else float(np.prod(np.arange(n - 1, 0, -2))) if n > 1 else 1.0


@lru_cache(maxsize=None)
def gaussian_gram(L: int) -> np.ndarray:
    ms = monomials(L)
    return np.array([[_moment(a + u) * _moment(b + v) * _moment(c + w) for (u, v, w) in ms] for (a, b, c) in ms])


def laplacian(L: int) -> np.ndarray:
    rows = {t: i for i, t in enumerate(monomials(L - 2))}
    D = np.zeros((len(rows), len(monomials(L))))
    for j, (a, b, c) in enumerate(monomials(L)):
        for e, sh in ((a, (2, 0, 0)), (b, (0, 2, 0)), (c, (0, 0, 2))):
            if e >= 2:
                D[rows[(a - sh[0], b - sh[1], c - sh[2])], j] += e * (e - 1)
    return D


@lru_cache(maxsize=None)
def harmonic_basis(l: int) -> np.ndarray:
    """(Dsym(l), 2l+1) G-orthonormal harmonic basis."""
    if l == 0:
        return np.ones((1, 1))
    if l == 1:
        return np.eye(3)
    import torch
    _, s, vh = torch.linalg.svd(torch.tensor(laplacian(l), dtype=torch.float64), full_matrices=True)
    rank = int((s > 1e-12).sum())
    B = vh[rank:].T.numpy()
    ev, U = np.linalg.eigh(B.T @ gaussian_gram(l) @ B)
    return B @ (U * (1.0 / np.sqrt(np.maximum(ev, 1e-14)))) @ U.T


def _r2k(l: int, k: int) -> np.ndarray:
    src = monomials(l)
    dst = {t: i for i, t in enumerate(monomials(l + 2 * k))}
    M = np.zeros((len(dst), len(src)))
    for j, (a, b, c) in enumerate(src):
        for u in range(k + 1):
            for v in range(k - u + 1):
                w = k - u - v
                M[dst[(a + 2 * u, b + 2 * v, c + 2 * w)], j] += (
                    math.factorial(k) / (math.factorial(u) * math.factorial(v) * math.factorial(w)))
    return M


@lru_cache(maxsize=None)
def coupling(l1: int, l2: int, l3: int) -> np.ndarray:
    """Normalised C[m1,m2,m3] (||C||_F = sqrt(2 l3 + 1)); zero when not allowed."""
    if not (abs(l1 - l2) <= l3 <= l1 + l2) or (l1 + l2 + l3) % 2:
        return np.zeros((2 * l1 + 1, 2 * l2 + 1, 2 * l3 + 1))
    L = l1 + l2
    V = _r2k(l3, (L - l3) // 2) @ harmonic_basis(l3)
    G = gaussian_gram(L)
    proj = np.linalg.solve(V.T @ G @ V, V.T @ G)                    # (2l3+1, Dsym(L))
    idx = {t: i for i, t in enumerate(monomials(L))}
    B1, B2 = harmonic_basis(l1), harmonic_basis(l2)
    prod = np.zeros((len(idx), 2 * l1 + 1, 2 * l2 + 1))           # polynomial product of basis pairs
    for i, u in enumerate(monomials(l1)):
        for j, v in enumerate(monomials(l2)):
            prod[idx[(u[0] + v[0], u[1] + v[1], u[2] + v[2])]] += np.outer(B1[i], B2[j])
    C = np.einsum("kd,dmn->mnk", proj, prod)
    return C * (math.sqrt(2 * l3 + 1) / np.linalg.norm(C))


@lru_cache(maxsize=None)
def harmonic_projection(l: int) -> tuple:
    """(exponents (D,3), multinomials (D,), P = G_l B_l (D, 2l+1)): Y_l(n) = (coef * n^abc) @ P."""
    ms = monomials(l)
    coef = np.array([math.factorial(l) / (math.factorial(a) * math.factorial(b) * math.factorial(c))
                     for a, b, c in ms])
    return np.array(ms), coef, gaussian_gram(l) @ harmonic_basis(l)


def canonical(l: int) -> tuple:
    return (l, 1 if l % 2 == 0 else -1)


def all_paths(keys, lmax: int) -> list:
    """Reference enumeration of (l1,p1,l2,p2,l3,p3) over active keys (models/ictd_irreps.py:1371-1380)."""
    ks = set(keys)
    out = []
    for l1, p1 in keys:
        for l2, p2 in keys:
            for l3 in range(abs(l1 - l2), min(l1 + l2, lmax) + 1):
                if (l1 + l2 + l3) % 2 == 0 and (l3, p1 * p2) in ks:
                    out.append((l1, p1, l2, p2, l3, p1 * p2))
    return out


@dataclass(frozen=True)
class Layout:
    """Active irreps of one trunk and the derived kernel tables."""

    name: str
    lmax: int
    keys: tuple

    @property
    def comp_off(self) -> dict:
        off, out = 0, {}
        for k in self.keys:
            out[k] = off
            off += 2 * k[0] + 1
        return out

    @property
    def M(self) -> int:
        return sum(2 * k[0] + 1 for k in self.keys)

    @property
    def NY(self) -> int:
        return (self.lmax + 1) ** 2

    def conv2_paths(self) -> list:
        """Live conv2 paths: second operand is a geometric harmonic Y_l (canonical key, active)."""
        offs, rows, koff, cgoff, boff = self.comp_off, [], 0, 0, 0
        for ref_idx, (l1, p1, l2, p2, l3, p3) in enumerate(all_paths(self.keys, self.lmax)):
            if (l2, p2) != canonical(l2):
                continue
            d1, d2, d3 = 2 * l1 + 1, 2 * l2 + 1, 2 * l3 + 1
            rows.append(dict(gate=ref_idx, o1=offs[(l1, p1)], d1=d1, oy=l2 * l2, d2=d2, oo=offs[(l3, p3)], d3=d3,
                             koff=koff, cgoff=cgoff, boff=boff, l=(l1, l2, l3)))
            koff += d3
            cgoff += d1 * d2 * d3
            boff += d1 * d3
        return rows

    def conv1_paths(self) -> list:
        """Live conv1 paths: (l, canonical) x (0e) -> (l, canonical); C(l,0,l) is the identity."""
        rows = []
        for ref_idx, (l1, p1, l2, p2, l3, p3) in enumerate(all_paths(self.keys, self.lmax)):
            if (l2, p2) == (0, 1) and (l1, p1) == canonical(l1) and l3 == l1:
                rows.append(dict(gate=ref_idx, oo=self.comp_off[(l1, p1)], d=2 * l1 + 1, oy=l1 * l1))
        return rows

    def n_ref_paths(self) -> int:
        return len(all_paths(self.keys, self.lmax))

    def cg_table(self) -> np.ndarray:
        """Concatenated normalised C[m1][m2][m3] of the live conv2 paths (float64)."""
        return np.concatenate([coupling(*r["l"]).reshape(-1) for r in self.conv2_paths()])


def layout_full(lmax: int) -> Layout:
    return Layout(f"full_l{lmax}", lmax, tuple(canonical(l) for l in range(lmax + 1)))


def layout_o3(lmax: int, keys) -> Layout:
    ks = tuple(sorted(set((int(l), int(p)) for l, p in keys), key=lambda k: (k[0], 0 if k[1] > 0 else 1)))
    tag = "".join(f"{l}{'e' if p > 0 else 'o'}" for l, p in ks)
    return Layout(f"o3_l{lmax}_{tag}", lmax, ks)


# Layouts compiled into the HIP library (the benchmark configurations and their test sizes).
COMPILED_LAYOUTS = [layout_full(2), layout_full(3), layout_o3(2, [(0, 1), (1, 1), (1, -1), (2, 1)])]
