"""Seeded synthetic atomic systems and seeded model parameters.

The benchmark workloads are random atomic systems, not datasets:

* positions by random sequential addition in a cubic box (periodic or not),
  rejecting any candidate closer than ``min_dist`` to an accepted atom;
* species drawn uniformly from a fixed list of atomic numbers;
* the radius graph: every ordered pair (src, dst, shift) with
  ``|pos[dst] - pos[src] + shift @ cell| < cutoff``, shifts in {-1, 0, 1}^3
  (the convention of ``utils/graph_utils.py:192-257`` and
  ``models/pure_cartesian_sparse_layers.py:751-756``), sorted by receiver.

Parameters are drawn per state_dict key from an independent PCG64 stream
seeded by ``(seed, crc32(key))``, so any implementation that shares the
reference's state_dict keys and shapes gets bit-identical values without
sharing initialisation order.  The tensors the reference initialises to zero
(``weighted_sum.weights``, ``external_tensor_scale_*``) get random values too,
otherwise energies and forces would be identically zero.
"""

from __future__ import annotations

import math
import zlib
from dataclasses import dataclass

import numpy as np

SPECIES_4 = (1, 6, 7, 8)
SPECIES_8 = (1, 2, 3, 4, 5, 6, 7, 8)


@dataclass
class AtomicSystem:
    """One periodic or open system with its receiver-sorted radius graph."""

    pos: np.ndarray          # (N, 3) float64, Angstrom
    species: np.ndarray      # (N,) int64 atomic numbers
    cell: np.ndarray         # (1, 3, 3) float64, rows are lattice vectors
    periodic: bool
    edge_src: np.ndarray     # (E,) int64
    edge_dst: np.ndarray     # (E,) int64, non-decreasing
    edge_shifts: np.ndarray  # (E, 3) float64 integer-valued image shifts

    @property
    def num_atoms(self) -> int:
        return int(self.pos.shape[0])

    @property
    def num_edges(self) -> int:
        return int(self.edge_src.shape[0])


def random_positions(n: int, box: float, min_dist: float, periodic: bool,
                     rng: np.random.Generator, max_tries: int = 2000) -> np.ndarray:
    """Random sequential addition with a cell grid for the exclusion test."""
    ncell = max(1, int(box // min_dist))
    csize = box / ncell
    grid: dict[tuple[int, int, int], list[int]] = {}
    pos = np.empty((n, 3), dtype=np.float64)
    md2 = min_dist * min_dist
    k = 0
    while k < n:
        for _ in range(max_tries):
            cand = rng.random(3) * box
            ci = tuple(int(v) % ncell for v in (cand // csize))
            ok = True
            for dx in (-1, 0, 1):
                for dy in (-1, 0, 1):
                    for dz in (-1, 0, 1):
                        nb = (ci[0] + dx, ci[1] + dy, ci[2] + dz)
                        if periodic:
                            nb = (nb[0] % ncell, nb[1] % ncell, nb[2] % ncell)
                        elif min(nb) < 0 or max(nb) >= ncell:
                            continue
                        for j in grid.get(nb, ()):
                            d = pos[j] - cand
                            if periodic:
                                d -= box * np.round(d / box)
                            if d @ d < md2:
                                ok = False
                                break
                        if not ok:
                            break
                    if not ok:
                        break
                if not ok:
                    break
            if ok:
                pos[k] = cand
                grid.setdefault(ci, []).append(k)
                k += 1
                break
        else:
            raise RuntimeError(f"random sequential addition stalled at {k}/{n} atoms")
    return pos


def radius_graph(pos: np.ndarray, cell: np.ndarray, periodic: bool, cutoff: float):
    """All ordered pairs within ``cutoff``; returns receiver-sorted (src, dst, shifts)."""
    n = pos.shape[0]
    lat = cell.reshape(3, 3)
    box = float(lat[0, 0])
    if periodic and box > 2.0 * cutoff + 1e-9:
        from scipy.spatial import cKDTree
        wrapped = np.mod(pos, box)
        tree = cKDTree(wrapped, boxsize=box)
        pairs = tree.query_pairs(cutoff, output_type="ndarray")
        i = np.concatenate([pairs[:, 0], pairs[:, 1]])
        j = np.concatenate([pairs[:, 1], pairs[:, 0]])
        d = pos[j] - pos[i]
        shifts = -np.round(d / box)
        vec = d + shifts * box
        keep = np.einsum("ij,ij->i", vec, vec) < cutoff * cutoff
        src, dst, sh = i[keep], j[keep], shifts[keep]
    elif not periodic:
        from scipy.spatial import cKDTree
        tree = cKDTree(pos)
        pairs = tree.query_pairs(cutoff, output_type="ndarray")
        src = np.concatenate([pairs[:, 0], pairs[:, 1]])
        dst = np.concatenate([pairs[:, 1], pairs[:, 0]])
        sh = np.zeros((src.shape[0], 3))
    else:
        # small periodic box: brute force over the 27 images
        srcs, dsts, shs = [], [], []
        for s in np.array(np.meshgrid([-1, 0, 1], [-1, 0, 1], [-1, 0, 1], indexing="ij")).reshape(3, -1).T:
            vec = pos[None, :, :] - pos[:, None, :] + (s @ lat)[None, None, :]
            d2 = np.einsum("ijk,ijk->ij", vec, vec)
            mask = d2 < cutoff * cutoff
            if not s.any():
                np.fill_diagonal(mask, False)
            ii, jj = np.nonzero(mask)
            srcs.append(ii)
            dsts.append(jj)
            shs.append(np.broadcast_to(s, (ii.shape[0], 3)))
        src = np.concatenate(srcs)
        dst = np.concatenate(dsts)
        sh = np.concatenate(shs).astype(np.float64)
    order = np.lexsort((sh[:, 2], sh[:, 1], sh[:, 0], src, dst))
    return (src[order].astype(np.int64), dst[order].astype(np.int64),
            np.ascontiguousarray(sh[order], dtype=np.float64))


def make_system(n_atoms: int, *, density: float | None = 0.1, box: float | None = None,
                periodic: bool = True, species=SPECIES_4, cutoff: float = 5.0,
                min_dist: float = 0.9, seed: int = 0) -> AtomicSystem:
    """Seeded system: box side from ``density`` (atoms/A^3) unless ``box`` is given."""
    rng = np.random.Generator(np.random.PCG64(seed))
    if box is None:
        box = (n_atoms / density) ** (1.0 / 3.0)
    pos = random_positions(n_atoms, box, min_dist, periodic, rng)
    spec = np.asarray(species, dtype=np.int64)[rng.integers(0, len(species), size=n_atoms)]
    cell = (np.eye(3) * (box if periodic else 100.0))[None]
    src, dst, sh = radius_graph(pos, cell, periodic, cutoff)
    return AtomicSystem(pos=pos, species=spec, cell=cell, periodic=periodic,
                        edge_src=src, edge_dst=dst, edge_shifts=sh)


def workload_system(name: str, n_atoms: int | None = None, seed: int | None = None) -> AtomicSystem:
    """The named benchmark systems (sizes and recipes of the benchmark configurations)."""
    if name == "sparse-32-open":
        return make_system(32 if n_atoms is None else n_atoms, box=10.0, periodic=False,
                           species=SPECIES_4, seed=11 if seed is None else seed)
    if name == "sparse-periodic":
        return make_system(1000 if n_atoms is None else n_atoms, density=0.1, periodic=True,
                           species=SPECIES_4, seed=22 if seed is None else seed)
    if name == "ictd-periodic":
        return make_system(10000 if n_atoms is None else n_atoms, density=0.1, periodic=True,
                           species=SPECIES_8, seed=33 if seed is None else seed)
    raise KeyError(name)


# --------------------------------------------------------------------------- parameters

def _key_rng(seed: int, key: str) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(np.random.SeedSequence([int(seed), zlib.crc32(key.encode())])))


def seeded_value(key: str, shape, seed: int) -> np.ndarray:
    """Deterministic float64 value for one state_dict entry.

    Scale rules: LayerNorm gain 1+0.1N, LayerNorm/Linear bias 0.1N, Linear weight
    N/sqrt(fan_in), per-path tensor-product weight (P, out, in1, in2) N/sqrt(in1*in2),
    embedding N, bilinear readout weights 0.02N, zero-initialised scalars (weighted
    sums, external-field scales) 0.1N.
    """
    rng = _key_rng(seed, key)
    shape = tuple(int(s) for s in shape)
    z = rng.standard_normal(shape) if shape else np.asarray(rng.standard_normal())
    leaf = key.rsplit(".", 1)[-1]
    owner = key.rsplit(".", 2)[-2] if key.count(".") >= 1 else ""
    is_norm = ("norm" in owner) or (".layer_norms." in key) or key.startswith("layer_norms.")
    if is_norm and leaf == "weight":
        return 1.0 + 0.1 * z
    if leaf == "bias":
        return 0.1 * z
    if "embedding" in key and leaf == "weight":
        return z
    if key.startswith(("product_3.W", "W_read.")) or ".product_3.W" in key:
        return 0.02 * z
    if leaf == "weight" and len(shape) == 2:
        return z / math.sqrt(shape[1])
    if leaf == "weight" and len(shape) >= 3:
        return z / math.sqrt(float(np.prod(shape[2:])))      # per-path (out, in1, in2): fan-in in1*in2
    return 0.1 * z


def seeded_state_dict(named_shapes, seed: int) -> dict[str, np.ndarray]:
    """``{key: float64 array}`` for an iterable of ``(key, shape)``."""
    return {k: seeded_value(k, s, seed) for k, s in named_shapes}


def apply_seeded_parameters(module, seed: int) -> None:
    """Overwrite every parameter of ``module`` with ``seeded_value(name, shape, seed)``."""
    import torch
    with torch.no_grad():
        for name, p in module.named_parameters():
            p.copy_(torch.from_numpy(seeded_value(name, tuple(p.shape), seed)).to(p.dtype))
