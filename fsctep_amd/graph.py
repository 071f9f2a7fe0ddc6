"""Receiver-sorted graph structures consumed by the kernels.

Built once per neighbour list (as in MD between list rebuilds) from the reference's
edge arrays (``edge_src``, ``edge_dst``, ``edge_shifts``; ``models/pure_cartesian_sparse_layers.py:745-748``
sorts them by receiver on every call, here the sort is hoisted out of the step).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass
class Graph:
    n_nodes: int
    n_edges: int
    src: torch.Tensor          # (E,) int64, receiver-sorted
    dst: torch.Tensor          # (E,) int64, non-decreasing
    shifts: torch.Tensor       # (E, 3) float, receiver-sorted
    dst_ptr: torch.Tensor      # (N+1,) int32 receiver CSR
    src_ptr: torch.Tensor      # (N+1,) int32 source CSR over src_perm
    src_perm: torch.Tensor     # (E,) int32 receiver-sorted ids grouped by source (stable)
    dst32: torch.Tensor        # (E,) int32
    src32: torch.Tensor        # (E,) int32
    in_degree: torch.Tensor    # (N,) int64
    species_index: torch.Tensor | None = None   # (N,) int64 index into `species`
    species: torch.Tensor | None = None         # (S,) int64 distinct atomic numbers (sorted)
    edge_pair: torch.Tensor | None = None       # (E,) int32 species-pair index src*S+dst
    pair_tiles: torch.Tensor | None = None      # (17*T,) int32: edge ids by pair in 16-tiles | tile pairs
    species_index32: torch.Tensor | None = None # (N,) int32


def prepare_graph(edge_src: torch.Tensor, edge_dst: torch.Tensor, edge_shifts: torch.Tensor,
                  n_nodes: int, species: torch.Tensor | None = None) -> Graph:
    """Sort by receiver (stable) and build the CSR / source-grouped permutations."""
    dev = edge_dst.device
    E = int(edge_dst.shape[0])
    if E >= 2 ** 31 or n_nodes >= 2 ** 31:
        raise ValueError("graph exceeds int32 indexing")
    order = torch.argsort(edge_dst, stable=True)
    src = edge_src[order].long().contiguous()
    dst = edge_dst[order].long().contiguous()
    shifts = edge_shifts[order].contiguous()
    deg = torch.bincount(dst, minlength=n_nodes) if E else torch.zeros(n_nodes, dtype=torch.long, device=dev)
    dst_ptr = torch.zeros(n_nodes + 1, dtype=torch.int64, device=dev)
    dst_ptr[1:] = torch.cumsum(deg, 0)
    src_perm = torch.argsort(src, stable=True) if E else torch.zeros(0, dtype=torch.long, device=dev)
    odeg = torch.bincount(src, minlength=n_nodes) if E else torch.zeros(n_nodes, dtype=torch.long, device=dev)
    src_ptr = torch.zeros(n_nodes + 1, dtype=torch.int64, device=dev)
    src_ptr[1:] = torch.cumsum(odeg, 0)
    g = Graph(n_nodes=n_nodes, n_edges=E, src=src, dst=dst, shifts=shifts,
              dst_ptr=dst_ptr.to(torch.int32), src_ptr=src_ptr.to(torch.int32),
              src_perm=src_perm.to(torch.int32).contiguous(), dst32=dst.to(torch.int32),
              src32=src.to(torch.int32), in_degree=deg)
    if species is not None:
        uniq, inv = torch.unique(species.long(), sorted=True, return_inverse=True)
        g.species = uniq
        g.species_index = inv
        g.species_index32 = inv.to(torch.int32).contiguous()
        S = int(uniq.shape[0])
        g.edge_pair = (inv[src] * S + inv[dst]).to(torch.int32).contiguous()
        g.pair_tiles = pair_tiles(g.edge_pair, S * S)
    return g


def pair_tiles(edge_pair: torch.Tensor, n_pairs: int) -> torch.Tensor:
    """Edge ids grouped by species pair, each group padded with -1 to a multiple of 16, followed by
    the pair of each 16-entry tile: [16*T ids | T pairs] (int32).  The sparse conv1 runs one small
    GEMM per tile with that pair's table."""
    dev = edge_pair.device
    E = int(edge_pair.shape[0])
    pair = edge_pair.long()
    counts = torch.bincount(pair, minlength=n_pairs) if E else torch.zeros(n_pairs, dtype=torch.long, device=dev)
    tiles_per = (counts + 15) // 16
    T = int(tiles_per.sum())
    tile_start = torch.cumsum(tiles_per, 0) - tiles_per            # first tile of each pair
    order = torch.argsort(pair, stable=True) if E else torch.zeros(0, dtype=torch.long, device=dev)
    sorted_pair = pair[order]
    first = torch.cumsum(counts, 0) - counts                        # first sorted position of each pair
    pos = tile_start[sorted_pair] * 16 + (torch.arange(E, device=dev) - first[sorted_pair])
    ids = torch.full((16 * T,), -1, dtype=torch.int32, device=dev)
    ids[pos] = order.to(torch.int32)
    tpair = torch.repeat_interleave(torch.arange(n_pairs, device=dev), tiles_per).to(torch.int32)
    return torch.cat([ids, tpair]).contiguous()
