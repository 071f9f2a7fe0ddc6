"""Receiver-sorted graph structures consumed by the kernels, built on the device.

``prepare_graph`` runs ``torch.ops.fsctep.graph_prepare`` (``fsc_graph_prepare``): the stable receiver
sort of the reference's edge arrays (``edge_src``, ``edge_dst``, ``edge_shifts``), the receiver CSR, the
source grouping, and the species-pair ids and tiles.  The reference sorts on every call
(``models/pure_cartesian_sparse_layers.py:745-748``, ``models/pure_cartesian_ictd_layers_full.py:896-899``);
the trunks' ``forward`` does the same through this function.  Nothing here synchronises the host and
every tensor's size follows from (N, E, n_species), so the preparation can sit inside a traced graph.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib

_lib.load_torch_ops()


@dataclass
class Graph:
    order: torch.Tensor        # (E,) int32: receiver-sorted position -> input edge id
    src32: torch.Tensor        # (E,) int32 source of each receiver-sorted edge
    dst32: torch.Tensor        # (E,) int32 receiver, non-decreasing
    dst_ptr: torch.Tensor      # (N+1,) int32 receiver CSR
    src_ptr: torch.Tensor      # (N+1,) int32 source CSR over src_perm
    src_perm: torch.Tensor     # (E,) int32 receiver-sorted ids grouped by source (ascending within a source)
    shifts: torch.Tensor       # (E, 3) float, receiver-sorted
    node_species: torch.Tensor  # (N,) int32 species-table row of each node (empty without species)
    edge_pair: torch.Tensor    # (E,) int32 species pair node_species[src]*n_species + node_species[dst]
    pair_tiles: torch.Tensor   # (17*T,) int32: edge ids by pair in 16-tiles | tile pairs (unused tiles last)
    status: torch.Tensor       # (1,) int32: nonzero if an edge or species id was out of range
    n_species: int = 0
    node_order: torch.Tensor | None = None   # (N,) int32 spatial order of the nodes, or empty (identity)

    @property
    def n_nodes(self) -> int:
        return int(self.dst_ptr.shape[0]) - 1

    @property
    def n_edges(self) -> int:
        return int(self.src32.shape[0])

    @property
    def src(self) -> torch.Tensor:
        return self.src32.long()

    @property
    def dst(self) -> torch.Tensor:
        return self.dst32.long()


def prepare_graph(edge_src: torch.Tensor, edge_dst: torch.Tensor, edge_shifts: torch.Tensor,
                  n_nodes: int | None = None, species: torch.Tensor | None = None, n_species: int = 0,
                  pos: torch.Tensor | None = None) -> Graph:
    """Stable receiver sort and index structures of one neighbour list.

    ``species`` (N,) holds the atomic numbers used as rows of the model's species table of
    ``n_species`` rows (<= 16); without species pass ``n_nodes`` (the pair structures stay empty).
    With ``pos`` (N, 3) the graph also carries the spatial order of the atoms, which the per-node
    kernels walk (XCD by XCD) so that neighbouring blocks share gathered rows in L2; results do not
    depend on it."""
    if species is None:
        if n_nodes is None:
            raise ValueError("prepare_graph needs species or n_nodes")
        species = torch.zeros(int(n_nodes), dtype=torch.long, device=edge_dst.device)
        n_species = 0
    elif n_nodes is not None and int(n_nodes) != species.shape[0]:
        raise ValueError(f"n_nodes {n_nodes} != len(species) {species.shape[0]}")
    (order, src32, dst32, dst_ptr, src_ptr, src_perm, node_species, edge_pair, pair_tiles,
     status) = torch.ops.fsctep.graph_prepare(edge_src, edge_dst, species, int(n_species))
    shifts = edge_shifts.index_select(0, order)
    if pos is not None:
        node_order = torch.ops.fsctep.spatial_order(pos.detach())
    else:
        node_order = torch.empty(0, dtype=torch.int32, device=edge_dst.device)
    return Graph(order=order, src32=src32, dst32=dst32, dst_ptr=dst_ptr, src_ptr=src_ptr, src_perm=src_perm,
                 shifts=shifts, node_species=node_species, edge_pair=edge_pair, pair_tiles=pair_tiles,
                 status=status, n_species=int(n_species), node_order=node_order)


def poison_invalid(e: torch.Tensor, graph: Graph) -> torch.Tensor:
    """NaN energies when the graph preparation found an out-of-range edge or species id (the ids were
    clamped to keep every access in bounds), without a host synchronisation."""
    return e + torch.where(graph.status != 0, float("nan"), 0.0).to(e.dtype)
