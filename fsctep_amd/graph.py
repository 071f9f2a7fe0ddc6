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
    species_z: torch.Tensor | None = None    # (n_species,) int64 atomic number of each species-table row,
    #                                          or None: row i is atomic number i

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


TABLE_ROWS = 16   # species-table rows the conv kernels take


def map_species(A: torch.Tensor, max_atomvalue: int, rows: int = TABLE_ROWS):
    """Atomic numbers -> rows of a species table of at most ``rows`` entries, on the device.

    The reference embeds atomic numbers 0..max_atomvalue-1 (``nn.Embedding(max_atomvalue, ...)``); the
    kernels take at most 16 table rows.  The species present get rows in ascending atomic number: a
    presence bitmap over the max_atomvalue numbers, then its prefix sum.  Returns (node rows (N,) int64,
    atomic number of each row (rows,) int64, status (1,) int32: 2 if an atomic number lies outside
    0..max_atomvalue-1, 4 if more than ``rows`` species are present).  No host synchronisation."""
    Z = int(max_atomvalue)
    a = A.long()
    dev = a.device
    ac = a.clamp(0, Z - 1)
    present = torch.zeros(Z, dtype=torch.int32, device=dev).index_fill_(0, ac, 1)
    row_of_z = torch.cumsum(present, 0) - 1                      # int64; row of each present number
    node_rows = row_of_z.index_select(0, ac).clamp_(0, rows - 1)
    slot = torch.where((present > 0) & (row_of_z < rows), row_of_z, torch.full_like(row_of_z, rows))
    # every present number lands in its own slot; the absent ones all land in the spare slot `rows`
    species_z = torch.zeros(rows + 1, dtype=torch.long, device=dev).scatter_(
        0, slot, torch.arange(Z, device=dev))[:rows]
    out_of_range = ((a < 0) | (a >= Z)).any().to(torch.int32) * 2
    too_many = (row_of_z[-1] >= rows).to(torch.int32) * 4
    return node_rows, species_z, (out_of_range | too_many).view(1)


def prepare_species_graph(edge_src: torch.Tensor, edge_dst: torch.Tensor, edge_shifts: torch.Tensor,
                          A: torch.Tensor, max_atomvalue: int, pos: torch.Tensor | None = None) -> Graph:
    """``prepare_graph`` for a model whose species table has ``max_atomvalue`` rows: up to 16 rows the
    atomic number is the row; beyond, the species present are mapped to at most 16 rows (map_species)."""
    if int(max_atomvalue) <= TABLE_ROWS:
        return prepare_graph(edge_src, edge_dst, edge_shifts, A.shape[0], species=A, n_species=int(max_atomvalue),
                             pos=pos)
    rows, species_z, st = map_species(A, max_atomvalue)
    g = prepare_graph(edge_src, edge_dst, edge_shifts, A.shape[0], species=rows, n_species=TABLE_ROWS, pos=pos)
    g.status = g.status | st
    g.species_z = species_z
    return g


def species_rows(graph: Graph, device) -> torch.Tensor:
    """Atomic number of each species-table row of ``graph`` (the argument of the atom embedding)."""
    if graph.species_z is not None:
        return graph.species_z
    return torch.arange(graph.n_species, device=device)


def poison_invalid(e: torch.Tensor, graph: Graph, pos: torch.Tensor | None = None,
                   edge_vec: torch.Tensor | None = None) -> torch.Tensor:
    """NaN energies when the graph preparation found an out-of-range edge or species id (the ids were
    clamped to keep every access in bounds), without a host synchronisation.  The same NaN, times the
    differentiated input (``pos`` (N, 3), or ``edge_vec`` (E, 3) in the caller's edge order, gathered to
    the receivers), is added to every atom's energy, so the gradients, i.e. the forces, are NaN too.
    No reduction across atoms: the step stays free of multi-block reductions."""
    bad = torch.where(graph.status != 0, float("nan"), 0.0).to(e.dtype)
    out = e + bad
    # unconditional (not only when the input requires grad), so a traced graph keeps the terms
    if pos is not None:
        out = out + (bad * pos.to(e.dtype)).sum(-1, keepdim=True)
    if edge_vec is not None:
        v = (bad * edge_vec.to(e.dtype)).sum(-1, keepdim=True).index_select(0, graph.order.long())
        out = out + torch.zeros_like(e).index_add(0, graph.dst, v)
    return out
