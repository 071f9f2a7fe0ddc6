"""Radius graph with periodic images on the GPU: ``torch.ops.fsctep.neighbor_list`` (cell list,
``csrc/neighbors.hip``).

``radius_graph_pbc_gpu`` keeps the signature and the edge convention of the reference function of the
same name (``molecular_force_field/utils/graph_utils.py:192-257``): ``edge_src`` i, ``edge_dst`` j and
the integer image ``edge_shifts`` s (float64) of every pair with ``|pos[j] + s @ cell - pos[i]| < r``,
s in {-1, 0, 1} on periodic axes, self pairs only across images.  Edges come receiver-sorted (then by
source and image), so ``prepare_graph`` keeps their order.  The reference's ``max_num_neighbors`` cap
of torch_cluster is not applied (every pair within ``r`` is returned).
"""

from __future__ import annotations

import torch

from . import _lib

_lib.load_torch_ops()


def _pbc_flags(pbc) -> list[int]:
    if pbc is None:
        return [1, 1, 1]
    if isinstance(pbc, torch.Tensor):
        pbc = pbc.detach().cpu().reshape(-1).tolist()
    elif isinstance(pbc, bool):
        pbc = [pbc]
    pbc = [int(bool(p)) for p in pbc]
    if len(pbc) == 1:
        pbc = pbc * 3
    if len(pbc) != 3:
        raise ValueError(f"pbc must have length 3, got {len(pbc)}")
    return pbc


def radius_graph_pbc_gpu(pos: torch.Tensor, r: float, cell: torch.Tensor, max_num_neighbors: int | None = None,
                         pbc=None):
    """(edge_src, edge_dst, edge_shifts) of one periodic (or partly periodic) system, on pos's GPU."""
    del max_num_neighbors   # no cap: every pair within r
    cell = cell.to(pos.device)
    src, dst, shifts, _ = torch.ops.fsctep.neighbor_list(pos, cell, float(r), _pbc_flags(pbc))
    return src, dst, shifts


def neighbor_csr(pos: torch.Tensor, r: float, cell: torch.Tensor, pbc=None):
    """(edge_src, edge_dst, edge_shifts, dst_ptr): the same edges and their receiver CSR (N+1, int32)."""
    src, dst, shifts, dst_ptr = torch.ops.fsctep.neighbor_list(pos, cell.to(pos.device), float(r), _pbc_flags(pbc))
    return src, dst, shifts, dst_ptr
