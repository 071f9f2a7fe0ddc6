"""Sparse-Cartesian ops: ``torch.ops.fsctep.sparse_*``.

The ops are registered in C++ by ``libfsctep_torch.so`` (``csrc/torch_ops.cpp``): a device kernel
over the C ABI of ``libfsctep_hip.so`` launched on the current stream, a Meta kernel (shapes only,
for ``make_fx`` / ``torch.export`` / tracing) and an autograd kernel whose backward is itself an op.
There is no CPU implementation: calling an op with CPU tensors raises.  Parameter gradients are produced
only by the conv2..n op, for the last radial layer passed as w_last / b_last (training; its backward is
differentiable once, for force losses); the other ops serve energy + forces.

    sparse_prepare_weights(w_last, b_last, channels) -> (bk1, bk6)
    sparse_conv(x, h, n, bk1, bk6, dst_ptr, src_ptr, src_perm, edge_dst, node_order, precision=0,
                w_last=None, b_last=None) -> (out, S, P)
    sparse_conv_backward(grad_out, h, n, bk6, S, P, dst_ptr, src_ptr, src_perm, edge_dst, node_order, precision=0)
        -> (dx, dh, dn, dS)
        precision 0: fp32-accurate products; 1: the bf16 channel-mix variant (one bf16 MFMA per product)
    sparse_conv_direction(P, n, u, dst_ptr, channels), sparse_conv_direction_backward(...): the derivative of
        the receiver assembly along edge directions u and its gradients (double backward)
    sparse_conv1_pair_table(w_last, b_last, atom_table, channels) -> (mf, mb)
    sparse_conv1(h, n, mf, mb, dst_ptr, pair_tiles, channels) -> (out, Q)
    sparse_conv1_backward(grad_out, n, mf, Q, dst_ptr, pair_tiles) -> (dh, dn)
    graph_prepare(edge_src, edge_dst, species, n_species) -> [order, src32, dst32, dst_ptr, src_ptr,
                                                              src_perm, node_species, edge_pair, pair_tiles, status]
    edge_geometry(pos, shift, edge_src, edge_dst, dst_ptr, src_ptr, src_perm) -> (n, r)
    edge_vec_geometry(edge_vec, order) -> (n, r)
    spatial_order(pos) -> node_order (N,) int32, the Morton order of the atoms (empty node_order: identity)
    radial_mlp(r, w0, b0, w2, b2, w4?, b4?, r_cut, basis) -> h (E,64) or the fused last Linear (E,P)

Sizes are read from the tensors inside the ops (the conv2..n normalisation 1/max(E/N, 1e-8) included),
so a traced graph holds no size constants.
"""

from __future__ import annotations

from . import _lib

_lib.load_torch_ops()

import torch  # noqa: E402


def sparse_conv_apply(x, h, n, bk1, bk6, graph, precision: int = 0, w_last=None, b_last=None):
    """Differentiable conv2..n message passing: (N,13,C) -> (N,13,C), normalised by 1/max(E/N, 1e-8).
    With ``w_last``/``b_last`` (the layer bk1/bk6 were prepared from) their gradients are produced too."""
    out, _, _ = torch.ops.fsctep.sparse_conv(x, h, n, bk1, bk6, graph.dst_ptr, graph.src_ptr,
                                             graph.src_perm, graph.dst32, graph.node_order, int(precision),
                                             w_last, b_last)
    return out


def sparse_conv1_apply(h, n, mf, mb, graph, channels: int):
    """Differentiable conv1 message passing from the species-pair tables: -> (N,13,C)."""
    out, _ = torch.ops.fsctep.sparse_conv1(h, n, mf, mb, graph.dst_ptr, graph.pair_tiles, int(channels))
    return out


# radial bases of e3nn's soft_one_hot_linspace that the reference offers (cli/train.py:589-590)
BASIS = {"bessel": 0, "gaussian": 1, "fourier": 2, "cosine": 3, "smooth_finite": 4}


def check_basis(basis: str) -> int:
    """The kernel code of a radial basis name; raises for a name the reference does not offer."""
    if basis not in BASIS:
        raise ValueError(f"radial basis {basis!r}: expected one of {sorted(BASIS)}")
    return BASIS[basis]


def edge_geometry(pos, shift_vec, graph):
    """Differentiable (w.r.t. ``pos``) unit vectors n (E,3) and lengths r (E,) of the receiver-sorted edges;
    ``shift_vec`` = edge_shifts @ cell (no gradient)."""
    return torch.ops.fsctep.edge_geometry(pos, shift_vec.detach(), graph.src32, graph.dst32, graph.dst_ptr,
                                          graph.src_ptr, graph.src_perm)


def edge_vec_geometry(edge_vec, graph):
    """Differentiable (w.r.t. ``edge_vec``, given in the caller's edge order) unit vectors n (E,3) and
    lengths r (E,) of the receiver-sorted edges."""
    return torch.ops.fsctep.edge_vec_geometry(edge_vec, graph.order)


def radial_hidden(r, fc, r_cut: float, basis: str):
    """fc[:4](radial_basis(r)) = silu(fc[2](silu(fc[0](emb)))) on the device: (E, 64)."""
    return torch.ops.fsctep.radial_mlp(r, fc[0].weight.detach(), fc[0].bias.detach(), fc[2].weight.detach(),
                                       fc[2].bias.detach(), None, None, float(r_cut), check_basis(basis))


def radial_full(r, fc, r_cut: float, basis: str):
    """The whole radial MLP fc(radial_basis(r)) including its last Linear (<= 64 outputs): (E, P)."""
    return torch.ops.fsctep.radial_mlp(r, fc[0].weight.detach(), fc[0].bias.detach(), fc[2].weight.detach(),
                                       fc[2].bias.detach(), fc[4].weight.detach(), fc[4].bias.detach(),
                                       float(r_cut), check_basis(basis))
