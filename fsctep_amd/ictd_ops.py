"""ICTD custom ops (``torch.ops.fsctep.ictd_*``) over the C ABI, and the kernel layout tables.

A layout (active irreps + live paths, see ``ictd_basis.Layout``) is turned into the C struct
``FscIctdLayout`` once and registered under an integer id that the ops carry.
"""

from __future__ import annotations

import ctypes

import numpy as np
import torch
from torch import Tensor

from . import _lib
from .ictd_basis import Layout

_i32 = ctypes.c_int32


class FscIctdLayout(ctypes.Structure):
    _fields_ = [(n, _i32) for n in ("M", "NY", "KT", "NP", "NG", "NREF", "NBGP", "KTT")] + \
        [(n, _i32 * 8) for n in ("g_o1", "g_d1", "g_kstart", "g_kcount", "g_kpad", "g_bgoff", "g_tile0")] + \
        [("tile_group", _i32 * 16)] + \
        [(n, _i32 * 64) for n in ("p_gate", "p_oy", "p_d2", "p_d3", "p_koff", "p_cgoff", "p_group", "p_oo")] + \
        [("kk_path", _i32 * 128), ("NK", _i32), ("k_oo", _i32 * 16), ("k_d", _i32 * 16),
         ("NP1", _i32), ("y_path1", _i32 * 16), ("y_oo1", _i32 * 16), ("c1_gate", _i32 * 16)]


def build_layout_struct(lay: Layout) -> FscIctdLayout:
    paths = lay.conv2_paths()
    s = FscIctdLayout()
    s.M, s.NY, s.NREF = lay.M, lay.NY, lay.n_ref_paths()
    s.NP = len(paths)
    s.KT = sum(p["d3"] for p in paths)
    groups = []
    for i, p in enumerate(paths):
        if not groups or groups[-1]["o1"] != p["o1"]:
            groups.append(dict(o1=p["o1"], d1=p["d1"], kstart=p["koff"], kcount=0, paths=[]))
        groups[-1]["kcount"] += p["d3"]
        groups[-1]["paths"].append(i)
    bgoff = tile0 = 0
    tiles = []
    for gi, g in enumerate(groups):
        g["kpad"] = 16 * ((g["kcount"] + 15) // 16)
        g["bgoff"], g["tile0"] = bgoff, tile0
        bgoff += g["d1"] * g["kpad"]
        tile0 += g["kpad"] // 16
        tiles += [gi] * (g["kpad"] // 16)
        for name in ("o1", "d1", "kstart", "kcount", "kpad", "bgoff", "tile0"):
            getattr(s, "g_" + name)[gi] = g[name]
    s.NG, s.NBGP, s.KTT = len(groups), bgoff, tile0
    for t, gi in enumerate(tiles):
        s.tile_group[t] = gi
    for i, p in enumerate(paths):
        s.p_gate[i], s.p_oy[i], s.p_d2[i], s.p_d3[i] = p["gate"], p["oy"], p["d2"], p["d3"]
        s.p_koff[i], s.p_cgoff[i], s.p_oo[i] = p["koff"], p["cgoff"], p["oo"]
        s.p_group[i] = next(gi for gi, g in enumerate(groups) if i in g["paths"])
        for k in range(p["d3"]):
            s.kk_path[p["koff"] + k] = i
    offs = lay.comp_off
    s.NK = len(lay.keys)
    for i, k in enumerate(lay.keys):
        s.k_oo[i], s.k_d[i] = offs[k], 2 * k[0] + 1
    c1 = lay.conv1_paths()
    s.NP1 = len(c1)
    for y in range(16):
        s.y_path1[y] = -1
    for i, p in enumerate(c1):
        s.c1_gate[i] = p["gate"]
        for k in range(p["d"]):
            s.y_path1[p["oy"] + k] = i
            s.y_oo1[p["oy"] + k] = p["oo"] + k
    if sum(g["d1"] for g in groups) != lay.M:
        raise ValueError(f"layout {lay.name}: every input irrep needs a live tensor-product path")
    return s


_LAYOUTS: list = []


def register_layout(lay: Layout) -> int:
    """Id of the C layout table for ``lay`` (built once)."""
    for i, (name, _, _) in enumerate(_LAYOUTS):
        if name == lay.name:
            return i
    _LAYOUTS.append((lay.name, lay, build_layout_struct(lay)))
    return len(_LAYOUTS) - 1


def layout_struct(layout_id: int) -> FscIctdLayout:
    return _LAYOUTS[layout_id][2]


def _ref(layout_id: int) -> int:
    return ctypes.addressof(layout_struct(layout_id))


def _require_cuda(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise RuntimeError("fsctep ops run on the GPU only (HIP kernels); got a CPU tensor")


def _c(t: Tensor) -> Tensor:
    t = t if t.dtype == torch.float32 else t.float()
    return t if t.is_contiguous() else t.contiguous()


# ----------------------------------------------------------------------------- conv2..n

@torch.library.custom_op("fsctep::ictd_prepare_weights", mutates_args=())
def ictd_prepare_weights(W: Tensor) -> Tensor:
    _require_cuda(W)
    P, C = W.shape[0], W.shape[1]
    Wc = _c(W.reshape(P, C, C))
    Wt = torch.empty_like(Wc)
    _lib.call("fsc_ictd_prepare_weights", _lib.ptr(Wc), P, C, _lib.ptr(Wt), _lib.stream_handle(W.device))
    return Wt


@ictd_prepare_weights.register_fake
def _(W):
    return W.new_empty(W.shape[0], W.shape[1], W.shape[1])


@torch.library.custom_op("fsctep::ictd_conv", mutates_args=())
def ictd_conv(x: Tensor, Y: Tensor, gates: Tensor, W: Tensor, Wt: Tensor, cg: Tensor, dst_ptr: Tensor,
              edge_src: Tensor, src_ptr: Tensor, src_perm: Tensor, layout_id: int) -> Tensor:
    """x (N,M,C), Y (E,NY), gates (E,NREF), W (NREF,C,C[,1]) -> (N,M,C).  Wt, src_ptr, src_perm: backward."""
    _require_cuda(x, Y, gates, W, cg)
    L = layout_struct(layout_id)
    N, M, C = x.shape
    E = Y.shape[0]
    x, Y, gates = _c(x), _c(Y), _c(gates)
    W = _c(W.reshape(W.shape[0], C, C))
    z = torch.empty(N, L.KT, C, device=x.device, dtype=torch.float32)
    out = torch.empty(N, M, C, device=x.device, dtype=torch.float32)
    _lib.call("fsc_ictd_conv_forward", _ref(layout_id), N, E, C, _lib.ptr(dst_ptr), _lib.ptr(edge_src),
              _lib.ptr(x), _lib.ptr(Y), _lib.ptr(gates), _lib.ptr(cg), _lib.ptr(W), _lib.ptr(z), _lib.ptr(out),
              _lib.stream_handle(x.device))
    return out


@ictd_conv.register_fake
def _(x, Y, gates, W, Wt, cg, dst_ptr, edge_src, src_ptr, src_perm, layout_id):
    return torch.empty_like(x)


@torch.library.custom_op("fsctep::ictd_conv_backward", mutates_args=())
def ictd_conv_backward(grad_out: Tensor, x: Tensor, Y: Tensor, gates: Tensor, Wt: Tensor, cg: Tensor,
                       dst_ptr: Tensor, edge_src: Tensor, src_ptr: Tensor, src_perm: Tensor,
                       layout_id: int) -> tuple[Tensor, Tensor, Tensor]:
    _require_cuda(grad_out, x, Y, gates, Wt, cg)
    L = layout_struct(layout_id)
    N, M, C = x.shape
    E = Y.shape[0]
    g, x, Y, gates = _c(grad_out), _c(x), _c(Y), _c(gates)
    dz = torch.empty(N, L.KT, C, device=x.device, dtype=torch.float32)
    dxe = torch.empty(E, M, C, device=x.device, dtype=torch.float32)
    dx = torch.empty(N, M, C, device=x.device, dtype=torch.float32)
    dgates = torch.zeros(E, L.NREF, device=x.device, dtype=torch.float32)
    dY = torch.empty(E, L.NY, device=x.device, dtype=torch.float32)
    _lib.call("fsc_ictd_conv_backward", _ref(layout_id), N, E, C, _lib.ptr(dst_ptr), _lib.ptr(edge_src),
              _lib.ptr(src_ptr), _lib.ptr(src_perm), _lib.ptr(g), _lib.ptr(x), _lib.ptr(Y), _lib.ptr(gates),
              _lib.ptr(cg), _lib.ptr(Wt), _lib.ptr(dz), _lib.ptr(dxe), _lib.ptr(dx), _lib.ptr(dgates),
              _lib.ptr(dY), _lib.stream_handle(x.device))
    return dx, dgates, dY


@ictd_conv_backward.register_fake
def _(grad_out, x, Y, gates, Wt, cg, dst_ptr, edge_src, src_ptr, src_perm, layout_id):
    return torch.empty_like(x), torch.empty_like(gates), torch.empty_like(Y)


def _ictd_conv_setup(ctx, inputs, output):
    x, Y, gates, W, Wt, cg, dst_ptr, edge_src, src_ptr, src_perm, layout_id = inputs
    ctx.save_for_backward(x, Y, gates, Wt, cg, dst_ptr, edge_src, src_ptr, src_perm)
    ctx.layout_id = layout_id


def _ictd_conv_bwd(ctx, grad_out):
    x, Y, gates, Wt, cg, dst_ptr, edge_src, src_ptr, src_perm = ctx.saved_tensors
    if ctx.needs_input_grad[3] or ctx.needs_input_grad[4] or ctx.needs_input_grad[5]:
        raise NotImplementedError("parameter gradients of the ICTD conv are not implemented "
                                  "(energy/force inference only)")
    dx, dgates, dY = torch.ops.fsctep.ictd_conv_backward(grad_out, x, Y, gates, Wt, cg, dst_ptr, edge_src,
                                                         src_ptr, src_perm, ctx.layout_id)
    return dx, dY, dgates, None, None, None, None, None, None, None, None


torch.library.register_autograd("fsctep::ictd_conv", _ictd_conv_bwd, setup_context=_ictd_conv_setup)


def ictd_conv_apply(x, Y, gates, W, Wt, cg, graph, layout_id: int):
    return torch.ops.fsctep.ictd_conv(x, Y, gates, W, Wt, cg, graph.dst_ptr, graph.src32, graph.src_ptr,
                                      graph.src_perm, int(layout_id))


# ----------------------------------------------------------------------------- conv1

@torch.library.custom_op("fsctep::ictd_conv1", mutates_args=())
def ictd_conv1(F: Tensor, gates: Tensor, qtab: Tensor, dst_ptr: Tensor, edge_pair: Tensor, node_species: Tensor,
               n_nodes: int, n_species: int, layout_id: int) -> Tensor:
    """F (E,NY) harmonics (+ field), gates (E,NREF), qtab (NS*NS,NP1,C) -> (N,M,C)."""
    _require_cuda(F, gates, qtab)
    L = layout_struct(layout_id)
    C = qtab.shape[-1]
    E = F.shape[0]
    F, gates, qtab = _c(F), _c(gates), _c(qtab)
    out = torch.empty(n_nodes, L.M, C, device=F.device, dtype=torch.float32)
    _lib.call("fsc_ictd_conv1_forward", _ref(layout_id), n_nodes, E, C, _lib.ptr(dst_ptr), _lib.ptr(edge_pair),
              _lib.ptr(F), _lib.ptr(gates), _lib.ptr(qtab), _lib.ptr(out), _lib.stream_handle(F.device))
    return out


@ictd_conv1.register_fake
def _(F, gates, qtab, dst_ptr, edge_pair, node_species, n_nodes, n_species, layout_id):
    return F.new_empty(n_nodes, layout_struct(layout_id).M, qtab.shape[-1])


@torch.library.custom_op("fsctep::ictd_conv1_backward", mutates_args=())
def ictd_conv1_backward(grad_out: Tensor, F: Tensor, gates: Tensor, qtab: Tensor, dst_ptr: Tensor,
                        edge_pair: Tensor, node_species: Tensor, n_species: int,
                        layout_id: int) -> tuple[Tensor, Tensor]:
    _require_cuda(grad_out, F, gates, qtab)
    N, M, C = grad_out.shape
    E = F.shape[0]
    g, F, gates, qtab = _c(grad_out), _c(F), _c(gates), _c(qtab)
    dF = torch.empty_like(F)
    dgates = torch.zeros_like(gates)
    _lib.call("fsc_ictd_conv1_backward", _ref(layout_id), N, E, C, n_species, _lib.ptr(dst_ptr),
              _lib.ptr(edge_pair), _lib.ptr(node_species), _lib.ptr(g), _lib.ptr(F), _lib.ptr(gates),
              _lib.ptr(qtab), _lib.ptr(dF), _lib.ptr(dgates), _lib.stream_handle(F.device))
    return dF, dgates


@ictd_conv1_backward.register_fake
def _(grad_out, F, gates, qtab, dst_ptr, edge_pair, node_species, n_species, layout_id):
    return torch.empty_like(F), torch.empty_like(gates)


def _ictd_conv1_setup(ctx, inputs, output):
    F, gates, qtab, dst_ptr, edge_pair, node_species, n_nodes, n_species, layout_id = inputs
    ctx.save_for_backward(F, gates, qtab, dst_ptr, edge_pair, node_species)
    ctx.n_species, ctx.layout_id = n_species, layout_id


def _ictd_conv1_bwd(ctx, grad_out):
    F, gates, qtab, dst_ptr, edge_pair, node_species = ctx.saved_tensors
    if ctx.needs_input_grad[2]:
        raise NotImplementedError("parameter gradients of the ICTD conv1 are not implemented")
    dF, dgates = torch.ops.fsctep.ictd_conv1_backward(grad_out, F, gates, qtab, dst_ptr, edge_pair, node_species,
                                                      ctx.n_species, ctx.layout_id)
    return dF, dgates, None, None, None, None, None, None, None


torch.library.register_autograd("fsctep::ictd_conv1", _ictd_conv1_bwd, setup_context=_ictd_conv1_setup)


def ictd_conv1_apply(F, gates, qtab, graph, layout_id: int):
    return torch.ops.fsctep.ictd_conv1(F, gates, qtab, graph.dst_ptr, graph.edge_pair, graph.species_index32,
                                       graph.n_nodes, int(graph.species.shape[0]), int(layout_id))
