"""ICTD kernel layout tables and helpers over the ``torch.ops.fsctep.ictd_*`` ops.

A layout (active irreps + live paths, see ``ictd_basis.Layout``) is turned into the C struct
``FscIctdLayout`` once, registered under an integer id, and handed to the ops as the list of the
struct's int32 words (an ``int[]`` argument).  The ops are registered in C++ by ``libfsctep_torch.so``:

    ictd_prepare_weights(W) -> Wt   (split-fp16 channel-mix weights, opaque)
    ictd_conv(x, Y, gates, W, Wt, cg, dst_ptr, edge_src, src_ptr, src_perm, edge_dst, node_order, layout) -> out
    ictd_conv_backward(grad_out, x, Y, gates, Wt, cg, dst_ptr, edge_src, src_ptr, src_perm, edge_dst, node_order,
                       layout)
    ictd_conv1(F, gates, qtab, dst_ptr, edge_pair, node_species, n_species, n_comps, layout)
    ictd_conv1_backward(grad_out, F, gates, qtab, dst_ptr, edge_pair, node_species, n_species, layout)
"""

from __future__ import annotations

import ctypes

import numpy as np
import torch
from torch import Tensor

from . import _lib
from .ictd_basis import Layout
from .ops import edge_geometry, edge_vec_geometry, radial_full, radial_hidden  # noqa: F401  (shared geometry / radial ops)

_lib.load_torch_ops()

_i32 = ctypes.c_int32


class FscIctdLayout(ctypes.Structure):
    _fields_ = [(n, _i32) for n in ("M", "NY", "KT", "NP", "NG", "NREF", "NBGP", "KTT")] + \
        [(n, _i32 * 8) for n in ("g_o1", "g_d1", "g_kstart", "g_kcount", "g_kpad", "g_bgoff", "g_tile0")] + \
        [("tile_group", _i32 * 16)] + \
        [(n, _i32 * 64) for n in ("p_gate", "p_oy", "p_d2", "p_d3", "p_koff", "p_cgoff", "p_group", "p_oo")] + \
        [("kk_path", _i32 * 128), ("NK", _i32), ("k_oo", _i32 * 16), ("k_d", _i32 * 16),
         ("NP1", _i32), ("y_path1", _i32 * 16), ("y_oo1", _i32 * 16), ("c1_gate", _i32 * 16)]


def kernel_limits(lay: Layout) -> list:
    """What of ``lay`` exceeds the ICTD kernels' tables (empty: the kernels run it): at most 32 components
    and 16 harmonic components, 64 live paths and 128 kk rows, 8 path groups of at most 32 kk rows and 8 kk
    tiles in all, in the layout and in its dual (the paths reversed, grouped by output key)."""
    paths = lay.conv2_paths()
    out = []
    if lay.M > 32:
        out.append(f"{lay.M} components per channel (at most 32)")
    if lay.NY > 16:
        out.append(f"{lay.NY} harmonic components (at most 16, lmax <= 3)")
    if len(paths) > 64:
        out.append(f"{len(paths)} live paths (at most 64)")
    for name, key in (("", "o1"), ("dual ", "oo")):
        size = "d3" if key == "o1" else "d1"
        groups: dict = {}
        for p in paths:
            groups[p[key]] = groups.get(p[key], 0) + p[size]
        rows = sum(groups.values())
        tiles = sum((k + 15) // 16 for k in groups.values())
        if rows > 128:
            out.append(f"{name}kk rows {rows} (at most 128)")
        if len(groups) > 8:
            out.append(f"{len(groups)} {name}path groups (at most 8)")
        if max(groups.values(), default=0) > 32:
            out.append(f"a {name}path group of {max(groups.values())} kk rows (at most 32)")
        if tiles > 8:
            out.append(f"{tiles} {name}kk tiles (at most 8)")
    return out


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


def struct_words(st) -> list:
    """A ctypes struct of 32-bit fields as the list of its int32 words (the ``int[]`` table arguments of the
    ops: host values, so a traced graph keeps them on the host whatever device it is loaded to)."""
    return np.frombuffer(ctypes.string_at(ctypes.addressof(st), ctypes.sizeof(st)), dtype=np.int32).tolist()


def layout_words(layout_id: int) -> list:
    """The layout table as the int32 word list the ops take (one per layout, cached)."""
    name, lay, st = _LAYOUTS[layout_id]
    key = ("words", layout_id)
    if key not in _TABLES:
        _TABLES[key] = struct_words(st)
    return _TABLES[key]


_TABLES: dict = {}


class FscHarmTable(ctypes.Structure):
    _fields_ = [("lmax", _i32), ("nmono", _i32), ("mono_l", _i32 * 20), ("mono_exp", (_i32 * 3) * 20),
                ("coef", (ctypes.c_float * 7) * 20)]


def harmonics_table(lmax: int) -> list:
    """The ICTD direction-harmonics table (degree-l monomials and multinomial * G_l B_l, lmax <= 3) as the
    int32 word list the ``edge_harmonics`` op takes (cached)."""
    from .ictd_basis import harmonic_projection
    key = ("harm", lmax)
    if key not in _TABLES:
        if not 0 <= lmax <= 3:
            raise NotImplementedError("the HIP direction harmonics support lmax <= 3")
        t = FscHarmTable()
        t.lmax = lmax
        k = 0
        for l in range(lmax + 1):
            exps, coef, P = harmonic_projection(l)
            M = coef[:, None] * P
            for i in range(len(exps)):
                t.mono_l[k] = l
                for j in range(3):
                    t.mono_exp[k][j] = int(exps[i][j])
                for j in range(2 * l + 1):
                    t.coef[k][j] = float(M[i][j])
                k += 1
        t.nmono = k
        _TABLES[key] = struct_words(t)
    return _TABLES[key]


def edge_harmonics(n: Tensor, lmax: int) -> Tensor:
    """Differentiable Y (E, (lmax+1)^2) of the unit edge vectors n (E, 3) in the ICTD basis."""
    return torch.ops.fsctep.edge_harmonics(n, harmonics_table(lmax))


def ictd_conv_apply(x, Y, gates, W, Wt, cg, graph, layout_id: int):
    """Differentiable conv2..n: x (N,M,C), Y (E,NY), gates (E,NREF) -> (N,M,C)."""
    return torch.ops.fsctep.ictd_conv(x, Y, gates, W, Wt, cg, graph.dst_ptr, graph.src32, graph.src_ptr,
                                      graph.src_perm, graph.dst32, graph.node_order, layout_words(layout_id))


def ictd_conv1_apply(F, gates, qtab, graph, layout_id: int):
    """Differentiable conv1: F (E,NY) harmonics (+ field), gates (E,NREF), qtab (NS*NS,NP1,C) -> (N,M,C)."""
    return torch.ops.fsctep.ictd_conv1(F, gates, qtab, graph.dst_ptr, graph.edge_pair, graph.node_species,
                                       int(graph.n_species), layout_struct(layout_id).M, layout_words(layout_id))
