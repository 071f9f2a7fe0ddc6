"""Fused invariant Gram bilinear of the readout as ``torch.ops.fsctep.*`` custom ops.

``gram_bilinear(t, Wf, Wb, scale)`` computes ``out[n][o] = sum_{i,j} W[o][i][j] G_n[i][j]`` with
``G_n = scale * t_n^T t_n`` for ``t`` of shape (N, D, nC), without materialising ``G``.  It serves
``PureCartesianSparseInvariantBilinear`` (models/pure_cartesian_sparse_layers.py:424-456) and the
Gram x ``W_read`` readout of the ICTD trunks (models/pure_cartesian_ictd_layers_full.py:999-1000,
models/pure_cartesian_ictd_layers_o3.py:1017-1018).  ``Wf``/``Wb`` are the block-pair layouts of
``W`` made by ``gram_prepare_weights``; the autograd formula returns the gradient w.r.t. ``t`` only
(weights are constants of the energy/force path).  The ops are registered in C++ by
``libfsctep_torch.so``:

    gram_prepare_weights(W) -> (Wf, Wb)
    gram_bilinear(t, Wf, Wb, scale) -> out
    gram_bilinear_backward(grad_out, t, Wb, scale) -> grad_t

``readout_features(layers, Wf, Wb, scales, srcmap, gmap, table) -> (scalars, sq)`` assembles the readout
from the per-layer features in one gather: the Gram inputs of every key (the sum of their Gram bilinears
is ``scalars``) and the per-key squared norms ``sq`` (N, n_keys, n_layers*C); its backward is the Gram
backward of each key plus one scatter kernel.  ``ReadoutMaps`` holds the column maps of a readout
layout: the sparse trunk's per-rank layer concatenation
(models/pure_cartesian_sparse_layers.py:769-833) or the ICTD trunks' channel-major flatten, layer
concatenation and re-split by key (models/pure_cartesian_ictd_layers_full.py:977-1001,
models/pure_cartesian_ictd_layers_o3.py:987-1019).
"""

from __future__ import annotations

import ctypes

import numpy as np
import torch
from torch import Tensor

from . import _lib

_lib.load_torch_ops()


def gram_sizes(n_nodes: int, nC: int, S: int) -> tuple[int, int, int]:
    """(floats of the prepared Wf, floats of the prepared Wb, floats of the forward workspace)."""
    wf, wb, ws = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
    _lib.call("fsc_gram_sizes", int(n_nodes), int(nC), int(S), ctypes.byref(wf), ctypes.byref(wb), ctypes.byref(ws))
    return int(wf.value), int(wb.value), int(ws.value)


def prepare_gram(W: Tensor):
    """(Wf, Wb) of one ``W`` parameter, made from its current values on every call: a cache keyed on the
    parameter's version would miss in-place updates through ``.data`` (EMA weights), and the preparation
    reads W once (~0.15 GB/step for the ICTD 10k readout)."""
    with torch.no_grad():
        return torch.ops.fsctep.gram_prepare_weights(W.detach())


class FscReadoutTable(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in ("n_layers", "M", "C", "n_keys")] + \
        [("key_comp0", ctypes.c_int32 * 8), ("key_dim", ctypes.c_int32 * 8)]


class ReadoutMaps:
    """Column maps of the readout Gram inputs for ``n_layers`` layers of (N, M, C) features whose
    components split into keys of ``key_dims`` components (in order).

    ``resplit=False``: t_k[n][m'][l*C + c] = X_l[n][comp0_k + m'][c] (sparse trunk).
    ``resplit=True``: each layer is flattened key by key channel-major (index c*d + m within a key),
    the layers are concatenated and the result is cut into consecutive blocks of n_layers*C*d_k
    columns, block k read as (n_layers*C, d_k) and transposed (ICTD trunks).
    ``srcmap[j]`` = l*M*C + m*C + c for key-major destination column j (t_0 then t_1 ...);
    ``gmap`` is its inverse (with the re-split an entry may land in another key's Gram input)."""

    def __init__(self, n_layers: int, C: int, key_dims, resplit: bool):
        dims = [int(d) for d in key_dims]
        if not (1 <= n_layers <= 4 and 1 <= len(dims) <= 8):
            raise ValueError("readout maps: 1..4 layers and 1..8 keys")
        M = sum(dims)
        comp0 = np.concatenate([[0], np.cumsum(dims)[:-1]]).astype(np.int64)
        nC = n_layers * C
        src = []
        if not resplit:
            for k, d in enumerate(dims):
                m, cc = np.meshgrid(np.arange(d), np.arange(nC), indexing="ij")
                l, c = cc // C, cc % C
                src.append((l * M * C + (comp0[k] + m) * C + c).reshape(-1))
        else:
            # fc column J of a node: layer l = J // (C*M); within the layer, key block k2 at
            # C * comp0[k2], entry c*d2 + m2  ->  X_l[comp0[k2] + m2][c]
            kcol = C * comp0
            J_src = np.empty(n_layers * M * C, dtype=np.int64)
            for l in range(n_layers):
                for k2, d2 in enumerate(dims):
                    c, m2 = np.meshgrid(np.arange(C), np.arange(d2), indexing="ij")
                    J = l * C * M + kcol[k2] + c * d2 + m2
                    J_src[J.reshape(-1)] = (l * M * C + (comp0[k2] + m2) * C + c).reshape(-1)
            off = 0
            for k, d in enumerate(dims):
                m, cc = np.meshgrid(np.arange(d), np.arange(nC), indexing="ij")   # t_k[m'][c'] = fc[off + c'*d + m']
                src.append(J_src[off + cc * d + m].reshape(-1))
                off += nC * d
        srcmap = np.concatenate(src)
        P = n_layers * M * C
        if sorted(srcmap.tolist()) != list(range(P)):
            raise AssertionError("readout map is not a permutation")
        gmap = np.empty(P, dtype=np.int64)
        gmap[srcmap] = np.arange(P)
        t = FscReadoutTable()
        t.n_layers, t.M, t.C, t.n_keys = n_layers, M, C, len(dims)
        for k, d in enumerate(dims):
            t.key_comp0[k], t.key_dim[k] = int(comp0[k]), d
        self.table = np.frombuffer(ctypes.string_at(ctypes.addressof(t), ctypes.sizeof(t)), dtype=np.int32).tolist()
        self.srcmap = torch.from_numpy(srcmap.astype(np.int32))
        self.gmap = torch.from_numpy(gmap.astype(np.int32))
        self.n_layers, self.M, self.C, self.key_dims = n_layers, M, C, dims
        self._dev = {}

    def on(self, device):
        """(srcmap, gmap) on ``device`` (copied once)."""
        key = str(device)
        if key not in self._dev:
            self._dev[key] = (self.srcmap.to(device), self.gmap.to(device))
        return self._dev[key]


def readout_features(layers, grams, scales, maps: ReadoutMaps):
    """(scalars (N, S) = sum_k gram_bilinear(t_k, Wf_k, Wb_k, scale_k), sq (N, n_keys, n_layers*C)).
    ``grams``: prepared (Wf, Wb) per key.  Differentiable w.r.t. the layers."""
    srcmap, gmap = maps.on(layers[0].device)
    return torch.ops.fsctep.readout_features(list(layers), [g[0] for g in grams], [g[1] for g in grams],
                                             [float(s) for s in scales], srcmap, gmap, maps.table)
