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
"""

from __future__ import annotations

import ctypes

import torch
from torch import Tensor

from . import _lib

_lib.load_torch_ops()


def gram_sizes(n_nodes: int, nC: int, S: int) -> tuple[int, int]:
    """(floats of one prepared weight layout, floats of the forward workspace)."""
    w, ws = ctypes.c_int64(), ctypes.c_int64()
    _lib.call("fsc_gram_sizes", int(n_nodes), int(nC), int(S), ctypes.byref(w), ctypes.byref(ws))
    return int(w.value), int(ws.value)


class GramWeights:
    """Prepared (Wf, Wb) of one ``W`` parameter, rebuilt when the parameter changes."""

    def __init__(self):
        self._key = None
        self._val = None

    def get(self, W: Tensor):
        key = (W.data_ptr(), W._version, tuple(W.shape), W.device)
        if key != self._key:
            with torch.no_grad():
                self._val = torch.ops.fsctep.gram_prepare_weights(W.detach())
            self._key = key
        return self._val
