"""Fused invariant Gram bilinear of the readout as ``torch.ops.fsctep.*`` custom ops.

``gram_bilinear(t, Wf, Wb, scale)`` computes ``out[n][o] = sum_{i,j} W[o][i][j] G_n[i][j]`` with
``G_n = scale * t_n^T t_n`` for ``t`` of shape (N, D, nC), without materialising ``G``.  It serves
``PureCartesianSparseInvariantBilinear`` (models/pure_cartesian_sparse_layers.py:424-456) and the
Gram x ``W_read`` readout of the ICTD trunks (models/pure_cartesian_ictd_layers_full.py:999-1000,
models/pure_cartesian_ictd_layers_o3.py:1017-1018).  ``Wf``/``Wb`` are the block-pair layouts of
``W`` made by ``gram_prepare_weights``; the autograd formula returns the gradient w.r.t. ``t`` only
(weights are constants of the energy/force path).
"""

from __future__ import annotations

import ctypes

import torch
from torch import Tensor

from . import _lib


def _require_cuda(*ts: Tensor) -> None:
    for t in ts:
        if t is not None and not t.is_cuda:
            raise RuntimeError("fsctep ops run on the GPU only (HIP kernels); got a CPU tensor")


def _c(t: Tensor) -> Tensor:
    t = t if t.dtype == torch.float32 else t.float()
    return t if t.is_contiguous() else t.contiguous()


def gram_sizes(n_nodes: int, nC: int, S: int) -> tuple[int, int]:
    """(floats of one prepared weight layout, floats of the forward workspace)."""
    w, ws = ctypes.c_int64(), ctypes.c_int64()
    _lib.call("fsc_gram_sizes", int(n_nodes), int(nC), int(S), ctypes.byref(w), ctypes.byref(ws))
    return int(w.value), int(ws.value)


@torch.library.custom_op("fsctep::gram_prepare_weights", mutates_args=())
def gram_prepare_weights(W: Tensor) -> tuple[Tensor, Tensor]:
    """W (S, nC, nC) -> (Wf (P, 16, S, 16), Wb (P, 256, S)) over the P = nb(nb+1)/2 block pairs."""
    _require_cuda(W)
    S, nC = int(W.shape[0]), int(W.shape[1])
    W = _c(W)
    wn, _ = gram_sizes(0, nC, S)
    P = wn // (256 * S)
    Wf = torch.empty(P, 16, S, 16, device=W.device, dtype=torch.float32)
    Wb = torch.empty(P, 256, S, device=W.device, dtype=torch.float32)
    _lib.call("fsc_gram_prepare_weights", _lib.ptr(W), S, nC, _lib.ptr(Wf), _lib.ptr(Wb),
              _lib.stream_handle(W.device))
    return Wf, Wb


@gram_prepare_weights.register_fake
def _(W):
    S, nC = W.shape[0], W.shape[1]
    nb = nC // 16
    P = nb * (nb + 1) // 2
    return W.new_empty(P, 16, S, 16), W.new_empty(P, 256, S)


@torch.library.custom_op("fsctep::gram_bilinear", mutates_args=())
def gram_bilinear(t: Tensor, Wf: Tensor, Wb: Tensor, scale: float) -> Tensor:
    """t (N, D, nC) -> (N, S)."""
    _require_cuda(t, Wf, Wb)
    N, D, nC = (int(v) for v in t.shape)
    S = int(Wb.shape[2])
    t = _c(t)
    _, wsn = gram_sizes(N, nC, S)
    ws = torch.empty(max(wsn, 1), device=t.device, dtype=torch.float32)
    out = torch.empty(N, S, device=t.device, dtype=torch.float32)
    _lib.call("fsc_gram_forward", N, D, nC, S, float(scale), _lib.ptr(t), _lib.ptr(Wf), _lib.ptr(ws),
              _lib.ptr(out), _lib.stream_handle(t.device))
    return out


@gram_bilinear.register_fake
def _(t, Wf, Wb, scale):
    return t.new_empty(t.shape[0], Wb.shape[2])


@torch.library.custom_op("fsctep::gram_bilinear_backward", mutates_args=())
def gram_bilinear_backward(grad_out: Tensor, t: Tensor, Wb: Tensor, scale: float) -> Tensor:
    _require_cuda(grad_out, t, Wb)
    N, D, nC = (int(v) for v in t.shape)
    S = int(Wb.shape[2])
    g, t = _c(grad_out), _c(t)
    dt = torch.empty(N, D, nC, device=t.device, dtype=torch.float32)
    _lib.call("fsc_gram_backward", N, D, nC, S, float(scale), _lib.ptr(g), _lib.ptr(t), _lib.ptr(Wb),
              _lib.ptr(dt), _lib.stream_handle(t.device))
    return dt


@gram_bilinear_backward.register_fake
def _(grad_out, t, Wb, scale):
    return torch.empty_like(t)


def _gram_setup(ctx, inputs, output):
    t, Wf, Wb, scale = inputs
    ctx.save_for_backward(t, Wb)
    ctx.scale = scale


def _gram_bwd(ctx, grad_out):
    t, Wb = ctx.saved_tensors
    if ctx.needs_input_grad[1] or ctx.needs_input_grad[2]:
        raise NotImplementedError("gradients w.r.t. the readout weights are not implemented "
                                  "(energy/force inference only)")
    return torch.ops.fsctep.gram_bilinear_backward(grad_out, t, Wb, ctx.scale), None, None, None


torch.library.register_autograd("fsctep::gram_bilinear", _gram_bwd, setup_context=_gram_setup)


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
