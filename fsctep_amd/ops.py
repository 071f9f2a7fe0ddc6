"""PyTorch custom ops (``torch.ops.fsctep.*``) over the C ABI of ``libfsctep_hip.so``.

Each op has a device implementation (the HIP kernels through ctypes), a fake/meta
implementation (shapes only, for ``make_fx`` / ``torch.export`` / tracing) and an
autograd formula whose backward is itself a custom op.  Ops launch on the current
stream of the input's device.  There is no CPU implementation: calling an op with CPU
tensors raises.

Parameter gradients are not produced (the path serves energy + forces); the model
classes refuse training-mode calls that would need them.
"""

from __future__ import annotations

import ctypes

import torch
from torch import Tensor

from . import _lib

_KH = 64


def _require_cuda(*ts: Tensor) -> None:
    for t in ts:
        if t is not None and not t.is_cuda:
            raise RuntimeError("fsctep ops run on the GPU only (HIP kernels); got a CPU tensor")


def _c(t: Tensor) -> Tensor:
    return t if t.is_contiguous() else t.contiguous()


# ----------------------------------------------------------------------------- weight preparation

@torch.library.custom_op("fsctep::sparse_prepare_weights", mutates_args=())
def sparse_prepare_weights(w_last: Tensor, b_last: Tensor, channels: int) -> tuple[Tensor, Tensor]:
    _require_cuda(w_last, b_last)
    C = int(channels)
    if w_last.shape != (6 * C * C, _KH) or b_last.shape != (6 * C * C,):
        raise ValueError(f"fc.4 of a sparse conv2 layer must be ({6 * C * C}, {_KH}); got {tuple(w_last.shape)}")
    w, b = _c(w_last.float()), _c(b_last.float())
    bk1 = torch.empty(6 * 65 * C * C, device=w.device, dtype=torch.float32)
    bk6 = torch.empty_like(bk1)
    _lib.call("fsc_sparse_conv_prepare_weights", _lib.ptr(w), _lib.ptr(b), C, _lib.ptr(bk1),
              _lib.ptr(bk6), _lib.stream_handle(w.device))
    return bk1, bk6


@sparse_prepare_weights.register_fake
def _(w_last, b_last, channels):
    n = 6 * 65 * channels * channels
    return w_last.new_empty(n, dtype=torch.float32), w_last.new_empty(n, dtype=torch.float32)


# ----------------------------------------------------------------------------- sparse conv2..n

def _ws_sizes(N: int, E: int, C: int) -> tuple[int, int]:
    s = ctypes.c_int64()
    p = ctypes.c_int64()
    _lib.call("fsc_sparse_conv_workspace", N, E, C, ctypes.byref(s), ctypes.byref(p))
    return s.value, p.value


@torch.library.custom_op("fsctep::sparse_conv", mutates_args=())
def sparse_conv(x: Tensor, h: Tensor, n: Tensor, bk1: Tensor, bk6: Tensor, dst_ptr: Tensor,
                src_ptr: Tensor, src_perm: Tensor, edge_dst: Tensor,
                inv_norm: float) -> tuple[Tensor, Tensor, Tensor]:
    """x (N,13,C), h (E,64), n (E,3) -> (out (N,13,C), S workspace, P workspace).

    bk6 and edge_dst are used by the backward only."""
    _require_cuda(x, h, n, bk1)
    N, _, C = x.shape
    E = h.shape[0]
    x, h, n = _c(x), _c(h), _c(n)
    s_f, p_f = _ws_sizes(N, E, C)
    S = torch.empty(s_f, device=x.device, dtype=torch.float32)
    P = torch.empty(p_f, device=x.device, dtype=torch.float32)
    out = torch.empty(N, 13, C, device=x.device, dtype=torch.float32)
    _lib.call("fsc_sparse_conv_forward", N, E, C, _lib.ptr(dst_ptr), _lib.ptr(src_ptr), _lib.ptr(src_perm),
              _lib.ptr(x), _lib.ptr(h), _lib.ptr(n), _lib.ptr(bk1), float(inv_norm), _lib.ptr(S),
              _lib.ptr(P), _lib.ptr(out), _lib.stream_handle(x.device))
    return out, S, P


@sparse_conv.register_fake
def _(x, h, n, bk1, bk6, dst_ptr, src_ptr, src_perm, edge_dst, inv_norm):
    N, _, C = x.shape
    E = h.shape[0]
    return (x.new_empty(N, 13, C), x.new_empty(N * 18 * 65 * C), x.new_empty(E * 18 * C))


@torch.library.custom_op("fsctep::sparse_conv_backward", mutates_args=())
def sparse_conv_backward(grad_out: Tensor, h: Tensor, n: Tensor, bk6: Tensor, S: Tensor, P: Tensor,
                         dst_ptr: Tensor, src_ptr: Tensor, src_perm: Tensor, edge_dst: Tensor,
                         inv_norm: float) -> tuple[Tensor, Tensor, Tensor]:
    _require_cuda(grad_out, h, n, bk6, S, P)
    N, _, C = grad_out.shape
    E = h.shape[0]
    g = _c(grad_out.float())
    dS = torch.empty_like(S)
    dx = torch.empty(N, 13, C, device=g.device, dtype=torch.float32)
    dh = torch.empty(E, _KH, device=g.device, dtype=torch.float32)
    dn = torch.empty(E, 3, device=g.device, dtype=torch.float32)
    _lib.call("fsc_sparse_conv_backward", N, E, C, _lib.ptr(dst_ptr), _lib.ptr(src_ptr), _lib.ptr(src_perm),
              _lib.ptr(edge_dst), _lib.ptr(g), _lib.ptr(h), _lib.ptr(n), _lib.ptr(bk6), _lib.ptr(S),
              _lib.ptr(P), float(inv_norm), _lib.ptr(dS), _lib.ptr(dx), _lib.ptr(dh), _lib.ptr(dn),
              _lib.stream_handle(g.device))
    return dx, dh, dn


@sparse_conv_backward.register_fake
def _(grad_out, h, n, bk6, S, P, dst_ptr, src_ptr, src_perm, edge_dst, inv_norm):
    N, _, C = grad_out.shape
    E = h.shape[0]
    return grad_out.new_empty(N, 13, C), h.new_empty(E, _KH), n.new_empty(E, 3)


def _sparse_conv_setup(ctx, inputs, output):
    x, h, n, bk1, bk6, dst_ptr, src_ptr, src_perm, edge_dst, inv_norm = inputs
    _, S, P = output
    ctx.save_for_backward(h, n, bk6, S, P, dst_ptr, src_ptr, src_perm, edge_dst)
    ctx.inv_norm = inv_norm
    ctx.mark_non_differentiable(S, P)
    ctx.set_materialize_grads(False)     # S and P are saved workspaces: no zero-filled gradients for them


def _sparse_conv_bwd(ctx, grad_out, grad_s, grad_p):
    h, n, bk6, S, P, dst_ptr, src_ptr, src_perm, edge_dst = ctx.saved_tensors
    if grad_out is None:
        return (None,) * 10
    if ctx.needs_input_grad[3] or ctx.needs_input_grad[4]:
        raise NotImplementedError("parameter gradients of the sparse conv are not implemented "
                                  "(energy/force inference only)")
    dx, dh, dn = torch.ops.fsctep.sparse_conv_backward(grad_out, h, n, bk6, S, P, dst_ptr, src_ptr,
                                                       src_perm, edge_dst, ctx.inv_norm)
    return dx, dh, dn, None, None, None, None, None, None, None


torch.library.register_autograd("fsctep::sparse_conv", _sparse_conv_bwd, setup_context=_sparse_conv_setup)


def sparse_conv_apply(x, h, n, bk1, bk6, graph, inv_norm: float):
    """Differentiable conv2..n message passing: (N,13,C) -> (N,13,C)."""
    out, _, _ = torch.ops.fsctep.sparse_conv(x, h, n, bk1, bk6, graph.dst_ptr, graph.src_ptr,
                                             graph.src_perm, graph.dst32, float(inv_norm))
    return out


# ----------------------------------------------------------------------------- sparse conv1

@torch.library.custom_op("fsctep::sparse_conv1_pair_table", mutates_args=())
def sparse_conv1_pair_table(w_last: Tensor, b_last: Tensor, atom_table: Tensor, channels: int) -> tuple[Tensor, Tensor]:
    _require_cuda(w_last, b_last, atom_table)
    C = int(channels)
    S = int(atom_table.shape[0])
    if atom_table.shape[1] != 8 or w_last.shape != (6 * C * 64, _KH):
        raise ValueError("conv1 pair table needs output_size 8 and fc.4 of shape (6*C*64, 64)")
    w, b, a = _c(w_last.float()), _c(b_last.float()), _c(atom_table.float())
    mf = torch.empty(S * S * 3 * 65 * C, device=w.device, dtype=torch.float32)
    mb = torch.empty_like(mf)
    _lib.call("fsc_sparse_conv1_pair_table", _lib.ptr(w), _lib.ptr(b), _lib.ptr(a), S, C, _lib.ptr(mf),
              _lib.ptr(mb), _lib.stream_handle(w.device))
    return mf, mb


@sparse_conv1_pair_table.register_fake
def _(w_last, b_last, atom_table, channels):
    S = atom_table.shape[0]
    n = S * S * 3 * 65 * channels
    return w_last.new_empty(n), w_last.new_empty(n)


@torch.library.custom_op("fsctep::sparse_conv1", mutates_args=())
def sparse_conv1(h: Tensor, n: Tensor, mf: Tensor, mb: Tensor, dst_ptr: Tensor, edge_pair: Tensor,
                 n_nodes: int, channels: int) -> tuple[Tensor, Tensor]:
    """h (E,64), n (E,3) -> (out (N,13,C), Q workspace); mb is used by the backward only."""
    _require_cuda(h, n, mf)
    E = h.shape[0]
    C = int(channels)
    h, n = _c(h), _c(n)
    Q = torch.empty(E * 3 * C, device=h.device, dtype=torch.float32)
    out = torch.empty(n_nodes, 13, C, device=h.device, dtype=torch.float32)
    _lib.call("fsc_sparse_conv1_forward", n_nodes, E, C, _lib.ptr(dst_ptr), _lib.ptr(edge_pair), _lib.ptr(h),
              _lib.ptr(n), _lib.ptr(mf), _lib.ptr(Q), _lib.ptr(out), _lib.stream_handle(h.device))
    return out, Q


@sparse_conv1.register_fake
def _(h, n, mf, mb, dst_ptr, edge_pair, n_nodes, channels):
    return h.new_empty(n_nodes, 13, channels), h.new_empty(h.shape[0] * 3 * channels)


@torch.library.custom_op("fsctep::sparse_conv1_backward", mutates_args=())
def sparse_conv1_backward(grad_out: Tensor, n: Tensor, mb: Tensor, Q: Tensor, dst_ptr: Tensor,
                          edge_pair: Tensor) -> tuple[Tensor, Tensor]:
    _require_cuda(grad_out, n, mb, Q)
    N, _, C = grad_out.shape
    E = n.shape[0]
    g = _c(grad_out.float())
    dh = torch.empty(E, _KH, device=g.device, dtype=torch.float32)
    dn = torch.empty(E, 3, device=g.device, dtype=torch.float32)
    _lib.call("fsc_sparse_conv1_backward", N, E, C, _lib.ptr(dst_ptr), _lib.ptr(edge_pair), _lib.ptr(g),
              _lib.ptr(n), _lib.ptr(mb), _lib.ptr(Q), _lib.ptr(dh), _lib.ptr(dn), _lib.stream_handle(g.device))
    return dh, dn


@sparse_conv1_backward.register_fake
def _(grad_out, n, mb, Q, dst_ptr, edge_pair):
    E = n.shape[0]
    return n.new_empty(E, _KH), n.new_empty(E, 3)


def _sparse_conv1_setup(ctx, inputs, output):
    h, n, mf, mb, dst_ptr, edge_pair, n_nodes, channels = inputs
    _, Q = output
    ctx.save_for_backward(n, mb, Q, dst_ptr, edge_pair)
    ctx.mark_non_differentiable(Q)
    ctx.set_materialize_grads(False)


def _sparse_conv1_bwd(ctx, grad_out, grad_q):
    n, mb, Q, dst_ptr, edge_pair = ctx.saved_tensors
    if grad_out is None:
        return (None,) * 8
    if ctx.needs_input_grad[2] or ctx.needs_input_grad[3]:
        raise NotImplementedError("parameter gradients of the sparse conv1 are not implemented "
                                  "(energy/force inference only)")
    dh, dn = torch.ops.fsctep.sparse_conv1_backward(grad_out, n, mb, Q, dst_ptr, edge_pair)
    return dh, dn, None, None, None, None, None, None


torch.library.register_autograd("fsctep::sparse_conv1", _sparse_conv1_bwd, setup_context=_sparse_conv1_setup)


def sparse_conv1_apply(h, n, mf, mb, graph, channels: int):
    out, _ = torch.ops.fsctep.sparse_conv1(h, n, mf, mb, graph.dst_ptr, graph.edge_pair, graph.n_nodes,
                                           int(channels))
    return out
