"""Training derivatives of the sparse conv2..n op (``torch.ops.fsctep.sparse_conv`` with ``w_last``/``b_last``):
the gradient of the last radial layer and the double backward of force training, against torch autograd of
the oracle chain (models/pure_cartesian_sparse_layers.py:382-421 restated in the oracle) in fp64.  The
receiver assembly is quadratic in the edge directions, so the second derivatives include the direction
Hessian term (``sparse_conv_direction_backward``).  Bars as for the ICTD conv: 1e-5 relative (max norm) for
first derivatives, 2e-5 for second derivatives."""

import numpy as np
import pytest
import torch

from sparse_helpers import oracle_conv2, rel_inf
from test_sparse_gpu import _graph_with_edge_cases

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL1, TOL2 = 1e-5, 2e-5


def _case(C, seed, N=30, E_rand=260):
    g = torch.Generator().manual_seed(seed)
    src, dst = _graph_with_edge_cases(N, E_rand, seed)
    order = torch.argsort(dst, stable=True)
    src, dst = src[order], dst[order]
    E = src.shape[0]
    x = torch.randn(N, 13, C, generator=g, dtype=torch.float64)
    h = torch.randn(E, 64, generator=g, dtype=torch.float64)
    v = torch.randn(E, 3, generator=g, dtype=torch.float64)
    n = v / v.norm(dim=1, keepdim=True)
    L = torch.randn(6 * C * C, 64, generator=g, dtype=torch.float64) / 8
    b = torch.randn(6 * C * C, generator=g, dtype=torch.float64) * 0.1
    x, h, n, L, b = (t.float().double() for t in (x, h, n, L, b))
    return src, dst, N, x, h, n, L, b, g


def _device_conv(src, dst, N, C):
    from fsctep_amd import ops
    from fsctep_amd.graph import prepare_graph
    gr = prepare_graph(src.to(DEV), dst.to(DEV), torch.zeros(src.shape[0], 3, device=DEV), N)

    def conv(x, h, n, L, b):
        bk1, bk6 = torch.ops.fsctep.sparse_prepare_weights(L.detach(), b.detach(), C)
        return ops.sparse_conv_apply(x, h, n, bk1, bk6, gr, 0, L, b)
    return conv


def _oracle(src, dst, N):
    E = src.shape[0]

    def conv(x, h, n, L, b):
        return oracle_conv2(x, h, n, L, b, src, dst, N, 1.0 / (E / N))
    return conv


def _leaves(ts, dev=None, dtype=None):
    return [t.detach().to(device=dev or t.device, dtype=dtype or t.dtype).requires_grad_(True) for t in ts]


@pytest.mark.parametrize("C", [64, 32, 128])
def test_weight_gradient_matches_oracle(C):
    src, dst, N, x, h, n, L, b, g = _case(C, 3)
    ref_leaves = _leaves((x, h, n, L, b))
    ref = _oracle(src, dst, N)(*ref_leaves)
    G = torch.randn(ref.shape, generator=g, dtype=torch.float64).float().double()
    want = torch.autograd.grad((ref * G).sum(), ref_leaves)
    dev_leaves = _leaves((x, h, n, L, b), DEV, torch.float32)
    out = _device_conv(src, dst, N, C)(*dev_leaves)
    got = torch.autograd.grad(out, dev_leaves, G.float().to(DEV))
    torch.cuda.synchronize()
    assert rel_inf(out, ref) < TOL1
    for name, a, b_ in zip(("x", "h", "n", "L", "b"), got, want):
        assert a.shape == b_.shape, name
        assert rel_inf(a, b_) < TOL1, name


@pytest.mark.parametrize("C", [64, 32, 128])
def test_double_backward_matches_oracle(C):
    """s = <Vx,dx> + <Vh,dh> + <Vn,dn> + <VL,dL> + <Vb,db> of the conv's backward at G (create_graph), then
    the gradient of s with respect to x, h, n, L, b and G."""
    src, dst, N, x, h, n, L, b, g = _case(C, 7)
    G = torch.randn(N, 13, C, generator=g, dtype=torch.float64).float().double()
    V = [torch.randn(t.shape, generator=g, dtype=torch.float64).float().double() for t in (x, h, n, L, b)]

    def second(conv, leaves, Vs):
        xa, ha, na, La, ba, Ga = leaves
        out = conv(xa, ha, na, La, ba)
        d = torch.autograd.grad((out * Ga).sum(), (xa, ha, na, La, ba), create_graph=True)
        s = sum((di * vi).sum() for di, vi in zip(d, Vs))
        return torch.autograd.grad(s, leaves)

    want = second(_oracle(src, dst, N), _leaves((x, h, n, L, b, G)), V)
    got = second(_device_conv(src, dst, N, C), _leaves((x, h, n, L, b, G), DEV, torch.float32),
                 [v.float().to(DEV) for v in V])
    torch.cuda.synchronize()
    for name, a, b_ in zip(("x", "h", "n", "L", "b", "G"), got, want):
        assert a.shape == b_.shape, name
        assert rel_inf(a, b_) < TOL2, name


def test_force_loss_parameter_gradients_match_oracle():
    """Force training through the conv: pos -> edge vectors -> n, r (torch) -> radial hidden features (a torch
    MLP) -> conv (the op, with its last radial layer L, b) -> a quadratic atom energy; forces by create_graph,
    loss = sum F^2, then the gradients of every parameter and of the positions.  Everything but the conv is
    torch in fp64 on the host for both sides; the device side runs the op in fp32 (inputs cast at its
    boundary), so the comparison isolates the op's first and second derivatives."""
    C = 32
    g = torch.Generator().manual_seed(29)
    N = 24
    pos0 = (torch.rand(N, 3, generator=g, dtype=torch.float64) * 6.0).float().double()
    d = (pos0[None] - pos0[:, None]).norm(dim=-1)
    src, dst = torch.nonzero((d < 3.5) & (d > 0), as_tuple=True)
    order = torch.argsort(dst, stable=True)
    src, dst = src[order], dst[order]
    params0 = {
        "x": torch.randn(N, 13, C, generator=g, dtype=torch.float64),
        "L": torch.randn(6 * C * C, 64, generator=g, dtype=torch.float64) / 8,
        "b": torch.randn(6 * C * C, generator=g, dtype=torch.float64) * 0.1,
        "w1": torch.randn(8, 64, generator=g, dtype=torch.float64) / np.sqrt(8),
        "ro": torch.randn(C, generator=g, dtype=torch.float64) / np.sqrt(C),
    }
    params0 = {k: v.float().double() for k, v in params0.items()}

    def loss_and_grads(conv):
        p = {k: v.detach().clone().requires_grad_(True) for k, v in params0.items()}
        pos = pos0.detach().clone().requires_grad_(True)
        vec = pos[src] - pos[dst]
        r = vec.norm(dim=-1, keepdim=True)
        n = vec / r
        mu = torch.linspace(0.5, 3.5, 8, dtype=torch.float64)
        h = torch.tanh(torch.exp(-((r - mu) ** 2) / 0.5) @ p["w1"])
        out = conv(p["x"], h, n, p["L"], p["b"])
        e = (out[:, 0, :] @ p["ro"]) + 0.5 * (out ** 2).sum(dim=(1, 2))
        F = -torch.autograd.grad(e.sum(), pos, create_graph=True)[0]
        loss = (F ** 2).sum()
        grads = torch.autograd.grad(loss, [p[k] for k in p] + [pos])
        return float(loss), dict(zip(list(p) + ["pos"], grads)), F.detach()

    dconv = _device_conv(src, dst, N, C)

    def device_conv(x, h, n, L, b):
        return dconv(*[t.to(DEV, torch.float32) for t in (x, h, n, L, b)]).double().cpu()

    loss_ref, g_ref, F_ref = loss_and_grads(_oracle(src, dst, N))
    loss_dev, g_dev, F_dev = loss_and_grads(device_conv)
    torch.cuda.synchronize()
    assert rel_inf(F_dev, F_ref) < TOL1
    assert abs(loss_dev - loss_ref) / abs(loss_ref) < TOL1
    for k in g_ref:
        assert rel_inf(g_dev[k], g_ref[k]) < TOL2, k


def test_without_weights_and_third_derivative():
    """Without w_last/b_last the op serves forces as before and refuses a weight-dependent second
    derivative through h; create_graph through the double backward (third derivatives) raises."""
    from fsctep_amd import ops
    from fsctep_amd.graph import prepare_graph
    C = 32
    src, dst, N, x, h, n, L, b, g = _case(C, 11)
    gr = prepare_graph(src.to(DEV), dst.to(DEV), torch.zeros(src.shape[0], 3, device=DEV), N)
    Ld, bd = L.float().to(DEV), b.float().to(DEV)
    bk1, bk6 = torch.ops.fsctep.sparse_prepare_weights(Ld, bd, C)
    xd, hd, nd = _leaves((x, h, n), DEV, torch.float32)
    out = ops.sparse_conv_apply(xd, hd, nd, bk1, bk6, gr)
    (dh,) = torch.autograd.grad(out.sum(), (hd,), create_graph=True)
    with pytest.raises(RuntimeError, match="needs w_last and b_last"):
        torch.autograd.grad((dh ** 2).sum(), (xd,))
    Lw, bw = _leaves((L, b), DEV, torch.float32)
    out = _device_conv(src, dst, N, C)(xd, hd, nd, Lw, bw)
    (dx,) = torch.autograd.grad(out.sum(), (xd,), create_graph=True)
    (dn2,) = torch.autograd.grad((dx ** 2).sum(), (nd,))
    assert torch.isfinite(dn2).all()
    (dx,) = torch.autograd.grad(out.sum(), (xd,), create_graph=True)
    with pytest.raises(RuntimeError, match="third derivatives"):
        torch.autograd.grad((dx ** 2).sum(), (nd,), create_graph=True)
