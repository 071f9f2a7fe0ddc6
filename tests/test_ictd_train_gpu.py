"""Training derivatives of the ICTD conv op (``torch.ops.fsctep.ictd_conv``): the weight gradient and the
double backward of force training (create_graph through the conv's backward), against torch autograd of
the oracle tensor product in fp64.  The reference covers the same derivatives of its tensor-product
extension with its double-backward kernels (csrc/ictd_tp_cuda.cu:536-971) and tests them against its
einsum path (test/test_ictd_tp_backend.py:383-714, fp32 rtol 5e-5 / atol 5e-6); the bar here is 1e-5
relative (max norm) for first derivatives and 2e-5 for second derivatives, which sum four products of
first-derivative size."""

import numpy as np
import pytest
import torch

from oracle import ictd_ref as I
from test_ictd_gpu import _edges, _oracle_conv, rel_inf

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL1, TOL2 = 1e-5, 2e-5

LAYOUTS = {"full_l2": lambda B: B.layout_full(2), "full_l3": lambda B: B.layout_full(3),
           "o3": lambda B: B.layout_o3(2, [(0, 1), (1, 1), (1, -1), (2, 1)])}


def _case(lname, C, seed):
    from fsctep_amd import ictd_basis as B
    lay = LAYOUTS[lname](B)
    g = torch.Generator().manual_seed(seed)
    N = 30
    src, dst = _edges(N, seed + 4)
    order = torch.argsort(dst, stable=True)
    src, dst = src[order], dst[order]
    E = src.shape[0]
    n = torch.randn(E, 3, generator=g, dtype=torch.float64)
    n = n / n.norm(dim=1, keepdim=True)
    Y = torch.cat([I.direction_harmonics(n, l) for l in range(lay.lmax + 1)], dim=-1)
    x = torch.randn(N, lay.M, C, generator=g, dtype=torch.float64)
    P = lay.n_ref_paths()
    gates = torch.randn(E, P, generator=g, dtype=torch.float64)
    W = torch.randn(P, C, C, 1, generator=g, dtype=torch.float64) / np.sqrt(C)
    # round every input to fp32 so that both sides see the same values
    x, Y, gates, W = (t.float().double() for t in (x, Y, gates, W))
    return lay, src, dst, N, x, Y, gates, W, g


def _device_conv(lay, src, dst, N):
    from fsctep_amd import ictd_ops
    from fsctep_amd.graph import prepare_graph
    lid = ictd_ops.register_layout(lay)
    gr = prepare_graph(src.to(DEV), dst.to(DEV), torch.zeros(src.shape[0], 3, device=DEV), N)
    cg = torch.tensor(lay.cg_table(), dtype=torch.float32, device=DEV)

    def conv(x, Y, gates, W):
        Wt = torch.ops.fsctep.ictd_prepare_weights(W.detach())
        return ictd_ops.ictd_conv_apply(x, Y, gates, W, Wt, cg, gr, lid)
    return conv


def _leaves(ts, dev=None, dtype=None):
    return [t.detach().to(device=dev or t.device, dtype=dtype or t.dtype).requires_grad_(True) for t in ts]


@pytest.mark.parametrize("lname,C", [("full_l2", 32), ("full_l3", 128), ("o3", 64)])
def test_weight_gradient_matches_oracle(lname, C):
    lay, src, dst, N, x, Y, gates, W, g = _case(lname, C, 5)
    xo, Yo, go, Wo = _leaves((x, Y, gates, W))
    ref = _oracle_conv(xo, Yo, go, Wo, src, dst, N, lay)
    G = torch.randn(ref.shape, generator=g, dtype=torch.float64).float().double()
    want = torch.autograd.grad((ref * G).sum(), (xo, Yo, go, Wo))

    conv = _device_conv(lay, src, dst, N)
    xd, Yd, gd, Wd = _leaves((x, Y, gates, W), DEV, torch.float32)
    out = conv(xd, Yd, gd, Wd)
    got = torch.autograd.grad(out, (xd, Yd, gd, Wd), G.float().to(DEV))
    torch.cuda.synchronize()
    assert rel_inf(out, ref) < TOL1
    for a, b in zip(got, want):
        assert a.shape == b.shape
        assert rel_inf(a, b) < TOL1
    # weight slots of paths without a geometric operand get no gradient
    live = set(int(p) for p in _live_gates(lay))
    dead = [p for p in range(W.shape[0]) if p not in live]
    if dead:
        assert float(got[3][dead].abs().max()) == 0.0


def _live_gates(lay):
    from fsctep_amd.ictd_ops import build_layout_struct
    s = build_layout_struct(lay)
    return [s.p_gate[p] for p in range(s.NP)]


@pytest.mark.parametrize("lname,C", [("full_l2", 32), ("full_l3", 128), ("o3", 64)])
def test_double_backward_matches_oracle(lname, C):
    """s = <Vx, dx> + <VY, dY> + <Vg, dgates> + <VW, dW> with (dx, dY, dgates, dW) the conv's backward at G
    (create_graph), then the gradient of s with respect to G, x, Y, gates and W."""
    lay, src, dst, N, x, Y, gates, W, g = _case(lname, C, 9)
    G = torch.randn(N, lay.M, C, generator=g, dtype=torch.float64).float().double()
    V = [torch.randn(t.shape, generator=g, dtype=torch.float64).float().double() for t in (x, Y, gates, W)]

    def second(conv, leaves, Vs):
        xa, Ya, ga, Wa, Ga = leaves
        out = conv(xa, Ya, ga, Wa)
        d = torch.autograd.grad((out * Ga).sum(), (xa, Ya, ga, Wa), create_graph=True)
        s = sum((di * vi).sum() for di, vi in zip(d, Vs))
        return torch.autograd.grad(s, leaves)

    ref_leaves = _leaves((x, Y, gates, W, G))
    want = second(lambda *a: _oracle_conv(*a, src, dst, N, lay), ref_leaves, V)

    conv = _device_conv(lay, src, dst, N)
    dev_leaves = _leaves((x, Y, gates, W, G), DEV, torch.float32)
    got = second(conv, dev_leaves, [v.float().to(DEV) for v in V])
    torch.cuda.synchronize()
    for name, a, b in zip(("x", "Y", "gates", "W", "G"), got, want):
        assert a.shape == b.shape, name
        assert rel_inf(a, b) < TOL2, name


def test_force_loss_parameter_gradients_match_oracle():
    """Force training through the conv: a small model pos -> edge geometry -> harmonics and gates (a radial
    MLP) -> conv -> a quadratic atom energy; forces by create_graph, loss = sum F^2, then the gradients of
    every parameter (conv weight, radial MLP, node features) and of the positions.  Everything but the conv
    is torch in fp64 on the host for both sides; the device side runs the conv op in fp32 on the GPU (inputs
    cast at its boundary, output cast back), so the comparison isolates the op's first and second
    derivatives."""
    from fsctep_amd import ictd_basis as B
    lay, C = B.layout_full(2), 32
    g = torch.Generator().manual_seed(17)
    N = 24
    pos0 = torch.rand(N, 3, generator=g, dtype=torch.float64) * 6.0
    d = (pos0[None] - pos0[:, None]).norm(dim=-1)
    src, dst = torch.nonzero((d < 3.5) & (d > 0), as_tuple=True)
    order = torch.argsort(dst, stable=True)
    src, dst = src[order], dst[order]
    P = lay.n_ref_paths()
    params0 = {
        "x": torch.randn(N, lay.M, C, generator=g, dtype=torch.float64),
        "W": torch.randn(P, C, C, 1, generator=g, dtype=torch.float64) / np.sqrt(C),
        "w1": torch.randn(8, 16, generator=g, dtype=torch.float64) / np.sqrt(8),
        "w2": torch.randn(16, P, generator=g, dtype=torch.float64) / 4.0,
        "ro": torch.randn(C, generator=g, dtype=torch.float64) / np.sqrt(C),
    }
    params0 = {k: v.float().double() for k, v in params0.items()}
    pos0 = pos0.float().double()

    def loss_and_grads(conv):
        p = {k: v.detach().clone().requires_grad_(True) for k, v in params0.items()}
        pos = pos0.detach().clone().requires_grad_(True)
        vec = pos[src] - pos[dst]
        r = vec.norm(dim=-1, keepdim=True)
        n = vec / r
        Y = torch.cat([I.direction_harmonics(n, l) for l in range(lay.lmax + 1)], dim=-1)
        mu = torch.linspace(0.5, 3.5, 8, dtype=torch.float64)
        emb = torch.exp(-((r - mu) ** 2) / 0.5)
        gates = torch.tanh(emb @ p["w1"]) @ p["w2"]
        out = conv(p["x"], Y, gates, p["W"])
        e = (out[:, 0, :] @ p["ro"]) + 0.5 * (out ** 2).sum(dim=(1, 2))
        E = e.sum()
        F = -torch.autograd.grad(E, pos, create_graph=True)[0]
        loss = (F ** 2).sum()
        names = list(p) + ["pos"]
        grads = torch.autograd.grad(loss, [p[k] for k in p] + [pos])
        return float(loss), dict(zip(names, grads)), F.detach()

    dconv = _device_conv(lay, src, dst, N)

    def device_conv(x, Y, ga, W):
        f32 = [t.to(DEV, torch.float32) for t in (x, Y, ga, W)]
        return dconv(*f32).double().cpu()

    loss_ref, g_ref, F_ref = loss_and_grads(lambda x, Y, ga, W: _oracle_conv(x, Y, ga, W, src, dst, N, lay))
    loss_dev, g_dev, F_dev = loss_and_grads(device_conv)
    torch.cuda.synchronize()
    assert rel_inf(F_dev, F_ref) < TOL1
    assert abs(loss_dev - loss_ref) / abs(loss_ref) < TOL1
    for k in g_ref:
        assert rel_inf(g_dev[k], g_ref[k]) < TOL2, k


def test_third_derivative_is_refused():
    lay, src, dst, N, x, Y, gates, W, g = _case("full_l2", 32, 2)
    conv = _device_conv(lay, src, dst, N)
    xd, Yd, gd, Wd = _leaves((x, Y, gates, W), DEV, torch.float32)
    out = conv(xd, Yd, gd, Wd)
    (dx,) = torch.autograd.grad(out.sum(), (xd,), create_graph=True)
    (dg,) = torch.autograd.grad((dx ** 2).sum(), (gd,))          # second derivatives: supported
    assert torch.isfinite(dg).all()
    (dx,) = torch.autograd.grad(out.sum(), (xd,), create_graph=True)
    with pytest.raises(RuntimeError, match="third derivatives"):
        torch.autograd.grad((dx ** 2).sum(), (gd,), create_graph=True)
