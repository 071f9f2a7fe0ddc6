"""Pins of the oracle of the per-edge (bucketed) ICTD tensor product (oracle/ictd_bucket_ref.py), CPU only.

* The projection equals brute-force loops and the extension's second (ATen) formulation, which fixes the
  (B, P, K, I*J) output layout independently of the einsum.
* Every transpose equals the autograd vector-Jacobian product of its forward; every double-backward sum
  equals the directional derivative (torch.func.jvp) of the first-order function it differentiates.
* Summed over the bucket table, project + mix reproduces the fully connected TP of the trunk oracle
  (oracle.ictd_ref.fctp), which the reference's golden energies and forces pin.
A planted mistake (a transposed operand in the mix) fails the VJP check.
"""

import itertools

import pytest
import torch

from oracle import ictd_bucket_ref as BR
from oracle import ictd_ref as R

torch.manual_seed(0)
D = torch.float64


def _proj_args(B=3, I=4, J=1, m1=3, m2=5, P=2, K=3):
    g = torch.Generator().manual_seed(B * 131 + I * 7 + m1 + 11 * m2 + 3 * P + K)
    mk = lambda *s: torch.randn(*s, generator=g, dtype=D)
    return mk(B, I, m1), mk(B, J, m2), mk(m1 * m2, P * K), P


def _mix_args(B=3, P=2, K=5, IJ=6, O=4):
    g = torch.Generator().manual_seed(B + 17 * P + K + 5 * IJ + O)
    mk = lambda *s: torch.randn(*s, generator=g, dtype=D)
    return mk(B, P, K, IJ), mk(P, O, IJ), mk(B, P)


@pytest.mark.parametrize("J", [1, 2])
def test_projection_brute_force_and_aten_route(J):
    a, b, u, P = _proj_args(J=J)
    y = BR.project_forward(a, b, u, P)
    B, I, m1 = a.shape
    m2, K = b.shape[2], u.shape[1] // P
    ref = torch.zeros(B, P, K, I * J, dtype=D)
    for bb, p, k, i, j in itertools.product(range(B), range(P), range(K), range(I), range(J)):
        s = 0.0
        for m, n in itertools.product(range(m1), range(m2)):
            s += float(a[bb, i, m] * b[bb, j, n] * u[m * m2 + n, p * K + k])
        ref[bb, p, k, i * J + j] = s
    assert torch.allclose(y, ref, rtol=1e-12, atol=1e-12)
    assert torch.allclose(BR.project_forward_aten(a, b, u, P), ref, rtol=1e-12, atol=1e-12)


def test_mix_brute_force():
    y, w, g = _mix_args()
    out = BR.mix_forward(y, w, g)
    B, P, K, IJ = y.shape
    O = w.shape[1]
    ref = torch.zeros(B, O, K, dtype=D)
    for bb, o, k in itertools.product(range(B), range(O), range(K)):
        ref[bb, o, k] = sum(float(g[bb, p] * y[bb, p, k, q] * w[p, o, q]) for p in range(P) for q in range(IJ))
    assert torch.allclose(out, ref, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("J", [1, 2])
def test_projection_transposes_are_vjps(J):
    a, b, u, P = _proj_args(J=J, m1=5, m2=3)
    a, b, u = (t.clone().requires_grad_() for t in (a, b, u))
    y = BR.project_forward(a, b, u, P)
    gy = torch.randn_like(y)
    va, vb, vu = torch.autograd.grad(y, (a, b, u), gy)
    ta, tb, tu = BR.project_transpose(gy, a.detach(), b.detach(), u.detach())
    for x, ref in ((ta, va), (tb, vb), (tu, vu)):
        assert torch.allclose(x, ref, rtol=1e-12, atol=1e-12)


def _mix_transpose_planted(grad_out, y, w, gates):
    gated = grad_out[:, None, :, :] * gates[:, :, None, None]
    return torch.einsum("bpok,poq->bpkq", gated, w.transpose(1, 2).reshape(w.shape)), None, None


@pytest.mark.parametrize("planted", [False, True])
def test_mix_transposes_are_vjps(planted):
    y, w, g = _mix_args(IJ=4, O=4)
    y, w, g = (t.clone().requires_grad_() for t in (y, w, g))
    out = BR.mix_forward(y, w, g)
    go = torch.randn_like(out)
    vy, vw, vg = torch.autograd.grad(out, (y, w, g), go)
    if planted:
        ty = _mix_transpose_planted(go, y.detach(), w.detach(), g.detach())[0]
        assert not torch.allclose(ty, vy, rtol=1e-6, atol=1e-6)
        return
    ty, tw, tg = BR.mix_transpose(go, y.detach(), w.detach(), g.detach())
    for x, ref in ((ty, vy), (tw, vw), (tg, vg)):
        assert torch.allclose(x, ref, rtol=1e-12, atol=1e-12)


def test_projection_double_backward_is_the_directional_derivative():
    a, b, u, P = _proj_args(B=2, I=3, m1=3, m2=3, P=2, K=3)
    gga, ggb, ggu = torch.randn_like(a), torch.randn_like(b), torch.randn_like(u)
    h = torch.randn(2, P, 3, 3, dtype=D)
    gh, ga, gb, gu = BR.project_dbl_bwd(h, a, gga, b, ggb, u, ggu, P)
    f = lambda a_, b_, u_: BR.project_forward(a_, b_, u_, P)
    assert torch.allclose(gh, torch.func.jvp(f, (a, b, u), (gga, ggb, ggu))[1], rtol=1e-12, atol=1e-12)
    pat = lambda b_, u_: BR.project_transpose(h, a, b_, u_)[0]
    assert torch.allclose(ga, torch.func.jvp(pat, (b, u), (ggb, ggu))[1], rtol=1e-12, atol=1e-12)
    pbt = lambda a_, u_: BR.project_transpose(h, a_, b, u_)[1]
    assert torch.allclose(gb, torch.func.jvp(pbt, (a, u), (gga, ggu))[1], rtol=1e-12, atol=1e-12)
    put = lambda a_, b_: BR.project_transpose(h, a_, b_, u)[2]
    assert torch.allclose(gu, torch.func.jvp(put, (a, b), (gga, ggb))[1], rtol=1e-12, atol=1e-12)


def test_mix_double_backward_is_the_directional_derivative():
    y, w, g = _mix_args()
    ggy, ggw, ggg = torch.randn_like(y), torch.randn_like(w), torch.randn_like(g)
    G = torch.randn(y.shape[0], w.shape[1], y.shape[2], dtype=D)
    go, gy, gw, gg = BR.mix_dbl_bwd(G, y, ggy, w, ggw, g, ggg)
    assert torch.allclose(go, torch.func.jvp(BR.mix_forward, (y, w, g), (ggy, ggw, ggg))[1], rtol=1e-12, atol=1e-12)
    myt = lambda w_, g_: BR.mix_transpose(G, y, w_, g_)[0]
    assert torch.allclose(gy, torch.func.jvp(myt, (w, g), (ggw, ggg))[1], rtol=1e-12, atol=1e-12)
    mwt = lambda y_, g_: BR.mix_transpose(G, y_, w, g_)[1]
    assert torch.allclose(gw, torch.func.jvp(mwt, (y, g), (ggy, ggg))[1], rtol=1e-12, atol=1e-12)
    mgt = lambda y_, w_: BR.mix_transpose(G, y_, w_, g)[2]
    assert torch.allclose(gg, torch.func.jvp(mgt, (y, w), (ggy, ggw))[1], rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("lmax,o3", [(2, False), (3, False), (2, True)])
def test_bucketed_tp_equals_the_fully_connected_tp(lmax, o3):
    if o3:
        keys = [(0, 1), (1, 1), (1, -1), (2, 1)]
        ykeys = [(0, 1), (1, -1), (2, 1)]
    else:
        keys = [(l, (-1) ** l) for l in range(lmax + 1)]
        ykeys = keys
    paths = R.tp_paths(keys, ykeys, keys, lmax)
    E, C = 5, 4
    x1 = {k: torch.randn(E, C, 2 * k[0] + 1, dtype=D) for k in keys}
    x2 = {k: torch.randn(E, 1, 2 * k[0] + 1, dtype=D) for k in ykeys}
    W = torch.randn(len(paths), C, C, 1, dtype=D)
    gates = torch.randn(E, len(paths), dtype=D)
    ref = R.fctp(x1, x2, W, gates, paths, keys)
    out = {k: torch.zeros(E, C, 2 * k[0] + 1, dtype=D) for k in keys}
    table = BR.buckets(paths)
    assert sum(len(t[4]) for t in table) == len(paths)
    for k1, k2, k3, kdim, pidx, U in table:
        y = BR.project_forward(x1[k1], x2[k2], U, len(pidx))
        out[k3] = out[k3] + BR.mix_forward(y, W[pidx].reshape(len(pidx), C, C), gates[:, pidx])
    for k in keys:
        assert torch.allclose(out[k], ref[k], rtol=1e-11, atol=1e-11), k
