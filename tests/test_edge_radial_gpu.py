"""The fused edge geometry and radial MLP ops against an fp64 torch evaluation of the same
formulas: the radial basis from the oracle's restatement of e3nn's soft_one_hot_linspace
(``oracle/radial.py``), torch Linear/SiLU for fc[:4], torch autograd for the force backward."""

import math

import pytest
import torch
import torch.nn.functional as F

from oracle.radial import soft_one_hot_linspace

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def rel(a, b):
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    return float((a - b).abs().max() / b.abs().max().clamp(min=1e-30))


def _hidden_ref(r, w0, b0, w2, b2, rc, nb, basis):
    emb = soft_one_hot_linspace(r, 0.0, rc, nb, basis, True) * math.sqrt(nb)
    return F.silu(F.silu(emb @ w0.T + b0) @ w2.T + b2)


@pytest.mark.parametrize("basis,nb", [("bessel", 8), ("gaussian", 8), ("bessel", 5), ("gaussian", 3), ("bessel", 16),
                                      ("fourier", 8), ("cosine", 8), ("smooth_finite", 8), ("cosine", 5),
                                      ("smooth_finite", 16)])
def test_radial_mlp_matches_torch(basis, nb):
    from fsctep_amd import ops
    g = torch.Generator().manual_seed(nb + 100 * len(basis))
    E, rc = 3001, 5.0
    r = torch.rand(E, generator=g, dtype=torch.float64) * 6.0 + 0.05     # includes r beyond the cutoff
    r[:3] = torch.tensor([rc, rc * (1 - 1e-7), 1e-3], dtype=torch.float64)
    w0 = torch.randn(64, nb, generator=g, dtype=torch.float64) * 0.5
    b0 = torch.randn(64, generator=g, dtype=torch.float64) * 0.1
    w2 = torch.randn(64, 64, generator=g, dtype=torch.float64) * 0.2
    b2 = torch.randn(64, generator=g, dtype=torch.float64) * 0.1
    dh = torch.randn(E, 64, generator=g, dtype=torch.float64)
    dev = lambda t: t.float().to(DEV)
    rd = dev(r).requires_grad_(True)
    h = torch.ops.fsctep.radial_mlp(rd, dev(w0), dev(b0), dev(w2), dev(b2), None, None, rc, ops.BASIS[basis])
    (gr,) = torch.autograd.grad(h, rd, dev(dh))
    rr = r.clone().requires_grad_(True)
    href = _hidden_ref(rr, w0, b0, w2, b2, rc, nb, basis)
    (grr,) = torch.autograd.grad(href, rr, dh)
    assert rel(h, href) < 1e-5
    # d/dr of the basis: relative to the largest entry; near r -> 0 the Bessel slope is large.  The cosine
    # bumps have a kink one step from their centre (slope pi/(2 step) inside, 0 outside): points within
    # 1e-5 steps of a kink fall on either side in fp32 and fp64, so they are left out of the slope check.
    keep = torch.ones(E, dtype=torch.bool)
    if basis == "cosine":
        step = rc / (nb + 1)
        d = (r[:, None] - step * torch.arange(1, nb + 1, dtype=torch.float64)) / step
        keep = ((d.abs() - 1).abs() > 1e-5).all(1)
    assert rel(gr.cpu()[keep], grr[keep]) < 1e-5


@pytest.mark.parametrize("P", [23, 17, 64, 1])
def test_radial_mlp_with_last_linear(P):
    from fsctep_amd import ops
    g = torch.Generator().manual_seed(P)
    E, rc, nb = 2049, 5.0, 8
    r = torch.rand(E, generator=g, dtype=torch.float64) * 5.5 + 0.5
    w0 = torch.randn(64, nb, generator=g, dtype=torch.float64) * 0.5
    b0 = torch.randn(64, generator=g, dtype=torch.float64) * 0.1
    w2 = torch.randn(64, 64, generator=g, dtype=torch.float64) * 0.2
    b2 = torch.randn(64, generator=g, dtype=torch.float64) * 0.1
    w4 = torch.randn(P, 64, generator=g, dtype=torch.float64) * 0.2
    b4 = torch.randn(P, generator=g, dtype=torch.float64) * 0.1
    dg = torch.randn(E, P, generator=g, dtype=torch.float64)
    dev = lambda t: t.float().to(DEV)
    rd = dev(r).requires_grad_(True)
    out = torch.ops.fsctep.radial_mlp(rd, dev(w0), dev(b0), dev(w2), dev(b2), dev(w4), dev(b4), rc, 0)
    (gr,) = torch.autograd.grad(out, rd, dev(dg))
    rr = r.clone().requires_grad_(True)
    ref = _hidden_ref(rr, w0, b0, w2, b2, rc, nb, "bessel") @ w4.T + b4
    (grr,) = torch.autograd.grad(ref, rr, dg)
    assert out.shape == (E, P)
    assert rel(out, ref) < 1e-5 and rel(gr, grr) < 1e-5


def _periodic_graph(N, E, seed):
    g = torch.Generator().manual_seed(seed)
    L = 12.0
    pos = torch.rand(N, 3, generator=g, dtype=torch.float64) * L
    src = torch.randint(0, N, (E,), generator=g)
    dst = torch.randint(0, N, (E,), generator=g)
    dst[src == dst] = (dst[src == dst] + 1) % N
    shifts = torch.randint(-1, 2, (E, 3), generator=g).double()
    return pos, src, dst, shifts * L


@pytest.mark.parametrize("which", ["both", "n_only", "r_only"])
def test_edge_geometry_forward_and_forces(which):
    from fsctep_amd import ops
    from fsctep_amd.graph import prepare_graph
    N, E = 300, 5000
    pos, src, dst, shift = _periodic_graph(N, E, 7)
    g = prepare_graph(src.to(DEV), dst.to(DEV), torch.zeros(E, 3, device=DEV), N)
    order = torch.argsort(dst, stable=True)
    src_s, dst_s, shift_s = src[order], dst[order], shift[order]
    gen = torch.Generator().manual_seed(3)
    gn = torch.randn(E, 3, generator=gen, dtype=torch.float64)
    gr = torch.randn(E, generator=gen, dtype=torch.float64)
    if which == "n_only":
        gr = gr * 0
    if which == "r_only":
        gn = gn * 0
    p = pos.float().to(DEV).requires_grad_(True)
    n, r = ops.edge_geometry(p, shift_s.float().to(DEV), g)
    outs, grads = [], []
    if which != "r_only":
        outs.append(n), grads.append(gn.float().to(DEV))
    if which != "n_only":
        outs.append(r), grads.append(gr.float().to(DEV))
    (gp,) = torch.autograd.grad(outs, p, grads)
    pr = pos.clone().requires_grad_(True)
    vec = pr[dst_s] - pr[src_s] + shift_s
    rr = vec.norm(dim=1)
    nr = vec / rr.clamp(min=1e-8).unsqueeze(-1)
    (gpr,) = torch.autograd.grad((nr * gn).sum() + (rr * gr).sum(), pr)
    assert rel(n, nr) < 1e-6 and rel(r, rr) < 1e-6
    assert rel(gp, gpr) < 1e-5


def test_edge_geometry_empty_graph():
    from fsctep_amd import ops
    from fsctep_amd.graph import prepare_graph
    e = torch.zeros(0, dtype=torch.long, device=DEV)
    g = prepare_graph(e, e, torch.zeros(0, 3, device=DEV), 5)
    p = torch.rand(5, 3, device=DEV, requires_grad=True)
    n, r = ops.edge_geometry(p, torch.zeros(0, 3, device=DEV), g)
    assert n.shape == (0, 3) and r.shape == (0,)
    (gp,) = torch.autograd.grad((n.sum() + r.sum()), p, allow_unused=True)
    assert gp is None or float(gp.abs().max()) == 0.0


@pytest.mark.parametrize("lmax", [1, 2, 3])
def test_edge_harmonics_match_oracle(lmax):
    from fsctep_amd import ictd_ops
    from oracle.ictd_ref import direction_harmonics
    g = torch.Generator().manual_seed(lmax)
    v = torch.randn(4097, 3, generator=g, dtype=torch.float64)
    n = v / v.norm(dim=1, keepdim=True)
    dY = torch.randn(4097, (lmax + 1) ** 2, generator=g, dtype=torch.float64)
    nd = n.float().to(DEV).requires_grad_(True)
    Y = ictd_ops.edge_harmonics(nd, lmax)
    (gn,) = torch.autograd.grad(Y, nd, dY.float().to(DEV))
    nr = n.clone().requires_grad_(True)
    Yr = torch.cat([direction_harmonics(nr, l) for l in range(lmax + 1)], dim=-1)
    (gnr,) = torch.autograd.grad(Yr, nr, dY)
    assert Y.shape == Yr.shape
    assert rel(Y, Yr) < 1e-6 and rel(gn, gnr) < 1e-5
