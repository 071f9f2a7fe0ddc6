"""GPU parity of the fused readout head, ``torch.ops.fsctep.readout_mlp`` (input LayerNorm, hidden
Linear -> LayerNorm -> SiLU layers, output Linear and weighted sum: MainNet and RobustScalarWeightedSum,
reference models/mlp.py:8-66, :117-133), against a float64 PyTorch evaluation of the same modules on the
CPU and the float32 torch modules on the GPU: per-atom energy and its input gradient, 1e-5 relative
(max-norm)."""

import copy

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL = 1e-5


def rel_inf(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).abs().max() / b.abs().max().clamp_min(1e-30))


def _head(K, hidden, seed):
    from fsctep_amd.sparse import MainNet, RobustScalarWeightedSum
    torch.manual_seed(seed)
    net = MainNet(K, hidden, 17).double()
    ws = RobustScalarWeightedSum(17, init_weights="rand").double()
    g = torch.Generator().manual_seed(seed + 1)
    with torch.no_grad():
        # non-trivial affine LayerNorms and biases, so that every folded term counts
        for ln in [net.input_norm, *net.layer_norms]:
            ln.weight.copy_(1 + 0.3 * torch.randn(ln.weight.shape, generator=g, dtype=torch.float64))
            ln.bias.copy_(0.2 * torch.randn(ln.bias.shape, generator=g, dtype=torch.float64))
        for lin in [*net.layers, net.output]:
            lin.bias.copy_(0.1 * torch.randn(lin.bias.shape, generator=g, dtype=torch.float64))
        net.output.weight.mul_(30.0)
    return net, ws


# (N, K, hidden, x offset): the sparse 10k head (K 640) with ragged row tiles, the ICTD head (K 1600),
# K not a multiple of 16, one row, one 256-wide layer, four 64-wide layers, inputs with a mean far from 0
CASES = [(37, 640, [128, 128, 128], 0.0), (300, 1600, [128, 128, 128], 0.0), (1, 20, [64, 64], 0.0),
         (17, 36, [256], 0.5), (50, 100, [64, 64, 64, 64], 0.0), (65, 1024, [128, 128], 8.0)]


@pytest.mark.parametrize("N,K,hidden,offset", CASES)
def test_readout_mlp_matches_reference(N, K, hidden, offset):
    from fsctep_amd.sparse import readout_energy
    net, ws = _head(K, hidden, N + K)
    g = torch.Generator().manual_seed(N * 3 + K)
    x = torch.randn(N, K, generator=g, dtype=torch.float64) * (1 + torch.rand(N, 1, generator=g, dtype=torch.float64))
    x = x + offset
    G = torch.randn(N, 1, generator=g, dtype=torch.float64)
    xo = x.clone().requires_grad_(True)
    ref = ws(net(xo))
    (gref,) = torch.autograd.grad(ref, xo, G)

    netf, wsf = copy.deepcopy(net).float().to(DEV), copy.deepcopy(ws).float().to(DEV)
    xd = x.float().to(DEV).requires_grad_(True)
    e = readout_energy(netf, wsf, xd)
    assert "ReadoutMlp" in e.grad_fn.name()
    (gx,) = torch.autograd.grad(e, xd, G.float().to(DEV))
    # the float32 torch modules on the GPU, for scale
    xt = x.float().to(DEV).requires_grad_(True)
    et = wsf(netf(xt))
    (gt,) = torch.autograd.grad(et, xt, G.float().to(DEV))
    torch.cuda.synchronize()
    assert e.shape == (N, 1)
    assert rel_inf(e, ref) < TOL, (rel_inf(e, ref), rel_inf(et, ref))
    assert rel_inf(gx, gref) < TOL, (rel_inf(gx, gref), rel_inf(gt, gref))


def test_readout_mlp_energy_sum_gradient_and_repeat():
    """The forces' pattern, grad of e.sum() (an expanded upstream gradient), twice in a row: identical."""
    from fsctep_amd.sparse import readout_energy
    net, ws = _head(640, [128, 128, 128], 3)
    netf, wsf = net.float().to(DEV), ws.float().to(DEV)
    x = torch.randn(1000, 640, device=DEV).abs().requires_grad_(True)
    outs = []
    for _ in range(2):
        e = readout_energy(netf, wsf, x)
        (gx,) = torch.autograd.grad(e.sum(), x)
        outs.append((e.detach(), gx))
    (ge2,) = torch.autograd.grad(wsf(netf(x)).sum(), x)
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    assert rel_inf(outs[0][1], ge2) < 1e-4


def test_readout_mlp_empty_and_fallback():
    """Zero atoms give an empty energy; a head the kernels do not cover (8-wide layers) runs as the torch
    modules."""
    from fsctep_amd.sparse import readout_energy
    net, ws = _head(64, [128, 128], 5)
    netf, wsf = net.float().to(DEV), ws.float().to(DEV)
    e = readout_energy(netf, wsf, torch.empty(0, 64, device=DEV))
    assert e.shape == (0, 1)
    small, sws = _head(12, [8, 8], 6)
    small, sws = small.float().to(DEV), sws.float().to(DEV)
    x = torch.randn(5, 12, device=DEV, requires_grad=True)
    e = readout_energy(small, sws, x)
    assert "ReadoutMlp" not in e.grad_fn.name()
    assert torch.equal(e, sws(small(x)))
