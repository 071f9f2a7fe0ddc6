"""The fused readout op (Gram inputs gathered through the readout column map, per-key Gram bilinears
summed, per-key squared norms; backward by the Gram backward and one scatter kernel) against an fp64
torch evaluation of the reference readout glue (slicing, concatenation, re-split, materialised Gram
matrix, (T*T).sum(1); models/pure_cartesian_sparse_layers.py:769-833,
models/pure_cartesian_ictd_layers_full.py:977-1024)."""

import math

import pytest
import torch

from fsctep_amd.readout_ops import ReadoutMaps, readout_features
from test_readout_maps import ictd_reference_inputs, sparse_reference_blocks

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def rel(a, b):
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    return float((a - b).abs().max() / b.abs().max().clamp(min=1e-30))


def reference(feats, Ws, scales, dims, resplit):
    """scalars = sum_k sum_{ij} W_k[o][i][j] G_k[n][i][j] and sq[n][k][l*C + c] in fp64."""
    ts = ictd_reference_inputs(feats, dims) if resplit else sparse_reference_blocks(feats)
    scal = 0
    for t, W, s in zip(ts, Ws, scales):
        G = s * torch.einsum("nmi,nmj->nij", t, t)
        scal = scal + torch.einsum("oij,nij->no", W, G)
    sq, off = [], 0
    for d in dims:
        T = torch.cat([f[:, off:off + d, :] for f in feats], dim=2)
        sq.append((T * T).sum(1))
        off += d
    return scal, torch.stack(sq, dim=1)


@pytest.mark.parametrize("case", ["sparse", "ictd", "ictd_small"])
def test_readout_features_forward_and_backward(case):
    if case == "sparse":
        dims, C, nL, S, resplit, N = [1, 3, 9], 64, 3, 64, False, 517
    elif case == "ictd":
        dims, C, nL, S, resplit, N = [1, 3, 5, 7], 32, 3, 64, True, 333
    else:
        dims, C, nL, S, resplit, N = [1, 3, 3, 5], 16, 2, 32, True, 129
    g = torch.Generator().manual_seed(len(case) + C)
    M, nC = sum(dims), nL * C
    feats = [torch.randn(N, M, C, generator=g, dtype=torch.float64) for _ in range(nL)]
    Ws = [torch.randn(S, nC, nC, generator=g, dtype=torch.float64) * 0.05 for _ in dims]
    scales = [1.0 / math.sqrt(d) for d in dims]
    gs = torch.randn(N, S, generator=g, dtype=torch.float64)
    gq = torch.randn(N, len(dims), nC, generator=g, dtype=torch.float64)

    fr = [f.clone().requires_grad_(True) for f in feats]
    scal_r, sq_r = reference(fr, Ws, scales, dims, resplit)
    dref = torch.autograd.grad((scal_r * gs).sum() + (sq_r * gq).sum(), fr)

    maps = ReadoutMaps(nL, C, dims, resplit=resplit)
    fd = [f.float().to(DEV).requires_grad_(True) for f in feats]
    grams = [torch.ops.fsctep.gram_prepare_weights(W.float().to(DEV)) for W in Ws]
    scal, sq = readout_features(fd, grams, scales, maps)
    d = torch.autograd.grad((scal * gs.float().to(DEV)).sum() + (sq * gq.float().to(DEV)).sum(), fd,
                            retain_graph=True)
    assert rel(scal, scal_r) < 1e-5
    assert rel(sq, sq_r) < 1e-5
    for a, b in zip(d, dref):
        assert rel(a, b) < 1e-5
    # only one of the two outputs feeding the loss
    (d1,) = torch.autograd.grad((sq * gq.float().to(DEV)).sum(), fd[:1])
    assert rel(d1, 2 * feats[0] * _sq_grad_expand(gq, dims, 0, C)) < 1e-5


def _sq_grad_expand(gq, dims, layer, C):
    """d/dX_l of sum(sq * gq): 2 X_l[n][m][c] gq[n][k(m)][l*C + c]; returns gq expanded to (N, M, C)."""
    parts = []
    for k, d in enumerate(dims):
        parts.append(gq[:, k:k + 1, layer * C:(layer + 1) * C].expand(-1, d, -1))
    return torch.cat(parts, dim=1)


def test_readout_features_misaligned_views():
    """Feature layers that are views at an odd float offset (not 16-byte aligned) take the blocked
    gather after a copy and give the same scalars, norms and gradients as aligned tensors, bit for bit;
    with autograd off (the op's own device kernel) too."""
    dims, C, nL, S, N = [1, 3, 9], 64, 3, 64, 300
    M, nC = sum(dims), nL * C
    g = torch.Generator(device=DEV).manual_seed(11)
    feats = [torch.randn(N, M, C, device=DEV, generator=g) for _ in range(nL)]
    grams = [torch.ops.fsctep.gram_prepare_weights(torch.randn(S, nC, nC, device=DEV, generator=g) * 0.05)
             for _ in dims]
    scales = [1.0 / math.sqrt(d) for d in dims]
    maps = ReadoutMaps(nL, C, dims, resplit=False)
    views = []
    for f in feats:
        buf = torch.empty(f.numel() + 1, device=DEV)
        v = buf[1:].view(N, M, C)
        v.copy_(f)
        assert v.data_ptr() % 16 != 0
        views.append(v)
    gs = torch.randn(N, S, device=DEV, generator=g)
    outs = []
    for src in (feats, views):
        x = [t.detach().requires_grad_(True) for t in src]
        scal, sq = readout_features(x, grams, scales, maps)
        d = torch.autograd.grad((scal * gs).sum() + sq.sum(), x)
        with torch.inference_mode():   # autograd keys excluded: the op's device kernel itself
            scal0, sq0 = readout_features([t.detach() for t in src], grams, scales, maps)
        outs.append((scal, sq, d, scal0, sq0))
    (a_s, a_q, a_d, a_s0, a_q0), (b_s, b_q, b_d, b_s0, b_q0) = outs
    assert torch.equal(a_s, b_s) and torch.equal(a_q, b_q)
    assert torch.equal(a_s0, a_s) and torch.equal(b_s0, b_s) and torch.equal(b_q0, b_q)
    for u, w in zip(a_d, b_d):
        assert torch.equal(u, w)
