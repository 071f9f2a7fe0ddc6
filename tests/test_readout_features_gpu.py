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
