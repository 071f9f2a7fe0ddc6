"""Readout assembly kernels on their own (the readout_gather / readout_scatter ops), against torch
indexing through the same column maps: the permutation must be exact (bit-for-bit), the squared norms
and the backward's 2 X dsq term within fp32 rounding.  Rows of n_layers*M*C entries up to 12288 run in
one block per node out of LDS, larger ones element-wise; both paths are covered."""

import pytest
import torch

from fsctep_amd.readout_ops import ReadoutMaps

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")

CASES = {
    # name: (key dims, C, n_layers, resplit)  -> n_layers*M*C
    "sparse_node": ([1, 3, 9], 64, 3, False),        # 2496: per-node path
    "ictd_node": ([1, 3, 5, 7], 128, 3, True),       # 6144: per-node path
    "ictd_rowwise": ([1, 3, 5, 7], 256, 4, True),    # 16384: element-wise path
    "sparse_rowwise": ([1, 3, 9], 512, 2, False),    # 13312: element-wise path
}


def _key_blocks(flat, maps, N):
    """Key-major gathered buffer t_all (t_0 then t_1 ...; t_k is (N, d_k * nC)) from (N, P) columns."""
    nC = maps.n_layers * maps.C
    out, col0 = [], 0
    for d in maps.key_dims:
        out.append(flat[:, col0:col0 + d * nC].reshape(-1))
        col0 += d * nC
    return torch.cat(out)


@pytest.mark.parametrize("case", sorted(CASES))
def test_gather_and_norms(case):
    dims, C, nL, resplit = CASES[case]
    N = 37
    maps = ReadoutMaps(nL, C, dims, resplit=resplit)
    srcmap, _ = maps.on(DEV)
    g = torch.Generator(device=DEV).manual_seed(len(case))
    X = [torch.randn(N, maps.M, C, device=DEV, generator=g) for _ in range(nL)]
    t_all, sq = torch.ops.fsctep.readout_gather(X, srcmap, maps.table)
    flat = torch.cat([x.reshape(N, -1) for x in X], dim=1)
    assert torch.equal(t_all, _key_blocks(flat[:, srcmap.long()], maps, N))
    ref, c0 = [], 0
    for d in dims:
        ref.append(torch.cat([(x[:, c0:c0 + d, :].double() ** 2).sum(1) for x in X], dim=1))
        c0 += d
    ref = torch.stack(ref, dim=1)
    assert ((sq.double() - ref).abs() / ref.abs().max()).max().item() < 1e-6


@pytest.mark.parametrize("case", sorted(CASES))
@pytest.mark.parametrize("with_sq", [False, True])
def test_scatter(case, with_sq):
    dims, C, nL, resplit = CASES[case]
    N = 29
    maps = ReadoutMaps(nL, C, dims, resplit=resplit)
    _, gmap = maps.on(DEV)
    nC = nL * C
    g = torch.Generator(device=DEV).manual_seed(7 + len(case))
    X = [torch.randn(N, maps.M, C, device=DEV, generator=g) for _ in range(nL)]
    dt = [torch.randn(N, d, nC, device=DEV, generator=g) for d in dims]
    dt[1] = None                      # no gradient through key 1: its entries contribute zero
    dsq = torch.randn(N, len(dims), nC, device=DEV, generator=g) if with_sq else None
    dX = torch.ops.fsctep.readout_scatter(dt, dsq, X, gmap, maps.table)
    cols = torch.cat([(t if t is not None else torch.zeros(N, d, nC, device=DEV)).reshape(N, -1)
                      for t, d in zip(dt, dims)], dim=1)            # (N, P) in key-major column order
    back = cols[:, gmap.long()]                                     # (N, P) in (layer, comp, channel) order
    key_of_comp = torch.repeat_interleave(torch.arange(len(dims), device=DEV), torch.tensor(dims, device=DEV))
    MC = maps.M * C
    for l in range(nL):
        ref = back[:, l * MC:(l + 1) * MC].reshape(N, maps.M, C)
        if not with_sq:
            assert torch.equal(dX[l], ref)
        else:
            q = dsq[:, key_of_comp, l * C:(l + 1) * C]               # (N, M, C)
            ref = ref.double() + 2.0 * X[l].double() * q.double()
            assert ((dX[l].double() - ref).abs() / ref.abs().max()).max().item() < 1e-6
