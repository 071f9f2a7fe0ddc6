"""Column maps of the fused readout (host logic, no GPU): gathering the per-layer features through
``ReadoutMaps.srcmap`` reproduces the Gram inputs the reference readouts build by slicing,
concatenating and re-splitting (models/pure_cartesian_sparse_layers.py:769-833,
models/pure_cartesian_ictd_layers_full.py:977-1001), and ``gmap`` inverts it."""

import numpy as np
import pytest
import torch

from fsctep_amd.readout_ops import ReadoutMaps


def gather(maps, feats):
    N = feats[0].shape[0]
    flat = torch.cat([f.reshape(N, -1) for f in feats], dim=1)
    t_all = flat[:, maps.srcmap.long()]
    out, col0 = [], 0
    nC = maps.n_layers * maps.C
    for d in maps.key_dims:
        out.append(t_all[:, col0:col0 + d * nC].reshape(N, d, nC))
        col0 += d * nC
    return out


def sparse_reference_blocks(feats):
    comps = [(0, 1), (1, 4), (4, 13)]
    return [torch.cat([f[:, a:b, :] for f in feats], dim=2) for (a, b) in comps]


def ictd_reference_inputs(feats, dims):
    """Channel-major flatten per key, layer concatenation, re-split by key, transpose."""
    N, C = feats[0].shape[0], feats[0].shape[2]
    nC = C * len(feats)

    def ref_flat(f):
        parts, off = [], 0
        for d in dims:
            parts.append(f[:, off:off + d, :].transpose(1, 2).reshape(N, -1))
            off += d
        return torch.cat(parts, dim=-1)

    fc = torch.cat([ref_flat(f) for f in feats], dim=-1)
    out, off = [], 0
    for d in dims:
        out.append(fc[:, off:off + nC * d].reshape(N, nC, d).transpose(1, 2))
        off += nC * d
    return out


def test_sparse_map_is_the_layer_concatenation():
    g = torch.Generator().manual_seed(0)
    feats = [torch.randn(5, 13, 8, generator=g) for _ in range(3)]
    maps = ReadoutMaps(3, 8, [1, 3, 9], resplit=False)
    for got, ref in zip(gather(maps, feats), sparse_reference_blocks(feats)):
        assert torch.equal(got, ref)


@pytest.mark.parametrize("dims,layers", [([1, 3, 5, 7], 3), ([1, 3, 3, 5], 3), ([1, 3, 5], 2), ([1, 3], 4)])
def test_ictd_map_is_the_reference_resplit(dims, layers):
    g = torch.Generator().manual_seed(1)
    C = 4
    feats = [torch.randn(3, sum(dims), C, generator=g) for _ in range(layers)]
    maps = ReadoutMaps(layers, C, dims, resplit=True)
    for got, ref in zip(gather(maps, feats), ictd_reference_inputs(feats, dims)):
        assert torch.equal(got, ref)


def test_resplit_mixes_keys_and_layers():
    """The re-split is not the per-key layer concatenation (it takes columns across key boundaries)."""
    maps_r = ReadoutMaps(3, 4, [1, 3, 5, 7], resplit=True)
    maps_s = ReadoutMaps(3, 4, [1, 3, 5, 7], resplit=False)
    assert not torch.equal(maps_r.srcmap, maps_s.srcmap)


@pytest.mark.parametrize("resplit", [False, True])
def test_gmap_inverts_srcmap(resplit):
    maps = ReadoutMaps(3, 16, [1, 3, 5, 7], resplit=resplit)
    src, gm = maps.srcmap.numpy(), maps.gmap.numpy()
    assert np.array_equal(gm[src], np.arange(src.size))
    assert sorted(src.tolist()) == list(range(3 * 16 * 16))


def test_resplit_moves_entries_across_keys():
    """With the re-split some component's entries land in another key's Gram input, so the backward
    must locate the destination key from the column, not from the component."""
    dims, C, nL = [1, 3, 5, 7], 4, 3
    maps = ReadoutMaps(nL, C, dims, resplit=True)
    nC, M = nL * C, sum(dims)
    comp_key = np.repeat(np.arange(len(dims)), dims)
    col_key = np.repeat(np.arange(len(dims)), [d * nC for d in dims])
    src = maps.srcmap.numpy()
    m_of_src = (src % (M * C)) // C
    assert (comp_key[m_of_src] != col_key).any()
    sparse = ReadoutMaps(nL, C, dims, resplit=False).srcmap.numpy()
    assert (comp_key[(sparse % (M * C)) // C] == col_key).all()


def test_table_layout():
    maps = ReadoutMaps(3, 64, [1, 3, 9], resplit=False)
    t = np.asarray(maps.table)
    assert t[:4].tolist() == [3, 13, 64, 3]
    assert t[4:7].tolist() == [0, 1, 4] and t[12:15].tolist() == [1, 3, 9]
