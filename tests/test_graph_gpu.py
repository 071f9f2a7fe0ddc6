"""Graph preparation on the device (``fsc_graph_prepare``): the receiver sort must equal numpy's stable
argsort of ``edge_dst`` (the reference sorts with ``argsort(edge_dst)``,
models/pure_cartesian_sparse_layers.py:745-748), the CSR pointers the bincount prefix sums, the source
grouping the stable argsort of the sorted sources, and the species-pair tiles must list every edge once.
Integer results: bit-exact.  The sizes query and the Meta kernel run without a GPU."""

import ctypes

import numpy as np
import pytest
import torch

from fsctep_amd import _lib

DEV = "cuda"


def _graph(N, E, NS, seed, hub=None):
    rng = np.random.default_rng(seed)
    src = rng.integers(0, N, E)
    dst = rng.integers(0, N, E)
    if hub is not None and E:
        dst[: E // 2] = hub                      # one receiver with half the edges
        src[E // 2: 3 * E // 4] = hub            # and a quarter of the sources
    if N > 1 and E:
        dst[dst == N - 1] = 0                    # node N-1 receives nothing
    species = rng.integers(0, NS, N) if NS else np.zeros(N, dtype=np.int64)
    return src.astype(np.int64), dst.astype(np.int64), species.astype(np.int64)


def _run(src, dst, species, NS):
    from fsctep_amd.graph import prepare_graph
    E = src.shape[0]
    sh = torch.arange(3 * E, dtype=torch.float32).view(E, 3)
    return prepare_graph(torch.from_numpy(src).to(DEV), torch.from_numpy(dst).to(DEV), sh.to(DEV),
                         species.shape[0], species=torch.from_numpy(species).to(DEV), n_species=NS), sh


def _check(src, dst, species, NS, g, sh):
    N, E = species.shape[0], src.shape[0]
    order = np.argsort(dst, kind="stable")
    np.testing.assert_array_equal(g.order.cpu().numpy(), order)
    s_sorted, d_sorted = src[order], dst[order]
    np.testing.assert_array_equal(g.src32.cpu().numpy(), s_sorted)
    np.testing.assert_array_equal(g.dst32.cpu().numpy(), d_sorted)
    np.testing.assert_array_equal(g.shifts.cpu().numpy(), sh.numpy()[order])
    np.testing.assert_array_equal(g.dst_ptr.cpu().numpy(), np.concatenate([[0], np.cumsum(np.bincount(dst, minlength=N))]))
    np.testing.assert_array_equal(g.src_ptr.cpu().numpy(), np.concatenate([[0], np.cumsum(np.bincount(src, minlength=N))]))
    np.testing.assert_array_equal(g.src_perm.cpu().numpy(), np.argsort(s_sorted, kind="stable"))
    assert int(g.status.cpu()[0]) == 0
    if NS:
        np.testing.assert_array_equal(g.node_species.cpu().numpy(), species)
        pair = species[s_sorted] * NS + species[d_sorted]
        np.testing.assert_array_equal(g.edge_pair.cpu().numpy(), pair)
        t = g.pair_tiles.cpu().numpy()
        T = t.shape[0] // 17
        assert t.shape[0] == 17 * T and T == (E + 15) // 16 + NS * NS
        ids, tp = t[:16 * T].reshape(T, 16), t[16 * T:]
        np.testing.assert_array_equal(np.sort(ids[ids >= 0]), np.arange(E))     # every edge exactly once
        used = ids[:, 0] >= 0
        n_used = int(used.sum())
        assert used[:n_used].all() and not used[n_used:].any()                  # unused tiles last
        assert (ids[n_used:] == -1).all() and (tp[n_used:] == 0).all()
        assert n_used == int(sum((np.bincount(pair, minlength=NS * NS) + 15) // 16))
        assert (np.diff(tp[:n_used]) >= 0).all()                                # a pair's tiles are contiguous
        for k in range(n_used):
            e = ids[k][ids[k] >= 0]
            assert (pair[e] == tp[k]).all()
            assert (ids[k][: e.shape[0]] >= 0).all()                           # padding only at the end
        real = ids[ids >= 0]
        np.testing.assert_array_equal(real, np.argsort(pair, kind="stable"))   # ascending within a pair


@pytest.mark.gpu
@pytest.mark.parametrize("N,E,NS,seed,hub", [(50, 400, 4, 0, None), (40, 0, 3, 1, None), (40, 1, 3, 2, None),
                                              (40, 15, 3, 3, None), (40, 16, 3, 4, None), (40, 17, 10, 5, None),
                                              (300, 9000, 10, 6, 7), (1, 5, 1, 7, None), (2000, 104000, 16, 8, None),
                                              (37, 500, 0, 9, 3)])
def test_graph_prepare_matches_stable_sort(N, E, NS, seed, hub):
    src, dst, species = _graph(N, E, NS, seed, hub)
    g, sh = _run(src, dst, species, NS)
    _check(src, dst, species, NS, g, sh)
    g2, _ = _run(src, dst, species, NS)             # deterministic: a second call gives the same bits
    for a, b in ((g.order, g2.order), (g.src_perm, g2.src_perm), (g.dst_ptr, g2.dst_ptr)):
        assert torch.equal(a, b)


@pytest.mark.gpu
def test_graph_prepare_flags_out_of_range_ids():
    src, dst, species = _graph(20, 100, 4, 11)
    dst[3], src[5], species[2] = 20, -1, 4
    g, _ = _run(src, dst, species, 4)
    assert int(g.status.cpu()[0]) == 3
    for t, hi in ((g.src32, 20), (g.dst32, 20), (g.node_species, 4), (g.edge_pair, 16)):
        a = t.cpu().numpy()
        assert a.min() >= 0 and a.max() < hi
    from fsctep_amd.graph import poison_invalid
    e = torch.ones(20, 1, device=DEV)
    assert torch.isnan(poison_invalid(e, g)).all()


def test_graph_sizes_without_gpu():
    lib = _lib.load()
    t, w = ctypes.c_int64(), ctypes.c_int64()
    assert lib.fsc_graph_sizes(10000, 519338, 10, ctypes.byref(t), ctypes.byref(w)) == 0
    assert t.value == (519338 + 15) // 16 + 100
    nb, nchunk = (10000 + 1 + 2047) // 2048, (519338 + 2047) // 2048
    assert w.value == 4 * 10000 + 2 * nb + 2 * 100 + 100 * nchunk + 519338
    assert lib.fsc_graph_sizes(10, 10, 17, ctypes.byref(t), ctypes.byref(w)) == 1
    assert b"n_species" in lib.fsc_last_error()


def test_graph_prepare_meta_shapes():
    from torch._subclasses.fake_tensor import FakeTensorMode
    _lib.load_torch_ops()
    with FakeTensorMode():
        src = torch.empty(100, dtype=torch.long)
        out = torch.ops.fsctep.graph_prepare(src, src, torch.empty(12, dtype=torch.long), 4)
        shapes = [tuple(o.shape) for o in out]
    assert shapes == [(100,), (100,), (100,), (13,), (13,), (100,), (12,), (100,), (17 * (7 + 16),), (1,)]
    assert all(o.dtype == torch.int32 for o in out)
