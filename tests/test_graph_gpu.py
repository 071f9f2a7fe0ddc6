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


# ---------------------------------------------------------------- spatial node order (fsc_spatial_order)

def _spread3(v):
    v = v.astype(np.int64) & 0xFF
    v = (v | (v << 8)) & 0x0F00F
    v = (v | (v << 4)) & 0x0C30C3
    v = (v | (v << 2)) & 0x249249
    return v


def _morton_order(pos):
    """numpy statement of the order: Morton code of the cell on a G^3 grid over the bounding box of the
    finite coordinates (G the smallest power of two <= 256 with 2 G^3 >= N), ascending id within a cell."""
    N = pos.shape[0]
    G = 1
    while G < 256 and 2 * G ** 3 < N:
        G *= 2
    p = pos.astype(np.float32)
    fin = np.isfinite(p)
    lo = np.array([p[fin[:, k], k].min() if fin[:, k].any() else np.inf for k in range(3)], np.float32)
    hi = np.array([p[fin[:, k], k].max() if fin[:, k].any() else -np.inf for k in range(3)], np.float32)
    c = np.zeros((N, 3), np.int64)
    for k in range(3):
        if hi[k] > lo[k]:
            with np.errstate(invalid="ignore"):
                t = (p[:, k] - lo[k]) * (np.float32(G) / (hi[k] - lo[k]))
            t = np.where(np.isnan(t), np.float32(0), t)
            c[:, k] = np.clip(t, 0, G - 1).astype(np.int64)
    code = _spread3(c[:, 0]) | (_spread3(c[:, 1]) << 1) | (_spread3(c[:, 2]) << 2)
    return np.argsort(code, kind="stable")


@pytest.mark.gpu
@pytest.mark.parametrize("N,kind", [(1, "box"), (7, "box"), (1000, "box"), (10000, "box"), (3000, "zeros"),
                                    (500, "nan"), (40000, "slab")])
def test_spatial_order_is_the_morton_permutation(N, kind):
    rng = np.random.default_rng(N)
    pos = rng.uniform(-3.0, 40.0, (N, 3)).astype(np.float32)
    if kind == "zeros":
        pos[:] = 0.0                               # edge-vector callers pass zero positions: identity
    elif kind == "nan":
        pos[::7, 1] = np.nan
    elif kind == "slab":
        pos[:, 2] *= 0.01
    order = torch.ops.fsctep.spatial_order(torch.from_numpy(pos).to(DEV)).cpu().numpy()
    np.testing.assert_array_equal(np.sort(order), np.arange(N))
    np.testing.assert_array_equal(order, _morton_order(pos))
    if kind == "zeros":
        np.testing.assert_array_equal(order, np.arange(N))


@pytest.mark.gpu
def test_conv_results_do_not_depend_on_the_node_order():
    """The per-node kernels walk graph.node_order: energies and forces are bitwise those of the identity."""
    import bench
    from fsctep_amd.ictd import energy_forces
    from fsctep_amd.sparse import energy_and_forces
    for mode, atoms in (("sparse", 1500), ("ictd-o3", 1200)):
        w = bench.WORKLOADS[mode]
        s = bench._system(mode, atoms, w["seed"])
        model = bench.build_model(mode, torch.device(DEV))
        pos = torch.tensor(s.pos, dtype=torch.float32, device=DEV)
        A = torch.tensor(s.species, device=DEV)
        batch = torch.zeros(atoms, dtype=torch.long, device=DEV)
        cell = torch.tensor(s.cell, dtype=torch.float32, device=DEV)
        args = (torch.tensor(s.edge_src, device=DEV), torch.tensor(s.edge_dst, device=DEV),
                torch.tensor(s.edge_shifts, dtype=torch.float32, device=DEV), atoms, A)
        g0 = model.prepare(*args)
        g1 = model.prepare(*args, pos=pos)
        assert g0.node_order.numel() == 0 and g1.node_order.numel() == atoms
        assert not torch.equal(g1.node_order.cpu(), torch.arange(atoms, dtype=torch.int32))
        if mode == "sparse":
            r0, r1 = (energy_and_forces(model, pos, batch, cell, g) for g in (g0, g1))
        else:
            fld = torch.tensor(bench._field(1, w["seed"]), dtype=torch.float32, device=DEV)
            r0, r1 = (energy_forces(model, pos, batch, cell, g, external_tensor=fld)[:2] for g in (g0, g1))
        assert torch.equal(r0[0], r1[0]) and torch.equal(r0[1], r1[1]), mode
