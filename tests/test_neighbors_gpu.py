"""The GPU radius graph (``fsctep_amd.neighbors``, cell list in ``csrc/neighbors.hip``) against the host
list of ``fsctep_amd.synthetic.radius_graph`` (scipy cKDTree, minimum image) and against a brute-force
numpy statement of the reference semantics (utils/graph_utils.py:192-257: every image s in {-1,0,1} on
periodic axes, |pos[j] + s @ cell - pos[i]| < r, no self pair at s = 0).  Integer output: bit-exact, in
the same receiver-sorted order (then by source and image)."""

import time

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _gpu(pos, cell, r, pbc=None):
    from fsctep_amd.neighbors import neighbor_csr
    src, dst, sh, dst_ptr = neighbor_csr(torch.tensor(pos, dtype=torch.float64, device=DEV),
                                         r, torch.tensor(np.asarray(cell).reshape(3, 3), dtype=torch.float64), pbc)
    return src.cpu().numpy(), dst.cpu().numpy(), sh.cpu().numpy(), dst_ptr.cpu().numpy()


def _brute(pos, cell, r, pbc):
    """The reference's edge set by brute force over all pairs and images, sorted (dst, src, shift)."""
    cell = np.asarray(cell, np.float64).reshape(3, 3)
    rng = [(-1, 0, 1) if p else (0,) for p in pbc]
    S, D, SH = [], [], []
    for sx in rng[0]:
        for sy in rng[1]:
            for sz in rng[2]:
                s = np.array([sx, sy, sz], np.float64)
                sv = (s[0] * cell[0] + s[1] * cell[1]) + s[2] * cell[2]
                d = (pos[None, :, :] - pos[:, None, :]) + sv          # [i][j] = (pos_j - pos_i) + s.cell
                d2 = (d[..., 0] * d[..., 0] + d[..., 1] * d[..., 1]) + d[..., 2] * d[..., 2]
                m = d2 < r * r
                if not s.any():
                    np.fill_diagonal(m, False)
                ii, jj = np.nonzero(m)
                S.append(ii)
                D.append(jj)
                SH.append(np.broadcast_to(s, (ii.shape[0], 3)))
    src, dst, sh = np.concatenate(S), np.concatenate(D), np.concatenate(SH)
    o = np.lexsort((sh[:, 2], sh[:, 1], sh[:, 0], src, dst))
    return src[o], dst[o], sh[o]


def _equal(got, want, N):
    src, dst, sh, dst_ptr = got
    np.testing.assert_array_equal(dst, want[1])
    np.testing.assert_array_equal(src, want[0])
    np.testing.assert_array_equal(sh, want[2])
    np.testing.assert_array_equal(dst_ptr, np.concatenate([[0], np.cumsum(np.bincount(want[1], minlength=N))]))


@pytest.mark.parametrize("mode,atoms", [("sparse", 1000), ("sparse", 10000), ("ictd-o3", 4000)])
def test_matches_host_list_of_the_benchmark_systems(mode, atoms):
    import bench
    s = bench._system(mode, atoms, bench.WORKLOADS[mode]["seed"])
    got = _gpu(s.pos, s.cell, 5.0)
    _equal(got, (s.edge_src, s.edge_dst, s.edge_shifts), atoms)
    # the timed rebuild (count pass, edge-count read back, fill pass)
    from fsctep_amd.neighbors import radius_graph_pbc_gpu
    pos = torch.tensor(s.pos, dtype=torch.float64, device=DEV)
    cell = torch.tensor(s.cell, dtype=torch.float64, device=DEV)
    radius_graph_pbc_gpu(pos, 5.0, cell)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(5):
        radius_graph_pbc_gpu(pos, 5.0, cell)
    torch.cuda.synchronize()
    print(f"{mode} {atoms} atoms, {got[0].shape[0]} edges: rebuild {(time.perf_counter() - t0) / 5 * 1e3:.3f} ms")


def test_small_box_many_images_and_open_system():
    from fsctep_amd.synthetic import radius_graph
    rng = np.random.default_rng(3)
    # box 7 A < 2 r: several images of one pair within the cutoff (the host's brute-force branch)
    pos = rng.uniform(0.0, 7.0, (40, 3))
    cell = np.eye(3)[None] * 7.0
    want = radius_graph(pos, cell, True, 5.0)
    _equal(_gpu(pos, cell, 5.0), want, 40)
    _equal(_gpu(pos, cell, 5.0), _brute(pos, cell, 5.0, (1, 1, 1)), 40)
    # open system (kd-tree branch of the host list)
    pos = rng.uniform(0.0, 20.0, (300, 3))
    want = radius_graph(pos, np.eye(3)[None] * 100.0, False, 5.0)
    _equal(_gpu(pos, np.eye(3) * 100.0, 5.0, pbc=False), want, 300)


@pytest.mark.parametrize("pbc", [(1, 1, 1), (1, 1, 0), (0, 0, 0), (0, 1, 0)])
def test_triclinic_partial_pbc_unwrapped_positions(pbc):
    rng = np.random.default_rng(sum(pbc) + 10)
    cell = np.array([[11.0, 0.0, 0.0], [3.1, 10.2, 0.0], [-2.2, 1.7, 12.5]])
    frac = rng.uniform(-0.1, 1.1, (220, 3))                   # some atoms outside the cell
    pos = frac @ cell
    _equal(_gpu(pos, cell, 4.5, pbc), _brute(pos, cell, 4.5, pbc), 220)


def test_degenerate_inputs():
    cell = np.eye(3) * 10.0
    for N in (0, 1):
        src, dst, sh, dst_ptr = _gpu(np.zeros((N, 3)) + 1.0, cell, 5.0)
        assert src.shape == (0,) and sh.shape == (0, 3) and dst_ptr.tolist() == [0] * (N + 1)
    # one atom in a box smaller than the cutoff sees its own images (s != 0), as in the reference
    got = _gpu(np.array([[0.5, 0.5, 0.5]]), np.eye(3) * 4.0, 5.0)
    _equal(got, _brute(np.array([[0.5, 0.5, 0.5]]), np.eye(3) * 4.0, 5.0, (1, 1, 1)), 1)
    assert got[0].shape[0] == 6                               # the 6 face images at 4 A (edge images: 5.66 A)
    # all atoms at one point (no extent): every pair at distance 0
    got = _gpu(np.zeros((5, 3)), cell, 1.0, pbc=False)
    assert got[0].shape[0] == 20


def test_feeds_graph_preparation_unchanged():
    """The list is already receiver-sorted and stable: prepare_graph's order is the identity."""
    import bench
    from fsctep_amd.graph import prepare_graph
    s = bench._system("sparse", 1000, 22)
    src, dst, sh, _ = [torch.as_tensor(a).to(DEV) for a in _gpu(s.pos, s.cell, 5.0)]
    g = prepare_graph(src, dst, sh, 1000)
    assert torch.equal(g.order.cpu(), torch.arange(src.shape[0], dtype=torch.int32))
