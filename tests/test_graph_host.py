"""Host logic of the receiver-sorted graph: CSR pointers, the source grouping and the
species-pair tiles consumed by the sparse conv1 kernels (CPU only)."""

import torch

from fsctep_amd.graph import pair_tiles, prepare_graph


def _random_graph(N, E, S, seed):
    g = torch.Generator().manual_seed(seed)
    src = torch.randint(0, N, (E,), generator=g)
    dst = torch.randint(0, N, (E,), generator=g)
    species = torch.tensor([1, 6, 7, 8][:S])[torch.randint(0, S, (N,), generator=g)]
    return src, dst, torch.zeros(E, 3), species


def test_csr_and_source_grouping():
    src, dst, sh, sp = _random_graph(50, 400, 4, 0)
    g = prepare_graph(src, dst, sh, 50, species=sp)
    assert torch.all(g.dst[1:] >= g.dst[:-1])
    assert torch.equal(g.dst_ptr.long()[1:] - g.dst_ptr.long()[:-1], torch.bincount(g.dst, minlength=50))
    srcs = g.src[g.src_perm.long()]
    assert torch.all(srcs[1:] >= srcs[:-1])
    for m in range(50):
        a, b = int(g.src_ptr[m]), int(g.src_ptr[m + 1])
        assert torch.all(g.src[g.src_perm[a:b].long()] == m)
    # the receiver sort is stable: edges of one receiver keep their input order
    order = torch.argsort(dst, stable=True)
    assert torch.equal(g.src, src[order])


def test_pair_tiles_cover_every_edge_once():
    for E, seed in ((0, 1), (1, 2), (15, 3), (16, 4), (17, 5), (999, 6)):
        src, dst, sh, sp = _random_graph(40, E, 3, seed)
        g = prepare_graph(src, dst, sh, 40, species=sp)
        t = g.pair_tiles.long()
        assert t.numel() % 17 == 0
        T = t.numel() // 17
        ids, tp = t[:16 * T].view(T, 16), t[16 * T:]
        real = ids[ids >= 0]
        assert torch.equal(torch.sort(real).values, torch.arange(E))        # each edge exactly once
        assert torch.all(ids[:, 0] >= 0)                                    # tiles start with an edge
        for k in range(T):                                                  # one pair per tile
            e = ids[k][ids[k] >= 0]
            assert torch.all(g.edge_pair[e].long() == tp[k])
        # tiles of one pair are contiguous and padded only at the pair's end
        assert torch.all(tp[1:] >= tp[:-1])


def test_pair_tiles_counts():
    ep = torch.tensor([3, 0, 3, 3, 0, 2] + [1] * 20, dtype=torch.int32)
    t = pair_tiles(ep, 4).long()
    T = t.numel() // 17
    assert T == 1 + 2 + 1 + 1            # pair 0: 2 edges, pair 1: 20, pair 2: 1, pair 3: 3
    assert t[16 * T:].tolist() == [0, 1, 1, 2, 3]
    assert t[:16].tolist()[:2] == [1, 4] and t[2:16].tolist() == [-1] * 14
