"""fsc_graph_prepare_noalloc (static device scratch, no allocation) against fsc_graph_prepare (caller
workspace), both called through the C ABI on the current stream: bit-identical outputs on two calls
in a row, the second with a smaller graph (the shared scratch keeps the first call's contents), and
the size limit reported as an argument error."""

import ctypes

import numpy as np
import pytest
import torch

from fsctep_amd import _lib

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs(N, E, NS, seed):
    rng = np.random.default_rng(seed)
    src = torch.from_numpy(rng.integers(0, N, E)).to(DEV)
    dst = torch.from_numpy(rng.integers(0, N, E)).to(DEV)
    dst[: E // 3] = 1                                         # a hub receiver
    species = torch.from_numpy(rng.integers(0, NS, N)).to(DEV)
    return src, dst, species


def _outputs(N, E, NS):
    t, w = ctypes.c_int64(), ctypes.c_int64()
    _lib.call("fsc_graph_sizes", N, E, NS, ctypes.byref(t), ctypes.byref(w))
    T = t.value
    mk = lambda n: torch.full((n,), -7, dtype=torch.int32, device=DEV)   # poisoned: every entry must be written
    outs = dict(order=mk(E), src32=mk(E), dst32=mk(E), dst_ptr=mk(N + 1), src_ptr=mk(N + 1), src_perm=mk(E),
                node_species=mk(N), edge_pair=mk(E), pair_tiles=mk(17 * T), status=mk(1))
    return outs, w.value


def _call(noalloc, N, E, NS, src, dst, species):
    outs, ws_ints = _outputs(N, E, NS)
    p = _lib.ptr
    args = [N, E, NS, p(src), p(dst), p(species)] + [p(outs[k]) for k in ("order", "src32", "dst32", "dst_ptr",
                                                                          "src_ptr", "src_perm", "node_species",
                                                                          "edge_pair", "pair_tiles", "status")]
    stream = _lib.stream_handle(torch.device(DEV))
    if noalloc:
        _lib.call("fsc_graph_prepare_noalloc", *args, stream)
    else:
        ws = torch.empty(ws_ints, dtype=torch.int32, device=DEV)
        _lib.call("fsc_graph_prepare", *args, p(ws), stream)
        torch.cuda.synchronize()
    torch.cuda.synchronize()
    return outs


def test_noalloc_matches_workspace_entry_point_twice():
    for N, E, NS, seed in ((3000, 160000, 10, 1), (700, 20000, 4, 2)):    # second call smaller
        src, dst, species = _inputs(N, E, NS, seed)
        ref = _call(False, N, E, NS, src, dst, species)
        got = _call(True, N, E, NS, src, dst, species)
        assert int(ref["status"][0]) == 0
        for k in ref:
            assert torch.equal(ref[k], got[k]), (N, E, k)
        order = np.argsort(dst.cpu().numpy(), kind="stable")
        np.testing.assert_array_equal(got["order"].cpu().numpy(), order)


def test_noalloc_rejects_graphs_above_the_scratch():
    t, w = ctypes.c_int64(), ctypes.c_int64()
    N, E = 100000, 9_000_000
    _lib.call("fsc_graph_sizes", N, E, 10, ctypes.byref(t), ctypes.byref(w))
    assert w.value > (1 << 23)
    lib = _lib.load()
    rc = lib.fsc_graph_prepare_noalloc(N, E, 10, *([None] * 14))
    assert rc == 1 and b"static scratch" in lib.fsc_last_error()
