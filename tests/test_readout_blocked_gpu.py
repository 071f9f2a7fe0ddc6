"""The blocked Gram-input entry points through the C ABI (fsc_readout_gather_blocked,
fsc_gram_forward_blocked, fsc_gram_backward_blocked) against the standard-layout ones: the blocked
gather must write exactly the quad-major transpose [nC/4][d_k][N][4] of each standard t_k
[N][d_k][nC] and the same squared norms, and the blocked Gram products must equal the standard ones
bit for bit (the same arithmetic in the same order, only the operand addresses differ).  The
standard entry points are checked against the PyTorch evaluation of the reference formula in
test_readout_gpu.py and test_readout_assembly_gpu.py."""

import ctypes

import pytest
import torch

from fsctep_amd import _lib
from fsctep_amd.readout_ops import FscReadoutTable, ReadoutMaps

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _blocked(t):
    """(N, D, nC) -> the quad-major order [nC/4][D][N][4], flattened."""
    N, D, nC = t.shape
    return t.reshape(N, D, nC // 4, 4).permute(2, 1, 0, 3).contiguous().reshape(-1)


def _table(maps):
    t = FscReadoutTable()
    ctypes.memmove(ctypes.addressof(t), (ctypes.c_int32 * len(maps.table))(*maps.table), ctypes.sizeof(t))
    return t


def _gather(name, maps, X, srcmap):
    N, nC = X[0].shape[0], maps.n_layers * maps.C
    t_all = torch.full((N * maps.M * nC,), float("nan"), device=DEV)
    sq = torch.full((N, len(maps.key_dims), nC), float("nan"), device=DEV)
    layers = (ctypes.c_void_p * len(X))(*[_lib.ptr(x) for x in X])
    T = _table(maps)
    _lib.call(name, ctypes.byref(T), N, layers, _lib.ptr(srcmap), _lib.ptr(t_all), _lib.ptr(sq),
              _lib.stream_handle(DEV))
    torch.cuda.synchronize()
    return t_all, sq


# (key dims, C, n_layers, resplit, N): sparse and ICTD readout rows; N below 8 (no node remap), below
# and above the gather's 2048 blocks, not a multiple of 8
GATHER = {
    "sparse_37": ([1, 3, 9], 64, 3, False, 37),
    "sparse_5": ([1, 3, 9], 64, 3, False, 5),
    "ictd_2051": ([1, 3, 5, 7], 128, 3, True, 2051),
    "ictd_o3_300": ([1, 3, 5, 7], 64, 2, True, 300),
}


@pytest.mark.parametrize("case", sorted(GATHER))
def test_blocked_gather_is_the_transpose(case):
    dims, C, nL, resplit, N = GATHER[case]
    print(f"blocked gather {case}", flush=True)
    maps = ReadoutMaps(nL, C, dims, resplit=resplit)
    srcmap, _ = maps.on(DEV)
    g = torch.Generator(device=DEV).manual_seed(N)
    X = [torch.randn(N, maps.M, C, device=DEV, generator=g) for _ in range(nL)]
    t_std, sq_std = _gather("fsc_readout_gather", maps, X, srcmap)
    t_blk, sq_blk = _gather("fsc_readout_gather_blocked", maps, X, srcmap)
    nC, off = nL * C, 0
    for d in dims:
        n = N * d * nC
        assert torch.equal(t_blk[off:off + n], _blocked(t_std[off:off + n].view(N, d, nC)))
        off += n
    assert torch.equal(sq_blk, sq_std)


def test_blocked_gather_refuses_long_rows():
    maps = ReadoutMaps(4, 256, [1, 3, 5, 7], resplit=True)   # 16384 entries a node
    srcmap, _ = maps.on(DEV)
    X = [torch.zeros(3, maps.M, 256, device=DEV) for _ in range(4)]
    with pytest.raises(RuntimeError, match="fsc_readout_gather_blocked"):
        _gather("fsc_readout_gather_blocked", maps, X, srcmap)


# (N, D, nC, S): few nodes (the first four: fp32 forward kernel), many nodes (the rest: split-fp16
# forward, 3500 nodes with chunks of 8 block pairs, the others of 16), partial tiles, D 1..9, nC 16 (one
# block), the 10k-atom channel widths
GRAM = [(70, 1, 64, 32), (130, 9, 192, 64), (1, 3, 16, 64), (1100, 5, 128, 32), (3500, 3, 192, 64),
        (2500, 7, 384, 64), (2000, 5, 384, 32), (6700, 9, 192, 64), (7100, 1, 192, 64)]


@pytest.mark.parametrize("N,D,nC,S", GRAM)
def test_blocked_gram_matches_standard(N, D, nC, S):
    print(f"blocked gram N={N} D={D} nC={nC} S={S}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(N + D)
    t = torch.randn(N, D, nC, device=DEV, generator=g)
    t[::7] *= 1e-3                                  # per-node scales spread over a few binades
    W = torch.randn(S, nC, nC, device=DEV, generator=g) * 0.02
    G = torch.randn(N, S, device=DEV, generator=g)
    st = _lib.stream_handle(DEV)
    wf, wb, ws = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
    _lib.call("fsc_gram_sizes", N, nC, S, ctypes.byref(wf), ctypes.byref(wb), ctypes.byref(ws))
    Wf = torch.empty(wf.value, device=DEV)
    Wb = torch.empty(wb.value, device=DEV)
    _lib.call("fsc_gram_prepare_weights", _lib.ptr(W), S, nC, _lib.ptr(Wf), _lib.ptr(Wb), st)
    tb = _blocked(t)
    scale = 1.0 / D ** 0.5
    outs, grads = [], []
    for fwd, bwd, src in (("fsc_gram_forward", "fsc_gram_backward", t),
                          ("fsc_gram_forward_blocked", "fsc_gram_backward_blocked", tb)):
        part = torch.empty(max(ws.value, 1), device=DEV)
        out = torch.full((N, S), float("nan"), device=DEV)
        dt = torch.full((N, D, nC), float("nan"), device=DEV)
        _lib.call(fwd, N, D, nC, S, ctypes.c_float(scale), _lib.ptr(src), _lib.ptr(Wf), _lib.ptr(part),
                  _lib.ptr(out), st)
        _lib.call(bwd, N, D, nC, S, ctypes.c_float(scale), _lib.ptr(G), _lib.ptr(src), _lib.ptr(Wb),
                  _lib.ptr(dt), st)
        torch.cuda.synchronize()
        outs.append(out)
        grads.append(dt)
    assert torch.isfinite(outs[0]).all() and torch.isfinite(grads[0]).all()
    assert torch.equal(outs[1], outs[0])
    assert torch.equal(grads[1], grads[0])
