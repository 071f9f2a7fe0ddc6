"""The C ABI library loads (no GPU needed) and exports every symbol of include/fsctep.h;
the model mirror holds the reference's state_dict keys and shapes."""

import ctypes
import json
import os
import re

import pytest
import torch

from conftest import GOLDEN, ROOT
from fsctep_amd import _lib


def header_symbols():
    text = open(os.path.join(ROOT, "include", "fsctep.h")).read()
    return sorted(set(re.findall(r"\b(fsc_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    syms = header_symbols()
    assert len(syms) >= 9
    for s in syms:
        assert hasattr(lib, s), s
    assert lib.fsc_abi_version() == 2
    # every declared entry point has a ctypes signature (or is a metadata call)
    for s in syms:
        assert s in _lib.SIGNATURES or s in ("fsc_last_error", "fsc_abi_version"), s


def test_argument_errors_are_reported_without_a_gpu():
    lib = _lib.load()
    s, p = ctypes.c_int64(), ctypes.c_int64()
    assert lib.fsc_sparse_conv_workspace(10, 20, 64, ctypes.byref(s), ctypes.byref(p)) == 0
    # the tail holds ks partial input gradients of the node-expansion gradient: ks = 16 for ten nodes (six
    # row tiles), 2 from about 5,000 nodes on; below 2,048 nodes the message gradient is split over 2 (4 up
    # to 256 nodes) blocks per node, whose partial dh (E x 64), dn (E x 3) and dS maxima (N) follow,
    # 256-byte aligned
    tail = 10 * 18 * 65 * 64 + 16 * 18 * 10 * 64 + 10
    assert s.value == (tail + 63) // 64 * 64 + 4 * (20 * 67 + 10) and p.value == 20 * 18 * 64
    assert lib.fsc_sparse_conv_workspace(10000, 20, 64, ctypes.byref(s), ctypes.byref(p)) == 0
    assert s.value == 10000 * 18 * 65 * 64 + 2 * 18 * 10000 * 64 + 10000
    assert lib.fsc_sparse_conv_workspace(10, 20, 48, ctypes.byref(s), ctypes.byref(p)) == 1
    assert b"channels" in lib.fsc_last_error()
    with pytest.raises(RuntimeError, match="negative"):
        _lib.call("fsc_sparse_conv_workspace", -1, 0, 64, ctypes.byref(s), ctypes.byref(p))


@pytest.mark.parametrize("name,channels,layers", [("sparse_open32_c32_l2", 32, 2), ("sparse_pbc100_c64_l3", 64, 3)])
def test_state_dict_keys_match_reference(name, channels, layers):
    from sparse_helpers import seeded_hip_model
    ref = json.load(open(os.path.join(GOLDEN, name + "_state_dict.json")))
    m = seeded_hip_model(channels, layers, 0)
    mine = [[k, list(v.shape)] for k, v in m.state_dict().items()]
    assert sorted(map(tuple, map(lambda kv: (kv[0], tuple(kv[1])), mine))) == \
        sorted(map(lambda kv: (kv[0], tuple(kv[1])), ref))


def test_ops_refuse_cpu_tensors():
    from fsctep_amd import ops  # noqa: F401
    w = torch.zeros(6 * 32 * 32, 64)
    b = torch.zeros(6 * 32 * 32)
    with pytest.raises(RuntimeError, match="GPU only"):
        torch.ops.fsctep.sparse_prepare_weights(w, b, 32)


def test_fake_kernels_trace_shapes():
    from torch._subclasses.fake_tensor import FakeTensorMode
    from fsctep_amd import ops  # noqa: F401
    with FakeTensorMode():
        x = torch.empty(10, 13, 64)
        h = torch.empty(30, 64)
        n = torch.empty(30, 3)
        bk = torch.empty(6 * 65 * 64 * 64 + 512)
        i = torch.empty(11, dtype=torch.int32)
        e = torch.empty(30, dtype=torch.int32)
        out, S, P = torch.ops.fsctep.sparse_conv(x, h, n, bk, bk, i, i, e, e, torch.empty(0, dtype=torch.int32))
        tail = 10 * 18 * 65 * 64 + 16 * 18 * 10 * 64 + 10
        assert out.shape == (10, 13, 64) and S.shape == ((tail + 63) // 64 * 64 + 4 * (30 * 67 + 10),)
        assert P.shape == (30 * 18 * 64,)


def test_gram_sizes_and_fake_kernels():
    from torch._subclasses.fake_tensor import FakeTensorMode
    from fsctep_amd import readout_ops
    # 24 blocks -> 300 pairs; 1,000 nodes: 38 chunks of 8 x 4 tiles of 256 nodes (16-pair chunks would leave
    # 76 <= 128 workgroups); 10,000 nodes: 19 chunks of 16 x 40 tiles; node scales
    wf, wb, ws = readout_ops.gram_sizes(1000, 384, 64)
    assert ws == 38 * 1000 * 64 + 1000
    _, _, ws = readout_ops.gram_sizes(10000, 384, 64)
    assert ws == 19 * 10000 * 64 + 10000
    assert wf == wb == 300 * 256 * 64 * 2 + 512              # fp32 pairs + two fp16 planes + scale/maxima tail
    with pytest.raises(RuntimeError, match="multiple of 16"):
        readout_ops.gram_sizes(10, 40, 64)
    with FakeTensorMode():
        W = torch.empty(64, 192, 192)
        Wf, Wb = torch.ops.fsctep.gram_prepare_weights(W)
        assert Wf.shape == Wb.shape == (78 * 256 * 64 * 2 + 512,)
        out = torch.ops.fsctep.gram_bilinear(torch.empty(7, 9, 192), Wf, Wb, 1.0)
        assert out.shape == (7, 64)


def test_readout_mlp_sizes_errors_and_fake_kernels():
    """Folded-weight buffer of the readout head: W1 diag(g0) and its transpose (2 H K), c1 and u1 (2 H), the
    hidden LayerNorms (2 H each), the H x H layers and their transposes with biases, v (H) and e0 (4)."""
    from torch._subclasses.fake_tensor import FakeTensorMode
    from fsctep_amd import ops  # noqa: F401

    class Dims(ctypes.Structure):
        _fields_ = [("K", ctypes.c_int32), ("H", ctypes.c_int32), ("NH", ctypes.c_int32), ("O", ctypes.c_int32),
                    ("eps0", ctypes.c_float), ("eps", ctypes.c_float * 4)]

    lib = _lib.load()
    n = ctypes.c_int64()
    d = Dims(1600, 128, 3, 17, 1e-5, (ctypes.c_float * 4)(1e-5, 1e-5, 1e-5, 0.0))
    assert lib.fsc_readout_mlp_weights_floats(ctypes.byref(d), ctypes.byref(n)) == 0
    H, K = 128, 1600
    assert n.value == 2 * H * K + 2 * H + 3 * 2 * H + 2 * (2 * H * H + H) + H + 4
    for bad, msg in ((Dims(1602, 128, 3, 17, 1e-5), b"multiple of 4"), (Dims(640, 96, 3, 17, 1e-5), b"hidden width"),
                     (Dims(640, 128, 5, 17, 1e-5), b"hidden layers")):
        bad.eps = (ctypes.c_float * 4)(1e-5, 1e-5, 1e-5, 1e-5)
        assert lib.fsc_readout_mlp_weights_floats(ctypes.byref(bad), ctypes.byref(n)) == 1
        assert msg in lib.fsc_last_error()
    with FakeTensorMode():
        K, H = 640, 64
        ps = [torch.empty(K), torch.empty(K), torch.empty(H, K), torch.empty(H), torch.empty(H), torch.empty(H),
              torch.empty(H, H), torch.empty(H), torch.empty(H), torch.empty(H), torch.empty(17, H), torch.empty(17),
              torch.empty(17)]
        w = torch.ops.fsctep.readout_mlp_prepare(ps, [K, H, 2, 17], [1e-5] * 3)
        assert w.shape == (2 * H * K + 2 * H + 2 * 2 * H + (2 * H * H + H) + H + 4,)
        e = torch.ops.fsctep.readout_mlp(torch.empty(9, K), w, [K, H, 2, 17], [1e-5] * 3)
        assert e.shape == (9, 1)
        dx = torch.ops.fsctep.readout_mlp_backward(torch.empty(9, 1), torch.empty(9, K), w, [K, H, 2, 17], [1e-5] * 3)
        assert dx.shape == (9, K)
