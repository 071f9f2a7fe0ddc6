"""The per-edge (bucketed) ICTD operations under the reference extension's names
(molecular_force_field._C_ictd_tp, csrc/ictd_tp.cpp:498-522), run through fsctep_amd.ictd_tp_ext on the
HIP kernels, against the fp64 oracle (oracle/ictd_bucket_ref.py, pinned in tests/test_oracle_bucket.py),
in float32 and float64 (the reference's kernels dispatch both, csrc/ictd_tp_cuda.cu:1230-1236).
Tolerance: max-norm relative error per output, 1e-5 in float32 (fp32 products and sums) and 1e-10 in
float64 (the reference's fp64 rtol, test/test_ictd_tp_backend.py:383-714).  Also: summed over the bucket
table the ops reproduce the trunk's fully connected TP (oracle fctp); argument errors; an empty batch;
bitwise-deterministic batch sums; the module passes the reference's availability probe."""

import sys

import pytest
import torch

from oracle import ictd_bucket_ref as BR
from oracle import ictd_ref as R

pytestmark = pytest.mark.gpu
TOLS = {torch.float32: 1e-5, torch.float64: 1e-10}
DTYPES = pytest.mark.parametrize("dt", [torch.float32, torch.float64], ids=["fp32", "fp64"])
TOL = TOLS[torch.float32]
DEV = "cuda"


def ext():
    from fsctep_amd import ictd_tp_ext
    return ictd_tp_ext


def rel(x, ref):
    ref = ref.double()
    return float((x.double().cpu() - ref).abs().max() / ref.abs().max().clamp_min(1e-30))


def rnd(*shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g, dtype=torch.float64)


def gpu(t, dt=torch.float32):
    return t.to(DEV, dt)


# (B, I, m1, m2, P, K)
PROJ = [(37, 32, 3, 3, 2, 3), (200, 128, 7, 7, 1, 7), (64, 64, 5, 3, 3, 5), (1, 16, 1, 5, 2, 5),
        (300, 128, 7, 5, 2, 3), (70, 36, 9, 1, 4, 1)]
# (B, P, K, I, O)
MIX = [(37, 2, 3, 32, 32), (200, 1, 7, 128, 128), (50, 3, 5, 64, 144), (1, 4, 1, 16, 8), (130, 2, 1, 128, 64),
       (33, 2, 9, 20, 12)]


@DTYPES
@pytest.mark.parametrize("case", PROJ)
def test_projection_ops(case, dt):
    B, I, m1, m2, P, K = case
    E = ext()
    TOL = TOLS[dt]
    gpu = lambda t: t.to(DEV, dt)
    s = sum(case)
    a, b, u = rnd(B, I, m1, seed=s), rnd(B, 1, m2, seed=s + 1), rnd(m1 * m2, P * K, seed=s + 2)
    gy = rnd(B, P, K, I, seed=s + 3)
    y = E.project_bucket_forward(gpu(a), gpu(b), gpu(u), P)
    assert y.shape == (B, P, K, I) and y.dtype == dt
    assert rel(y, BR.project_forward(a, b, u, P)) < TOL
    ta, tb, tu = BR.project_transpose(gy, a, b, u)
    ga = E.project_bucket_transpose_a(gpu(gy), gpu(b), gpu(u))
    gb = E.project_bucket_transpose_b(gpu(gy), gpu(a), gpu(u))
    gu = E.project_bucket_transpose_u(gpu(gy), gpu(a), gpu(b))
    assert ga.shape == ta.shape and gb.shape == tb.shape and gu.shape == tu.shape
    errs = {"a": rel(ga, ta), "b": rel(gb, tb), "u": rel(gu, tu)}
    assert max(errs.values()) < TOL, errs


@DTYPES
@pytest.mark.parametrize("case", MIX)
def test_mix_ops(case, dt):
    B, P, K, I, O = case
    E = ext()
    TOL = TOLS[dt]
    gpu = lambda t: t.to(DEV, dt)
    s = sum(case) + 1000
    y, w, g = rnd(B, P, K, I, seed=s), rnd(P, O, I, seed=s + 1), rnd(B, P, seed=s + 2)
    go = rnd(B, O, K, seed=s + 3)
    out = E.mix_bucket_forward(gpu(y), gpu(w), gpu(g))
    assert out.shape == (B, O, K) and out.dtype == dt
    assert rel(out, BR.mix_forward(y, w, g)) < TOL
    ty, tw, tg = BR.mix_transpose(go, y, w, g)
    gy = E.mix_bucket_transpose_y(gpu(go), gpu(w), gpu(g))
    gw = E.mix_bucket_transpose_w(gpu(go), gpu(y), gpu(g))
    gg = E.mix_bucket_transpose_g(gpu(go), gpu(y), gpu(w))
    assert gy.shape == ty.shape and gw.shape == tw.shape and gg.shape == tg.shape
    errs = {"y": rel(gy, ty), "w": rel(gw, tw), "g": rel(gg, tg)}
    assert max(errs.values()) < TOL, errs


@DTYPES
def test_bucketed_tp_forward_and_double_backward(dt):
    E = ext()
    TOL = TOLS[dt]
    gpu = lambda t: t.to(DEV, dt)
    B, I, m1, m2, P, K, O = 90, 64, 5, 3, 2, 3, 64
    a, b, u = rnd(B, I, m1, seed=1), rnd(B, 1, m2, seed=2), rnd(m1 * m2, P * K, seed=3)
    gga, ggb, ggu = rnd(B, I, m1, seed=4), rnd(B, 1, m2, seed=5), rnd(m1 * m2, P * K, seed=6)
    w, g = rnd(P, O, I, seed=7), rnd(B, P, seed=8)
    out = E.bucketed_tp_forward(gpu(a), gpu(b), gpu(u), gpu(w), gpu(g))
    assert rel(out, BR.mix_forward(BR.project_forward(a, b, u, P), w, g)) < TOL
    h = rnd(B, P, K, I, seed=9)
    ref = BR.project_dbl_bwd(h, a, gga, b, ggb, u, ggu, P)
    got = (E.project_dbl_bwd_grad_h(gpu(a), gpu(gga), gpu(b), gpu(ggb), gpu(u), gpu(ggu), P),
           E.project_dbl_bwd_grad_a(gpu(h), gpu(b), gpu(ggb), gpu(u), gpu(ggu)),
           E.project_dbl_bwd_grad_b(gpu(h), gpu(a), gpu(gga), gpu(u), gpu(ggu)),
           E.project_dbl_bwd_grad_u(gpu(h), gpu(a), gpu(gga), gpu(b), gpu(ggb)))
    errs = [rel(x, r) for x, r in zip(got, ref)]
    assert all(x.shape == r.shape for x, r in zip(got, ref))
    assert max(errs) < TOL, errs
    y, ggy, ggw, ggg = rnd(B, P, K, I, seed=10), rnd(B, P, K, I, seed=11), rnd(P, O, I, seed=12), rnd(B, P, seed=13)
    G = rnd(B, O, K, seed=14)
    ref = BR.mix_dbl_bwd(G, y, ggy, w, ggw, g, ggg)
    got = (E.mix_dbl_bwd_grad_g_out(gpu(y), gpu(ggy), gpu(w), gpu(ggw), gpu(g), gpu(ggg)),
           E.mix_dbl_bwd_grad_y(gpu(G), gpu(w), gpu(ggw), gpu(g), gpu(ggg)),
           E.mix_dbl_bwd_grad_w(gpu(G), gpu(y), gpu(ggy), gpu(g), gpu(ggg)),
           E.mix_dbl_bwd_grad_g(gpu(G), gpu(y), gpu(ggy), gpu(w), gpu(ggw)))
    errs = [rel(x, r) for x, r in zip(got, ref)]
    assert all(x.shape == r.shape for x, r in zip(got, ref))
    assert max(errs) < TOL, errs


@DTYPES
def test_buckets_reproduce_the_fully_connected_tp(dt):
    """The reference trunk's cuda_ext dispatch (models/ictd_irreps.py:1035-1070) over the bucket table, with
    these ops, equals the fully connected TP at C 64, lmax 3."""
    E = ext()
    TOL = TOLS[dt]
    gpu = lambda t: t.to(DEV, dt)
    lmax, C, n = 3, 64, 300
    keys = [(l, (-1) ** l) for l in range(lmax + 1)]
    paths = R.tp_paths(keys, keys, keys, lmax)
    x1 = {k: rnd(n, C, 2 * k[0] + 1, seed=20 + k[0]) for k in keys}
    x2 = {k: rnd(n, 1, 2 * k[0] + 1, seed=30 + k[0]) for k in keys}
    W = rnd(len(paths), C, C, 1, seed=40) / C
    gates = rnd(n, len(paths), seed=41)
    ref = R.fctp(x1, x2, W, gates, paths, keys)
    out = {k: torch.zeros(n, C, 2 * k[0] + 1, device=DEV, dtype=dt) for k in keys}
    for k1, k2, k3, kdim, pidx, U in BR.buckets(paths):
        out[k3] += E.bucketed_tp_forward(gpu(x1[k1]), gpu(x2[k2]), gpu(U), gpu(W[pidx].reshape(len(pidx), C, C)),
                                         gpu(gates[:, pidx]))
    errs = {k: rel(out[k], ref[k]) for k in keys}
    assert max(errs.values()) < TOL, errs


def test_argument_errors():
    E = ext()
    a, b, u = torch.randn(4, 8, 3, device=DEV), torch.randn(4, 1, 3, device=DEV), torch.randn(9, 6, device=DEV)
    with pytest.raises(RuntimeError, match="float32 or float64"):
        E.project_bucket_forward(a.half(), b.half(), u.half(), 2)
    with pytest.raises(RuntimeError, match="same dtype"):
        E.project_bucket_forward(a.double(), b, u, 2)
    with pytest.raises(RuntimeError, match="mul_in2"):
        E.project_bucket_forward(a, torch.randn(4, 2, 3, device=DEV), torch.randn(9, 6, device=DEV), 2)
    with pytest.raises(RuntimeError, match="a and b batch dimensions must match"):
        E.project_bucket_forward(a, b[:3], u, 2)
    with pytest.raises(RuntimeError, match="divisible by num_paths"):
        E.project_bucket_forward(a, b, u, 4)
    with pytest.raises(RuntimeError, match="GPU"):
        E.project_bucket_forward(a.cpu(), b.cpu(), u.cpu(), 2)
    y, w, g = torch.randn(4, 2, 3, 8, device=DEV), torch.randn(2, 5, 8, device=DEV), torch.randn(4, 2, device=DEV)
    with pytest.raises(RuntimeError, match="w IJ dim must match y"):
        E.mix_bucket_forward(y, w[:, :, :4], g)
    with pytest.raises(RuntimeError, match="multiples of 4"):
        E.mix_bucket_forward(torch.randn(4, 2, 3, 6, device=DEV), torch.randn(2, 5, 6, device=DEV), g)


def test_empty_batch():
    E = ext()
    a, b, u = torch.zeros(0, 8, 3, device=DEV), torch.zeros(0, 1, 3, device=DEV), torch.randn(9, 6, device=DEV)
    gy = torch.zeros(0, 2, 3, 8, device=DEV)
    assert E.project_bucket_forward(a, b, u, 2).shape == (0, 2, 3, 8)
    gu = E.project_bucket_transpose_u(gy, a, b)
    assert gu.shape == (9, 6) and not gu.abs().any()
    y, g, go = torch.zeros(0, 2, 3, 8, device=DEV), torch.zeros(0, 2, device=DEV), torch.zeros(0, 4, 3, device=DEV)
    gw = E.mix_bucket_transpose_w(go, y, g)
    assert gw.shape == (2, 4, 8) and not gw.abs().any()
    assert E.mix_bucket_forward(y, torch.randn(2, 4, 8, device=DEV), g).shape == (0, 4, 3)


@DTYPES
def test_batch_sums_are_deterministic(dt):
    E = ext()
    TOL = TOLS[dt]
    gpu = lambda t: t.to(DEV, dt)
    B, I, m1, m2, P, K, O = 5000, 64, 5, 5, 2, 5, 64
    a, b, u = gpu(rnd(B, I, m1, seed=50)), gpu(rnd(B, 1, m2, seed=51)), gpu(rnd(m1 * m2, P * K, seed=52))
    gy, g, go = gpu(rnd(B, P, K, I, seed=53)), gpu(rnd(B, P, seed=54)), gpu(rnd(B, O, K, seed=55))
    u1, u2 = E.project_bucket_transpose_u(gy, a, b), E.project_bucket_transpose_u(gy, a, b)
    w1, w2 = E.mix_bucket_transpose_w(go, gy, g), E.mix_bucket_transpose_w(go, gy, g)
    assert torch.equal(u1, u2) and torch.equal(w1, w2)
    ref = BR.mix_transpose(go.double().cpu(), gy.double().cpu(), torch.zeros(P, O, I, dtype=torch.float64),
                           g.double().cpu())[1]
    assert rel(w1, ref) < TOL


def test_module_passes_the_reference_availability_probe():
    """models/ictd_irreps_cuda.py:28-47: all nine names present and has_cuda() true."""
    E = ext()
    required = ("project_bucket_forward", "project_bucket_transpose_a", "project_bucket_transpose_b",
                "project_bucket_transpose_u", "mix_bucket_forward", "mix_bucket_transpose_y",
                "mix_bucket_transpose_w", "mix_bucket_transpose_g", "bucketed_tp_forward")
    name = "molecular_force_field._C_ictd_tp"
    try:
        E.install(name)
        mod = sys.modules[name]
        assert all(hasattr(mod, n) for n in required) and mod.has_cuda()
        assert all(callable(getattr(mod, n)) for n in E.FUNCTIONS)
    finally:
        sys.modules.pop(name, None)
