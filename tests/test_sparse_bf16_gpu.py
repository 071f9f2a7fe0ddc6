"""The bf16 channel-mix variant of the sparse conv (precision 1: one bf16 MFMA per product in the node
expansion, the edge message and the node-expansion gradient, fp32 accumulation), against the fp64 oracle
(op level) and against the fp32-accurate path (whole model).  bf16 keeps 8 significant bits, so the
bound here is a bf16 one: 2e-2 relative (max-norm) at the op level, where every output sums 64 to 4160
rounded products; the measured errors are printed.  The variant must also be deterministic and really
differ from the fp32 path."""

import numpy as np
import pytest
import torch

from sparse_helpers import oracle_conv2, rel_inf

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL_BF16 = 2e-2


@pytest.mark.parametrize("C", [64, 32, 128])
def test_bf16_conv2_op_against_oracle(C):
    from fsctep_amd import ops
    from fsctep_amd.graph import prepare_graph
    from test_sparse_gpu import _graph_with_edge_cases
    torch.manual_seed(3)
    N = 40
    src, dst = _graph_with_edge_cases(N, 400, 7)
    E = src.shape[0]
    x = torch.randn(N, 13, C, dtype=torch.float64)
    h = torch.randn(E, 64, dtype=torch.float64)
    v = torch.randn(E, 3, dtype=torch.float64)
    n = v / v.norm(dim=1, keepdim=True)
    L = torch.randn(6 * C * C, 64, dtype=torch.float64) / 8
    b = torch.randn(6 * C * C, dtype=torch.float64) * 0.1
    gr = prepare_graph(src.to(DEV), dst.to(DEV), torch.zeros(E, 3, device=DEV), N)
    order = torch.argsort(dst, stable=True)
    xo, ho, no = (t.clone().requires_grad_(True) for t in (x, h[order], n[order]))
    ref = oracle_conv2(xo, ho, no, L, b, src[order], dst[order], N, 1.0 / (E / N))
    G = torch.randn_like(ref)
    gx, gh, gn = torch.autograd.grad((ref * G).sum(), (xo, ho, no))
    bk1, bk6 = torch.ops.fsctep.sparse_prepare_weights(L.float().to(DEV), b.float().to(DEV), C)
    res = {}
    for prec in (0, 1):
        xd = x.float().to(DEV).requires_grad_(True)
        hd = h[order].float().to(DEV).requires_grad_(True)
        nd = n[order].float().to(DEV).requires_grad_(True)
        out = ops.sparse_conv_apply(xd, hd, nd, bk1, bk6, gr, precision=prec)
        grads = torch.autograd.grad(out, (xd, hd, nd), G.float().to(DEV))
        res[prec] = (out.detach(), *grads)
    errs = [rel_inf(a, r) for a, r in zip(res[1], (ref, gx, gh, gn))]
    print(f"C {C}: bf16 variant vs fp64 oracle: out {errs[0]:.2e}, dx {errs[1]:.2e}, dh {errs[2]:.2e}, dn {errs[3]:.2e}")
    assert max(errs) < TOL_BF16, errs
    assert rel_inf(res[1][0], res[0][0]) > 1e-5          # the bf16 products really ran
    assert rel_inf(res[0][0], ref) < 1e-5                 # and the default path is the fp32-accurate one


def test_bf16_model_against_fp32_path_and_deterministic():
    import bench
    from fsctep_amd.sparse import energy_and_forces
    s = bench._system("sparse", 3000, 22)
    m = bench.build_model("sparse", torch.device(DEV))
    pos = torch.tensor(s.pos, dtype=torch.float32, device=DEV)
    A = torch.tensor(s.species, device=DEV)
    batch = torch.zeros(3000, dtype=torch.long, device=DEV)
    cell = torch.tensor(s.cell, dtype=torch.float32, device=DEV)
    g = m.prepare(torch.tensor(s.edge_src, device=DEV), torch.tensor(s.edge_dst, device=DEV),
                  torch.tensor(s.edge_shifts, dtype=torch.float32, device=DEV), 3000, A, pos=pos)
    e32, f32 = energy_and_forces(m, pos, batch, cell, g)
    m.channel_mix_precision = "bf16"
    e16, f16 = energy_and_forces(m, pos, batch, cell, g)
    e16b, f16b = energy_and_forces(m, pos, batch, cell, g)
    assert torch.equal(e16, e16b) and torch.equal(f16, f16b)
    er, fr = rel_inf(e16, e32), rel_inf(f16, f32)
    print(f"3000 atoms: bf16 variant vs fp32 path: energies {er:.2e}, forces {fr:.2e}")
    assert er > 1e-7 and er < 5e-2 and fr < 5e-2
    m.channel_mix_precision = "fp16"
    with pytest.raises(ValueError):
        energy_and_forces(m, pos, batch, cell, g)
