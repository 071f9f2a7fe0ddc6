"""ICTD trunks at lmax 0 and 1 and the larger O3 irrep sets (the kernels take lmax 0 to 3 and up to 32
components per channel; the reference takes any lmax).

* the conv2..n op against the reference conv2 semantics of the oracle (fctp per path, scatter, / in-degree),
  forward and the three input gradients: full layouts at lmax 0 and 1, O3 layouts at lmax 1 and the O3
  presets "balanced" (17 components) and "full" (18) at lmax 2;
* whole trunks (energies and forces; O3 with an external field and the dipole head) against the fp64 oracle
  (oracle/ictd_ref.py, the restatement pinned by the reference golden vectors at lmax 2 and 3, whose code
  is the same for every lmax) on the 32-atom golden system, with seeded parameters shared by name.
1e-5 relative, max-norm, fp32 on the GPU."""

import numpy as np
import pytest
import torch

from conftest import load_golden
from fsctep_amd.synthetic import seeded_value
from oracle import ictd_ref as I
from test_ictd_gpu import _edges, _oracle_conv, rel_inf

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL = 1e-5


O3_BALANCED_L2 = [(0, 1), (1, 1), (1, -1), (2, 1), (2, -1)]
O3_FULL_L2 = [(0, 1), (0, -1), (1, 1), (1, -1), (2, 1), (2, -1)]


@pytest.mark.parametrize("lname,C", [("full_l0", 32), ("full_l1", 64), ("o3_l1", 32), ("o3_balanced_l2", 32),
                                     ("o3_full_l2", 64), ("o3_full_l2", 128)])
def test_ictd_conv_op_at_low_lmax(lname, C):
    from fsctep_amd import ictd_basis as B, ictd_ops
    from fsctep_amd.graph import prepare_graph
    lay = {"full_l0": B.layout_full(0), "full_l1": B.layout_full(1),
           "o3_l1": B.layout_o3(1, [(0, 1), (1, 1), (1, -1)]),
           "o3_balanced_l2": B.layout_o3(2, O3_BALANCED_L2), "o3_full_l2": B.layout_o3(2, O3_FULL_L2)}[lname]
    lid = ictd_ops.register_layout(lay)
    torch.manual_seed(11)
    N = 30
    src, dst = _edges(N, 5)
    order = torch.argsort(dst, stable=True)
    src, dst = src[order], dst[order]
    E = src.shape[0]
    n = torch.randn(E, 3, dtype=torch.float64)
    n = n / n.norm(dim=1, keepdim=True)
    Y = torch.cat([I.direction_harmonics(n, l) for l in range(lay.lmax + 1)], dim=-1)
    x = torch.randn(N, lay.M, C, dtype=torch.float64)
    P = lay.n_ref_paths()
    gates = torch.randn(E, P, dtype=torch.float64)
    W = torch.randn(P, C, C, 1, dtype=torch.float64) / np.sqrt(C)
    xo, Yo, go = (t.clone().requires_grad_(True) for t in (x, Y, gates))
    ref = _oracle_conv(xo, Yo, go, W, src, dst, N, lay)
    G = torch.randn_like(ref)
    gx, gY, gg = torch.autograd.grad((ref * G).sum(), (xo, Yo, go))

    gr = prepare_graph(src.to(DEV), dst.to(DEV), torch.zeros(E, 3, device=DEV), N)
    cg = torch.tensor(lay.cg_table(), dtype=torch.float32, device=DEV)
    Wd = W.float().to(DEV)
    Wt = torch.ops.fsctep.ictd_prepare_weights(Wd)
    xd, Yd, gd = (t.float().to(DEV).requires_grad_(True) for t in (x, Y, gates))
    out = ictd_ops.ictd_conv_apply(xd, Yd, gd, Wd, Wt, cg, gr, lid)
    dx, dY, dg = torch.autograd.grad(out, (xd, Yd, gd), G.float().to(DEV))
    torch.cuda.synchronize()
    assert rel_inf(out, ref) < TOL
    assert rel_inf(dx, gx) < TOL
    assert rel_inf(dY, gY) < TOL
    assert rel_inf(dg, gg) < TOL


KW = dict(max_embed_radius=5.0, main_max_radius=5.0, main_number_of_basis=8, hidden_dim_conv=32, hidden_dim_sh=32,
          hidden_dim=64, channel_in2=32, embedding_dim=16, max_atomvalue=10, output_size=8,
          embed_size=[128, 128, 128], num_interaction=2, function_type_main="gaussian",
          ictd_tp_path_policy="full", invariant_channels=32)


@pytest.mark.parametrize("lmax,o3", [(0, False), (1, False), (1, "0e,1o"), (2, "full"), (2, "balanced")])
def test_ictd_trunk_at_low_lmax_matches_oracle(lmax, o3):
    from fsctep_amd.ictd import (PureCartesianICTDO3TransformerLayer, PureCartesianICTDTransformerLayer,
                                 energy_forces)
    g = load_golden("ictd_open32_c32_l2")          # the geometry of the reference's 32-atom system
    seed = 17
    if o3:
        irreps = {"o3_active_irreps": o3} if "," in o3 else {"o3_irrep_preset": o3}
        m = PureCartesianICTDO3TransformerLayer(
            **KW, lmax=lmax, **irreps, external_tensor_rank=1, external_tensor_irrep="1o",
            physical_tensor_outputs={"dipole": {"irreps": ["1o"], "channels_out": 1, "reduce": "sum"}})
    else:
        m = PureCartesianICTDTransformerLayer(**KW, lmax=lmax)
    with torch.no_grad():
        for name, p in m.named_parameters():
            p.copy_(torch.from_numpy(seeded_value(name, tuple(p.shape), seed)).to(p.dtype))
    m = m.eval().requires_grad_(False).to(DEV)
    o3 = bool(o3)
    cfg = I.ICTDConfig(channels=32, lmax=lmax, num_interaction=2, function_type="gaussian", o3=o3,
                       active=tuple(m.keys) if o3 else (), external_field=o3, dipole=o3)
    prm = {k: torch.tensor(seeded_value(k, s, seed), dtype=torch.float64) for k, s in I.param_shapes(cfg)}
    assert set(prm) == {k for k, _ in m.named_parameters()}
    n = g["pos"].shape[0]
    field = torch.tensor([[0.05, -0.02, 0.03]], dtype=torch.float64) if o3 else None
    pos64 = torch.tensor(g["pos"], dtype=torch.float32).double().requires_grad_(True)
    args = (torch.tensor(g["species"]), torch.zeros(n, dtype=torch.long), torch.tensor(g["edge_src"]),
            torch.tensor(g["edge_dst"]), torch.tensor(g["edge_shifts"], dtype=torch.float32).double(),
            torch.tensor(g["cell"], dtype=torch.float32).double())
    res = I.forward(pos64, *args, prm, cfg, field)
    e_ref = res[0]
    (f_ref,) = torch.autograd.grad(e_ref.sum(), pos64)
    f_ref = -f_ref

    pos = torch.tensor(g["pos"], dtype=torch.float32, device=DEV)
    A = torch.tensor(g["species"], device=DEV)
    batch = torch.zeros(n, dtype=torch.long, device=DEV)
    cell = torch.tensor(g["cell"], dtype=torch.float32, device=DEV)
    gr = m.prepare(torch.tensor(g["edge_src"], device=DEV), torch.tensor(g["edge_dst"], device=DEV),
                   torch.tensor(g["edge_shifts"], dtype=torch.float32, device=DEV), n, A)
    e, f, dip = energy_forces(m, pos, batch, cell, gr,
                              external_tensor=None if field is None else field.float().to(DEV))
    torch.cuda.synchronize()
    assert rel_inf(e.reshape(-1), e_ref.detach().reshape(-1)) < TOL
    assert rel_inf(f, f_ref) < TOL
    if o3:
        assert rel_inf(dip.reshape(-1), res[1].detach().reshape(-1)) < TOL
