"""GPU parity of the ICTD HIP path (pure-cartesian-ictd and -o3) against the oracle and the
reference's golden vectors (fp32 on the GPU; 1e-5 relative, max-norm)."""

import numpy as np
import pytest
import torch

from conftest import load_golden
from fsctep_amd.synthetic import seeded_value
from oracle import ictd_ref as I

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL = 1e-5


def rel_inf(a, b):
    a = np.asarray(a.detach().cpu() if torch.is_tensor(a) else a, np.float64)
    b = np.asarray(b.detach().cpu() if torch.is_tensor(b) else b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def _edges(N, seed):
    g = torch.Generator().manual_seed(seed)
    src = torch.randint(0, N - 1, (300,), generator=g)
    dst = torch.randint(0, N - 1, (300,), generator=g)
    src = torch.cat([src, torch.zeros(70, dtype=torch.long), torch.randint(2, N - 1, (70,), generator=g)])
    dst = torch.cat([dst, torch.randint(2, N - 1, (70,), generator=g), torch.ones(70, dtype=torch.long)])
    return src, dst       # node N-1 isolated, node 0 a 70-out-edge hub, node 1 a 70-in-edge receiver


def _oracle_conv(x, Y, gates, W, src, dst, N, lay):
    """Reference conv2 semantics on component-major tensors: fctp per path, scatter, / in-degree."""
    keys = list(lay.keys)
    offs = lay.comp_off
    x1 = {k: x[src][:, offs[k]:offs[k] + 2 * k[0] + 1, :].transpose(1, 2) for k in keys}
    x2 = {}
    for l in range(lay.lmax + 1):
        k = (l, 1 if l % 2 == 0 else -1)
        if k in keys:
            x2[k] = Y[:, l * l:(l + 1) ** 2].unsqueeze(1)
    paths = I.tp_paths(keys, keys, keys, lay.lmax)
    out = I.fctp(x1, x2, W, gates, paths, keys)
    msg = torch.cat([out[k].transpose(1, 2) for k in keys], dim=1)
    cnt = torch.zeros(N, dtype=x.dtype).index_add(0, dst, torch.ones_like(dst, dtype=x.dtype)).clamp(min=1)
    return torch.zeros(N, *msg.shape[1:], dtype=x.dtype).index_add(0, dst, msg) / cnt[:, None, None]


@pytest.mark.parametrize("lname,C", [("full_l2", 32), ("full_l3", 128), ("o3", 64)])
def test_ictd_conv_op_matches_oracle(lname, C):
    from fsctep_amd import ictd_basis as B, ictd_ops
    from fsctep_amd.graph import prepare_graph
    lay = {"full_l2": B.layout_full(2), "full_l3": B.layout_full(3),
           "o3": B.layout_o3(2, [(0, 1), (1, 1), (1, -1), (2, 1)])}[lname]
    lid = ictd_ops.register_layout(lay)
    torch.manual_seed(3)
    N = 30
    src, dst = _edges(N, 7)
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
    assert float(out.detach()[N - 1].abs().max()) == 0.0 and float(dx[N - 1].abs().max()) == 0.0


def _rowwise_rel(a, b):
    """max over rows (first axis) of |a_r - b_r|_inf / |b_r|_inf; rows where b is zero must be zero."""
    a = a.detach().double().cpu().reshape(a.shape[0], -1)
    b = b.detach().double().cpu().reshape(b.shape[0], -1)
    den, err = b.abs().amax(1), (a - b).abs().amax(1)
    nz = den > 0
    if (~nz).any():
        assert float(err[~nz].max()) == 0.0
    return float((err[nz] / den[nz]).max())


def test_ictd_conv_op_wide_dynamic_range():
    """The split-fp16 channel mix scales the projections of each receiver and the output gradient of each
    node by their own powers of two: with node features and output gradients spread over 8 decades and an
    all-zero node, every receiver's output and every node's input gradient keep their relative accuracy."""
    from fsctep_amd import ictd_basis as B, ictd_ops
    from fsctep_amd.graph import prepare_graph
    lay, C = B.layout_full(3), 128
    lid = ictd_ops.register_layout(lay)
    g = torch.Generator().manual_seed(23)
    N = 30
    src, dst = _edges(N, 11)
    order = torch.argsort(dst, stable=True)
    src, dst = src[order], dst[order]
    E = src.shape[0]
    n = torch.randn(E, 3, generator=g, dtype=torch.float64)
    n = n / n.norm(dim=1, keepdim=True)
    Y = torch.cat([I.direction_harmonics(n, l) for l in range(lay.lmax + 1)], dim=-1).float().double()
    x = (torch.randn(N, lay.M, C, generator=g, dtype=torch.float64) *
         10.0 ** (8 * torch.rand(N, 1, 1, generator=g, dtype=torch.float64) - 4)).float().double()
    x[4] = 0.0
    P = lay.n_ref_paths()
    gates = torch.randn(E, P, generator=g, dtype=torch.float64).float().double()
    W = (torch.randn(P, C, C, 1, generator=g, dtype=torch.float64) / np.sqrt(C)).float().double()
    xo, Yo, go = (t.clone().requires_grad_(True) for t in (x, Y, gates))
    ref = _oracle_conv(xo, Yo, go, W, src, dst, N, lay)
    G = (torch.randn(ref.shape, generator=g, dtype=torch.float64) *
         10.0 ** (8 * torch.rand(N, 1, 1, generator=g, dtype=torch.float64) - 4)).float().double()
    gx, gY, gg = torch.autograd.grad((ref * G).sum(), (xo, Yo, go))

    gr = prepare_graph(src.to(DEV), dst.to(DEV), torch.zeros(E, 3, device=DEV), N)
    cg = torch.tensor(lay.cg_table(), dtype=torch.float32, device=DEV)
    Wd = W.float().to(DEV)
    Wt = torch.ops.fsctep.ictd_prepare_weights(Wd)
    xd, Yd, gd = (t.float().to(DEV).requires_grad_(True) for t in (x, Y, gates))
    out = ictd_ops.ictd_conv_apply(xd, Yd, gd, Wd, Wt, cg, gr, lid)
    dx, dY, dg = torch.autograd.grad(out, (xd, Yd, gd), G.float().to(DEV))
    torch.cuda.synchronize()
    assert _rowwise_rel(out, ref) < TOL      # per receiver
    assert _rowwise_rel(dx, gx) < TOL        # per source
    assert _rowwise_rel(dY, gY) < TOL        # per edge
    assert _rowwise_rel(dg, gg) < TOL


CASES = ["ictd_open32_c32_l2", "ictd_pbc64_c128_l3", "ictdo3_pbc64_c64_l2_field"]


def _model(g):
    from fsctep_amd.ictd import PureCartesianICTDO3TransformerLayer, PureCartesianICTDTransformerLayer
    o3 = bool(g["o3"])
    kw = dict(max_embed_radius=5.0, main_max_radius=5.0, main_number_of_basis=8,
              hidden_dim_conv=int(g["channels"]), hidden_dim_sh=int(g["channels"]), hidden_dim=64,
              channel_in2=32, embedding_dim=16, max_atomvalue=10, output_size=8, embed_size=[128, 128, 128],
              num_interaction=int(g["layers"]), function_type_main=str(g["function_type"]), lmax=int(g["lmax"]),
              ictd_tp_path_policy="full", invariant_channels=32)
    if o3:
        m = PureCartesianICTDO3TransformerLayer(
            **kw, o3_active_irreps="0e,1e,1o,2e", external_tensor_rank=1, external_tensor_irrep="1o",
            physical_tensor_outputs={"dipole": {"irreps": ["1o"], "channels_out": 1, "reduce": "sum"}})
    else:
        m = PureCartesianICTDTransformerLayer(**kw)
    with torch.no_grad():
        for name, p in m.named_parameters():
            p.copy_(torch.from_numpy(seeded_value(name, tuple(p.shape), int(g["param_seed"]))).to(p.dtype))
    return m.eval().requires_grad_(False).to(DEV)


@pytest.mark.parametrize("name", CASES)
def test_ictd_model_matches_reference_golden(name):
    from fsctep_amd.ictd import energy_forces
    g = load_golden(name)
    m = _model(g)
    n = g["pos"].shape[0]
    pos = torch.tensor(g["pos"], dtype=torch.float32, device=DEV)
    A = torch.tensor(g["species"], device=DEV)
    batch = torch.zeros(n, dtype=torch.long, device=DEV)
    cell = torch.tensor(g["cell"], dtype=torch.float32, device=DEV)
    gr = m.prepare(torch.tensor(g["edge_src"], device=DEV), torch.tensor(g["edge_dst"], device=DEV),
                   torch.tensor(g["edge_shifts"], dtype=torch.float32, device=DEV), n, A)
    field = torch.tensor(g["external_field"], dtype=torch.float32, device=DEV) if "external_field" in g else None
    e, f, dip = energy_forces(m, pos, batch, cell, gr, external_tensor=field)
    assert rel_inf(e, g["energy_f64"]) < TOL
    assert rel_inf(f, g["forces_f64"]) < TOL
    if "dipole_f64" in g:
        assert rel_inf(dip, g["dipole_f64"]) < TOL
