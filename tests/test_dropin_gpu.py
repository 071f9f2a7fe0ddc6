"""The reference-signature ``forward()`` of the trunks: the graph is rebuilt on every call (fresh edge
tensors of the same shape but different content, allocated where the previous ones were freed, must
give their own energies), parameter updates made in place through ``.data`` (as an EMA update does,
training/trainer.py:1424) are seen by the next call, and the ICTD trunks take ``precomputed_edge_vec``
(models/pure_cartesian_ictd_layers_full.py:901-902, _o3.py:928-929) with forces flowing back through it.
Checked against the fp64 oracle and the reference golden vectors at 1e-5 relative."""

import numpy as np
import pytest
import torch

from conftest import load_golden
from sparse_helpers import oracle_params, rel_inf, seeded_hip_model

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = 1e-5


def _edge_sets(g):
    """Two same-shape edge lists: the golden one and one with its last 12 edges replaced by copies of
    the first 12 (a multigraph; both are valid inputs with different energies)."""
    src, dst, sh = g["edge_src"].copy(), g["edge_dst"].copy(), g["edge_shifts"].copy()
    src2, dst2, sh2 = src.copy(), dst.copy(), sh.copy()
    src2[-12:], dst2[-12:], sh2[-12:] = src[:12], dst[:12], sh[:12]
    return [(src, dst, sh), (src2, dst2, sh2)]


def test_sparse_forward_rebuilds_graph_for_fresh_same_shape_edges():
    from oracle import sparse_ref as R
    g = load_golden("sparse_pbc100_c64_l3")
    C, L, seed = int(g["channels"]), int(g["layers"]), int(g["param_seed"])
    cfg, p = oracle_params(C, L, seed, torch.float64)
    n = g["pos"].shape[0]
    pos64, A = torch.tensor(g["pos"], dtype=torch.float64), torch.tensor(g["species"])
    batch, cell64 = torch.zeros(n, dtype=torch.long), torch.tensor(g["cell"], dtype=torch.float64)
    sets = _edge_sets(g)
    refs = [R.atom_energies(pos64, A, batch, torch.tensor(s), torch.tensor(d), torch.tensor(sh, dtype=torch.float64),
                            cell64, p, cfg).squeeze(-1) for s, d, sh in sets]
    assert rel_inf(refs[0], refs[1]) > 1e-3          # the two edge sets really differ
    m = seeded_hip_model(C, L, seed).to(DEV)
    pos, cell = pos64.float().to(DEV), cell64.float().to(DEV)
    for it in range(6):
        s, d, sh = sets[it % 2]
        es, ed = torch.tensor(s, device=DEV), torch.tensor(d, device=DEV)   # freshly allocated each call
        esh = torch.tensor(sh, dtype=torch.float32, device=DEV)
        e = m(pos, A.to(DEV), batch.to(DEV), es, ed, esh, cell).squeeze(-1)
        assert rel_inf(e, refs[it % 2]) < TOL, it
        del es, ed, esh


def test_sparse_in_place_parameter_update_is_seen():
    from oracle import sparse_ref as R
    g = load_golden("sparse_open32_c32_l2")
    C, L, seed = int(g["channels"]), int(g["layers"]), int(g["param_seed"])
    m = seeded_hip_model(C, L, seed).to(DEV)
    n = g["pos"].shape[0]
    args = [torch.tensor(g["pos"], dtype=torch.float32), torch.tensor(g["species"]), torch.zeros(n, dtype=torch.long),
            torch.tensor(g["edge_src"]), torch.tensor(g["edge_dst"]),
            torch.tensor(g["edge_shifts"], dtype=torch.float32), torch.tensor(g["cell"], dtype=torch.float32)]
    e0 = m(*[a.to(DEV) for a in args]).squeeze(-1)
    assert rel_inf(e0, g["energy_f64"]) < TOL
    keys = ("product_3.W.1", "e3_conv_layers.1.fc.4.weight", "e3_conv_layers.0.fc.4.weight")
    params = dict(m.named_parameters())
    for k in keys:
        params[k].data.mul_(1.5)                      # in place through .data: the version counter stays
    e1 = m(*[a.to(DEV) for a in args]).squeeze(-1)
    cfg, p = oracle_params(C, L, seed, torch.float64)
    for k in keys:
        p[k] = p[k] * 1.5
    a64 = [a.double() if a.is_floating_point() else a for a in args]
    ref = R.atom_energies(*a64, p, cfg).squeeze(-1)
    assert rel_inf(e1, ref) < TOL and rel_inf(e1, e0) > 1e-4


def _ictd_model(g):
    from test_ictd_gpu import _model
    return _model(g)


@pytest.mark.parametrize("name", ["ictd_pbc64_c128_l3", "ictdo3_pbc64_c64_l2_field"])
def test_ictd_precomputed_edge_vec(name):
    """pos enters only through edge_vec = pos[dst] - pos[src] + shifts @ cell, built by the caller as the
    LAMMPS engine does (mff_torch_engine.cpp:740-760); the trunk receives zeros for pos."""
    g = load_golden(name)
    m = _ictd_model(g)
    n = g["pos"].shape[0]
    pos = torch.tensor(g["pos"], dtype=torch.float32, device=DEV).requires_grad_(True)
    A = torch.tensor(g["species"], device=DEV)
    batch = torch.zeros(n, dtype=torch.long, device=DEV)
    src, dst = torch.tensor(g["edge_src"], device=DEV), torch.tensor(g["edge_dst"], device=DEV)
    sh = torch.tensor(g["edge_shifts"], dtype=torch.float32, device=DEV)
    cell = torch.tensor(g["cell"], dtype=torch.float32, device=DEV)
    edge_vec = pos.index_select(0, dst) - pos.index_select(0, src) + sh @ cell[0]
    kw = {}
    if "external_field" in g:
        kw = dict(external_tensor=torch.tensor(g["external_field"], dtype=torch.float32, device=DEV))
    e = m(torch.zeros_like(pos), A, batch, src, dst, sh, cell, precomputed_edge_vec=edge_vec, **kw)
    (gpos,) = torch.autograd.grad(e.sum(), pos)
    assert rel_inf(e.detach().squeeze(-1), g["energy_f64"]) < TOL
    assert rel_inf(-gpos, g["forces_f64"]) < TOL


@pytest.mark.parametrize("name", ["sparse_open32_c32_l2", "ictd_pbc64_c128_l3"])
def test_float64_inputs(name):
    """Inputs in float64 (the reference's default dtype, utils/config.py:16): the energies are those of the
    float32 inputs (the trunk computes in fp32) and the forces come back in float64."""
    g = load_golden(name)
    m = _ictd_model(g) if name.startswith("ictd") else seeded_hip_model(
        int(g["channels"]), int(g["layers"]), int(g["param_seed"])).to(DEV)
    n = g["pos"].shape[0]
    A = torch.tensor(g["species"], device=DEV)
    batch = torch.zeros(n, dtype=torch.long, device=DEV)
    src, dst = torch.tensor(g["edge_src"], device=DEV), torch.tensor(g["edge_dst"], device=DEV)
    out = {}
    for dt in (torch.float32, torch.float64):
        pos = torch.tensor(g["pos"], dtype=dt, device=DEV).requires_grad_(True)
        sh = torch.tensor(g["edge_shifts"], dtype=dt, device=DEV)
        cell = torch.tensor(g["cell"], dtype=dt, device=DEV).reshape(-1, 3, 3)
        e = m(pos, A, batch, src, dst, sh, cell)
        (f,) = torch.autograd.grad(e.sum(), pos)
        out[dt] = (e.detach(), -f)
    e32, f32 = out[torch.float32]
    e64, f64 = out[torch.float64]
    assert e64.dtype == torch.float32 and f64.dtype == torch.float64
    assert rel_inf(e64, e32) < 1e-6 and rel_inf(f64, f32) < 1e-5
