"""Inputs of the drop-in trunks beyond the single-graph benchmark systems, against the fp64 oracle at
1e-5 relative (max-norm):

* a batch of two periodic graphs with different cells, a field per graph and a dipole per graph (the
  trunks index ``cell[batch[src]]`` and ``field[batch[src]]``, models/pure_cartesian_ictd_layers_o3.py:924-936,
  497-519, and sum the dipole per graph, :978-1007);
* an ICTD system with no edges at all;
* a species table larger than 16 rows (max_atomvalue 30, elements up to Cu), served by mapping the species
  present to the kernels' 16 rows, and more than 16 species present, which must poison the result;
* an out-of-range edge id, which must make both energies and forces NaN (the ids are clamped on the
  device, so without the poison the forces would be finite and wrong);
* the O3 active-irrep preset 'auto' (models/pure_cartesian_ictd_layers_o3.py:149-180).
"""

import numpy as np
import pytest
import torch

from fsctep_amd.synthetic import make_system, seeded_value
from oracle import ictd_ref as I
from oracle import sparse_ref as R
from sparse_helpers import oracle_params, rel_inf, seeded_hip_model

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL = 1e-5
DIPOLE = {"dipole": {"irreps": ["1o"], "channels_out": 1, "reduce": "sum"}}


def _ictd_model(C, layers, lmax, o3=False, field=False, dipole=False, active=None, preset="auto",
                max_atomvalue=10, seed=5):
    from fsctep_amd.ictd import PureCartesianICTDO3TransformerLayer, PureCartesianICTDTransformerLayer
    kw = dict(max_embed_radius=5.0, main_max_radius=5.0, main_number_of_basis=8, hidden_dim_conv=C,
              hidden_dim_sh=C, hidden_dim=64, channel_in2=32, embedding_dim=16, max_atomvalue=max_atomvalue,
              output_size=8, embed_size=[128, 128, 128], num_interaction=layers, function_type_main="bessel",
              lmax=lmax, ictd_tp_path_policy="full", invariant_channels=32)
    if o3:
        extra = dict(o3_active_irreps=active, o3_irrep_preset=preset)
        if field:
            extra.update(external_tensor_rank=1, external_tensor_irrep="1o")
        if dipole:
            extra["physical_tensor_outputs"] = DIPOLE
        m = PureCartesianICTDO3TransformerLayer(**kw, **extra)
    else:
        m = PureCartesianICTDTransformerLayer(**kw)
    with torch.no_grad():
        for name, p in m.named_parameters():
            p.copy_(torch.from_numpy(seeded_value(name, tuple(p.shape), seed)).to(p.dtype))
    return m.eval().requires_grad_(False).to(DEV)


def _ictd_oracle(m, C, layers, lmax, o3=False, field=False, dipole=False, max_atomvalue=10, seed=5):
    cfg = I.ICTDConfig(channels=C, lmax=lmax, num_interaction=layers, function_type="bessel", o3=o3,
                       active=tuple(m.keys) if o3 else (), external_field=field, dipole=dipole,
                       max_atomvalue=max_atomvalue)
    p = {k: torch.tensor(seeded_value(k, s, seed), dtype=torch.float64) for k, s in I.param_shapes(cfg)}
    return cfg, p


def _two_graphs():
    """Two periodic graphs (40 atoms in an 11 A cube, 30 atoms in a 13 A cube), one batch."""
    a = make_system(40, box=11.0, periodic=True, seed=101)
    b = make_system(30, box=13.0, periodic=True, seed=202)
    na = a.num_atoms
    pos = np.concatenate([a.pos, b.pos])
    species = np.concatenate([a.species, b.species])
    batch = np.concatenate([np.zeros(na, np.int64), np.ones(b.num_atoms, np.int64)])
    src = np.concatenate([a.edge_src, b.edge_src + na])
    dst = np.concatenate([a.edge_dst, b.edge_dst + na])
    sh = np.concatenate([a.edge_shifts, b.edge_shifts])
    cell = np.concatenate([a.cell, b.cell])
    return pos, species, batch, src, dst, sh, cell


def _to_dev(pos, species, batch, src, dst, sh, cell):
    f = lambda x: torch.tensor(x, dtype=torch.float32, device=DEV)
    i = lambda x: torch.tensor(x, dtype=torch.long, device=DEV)
    return f(pos), i(species), i(batch), i(src), i(dst), f(sh), f(cell)


def _to_cpu64(pos, species, batch, src, dst, sh, cell):
    f = lambda x: torch.tensor(np.asarray(x, np.float32), dtype=torch.float64)
    i = lambda x: torch.tensor(x, dtype=torch.long)
    return f(pos), i(species), i(batch), i(src), i(dst), f(sh), f(cell)


def test_o3_two_graph_batch_with_fields_and_dipoles():
    from fsctep_amd.ictd import energy_forces
    sysd = _two_graphs()
    C, L = 32, 2
    m = _ictd_model(C, L, 2, o3=True, field=True, dipole=True, active="0e,1e,1o,2e")
    cfg, p = _ictd_oracle(m, C, L, 2, o3=True, field=True, dipole=True)
    fields = np.array([[0.05, -0.12, 0.08], [-0.09, 0.03, 0.15]], np.float32)
    pos, A, batch, src, dst, sh, cell = _to_dev(*sysd)
    g = m.prepare(src, dst, sh, pos.shape[0], A)
    e, f, dip = energy_forces(m, pos, batch, cell, g, external_tensor=torch.tensor(fields, device=DEV))
    e_ref, f_ref, d_ref = I.energy_forces(*_to_cpu64(*sysd), p, cfg, torch.tensor(fields, dtype=torch.float64))
    assert dip.shape == (2, 1, 3)
    assert rel_inf(e, e_ref) < TOL
    assert rel_inf(f, f_ref) < TOL
    assert rel_inf(dip, d_ref) < TOL
    # each graph sees its own field: with the fields swapped the dipoles follow the oracle's, and differ
    swapped = fields[::-1].copy()
    _, _, dip_sw = energy_forces(m, pos, batch, cell, g, external_tensor=torch.tensor(swapped, device=DEV))
    _, _, d_sw = I.energy_forces(*_to_cpu64(*sysd), p, cfg, torch.tensor(swapped, dtype=torch.float64))
    assert rel_inf(dip_sw, d_sw) < TOL
    assert rel_inf(d_sw, d_ref) > 1e-5


def test_sparse_two_graph_batch():
    from fsctep_amd.sparse import energy_and_forces
    sysd = _two_graphs()
    C, L, seed = 32, 3, 9
    m = seeded_hip_model(C, L, seed).to(DEV)
    cfg, p = oracle_params(C, L, seed, torch.float64)
    pos, A, batch, src, dst, sh, cell = _to_dev(*sysd)
    e, f = energy_and_forces(m, pos, batch, cell, m.prepare(src, dst, sh, pos.shape[0], A))
    e_ref, f_ref = R.energy_forces(*_to_cpu64(*sysd), p, cfg)
    assert rel_inf(e, e_ref) < TOL
    assert rel_inf(f, f_ref) < TOL


@pytest.mark.parametrize("o3", [False, True])
def test_ictd_system_without_edges(o3):
    from fsctep_amd.ictd import energy_forces
    s = make_system(12, box=10.0, periodic=False, seed=7)
    C, L = 32, 2
    kw = dict(o3=True, field=True, dipole=True, active="0e,1e,1o,2e") if o3 else {}
    m = _ictd_model(C, L, 2, **kw)
    okw = dict(o3=True, field=True, dipole=True) if o3 else {}
    cfg, p = _ictd_oracle(m, C, L, 2, **okw)
    empty_i = np.zeros(0, np.int64)
    sysd = (s.pos, s.species, np.zeros(12, np.int64), empty_i, empty_i, np.zeros((0, 3)), s.cell)
    pos, A, batch, src, dst, sh, cell = _to_dev(*sysd)
    fld = np.array([[0.1, 0.0, -0.2]], np.float32)
    ext = torch.tensor(fld, device=DEV) if o3 else None
    e, f, dip = energy_forces(m, pos, batch, cell, m.prepare(src, dst, sh, 12, A), external_tensor=ext)
    e_ref, f_ref, d_ref = I.energy_forces(*_to_cpu64(*sysd), p, cfg,
                                          torch.tensor(fld, dtype=torch.float64) if o3 else None)
    assert rel_inf(e, e_ref) < TOL
    assert float(f.abs().max()) == 0.0 and float(f_ref.abs().max()) == 0.0
    if o3:
        assert float(dip.abs().max()) == 0.0 and float(d_ref.abs().max()) == 0.0


def _heavy_system(species_set, n=40, seed=31):
    s = make_system(n, box=10.0, periodic=False, seed=seed)
    rng = np.random.Generator(np.random.PCG64(seed))
    species = np.asarray(species_set, np.int64)[rng.integers(0, len(species_set), size=n)]
    species[:len(species_set)] = species_set          # every listed species present
    return (s.pos, species, np.zeros(n, np.int64), s.edge_src, s.edge_dst, s.edge_shifts, s.cell)


ELEMENTS = [1, 6, 8, 17, 29]          # H, C, O, Cl, Cu: atomic numbers beyond the 16-row table


def test_sparse_species_table_beyond_16_rows():
    from fsctep_amd.sparse import PureCartesianSparseTransformerLayer, energy_and_forces
    C, L, seed = 32, 2, 13
    m = PureCartesianSparseTransformerLayer(
        max_embed_radius=5.0, main_max_radius=5.0, main_number_of_basis=8, hidden_dim_conv=C, max_atomvalue=30,
        num_interaction=L, function_type_main="bessel")
    with torch.no_grad():
        for name, prm in m.named_parameters():
            prm.copy_(torch.from_numpy(seeded_value(name, tuple(prm.shape), seed)).to(prm.dtype))
    m = m.eval().requires_grad_(False).to(DEV)
    cfg = R.SparseConfig(channels=C, num_interaction=L, function_type="bessel", max_atomvalue=30)
    p = {k: torch.tensor(seeded_value(k, s, seed), dtype=torch.float64) for k, s in R.param_shapes(cfg)}
    sysd = _heavy_system(ELEMENTS)
    pos, A, batch, src, dst, sh, cell = _to_dev(*sysd)
    e, f = energy_and_forces(m, pos, batch, cell, m.prepare(src, dst, sh, pos.shape[0], A))
    e_ref, f_ref = R.energy_forces(*_to_cpu64(*sysd), p, cfg)
    assert rel_inf(e, e_ref) < TOL
    assert rel_inf(f, f_ref) < TOL
    # 17 species present: more than the kernels' 16 rows -> energies and forces are NaN
    many = _heavy_system(list(range(1, 18)), n=40, seed=32)
    pos, A, batch, src, dst, sh, cell = _to_dev(*many)
    e, f = energy_and_forces(m, pos, batch, cell, m.prepare(src, dst, sh, pos.shape[0], A))
    assert torch.isnan(e).all() and torch.isnan(f).all()


def test_ictd_species_table_beyond_16_rows():
    from fsctep_amd.ictd import energy_forces
    C, L = 32, 2
    m = _ictd_model(C, L, 2, max_atomvalue=30)
    cfg, p = _ictd_oracle(m, C, L, 2, max_atomvalue=30)
    sysd = _heavy_system(ELEMENTS, seed=35)
    pos, A, batch, src, dst, sh, cell = _to_dev(*sysd)
    e, f, _ = energy_forces(m, pos, batch, cell, m.prepare(src, dst, sh, pos.shape[0], A))
    e_ref, f_ref, _ = I.energy_forces(*_to_cpu64(*sysd), p, cfg)
    assert rel_inf(e, e_ref) < TOL
    assert rel_inf(f, f_ref) < TOL


def test_bad_edge_id_poisons_energies_and_forces():
    from fsctep_amd.ictd import energy_forces
    from fsctep_amd.sparse import energy_and_forces
    s = make_system(32, box=10.0, periodic=False, seed=11)
    src = s.edge_src.copy()
    src[5] = 32 + 7                                   # out of range
    sysd = (s.pos, s.species, np.zeros(32, np.int64), src, s.edge_dst, s.edge_shifts, s.cell)
    pos, A, batch, esrc, edst, sh, cell = _to_dev(*sysd)
    m = seeded_hip_model(32, 2, 3).to(DEV)
    e, f = energy_and_forces(m, pos, batch, cell, m.prepare(esrc, edst, sh, 32, A))
    assert torch.isnan(e).all() and torch.isnan(f).all()
    mi = _ictd_model(32, 2, 2)
    e, f, _ = energy_forces(mi, pos, batch, cell, mi.prepare(esrc, edst, sh, 32, A))
    assert torch.isnan(e).all() and torch.isnan(f).all()
    # the LAMMPS-style path: geometry from caller edge vectors, forces through them
    ev = torch.randn(esrc.shape[0], 3, device=DEV).requires_grad_(True)
    en = mi(pos, A, batch, esrc, edst, sh, cell, precomputed_edge_vec=ev)
    (gv,) = torch.autograd.grad(en.sum(), ev)
    assert torch.isnan(en).all() and torch.isnan(gv).all()


def test_o3_auto_preset_matches_oracle():
    """preset 'auto' with a field and a dipole head: 0e, 1o, 2e (the field and the dipole need 1o)."""
    from fsctep_amd.ictd import energy_forces
    C, L = 32, 2
    m = _ictd_model(C, L, 2, o3=True, field=True, dipole=True, active=None, preset="auto")
    assert m.keys == [(0, 1), (1, -1), (2, 1)]
    cfg, p = _ictd_oracle(m, C, L, 2, o3=True, field=True, dipole=True)
    s = make_system(40, box=11.0, periodic=True, seed=303)
    sysd = (s.pos, s.species, np.zeros(40, np.int64), s.edge_src, s.edge_dst, s.edge_shifts, s.cell)
    pos, A, batch, src, dst, sh, cell = _to_dev(*sysd)
    fld = np.array([[0.07, -0.02, 0.11]], np.float32)
    e, f, dip = energy_forces(m, pos, batch, cell, m.prepare(src, dst, sh, 40, A),
                              external_tensor=torch.tensor(fld, device=DEV))
    e_ref, f_ref, d_ref = I.energy_forces(*_to_cpu64(*sysd), p, cfg, torch.tensor(fld, dtype=torch.float64))
    assert rel_inf(e, e_ref) < TOL
    assert rel_inf(f, f_ref) < TOL
    assert rel_inf(dip, d_ref) < TOL
