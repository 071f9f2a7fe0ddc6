"""Parity at the benchmark sizes (10k-atom sparse and ICTD, 4k-atom ICTD-O3 with a field, 100k-atom
sparse), where the oracle cannot run the whole system, through properties that do not depend on size:

* locality: an atom's energy depends only on atoms within 3 cutoffs (three message-passing layers), so
  the oracle evaluates a 15.5 A cluster cut around a few atoms and the centre energies must match the
  GPU values of the full periodic system (the sparse conv2 normalisation E/N is the one non-local
  term; the cluster is evaluated with its parent's E/N);
* determinism (bitwise equal repeats); translation invariance, exact: positions are snapped to a
  2^-16 A grid and shifted by grid multiples, so every fp32 coordinate and every edge vector is
  bit-identical before and after and so must be the energies and forces; sum of forces = 0; and, for
  the sparse trunk, invariance under the cubic box's axis permutation (an exact symmetry of the
  periodic system; the ICTD readout is not O(3)-invariant in the reference, see test_oracle_ictd).

Tolerance 1e-5 relative to the largest |e| (energies) or |F| (forces) of the system."""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL = 1e-5
RCUT = 5.0


def _gpu_eval(mode, system, seed):
    import bench
    model = bench.build_model(mode, torch.device(DEV))
    pos = torch.tensor(system.pos, dtype=torch.float32, device=DEV)
    A = torch.tensor(system.species, device=DEV)
    batch = torch.zeros(system.num_atoms, dtype=torch.long, device=DEV)
    cell = torch.tensor(system.cell, dtype=torch.float32, device=DEV)
    g = model.prepare(torch.tensor(system.edge_src, device=DEV), torch.tensor(system.edge_dst, device=DEV),
                      torch.tensor(system.edge_shifts, dtype=torch.float32, device=DEV), system.num_atoms, A)
    if mode == "sparse":
        from fsctep_amd.sparse import energy_and_forces

        def run(p):
            return energy_and_forces(model, p, batch, cell, g)
    else:
        from fsctep_amd.ictd import energy_forces
        field = torch.tensor(bench._field(1, seed), dtype=torch.float32, device=DEV) if mode == "ictd-o3" else None

        def run(p):
            e, f, _ = energy_forces(model, p, batch, cell, g, external_tensor=field)
            return e, f
    return run, pos


def _cluster(system, centre, radius):
    """Atoms within ``radius`` of ``centre`` (minimum image), centred, with an open radius graph."""
    from fsctep_amd.synthetic import radius_graph
    L = float(system.cell[0, 0, 0])
    assert 2 * radius < L
    d = system.pos - system.pos[centre]
    d -= L * np.round(d / L)
    keep = np.flatnonzero(np.linalg.norm(d, axis=1) < radius)
    pos = d[keep]
    cell = np.eye(3)[None] * 100.0
    src, dst, sh = radius_graph(pos, cell, False, RCUT)
    return keep, pos, system.species[keep], src, dst, sh, int(np.flatnonzero(keep == centre)[0])


def _oracle_cluster_energy(mode, system, centre, seed):
    from fsctep_amd.synthetic import seeded_value
    keep, pos, spec, src, dst, sh, ci = _cluster(system, centre, 3 * RCUT + 0.5)
    args = (torch.tensor(pos, dtype=torch.float64), torch.tensor(spec), torch.zeros(len(keep), dtype=torch.long),
            torch.tensor(src), torch.tensor(dst), torch.tensor(sh, dtype=torch.float64),
            torch.eye(3, dtype=torch.float64)[None] * 100.0)
    with torch.no_grad():
        if mode == "sparse":
            from oracle import sparse_ref as R
            cfg = R.SparseConfig(channels=64, num_interaction=3, function_type="bessel")
            p = {k: torch.tensor(seeded_value(k, s, 1), dtype=torch.float64) for k, s in R.param_shapes(cfg)}
            e = R.atom_energies(*args, p, cfg, avg_degree=system.num_edges / system.num_atoms)
        else:
            import bench
            from oracle import ictd_ref as R
            o3 = mode == "ictd-o3"
            w = bench.WORKLOADS[mode]
            cfg = R.ICTDConfig(channels=w["channels"], lmax=w["lmax"], num_interaction=w["layers"],
                               function_type="bessel", o3=o3,
                               active=((0, 1), (1, 1), (1, -1), (2, 1)) if o3 else (), external_field=o3, dipole=o3)
            p = {k: torch.tensor(seeded_value(k, s, 1), dtype=torch.float64) for k, s in R.param_shapes(cfg)}
            field = torch.tensor(bench._field(1, seed), dtype=torch.float64) if o3 else None
            e, _ = R.forward(*args, p, cfg, field)
    return float(e.squeeze(-1)[ci])


def _check(mode, n_atoms, seed, centres):
    import bench
    system = bench._system(mode, n_atoms, seed)
    system.pos = np.round(system.pos * 2.0 ** 16) / 2.0 ** 16        # exactly representable in fp32
    run, pos = _gpu_eval(mode, system, seed)
    e, f = run(pos)
    e2, f2 = run(pos)
    torch.cuda.synchronize()
    assert torch.equal(e, e2) and torch.equal(f, f2), "repeat evaluation is not bitwise identical"
    emax, fmax = float(e.abs().max()), float(f.abs().max())
    # sum of forces of a periodic system
    assert float(f.double().sum(0).abs().max()) < 1e-3 * fmax * max(1.0, (n_atoms / 1e4) ** 0.5)
    # translation by grid multiples: bit-identical edge vectors, so bit-identical results
    shift = torch.tensor([24231, -79298, 134349], dtype=torch.float64) / 2.0 ** 16     # (0.37, -1.21, 2.05) A
    pos_t = (torch.tensor(system.pos) + shift).to(torch.float32).to(DEV)
    assert torch.equal(pos_t.double().cpu() - shift, torch.tensor(system.pos))            # exact in fp32
    et, ft = run(pos_t)
    assert torch.equal(et, e) and torch.equal(ft, f)
    # local parity against the oracle
    ec = e.double().cpu().numpy()
    for c in centres:
        ref = _oracle_cluster_energy(mode, system, c, seed)
        assert abs(ec[c] - ref) < TOL * emax, (c, ec[c], ref)
    return system, run, pos, e, f


def test_sparse_10k_local_parity_and_invariances():
    system, run, pos, e, f = _check("sparse", 10000, 22, centres=[0, 4321])
    # the cubic box is invariant under x->y->z: energies equal, forces permuted
    perm = [1, 2, 0]
    from fsctep_amd.synthetic import AtomicSystem
    ps = AtomicSystem(pos=system.pos[:, perm], species=system.species, cell=system.cell, periodic=True,
                      edge_src=system.edge_src, edge_dst=system.edge_dst, edge_shifts=system.edge_shifts[:, perm])
    run_p, pos_p = _gpu_eval("sparse", ps, 22)
    ep, fp = run_p(pos_p)
    assert float((ep - e).abs().max()) < TOL * float(e.abs().max())
    assert float((fp - f[:, perm]).abs().max()) < TOL * float(f.abs().max())


def test_ictd_10k_local_parity_and_invariances():
    _check("ictd", 10000, 33, centres=[17])


def test_ictd_o3_field_4k_local_parity_and_invariances():
    _check("ictd-o3", 4000, 44, centres=[5, 2500])


def test_sparse_100k_local_parity():
    _check("sparse", 100000, 22, centres=[99999])
