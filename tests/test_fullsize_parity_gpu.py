"""Energies, forces (and the O3 dipole) of whole benchmark systems against the fp64 oracle.

The fixtures ``tests/golden/oracle_<mode>_<atoms>.npz`` hold the oracle's per-atom energies, forces and
dipole for the exact systems bench.py builds (seeded positions, neighbour list and parameters; the
system's sha256 is stored and checked here).  They are written on the CPU by
``tests/golden/make_fullsize_oracle.py``; the oracle itself is pinned by the reference golden vectors
(tests/test_oracle_*.py).  The GPU step runs here through the same entry points bench.py times.

Tolerance: 1e-5 relative to the largest |e| (energies), |F| (forces) or |dipole| of the system; the
measured margins are printed."""

import glob
import os

import numpy as np
import pytest
import torch

from conftest import GOLDEN

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL = 1e-5

FIXTURES = sorted(os.path.basename(p)[:-4] for p in glob.glob(os.path.join(GOLDEN, "oracle_*.npz")))


def _rel(a, b) -> float:
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def _gpu_step(mode, system, seed):
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
        e, f = energy_and_forces(model, pos, batch, cell, g)
        dip = None
    else:
        from fsctep_amd.ictd import energy_forces
        field = torch.tensor(bench._field(1, seed), dtype=torch.float32, device=DEV) if mode == "ictd-o3" else None
        e, f, dip = energy_forces(model, pos, batch, cell, g, external_tensor=field)
    torch.cuda.synchronize()
    return e.cpu().numpy(), f.cpu().numpy(), None if dip is None else dip.cpu().numpy().reshape(-1, 3)


@pytest.mark.skipif(not FIXTURES, reason="no full-size oracle fixture in tests/golden")
@pytest.mark.parametrize("name", FIXTURES)
def test_whole_system_matches_fp64_oracle(name):
    import bench
    fx = np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False)
    mode, atoms, seed = str(fx["mode"]), int(fx["atoms"]), int(fx["seed"])
    system = bench._system(mode, atoms, seed)
    assert bench.system_digest(system) == str(fx["system_sha256"]), "bench.py now builds another system"
    e, f, dip = _gpu_step(mode, system, seed)
    er, fr = _rel(e, fx["energy"]), _rel(f, fx["forces"])
    msg = f"{name}: energy {er:.2e}, forces {fr:.2e}"
    if dip is not None:
        dr = _rel(dip, fx["dipole"])
        msg += f", dipole {dr:.2e}"
        assert dr < TOL, msg
    print(msg)
    assert er < TOL and fr < TOL, msg
    # the total energy too (a sum of 1e3-1e5 terms of both signs)
    et = abs(float(np.sum(e, dtype=np.float64)) - float(fx["energy_total"])) / abs(float(fx["energy_total"]))
    assert et < TOL, (msg, et)
