"""The full-size fp64 oracle fixtures (tests/golden/oracle_<mode>_<atoms>.npz) describe the systems
bench.py builds today: same seed, same sha256 of positions, species, neighbour list and cell, and the
stored per-atom energies add up to the stored total."""

import glob
import os

import numpy as np
import pytest

from conftest import GOLDEN

FIXTURES = sorted(os.path.basename(p)[:-4] for p in glob.glob(os.path.join(GOLDEN, "oracle_*.npz")))


@pytest.mark.skipif(not FIXTURES, reason="no full-size oracle fixture in tests/golden")
@pytest.mark.parametrize("name", FIXTURES)
def test_fixture_matches_bench_system(name):
    import bench
    fx = np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False)
    mode, atoms, seed = str(fx["mode"]), int(fx["atoms"]), int(fx["seed"])
    assert name == f"oracle_{mode}_{atoms}" and seed == bench.WORKLOADS[mode]["seed"]
    system = bench._system(mode, atoms, seed)
    assert bench.system_digest(system) == str(fx["system_sha256"])
    assert fx["energy"].shape == (atoms,) and fx["forces"].shape == (atoms, 3) and int(fx["edges"]) == system.num_edges
    assert abs(float(fx["energy"].astype(np.float64).sum()) - float(fx["energy_total"])) < 1e-5 * abs(float(fx["energy_total"]))
    assert np.isfinite(fx["forces"]).all()
    # forces of a periodic system sum to zero (to the fp32 rounding of the stored values)
    assert float(np.abs(fx["forces"].astype(np.float64).sum(0)).max()) < 1e-5 * float(np.abs(fx["forces"]).max()) * atoms ** 0.5
