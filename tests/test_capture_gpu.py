"""HIP-graph replay of the energy + forces step (fsctep_amd.capture) against the eager step.

Each captured graph is replayed several times with the program's own eager work and synchronisations in
between (a memset node recorded by a library call would show up as a wrong replay after the first), and
with new positions copied in between replays; every replay must equal the eager step on the same
positions bit for bit (the kernels are deterministic: segmented sums, no float atomics), and the eager
step matches the reference golden vectors at 1e-5."""

import os

import numpy as np
import pytest
import torch

from conftest import GOLDEN, load_golden
from sparse_helpers import rel_inf, seeded_hip_model

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _inputs(g):
    n = g["pos"].shape[0]
    pos = torch.tensor(g["pos"], dtype=torch.float32, device=DEV)
    A = torch.tensor(g["species"], device=DEV)
    batch = torch.zeros(n, dtype=torch.long, device=DEV)
    cell = torch.tensor(g["cell"], dtype=torch.float32, device=DEV)
    src, dst = torch.tensor(g["edge_src"], device=DEV), torch.tensor(g["edge_dst"], device=DEV)
    sh = torch.tensor(g["edge_shifts"], dtype=torch.float32, device=DEV)
    return pos, A, batch, cell, src, dst, sh


def _check_replays(model, g, eager, ext=None):
    from fsctep_amd.capture import CapturedEnergyForces
    pos, A, batch, cell, src, dst, sh = _inputs(g)
    graph = model.prepare(src, dst, sh, pos.shape[0], A)
    cap = CapturedEnergyForces(model, pos, batch, cell, graph, external_tensor=ext)
    gen = torch.Generator(device="cpu").manual_seed(4)
    moved = pos + 0.01 * torch.randn(pos.shape, generator=gen).to(DEV)
    want0 = eager(pos, batch, cell, graph, ext)
    want1 = eager(moved, batch, cell, graph, ext)
    for it in range(4):
        p, want = (pos, want0) if it % 2 == 0 else (moved, want1)
        out = cap(p)
        torch.cuda.synchronize()
        for a, b in zip(out, want):
            if b is not None:
                assert torch.equal(a, b), f"replay {it} differs from the eager step"
        # eager work between replays (allocations, reductions, a separate step)
        junk = torch.randn(4096, device=DEV).sum()
        eager(moved, batch, cell, graph, ext)
        torch.cuda.synchronize()
        del junk
    return want0


def test_sparse_step_replays_equal_eager():
    from fsctep_amd.sparse import energy_and_forces
    g = load_golden("sparse_open32_c32_l2")
    m = seeded_hip_model(int(g["channels"]), int(g["layers"]), int(g["param_seed"])).to(DEV)

    def eager(pos, batch, cell, graph, ext):
        e, f = energy_and_forces(m, pos, batch, cell, graph)
        return e, f, None
    e, f, _ = _check_replays(m, g, eager)
    assert rel_inf(e, g["energy_f64"]) < 1e-5 and rel_inf(f, g["forces_f64"]) < 1e-5


@pytest.mark.parametrize("name", ["ictd_pbc64_c128_l3", "ictdo3_pbc64_c64_l2_field"])
def test_ictd_step_replays_equal_eager(name):
    from fsctep_amd.ictd import energy_forces
    from test_ictd_gpu import _model
    g = load_golden(name)
    m = _model(g)
    ext = torch.tensor(g["external_field"], dtype=torch.float32, device=DEV) if "external_field" in g else None

    def eager(pos, batch, cell, graph, ext):
        return energy_forces(m, pos, batch, cell, graph, external_tensor=ext)
    e, f, dip = _check_replays(m, g, eager, ext)
    assert rel_inf(e, g["energy_f64"]) < 1e-5 and rel_inf(f, g["forces_f64"]) < 1e-5
    if "dipole_f64" in g:
        assert rel_inf(dip, g["dipole_f64"]) < 1e-5


def test_sparse_1k_step_replays_equal_eager():
    """The 1,000-atom benchmark system (C 64, 3 layers), whose fp64 oracle values are a fixture."""
    import bench
    from fsctep_amd.capture import CapturedEnergyForces
    from fsctep_amd.sparse import energy_and_forces
    fx = np.load(os.path.join(GOLDEN, "oracle_sparse_1000.npz"), allow_pickle=False)
    s = bench._system("sparse", 1000, int(fx["seed"]))
    m = bench.build_model("sparse", torch.device(DEV))
    pos = torch.tensor(s.pos, dtype=torch.float32, device=DEV)
    A = torch.tensor(s.species, device=DEV)
    batch = torch.zeros(1000, dtype=torch.long, device=DEV)
    cell = torch.tensor(s.cell, dtype=torch.float32, device=DEV)
    graph = m.prepare(torch.tensor(s.edge_src, device=DEV), torch.tensor(s.edge_dst, device=DEV),
                      torch.tensor(s.edge_shifts, dtype=torch.float32, device=DEV), 1000, A, pos=pos)
    e0, f0 = energy_and_forces(m, pos, batch, cell, graph)
    cap = CapturedEnergyForces(m, pos, batch, cell, graph)
    for _ in range(3):
        e, f, _ = cap(pos)
        torch.cuda.synchronize()
        assert torch.equal(e, e0) and torch.equal(f, f0)
        energy_and_forces(m, pos, batch, cell, graph)
    assert rel_inf(e, fx["energy"]) < 1e-5 and rel_inf(f, fx["forces"]) < 1e-5
