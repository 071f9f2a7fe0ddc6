"""The exported TorchScript core (fsctep_amd.core, the contract of the reference's _TorchScriptEdgeVecCore,
interfaces/lammps_mliap.py:372-442): traced once on the reference's N=32, E=256 dummies, it must reproduce
the reference golden energies, forces (and the O3 dipole) of every golden system at other N and E, both in
Python and in a compiled LibTorch program with no Python that loads libfsctep_torch.so with dlopen and
takes forces by C++ autograd on the GPU, as the LAMMPS engine does (mff_torch_engine.cpp:226-255,740-864).
make_fx of energy + forces through the reference-signature forward() must trace and replay."""

import os
import subprocess

import numpy as np
import pytest
import torch

from conftest import ROOT, load_golden
from sparse_helpers import rel_inf, seeded_hip_model

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = 1e-5
CASES = ["sparse_open32_c32_l2", "sparse_pbc100_c64_l3", "ictd_open32_c32_l2", "ictd_pbc64_c128_l3",
         "ictdo3_pbc64_c64_l2_field"]
CORE_RUN = os.path.join(ROOT, "tests", "cpp", "core_run")


def _model(name, g):
    if name.startswith("sparse"):
        return seeded_hip_model(int(g["channels"]), int(g["layers"]), int(g["param_seed"])).to(DEV)
    from test_ictd_gpu import _model as ictd_model
    return ictd_model(g)


def _inputs(g):
    n, e = g["pos"].shape[0], g["edge_src"].shape[0]
    ext = g["external_field"].reshape(-1).astype(np.float32) if "external_field" in g else np.zeros(0, np.float32)
    return dict(pos=torch.tensor(g["pos"], dtype=torch.float32, device=DEV),
                A=torch.tensor(g["species"], device=DEV), batch=torch.zeros(n, dtype=torch.long, device=DEV),
                src=torch.tensor(g["edge_src"], device=DEV), dst=torch.tensor(g["edge_dst"], device=DEV),
                shifts=torch.tensor(g["edge_shifts"], dtype=torch.float32, device=DEV),
                cell=torch.tensor(g["cell"], dtype=torch.float32, device=DEV).reshape(1, 3, 3),
                ext=torch.tensor(ext, device=DEV), N=n, E=e)


def _engine_step(core, d):
    """mff_torch_engine.cpp:740-820 in Python: pos leaf, edge_vec from pos, forces by autograd."""
    pos = d["pos"].clone().detach().requires_grad_(True)
    shift_vec = (d["shifts"].unsqueeze(-1) * d["cell"].index_select(0, d["batch"].index_select(0, d["src"]))).sum(1)
    edge_vec = pos.index_select(0, d["dst"]) - pos.index_select(0, d["src"]) + shift_vec
    out = core(pos, d["A"], d["batch"], d["src"], d["dst"], d["shifts"], d["cell"], edge_vec, d["ext"])
    (grad,) = torch.autograd.grad(out[0].sum(), pos)
    return out, -grad


def _check(name, g, e, f, gphys, gmask):
    assert rel_inf(e, g["energy_f64"]) < TOL, name
    assert rel_inf(f, g["forces_f64"]) < TOL, name
    if "dipole_f64" in g:
        assert rel_inf(gphys[:, 1:4], g["dipole_f64"].reshape(-1, 3)) < TOL
        assert gmask.tolist() == [0.0, 1.0, 0.0, 0.0, 0.0]
    else:
        assert float(np.abs(gphys).max()) == 0.0 and float(np.abs(gmask).max()) == 0.0


@pytest.mark.parametrize("name", CASES)
def test_traced_core_python_and_libtorch(name, tmp_path):
    from fsctep_amd.core import export_core
    g = load_golden(name)
    m = _model(name, g)
    path = export_core(m, str(tmp_path / "core.pt"), device=DEV)
    assert os.path.exists(path + ".json")
    core = torch.jit.load(path, map_location=DEV)
    assert "fsctep::graph_prepare" in str(core.inlined_graph)
    d = _inputs(g)
    out, f = _engine_step(core, d)
    assert out[0].shape == (d["N"], 1) and out[1].shape == (1, 22) and out[2].shape == (d["N"], 31)
    assert out[5].shape == (d["N"], 0)
    _check(name, g, out[0].detach().cpu().numpy().reshape(-1), f.cpu().numpy(), out[1].detach().cpu().numpy(),
           out[3].detach().cpu().numpy())

    # the same core in a compiled LibTorch process without Python
    assert os.path.exists(CORE_RUN), "tests/cpp/core_run is built by fsctep_amd.build"
    io = tmp_path / "io"
    io.mkdir()
    (io / "meta.txt").write_text(f"{d['N']} {d['E']} {d['ext'].numel()}\n")
    for k, key, dt in (("pos", "pos.f32", np.float32), ("species", "A.i64", np.int64), ("edge_src", "src.i64", np.int64),
                       ("edge_dst", "dst.i64", np.int64), ("edge_shifts", "shifts.f32", np.float32),
                       ("cell", "cell.f32", np.float32)):
        np.ascontiguousarray(np.asarray(g[k]).astype(dt)).tofile(io / key)
    d["ext"].cpu().numpy().astype(np.float32).tofile(io / "external.f32")
    from fsctep_amd import _lib
    env = {k: v for k, v in os.environ.items() if not k.startswith("PYTHON")}
    run = subprocess.run([CORE_RUN, _lib.TORCH_LIB_PATH, path, str(io), "2"], capture_output=True, text=True,
                         timeout=240, env=env)
    assert run.returncode == 0, run.stdout + run.stderr
    res = np.fromfile(io / "out.f32", dtype=np.float32)
    N = d["N"]
    assert res.shape == (N + 3 * N + 22 + 5,)
    _check(name, g, res[:N], res[N:4 * N].reshape(N, 3), res[4 * N:4 * N + 22].reshape(1, 22), res[4 * N + 22:])


@pytest.mark.parametrize("name", ["sparse_pbc100_c64_l3", "ictd_pbc64_c128_l3", "ictdo3_pbc64_c64_l2_field"])
def test_make_fx_energy_forces(name):
    from torch.fx.experimental.proxy_tensor import make_fx
    g = load_golden(name)
    m = _model(name, g)
    d = _inputs(g)
    kw = {"external_tensor": d["ext"]} if d["ext"].numel() else {}

    def energy_forces(pos, A, batch, src, dst, shifts, cell):
        pos = pos.requires_grad_(True)
        e = m(pos, A, batch, src, dst, shifts, cell, **kw)
        (grad,) = torch.autograd.grad(e.sum(), pos)
        return e, -grad

    args = (d["pos"], d["A"], d["batch"], d["src"], d["dst"], d["shifts"], d["cell"])
    gm = make_fx(energy_forces)(*[a.clone() for a in args])
    text = str(gm.graph)
    assert "fsctep.graph_prepare" in text and "backward" in text
    e, f = gm(*[a.clone() for a in args])
    assert rel_inf(e.squeeze(-1), g["energy_f64"]) < TOL
    assert rel_inf(f, g["forces_f64"]) < TOL


@pytest.mark.parametrize("name", CASES)
def test_libtorch_core_under_hip_graph_capture(name, tmp_path):
    """The engine's CUDA-graph path (mff_torch_engine.cpp:648-737) in the Python-free runner: forward and
    force backward captured once on a pool stream over static inputs, replayed on three position sets
    with eager runs in between; every replay equals the eager step (energies bitwise, forces and dipole to
    1e-6 of their largest entry: torch's index_add backward of the engine-side edge_vec gather and the
    dipole's sum over atoms are atomic) and the first the golden."""
    from fsctep_amd import _lib
    from fsctep_amd.core import export_core
    g = load_golden(name)
    m = _model(name, g)
    path = export_core(m, str(tmp_path / "core.pt"), device=DEV)
    d = _inputs(g)
    io = tmp_path / "io"
    io.mkdir()
    (io / "meta.txt").write_text(f"{d['N']} {d['E']} {d['ext'].numel()}\n")
    for k, key, dt in (("pos", "pos.f32", np.float32), ("species", "A.i64", np.int64), ("edge_src", "src.i64", np.int64),
                       ("edge_dst", "dst.i64", np.int64), ("edge_shifts", "shifts.f32", np.float32),
                       ("cell", "cell.f32", np.float32)):
        np.ascontiguousarray(np.asarray(g[k]).astype(dt)).tofile(io / key)
    d["ext"].cpu().numpy().astype(np.float32).tofile(io / "external.f32")
    env = {k: v for k, v in os.environ.items() if not k.startswith("PYTHON")}
    run = subprocess.run([CORE_RUN, _lib.TORCH_LIB_PATH, path, str(io), "3", "graph"], capture_output=True, text=True,
                         timeout=240, env=env)
    assert run.returncode == 0, run.stdout + run.stderr
    assert "graph replays equal to eager: 3/3" in run.stdout, run.stdout
    res = np.fromfile(io / "out.f32", dtype=np.float32)
    N = d["N"]
    _check(name, g, res[:N], res[N:4 * N].reshape(N, 3), res[4 * N:4 * N + 22].reshape(1, 22), res[4 * N + 22:])
