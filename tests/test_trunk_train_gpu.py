"""Force-loss training through the drop-in trunks (training/trainer.py:1292-1297): in train() mode,
F = -dE/dpos with create_graph, loss = sum F^2, then the gradient of every parameter of the model.

The device side is the trunk itself on the GPU (fp32; conv2..n on the HIP ops with their double backward,
the rest on the differentiable formulations of fsctep_amd.train_ops); the reference side is the fp64
oracle (oracle/sparse_ref.py, oracle/ictd_ref.py, pinned by the reference golden vectors) differentiated
by torch autograd on the CPU, on the same systems and parameters.  Tolerance: each parameter's gradient
within 2e-5 of the oracle's, max-norm, relative to the largest entry of that gradient (floored at 1e-3 of
the largest gradient entry of the whole model: parameters the force loss barely reaches, such as the
final bias, which cancels from the forces, have gradients of pure rounding).  Energies and forces of the
training step also equal the golden vectors at 1e-5, and the training step's forces equal the inference
step's."""

import numpy as np
import pytest
import torch

from conftest import load_golden
from fsctep_amd.synthetic import seeded_value

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL = 2e-5


def _rel(a, b, floor):
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    return float((a - b).abs().max() / max(float(b.abs().max()), floor))


def _device_loss(model, g, ext=None):
    """(energies, forces, {name: gradient}) of sum F^2 on the GPU, model in train() mode."""
    n = g["pos"].shape[0]
    pos = torch.tensor(g["pos"], dtype=torch.float32, device=DEV).requires_grad_(True)
    A = torch.tensor(g["species"], device=DEV)
    batch = torch.zeros(n, dtype=torch.long, device=DEV)
    cell = torch.tensor(g["cell"], dtype=torch.float32, device=DEV)
    src, dst = torch.tensor(g["edge_src"], device=DEV), torch.tensor(g["edge_dst"], device=DEV)
    sh = torch.tensor(g["edge_shifts"], dtype=torch.float32, device=DEV)
    model.train().requires_grad_(True)
    kw = {} if ext is None else {"external_tensor": ext}
    e = model(pos, A, batch, src, dst, sh, cell, **kw)
    (gp,) = torch.autograd.grad(e.sum(), pos, create_graph=True)
    loss = (gp ** 2).sum()
    names = [k for k, p in model.named_parameters()]
    grads = torch.autograd.grad(loss, [p for _, p in model.named_parameters()], allow_unused=True)
    torch.cuda.synchronize()
    out = {k: (gr if gr is not None else torch.zeros_like(p)) for k, gr, p in
           zip(names, grads, [p for _, p in model.named_parameters()])}
    return e.detach().squeeze(-1), -gp.detach(), out


def _oracle_loss(energy_fn, params, g):
    """(energies, forces, {name: gradient}) of sum F^2 from the fp64 oracle."""
    p = {k: v.detach().clone().requires_grad_(True) for k, v in params.items()}
    pos = torch.tensor(g["pos"], dtype=torch.float32).double().requires_grad_(True)
    e = energy_fn(pos, p)
    (gp,) = torch.autograd.grad(e.sum(), pos, create_graph=True)
    loss = (gp ** 2).sum()
    grads = torch.autograd.grad(loss, list(p.values()), allow_unused=True)
    return e.detach().squeeze(-1), -gp.detach(), {k: (gr if gr is not None else torch.zeros_like(p[k]))
                                                   for k, gr in zip(p, grads)}


def _compare(dev, ref, golden):
    e, f, gd = dev
    er, fr, gr = ref
    assert _rel(e, torch.tensor(golden["energy_f64"]), 1e-30) < 1e-5
    assert _rel(f, torch.tensor(golden["forces_f64"]), 1e-30) < 1e-5
    assert _rel(f, fr, 1e-30) < 1e-5
    assert set(gd) == set(gr), set(gd) ^ set(gr)
    floor = 1e-3 * max(float(v.abs().max()) for v in gr.values())
    errs = {k: _rel(gd[k], gr[k], floor) for k in gr}
    worst = sorted(errs.items(), key=lambda kv: -kv[1])[:5]
    print("largest relative gradient errors:", [(k, f"{v:.2e}") for k, v in worst])
    assert max(errs.values()) < TOL, worst
    nonzero = sum(1 for v in gr.values() if float(v.abs().max()) > floor)
    assert nonzero >= len(gr) // 2          # the loss reaches most parameters


@pytest.mark.parametrize("name", ["sparse_open32_c32_l2", "sparse_pbc100_c64_l3"])
def test_sparse_force_loss_gradients(name):
    from oracle import sparse_ref as R
    from sparse_helpers import oracle_params, seeded_hip_model
    g = load_golden(name)
    C, L, seed = int(g["channels"]), int(g["layers"]), int(g["param_seed"])
    m = seeded_hip_model(C, L, seed).to(DEV)
    dev = _device_loss(m, g)
    cfg, p = oracle_params(C, L, seed, torch.float64)
    n = g["pos"].shape[0]
    args = (torch.tensor(g["species"]), torch.zeros(n, dtype=torch.long), torch.tensor(g["edge_src"]),
            torch.tensor(g["edge_dst"]), torch.tensor(g["edge_shifts"], dtype=torch.float32).double(),
            torch.tensor(g["cell"], dtype=torch.float32).double())
    ref = _oracle_loss(lambda pos, prm: R.atom_energies(pos, *args, prm, cfg), p, g)
    _compare(dev, ref, g)
    # the training step's forces are the inference step's
    m.eval().requires_grad_(False)
    from fsctep_amd.sparse import energy_and_forces
    pos = torch.tensor(g["pos"], dtype=torch.float32, device=DEV)
    gr = m.prepare(torch.tensor(g["edge_src"], device=DEV), torch.tensor(g["edge_dst"], device=DEV),
                   torch.tensor(g["edge_shifts"], dtype=torch.float32, device=DEV), n,
                   torch.tensor(g["species"], device=DEV))
    _, f_inf = energy_and_forces(m, pos, torch.zeros(n, dtype=torch.long, device=DEV),
                                 torch.tensor(g["cell"], dtype=torch.float32, device=DEV), gr)
    assert _rel(dev[1], f_inf, 1e-30) < 1e-5


@pytest.mark.parametrize("name", ["ictd_open32_c32_l2", "ictd_pbc64_c128_l3", "ictdo3_pbc64_c64_l2_field"])
def test_ictd_force_loss_gradients(name):
    from oracle import ictd_ref as I
    from test_ictd_gpu import _model
    g = load_golden(name)
    m = _model(g)
    o3 = bool(g["o3"])
    ext = torch.tensor(g["external_field"], dtype=torch.float32, device=DEV) if "external_field" in g else None
    dev = _device_loss(m, g, ext)
    cfg = I.ICTDConfig(channels=int(g["channels"]), lmax=int(g["lmax"]), num_interaction=int(g["layers"]),
                       function_type=str(g["function_type"]), o3=o3,
                       active=((0, 1), (1, 1), (1, -1), (2, 1)) if o3 else (), external_field=o3, dipole=o3)
    p = {k: torch.tensor(seeded_value(k, s, int(g["param_seed"])), dtype=torch.float64)
         for k, s in I.param_shapes(cfg)}
    n = g["pos"].shape[0]
    args = (torch.tensor(g["species"]), torch.zeros(n, dtype=torch.long), torch.tensor(g["edge_src"]),
            torch.tensor(g["edge_dst"]), torch.tensor(g["edge_shifts"], dtype=torch.float32).double(),
            torch.tensor(g["cell"], dtype=torch.float32).double())
    fld = None if ext is None else torch.tensor(g["external_field"], dtype=torch.float32).double()
    ref = _oracle_loss(lambda pos, prm: I.forward(pos, *args, prm, cfg, fld)[0], p, g)
    _compare(dev, ref, g)
