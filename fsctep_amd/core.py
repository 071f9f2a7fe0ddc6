"""TorchScript core for LibTorch / LAMMPS engines, traced over the HIP trunks.

``EdgeVecCore`` has the signature and return tuple of the reference's ``_TorchScriptEdgeVecCore``
(interfaces/lammps_mliap.py:372-442):

    forward(pos (N,3), A (N,) int64, batch (N,) int64, edge_src (E,) int64, edge_dst (E,) int64,
            edge_shifts (E,3), cell (G,3,3), edge_vec (E,3), external_tensor)
      -> (atom_energy (N,1), global_phys (G,22), atom_phys (N,31), global_mask (5,), atom_mask (5,),
          reciprocal_source (N,0))

``edge_vec`` is passed to the trunk as ``precomputed_edge_vec``: the ICTD trunks build their geometry from
it (forces then flow through it back to whatever the caller built it from, e.g. ``pos`` in
lammps_user_mfftorch/src/USER-MFFTORCH/mff_torch_engine.cpp:740-760); the sparse trunk, like the
reference's, ignores it and uses ``pos``.  The physical-tensor slots follow the reference layout
(lammps_mliap.py:84-116, 218-300): only the O3 dipole head exists here, written to global_phys[:, 1:4]
with global_mask[1] = 1.

``export_core`` traces the core the reference's way (``torch.jit.trace`` on N=32, E=256 dummies,
lammps_mliap.py:615-684) and writes ``<path>`` plus the metadata JSON ``<path>.json``
(cli/export_libtorch_core.py:437-525 names the keys kept here).  The traced graph calls
``torch.ops.fsctep.*`` by name, so a LibTorch process needs ``libfsctep_torch.so`` loaded first (the
engine's ``MFF_CUSTOM_OPS_LIB``, mff_torch_engine.cpp:226-249).  Every size the ops need is read from
the tensors at run time (graph preparation, the E/N normalisation), so the trace holds for any N and E.
"""

from __future__ import annotations

import json
import os

import torch
import torch.nn as nn

GLOBAL_PHYS_LAYOUT = (("charge", 1), ("dipole", 3), ("polarizability", 9), ("quadrupole", 9))
ATOM_PHYS_LAYOUT = (("charge_per_atom", 1), ("dipole_per_atom", 3), ("polarizability_per_atom", 9),
                    ("quadrupole_per_atom", 9), ("born_effective_charge_per_atom", 9))
GLOBAL_PHYS_DIM = sum(d for _, d in GLOBAL_PHYS_LAYOUT)            # 22
ATOM_PHYS_DIM = sum(d for _, d in ATOM_PHYS_LAYOUT)                # 31
PHYS_MASK_WIDTH = max(len(GLOBAL_PHYS_LAYOUT), len(ATOM_PHYS_LAYOUT))   # 5
DIPOLE_SLOT = (1, 1, 4)                                            # mask index, column range in global_phys


def _mode(model) -> str:
    from .ictd import PureCartesianICTDO3TransformerLayer, PureCartesianICTDTransformerLayer
    if isinstance(model, PureCartesianICTDO3TransformerLayer):
        return "pure-cartesian-ictd-o3"
    if isinstance(model, PureCartesianICTDTransformerLayer):
        return "pure-cartesian-ictd"
    return "pure-cartesian-sparse"


def external_numel(model) -> int:
    """Entries of the external tensor the model consumes (a rank-1 field: 3; none: 0)."""
    return 3 if getattr(model, "external_field", False) else 0


class EdgeVecCore(nn.Module):
    """The reference core wrapper's contract over a HIP trunk (interfaces/lammps_mliap.py:372-442)."""

    def __init__(self, model: nn.Module):
        super().__init__()
        self.model = model
        self.has_dipole = bool(getattr(model, "_dipole", False))
        self.external_total_numel = external_numel(model)

    def forward(self, pos, A, batch, edge_src, edge_dst, edge_shifts, cell, edge_vec, external_tensor):
        kw = {"precomputed_edge_vec": edge_vec}
        if self.has_dipole:
            kw["return_physical_tensors"] = True
        if self.external_total_numel > 0:
            kw["external_tensor"] = external_tensor
        out = self.model(pos, A, batch, edge_src, edge_dst, edge_shifts, cell, **kw)
        atom_energy = out[0] if isinstance(out, tuple) else out
        G = cell.size(0)
        global_phys = atom_energy.new_zeros(G, GLOBAL_PHYS_DIM)
        atom_phys = atom_energy.new_zeros(pos.size(0), ATOM_PHYS_DIM)
        global_mask = atom_energy.new_zeros(PHYS_MASK_WIDTH)
        atom_mask = atom_energy.new_zeros(PHYS_MASK_WIDTH)
        if self.has_dipole:
            dip = out[1]["dipole"][1]                                 # (G, 1, 3), reduce "sum"
            m, a, b = DIPOLE_SLOT
            global_phys = torch.cat([global_phys[:, :a], dip[:, 0, :].to(global_phys.dtype), global_phys[:, b:]], 1)
            global_mask = torch.cat([global_mask[:m], global_mask.new_ones(1), global_mask[m + 1:]])
        reciprocal_source = atom_energy.new_empty(pos.size(0), 0)
        return atom_energy, global_phys, atom_phys, global_mask, atom_mask, reciprocal_source


def trace_inputs(model, device, N: int = 32, E: int = 256, seed: int = 0):
    """The reference's dummy trace inputs (lammps_mliap.py:640-652): zeros for positions and shifts,
    species 1, one graph, random edges and edge vectors, a 100 A cubic cell."""
    g = torch.Generator().manual_seed(seed)
    ext = external_numel(model)
    return (torch.zeros(N, 3, device=device), torch.ones(N, dtype=torch.long, device=device),
            torch.zeros(N, dtype=torch.long, device=device),
            torch.randint(0, N, (E,), generator=g).to(device), torch.randint(0, N, (E,), generator=g).to(device),
            torch.zeros(E, 3, device=device), torch.eye(3, device=device).unsqueeze(0) * 100.0,
            torch.randn(E, 3, generator=g).to(device),
            torch.zeros(ext, device=device) if ext else torch.empty(0, device=device))


def trace_core(model, device="cuda") -> torch.jit.ScriptModule:
    """torch.jit.trace of EdgeVecCore(model) on the dummy inputs (eval mode, no parameter gradients)."""
    model = model.to(device).eval().requires_grad_(False)
    core = EdgeVecCore(model)
    inputs = trace_inputs(model, device)
    with torch.no_grad():
        core(*inputs)                                                 # fill the constant caches first
    ts = torch.jit.trace(core, inputs, check_trace=False, strict=False)
    return ts.eval()


def export_core(model, path: str, device="cuda", elements=None) -> str:
    """Trace and save ``path`` (TorchScript) and ``path + '.json'`` (metadata); returns ``path``."""
    ts = trace_core(model, device)
    os.makedirs(os.path.dirname(os.path.abspath(path)), exist_ok=True)
    torch.jit.save(ts, path)
    ext = external_numel(model)
    meta = {
        "elements": list(elements) if elements is not None else None,
        "tensor_product_mode": _mode(model),
        "device_exported_from": str(device),
        "max_radius": float(model.max_radius),
        "num_interaction": int(model.num_interaction),
        "dtype": "float32",
        "internal_compute_dtype_export": "float32",
        "embed_e0": False,
        "export_reciprocal_source": False,
        "forward_signature": ["pos(N,3)", "A(N,) atomic number (int64)", "batch(N,) (int64)", "edge_src(E,) (int64)",
                              "edge_dst(E,) (int64)", "edge_shifts(E,3)", "cell(1,3,3)", "edge_vec(E,3)",
                              "external_tensor(rank-dependent tensor or empty tensor)"],
        "external_tensor_rank": 1 if ext else None,
        "external_tensor_irrep": "1o" if ext else None,
        "external_tensor_total_numel": ext,
        "external_tensor_has_field_1o": bool(ext),
        "num_fidelity_levels": 0,
        "runtime_fidelity_input": False,
        "custom_ops_library": "libfsctep_torch.so (load before torch::jit::load, e.g. via MFF_CUSTOM_OPS_LIB)",
        "notes": ["Core model: outputs per-atom energy.",
                  "Forces: dE/d(pos) computed via autograd on C++ side.",
                  "Loadable: C++ torch::jit::load(path) after dlopen of libfsctep_torch.so (RTLD_GLOBAL).",
                  "external_tensor is required at runtime when external_tensor_rank is not null."],
    }
    with open(path + ".json", "w", encoding="utf-8") as fh:
        json.dump(meta, fh, indent=2)
    return path
