"""Write golden vectors of the reference ICTD trunks (``pure-cartesian-ictd`` and ``-o3``).

Runs ``PureCartesianICTDTransformerLayer`` (models/pure_cartesian_ictd_layers_full.py:476-1078) and
``PureCartesianICTDO3TransformerLayer`` (models/pure_cartesian_ictd_layers_o3.py:535-1074, with a
rank-1 "1o" external field and a dipole head) from the reference tree on seeded systems with
seeded parameters; stores inputs, the parameter seed, energies, forces (and dipole) in fp64/fp32
plus the reference state_dict keys.  Only run in a container that holds the reference.

    python tests/golden/make_ictd_golden.py
"""

from __future__ import annotations

import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import refimport  # noqa: E402
from fsctep_amd.synthetic import make_system, seeded_value, SPECIES_4, SPECIES_8  # noqa: E402

CASES = {
    "ictd_open32_c32_l2": dict(n=32, box=10.0, periodic=False, seed=13, species=SPECIES_4, channels=32,
                               lmax=2, layers=2, o3=False, pseed=303),
    "ictd_pbc64_c128_l3": dict(n=64, density=0.1, periodic=True, seed=33, species=SPECIES_8, channels=128,
                               lmax=3, layers=3, o3=False, pseed=404),
    "ictdo3_pbc64_c64_l2_field": dict(n=64, density=0.1, periodic=True, seed=44, species=SPECIES_4, channels=64,
                                      lmax=2, layers=3, o3=True, pseed=505, field_seed=7),
}


def build_reference(c, dtype):
    prev = torch.get_default_dtype()
    torch.set_default_dtype(dtype)
    common = dict(max_embed_radius=5.0, main_max_radius=5.0, main_number_of_basis=8,
                  hidden_dim_conv=c["channels"], hidden_dim_sh=c["channels"], hidden_dim=64, channel_in2=32,
                  embedding_dim=16, max_atomvalue=10, output_size=8, embed_size=[128, 128, 128],
                  num_interaction=c["layers"], device=torch.device("cpu"), function_type_main="bessel",
                  lmax=c["lmax"], ictd_tp_path_policy="full", internal_compute_dtype=dtype,
                  invariant_channels=32)
    try:
        if c["o3"]:
            mod = refimport.load("molecular_force_field.models.pure_cartesian_ictd_layers_o3")
            m = mod.PureCartesianICTDO3TransformerLayer(
                **common, o3_active_irreps="0e,1e,1o,2e", external_tensor_rank=1, external_tensor_irrep="1o",
                physical_tensor_outputs={"dipole": {"irreps": ["1o"], "channels_out": 1, "reduce": "sum"}})
        else:
            mod = refimport.load("molecular_force_field.models.pure_cartesian_ictd_layers_full")
            m = mod.PureCartesianICTDTransformerLayer(**common)
    finally:
        torch.set_default_dtype(prev)
    return m.to(dtype)


def apply_seeded(model, seed):
    with torch.no_grad():
        for name, p in model.named_parameters():
            p.copy_(torch.from_numpy(seeded_value(name, tuple(p.shape), seed)).to(p.dtype))


def run(model, s, dtype, field, o3):
    pos = torch.tensor(s.pos, dtype=dtype, requires_grad=True)
    args = (pos, torch.tensor(s.species), torch.zeros(s.num_atoms, dtype=torch.long), torch.tensor(s.edge_src),
            torch.tensor(s.edge_dst), torch.tensor(s.edge_shifts, dtype=dtype), torch.tensor(s.cell, dtype=dtype))
    dip = None
    if o3:
        e, phys = model(*args, external_tensor=torch.tensor(field, dtype=dtype), return_physical_tensors=True)
        dip = phys["dipole"][1].detach().numpy()
    else:
        e = model(*args)
    (g,) = torch.autograd.grad(e.sum(), pos)
    return e.detach().squeeze(-1).numpy(), (-g).numpy(), dip


def main():
    only = set(sys.argv[1:])
    for name, c in CASES.items():
        if only and name not in only:
            continue
        if c["periodic"]:
            s = make_system(c["n"], density=c["density"], periodic=True, species=c["species"], seed=c["seed"])
        else:
            s = make_system(c["n"], box=c["box"], periodic=False, species=c["species"], seed=c["seed"])
        field = None
        if c["o3"]:
            field = np.random.default_rng(c["field_seed"]).normal(0.0, 0.1, size=(1, 3))
        out = dict(pos=s.pos, species=s.species, cell=s.cell, periodic=np.asarray(s.periodic),
                   edge_src=s.edge_src, edge_dst=s.edge_dst, edge_shifts=s.edge_shifts,
                   channels=np.asarray(c["channels"]), layers=np.asarray(c["layers"]), lmax=np.asarray(c["lmax"]),
                   o3=np.asarray(c["o3"]), param_seed=np.asarray(c["pseed"]), function_type=np.asarray("bessel"))
        if field is not None:
            out["external_field"] = field
        for dt, tag in ((torch.float64, "f64"), (torch.float32, "f32")):
            m = build_reference(c, dt)
            apply_seeded(m, c["pseed"])
            e, f, dip = run(m, s, dt, field, c["o3"])
            out[f"energy_{tag}"] = e
            out[f"forces_{tag}"] = f
            if dip is not None:
                out[f"dipole_{tag}"] = dip
            print(name, tag, "E=", float(e.sum()), "max|e|=", float(np.abs(e).max()),
                  "max|F|=", float(np.abs(f).max()), "edges=", s.num_edges,
                  "dipole=", None if dip is None else dip.ravel(), flush=True)
        np.savez_compressed(os.path.join(HERE, name + ".npz"), **out)
        keys = [[k, list(v.shape)] for k, v in m.state_dict().items()]
        with open(os.path.join(HERE, name + "_state_dict.json"), "w") as fh:
            json.dump(keys, fh, indent=0)


if __name__ == "__main__":
    main()
