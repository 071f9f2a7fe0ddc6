"""Write golden vectors of the reference ``pure-cartesian-sparse`` trunk.

Runs ``PureCartesianSparseTransformerLayer`` from the reference tree
(``models/pure_cartesian_sparse_layers.py:459-855``) on seeded systems with seeded
parameters (``fsctep_amd.synthetic.seeded_value`` per state_dict key) and stores
inputs, the parameter seed and the outputs (per-atom energies, forces) in fp64 and
fp32.  Only run in a container that holds the reference; the ``.npz`` files it
writes are the committed fixtures.

    python tests/golden/make_sparse_golden.py
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
from fsctep_amd.synthetic import make_system, seeded_value, SPECIES_4  # noqa: E402

CASES = {
    # 32 atoms, open 10 A box, C 32, 2 layers (the CPU-runnable plumbing configuration)
    "sparse_open32_c32_l2": dict(n=32, box=10.0, periodic=False, seed=11, channels=32, layers=2, pseed=101),
    # periodic, density 0.1 A^-3, C 64, 3 layers: the 1k/10k/100k recipe at 100 atoms
    "sparse_pbc100_c64_l3": dict(n=100, density=0.1, periodic=True, seed=22, channels=64, layers=3, pseed=202),
}


def build_reference(channels: int, layers: int, dtype):
    mod = refimport.load("molecular_force_field.models.pure_cartesian_sparse_layers")
    prev = torch.get_default_dtype()
    torch.set_default_dtype(dtype)
    try:
        model = mod.PureCartesianSparseTransformerLayer(
            max_embed_radius=5.0, main_max_radius=5.0, main_number_of_basis=8,
            hidden_dim_conv=channels, hidden_dim_sh=channels, hidden_dim=64, channel_in2=32,
            embedding_dim=16, max_atomvalue=10, output_size=8, invariant_channels=32,
            embed_size=[128, 128, 128], num_interaction=layers, function_type_main="bessel",
            lmax=2, max_rank_other=1, k_policy="k0", device=torch.device("cpu"),
        )
    finally:
        torch.set_default_dtype(prev)
    return model.to(dtype)


def apply_seeded(model, seed: int) -> None:
    with torch.no_grad():
        for name, p in model.named_parameters():
            p.copy_(torch.from_numpy(seeded_value(name, tuple(p.shape), seed)).to(p.dtype))


def run(model, sys_, dtype):
    pos = torch.tensor(sys_.pos, dtype=dtype, requires_grad=True)
    A = torch.tensor(sys_.species)
    batch = torch.zeros(sys_.num_atoms, dtype=torch.long)
    src = torch.tensor(sys_.edge_src)
    dst = torch.tensor(sys_.edge_dst)
    sh = torch.tensor(sys_.edge_shifts, dtype=dtype)
    cell = torch.tensor(sys_.cell, dtype=dtype)
    e = model(pos, A, batch, src, dst, sh, cell)
    (g,) = torch.autograd.grad(e.sum(), pos)
    return e.detach().squeeze(-1).numpy(), (-g).numpy()


def main():
    for name, c in CASES.items():
        if c["periodic"]:
            s = make_system(c["n"], density=c["density"], periodic=True, species=SPECIES_4, seed=c["seed"])
        else:
            s = make_system(c["n"], box=c["box"], periodic=False, species=SPECIES_4, seed=c["seed"])
        out = dict(pos=s.pos, species=s.species, cell=s.cell, periodic=np.asarray(s.periodic),
                   edge_src=s.edge_src, edge_dst=s.edge_dst, edge_shifts=s.edge_shifts,
                   channels=np.asarray(c["channels"]), layers=np.asarray(c["layers"]),
                   param_seed=np.asarray(c["pseed"]), function_type=np.asarray("bessel"))
        for dt, tag in ((torch.float64, "f64"), (torch.float32, "f32")):
            m = build_reference(c["channels"], c["layers"], dt)
            apply_seeded(m, c["pseed"])
            e, f = run(m, s, dt)
            out[f"energy_{tag}"] = e
            out[f"forces_{tag}"] = f
            print(name, tag, "E=", float(e.sum()), "max|e|=", float(np.abs(e).max()),
                  "max|F|=", float(np.abs(f).max()), "edges=", s.num_edges)
        np.savez_compressed(os.path.join(HERE, name + ".npz"), **out)
        keys = [[k, list(v.shape)] for k, v in m.state_dict().items()]
        with open(os.path.join(HERE, name + "_state_dict.json"), "w") as fh:
            json.dump(keys, fh, indent=0)


if __name__ == "__main__":
    main()
