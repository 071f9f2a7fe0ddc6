"""Write the fp64 oracle's energies, forces (and dipole) for the benchmark workloads at full size.

    python tests/golden/make_fullsize_oracle.py sparse 10000
    python tests/golden/make_fullsize_oracle.py ictd 10000
    python tests/golden/make_fullsize_oracle.py ictd-o3 4000
    python tests/golden/make_fullsize_oracle.py sparse 1000

The system, the seeded parameters and the field are bench.py's for that workload.  The oracle
(oracle/sparse_ref.py, oracle/ictd_ref.py: the reference algorithm restated, pinned by the reference
golden vectors) runs on the CPU in fp64 on the fp32-rounded inputs the GPU sees, with its edge sum
chunked (oracle.sparse_ref.edge_chunked) so that the per-edge weights fit in memory.  Results are stored
as float32 (6e-8 relative rounding, far below the 1e-5 parity budget) with a checksum of the system, in
tests/golden/oracle_<mode>_<atoms>.npz; tests/test_fullsize_parity_gpu.py and bench.py compare with them.
"""

from __future__ import annotations

import os
import sys
import time

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)


def fixture_path(mode: str, atoms: int) -> str:
    return os.path.join(HERE, f"oracle_{mode}_{atoms}.npz")


def main(mode: str, atoms: int, edge_chunk: int = 2048):
    # glibc's dynamic mmap threshold would serve the per-chunk temporaries from the heap, which then
    # fragments and grows without bound; a fixed threshold returns every large block on free
    import ctypes
    ctypes.CDLL("libc.so.6").mallopt(-3, 131072)   # M_MMAP_THRESHOLD
    import bench
    from fsctep_amd.synthetic import seeded_value
    w = bench.WORKLOADS[mode]
    seed = w["seed"]
    s = bench._system(mode, atoms, seed)
    f64 = torch.float64
    args = (torch.tensor(s.pos, dtype=torch.float32).to(f64), torch.tensor(s.species),
            torch.zeros(atoms, dtype=torch.long), torch.tensor(s.edge_src), torch.tensor(s.edge_dst),
            torch.tensor(s.edge_shifts, dtype=torch.float32).to(f64), torch.tensor(s.cell, dtype=torch.float32).to(f64))
    t0 = time.time()
    dip = None
    if mode == "sparse":
        from oracle import sparse_ref as R
        cfg = R.SparseConfig(channels=w["channels"], num_interaction=w["layers"], function_type="bessel")
        p = {k: torch.tensor(seeded_value(k, sh, 1), dtype=f64) for k, sh in R.param_shapes(cfg)}
        e, f = R.energy_forces(*args, p, cfg, edge_chunk=edge_chunk)
    else:
        from oracle import ictd_ref as R
        o3 = mode == "ictd-o3"
        cfg = R.ICTDConfig(channels=w["channels"], lmax=w["lmax"], num_interaction=w["layers"],
                           function_type="bessel", o3=o3,
                           active=((0, 1), (1, 1), (1, -1), (2, 1)) if o3 else (), external_field=o3, dipole=o3)
        p = {k: torch.tensor(seeded_value(k, sh, 1), dtype=f64) for k, sh in R.param_shapes(cfg)}
        field = torch.tensor(bench._field(1, seed), dtype=torch.float32).to(f64) if o3 else None
        e, f, dip = R.energy_forces(*args, p, cfg, field, edge_chunk=edge_chunk)
    dt = time.time() - t0
    out = dict(mode=mode, atoms=atoms, seed=seed, edges=s.num_edges, param_seed=1, system_sha256=bench.system_digest(s),
               energy=e.numpy().astype(np.float32), forces=f.numpy().astype(np.float32),
               energy_total=np.float64(e.sum()), oracle_seconds=np.float64(dt), edge_chunk=edge_chunk,
               threads=torch.get_num_threads())
    if dip is not None:
        out["dipole"] = dip.numpy().reshape(-1, 3)
    np.savez_compressed(fixture_path(mode, atoms), **out)
    print(f"{mode} {atoms} atoms, {s.num_edges} edges: oracle {dt:.0f} s, E_total {float(e.sum()):.9f}", flush=True)


if __name__ == "__main__":
    main(sys.argv[1], int(sys.argv[2]), int(sys.argv[3]) if len(sys.argv) > 3 else 2048)
