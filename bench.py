"""Energy + forces throughput of the equivariant message-passing hot path on one MI355X.

    python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--mode sparse|ictd|ictd-o3] [--atoms N]

Workloads (``--mode``): ``sparse`` (default) is pure-cartesian-sparse, 3 layers, 64 channels,
ranks 0..2, 10,000 atoms of 4 species; ``ictd`` is pure-cartesian-ictd, 3 layers, 128 channels,
ranks 0..3, 10,000 atoms of 8 species; ``ictd-o3`` is pure-cartesian-ictd-o3 (0e,1e,1o,2e plus a
rank-1 external field, dipole head), 3 layers, 64 channels, 4,000 atoms.  All are periodic cubic
boxes at 0.1 atoms/A^3, cutoff 5 A, 8 Bessel radial functions, min pair distance 0.9 A.

One step = energy and forces (F = -dE/dpos) of the whole system: edge geometry, radial
basis and MLP, conv1..conv3 message passing (HIP kernels), readout, and the backward of
all of it w.r.t. positions.  Inputs (positions, neighbour list, parameters) are resident
in HBM before timing starts; the receiver-sorted graph is prepared once (as between MD list
rebuilds) for the headline figure.  The line also carries the step through the reference-signature
``forward()``, which prepares the graph on every call as the reference sorts on every call, and the
cold and warm graph-preparation times.

The default run (sparse, 10k atoms) prints the headline at the top level and, under ``workloads``, the
ICTD 10k and ICTD-O3 4k workloads, the 100k-atom sparse domain (fp32 and the bf16 channel-mix
variant), and the two launch-bound sparse systems (1,000 atoms, and the 32-atom golden system), which
are timed eagerly and replayed from a HIP graph.  Each carries its roofline kernel, a table of the
TP/scatter kernels' rates (MFMA kernels priced against the peak of their own product arithmetic), the
parity of its energies, forces (and dipole) against the fp64 oracle's full-system values where a
fixture for that exact system exists (tests/golden/oracle_<mode>_<atoms>.npz) or the reference golden
vector, and the CPU baseline.  Prints one JSON line.
"""

from __future__ import annotations

import argparse
import hashlib
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
FP32_MFMA_PEAK_TFLOPS = 157.3
FP16_MFMA_PEAK_TFLOPS = 2500.0          # dense fp16 and bf16 MFMA
PARITY_TOL = 1e-5

# Peak rate of fp32-accurate products for each product arithmetic: a split-fp16 product is 3 fp16 MFMA
# products (hh + hl + lh), a split-bf16 product 6 bf16 ones; "bf16" is one bf16 product (the bf16
# channel-mix variant).  A kernel's mfma_frac is its useful flops over the peak of its own arithmetic.
PRODUCT_PEAK_TFLOPS = {"fp32": FP32_MFMA_PEAK_TFLOPS, "split-fp16": FP16_MFMA_PEAK_TFLOPS / 3,
                       "split-bf16": FP16_MFMA_PEAK_TFLOPS / 6, "bf16": FP16_MFMA_PEAK_TFLOPS}
KERNEL_PRODUCTS = {"node_expand": "split-fp16", "node_expand_grad": "split-fp16", "edge_message": "split-bf16",
                   "edge_message_grad": "split-fp16", "receiver_sum": "fp32",
                   "ictd_project": "split-fp16", "ictd_project_grad": "split-fp16", "ictd_dual_project": "split-fp16",
                   "ictd_mix": "split-fp16", "ictd_mix_grad": "split-fp16", "ictd_dual_mix": "split-fp16"}
BF16_VARIANT = {"node_expand", "node_expand_grad", "edge_message"}


def kernel_products(name: str, precision: str = "fp32") -> str:
    if precision == "bf16" and name in BF16_VARIANT:
        return "bf16"
    return KERNEL_PRODUCTS.get(name, "fp32")

WORKLOADS = {
    "sparse": dict(atoms=10000, species=4, seed=22, channels=64, layers=3, lmax=2, kernel="edge_message_grad",
                   cpu_atoms=300,
                   table=["node_expand", "edge_message", "receiver_sum", "edge_message_grad", "node_expand_grad"]),
    "ictd": dict(atoms=10000, species=8, seed=33, channels=128, layers=3, lmax=3, kernel="ictd_project_grad",
                 cpu_atoms=200,
                 table=["ictd_project", "ictd_mix", "ictd_mix_grad", "ictd_project_grad", "ictd_dual_project",
                        "ictd_dual_mix"]),
    "ictd-o3": dict(atoms=4000, species=4, seed=44, channels=64, layers=3, lmax=2, kernel="ictd_project_grad",
                    cpu_atoms=200,
                    table=["ictd_project", "ictd_mix", "ictd_mix_grad", "ictd_project_grad", "ictd_dual_project",
                        "ictd_dual_mix"]),
}

# Arithmetic of the products in each kernel family (every sum accumulates in fp32).  "split-fp16": each
# operand times a power of two is split into two fp16 parts and a product keeps hh + hl + lh on fp16 MFMA
# (22 significant bits; the dropped ll term is below 2^-22 |ab|).  "split-bf16": three bf16 parts per
# operand, six of the nine part products on bf16 MFMA (the dropped ones are below 2^-23 |ab|).
PRODUCTS = {
    "sparse": {"node_expand": "split-fp16", "node_expand_grad": "split-fp16", "edge_message": "split-bf16",
               "edge_message_grad": "split-fp16", "conv1 pair GEMMs": "split-fp16 (forward), fp32 MFMA (gradient)",
               "radial_mlp": "fp32 MFMA (first layer), split-fp16 (64-wide layers)",
               "receiver_sum, edge geometry, readout assembly": "fp32 VALU",
               "gram_forward, gram_backward": "split-fp16",
               "readout_mlp (MainNet + weighted sum)": "fp32 MFMA", "atom MLP (species table)": "torch fp32"},
    "ictd": {"ictd_project, ictd_dual_project": "split-fp16 (main product), fp32 MFMA (coupling rows)",
             "ictd_project_grad": "split-fp16 (H = g x^T), fp32 MFMA (coupling rows, dY)",
             "ictd_mix, ictd_mix_grad": "split-fp16",
             "ictd_conv1, source_sum, edge geometry, harmonics, readout assembly": "fp32 VALU",
             "radial_mlp (gates)": "fp32 MFMA (first layer), split-fp16 (64-wide layers)",
             "gram_forward, gram_backward": "split-fp16",
             "readout_mlp (MainNet + weighted sum)": "fp32 MFMA", "atom MLP (species table)": "torch fp32"},
}
PRODUCTS["ictd-o3"] = PRODUCTS["ictd"]


# Per-kernel algorithmic work of one launch (one conv2..n layer with N nodes, E edges, C channels).
# flops: useful multiply-adds x2; bytes: compulsory fp32 traffic at the kernel's boundary (each
# array once, node gathers counted once per node).
def sparse_kernel_work(name: str, N: int, E: int, C: int) -> dict:
    K = 64
    s_bytes = 4 * N * 18 * 65 * C            # node expansion S (or dS)
    p_bytes = 4 * E * 18 * C                 # edge messages P
    if name == "edge_message_grad":
        # dh and dS products (split-fp16: their MFMA time is a fraction of the kernel's, which is set by
        # reading S and writing dS); the fused direction gradient reads P slots 1, 2, 6, 7, 8 and writes dn
        flops = 2 * (2 * E * 18 * C * K) + E * 18 * C + 2 * E * 30 * C
        byts = (s_bytes + s_bytes + 4 * E * K * 2 + 4 * N * 13 * C + 4 * E * 3 * 2 + 4 * E * 5 * C
                + 4 * E * 2)
        return dict(flops=flops, bytes=byts, bound="hbm")
    if name == "edge_message":
        flops = 2 * E * 18 * C * K
        byts = s_bytes + p_bytes + 4 * E * K + 4 * E
        return dict(flops=flops, bytes=byts, bound="hbm")
    if name == "node_expand":
        flops = 2 * N * 18 * 65 * C * C
        byts = s_bytes + 4 * N * 13 * C
        return dict(flops=flops, bytes=byts, bound="mfma")
    if name == "node_expand_grad":
        flops = 2 * N * 18 * 65 * C * C
        byts = s_bytes + 4 * 2 * 18 * N * C
        return dict(flops=flops, bytes=byts, bound="mfma")
    if name == "receiver_sum":
        return dict(flops=2 * E * 34 * C, bytes=p_bytes + 12 * E + 4 * N * 13 * C, bound="hbm")
    raise KeyError(name)


def ictd_kernel_work(name: str, L, N: int, E: int, C: int) -> dict:
    """``L`` is the layout table of the model (components M, coupled rows KT, paths, groups)."""
    M, KT, NY, NREF = L.M, L.KT, L.NY, L.NREF
    # useful (m1, kk) pairs per edge: input component m1 of group g couples to that group's rows
    pairs = sum(L.g_d1[g] * L.g_kcount[g] for g in range(L.NG))
    edge_in = 4 * E * (1 + NY + NREF)        # source index, harmonics, gates
    x_b, z_b = 4 * N * M * C, 4 * N * KT * C
    # The projections do 2 * pairs * C flop per edge on ~(M + KT) * C * 4 bytes per node: 50-100 flop per
    # algorithmic byte at 52 neighbours, above the fp32 MFMA ridge (157.3 TFLOP/s / 8 TB/s = 19.7), so their
    # roofline is the fp32 MFMA rate.
    if name == "ictd_project":
        return dict(flops=2 * E * pairs * C, bytes=x_b + z_b + edge_in + 4 * N, bound="mfma")
    if name == "ictd_project_grad":
        # H = x_src g^T per edge (the gate / harmonic gradients); writes dgates and dY
        return dict(flops=2 * E * pairs * C, bytes=z_b + x_b + edge_in + 4 * E * (NREF + NY), bound="mfma")
    if name == "ictd_dual_project":
        # R = projection of the receiver gradients over the source grouping (the reversed paths: KT' = KT
        # slots, the same pairs); reads G once per node, writes R
        return dict(flops=2 * E * pairs * C, bytes=x_b + z_b + edge_in + 4 * E + 4 * N, bound="mfma")
    if name in ("ictd_mix", "ictd_mix_grad", "ictd_dual_mix"):
        return dict(flops=2 * N * KT * C * C, bytes=z_b + x_b + 4 * L.NP * C * C, bound="mfma")
    raise KeyError(name)


def gpu_info():
    import torch
    p = torch.cuda.get_device_properties(0)
    return {"name": p.name, "arch": getattr(p, "gcnArchName", ""), "cus": p.multi_processor_count,
            "hbm_gib": round(p.total_memory / 2 ** 30, 1)}


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as fh:
            for ln in fh:
                if ln.startswith("model name"):
                    return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return ""


def host_cores() -> tuple[int, str]:
    """Cores available to this process: its affinity set, capped by a cgroup CPU quota if one is set."""
    aff = len(os.sched_getaffinity(0))
    quota = None
    try:
        with open("/sys/fs/cgroup/cpu.max") as fh:
            q, period = fh.read().split()[:2]
            if q != "max":
                quota = max(1, int(int(q) / int(period)))
    except (OSError, ValueError):
        pass
    cores = aff if quota is None else min(aff, quota)
    return cores, f"affinity {aff}" + ("" if quota is None else f", cgroup quota {quota}")


def _system(mode: str, n_atoms: int, seed: int):
    from fsctep_amd.synthetic import SPECIES_4, SPECIES_8, make_system
    w = WORKLOADS[mode]
    return make_system(n_atoms, density=0.1, periodic=True, species=SPECIES_8 if w["species"] == 8 else SPECIES_4,
                       seed=seed)


def _field(n_graphs: int, seed: int):
    """External field per graph, N(0, 0.1) V/A, seeded."""
    import numpy as np
    return np.random.Generator(np.random.PCG64(seed)).normal(0.0, 0.1, size=(n_graphs, 3))


def system_digest(s) -> str:
    """sha256 of the fp32/int64 arrays that define a system (the key of a full-size oracle fixture)."""
    import numpy as np
    h = hashlib.sha256()
    for a in (s.pos.astype(np.float32), s.species.astype(np.int64), s.edge_src.astype(np.int64),
              s.edge_dst.astype(np.int64), s.edge_shifts.astype(np.float32), s.cell.astype(np.float32)):
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def cpu_baseline(mode: str, n_atoms: int, steps: int, seed: int) -> dict:
    """The oracle (the reference's algorithm restated in PyTorch on the CPU) on the host cores."""
    import torch
    from fsctep_amd.synthetic import seeded_value
    w = WORKLOADS[mode]
    cores, cdesc = host_cores()
    torch.set_num_threads(cores)
    s = _system(mode, n_atoms, seed)
    args = (torch.tensor(s.pos, dtype=torch.float32), torch.tensor(s.species),
            torch.zeros(n_atoms, dtype=torch.long), torch.tensor(s.edge_src), torch.tensor(s.edge_dst),
            torch.tensor(s.edge_shifts, dtype=torch.float32), torch.tensor(s.cell, dtype=torch.float32))
    if mode == "sparse":
        from oracle import sparse_ref as R
        cfg = R.SparseConfig(channels=w["channels"], num_interaction=w["layers"], function_type="bessel")
        run = lambda p: R.energy_forces(*args, p, cfg)
        what = "materialised per-edge weights, per-path einsums, index_add"
    else:
        from oracle import ictd_ref as R
        o3 = mode == "ictd-o3"
        cfg = R.ICTDConfig(channels=w["channels"], lmax=w["lmax"], num_interaction=w["layers"],
                           function_type="bessel", o3=o3,
                           active=((0, 1), (1, 1), (1, -1), (2, 1)) if o3 else (), external_field=o3, dipole=o3)
        field = torch.tensor(_field(1, seed), dtype=torch.float32) if o3 else None
        run = lambda p: R.energy_forces(*args, p, cfg, field)
        what = "per-path CG contractions with materialised per-edge weights, index_add"
    p = {k: torch.tensor(seeded_value(k, sh, 1), dtype=torch.float32) for k, sh in R.param_shapes(cfg)}
    run(p)
    dts = []
    for _ in range(steps):
        t0 = time.perf_counter()
        run(p)
        dts.append(time.perf_counter() - t0)
    dt = statistics.median(dts)
    return {"value": round(n_atoms / dt, 3), "unit": "atom-steps/s", "cores": cores, "kind": "port",
            "sample": f"oracle ({what}), fp32, {n_atoms} atoms / {s.num_edges} edges of the same recipe, "
                      f"median of {steps} timed steps after 1 warm-up, {dt:.2f} s/step, {cores} threads "
                      f"({cdesc}) on {_cpu_model()}"}


def build_model(mode: str, dev):
    """Random-init (seeded) model of the workload, inference mode, on ``dev``."""
    from fsctep_amd.synthetic import apply_seeded_parameters
    w = WORKLOADS[mode]
    C = w["channels"]
    kw = dict(max_embed_radius=5.0, main_max_radius=5.0, main_number_of_basis=8, hidden_dim_conv=C,
              hidden_dim_sh=C, hidden_dim=64, channel_in2=32, embedding_dim=16, max_atomvalue=10,
              output_size=8, invariant_channels=32, embed_size=[128, 128, 128], num_interaction=w["layers"],
              function_type_main="bessel", lmax=w["lmax"])
    if mode == "sparse":
        from fsctep_amd.sparse import PureCartesianSparseTransformerLayer
        model = PureCartesianSparseTransformerLayer(**kw, max_rank_other=1, k_policy="k0")
    elif mode == "ictd":
        from fsctep_amd.ictd import PureCartesianICTDTransformerLayer
        model = PureCartesianICTDTransformerLayer(**kw, ictd_tp_path_policy="full")
    else:
        from fsctep_amd.ictd import PureCartesianICTDO3TransformerLayer
        model = PureCartesianICTDO3TransformerLayer(
            **kw, ictd_tp_path_policy="full", o3_active_irreps="0e,1e,1o,2e", external_tensor_rank=1,
            external_tensor_irrep="1o",
            physical_tensor_outputs={"dipole": {"irreps": ["1o"], "channels_out": 1, "reduce": "sum"}})
    apply_seeded_parameters(model, 1)
    return model.to(dev).eval().requires_grad_(False)


def workload_name(mode: str, N: int, E: int) -> str:
    w = WORKLOADS[mode]
    head = {"sparse": "pure-cartesian-sparse energy+forces",
            "ictd": "pure-cartesian-ictd energy+forces",
            "ictd-o3": "pure-cartesian-ictd-o3 (0e,1e,1o,2e + rank-1 external field) energy+forces+dipole"}[mode]
    return (f"{head}, {N} atoms, {E} edges, periodic cubic box, density 0.1/A^3, {w['species']} species, "
            f"{w['layers']} interaction layers, {w['channels']} channels, ranks 0..{w['lmax']}, "
            f"cutoff 5.0 A, 8 Bessel radial basis")


def _rel_inf(a, b) -> float:
    import numpy as np
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def parity_vs_fixture(mode: str, system, seed: int, e, f, dip) -> dict:
    """Max-norm relative errors of the step's outputs against the fp64 oracle's full-system values."""
    import numpy as np
    N = system.num_atoms
    path = os.path.join(ROOT, "tests", "golden", f"oracle_{mode}_{N}.npz")
    rel = os.path.relpath(path, ROOT)
    if not os.path.exists(path):
        return {"fixture": None, "note": f"no fp64 oracle fixture for this system ({rel})"}
    fx = np.load(path, allow_pickle=False)
    if str(fx["system_sha256"]) != system_digest(system) or int(fx["seed"]) != seed:
        return {"fixture": rel, "note": "fixture is for another system (digest mismatch): not compared"}
    out = {"fixture": rel, "reference": "fp64 oracle on the whole system", "tolerance": PARITY_TOL,
           "energy_rel": _rel_inf(e, fx["energy"]), "forces_rel": _rel_inf(f, fx["forces"]),
           "energy_total_rel": abs(float(np.sum(np.asarray(e, np.float64))) - float(fx["energy_total"]))
           / max(abs(float(fx["energy_total"])), 1e-30)}
    if dip is not None and "dipole" in fx:
        out["dipole_rel"] = _rel_inf(np.asarray(dip).reshape(-1, 3), fx["dipole"])
    out["within_tolerance"] = all(v < PARITY_TOL for k, v in out.items() if k.endswith("_rel"))
    for k in list(out):
        if k.endswith("_rel"):
            out[k] = float(f"{out[k]:.3e}")
    return out


def _rate(work: dict, avg_ms: float, products: str = "fp32") -> dict:
    """Achieved rate of one launch against its algorithmic bytes (HBM) and, for MFMA kernels, flops
    against the peak of the kernel's own product arithmetic (PRODUCT_PEAK_TFLOPS)."""
    gbs = work["bytes"] / (avg_ms * 1e-3) / 1e9
    r = {"avg_launch_ms": round(avg_ms, 4), "hbm_gbs": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
         "bound": work["bound"]}
    if work["bound"] == "mfma":
        tf = work["flops"] / (avg_ms * 1e-3) / 1e12
        peak = PRODUCT_PEAK_TFLOPS[products]
        r.update(tflops=round(tf, 2), products=products, mfma_peak_tflops=round(peak, 1),
                 mfma_frac=round(tf / peak, 4))
        if tf > peak:   # a useful-flop count above the arithmetic's peak means the accounting is wrong
            print(f"[bench] WARNING: {tf:.1f} TFLOP/s above the {products} peak {peak:.1f}", file=sys.stderr)
    return r


def measure(mode: str, n_atoms: int, seed: int, steps: int, warmup: int, kname: str, dev,
            table: bool = True, precision: str = "fp32", keep: bool = False, extras: bool = True,
            system=None) -> dict:
    import numpy as np
    import torch
    from fsctep_amd import _lib
    w = WORKLOADS[mode]
    t_build = time.perf_counter()
    system = _system(mode, n_atoms, seed) if system is None else system
    print(f"[bench] {mode}: {system.num_atoms} atoms, {system.num_edges} edges "
          f"({time.perf_counter() - t_build:.1f} s to build)", file=sys.stderr, flush=True)
    model = build_model(mode, dev)
    if precision != "fp32":
        model.channel_mix_precision = precision
    C = w["channels"]
    N, E = system.num_atoms, system.num_edges

    pos = torch.tensor(system.pos, dtype=torch.float32, device=dev)
    A = torch.tensor(system.species, device=dev)
    batch = torch.zeros(N, dtype=torch.long, device=dev)
    cell = torch.tensor(system.cell, dtype=torch.float32, device=dev)
    src = torch.tensor(system.edge_src, device=dev)
    dst = torch.tensor(system.edge_dst, device=dev)
    shifts = torch.tensor(system.edge_shifts, dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    t_g = time.perf_counter()
    graph = model.prepare(src, dst, shifts, N, A, pos=pos)
    torch.cuda.synchronize()
    t_cold = time.perf_counter() - t_g
    warm = []
    for _ in range(5):
        t_g = time.perf_counter()
        model.prepare(src, dst, shifts, N, A, pos=pos)
        torch.cuda.synchronize()
        warm.append(time.perf_counter() - t_g)

    field = torch.tensor(_field(1, seed), dtype=torch.float32, device=dev) if mode == "ictd-o3" else None
    if mode == "sparse":
        from fsctep_amd.sparse import energy_and_forces

        def step():
            e, f = energy_and_forces(model, pos, batch, cell, graph)
            return e, f, None
    else:
        from fsctep_amd.ictd import energy_forces

        def step():
            return energy_forces(model, pos, batch, cell, graph, external_tensor=field)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    print(f"[bench] {mode}: warm-up done ({warmup} steps)", file=sys.stderr, flush=True)

    # timed region: exactly `steps` steps, synchronised on both sides
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    with _lib.KernelTimer(kname) as kt:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ev[0].record()
        for i in range(steps):
            res = step()
            ev[i + 1].record()
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
    e, f, dip = res
    step_ms = [ev[i].elapsed_time(ev[i + 1]) for i in range(steps)]
    ms_per_step = elapsed * 1000.0 / steps
    assert torch.isfinite(e).all() and torch.isfinite(f).all()
    print(f"[bench] {mode}: timed {steps} steps: {ms_per_step:.3f} ms/step (median {statistics.median(step_ms):.3f}); "
          f"E={float(e.sum()):.6f} max|F|={float(f.abs().max()):.4f}", file=sys.stderr, flush=True)

    if mode == "sparse":
        work_of = lambda k: sparse_kernel_work(k, N, E, C)
    else:
        from fsctep_amd import ictd_ops
        lay = ictd_ops.layout_struct(model.layout_id)
        work_of = lambda k: ictd_kernel_work(k, lay, N, E, C)
    work = work_of(kname)
    avg_ms = kt.total_ms / max(kt.launches, 1)
    if work["bound"] == "mfma":
        achieved = work["flops"] / (avg_ms * 1e-3) / 1e12
        peak = PRODUCT_PEAK_TFLOPS[kernel_products(kname, precision)]
        roof = {"bound": "mfma", "achieved": round(achieved, 3), "peak": round(peak, 1), "unit": "TFLOP/s",
                "frac": round(achieved / peak, 4), "products": kernel_products(kname, precision)}
    else:
        achieved = work["bytes"] / (avg_ms * 1e-3) / 1e9
        roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4)}
    roof["traffic"] = None
    tfile = os.path.join(ROOT, "profiles", f"traffic_{kname}_{mode}{N}.json")
    if os.path.exists(tfile):
        with open(tfile) as fh:
            tinfo = json.load(fh)
        srcf = os.path.join(ROOT, tinfo.get("source", ""))
        if os.path.isfile(srcf) and hashlib.sha256(open(srcf, "rb").read()).hexdigest() == tinfo.get("source_sha256"):
            roof["traffic"] = tinfo.get("hbm_bytes_per_launch")   # measured for this exact kernel source
    roof["kernel"] = kname
    roof["avg_launch_ms"] = round(avg_ms, 4)
    roof["launches"] = kt.launches
    roof["algorithmic_per_launch"] = {"flops": work["flops"], "bytes": work["bytes"]}

    out = {"ms_per_step": round(ms_per_step, 4), "median_ms_per_step": round(statistics.median(step_ms), 4),
           "value": round(N / (ms_per_step * 1e-3), 1), "atoms": N, "edges": E, "roofline": roof}

    # per-kernel rates of the TP / scatter kernels (a separate pass per kernel, outside the timed region)
    if table:
        kt_steps = max(3, min(steps, 10))
        rates = {}
        for k in w["table"]:
            with _lib.KernelTimer(k) as t:
                for _ in range(kt_steps):
                    step()
                torch.cuda.synchronize()
            if t.launches:
                rates[k] = dict(_rate(work_of(k), t.total_ms / t.launches, kernel_products(k, precision)),
                                launches_per_step=t.launches // kt_steps)
        out["kernels"] = rates

    if keep:
        out["_ef"] = (e.double().cpu().numpy(), f.double().cpu().numpy())
    out["products"] = PRODUCTS[mode] if precision == "fp32" else {
        "node_expand, node_expand_grad, edge_message": "bf16 MFMA, one product, fp32 accumulation",
        "everything else": "as in the fp32 configuration"}
    out["config"] = {"workload": workload_name(mode, N, E), "mode": mode, "atoms": N, "edges": E,
                     "channel_mix_precision": precision}
    if not extras:
        return out

    # the reference-signature forward: the graph is prepared inside every call
    kw = {"external_tensor": field} if field is not None else {}

    def ref_step():
        p = pos.detach().requires_grad_(True)
        en = model(p, A, batch, src, dst, shifts, cell, **kw)
        (g,) = torch.autograd.grad(en.sum(), p)
        return en, g

    for _ in range(2):
        ref_step()
    torch.cuda.synchronize()
    rs = max(3, steps // 2)
    t0 = time.perf_counter()
    for _ in range(rs):
        ref_step()
    torch.cuda.synchronize()
    out["ms_per_step_with_graph_prepare"] = round((time.perf_counter() - t0) * 1000 / rs, 4)
    out["graph_prepare_ms"] = {"cold": round(t_cold * 1000, 3), "warm_median": round(statistics.median(warm) * 1000, 3)}

    # neighbour-list rebuild on the GPU (cell list, periodic images): the same edges as the host list
    from fsctep_amd.neighbors import radius_graph_pbc_gpu
    pos64 = torch.tensor(system.pos, dtype=torch.float64, device=dev)
    cell64 = torch.tensor(system.cell, dtype=torch.float64, device=dev)
    nl = radius_graph_pbc_gpu(pos64, 5.0, cell64)
    same = bool(nl[0].shape[0] == E and torch.equal(nl[0].cpu(), src.cpu()) and torch.equal(nl[1].cpu(), dst.cpu()))
    nl_t = []
    for _ in range(5):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        radius_graph_pbc_gpu(pos64, 5.0, cell64)
        torch.cuda.synchronize()
        nl_t.append(time.perf_counter() - t0)
    out["neighbor_list_ms"] = {"median": round(statistics.median(nl_t) * 1000, 3), "equals_host_list": same}

    out["parity"] = parity_vs_fixture(mode, system, seed, e.cpu().numpy(), f.cpu().numpy(),
                                      None if dip is None else dip.cpu().numpy())
    return out


# The two smaller sparse configurations: the 32-atom CPU-runnable plumbing system (the reference-written
# golden system itself: 32 atoms of 4 species in a 10 A open box, C 32, 2 layers) and the 1,000-atom
# periodic box (C 64, 3 layers).  Both are launch-bound, so each is timed eagerly and replayed from a
# HIP graph (fsctep_amd.capture); `value` is the replayed rate.
SMALL = {
    "sparse-1k": dict(atoms=1000, seed=22, channels=64, layers=3, kernel="edge_message_grad"),
    "sparse-32": dict(golden="sparse_open32_c32_l2", channels=32, layers=2, kernel="edge_message_grad"),
}


def _small_model(name: str, dev):
    from fsctep_amd.sparse import PureCartesianSparseTransformerLayer
    from fsctep_amd.synthetic import apply_seeded_parameters
    w = SMALL[name]
    seed = 1
    if "golden" in w:
        import numpy as np
        seed = int(np.load(os.path.join(ROOT, "tests", "golden", w["golden"] + ".npz"))["param_seed"])
    C = w["channels"]
    model = PureCartesianSparseTransformerLayer(
        max_embed_radius=5.0, main_max_radius=5.0, main_number_of_basis=8, hidden_dim_conv=C, hidden_dim_sh=C,
        hidden_dim=64, channel_in2=32, embedding_dim=16, max_atomvalue=10, output_size=8, invariant_channels=32,
        embed_size=[128, 128, 128], num_interaction=w["layers"], function_type_main="bessel", lmax=2,
        max_rank_other=1, k_policy="k0")
    apply_seeded_parameters(model, seed)
    return model.to(dev).eval().requires_grad_(False), seed


def _small_system(name: str):
    from fsctep_amd.synthetic import AtomicSystem
    w = SMALL[name]
    if "golden" in w:
        import numpy as np
        g = np.load(os.path.join(ROOT, "tests", "golden", w["golden"] + ".npz"), allow_pickle=False)
        return AtomicSystem(pos=g["pos"], species=g["species"], cell=g["cell"], periodic=bool(g["periodic"]),
                            edge_src=g["edge_src"], edge_dst=g["edge_dst"], edge_shifts=g["edge_shifts"]), g
    return _system("sparse", w["atoms"], w["seed"]), None


def measure_small(name: str, steps: int, warmup: int, dev) -> dict:
    """Eager and HIP-graph-replayed energy + forces of a small sparse system; parity of both against the
    reference golden (32 atoms) or the fp64 oracle fixture (1,000 atoms)."""
    import numpy as np
    import torch
    from fsctep_amd import _lib
    from fsctep_amd.capture import CapturedEnergyForces
    from fsctep_amd.sparse import energy_and_forces
    w = SMALL[name]
    system, golden = _small_system(name)
    model, pseed = _small_model(name, dev)
    N, E, C = system.num_atoms, system.num_edges, w["channels"]
    pos = torch.tensor(system.pos, dtype=torch.float32, device=dev)
    A = torch.tensor(system.species, device=dev)
    batch = torch.zeros(N, dtype=torch.long, device=dev)
    cell = torch.tensor(system.cell, dtype=torch.float32, device=dev)
    graph = model.prepare(torch.tensor(system.edge_src, device=dev), torch.tensor(system.edge_dst, device=dev),
                          torch.tensor(system.edge_shifts, dtype=torch.float32, device=dev), N, A, pos=pos)
    step = lambda: energy_and_forces(model, pos, batch, cell, graph)
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()

    def timed(fn, k):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(k):
            res = fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1000.0 / k, res

    with _lib.KernelTimer(w["kernel"]) as kt:
        eager_ms, (e_eager, f_eager) = timed(step, steps)
    cap = CapturedEnergyForces(model, pos, batch, cell, graph, warmup=2)
    for _ in range(warmup):
        cap()
    graph_ms, (e_cap, f_cap, _) = timed(cap, steps)
    same = bool(torch.equal(e_cap, e_eager) and torch.equal(f_cap, f_eager))
    print(f"[bench] {name}: {N} atoms, {E} edges: eager {eager_ms:.3f} ms/step, HIP graph {graph_ms:.3f} ms/step, "
          f"replay equals eager bitwise: {same}", file=sys.stderr, flush=True)

    work = sparse_kernel_work(w["kernel"], N, E, C)
    avg_ms = kt.total_ms / max(kt.launches, 1)
    if work["bound"] == "mfma":
        peak = PRODUCT_PEAK_TFLOPS[kernel_products(w["kernel"])]
        achieved = work["flops"] / (avg_ms * 1e-3) / 1e12
        roof = {"bound": "mfma", "achieved": round(achieved, 3), "peak": round(peak, 1), "unit": "TFLOP/s",
                "frac": round(achieved / peak, 4), "products": kernel_products(w["kernel"])}
    else:
        achieved = work["bytes"] / (avg_ms * 1e-3) / 1e9
        roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4)}
    launch_bound = graph_ms < 0.8 * eager_ms
    roof.update({"traffic": None, "kernel": w["kernel"], "avg_launch_ms": round(avg_ms, 4), "launches": kt.launches,
                 "algorithmic_per_launch": {"flops": work["flops"], "bytes": work["bytes"]},
                 "note": (f"HIP-graph replay {graph_ms:.3f} ms/step against {eager_ms:.3f} eager: "
                          + ("launch-bound at this size (the kernel is tens of microseconds)" if launch_bound else
                             "kernel-bound at this size (launches cost little)"))})
    e_np, f_np = e_cap.double().cpu().numpy(), f_cap.double().cpu().numpy()
    if golden is not None:
        parity = {"fixture": f"tests/golden/{w['golden']}.npz", "reference": "the reference trunk in fp64 "
                  "(golden vector written by the imported reference)", "tolerance": PARITY_TOL,
                  "energy_rel": float(f"{_rel_inf(e_np, golden['energy_f64']):.3e}"),
                  "forces_rel": float(f"{_rel_inf(f_np, golden['forces_f64']):.3e}")}
        parity["within_tolerance"] = parity["energy_rel"] < PARITY_TOL and parity["forces_rel"] < PARITY_TOL
    else:
        parity = parity_vs_fixture("sparse", system, w["seed"], e_np, f_np, None)
    return {"ms_per_step": round(graph_ms, 4), "value": round(N / (graph_ms * 1e-3), 1),
            "ms_per_step_eager": round(eager_ms, 4), "value_eager": round(N / (eager_ms * 1e-3), 1),
            "replay_equals_eager_bitwise": same, "roofline": roof, "parity": parity,
            "config": {"workload": f"pure-cartesian-sparse energy+forces, {N} atoms, {E} edges, "
                       + ("10 A open box (the reference golden system)" if golden is not None else
                          "periodic cubic box, density 0.1/A^3") + f", 4 species, {w['layers']} interaction layers, "
                       f"{C} channels, ranks 0..2, cutoff 5.0 A, 8 Bessel radial basis, parameters seed {pseed}; "
                       "step replayed from a HIP graph", "mode": "sparse", "atoms": N, "edges": E}}


def cpu_baseline_small(name: str, steps: int) -> dict:
    """The oracle on the host cores on the small system itself (the whole system, not a sample)."""
    import torch
    from fsctep_amd.synthetic import seeded_value
    from oracle import sparse_ref as R
    w = SMALL[name]
    cores, cdesc = host_cores()
    torch.set_num_threads(cores)
    s, _ = _small_system(name)
    _, pseed = _small_model(name, "cpu")
    n = s.num_atoms
    args = (torch.tensor(s.pos, dtype=torch.float32), torch.tensor(s.species), torch.zeros(n, dtype=torch.long),
            torch.tensor(s.edge_src), torch.tensor(s.edge_dst), torch.tensor(s.edge_shifts, dtype=torch.float32),
            torch.tensor(s.cell, dtype=torch.float32))
    cfg = R.SparseConfig(channels=w["channels"], num_interaction=w["layers"], function_type="bessel")
    p = {k: torch.tensor(seeded_value(k, sh, pseed), dtype=torch.float32) for k, sh in R.param_shapes(cfg)}
    R.energy_forces(*args, p, cfg)
    dts = []
    for _ in range(steps):
        t0 = time.perf_counter()
        R.energy_forces(*args, p, cfg)
        dts.append(time.perf_counter() - t0)
    dt = statistics.median(dts)
    return {"value": round(n / dt, 3), "unit": "atom-steps/s", "cores": cores, "kind": "port",
            "sample": f"oracle (materialised per-edge weights, per-path einsums, index_add), fp32, the whole "
                      f"{n}-atom / {s.num_edges}-edge system, median of {steps} timed steps after 1 warm-up, "
                      f"{dt:.3f} s/step, {cores} threads ({cdesc}) on {_cpu_model()}"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--mode", choices=sorted(WORKLOADS), default="sparse")
    ap.add_argument("--atoms", type=int, default=None)
    ap.add_argument("--seed", type=int, default=None)
    ap.add_argument("--roofline-kernel", default=None)
    ap.add_argument("--cpu-atoms", type=int, default=None)
    ap.add_argument("--cpu-steps", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true",
                    help="only the selected workload (by default the sparse headline also runs ICTD 10k and ICTD-O3 4k)")
    ap.add_argument("--no-kernel-table", action="store_true")
    ap.add_argument("--no-large", action="store_true",
                    help="skip the 100k-atom sparse workload (fp32 and the bf16 channel-mix variant)")
    ap.add_argument("--no-small", action="store_true",
                    help="skip the 32-atom and 1,000-atom sparse workloads (eager and HIP-graph replay)")
    ap.add_argument("--channel-mix", choices=["fp32", "bf16"], default="fp32",
                    help="products of the sparse channel mix for --mode sparse runs")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="after timing, copy a 1 GiB fp32 buffer 3 times (reference kernel for HBM counters)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the message passing would shard by receiver domain; not built here)", file=sys.stderr)
        sys.exit(2)
    w = WORKLOADS[args.mode]
    n_atoms = w["atoms"] if args.atoms is None else args.atoms
    seed = w["seed"] if args.seed is None else args.seed
    kname = w["kernel"] if args.roofline_kernel is None else args.roofline_kernel

    import torch
    dev = torch.device("cuda:0")
    head = measure(args.mode, n_atoms, seed, args.steps, args.warmup, kname, dev, table=not args.no_kernel_table,
                   precision=args.channel_mix if args.mode == "sparse" else "fp32")
    N, E = head["atoms"], head["edges"]
    out = {
        "metric": "atom-steps/sec (energy+forces) at 10k atoms; TP kernel HBM GB/s vs peak",
        "value": head["value"],
        "unit": "atom-steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "median_ms_per_step": head["median_ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "products": head["products"],
        "data": "synthetic (seeded random sequential addition, random-init seeded parameters)",
        "config": head["config"],
        "roofline": head["roofline"],
        "kernels": head.get("kernels"),
        "ms_per_step_with_graph_prepare": head["ms_per_step_with_graph_prepare"],
        "graph_prepare_ms": head["graph_prepare_ms"],
        "neighbor_list_ms": head["neighbor_list_ms"],
        "parity": head["parity"],
        "gpu": gpu_info(),
    }
    if args.copy_calibration:
        src_buf = torch.ones(256 * 2 ** 20, dtype=torch.float32, device=dev)
        dst_buf = torch.empty_like(src_buf)
        for _ in range(3):
            dst_buf.copy_(src_buf)
        torch.cuda.synchronize()
        del src_buf, dst_buf

    extra = []
    if not args.no_extra and args.mode == "sparse" and args.atoms is None:
        extra = ["ictd", "ictd-o3"]
    workloads = {}
    for m in extra:
        wm = WORKLOADS[m]
        r = measure(m, wm["atoms"], wm["seed"], args.steps, args.warmup, wm["kernel"], dev,
                    table=not args.no_kernel_table)
        r.pop("atoms")
        r.pop("edges")
        workloads[m] = r
    if extra and not args.no_large:
        # 100k-atom sparse domain: fp32-accurate products and the bf16 channel-mix variant, and the
        # variant's error against the fp32 path on the same system
        big = {}
        sys100k = _system("sparse", 100000, WORKLOADS["sparse"]["seed"])
        for prec in ("fp32", "bf16"):
            r = measure("sparse", 100000, WORKLOADS["sparse"]["seed"], max(3, args.steps // 2), 2, "edge_message_grad",
                        dev, table=False, precision=prec, keep=True, extras=False, system=sys100k)
            big[prec] = r
        (e32, f32), (e16, f16) = big["fp32"].pop("_ef"), big["bf16"].pop("_ef")
        big["bf16_vs_fp32"] = {"energy_rel": float(f"{_rel_inf(e16, e32):.3e}"),
                               "forces_rel": float(f"{_rel_inf(f16, f32):.3e}"),
                               "energy_total_rel": float(f"{abs(e16.sum() - e32.sum()) / abs(e32.sum()):.3e}"),
                               "speedup": round(big["fp32"]["ms_per_step"] / big["bf16"]["ms_per_step"], 3)}
        workloads["sparse-100k"] = big
    if extra and not args.no_small:
        for name in ("sparse-1k", "sparse-32"):
            workloads[name] = measure_small(name, max(args.steps, 50), args.warmup, dev)
    if workloads:
        out["workloads"] = workloads

    if not args.no_cpu_baseline:
        print("[bench] cpu baseline ...", file=sys.stderr, flush=True)
        cpu_atoms = w["cpu_atoms"] if args.cpu_atoms is None else args.cpu_atoms
        out["cpu_baseline"] = cpu_baseline(args.mode, cpu_atoms, args.cpu_steps, seed)
        out["cpu_baseline"]["gpu_over_cpu"] = round(out["value"] / out["cpu_baseline"]["value"], 1)
        for m, r in workloads.items():
            if m in SMALL:
                # the whole system: 32 atoms take ~0.04 s a step, 1,000 atoms ~15 s on 16 cores
                r["cpu_baseline"] = cpu_baseline_small(m, 10 if m == "sparse-32" else 1)
                r["cpu_baseline"]["gpu_over_cpu"] = round(r["value"] / r["cpu_baseline"]["value"], 1)
                continue
            if m not in WORKLOADS:        # the 100k-atom sparse domain: same per-atom oracle as the headline
                continue
            wm = WORKLOADS[m]
            r["cpu_baseline"] = cpu_baseline(m, wm["cpu_atoms"], args.cpu_steps, wm["seed"])
            r["cpu_baseline"]["gpu_over_cpu"] = round(r["value"] / r["cpu_baseline"]["value"], 1)
    else:
        out["cpu_baseline"] = None
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
