"""Time the reference extension's seam (``molecular_force_field._C_ictd_tp``, served by
``fsctep_amd.ictd_tp_ext``) on the per-edge conv2 of the ICTD trunk, driven the way the reference's
HarmonicFullyConnectedTensorProduct drives it (models/ictd_irreps.py:1035-1133): for each bucket of paths
with the same input keys (k1, k2) and output dimension, ``project_bucket_forward`` then
``mix_bucket_forward``, summed into the output key; backward, per bucket, ``mix_bucket_transpose_y/_w/_g``
and ``project_bucket_transpose_a/_b``.

    python -m fsctep_amd.seam_bench [--edges E] [--channels C] [--lmax L] [--reps R]

Random operands of the ICTD 10k shape by default (520,350 edges, C 128, lmax 3, the full path policy);
prints one JSON line with the forward and backward times per call (HIP events on the current stream, mean
over R calls after one warm-up) and the channel-mix flops of a forward.  The bucket table is built as the
reference builds it (models/ictd_irreps.py:97-120, 815-847, 886-915): paths grouped by (k1, k2) in sorted
order, each group's columns the coupling tensors reshaped (m1 m2, 2 l3 + 1) in path order, split into
buckets of equal output dimension, ascending.
"""

from __future__ import annotations

import argparse
import json

import torch

from . import ictd_tp_ext as X
from .ictd_basis import all_paths, canonical, coupling


def bucket_table(lmax: int, device):
    keys = [canonical(l) for l in range(lmax + 1)]
    paths = all_paths(keys, lmax)
    groups: dict = {}
    for p, (l1, p1, l2, p2, l3, p3) in enumerate(paths):
        groups.setdefault(((l1, p1), (l2, p2)), []).append((p, l3, p3))
    table = []
    for (k1, k2), items in sorted(groups.items()):
        by_kdim: dict = {}
        for p, l3, p3 in items:
            by_kdim.setdefault(2 * l3 + 1, []).append((p, l3, p3))
        for kdim, segs in sorted(by_kdim.items()):
            m1, m2 = 2 * k1[0] + 1, 2 * k2[0] + 1
            U = torch.cat([torch.from_numpy(coupling(k1[0], k2[0], l3)).reshape(m1 * m2, kdim)
                           for _, l3, _ in segs], dim=1)
            table.append((k1, k2, (segs[0][1], segs[0][2]), kdim, [p for p, _, _ in segs],
                          U.to(device=device, dtype=torch.float32)))
    return keys, paths, table


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--edges", type=int, default=520350)
    ap.add_argument("--channels", type=int, default=128)
    ap.add_argument("--lmax", type=int, default=3)
    ap.add_argument("--reps", type=int, default=3)
    args = ap.parse_args(argv)
    dev = torch.device("cuda:0")
    n, C = args.edges, args.channels
    keys, paths, table = bucket_table(args.lmax, dev)
    g = torch.Generator(device=dev).manual_seed(0)
    x1 = {k: torch.randn(n, C, 2 * k[0] + 1, device=dev, generator=g) for k in keys}
    x2 = {k: torch.randn(n, 1, 2 * k[0] + 1, device=dev, generator=g) for k in keys}
    W = torch.randn(len(paths), C, C, device=dev, generator=g) / C
    gates = torch.randn(n, len(paths), device=dev, generator=g)
    Ws = [W[t[4]].contiguous() for t in table]
    Gs = [gates[:, t[4]].contiguous() for t in table]

    def forward():
        out = {k: torch.zeros(n, C, 2 * k[0] + 1, device=dev) for k in keys}
        ys = []
        for (k1, k2, k3, kdim, pidx, U), w, gt in zip(table, Ws, Gs):
            y = X.project_bucket_forward(x1[k1], x2[k2], U, len(pidx))
            ys.append(y)
            out[k3] += X.mix_bucket_forward(y, w, gt)
        return out, ys

    def backward(ys, grad_out):
        for (k1, k2, k3, kdim, pidx, U), w, gt, y in zip(table, Ws, Gs, ys):
            go = grad_out[k3]
            gy = X.mix_bucket_transpose_y(go, w, gt)
            X.mix_bucket_transpose_w(go, y, gt)
            X.mix_bucket_transpose_g(go, y, w)
            X.project_bucket_transpose_a(gy, x2[k2], U)
            X.project_bucket_transpose_b(gy, x1[k1], U)

    out, ys = forward()
    grad_out = {k: torch.randn_like(v) for k, v in out.items()}
    backward(ys, grad_out)
    torch.cuda.synchronize()
    e0, e1, e2 = (torch.cuda.Event(enable_timing=True) for _ in range(3))
    e0.record()
    for _ in range(args.reps):
        out, ys = forward()
    e1.record()
    for _ in range(args.reps):
        backward(ys, grad_out)
    e2.record()
    torch.cuda.synchronize()
    fwd_ms, bwd_ms = e0.elapsed_time(e1) / args.reps, e1.elapsed_time(e2) / args.reps
    flops = 2 * n * sum(len(t[4]) * t[3] * C * C for t in table)
    print(json.dumps({"seam": "molecular_force_field._C_ictd_tp (fsctep_amd.ictd_tp_ext)",
                      "conv": f"ICTD conv2, full path policy, lmax {args.lmax}", "edges": n, "channels": C,
                      "paths": len(paths), "buckets": len(table), "forward_ms": round(fwd_ms, 3),
                      "backward_ms": round(bwd_ms, 3), "mix_gflop_forward": round(flops / 1e9, 1),
                      "mix_tflops_forward": round(flops / (fwd_ms * 1e-3) / 1e12, 1)}), flush=True)


if __name__ == "__main__":
    main()
