"""Energy + forces replayed from a HIP graph, for systems small enough to be launch-bound.

A 1,000-atom step issues about a hundred kernel launches whose work is a few microseconds each, so the
host's launch rate, not the GPU, sets the step time.  ``CapturedEnergyForces`` records one energy + forces
evaluation of a trunk on a prepared graph (edge geometry, radial MLPs, the three convolutions, the
readout and the autograd backward w.r.t. positions) into a ``torch.cuda.CUDAGraph`` and replays it: one
launch per step.  This is the Python counterpart of the LAMMPS engine's CUDA-graph path
(lammps_user_mfftorch/src/USER-MFFTORCH/mff_torch_engine.cpp:648-737), which captures the TorchScript
core the same way; as there, the graph (neighbour list) and the parameters are fixed for the life of the
capture and positions are copied into a static input buffer before each replay.

Requirements the capture relies on: no host synchronisation anywhere in the step (the trunks read every
size from tensor shapes, the dipole's graph count from ``cell``), no memset nodes (the ops' kernels clear
their own buffers), and outputs that are static tensors overwritten by each replay: copy them out before
the next call if they must be kept.
"""

from __future__ import annotations

import torch


def _step_fn(model, pos, batch, cell, graph, external_tensor):
    from .ictd import _ICTDTrunk, energy_forces
    from .sparse import energy_and_forces
    if isinstance(model, _ICTDTrunk):
        return lambda: energy_forces(model, pos, batch, cell, graph, external_tensor=external_tensor)

    def run():
        e, f = energy_and_forces(model, pos, batch, cell, graph)
        return e, f, None
    return run


class CapturedEnergyForces:
    """``(energies (N,), forces (N, 3), dipole or None)`` of ``model`` on ``graph``, one HIP-graph replay per call.

    ``pos``, ``batch``, ``cell`` and ``external_tensor`` are copied into static buffers at construction;
    ``__call__(pos)`` copies new positions in (same shape) and replays.  The model must be in eval mode
    with parameters that do not require grad; parameter values are read at replay time (in-place updates
    are seen), tensor identities are fixed."""

    def __init__(self, model, pos, batch, cell, graph, external_tensor=None, warmup: int = 3):
        if not pos.is_cuda:
            raise RuntimeError("CapturedEnergyForces runs on the GPU only")
        self.pos = pos.detach().to(torch.float32).clone()
        self.batch = batch.clone()
        self.cell = cell.detach().to(torch.float32).clone()
        self.ext = None if external_tensor is None else external_tensor.detach().to(torch.float32).clone()
        self.graph = graph
        fn = _step_fn(model, self.pos, self.batch, self.cell, graph, self.ext)
        cur = torch.cuda.current_stream(self.pos.device)
        side = torch.cuda.Stream(self.pos.device)          # default priority
        side.wait_stream(cur)
        with torch.cuda.stream(side):                        # fill the models' constant caches off-capture
            for _ in range(max(1, warmup)):
                fn()
        cur.wait_stream(side)
        torch.cuda.synchronize(self.pos.device)
        self.cuda_graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.cuda_graph):
            self.out = fn()
        torch.cuda.synchronize(self.pos.device)

    def __call__(self, pos=None, external_tensor=None):
        if pos is not None:
            if pos.shape != self.pos.shape:
                raise ValueError(f"positions of shape {tuple(pos.shape)}, captured for {tuple(self.pos.shape)}")
            self.pos.copy_(pos.detach())
        if external_tensor is not None:
            if self.ext is None or external_tensor.shape != self.ext.shape:
                raise ValueError("external_tensor does not match the captured one")
            self.ext.copy_(external_tensor.detach())
        self.cuda_graph.replay()
        return self.out
