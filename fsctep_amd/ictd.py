"""``pure-cartesian-ictd`` and ``pure-cartesian-ictd-o3`` trunks on the HIP kernels.

``PureCartesianICTDTransformerLayer`` (reference models/pure_cartesian_ictd_layers_full.py:476-1078) and
``PureCartesianICTDO3TransformerLayer`` (models/pure_cartesian_ictd_layers_o3.py:535-1074) take the
reference's constructor arguments and hold its parameters under the same state_dict keys.  Message
passing runs in ``libfsctep_hip.so`` (``torch.ops.fsctep.ictd_conv1`` / ``ictd_conv``), as do the edge geometry,
the direction harmonics and the radial MLPs (``edge_geometry``, ``edge_harmonics``, ``radial_mlp``); the readout
outside its Gram bilinear stays in PyTorch.  Node features are x[N][M][C]
(component-major over the active irreps); the readout rebuilds the reference's flat per-layer layout
because the reference re-splits the layer-concatenated vector with n_layers*C channels
(full :977-979, o3 :987-988) and its energy depends on that exact arrangement.
"""

from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn as nn
import torch.nn.functional as F

from . import ictd_ops
from .readout_ops import ReadoutMaps, prepare_gram, readout_features
from .graph import Graph, poison_invalid, prepare_species_graph, species_rows
from .ictd_basis import canonical, coupling, layout_full, layout_o3
from .sparse import MainNet, RobustScalarWeightedSum, _radial_mlp, readout_energy

LMAX_KERNELS = 3     # (lmax + 1)^2 <= 16 harmonic components in the projection and conv1 kernels


def _key_str(k) -> str:
    return f"{k[0]}{'e' if k[1] > 0 else 'o'}"


class _TPWeights(nn.Module):
    """Parameter holder of HarmonicFullyConnectedTensorProduct[O3] (internal weights (P, O, I, J))."""

    def __init__(self, num_paths, mul_out, mul_in1, mul_in2):
        super().__init__()
        self.num_paths = num_paths
        self.weight = nn.Parameter(torch.randn(num_paths, mul_out, mul_in1, mul_in2) * 0.02)


class _Conv1(nn.Module):
    """conv1 parameters: ICTDIrrepsE3Conv (:211-339) / ICTDO3E3Conv (:298-422)."""

    def __init__(self, o3, n_ref, n_keys, lmax, number_of_basis, channels_out, embedding_dim, max_atomvalue,
                 output_size, external_field):
        super().__init__()
        self.atom_embedding = nn.Embedding(max_atomvalue, embedding_dim)
        self.atom_mlp = nn.Sequential(nn.Linear(embedding_dim, 64), nn.SiLU(), nn.Linear(64, output_size))
        self.fidelity_embedding = None
        self.tp2 = _TPWeights(n_ref, channels_out, output_size, output_size)
        self.fc = _radial_mlp(n_ref, number_of_basis)
        if external_field:
            if o3:
                self.external_tensor_scale_by_irrep = nn.Parameter(torch.zeros(n_keys))
            else:
                self.external_tensor_scale_by_l = nn.Parameter(torch.zeros(lmax + 1))


class _ICTDTrunk(nn.Module):
    o3 = False

    def __init__(self, max_embed_radius, main_max_radius, main_number_of_basis, hidden_dim_conv,
                 hidden_dim_sh=None, hidden_dim=64, channel_in2=32, embedding_dim=16, max_atomvalue=10,
                 output_size=8, embed_size=None, main_hidden_sizes3=None, num_layers=1, num_interaction=2,
                 device=None, function_type_main="gaussian", lmax=2, ictd_tp_path_policy="full",
                 ictd_tp_max_rank_other=None, internal_compute_dtype=None, ictd_tp_backend="auto",
                 invariant_channels=32, physical_tensor_outputs=None, external_tensor_rank=None,
                 external_tensor_irrep=None, external_tensor_parity=None, external_tensor_specs=None,
                 o3_irrep_preset="auto", o3_active_irreps=None, num_fidelity_levels=0, long_range_mode="none",
                 **unsupported):
        super().__init__()
        for k in unsupported:
            if not k.startswith(("long_range_", "feature_spectral_", "external_tensor_", "multi_fidelity",
                                 "product5_muls_by_l", "max_rank_other", "k_policy", "ictd_Lmax")):
                raise TypeError(f"unexpected argument {k!r}")
        if unsupported.get("product5_muls_by_l") is not None:
            raise NotImplementedError("product5_muls_by_l adapters are outside the HIP path")
        if ictd_tp_path_policy != "full" or long_range_mode != "none" or num_fidelity_levels or external_tensor_specs:
            raise NotImplementedError("HIP ICTD path: path_policy 'full', no long-range, fidelity or multi-spec fields")
        if external_tensor_rank is not None and (int(external_tensor_rank) != 1 or
                                                 (external_tensor_irrep or "1o") != "1o"):
            raise NotImplementedError("HIP ICTD path: external field must be a rank-1 '1o' vector")
        embed_size = [128, 128, 128] if embed_size is None else list(embed_size)
        self.lmax = int(lmax)
        self.channels = int(hidden_dim_conv)
        self.num_interaction = int(num_interaction)
        if self.num_interaction < 2:
            raise ValueError(f"num_interaction must be >= 2, got {self.num_interaction}")
        if self.channels not in (32, 64, 128) or output_size != 8:
            raise NotImplementedError("HIP ICTD path: hidden_dim_conv 32/64/128 and output_size 8")
        if max_atomvalue < 1:
            raise ValueError(f"max_atomvalue must be >= 1, got {max_atomvalue}")
        from .ops import check_basis
        check_basis(function_type_main)
        if not 1 <= main_number_of_basis <= 16:
            raise NotImplementedError("HIP ICTD path: main_number_of_basis 1..16")
        self.n_species = int(max_atomvalue)
        self.invariant_channels = int(invariant_channels)
        self.max_radius = float(max_embed_radius)
        self.number_of_basis = int(main_number_of_basis)
        self.function_type = str(function_type_main)
        self.external_field = external_tensor_rank is not None
        self.layout = self._make_layout(o3_irrep_preset, o3_active_irreps, physical_tensor_outputs)
        self.keys = list(self.layout.keys)
        self.layout_id = ictd_ops.register_layout(self.layout)
        n_ref = self.layout.n_ref_paths()
        self.e3_conv_emb = _Conv1(self.o3, n_ref, len(self.keys), self.lmax, main_number_of_basis, self.channels,
                                  embedding_dim, max_atomvalue, output_size, self.external_field)
        self.tp2_layers = nn.ModuleList([_TPWeights(n_ref, self.channels, self.channels, 1)
                                         for _ in range(self.num_interaction - 1)])
        self.fc2_layers = nn.ModuleList([_radial_mlp(n_ref, main_number_of_basis)
                                         for _ in range(self.num_interaction - 1)])
        nC = self.channels * self.num_interaction
        S = (self.num_interaction - 1) * self.invariant_channels
        wr = [nn.Parameter(torch.randn(S, nC, nC) * 0.02) for _ in self.keys]
        if self.o3:
            self.W_read = nn.ParameterDict({_key_str(k): w for k, w in zip(self.keys, wr)})
        else:
            self.W_read = nn.ParameterList(wr)
        self.readout_linear = nn.Sequential(nn.Linear(S + nC * len(self.keys), embed_size[0]), nn.SiLU(),
                                            nn.Linear(embed_size[0], 17))
        self.weighted_sum = RobustScalarWeightedSum(17, init_weights="zero")
        self.proj_total = MainNet(self.num_interaction * self.channels * len(self.keys) + S, embed_size, 17)
        self.physical_tensor_heads = None
        self._dipole = False
        if physical_tensor_outputs:
            if set(physical_tensor_outputs) != {"dipole"}:
                raise NotImplementedError("HIP ICTD path: only a 'dipole' physical tensor head")
            spec = physical_tensor_outputs["dipole"]
            if spec.get("reduce", "sum") != "sum" or int(spec.get("channels_out", 1)) != 1:
                raise NotImplementedError("HIP ICTD path: dipole head with reduce 'sum', channels_out 1")
            self.physical_tensor_heads = nn.ModuleDict(
                {"dipole": nn.ModuleDict({"1": nn.Linear(nC, 1, bias=False)})})
            self._dipole = True
        self._cache = {}

    def _make_layout(self, preset, active, phys):
        return layout_full(self.lmax)

    # ------------------------------------------------------------------ device constants
    def _consts(self, device):
        key = ("consts", str(device))
        if key not in self._cache:
            cg = torch.tensor(self.layout.cg_table(), dtype=torch.float32, device=device)
            c1 = [p["gate"] for p in self.layout.conv1_paths()]
            factors = [float(coupling(k[0], k[0], 0)[0, 0, 0]) for k in self.keys]
            self._cache[key] = (cg, torch.tensor(c1, device=device), factors)
        return self._cache[key]

    @staticmethod
    def _wt(tp):
        """Channel-mix operand of tp.weight from its current values (no cache: see prepare_gram)."""
        with torch.no_grad():
            return torch.ops.fsctep.ictd_prepare_weights(tp.weight.detach())

    # ------------------------------------------------------------------ forward
    def prepare(self, edge_src, edge_dst, edge_shifts, num_nodes, A, pos=None) -> Graph:
        """The receiver-sorted graph of one neighbour list (device op, no host synchronisation); species
        tables above 16 rows are served by mapping the species present (at most 16) to rows."""
        if int(num_nodes) != A.shape[0]:
            raise ValueError(f"num_nodes {num_nodes} != len(A) {A.shape[0]}")
        return prepare_species_graph(edge_src, edge_dst, edge_shifts, A, self.n_species, pos=pos)

    def _training_step(self) -> bool:
        """True when parameter gradients are wanted (train() mode, grad enabled, parameters that require
        grad): the step is then built from differentiable parts (fsctep_amd.train_ops and the conv2..n op
        with its weight gradient and double backward), so that a force loss trains every parameter."""
        return self.training and torch.is_grad_enabled() and any(p.requires_grad for p in self.parameters())

    def forward(self, pos, A, batch, edge_src, edge_dst, edge_shifts, cell, *, precomputed_edge_vec=None,
                sync_after_scatter=None, external_tensor=None, external_tensor_blocks=None, fidelity_ids=None,
                return_physical_tensors=False, return_reciprocal_source=False):
        """Reference signature (full :867-884, o3 :902-920).  The graph is prepared on every call, as the
        reference sorts on every call.  With ``precomputed_edge_vec`` (E, 3) (caller edge order) the
        geometry comes from it and forces flow back through it, as the reference's branch at full
        :901-902 / o3 :928-929 (the LAMMPS / ML-IAP cores differentiate through edge_vec)."""
        if sync_after_scatter is not None or external_tensor_blocks is not None or fidelity_ids is not None:
            raise NotImplementedError("sync hooks, external blocks and fidelity ids are outside the HIP path")
        g = self.prepare(edge_src, edge_dst, edge_shifts, pos.shape[0], A, pos=pos)
        e, dip = self.forward_graph(pos, batch, cell, g, external_tensor=external_tensor,
                                    edge_vec=precomputed_edge_vec, with_dipole=bool(return_physical_tensors))
        if return_physical_tensors:
            return e, {"dipole": {1: dip}} if dip is not None else {}
        return e

    def forward_graph(self, pos, batch, cell, g: Graph, external_tensor=None, edge_vec=None, with_dipole=True):
        """((N,1) atomic energies, (G,1,3) dipole or None) for a prepared graph; ``edge_vec`` (E, 3), in the
        caller's edge order, replaces the geometry from ``pos`` (differentiable w.r.t. it).  The dipole head
        runs when the model has one and ``with_dipole`` is set; it has one row per graph of ``cell`` (G, 3, 3),
        which the reference sizes as max(batch) + 1 (pure_cartesian_ictd_layers_o3.py:983): the same for
        every batch whose last graph has atoms, and read here without a host synchronisation."""
        if not pos.is_cuda:
            raise RuntimeError("the HIP ICTD path runs on the GPU only")
        if self._training_step():
            return self._forward_train(pos, batch, cell, g, external_tensor, edge_vec, with_dipole)
        f32 = torch.float32
        pos, cell = pos.to(f32), cell.to(f32)
        cg, c1_gates, factors = self._consts(pos.device)
        src_batch = batch.index_select(0, g.src32)
        if edge_vec is not None:
            n, r = ictd_ops.edge_vec_geometry(edge_vec.to(f32), g)
        else:
            with torch.no_grad():
                shift_vec = (g.shifts.to(f32).unsqueeze(-1) * cell.index_select(0, src_batch)).sum(1)
            n, r = ictd_ops.edge_geometry(pos, shift_vec, g)
        Y = ictd_ops.edge_harmonics(n, self.lmax)

        c1 = self.e3_conv_emb
        NS = g.n_species
        with torch.no_grad():   # species-table rows
            atab = c1.atom_mlp(c1.atom_embedding(species_rows(g, pos.device))).detach()
            W1 = c1.tp2.weight.detach()[c1_gates]                                  # (NP1, C, 8, 8)
            qtab = torch.einsum("pcij,si,tj->stpc", W1, atab, atab).reshape(NS * NS, W1.shape[0], self.channels)
        F_in = self._field_term(Y, external_tensor, src_batch, detach=True)
        feats = [ictd_ops.ictd_conv1_apply(F_in, self._gates(c1.fc, r), qtab, g, self.layout_id)]
        for tp, fc2 in zip(self.tp2_layers, self.fc2_layers):
            feats.append(ictd_ops.ictd_conv_apply(feats[-1], Y, self._gates(fc2, r), tp.weight.detach(),
                                                  self._wt(tp), cg, g, self.layout_id))
        e, dip = self.readout(feats, batch, cell.shape[0], factors, with_dipole)
        return poison_invalid(e, g, pos, edge_vec), dip

    def _field_term(self, Y, external_tensor, src_batch, detach: bool):
        """Y plus the external field embedded in the l=1 block of conv1's first operand (z, y, x order)."""
        if not self.external_field:
            if external_tensor is not None:
                raise ValueError("external_tensor given but the model has no external field")
            return Y
        if external_tensor is None:
            raise ValueError("this model was built with an external field; pass external_tensor")
        c1 = self.e3_conv_emb
        fld = external_tensor.to(Y.dtype).reshape(-1, 3).flip(-1)
        if self.o3:
            s = c1.external_tensor_scale_by_irrep[self.keys.index((1, -1))]
        else:
            s = c1.external_tensor_scale_by_l[1]
        s = s.detach() if detach else s
        blk = fld.index_select(0, src_batch) * s
        return Y + torch.cat([torch.zeros_like(Y[:, :1]), blk, torch.zeros_like(Y[:, 4:])], dim=1)

    def _forward_train(self, pos, batch, cell, g: Graph, external_tensor, edge_vec, with_dipole):
        """The training step: geometry, harmonics, radial MLPs, conv1 and the readout Gram as differentiable
        GPU torch formulations (train_ops), conv2..n on the HIP op with its weight gradient and double
        backward."""
        from . import train_ops as T
        f32 = torch.float32
        pos, cell = pos.to(f32), cell.to(f32)
        cg, c1_gates, factors = self._consts(pos.device)
        src_batch = batch.index_select(0, g.src32)
        if edge_vec is not None:
            n, r = T.edge_vec_geometry(edge_vec.to(f32), g)
        else:
            shift_vec = (g.shifts.to(f32).unsqueeze(-1) * cell.index_select(0, src_batch)).sum(1)
            n, r = T.edge_geometry(pos, shift_vec, g)
        Y = T.harmonics(n, self.lmax)
        c1 = self.e3_conv_emb
        NS = g.n_species
        atab = c1.atom_mlp(c1.atom_embedding(species_rows(g, pos.device)))
        W1 = c1.tp2.weight.index_select(0, c1_gates)                                 # (NP1, C, 8, 8)
        qtab = torch.einsum("pcij,si,tj->stpc", W1, atab, atab).reshape(NS * NS, W1.shape[0], self.channels)
        F_in = self._field_term(Y, external_tensor, src_batch, detach=False)
        gates1 = T.radial_full(r, c1.fc, self.max_radius, self.function_type)
        feats = [T.ictd_conv1(F_in, gates1, qtab, g, self.layout)]
        for tp, fc2 in zip(self.tp2_layers, self.fc2_layers):
            gates = T.radial_full(r, fc2, self.max_radius, self.function_type)
            feats.append(ictd_ops.ictd_conv_apply(feats[-1], Y, gates, tp.weight, self._wt(tp), cg, g,
                                                  self.layout_id))
        e, dip = self.readout(feats, batch, cell.shape[0], factors, with_dipole, train=True)
        return poison_invalid(e, g, pos, edge_vec), dip

    def _gates(self, fc, r):
        """Per-path gates fc(radial_basis(r)) (E, P) by one fused kernel (P <= 64)."""
        if fc[4].weight.shape[0] > 64:
            h = ictd_ops.radial_hidden(r, fc, self.max_radius, self.function_type)
            return F.linear(h, fc[4].weight.detach(), fc[4].bias.detach())
        return ictd_ops.radial_full(r, fc, self.max_radius, self.function_type)

    def _wread(self, i, k):
        return self.W_read[_key_str(k)] if self.o3 else self.W_read[i]

    def readout(self, feats, batch, n_graphs, factors, with_dipole=True, train=False):
        """Gram bilinear + 0e products + MainNet (full :977-1033, o3 :987-1030), re-split included: the
        Gram inputs (the reference's channel-major flatten, layer concatenation and re-split by key)
        and the per-key squared norms of the layer concatenation come from one fused readout op
        (``train``: from its differentiable torch formulation, for parameter gradients)."""
        nL = len(feats)
        key = ("maps", nL)
        if key not in self._cache:
            self._cache[key] = ReadoutMaps(nL, self.channels, [2 * k[0] + 1 for k in self.keys], resplit=True)
        maps = self._cache[key]
        scales = [1.0 / math.sqrt(2 * k[0] + 1) for k in self.keys]
        if train:
            from . import train_ops as T
            scalars, sq_all = T.readout_features(feats, [self._wread(i, k) for i, k in enumerate(self.keys)],
                                                 scales, maps)
        else:
            grams = [prepare_gram(self._wread(i, k)) for i, k in enumerate(self.keys)]
            scalars, sq_all = readout_features(feats, grams, scales, maps)
        outs = []
        # unbind: its backward stacks the per-key gradients in one copy (a select per key would zero-fill,
        # copy and accumulate the whole (N, keys, n*C) gradient once per key)
        for i, (k, sq) in enumerate(zip(self.keys, sq_all.unbind(1))):
            if k == (0, 1):
                sq = torch.cat([sq, scalars * scalars], dim=-1)
            outs.append(sq * factors[i])
        f = torch.cat(outs, dim=-1)
        e = self.weighted_sum(self.proj_total(f)) if train else readout_energy(self.proj_total, self.weighted_sum, f)
        dip = None
        if self._dipole and with_dipole:
            # the (1, -1) Gram input, (N, d, n*C), by the same column map (differentiable gather)
            i = self.keys.index((1, -1))
            nC = nL * self.channels
            col0 = sum(d * nC for d in maps.key_dims[:i])
            idx = maps.on(feats[0].device)[0][col0:col0 + 3 * nC].long()
            t = torch.cat([f.flatten(1) for f in feats], dim=1).index_select(1, idx).view(-1, 3, nC)
            W = self.physical_tensor_heads["dipole"]["1"].weight
            y = torch.matmul(t, W.t().contiguous()).transpose(1, 2)          # (N, o, 3) = einsum("ncm,oc->nom")
            # per-graph sum as a (G, N) one-hot product: a fixed summation order (index_add's atomics are not)
            onehot = (torch.arange(n_graphs, device=batch.device).unsqueeze(1) == batch.unsqueeze(0)).to(y.dtype)
            dip = torch.matmul(onehot, y.reshape(-1, 3)).view(n_graphs, 1, 3)
        return e, dip


class PureCartesianICTDTransformerLayer(_ICTDTrunk):
    """Drop-in for the reference ``pure-cartesian-ictd`` trunk (lmax 0 to 3)."""

    o3 = False

    def _make_layout(self, preset, active, phys):
        if not 0 <= self.lmax <= LMAX_KERNELS:
            raise NotImplementedError(f"HIP ICTD path: lmax 0 to {LMAX_KERNELS} (the kernels take at most "
                                      "16 harmonic and 16 feature components)")
        return layout_full(self.lmax)


def _parse_irreps(spec, lmax: int) -> list:
    """'0e,1o + 2e' or ['0e', '1o'] -> [(l, parity)], multiplicity 1 only (models/pure_cartesian_ictd_layers_o3.py:66-86)."""
    items = spec.replace(",", " ").replace("+", " ").split() if isinstance(spec, str) else [str(x) for x in spec]
    out = []
    for it in items:
        it = it.strip()
        if not it:
            continue
        mul, _, ir = it.rpartition("x")
        if mul not in ("", "1") or len(ir) < 2 or ir[-1] not in "eo" or not ir[:-1].isdigit():
            raise ValueError(f"o3 irreps: multiplicity-1 entries like '1o' expected, got {it!r}")
        l = int(ir[:-1])
        if not 0 <= l <= lmax:
            raise ValueError(f"o3 irreps entry {it!r} outside 0..{lmax}")
        out.append((l, 1 if ir[-1] == "e" else -1))
    return out


def _sorted_keys(keys) -> list:
    return sorted(set(keys), key=lambda k: (k[0], 0 if k[1] > 0 else 1))


def resolve_o3_keys(lmax: int, preset="auto", explicit=None, external_irrep=None, physical_tensor_outputs=None):
    """Active irreps of the O3 trunk, as the reference resolves them
    (models/pure_cartesian_ictd_layers_o3.py:88-180): the required ones (0e, the external field's irrep,
    the physical-tensor heads' irreps) joined to an explicit list, or to the preset: 'auto' adds the
    geometric irreps (l, (-1)^l), 'full' is every (l, +-1), 'minimal' the required ones alone, and
    'balanced' the geometric and required ones plus every (l3, p1 p2) their products with the geometric
    irreps reach up to lmax."""
    required = [(0, 1)]
    if external_irrep is not None:
        required += [k for k in _parse_irreps(external_irrep, 10 ** 6) if k[0] <= lmax]
    for spec in (physical_tensor_outputs or {}).values():
        if spec.get("irreps") is not None:
            required += [k for k in _parse_irreps(spec["irreps"], 10 ** 6) if k[0] <= lmax]
        else:
            required += [canonical(int(l)) for l in spec.get("ls", [])]
    required = _sorted_keys(required)
    if explicit is not None and (not isinstance(explicit, str) or explicit.strip()):
        parsed = _parse_irreps(explicit, lmax)
        if parsed:
            return _sorted_keys(parsed + required)
    preset = str(preset or "auto").strip().lower()
    geom = [canonical(l) for l in range(lmax + 1)]
    if preset == "full":
        return _sorted_keys([(l, p) for l in range(lmax + 1) for p in (1, -1)])
    if preset == "minimal":
        return required
    if preset == "auto":
        return _sorted_keys(geom + required)
    if preset == "balanced":
        seed = _sorted_keys(geom + required)
        out = set(seed)
        for l1, p1 in seed:
            for l2, p2 in geom:
                for l3 in range(abs(l1 - l2), min(l1 + l2, lmax) + 1):
                    out.add((l3, p1 * p2))
        return _sorted_keys(out)
    raise ValueError(f"Unknown o3_irrep_preset={preset!r}; expected auto|minimal|balanced|full")


class PureCartesianICTDO3TransformerLayer(_ICTDTrunk):
    """Drop-in for the reference ``pure-cartesian-ictd-o3`` trunk: active irreps from ``o3_active_irreps``
    or the ``o3_irrep_preset`` (auto, minimal, balanced, full), resolved as the reference does."""

    o3 = True

    def _make_layout(self, preset, active, phys):
        if not 0 <= self.lmax <= LMAX_KERNELS:
            raise NotImplementedError(f"HIP ICTD-O3 path: lmax 0 to {LMAX_KERNELS} (the kernels take at most "
                                      "16 harmonic components)")
        keys = resolve_o3_keys(self.lmax, preset, active, "1o" if self.external_field else None, phys)
        for l in range(self.lmax + 1):
            if canonical(l) not in keys:
                raise NotImplementedError(f"HIP ICTD-O3 path: active irreps {keys} lack the geometric irrep "
                                          f"{canonical(l)}; the kernels need 0e,1o,2e,.. up to lmax")
        lay = layout_o3(self.lmax, keys)
        problems = ictd_ops.kernel_limits(lay)
        if problems:
            raise NotImplementedError(f"HIP ICTD-O3 path: active irreps {[_key_str(k) for k in keys]} exceed the "
                                      "kernels' tables: " + "; ".join(problems))
        return lay


def energy_forces(model, pos, batch, cell, graph, external_tensor=None):
    """(per-atom energies (N,), forces (N,3), dipole or None)."""
    pos = pos.detach().requires_grad_(True)
    e, dip = model.forward_graph(pos, batch, cell, graph, external_tensor=external_tensor)
    (grad,) = torch.autograd.grad(e.sum(), pos)
    return e.detach().squeeze(-1), -grad, (dip.detach() if dip is not None else None)
