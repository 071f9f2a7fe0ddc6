"""``pure-cartesian-sparse`` trunk on the HIP kernels.

``PureCartesianSparseTransformerLayer`` takes the reference's constructor arguments and
holds the reference's parameters under the same state_dict keys
(``models/pure_cartesian_sparse_layers.py:459-855``), so reference checkpoints load
unchanged.  Its message passing runs in ``libfsctep_hip.so``:

* conv1 (``:227-330``): ``torch.ops.fsctep.sparse_conv1`` on a species-pair table;
* conv2..n (``:382-421``): ``torch.ops.fsctep.sparse_conv``;
* readout Gram bilinear ``product_3`` (``:424-456``): ``torch.ops.fsctep.gram_bilinear``.

Edge geometry and the radial MLP fc[:4] (``:745-756``, ``:204-210``, ``:319-321``, ``:372-378``,
``:410-412``) run as ``torch.ops.fsctep.edge_geometry`` / ``radial_mlp``; the rest of the readout
(``:769-833``) stays in PyTorch, on the same internal feature layout x[N][13][C]
(component-major; the reference's pseudo half is identically zero and is not stored).  In train()
mode (force-loss training) the light ops switch to their differentiable formulations in
``train_ops`` and conv2..n keeps its HIP op, which gives its weight gradient and double backward.
"""

from __future__ import annotations

import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import ops
from .readout_ops import ReadoutMaps, prepare_gram, readout_features
from .graph import Graph, poison_invalid, prepare_species_graph, species_rows

_COMPS = ((0, 1), (1, 4), (4, 13))   # component ranges of ranks 0, 1, 2


class MainNet(nn.Module):
    """LayerNorm -> [Linear -> LayerNorm -> SiLU]* -> Linear (reference models/mlp.py:8-66)."""

    def __init__(self, input_size, hidden_sizes, output_size):
        super().__init__()
        self.input_norm = nn.LayerNorm(input_size)
        self.layers = nn.ModuleList()
        self.layer_norms = nn.ModuleList()
        prev = input_size
        for hsz in hidden_sizes:
            self.layers.append(nn.Linear(prev, hsz))
            self.layer_norms.append(nn.LayerNorm(hsz))
            prev = hsz
        self.output = nn.Linear(prev, output_size)
        for m in self.modules():
            if isinstance(m, nn.Linear):
                if m is self.output:
                    nn.init.normal_(m.weight, 0.0, 0.01)
                else:
                    nn.init.kaiming_normal_(m.weight, a=0, mode="fan_in", nonlinearity="relu")
                nn.init.zeros_(m.bias)

    def forward(self, x):
        x = self.input_norm(x)
        for lin, ln in zip(self.layers, self.layer_norms):
            x = F.silu(ln(lin(x)))
        return self.output(x)


class RobustScalarWeightedSum(nn.Module):
    """sum_i x_i w_i (reference models/mlp.py:117-133); zero-initialised like the reference."""

    def __init__(self, num_features, init_weights="zero"):
        super().__init__()
        self.weights = nn.Parameter(torch.zeros(num_features) if init_weights == "zero"
                                    else torch.randn(num_features) * 0.1)

    def forward(self, x):
        return (x * self.weights).sum(dim=-1, keepdim=True)


def readout_energy(net: MainNet, weighted_sum: RobustScalarWeightedSum, x: torch.Tensor) -> torch.Tensor:
    """weighted_sum(net(x)), (N, 1), by the fused readout-head kernels (``torch.ops.fsctep.readout_mlp``:
    one launch forward, one for the input gradient; no parameter gradients) where the head has their shape:
    fp32 GPU input with K % 4 == 0, 1 to 4 hidden layers all 64, 128 or 256 wide, affine LayerNorms and
    Linear biases.  Other heads run as the torch modules (reference models/mlp.py:8-66, :117-133)."""
    hid = [lin.out_features for lin in net.layers]
    norms = [net.input_norm, *net.layer_norms]
    K = x.shape[-1] if x.dim() == 2 else -1
    if not (x.is_cuda and x.dtype == torch.float32 and K % 4 == 0 and K >= 4 and 1 <= len(hid) <= 4
            and hid[0] in (64, 128, 256) and all(h == hid[0] for h in hid)
            and all(ln.weight is not None and ln.bias is not None and ln.weight.dim() == 1 for ln in norms)
            and all(lin.bias is not None for lin in (*net.layers, net.output))
            and weighted_sum.weights.numel() == net.output.out_features):
        return weighted_sum(net(x))
    dims = [K, hid[0], len(hid), net.output.out_features]
    eps = [float(ln.eps) for ln in norms]
    params = [net.input_norm.weight, net.input_norm.bias]
    for lin, ln in zip(net.layers, net.layer_norms):
        params += [lin.weight, lin.bias, ln.weight, ln.bias]
    params += [net.output.weight, net.output.bias, weighted_sum.weights]
    with torch.no_grad():
        w = torch.ops.fsctep.readout_mlp_prepare([p.detach() for p in params], dims, eps)
    return torch.ops.fsctep.readout_mlp(x, w, dims, eps)


def _radial_mlp(hidden_out: int, nb: int) -> nn.Sequential:
    return nn.Sequential(nn.Linear(nb, 64), nn.SiLU(), nn.Linear(64, 64), nn.SiLU(), nn.Linear(64, hidden_out))


class PureCartesianSparseE3Conv(nn.Module):
    """conv1 parameters (reference :134-226): atom embedding/MLP and the radial MLP fc."""

    def __init__(self, max_radius, number_of_basis, channels_out, embedding_dim=16, max_atomvalue=10,
                 output_size=8, Lmax=2, function_type="gaussian"):
        super().__init__()
        self.max_radius = max_radius
        self.number_of_basis = number_of_basis
        self.channels_out = channels_out
        self.output_size = output_size
        self.Lmax = Lmax
        self.function_type = function_type
        self.atom_embedding = nn.Embedding(max_atomvalue, embedding_dim)
        self.atom_mlp = nn.Sequential(nn.Linear(embedding_dim, 64), nn.SiLU(), nn.Linear(64, output_size))
        self.fidelity_embedding = None
        self.fc = _radial_mlp(6 * channels_out * output_size * output_size, number_of_basis)

    def atom_table(self, species: torch.Tensor) -> torch.Tensor:
        return self.atom_mlp(self.atom_embedding(species.long()))


class PureCartesianSparseE3Conv2(nn.Module):
    """conv2..n parameters (reference :333-380): the radial MLP fc."""

    def __init__(self, max_radius, number_of_basis, channels_in, channels_out, Lmax=2,
                 function_type="gaussian"):
        super().__init__()
        if channels_in != channels_out:
            raise ValueError("the HIP sparse conv needs channels_in == channels_out")
        self.max_radius = max_radius
        self.number_of_basis = number_of_basis
        self.channels_in = channels_in
        self.channels_out = channels_out
        self.Lmax = Lmax
        self.function_type = function_type
        self.fc = _radial_mlp(6 * channels_out * channels_in, number_of_basis)

    def prepared_weights(self):
        """The kernel operands (bk1, bk6) of fc.4, made from the current parameter values on every call
        (no cache: an in-place update through ``.data`` does not change a parameter's version)."""
        with torch.no_grad():
            return torch.ops.fsctep.sparse_prepare_weights(self.fc[4].weight.detach(), self.fc[4].bias.detach(),
                                                           self.channels_out)


class PureCartesianSparseInvariantBilinear(nn.Module):
    """product_3 parameters (reference :424-438)."""

    def __init__(self, channels, out_channels, Lmax):
        super().__init__()
        self.channels = channels
        self.out_channels = out_channels
        self.Lmax = Lmax
        self.W = nn.ParameterList([nn.Parameter(torch.randn(out_channels, channels, channels) * 0.02)
                                   for _ in range(Lmax + 1)])

    def forward(self, blocks):
        """blocks[L]: (N, 3^L, channels) -> (N, out_channels), by the fused Gram-bilinear kernel."""
        total = 0
        for L, t in enumerate(blocks):
            scale = 1.0 / math.sqrt(3 ** L) if L > 0 else 1.0
            Wf, Wb = prepare_gram(self.W[L])
            total = total + torch.ops.fsctep.gram_bilinear(t, Wf, Wb, scale)
        return total


class PureCartesianSparseTransformerLayer(nn.Module):
    """Drop-in for the reference class of the same name (lmax 2, max_rank_other 1, k_policy k0)."""

    def __init__(self, max_embed_radius, main_max_radius, main_number_of_basis, hidden_dim_conv,
                 hidden_dim_sh=None, hidden_dim=64, channel_in2=32, embedding_dim=16, max_atomvalue=10,
                 output_size=8, invariant_channels=32, embed_size=None, main_hidden_sizes3=None,
                 num_layers=1, num_interaction=2, device=None, function_type_main="gaussian", lmax=2,
                 max_rank_other=1, k_policy="k0", long_range_mode="none", external_tensor_rank=None,
                 external_tensor_specs=None, num_fidelity_levels=0, physical_tensor_outputs=None,
                 **unsupported):
        super().__init__()
        if lmax != 2 or max_rank_other != 1 or k_policy != "k0":
            raise NotImplementedError("HIP sparse path: lmax=2, max_rank_other=1, k_policy='k0' only")
        if long_range_mode != "none" or external_tensor_rank is not None or external_tensor_specs \
                or num_fidelity_levels or physical_tensor_outputs:
            raise NotImplementedError("HIP sparse path: long-range, external tensors, fidelity and "
                                      "physical tensor heads are outside this path")
        for k, v in unsupported.items():
            if k.startswith(("long_range_", "feature_spectral_")) or k in ("multi_fidelity_mode",
                                                                         "external_tensor_scale_init"):
                continue
            raise TypeError(f"unexpected argument {k!r}")
        if output_size != 8:
            raise NotImplementedError("HIP sparse conv1 needs output_size 8")
        if max_atomvalue < 1:
            raise ValueError(f"max_atomvalue must be >= 1, got {max_atomvalue}")
        ops.check_basis(function_type_main)
        if not 1 <= main_number_of_basis <= 16:
            raise NotImplementedError("HIP sparse path: main_number_of_basis 1..16")
        if hidden_dim_conv not in (32, 64, 128):
            raise NotImplementedError("HIP sparse path: hidden_dim_conv 32, 64 or 128")
        if num_interaction < 2:
            raise ValueError(f"num_interaction must be >= 2, got {num_interaction}")
        embed_size = [128, 128, 128] if embed_size is None else list(embed_size)
        self.Lmax = lmax
        self.lmax = lmax
        self.channels = hidden_dim_conv
        self.num_interaction = int(num_interaction)
        self.invariant_channels = int(invariant_channels)
        self.max_rank_other = max_rank_other
        self.k_policy = k_policy
        self.e3_conv_layers = nn.ModuleList()
        self.e3_conv_layers.append(PureCartesianSparseE3Conv(
            max_embed_radius, main_number_of_basis, self.channels, embedding_dim, max_atomvalue,
            output_size, lmax, function_type_main))
        self.e3_conv_emb = self.e3_conv_layers[0]
        for _ in range(1, self.num_interaction):
            self.e3_conv_layers.append(PureCartesianSparseE3Conv2(
                max_embed_radius, main_number_of_basis, self.channels, self.channels, lmax, function_type_main))
        self.combined_channels = self.channels * self.num_interaction
        scalar_channels = (self.num_interaction - 1) * self.invariant_channels
        self.product_3 = PureCartesianSparseInvariantBilinear(self.combined_channels, scalar_channels, lmax)
        self.proj_total = MainNet(self.num_interaction * self.channels * (lmax + 1) + scalar_channels,
                                  embed_size, 17)
        self.weighted_sum = RobustScalarWeightedSum(17, init_weights="zero")
        self.max_radius = max_embed_radius
        self.number_of_basis = main_number_of_basis
        self._readout_cache = {}
        self.function_type = function_type_main
        self.n_species = int(max_atomvalue)
        # products of the conv2..n channel mix: "fp32" (fp32-accurate split products, the default) or "bf16"
        # (one bf16 MFMA per product with fp32 accumulation; an MI355X option, not in the reference)
        self.channel_mix_precision = "fp32"

    # ------------------------------------------------------------------ graph handling
    def prepare(self, edge_src, edge_dst, edge_shifts, num_nodes, A, pos=None) -> Graph:
        """The receiver-sorted graph of one neighbour list (device op, no host synchronisation).  Reusing
        it across calls with unchanged edges is the caller's choice (``forward_graph``).  Up to 16
        species-table rows (max_atomvalue) the atomic number is the row; a larger table is served by
        mapping the species present (at most 16) to rows on the device."""
        if int(num_nodes) != A.shape[0]:
            raise ValueError(f"num_nodes {num_nodes} != len(A) {A.shape[0]}")
        return prepare_species_graph(edge_src, edge_dst, edge_shifts, A, self.n_species, pos=pos)

    # ------------------------------------------------------------------ forward
    def forward(self, pos, A, batch, edge_src, edge_dst, edge_shifts, cell, *, precomputed_edge_vec=None,
                external_tensor=None, fidelity_ids=None, return_physical_tensors=False,
                return_reciprocal_source=False, **_unused):
        """Reference signature (pure_cartesian_sparse_layers.py:723-735).  The graph is prepared on every
        call, as the reference sorts on every call; ``precomputed_edge_vec`` is ignored, as in the
        reference's sparse trunk (geometry from ``pos``, ``edge_shifts`` and ``cell``)."""
        if external_tensor is not None or fidelity_ids is not None or return_physical_tensors:
            raise NotImplementedError("external tensors / fidelity / physical tensors are outside the HIP path")
        g = self.prepare(edge_src, edge_dst, edge_shifts, pos.shape[0], A, pos=pos)
        e = self.forward_graph(pos, batch, cell, g)
        if return_reciprocal_source:
            return e, e.new_empty((e.shape[0], 0))
        return e

    def _training_step(self) -> bool:
        """True when parameter gradients are wanted (train() mode, grad enabled, parameters that require
        grad): the step is then built from differentiable parts (fsctep_amd.train_ops and the conv2..n op
        with its double backward), so that a force loss trains every parameter."""
        return self.training and torch.is_grad_enabled() and any(p.requires_grad for p in self.parameters())

    def forward_graph(self, pos, batch, cell, g: Graph):
        """(N, 1) atomic energies for a prepared graph; differentiable w.r.t. ``pos`` (and, in train() mode,
        twice differentiable w.r.t. ``pos`` and the parameters)."""
        if not pos.is_cuda:
            raise RuntimeError("the HIP sparse path runs on the GPU only")
        if self._training_step():
            return self._forward_train(pos, batch, cell, g)
        dtype = torch.float32
        pos = pos.to(dtype)
        cell = cell.to(dtype)
        with torch.no_grad():
            edge_cell = cell.index_select(0, batch.index_select(0, g.src32))
            shift_vec = (g.shifts.to(dtype).unsqueeze(-1) * edge_cell).sum(1)   # elementwise: no batched GEMM
        n, r = ops.edge_geometry(pos, shift_vec, g)

        conv1 = self.e3_conv_layers[0]
        # species-table rows, as atom_mlp(atom_embedding(A)) per atom
        with torch.no_grad():
            atab = conv1.atom_table(species_rows(g, pos.device)).to(dtype)
            mf, mb = torch.ops.fsctep.sparse_conv1_pair_table(conv1.fc[4].weight.detach(),
                                                              conv1.fc[4].bias.detach(), atab, self.channels)
        h1 = ops.radial_hidden(r, conv1.fc, self.max_radius, self.function_type)
        feats = [ops.sparse_conv1_apply(h1, n, mf, mb, g, self.channels)]
        for conv in self.e3_conv_layers[1:]:
            bk1, bk6 = conv.prepared_weights()
            h = ops.radial_hidden(r, conv.fc, self.max_radius, self.function_type)
            feats.append(ops.sparse_conv_apply(feats[-1], h, n, bk1, bk6, g, self._precision_code()))
        return poison_invalid(self.readout(feats), g, pos)

    def _forward_train(self, pos, batch, cell, g: Graph):
        """The training step: geometry, radial MLPs, conv1 and readout as differentiable GPU torch
        formulations (train_ops), conv2..n on the HIP op with its weight gradient and double backward."""
        from . import train_ops as T
        dtype = torch.float32
        pos = pos.to(dtype)
        cell = cell.to(dtype)
        edge_cell = cell.index_select(0, batch.index_select(0, g.src32))
        shift_vec = (g.shifts.to(dtype).unsqueeze(-1) * edge_cell).sum(1)
        n, r = T.edge_geometry(pos, shift_vec, g)
        conv1 = self.e3_conv_layers[0]
        atab = conv1.atom_table(species_rows(g, pos.device)).to(dtype)
        h1 = T.radial_hidden(r, conv1.fc, self.max_radius, self.function_type)
        feats = [T.sparse_conv1(h1, n, conv1.fc[4].weight, conv1.fc[4].bias, atab, g, self.channels)]
        for conv in self.e3_conv_layers[1:]:
            bk1, bk6 = conv.prepared_weights()
            h = T.radial_hidden(r, conv.fc, self.max_radius, self.function_type)
            feats.append(ops.sparse_conv_apply(feats[-1], h, n, bk1, bk6, g, self._precision_code(),
                                               conv.fc[4].weight, conv.fc[4].bias))
        return poison_invalid(self.readout(feats, train=True), g, pos)

    def _precision_code(self) -> int:
        prec = getattr(self, "channel_mix_precision", "fp32")
        if prec not in ("fp32", "bf16"):
            raise ValueError(f"channel_mix_precision must be 'fp32' or 'bf16', got {prec!r}")
        return 1 if prec == "bf16" else 0

    def readout(self, feats, train: bool = False):
        """pure_cartesian_sparse_layers.py:769-833 on x[N][13][C] features: the rank-L blocks of all
        layers (t_L = cat_l x_l[:, block L, :]) feed product_3 and their squared norms
        sum_m x^2 / 3^{L/2} the invariants, all assembled by one fused readout op (``train``: by its
        differentiable torch formulation, for parameter gradients)."""
        nL = len(feats)
        key = ("maps", nL)
        if key not in self._readout_cache:
            self._readout_cache[key] = ReadoutMaps(nL, self.channels, [b - a for (a, b) in _COMPS], resplit=False)
        maps = self._readout_cache[key]
        p3 = self.product_3
        scales = [1.0 / math.sqrt(3 ** L) for L in range(len(_COMPS))]
        if train:
            from . import train_ops as T
            f3, sq = T.readout_features(feats, [p3.W[L] for L in range(len(_COMPS))], scales, maps)
        else:
            grams = [prepare_gram(p3.W[L]) for L in range(len(_COMPS))]
            f3, sq = readout_features(feats, grams, scales, maps)
        skey = ("scales", str(sq.device))
        if skey not in self._readout_cache:
            self._readout_cache[skey] = torch.tensor(scales, dtype=sq.dtype, device=sq.device).view(1, -1, 1, 1)
        # invariants in the reference order: layer-major, then rank L
        invs = (sq.view(-1, len(_COMPS), nL, self.channels) * self._readout_cache[skey]).transpose(1, 2)
        f5 = torch.cat([invs.flatten(1), f3 * f3], dim=-1)
        if train:
            return self.weighted_sum(self.proj_total(f5))
        return readout_energy(self.proj_total, self.weighted_sum, f5)


def energy_and_forces(model: PureCartesianSparseTransformerLayer, pos, batch, cell, graph: Graph):
    """Per-atom energies (N,) and forces F = -dE/dpos (N, 3)."""
    pos = pos.detach().requires_grad_(True)
    e = model.forward_graph(pos, batch, cell, graph)
    (grad,) = torch.autograd.grad(e.sum(), pos)
    return e.detach().squeeze(-1), -grad
