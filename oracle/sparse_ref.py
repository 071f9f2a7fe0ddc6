"""CPU oracle for the ``pure-cartesian-sparse`` trunk (test infrastructure only).

A restatement, in plain PyTorch, of the reference algorithm: per-edge weights are
materialised by the radial MLP, every sparse path is an explicit einsum on the
O(3)-graded flat layout (true half + an all-zero pseudo half), and messages are
summed to receivers with ``index_add``.  Forces come from autograd.  Parameters are
a ``{state_dict key: tensor}`` mapping with the reference's keys.

Reference files followed (paths relative to the reference root):
  * trunk ``PureCartesianSparseTransformerLayer.forward``  models/pure_cartesian_sparse_layers.py:723-855
  * conv1 ``PureCartesianSparseE3Conv.forward``            models/pure_cartesian_sparse_layers.py:227-330
  * conv2..n ``PureCartesianSparseE3Conv2.forward``        models/pure_cartesian_sparse_layers.py:382-421
  * readout ``PureCartesianSparseInvariantBilinear``       models/pure_cartesian_sparse_layers.py:424-456
  * sparse tensor product (pseudo-zero branch)             models/pure_cartesian.py:790-863
  * path enumeration                                        models/pure_cartesian.py:353-418
  * layouts ``split/merge_by_rank_o3``                     models/pure_cartesian.py:69-143
  * 0e elementwise invariants                               models/pure_cartesian.py:146-221
  * rank powers                                             models/pure_cartesian.py:292-317
  * ``MainNet`` / ``RobustScalarWeightedSum``               models/mlp.py:8-66,117-133
  * scatter (index_add fallback)                            utils/scatter.py:63-116
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch
import torch.nn.functional as F

from .radial import soft_one_hot_linspace


@dataclass(frozen=True)
class SparseConfig:
    channels: int = 64            # hidden_dim_conv
    lmax: int = 2
    num_interaction: int = 3
    number_of_basis: int = 8
    max_radius: float = 5.0
    function_type: str = "bessel"
    embedding_dim: int = 16
    max_atomvalue: int = 10
    output_size: int = 8
    invariant_channels: int = 32
    embed_size: tuple = (128, 128, 128)
    radial_hidden: int = 64       # fixed by the reference's fc = Linear(nb,64)-SiLU-Linear(64,64)-SiLU-Linear(64,W)


# ----------------------------------------------------------------------------- layout

def rank_dim(L: int) -> int:
    return 3 ** L


def o3_dim(c: int, lmax: int) -> int:
    """True half + pseudo half (models/pure_cartesian.py:35-40)."""
    return 2 * c * sum(rank_dim(L) for L in range(lmax + 1))


def split_o3(x: torch.Tensor, c: int, lmax: int) -> dict:
    """(..., 2*c*sum 3^L) -> {(s, L): (..., c, 3, .., 3)}, s-major then L (models/pure_cartesian.py:69-90)."""
    lead = x.shape[:-1]
    out, off = {}, 0
    for s in (0, 1):
        for L in range(lmax + 1):
            d = c * rank_dim(L)
            out[(s, L)] = x[..., off:off + d].reshape(*lead, c, *([3] * L))
            off += d
    return out


def merge_o3(blocks: dict, c: int, lmax: int) -> torch.Tensor:
    """Inverse of ``split_o3`` (models/pure_cartesian.py:109-120)."""
    lead = blocks[(0, 0)].shape[:-1]
    return torch.cat([blocks[(s, L)].reshape(*lead, c * rank_dim(L))
                      for s in (0, 1) for L in range(lmax + 1)], dim=-1)


# ----------------------------------------------------------------------------- geometry

def edge_vectors(pos, batch, src, dst, shifts, cell):
    """edge_vec = pos[dst] - pos[src] + shifts @ cell[batch[src]] (pure_cartesian_sparse_layers.py:751-756)."""
    shift_vec = torch.einsum("ni,nij->nj", shifts, cell[batch[src]])
    return pos[dst] - pos[src] + shift_vec


def rank_powers(vec: torch.Tensor, lmax: int) -> dict:
    """{0: 1, 1: n, L: n^{(x)L}} with n = vec / max(|vec|, 1e-8) (models/pure_cartesian.py:292-317)."""
    n = vec / vec.norm(dim=-1, keepdim=True).clamp(min=1e-8)
    out = {0: torch.ones(*vec.shape[:-1], 1, dtype=vec.dtype)}
    if lmax >= 1:
        out[1] = n
    for L in range(2, lmax + 1):
        out[L] = out[L - 1].unsqueeze(-1) * n.view(*vec.shape[:-1], *([1] * (L - 1)), 3)
    return out


def radial_embedding(r: torch.Tensor, cfg: SparseConfig) -> torch.Tensor:
    """soft_one_hot_linspace(r, 0, rc, nb, basis, cutoff=True) * sqrt(nb)."""
    return soft_one_hot_linspace(r, 0.0, cfg.max_radius, cfg.number_of_basis,
                                 basis=cfg.function_type, cutoff=True) * (cfg.number_of_basis ** 0.5)


def linear(x, p, key):
    return F.linear(x, p[key + ".weight"], p[key + ".bias"])


def radial_mlp(emb, p, prefix):
    """fc = Linear(nb,64) SiLU Linear(64,64) SiLU Linear(64,W) (pure_cartesian_sparse_layers.py:204-210)."""
    h = F.silu(linear(emb, p, prefix + ".0"))
    h = F.silu(linear(h, p, prefix + ".2"))
    return linear(h, p, prefix + ".4")


# ----------------------------------------------------------------------------- tensor product

@dataclass(frozen=True)
class Path:
    L1: int
    L2: int
    Lout: int


def sparse_paths(lmax: int, max_rank_other: int = 1) -> list:
    """k_policy "k0", no epsilon (models/pure_cartesian.py:353-418): delta-free outer products."""
    out = []
    for L1 in range(lmax + 1):
        for L2 in range(lmax + 1):
            if min(L1, L2) > max_rank_other:
                continue
            if L1 + L2 <= lmax:
                out.append(Path(L1, L2, L1 + L2))
    return out


def sparse_tp(x1: torch.Tensor, x2: torch.Tensor, w: torch.Tensor, c1: int, c2: int, cout: int,
              lmax: int) -> torch.Tensor:
    """Pseudo-zero sparse TP with per-edge weights (models/pure_cartesian.py:790-863).

    w: (E, P*cout*c1*c2) laid out [path][cout][c1][c2]; out (E, o3_dim(cout)).
    Path tensors are outer products t1[a, I] (x) t2[b, J] -> [a, b, I, J].
    """
    E = x1.shape[0]
    A = split_o3(x1, c1, lmax)
    B = split_o3(x2, c2, lmax)
    out = {}
    for s in (0, 1):
        for L in range(lmax + 1):
            out[(s, L)] = x1.new_zeros(E, cout, *([3] * L))
    per = cout * c1 * c2
    for k, pth in enumerate(sparse_paths(lmax)):
        Wp = w[:, k * per:(k + 1) * per].reshape(E, cout, c1, c2)
        t1 = A[(0, pth.L1)].reshape(E, c1, rank_dim(pth.L1))
        t2 = B[(0, pth.L2)].reshape(E, c2, rank_dim(pth.L2))
        outer = torch.einsum("eai,ebj->eabij", t1, t2).reshape(E, c1, c2, rank_dim(pth.Lout))
        msg = torch.einsum("ecab,eabk->eck", Wp, outer)
        out[(0, pth.Lout)] = out[(0, pth.Lout)] + msg.reshape(E, cout, *([3] * pth.Lout))
    return merge_o3(out, cout, lmax)


def scatter_sum(src: torch.Tensor, index: torch.Tensor, n: int) -> torch.Tensor:
    """index_add segment sum (utils/scatter.py:99-105)."""
    return src.new_zeros((n,) + src.shape[1:]).index_add(0, index, src)


class _Recomputed(torch.autograd.Function):
    """y = part(*inputs) that keeps only its inputs for the backward and recomputes part there (the
    per-edge intermediates of a chunk live only while that chunk's gradient is formed)."""

    @staticmethod
    def forward(ctx, part, *inputs):
        ctx.part = part
        ctx.save_for_backward(*inputs)
        with torch.no_grad():
            return part(*inputs)

    @staticmethod
    def backward(ctx, gy):
        inputs = [t.detach().requires_grad_(t.is_floating_point()) for t in ctx.saved_tensors]
        want = [t for t in inputs if t.requires_grad]
        with torch.enable_grad():
            y = ctx.part(*inputs)
        got = iter(torch.autograd.grad(y, want, gy, allow_unused=True))
        return (None,) + tuple(next(got) if t.requires_grad else None for t in inputs)


def edge_chunked(part, edge_chunk, dst, n_nodes, node_input, *edge_tensors):
    """scatter_sum(part(node_input, *edge_tensors), dst, n_nodes) for a `part` that returns per-edge messages.

    An evaluation device for large systems, not part of the algorithm: the edges are taken in chunks of
    `edge_chunk` whose per-edge intermediates (the materialised weights) are recomputed in the backward
    instead of stored, and each chunk's messages are added into the receiver sum as they come (the same
    sum in another order).  None: one chunk."""
    E = dst.shape[0]
    if edge_chunk is None or E <= edge_chunk:
        return scatter_sum(part(node_input, *edge_tensors), dst, n_nodes)
    out = None
    for a in range(0, E, edge_chunk):
        sl = [t[a:a + edge_chunk] for t in edge_tensors]
        msg = _Recomputed.apply(part, node_input, *sl)
        if out is None:
            out = msg.new_zeros((n_nodes,) + msg.shape[1:])
        # in place, and index_put_ saves no messages for the backward
        out.index_put_((dst[a:a + edge_chunk],), msg, accumulate=True)
    return out


# ----------------------------------------------------------------------------- convolutions

def atom_features(A, p, prefix="e3_conv_layers.0"):
    """Ai = atom_mlp(atom_embedding(A)) (pure_cartesian_sparse_layers.py:258-259)."""
    e = F.embedding(A.long(), p[prefix + ".atom_embedding.weight"])
    h = F.silu(linear(e, p, prefix + ".atom_mlp.0"))
    return linear(h, p, prefix + ".atom_mlp.2")


def conv1(A, vec, src, dst, n_nodes, p, cfg: SparseConfig, edge_chunk=None):
    """pure_cartesian_sparse_layers.py:227-330 (no external tensor, no fidelity)."""
    Ai = atom_features(A, p)
    cnt = scatter_sum(torch.ones_like(dst), dst, n_nodes).clamp(min=1).to(Ai.dtype)
    out = edge_chunked(lambda Ai, vec, src, dst: _conv1_msg(Ai, vec, src, dst, p, cfg), edge_chunk, dst, n_nodes,
                       Ai, vec, src, dst)
    return out / cnt.unsqueeze(-1)


def _conv1_msg(Ai, vec, src, dst, p, cfg: SparseConfig):
    C8, lmax, E = cfg.output_size, cfg.lmax, vec.shape[0]
    e = rank_powers(vec, lmax)
    a_src = Ai[src]
    f1 = {(0, 0): a_src, (1, 0): torch.zeros_like(a_src)}
    for L in range(1, lmax + 1):
        base = a_src.view(E, C8, *([1] * L)) * e[L].view(E, 1, *([3] * L))
        f1[(0, L)] = base
        f1[(1, L)] = torch.zeros_like(base)
    f_in = merge_o3(f1, C8, lmax)
    a_dst = Ai[dst]
    x2b = {(0, 0): a_dst, (1, 0): torch.zeros_like(a_dst)}
    for L in range(1, lmax + 1):
        z = a_dst.new_zeros(E, C8, *([3] * L))
        x2b[(0, L)] = z
        x2b[(1, L)] = z
    x2 = merge_o3(x2b, C8, lmax)
    emb = radial_embedding(vec.norm(dim=1), cfg)
    w = radial_mlp(emb, p, "e3_conv_layers.0.fc")
    return sparse_tp(f_in, x2, w, C8, C8, cfg.channels, lmax)


def conv2(f, vec, src, dst, n_nodes, p, layer: int, cfg: SparseConfig, avg_degree: float | None = None,
          edge_chunk=None):
    """pure_cartesian_sparse_layers.py:382-421: x1 = f[src], x2 = [1, n, n(x)n] with C2=1, / (E/N).

    ``avg_degree`` replaces E/N, so that a cluster cut out of a larger system is normalised like
    its parent system (the normalisation is the only non-local term of the trunk)."""
    E = vec.shape[0]
    out = edge_chunked(lambda f, vec, src: _conv2_msg(f, vec, src, p, layer, cfg), edge_chunk, dst, n_nodes,
                       f, vec, src)
    avg = out.new_tensor(E / max(n_nodes, 1) if avg_degree is None else avg_degree).clamp_min(1e-8)
    return out / avg


def _conv2_msg(f, vec, src, p, layer: int, cfg: SparseConfig):
    lmax, E = cfg.lmax, vec.shape[0]
    e = rank_powers(vec, lmax)
    eb = {(0, 0): e[0].view(E, 1), (1, 0): torch.zeros(E, 1, dtype=vec.dtype)}
    for L in range(1, lmax + 1):
        base = e[L].view(E, 1, *([3] * L))
        eb[(0, L)] = base
        eb[(1, L)] = torch.zeros_like(base)
    x2 = merge_o3(eb, 1, lmax)
    emb = radial_embedding(vec.norm(dim=1), cfg)
    w = radial_mlp(emb, p, f"e3_conv_layers.{layer}.fc")
    return sparse_tp(f[src], x2, w, cfg.channels, 1, cfg.channels, lmax)


# ----------------------------------------------------------------------------- readout

def invariant_bilinear(x, W: list, c: int, lmax: int):
    """Gram of true+pseudo blocks per rank, contracted with W[L] (pure_cartesian_sparse_layers.py:440-456)."""
    blocks = split_o3(x, c, lmax)
    N = x.shape[0]
    total = 0
    for L in range(lmax + 1):
        t0 = blocks[(0, L)].reshape(N, c, -1)
        t1 = blocks[(1, L)].reshape(N, c, -1)
        scale = 1.0 / math.sqrt(3 ** L) if L > 0 else 1.0
        gram = (t0 @ t0.transpose(1, 2) + t1 @ t1.transpose(1, 2)) * scale
        total = total + torch.einsum("ocd,ncd->no", W[L], gram)
    return total


def elementwise_0e(x, c: int, lmax: int):
    """<x_L, x_L> per channel over true and pseudo halves / sqrt(3^L) (models/pure_cartesian.py:146-195)."""
    b = split_o3(x, c, lmax)
    N = x.shape[0]
    outs = []
    for L in range(lmax + 1):
        t0 = b[(0, L)].reshape(N, c, -1)
        t1 = b[(1, L)].reshape(N, c, -1)
        outs.append(((t0 * t0).sum(-1) + (t1 * t1).sum(-1)) / math.sqrt(rank_dim(L)))
    return torch.cat(outs, dim=-1)


def main_net(x, p, prefix, n_hidden: int):
    """LayerNorm -> [Linear -> LayerNorm -> SiLU]* -> Linear (models/mlp.py:56-66)."""
    def ln(v, key):
        return F.layer_norm(v, (v.shape[-1],), p[key + ".weight"], p[key + ".bias"])
    h = ln(x, prefix + ".input_norm")
    for i in range(n_hidden):
        h = F.silu(ln(linear(h, p, f"{prefix}.layers.{i}"), f"{prefix}.layer_norms.{i}"))
    return linear(h, p, prefix + ".output")


def readout(features: list, p, cfg: SparseConfig):
    """pure_cartesian_sparse_layers.py:769-814 (no physical tensors, no long range)."""
    C, lmax, nL = cfg.channels, cfg.lmax, len(features)
    blocks = [split_o3(f, C, lmax) for f in features]
    comb = {k: torch.cat([b[k] for b in blocks], dim=1) for k in blocks[0]}
    f_comb = merge_o3(comb, C * nL, lmax)
    W = [p[f"product_3.W.{L}"] for L in range(lmax + 1)]
    f3 = invariant_bilinear(f_comb, W, C * nL, lmax)
    invs = [elementwise_0e(f, C, lmax) for f in features]
    f5 = torch.cat(invs + [f3 * f3], dim=-1)
    proj = main_net(f5, p, "proj_total", len(cfg.embed_size))
    return (proj * p["weighted_sum.weights"]).sum(dim=-1, keepdim=True)


# ----------------------------------------------------------------------------- trunk

def atom_energies(pos, A, batch, src, dst, shifts, cell, p: dict, cfg: SparseConfig,
                  avg_degree: float | None = None, edge_chunk=None):
    """(N, 1) atomic energies of the sparse trunk (pure_cartesian_sparse_layers.py:723-855)."""
    dtype = p["weighted_sum.weights"].dtype
    pos, cell, shifts = pos.to(dtype), cell.to(dtype), shifts.to(dtype)
    order = torch.argsort(dst, stable=True)
    src, dst, shifts = src[order], dst[order], shifts[order]
    vec = edge_vectors(pos, batch, src, dst, shifts, cell)
    N = pos.shape[0]
    feats = [conv1(A, vec, src, dst, N, p, cfg, edge_chunk)]
    for layer in range(1, cfg.num_interaction):
        feats.append(conv2(feats[-1], vec, src, dst, N, p, layer, cfg, avg_degree, edge_chunk))
    return readout(feats, p, cfg)


def energy_forces(pos, A, batch, src, dst, shifts, cell, p: dict, cfg: SparseConfig, edge_chunk=None):
    """(per-atom energies (N,), forces (N,3)) with F = -dE/dpos."""
    pos = pos.detach().clone().requires_grad_(True)
    e = atom_energies(pos, A, batch, src, dst, shifts, cell, p, cfg, edge_chunk=edge_chunk)
    (g,) = torch.autograd.grad(e.sum(), pos)
    return e.detach().squeeze(-1), -g


def param_shapes(cfg: SparseConfig) -> list:
    """(key, shape) of every parameter of the reference trunk, in registration order."""
    C, C8, nb, H = cfg.channels, cfg.output_size, cfg.number_of_basis, cfg.radial_hidden
    n_paths = len(sparse_paths(cfg.lmax))
    out = [
        ("e3_conv_layers.0.atom_embedding.weight", (cfg.max_atomvalue, cfg.embedding_dim)),
        ("e3_conv_layers.0.atom_mlp.0.weight", (64, cfg.embedding_dim)),
        ("e3_conv_layers.0.atom_mlp.0.bias", (64,)),
        ("e3_conv_layers.0.atom_mlp.2.weight", (C8, 64)),
        ("e3_conv_layers.0.atom_mlp.2.bias", (C8,)),
    ]
    for layer in range(cfg.num_interaction):
        wn = n_paths * C * (C8 * C8 if layer == 0 else C)
        pre = f"e3_conv_layers.{layer}.fc"
        out += [(pre + ".0.weight", (H, nb)), (pre + ".0.bias", (H,)),
                (pre + ".2.weight", (H, H)), (pre + ".2.bias", (H,)),
                (pre + ".4.weight", (wn, H)), (pre + ".4.bias", (wn,))]
    S = (cfg.num_interaction - 1) * cfg.invariant_channels
    CC = C * cfg.num_interaction
    out += [(f"product_3.W.{L}", (S, CC, CC)) for L in range(cfg.lmax + 1)]
    fin = cfg.num_interaction * C * (cfg.lmax + 1) + S
    out += [("proj_total.input_norm.weight", (fin,)), ("proj_total.input_norm.bias", (fin,))]
    prev = fin
    for i, h in enumerate(cfg.embed_size):
        out += [(f"proj_total.layers.{i}.weight", (h, prev)), (f"proj_total.layers.{i}.bias", (h,)),
                (f"proj_total.layer_norms.{i}.weight", (h,)), (f"proj_total.layer_norms.{i}.bias", (h,))]
        prev = h
    out += [("proj_total.output.weight", (17, prev)), ("proj_total.output.bias", (17,)),
            ("weighted_sum.weights", (17,))]
    return out
