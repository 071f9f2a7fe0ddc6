"""Differentiable formulations of the light ops of the trunks, for force-loss training.

A force loss (training/trainer.py:1292-1297: F = -dE/dpos with create_graph=True, then loss.backward())
differentiates the whole energy twice, parameters included.  In ``train()`` mode the trunks therefore
build the step from:

* the conv2..n tensor products on their HIP kernels (``sparse_conv`` / ``ictd_conv``), whose C++ autograd
  gives the parameter gradients and a differentiable backward (the analogues of the reference's
  double-backward kernels, csrc/ictd_tp_cuda.cu:536-971): these carry almost all of the step's work;
* the functions below for the rest: edge geometry, radial basis and radial MLP, ICTD direction harmonics,
  the conv1 species-pair contraction and the readout's Gram bilinear and squared norms.  They are the same
  formulas as the inference kernels (``edge_radial.hip``, ``sparse_conv.hip`` conv1, ``ictd_conv.hip`` conv1,
  ``gram_readout.hip``, ``readout_gather.hip``) written as torch operations on the GPU, so autograd
  differentiates them to any order; the inference kernels stay the energy/force path.

Every function takes the receiver-sorted graph of ``fsctep_amd.graph`` and works on the internal layouts
(sparse x[N][13][C], ICTD x[N][M][C]).
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from .graph import Graph


# ------------------------------------------------------------------ edge geometry (edge_radial.hip)
def edge_geometry(pos, shift_vec, g: Graph):
    """vec = pos[dst] - pos[src] + shift, r = |vec|, n = vec / max(r, 1e-8) over the receiver-sorted edges
    (models/pure_cartesian_sparse_layers.py:751-756)."""
    vec = pos.index_select(0, g.dst) - pos.index_select(0, g.src) + shift_vec
    return _unit(vec)


def edge_vec_geometry(edge_vec, g: Graph):
    """The same from caller edge vectors (in the caller's edge order)."""
    return _unit(edge_vec.index_select(0, g.order.long()))


def _unit(vec):
    r = vec.norm(dim=1)
    return vec / r.clamp(min=1e-8).unsqueeze(-1), r


# ------------------------------------------------------------------ radial basis and MLP
def radial_basis(r, r_cut: float, nb: int, basis: str):
    """soft_one_hot_linspace(r, 0, r_cut, nb, basis, cutoff=True) * sqrt(nb) (e3nn's published definition,
    restated; models/pure_cartesian_sparse_layers.py:319-321).  Where a branch is cut off the value is a
    select of a finite expression, so every derivative stays finite."""
    step = r_cut / (nb + 1)
    k = torch.arange(1, nb + 1, dtype=r.dtype, device=r.device)
    x = r.unsqueeze(-1)
    if basis in ("bessel", "fourier"):
        inside = (x > 0) & (x < r_cut)
        xs = torch.where(inside, x, torch.full_like(x, 0.5 * r_cut))
        s = torch.sin(k * (math.pi / r_cut) * xs)
        if basis == "bessel":
            val = math.sqrt(2.0 / r_cut) * s / xs
        else:
            val = s / math.sqrt(0.25 + nb / 2)
        out = torch.where(inside, val, torch.zeros_like(val))
    else:
        d = (x - k * step) / step
        if basis == "gaussian":
            out = torch.exp(-d * d) / 1.12
        elif basis == "cosine":
            inside = (d > -1) & (d < 1)
            out = torch.where(inside, torch.cos(0.5 * math.pi * d), torch.zeros_like(d))
        elif basis == "smooth_finite":
            inside = (d > -1) & (d < 1)
            q = torch.where(inside, 1 - d * d, torch.ones_like(d))
            out = torch.where(inside, 1.14136 * math.exp(2.0) * torch.exp(-2.0 / q), torch.zeros_like(d))
        else:
            raise ValueError(f"radial basis {basis!r}")
    return out * math.sqrt(nb)


def radial_hidden(r, fc, r_cut: float, basis: str):
    """fc[:4](emb): silu(fc[2](silu(fc[0](emb)))) (E, 64)."""
    emb = radial_basis(r, r_cut, fc[0].in_features, basis)
    return F.silu(fc[2](F.silu(fc[0](emb))))


def radial_full(r, fc, r_cut: float, basis: str):
    """The whole radial MLP fc(emb) (E, P)."""
    return fc[4](radial_hidden(r, fc, r_cut, basis))


# ------------------------------------------------------------------ ICTD direction harmonics
_HARM = {}


def harmonics(n, lmax: int):
    """Y (E, (lmax+1)^2): block l at l^2, Y_l = sum over degree-l monomials n_x^a n_y^b n_z^c of
    multinomial * (G_l B_l) (models/ictd_irreps.py:371-402), the table edge_harmonics uses."""
    from .ictd_basis import harmonic_projection
    key = (lmax, str(n.device), n.dtype)
    if key not in _HARM:
        blocks = []
        for l in range(lmax + 1):
            exps, coef, P = harmonic_projection(l)
            M = torch.tensor(coef[:, None] * P, dtype=n.dtype, device=n.device)        # (monomials, 2l+1)
            blocks.append(([tuple(int(v) for v in e) for e in exps], M))
        _HARM[key] = blocks
    ones = torch.ones_like(n[:, 0])
    pw = []                                        # pw[axis][p] = n_axis^p, p <= lmax
    for axis in range(3):
        col = [ones]
        for _ in range(lmax):
            col.append(col[-1] * n[:, axis])
        pw.append(col)
    out = []
    for exps, M in _HARM[key]:
        mono = torch.stack([pw[0][a] * pw[1][b] * pw[2][c] for (a, b, c) in exps], dim=1)
        out.append(mono @ M)
    return torch.cat(out, dim=1)


# ------------------------------------------------------------------ conv1 (species-pair contractions)
_SPARSE_CONV1_PATHS = (0, 3, 5)       # (0,0->0), (1,0->1), (2,0->2): the paths with a rank-0 second operand


def sparse_conv1(h, n, w_last, b_last, atab, g: Graph, channels: int):
    """Sparse conv1 (models/pure_cartesian_sparse_layers.py:227-330) from the radial hidden h (E, 64):
    with W_e = h_e w_last^T + b_last in the [path][Cout][C1][C2] layout, x1 = A_src (x) n^L and x2 = A_dst,
    the message of rank L is Q_e[L][c] n^{(x)L}, Q_e[L][c] = sum_ab W_e[p_L][c][a][b] A_src[a] A_dst[b]
    = h_e . T[pair][L][c] + Tb[pair][L][c], summed to receivers / max(in-degree, 1).  The per-pair
    products run over the graph's 16-edge species-pair tiles (one batched GEMM)."""
    C, NS = channels, g.n_species
    K = h.shape[1]
    c8 = atab.shape[1]
    idx = torch.tensor(_SPARSE_CONV1_PATHS, device=h.device)
    W4 = w_last.view(6, C, c8, c8, K).index_select(0, idx)                       # (3, C, a, b, k)
    B4 = b_last.view(6, C, c8, c8).index_select(0, idx)
    T = torch.einsum("lcabk,sa,tb->stklc", W4, atab, atab).reshape(NS * NS, K, 3 * C)   # columns (L, c)
    Tb = torch.einsum("lcab,sa,tb->stlc", B4, atab, atab).reshape(NS * NS, 3 * C)
    E = h.shape[0]
    nt = g.pair_tiles.shape[0] // 17
    ids = g.pair_tiles[:16 * nt].view(nt, 16).long()
    tile_pair = g.pair_tiles[16 * nt:].long()
    valid = ids >= 0
    ht = h.index_select(0, ids.clamp(min=0).reshape(-1)).view(nt, 16, K) * valid.unsqueeze(-1).to(h.dtype)
    qt = torch.bmm(ht, T.index_select(0, tile_pair))                            # (nt, 16, 3C)
    slot = torch.where(valid, ids, torch.full_like(ids, E)).reshape(-1)
    Q = h.new_zeros(E + 1, 3 * C).index_copy(0, slot, qt.reshape(-1, 3 * C))[:E]
    Q = (Q + Tb.index_select(0, g.edge_pair.long())).view(E, 3, C)
    nn_ = (n.unsqueeze(-1) * n.unsqueeze(-2)).reshape(E, 9)
    msg = torch.cat([Q[:, 0:1, :], Q[:, 1:2, :] * n.unsqueeze(-1), Q[:, 2:3, :] * nn_.unsqueeze(-1)], dim=1)
    return _receiver_mean(msg, g)


def ictd_conv1(Fe, gates, qtab, g: Graph, layout):
    """ICTD conv1 (models/pure_cartesian_ictd_layers_full.py:341-473, _o3.py:424-532): for each live path
    (l, canonical) x (0e) -> (l, canonical), whose coupling is the identity, the message of component k of
    the output block is gate[e][p] Q[pair][p] F[e][l^2 + k], Q[pair][p][o] = sum_ij W1[p][o][i][j] A_src[i]
    A_dst[j]; summed to receivers / max(in-degree, 1)."""
    E = Fe.shape[0]
    C = qtab.shape[2]
    Qe = qtab.index_select(0, g.edge_pair.long())                                 # (E, NP1, C)
    msg = Fe.new_zeros(E, layout.M, C)
    parts = []
    for i, p in enumerate(layout.conv1_paths()):
        w = gates[:, p["gate"]].unsqueeze(-1) * Qe[:, i, :]                       # (E, C)
        parts.append((p["oo"], p["d"], Fe[:, p["oy"]:p["oy"] + p["d"]].unsqueeze(-1) * w.unsqueeze(1)))
    msg = _place(msg, parts)
    return _receiver_mean(msg, g)


def _place(buf, parts):
    """buf with the (offset, width, block) parts written along dim 1 (differentiable, no in-place update
    of a tensor autograd needs)."""
    pieces, pos = [], 0
    for off, d, blk in sorted(parts, key=lambda t: t[0]):
        if off > pos:
            pieces.append(buf[:, pos:off])
        pieces.append(blk)
        pos = off + d
    if pos < buf.shape[1]:
        pieces.append(buf[:, pos:])
    return torch.cat(pieces, dim=1)


def _receiver_mean(msg, g: Graph):
    N = g.n_nodes
    deg = (g.dst_ptr[1:] - g.dst_ptr[:-1]).to(msg.dtype).clamp(min=1)
    out = msg.new_zeros((N,) + tuple(msg.shape[1:])).index_add(0, g.dst, msg)
    return out / deg.view(-1, *([1] * (msg.dim() - 1)))


# ------------------------------------------------------------------ readout (gram_readout.hip, readout_gather.hip)
def gram_bilinear(t, W, scale: float):
    """out[n][o] = scale sum_ij W[o][i][j] sum_m t[n][m][i] t[n][m][j] for t (N, D, nC), W (S, nC, nC)."""
    N, D, nC = t.shape
    S = W.shape[0]
    tw = torch.matmul(t.reshape(N * D, nC), W.permute(1, 0, 2).reshape(nC, S * nC))   # (N D, S nC): t_i W[o][i][j]
    return scale * (tw.view(N, D, S, nC) * t.unsqueeze(2)).sum(dim=(1, 3))


def readout_features(feats, Ws, scales, maps):
    """(scalars (N, S) = sum_k gram_bilinear(t_k, W_k, scale_k), sq (N, n_keys, n_layers*C)), the readout
    op's outputs: t_k are the Gram inputs the readout maps lay out (srcmap over the layers' flattened
    features), sq[n][k][l*C + c] = sum over the components m of key k of X_l[n][m][c]^2."""
    N = feats[0].shape[0]
    srcmap, _ = maps.on(feats[0].device)
    X = torch.cat([f.reshape(N, -1) for f in feats], dim=1)
    T = X.index_select(1, srcmap.long())
    nC = maps.n_layers * maps.C
    scalars, off, sqs, comp = 0, 0, [], 0
    for k, d in enumerate(maps.key_dims):
        t = T[:, off:off + d * nC].view(N, d, nC)
        scalars = scalars + gram_bilinear(t, Ws[k], scales[k])
        off += d * nC
        sqs.append(torch.cat([(f[:, comp:comp + d, :] ** 2).sum(1) for f in feats], dim=1))
        comp += d
    return scalars, torch.stack(sqs, dim=1)
