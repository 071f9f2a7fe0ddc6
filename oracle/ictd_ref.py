"""CPU oracle for the ICTD trunks, ``pure-cartesian-ictd`` and ``-o3`` (test infrastructure only).

A restatement in plain PyTorch of the reference algorithm:
  * harmonic ("ICTD") basis: null space of the Laplacian on Sym^L, orthonormalised under the
    isotropic-Gaussian Gram matrix            models/ictd_irreps.py:144-185, models/ictd_fast.py:41-114
  * trace-chain projectors via r^{2k} lifts    models/ictd_irreps.py:229-254, models/ictd_fast.py:240-266
  * CG tensors by polynomial multiplication    models/ictd_irreps.py:531-581 (normalisation :869-876)
  * direction harmonics                        models/ictd_irreps.py:278-300, 371-402, 489-494
  * fully connected TP with per-path gates     models/ictd_irreps.py:971-1253 (O3 keys :1325-1695),
    evaluated per path as the reference's fallback einsum (:1224-1251)
  * conv1 / conv2..n / readout                 models/pure_cartesian_ictd_layers_full.py:341-473, 867-1078
                                               models/pure_cartesian_ictd_layers_o3.py:424-532, 902-1074
  * rank-1 external field embedding            models/pure_cartesian_ictd_layers.py:155-379
Irreps are keyed (l, parity); the "full" trunk is the O(3) one restricted to the canonical
parities (-1)^l, which the path rule p3 = p1*p2 preserves.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from functools import lru_cache

import torch
import torch.nn.functional as F

from .radial import soft_one_hot_linspace
from .sparse_ref import edge_chunked
from .sparse_ref import linear, main_net, edge_vectors, scatter_sum

# ----------------------------------------------------------------------------- basis (float64)


def counts(L: int) -> list:
    """Monomials x^a y^b z^c of degree L in the reference order (models/ictd_fast.py:41-48)."""
    return [(a, b, L - a - b) for a in range(L + 1) for b in range(L - a + 1)]


def sym_dim(L: int) -> int:
    return (L + 1) * (L + 2) // 2


def laplacian(L: int) -> torch.Tensor:
    """Delta: Sym^L -> Sym^{L-2} on monomial coefficients (models/ictd_fast.py:87-114)."""
    dst = {t: i for i, t in enumerate(counts(L - 2))}
    D = torch.zeros(len(dst), sym_dim(L), dtype=torch.float64)
    for col, (a, b, c) in enumerate(counts(L)):
        if a >= 2:
            D[dst[(a - 2, b, c)], col] += a * (a - 1)
        if b >= 2:
            D[dst[(a, b - 2, c)], col] += b * (b - 1)
        if c >= 2:
            D[dst[(a, b, c - 2)], col] += c * (c - 1)
    return D


def _gauss_moment(n: int) -> float:
    if n % 2:
        return 0.0
    out = 1
    for k in range(n - 1, 0, -2):
        out *= k
    return float(out)


@lru_cache(maxsize=None)
def gram(L: int) -> torch.Tensor:
    """<x^a y^b z^c, x^a' y^b' z^c'> under the standard Gaussian (models/ictd_irreps.py:144-159)."""
    cs = counts(L)
    G = torch.zeros(len(cs), len(cs), dtype=torch.float64)
    for i, (a, b, c) in enumerate(cs):
        for j, (a2, b2, c2) in enumerate(cs):
            G[i, j] = _gauss_moment(a + a2) * _gauss_moment(b + b2) * _gauss_moment(c + c2)
    return G


@lru_cache(maxsize=None)
def harmonic_basis(L: int) -> torch.Tensor:
    """(Dsym(L), 2L+1): ker(Delta), symmetrically orthonormalised under gram(L) (models/ictd_irreps.py:162-185)."""
    if L == 0:
        return torch.ones(1, 1, dtype=torch.float64)
    if L == 1:
        return torch.eye(3, dtype=torch.float64)
    _, s, vh = torch.linalg.svd(laplacian(L), full_matrices=True)
    rank = int((s > 1e-12).sum())
    B = vh[rank:].T.contiguous()
    ev, U = torch.linalg.eigh(B.T @ gram(L) @ B)
    return B @ (U @ torch.diag(ev.clamp(min=1e-14).rsqrt()) @ U.T)


def lift(l: int, k: int) -> torch.Tensor:
    """Multiplication by (x^2+y^2+z^2)^k: Sym^l -> Sym^{l+2k} (models/ictd_fast.py:240-266)."""
    src = counts(l)
    if k == 0:
        return torch.eye(len(src), dtype=torch.float64)
    dst = {t: i for i, t in enumerate(counts(l + 2 * k))}
    M = torch.zeros(len(dst), len(src), dtype=torch.float64)
    for col, (a, b, c) in enumerate(src):
        for u in range(k + 1):
            for v in range(k - u + 1):
                w = k - u - v
                coef = math.factorial(k) / (math.factorial(u) * math.factorial(v) * math.factorial(w))
                M[dst[(a + 2 * u, b + 2 * v, c + 2 * w)], col] += coef
    return M


@lru_cache(maxsize=None)
def projector(L: int, l: int) -> torch.Tensor:
    """(2l+1, Dsym(L)) Gram-weighted least-squares coordinates of r^{L-l} Harm^l (models/ictd_irreps.py:229-254)."""
    V = lift(l, (L - l) // 2) @ harmonic_basis(l)
    G = gram(L)
    return torch.linalg.solve(V.T @ G @ V, V.T @ G)


@lru_cache(maxsize=None)
def cg_raw(l1: int, l2: int, l3: int) -> torch.Tensor:
    """C[m1,m2,m3]: project the product polynomial (degree l1+l2) onto Harm^l3 (models/ictd_irreps.py:550-581)."""
    if not (abs(l1 - l2) <= l3 <= l1 + l2) or (l1 + l2 + l3) % 2:
        return torch.zeros(2 * l1 + 1, 2 * l2 + 1, 2 * l3 + 1, dtype=torch.float64)
    L = l1 + l2
    idx = {t: i for i, t in enumerate(counts(L))}
    c1, c2 = counts(l1), counts(l2)
    Mp = torch.zeros(len(idx), len(c1) * len(c2), dtype=torch.float64)
    for i, u in enumerate(c1):
        for j, v in enumerate(c2):
            Mp[idx[(u[0] + v[0], u[1] + v[1], u[2] + v[2])], i * len(c2) + j] = 1.0
    B1, B2 = harmonic_basis(l1), harmonic_basis(l2)
    outer = torch.einsum("im,jn->ijmn", B1, B2).reshape(len(c1) * len(c2), -1)
    c3 = projector(L, l3) @ (Mp @ outer)
    return c3.T.reshape(2 * l1 + 1, 2 * l2 + 1, 2 * l3 + 1).contiguous()


@lru_cache(maxsize=None)
def cg(l1: int, l2: int, l3: int) -> torch.Tensor:
    """"component" normalisation: C * sqrt(2 l3 + 1) / ||C||_F (models/ictd_irreps.py:869-876)."""
    C = cg_raw(l1, l2, l3)
    f = float(C.norm())
    return C * (math.sqrt(2 * l3 + 1) / f) if f > 1e-30 else C


def direction_harmonics(n: torch.Tensor, l: int) -> torch.Tensor:
    """Y_l(n) = B_l^T G_l t(n), t_abc = multinomial * n_x^a n_y^b n_z^c (models/ictd_irreps.py:278-300)."""
    if l == 0:
        return torch.ones(*n.shape[:-1], 1, dtype=n.dtype)
    cols = []
    for a, b, c in counts(l):
        coef = math.factorial(l) / (math.factorial(a) * math.factorial(b) * math.factorial(c))
        cols.append(coef * n[..., 0] ** a * n[..., 1] ** b * n[..., 2] ** c)
    t = torch.stack(cols, dim=-1)
    P = (gram(l) @ harmonic_basis(l)).to(n.dtype)
    return t @ P


# ----------------------------------------------------------------------------- tensor product

def tp_paths(keys1, keys2, keys_out, lmax) -> list:
    """(l1,p1,l2,p2,l3,p3) in the reference enumeration order (models/ictd_irreps.py:781-788, :1371-1380)."""
    out_set = set(keys_out)
    paths = []
    for l1, p1 in keys1:
        for l2, p2 in keys2:
            for l3 in range(abs(l1 - l2), min(l1 + l2, lmax) + 1):
                if (l1 + l2 + l3) % 2:
                    continue
                if (l3, p1 * p2) in out_set:
                    paths.append((l1, p1, l2, p2, l3, p1 * p2))
    return paths


def fctp(x1: dict, x2: dict, W: torch.Tensor, gates: torch.Tensor, paths, keys_out) -> dict:
    """out[k3][e,o,m3] = sum_p gate[e,p] sum_{i,j,m1,m2} W[p,o,i,j] x1[k1][e,i,m1] x2[k2][e,j,m2] C[m1,m2,m3]."""
    some = next(iter(x1.values()))
    E = some.shape[0]
    out = {k: some.new_zeros(E, W.shape[1], 2 * k[0] + 1) for k in keys_out}
    for p, (l1, p1, l2, p2, l3, p3) in enumerate(paths):
        a, b = x1.get((l1, p1)), x2.get((l2, p2))
        if a is None or b is None:
            continue
        C = cg(l1, l2, l3).to(a.dtype)
        y = torch.einsum("eim,ejn,mnk,oij->eok", a, b, C, W[p])
        out[(l3, p3)] = out[(l3, p3)] + y * gates[:, p, None, None]
    return out


# ----------------------------------------------------------------------------- trunk

@dataclass(frozen=True)
class ICTDConfig:
    channels: int = 64
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
    o3: bool = False                  # False: pure-cartesian-ictd; True: pure-cartesian-ictd-o3
    active: tuple = ()                # O3 active irreps ((l, p), ...) sorted (l, even first); () -> canonical
    external_field: bool = False      # rank-1 "1o" external field injected in conv1
    dipole: bool = False              # physical tensor head "dipole" on 1o, reduce sum


def active_keys(cfg: ICTDConfig) -> list:
    if cfg.o3 and cfg.active:
        return sorted(set(cfg.active), key=lambda k: (k[0], 0 if k[1] > 0 else 1))
    return [(l, 1 if l % 2 == 0 else -1) for l in range(cfg.lmax + 1)]


def key_str(k) -> str:
    return f"{k[0]}{'e' if k[1] > 0 else 'o'}"


def paths_conv1(cfg):
    k = active_keys(cfg)
    return tp_paths(k, k, k, cfg.lmax)


def paths_conv2(cfg):
    k = active_keys(cfg)
    return tp_paths(k, k, k, cfg.lmax)


def split_keys(x: torch.Tensor, C: int, keys) -> dict:
    out, off = {}, 0
    for k in keys:
        d = C * (2 * k[0] + 1)
        out[k] = x[..., off:off + d].reshape(*x.shape[:-1], C, 2 * k[0] + 1)
        off += d
    return out


def merge_keys(blocks: dict, keys) -> torch.Tensor:
    return torch.cat([blocks[k].reshape(*blocks[k].shape[:-2], blocks[k].shape[-2] * blocks[k].shape[-1])
                      for k in keys], dim=-1)


def radial_embedding(r, cfg):
    return soft_one_hot_linspace(r, 0.0, cfg.max_radius, cfg.number_of_basis, basis=cfg.function_type,
                                 cutoff=True) * (cfg.number_of_basis ** 0.5)


def radial_mlp(emb, p, prefix):
    h = F.silu(linear(emb, p, prefix + ".0"))
    h = F.silu(linear(h, p, prefix + ".2"))
    return linear(h, p, prefix + ".4")


def conv1(A, n, r, src, dst, batch, N, p, cfg, ext_field=None, edge_chunk=None):
    """ICTDIrrepsE3Conv.forward (full :341-473) / ICTDO3E3Conv.forward (o3 :424-532)."""
    e = F.embedding(A.long(), p["e3_conv_emb.atom_embedding.weight"])
    Ai = linear(F.silu(linear(e, p, "e3_conv_emb.atom_mlp.0")), p, "e3_conv_emb.atom_mlp.2")
    cnt = scatter_sum(torch.ones_like(dst), dst, N).clamp(min=1).to(Ai.dtype)
    eb = batch[src]
    out = edge_chunked(lambda Ai, n, r, src, dst, eb: _conv1_msg(Ai, n, r, src, dst, eb, p, cfg, ext_field),
                       edge_chunk, dst, N, Ai, n, r, src, dst, eb)
    return out / cnt.unsqueeze(-1)


def _conv1_msg(Ai, n, r, src, dst, edge_batch, p, cfg, ext_field):
    keys = active_keys(cfg)
    E = n.shape[0]
    C8 = cfg.output_size
    f_in = {k: Ai.new_zeros(E, C8, 2 * k[0] + 1) for k in keys}
    for l in range(cfg.lmax + 1):
        k = (l, 1 if l % 2 == 0 else -1)
        if k in f_in:
            f_in[k] = Ai[src].unsqueeze(-1) * direction_harmonics(n, l).unsqueeze(-2)
    if ext_field is not None:
        # rank-1 cartesian field -> l=1 block in monomial order (z, y, x) (pure_cartesian_ictd_layers.py:68-110,303-379)
        t = ext_field[:, [2, 1, 0]][edge_batch].unsqueeze(-2) * Ai[src].unsqueeze(-1)
        if cfg.o3:
            scale = p["e3_conv_emb.external_tensor_scale_by_irrep"][keys.index((1, -1))]
        else:
            scale = p["e3_conv_emb.external_tensor_scale_by_l"][1]
        f_in[(1, -1)] = f_in[(1, -1)] + t * scale
    x2 = {k: Ai.new_zeros(E, C8, 2 * k[0] + 1) for k in keys}
    x2[(0, 1)] = Ai[dst].unsqueeze(-1)
    gates = radial_mlp(radial_embedding(r, cfg), p, "e3_conv_emb.fc")
    out = fctp(f_in, x2, p["e3_conv_emb.tp2.weight"], gates, paths_conv1(cfg), keys)
    return merge_keys(out, keys)


def conv2(f, n, r, src, dst, N, p, layer, cfg, edge_chunk=None):
    """conv2..n loop (full :938-954, o3 :956-973): gates = fc2(emb), x2 = Y_l, / in-degree."""
    cnt = scatter_sum(torch.ones_like(dst), dst, N).clamp(min=1).to(f.dtype)
    out = edge_chunked(lambda f, n, r, src: _conv2_msg(f, n, r, src, p, layer, cfg), edge_chunk, dst, N,
                       f, n, r, src)
    return out / cnt.unsqueeze(-1)


def _conv2_msg(f, n, r, src, p, layer, cfg):
    keys = active_keys(cfg)
    x1 = {k: v[src] for k, v in split_keys(f, cfg.channels, keys).items()}
    Y = {}
    for l in range(cfg.lmax + 1):
        k = (l, 1 if l % 2 == 0 else -1)
        if k in keys:
            Y[k] = direction_harmonics(n, l).unsqueeze(-2)
    gates = radial_mlp(radial_embedding(r, cfg), p, f"fc2_layers.{layer}")
    out = fctp(x1, Y, p[f"tp2_layers.{layer}.weight"], gates, paths_conv2(cfg), keys)
    return merge_keys(out, keys)


def wread_key(cfg, k) -> str:
    return f"W_read.{key_str(k)}" if cfg.o3 else f"W_read.{k[0]}"


def readout(features, p, cfg, batch=None):
    """Gram bilinear + 0e products + MainNet + weighted sum (full :977-1033, o3 :1005-1030)."""
    keys = active_keys(cfg)
    nC = cfg.channels * cfg.num_interaction
    xb = split_keys(torch.cat(features, dim=-1), nC, keys)
    scalars = 0
    for k in keys:
        t = xb[k]
        g = torch.einsum("ncm,ndm->ncd", t, t) / math.sqrt(2 * k[0] + 1)
        scalars = scalars + torch.einsum("ocd,ncd->no", p[wread_key(cfg, k)], g)
    splits = [split_keys(f, cfg.channels, keys) for f in features]
    outs = []
    for k in keys:
        T = torch.cat([s[k] for s in splits], dim=-2)
        if k == (0, 1):
            T = torch.cat([T, scalars.unsqueeze(-1)], dim=-2)
        factor = float(cg_raw(k[0], k[0], 0)[0, 0, 0] / cg_raw(k[0], k[0], 0).norm())
        outs.append((T * T).sum(-1) * factor)
    f5 = torch.cat(outs, dim=-1)
    proj = main_net(f5, p, "proj_total", len(cfg.embed_size))
    e = (proj * p["weighted_sum.weights"]).sum(dim=-1, keepdim=True)
    dip = None
    if cfg.dipole:
        y = torch.einsum("ncm,oc->nom", xb[(1, -1)], p["physical_tensor_heads.dipole.1.weight"])
        G = int(batch.max()) + 1 if batch.numel() else 0
        dip = scatter_sum(y, batch, G)
    return e, dip


def forward(pos, A, batch, src, dst, shifts, cell, p, cfg, ext_field=None, edge_chunk=None):
    """(atomic energies (N,1), dipole (G,1,3) or None); ``edge_chunk`` as in sparse_ref.edge_chunked."""
    dtype = p["weighted_sum.weights"].dtype
    pos, cell, shifts = pos.to(dtype), cell.to(dtype), shifts.to(dtype)
    order = torch.argsort(dst, stable=True)
    src, dst, shifts = src[order], dst[order], shifts[order]
    vec = edge_vectors(pos, batch, src, dst, shifts, cell)
    r = vec.norm(dim=1)
    n = vec / r.clamp(min=1e-8).unsqueeze(-1)
    N = pos.shape[0]
    feats = [conv1(A, n, r, src, dst, batch, N, p, cfg, ext_field, edge_chunk)]
    for layer in range(cfg.num_interaction - 1):
        feats.append(conv2(feats[-1], n, r, src, dst, N, p, layer, cfg, edge_chunk))
    return readout(feats, p, cfg, batch)


def energy_forces(pos, A, batch, src, dst, shifts, cell, p, cfg, ext_field=None, edge_chunk=None):
    pos = pos.detach().clone().requires_grad_(True)
    e, dip = forward(pos, A, batch, src, dst, shifts, cell, p, cfg, ext_field, edge_chunk)
    (g,) = torch.autograd.grad(e.sum(), pos)
    return e.detach().squeeze(-1), -g, (dip.detach() if dip is not None else None)


def param_shapes(cfg: ICTDConfig) -> list:
    """(key, shape) of the trunk's parameters (state_dict order of the reference classes)."""
    keys = active_keys(cfg)
    C, C8, nb = cfg.channels, cfg.output_size, cfg.number_of_basis
    P1, P2 = len(paths_conv1(cfg)), len(paths_conv2(cfg))
    nC = C * cfg.num_interaction
    S = (cfg.num_interaction - 1) * cfg.invariant_channels
    out = [("e3_conv_emb.atom_embedding.weight", (cfg.max_atomvalue, cfg.embedding_dim)),
           ("e3_conv_emb.atom_mlp.0.weight", (64, cfg.embedding_dim)), ("e3_conv_emb.atom_mlp.0.bias", (64,)),
           ("e3_conv_emb.atom_mlp.2.weight", (C8, 64)), ("e3_conv_emb.atom_mlp.2.bias", (C8,)),
           ("e3_conv_emb.tp2.weight", (P1, C, C8, C8))]
    for pre, P in [("e3_conv_emb.fc", P1)] + [(f"fc2_layers.{i}", P2) for i in range(cfg.num_interaction - 1)]:
        out += [(pre + ".0.weight", (64, nb)), (pre + ".0.bias", (64,)), (pre + ".2.weight", (64, 64)),
                (pre + ".2.bias", (64,)), (pre + ".4.weight", (P, 64)), (pre + ".4.bias", (P,))]
    if cfg.external_field:
        if cfg.o3:
            out.append(("e3_conv_emb.external_tensor_scale_by_irrep", (len(keys),)))
        else:
            out.append(("e3_conv_emb.external_tensor_scale_by_l", (cfg.lmax + 1,)))
    out += [(f"tp2_layers.{i}.weight", (P2, C, C, 1)) for i in range(cfg.num_interaction - 1)]
    out += [(wread_key(cfg, k), (S, nC, nC)) for k in keys]
    out += [("readout_linear.0.weight", (cfg.embed_size[0], S + nC * len(keys))),
            ("readout_linear.0.bias", (cfg.embed_size[0],)),
            ("readout_linear.2.weight", (17, cfg.embed_size[0])), ("readout_linear.2.bias", (17,)),
            ("weighted_sum.weights", (17,))]
    fin = cfg.num_interaction * C * len(keys) + S
    out += [("proj_total.input_norm.weight", (fin,)), ("proj_total.input_norm.bias", (fin,))]
    prev = fin
    for i, h in enumerate(cfg.embed_size):
        out += [(f"proj_total.layers.{i}.weight", (h, prev)), (f"proj_total.layers.{i}.bias", (h,)),
                (f"proj_total.layer_norms.{i}.weight", (h,)), (f"proj_total.layer_norms.{i}.bias", (h,))]
        prev = h
    out += [("proj_total.output.weight", (17, prev)), ("proj_total.output.bias", (17,))]
    if cfg.dipole:
        out.append(("physical_tensor_heads.dipole.1.weight", (1, nC)))
    return out
