"""CPU oracle of the per-edge ("bucketed") ICTD tensor product behind the reference's native extension
``molecular_force_field._C_ictd_tp`` (test infrastructure only).

Restated from the reference's PyTorch definitions of the extension's operations:
  * projection and its transposes        models/ictd_irreps_cuda.py:169-180, 200-227
  * gated channel mix and its transposes models/ictd_irreps_cuda.py:251-258, 269-288
  * double-backward sums                 csrc/ictd_tp_cuda.cu:528-533, 796-802
  * the bucketing of a fully connected TP (paths grouped by (l1, l2), each group's projection
    U_g = [C_p reshaped (m1*m2, 2l3+1)] in path order, buckets of equal kdim)
                                         models/ictd_irreps.py:97-120, 815-847, 886-915, 1003-1063
and, as a second formulation of the projection, the ATen route of the extension's CPU branch
(csrc/ictd_tp.cpp:110-117, 155-175).  Shapes: a (B, I, m1), b (B, J, m2), u (m1*m2, P*K),
y (B, P, K, I*J), w (P, O, I*J), gates (B, P), out (B, O, K).
"""

from __future__ import annotations

import torch

from .ictd_ref import cg


def project_forward(a, b, u, num_paths: int):
    """y[b,p,k,(i,j)] = sum_{m,n} a[b,i,m] b[b,j,n] u[(m,n),(p,k)] (models/ictd_irreps_cuda.py:169-180)."""
    B, I, m1 = a.shape
    J, m2 = b.shape[1], b.shape[2]
    pk = u.shape[1]
    y = torch.einsum("bim,bjn,mnp->bijp", a, b, u.reshape(m1, m2, pk))
    return y.reshape(B, I * J, num_paths, pk // num_paths).permute(0, 2, 3, 1).contiguous()


def project_forward_aten(a, b, u, num_paths: int):
    """The same projection by the extension's CPU route (csrc/ictd_tp.cpp:110-117, 155-175): u packed to
    (m1, P*K*m2), one matmul over (b, i) rows, then a batched product with b."""
    B, I, m1 = a.shape
    J, m2 = b.shape[1], b.shape[2]
    pk = u.shape[1]
    u_stage1 = u.reshape(m1, m2, pk).permute(0, 2, 1).reshape(m1, pk * m2)
    tmp = (a.reshape(B * I, m1) @ u_stage1).reshape(B, I * pk, m2)
    y_rows = torch.bmm(tmp, b.transpose(1, 2))                                   # (B, I*pk, J)
    return (y_rows.reshape(B, I, num_paths, pk // num_paths, J).permute(0, 2, 3, 1, 4)
            .reshape(B, num_paths, pk // num_paths, I * J))


def project_transpose(grad_y, a, b, u):
    """(grad_a, grad_b, grad_u) of the projection (models/ictd_irreps_cuda.py:200-227)."""
    B, P, K, _ = grad_y.shape
    I, J, m1, m2 = a.shape[1], b.shape[1], a.shape[2], b.shape[2]
    g = grad_y.reshape(B, P, K, I, J).permute(0, 3, 4, 1, 2).reshape(B, I, J, P * K)
    u3 = u.reshape(m1, m2, P * K)
    grad_a = torch.einsum("bijp,bjn,mnp->bim", g, b, u3)
    grad_b = torch.einsum("bijp,bim,mnp->bjn", g, a, u3)
    grad_u = torch.einsum("bijp,bim,bjn->mnp", g, a, b).reshape(m1 * m2, P * K)
    return grad_a, grad_b, grad_u


def mix_forward(y, w, gates):
    """out[b,o,k] = sum_p gates[b,p] sum_q y[b,p,k,q] w[p,o,q] (models/ictd_irreps_cuda.py:251-258)."""
    out_per = torch.einsum("bpkq,poq->bpok", y, w)
    return (out_per * gates[:, :, None, None]).sum(dim=1)


def mix_transpose(grad_out, y, w, gates):
    """(grad_y, grad_w, grad_gates) of the channel mix (models/ictd_irreps_cuda.py:269-288)."""
    gated = grad_out[:, None, :, :] * gates[:, :, None, None]
    grad_y = torch.einsum("bpok,poq->bpkq", gated, w)
    grad_w = torch.einsum("bpok,bpkq->poq", gated, y)
    grad_g = (grad_out[:, None, :, :] * torch.einsum("bpkq,poq->bpok", y, w)).sum(dim=(2, 3))
    return grad_y, grad_w, grad_g


def project_dbl_bwd(h, a, gga, b, ggb, u, ggu, num_paths: int):
    """(grad_h, grad_a, grad_b, grad_u) of csrc/ictd_tp_cuda.cu:528-533:
    PF(gga,b,u) + PF(a,ggb,u) + PF(a,b,ggu); PAT(h,ggb,u) + PAT(h,b,ggu); PBT(h,gga,u) + PBT(h,a,ggu);
    PUT(h,gga,b) + PUT(h,a,ggb)."""
    grad_h = project_forward(gga, b, u, num_paths) + project_forward(a, ggb, u, num_paths) \
        + project_forward(a, b, ggu, num_paths)
    grad_a = project_transpose(h, a, ggb, u)[0] + project_transpose(h, a, b, ggu)[0]
    grad_b = project_transpose(h, gga, b, u)[1] + project_transpose(h, a, b, ggu)[1]
    grad_u = project_transpose(h, gga, b, u)[2] + project_transpose(h, a, ggb, u)[2]
    return grad_h, grad_a, grad_b, grad_u


def mix_dbl_bwd(g_out, y, ggy, w, ggw, gates, ggg):
    """(grad_g_out, grad_y, grad_w, grad_gates) of csrc/ictd_tp_cuda.cu:796-802:
    MF(ggy,w,g) + MF(y,ggw,g) + MF(y,w,ggg); MYT(G,ggw,g) + MYT(G,w,ggg); MWT(G,ggy,g) + MWT(G,y,ggg);
    MGT(G,ggy,w) + MGT(G,y,ggw)."""
    grad_go = mix_forward(ggy, w, gates) + mix_forward(y, ggw, gates) + mix_forward(y, w, ggg)
    grad_y = mix_transpose(g_out, y, ggw, gates)[0] + mix_transpose(g_out, y, w, ggg)[0]
    grad_w = mix_transpose(g_out, ggy, w, gates)[1] + mix_transpose(g_out, y, w, ggg)[1]
    grad_g = mix_transpose(g_out, ggy, w, gates)[2] + mix_transpose(g_out, y, ggw, gates)[2]
    return grad_go, grad_y, grad_w, grad_g


def buckets(paths):
    """The bucket table of a fully connected TP with per-path gates and mul_in2 == 1 (models/ictd_irreps.py:97-120,
    815-847, 886-915): paths grouped by their input keys (k1, k2) in sorted order, each group's columns the
    CG tensors C_p reshaped (m1*m2, 2 l3 + 1) in path order, split into buckets of equal kdim (ascending).
    Returns [(k1, k2, k3, kdim, [path indices], U_bucket (float64))]."""
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
            U = torch.cat([cg(k1[0], k2[0], l3).reshape(m1 * m2, kdim) for _, l3, _ in segs], dim=1)
            table.append((k1, k2, (segs[0][1], segs[0][2]), kdim, [p for p, _, _ in segs], U))
    return table
