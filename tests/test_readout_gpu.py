"""GPU parity of the fused Gram-bilinear readout op against a float64 PyTorch evaluation of the
reference formula (einsum("ocd,ncd->no", W, gram), models/pure_cartesian_sparse_layers.py:424-456,
models/pure_cartesian_ictd_layers_full.py:999-1000), forward and gradient w.r.t. t; 1e-5 relative."""

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL = 1e-5


def _ref(t, W, scale):
    gram = torch.einsum("nmi,nmj->nij", t, t) * scale
    return torch.einsum("oij,nij->no", W, gram)


def rel_inf(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).abs().max() / b.abs().max().clamp_min(1e-30))


# (N, D, nC, S): rank 0..2 sparse blocks (D = 3^L), ICTD irreps (D = 2l+1), partial node tiles,
# odd block counts (nC = 48, 160), the 10k-atom channel widths (192, 384)
CASES = [(70, 1, 64, 32), (65, 3, 48, 64), (130, 9, 192, 64), (20, 7, 160, 32), (200, 5, 384, 64),
         (1, 3, 16, 64)]


@pytest.mark.parametrize("N,D,nC,S", CASES)
def test_gram_bilinear_matches_reference(N, D, nC, S):
    from fsctep_amd import readout_ops  # noqa: F401  (registers the ops)
    g = torch.Generator().manual_seed(N * 7 + D)
    t = torch.randn(N, D, nC, generator=g, dtype=torch.float64)
    W = torch.randn(S, nC, nC, generator=g, dtype=torch.float64) * 0.02
    G = torch.randn(N, S, generator=g, dtype=torch.float64)
    scale = 1.0 / D ** 0.5
    to = t.clone().requires_grad_(True)
    ref = _ref(to, W, scale)
    (gref,) = torch.autograd.grad(ref, to, G)

    Wd = W.float().to(DEV)
    Wf, Wb = torch.ops.fsctep.gram_prepare_weights(Wd)
    td = t.float().to(DEV).requires_grad_(True)
    out = torch.ops.fsctep.gram_bilinear(td, Wf, Wb, scale)
    (gt,) = torch.autograd.grad(out, td, G.float().to(DEV))
    torch.cuda.synchronize()
    assert rel_inf(out, ref) < TOL
    assert rel_inf(gt, gref) < TOL


def test_gram_bilinear_strided_input_and_empty():
    """A transposed (non-contiguous) view gives the same result; zero nodes give an empty output."""
    from fsctep_amd import readout_ops  # noqa: F401
    g = torch.Generator().manual_seed(5)
    t = torch.randn(40, 64, 3, generator=g).to(DEV)          # ICTD layout (N, nC, d)
    W = (torch.randn(32, 64, 64, generator=g) * 0.02).to(DEV)
    Wf, Wb = torch.ops.fsctep.gram_prepare_weights(W)
    a = torch.ops.fsctep.gram_bilinear(t.transpose(1, 2), Wf, Wb, 0.5)
    b = torch.ops.fsctep.gram_bilinear(t.transpose(1, 2).contiguous(), Wf, Wb, 0.5)
    assert torch.equal(a, b)
    e = torch.ops.fsctep.gram_bilinear(torch.zeros(0, 3, 64, device=DEV), Wf, Wb, 0.5)
    assert e.shape == (0, 32)


class _GramProbe(torch.nn.Module):
    def forward(self, t: torch.Tensor, Wf: torch.Tensor, Wb: torch.Tensor) -> torch.Tensor:
        return torch.ops.fsctep.gram_bilinear(t, Wf, Wb, 0.25)


def test_scripted_graph_matches_eager_with_cpp_autograd():
    """TorchScript runs the same C++-registered op, forward and backward (the core.pt route)."""
    from fsctep_amd import readout_ops  # noqa: F401
    g = torch.Generator().manual_seed(9)
    t = torch.randn(90, 5, 128, generator=g).to(DEV)
    W = (torch.randn(64, 128, 128, generator=g) * 0.02).to(DEV)
    Wf, Wb = torch.ops.fsctep.gram_prepare_weights(W)
    m = torch.jit.script(_GramProbe())
    t1 = t.clone().requires_grad_(True)
    t2 = t.clone().requires_grad_(True)
    y1 = m(t1, Wf, Wb)
    y2 = torch.ops.fsctep.gram_bilinear(t2, Wf, Wb, 0.25)
    (g1,) = torch.autograd.grad(y1.square().sum(), t1)
    (g2,) = torch.autograd.grad(y2.square().sum(), t2)
    assert torch.equal(y1, y2) and torch.equal(g1, g2)


def _per_node_rel(a, b):
    """max over nodes of |a_n - b_n|_inf / |b_n|_inf; rows where b is zero must be exactly zero."""
    a = a.detach().double().cpu().reshape(a.shape[0], -1)
    b = b.detach().double().cpu().reshape(b.shape[0], -1)
    den, err = b.abs().amax(1), (a - b).abs().amax(1)
    nz = den > 0
    assert torch.equal(err[~nz], torch.zeros_like(err[~nz]))
    return float((err[nz] / den[nz]).max())


def _ref_chunked(t, W, G, scale, chunk=256):
    """float64 forward and gradient on the GPU, 256 nodes at a time (the Gram of 10^3 nodes is GBs)."""
    S, nC = W.shape[0], W.shape[1]
    Wm = W.reshape(S, -1)
    Ws = (W + W.transpose(1, 2)).reshape(S, -1)
    outs, grads = [], []
    for n0 in range(0, t.shape[0], chunk):
        tc = t[n0:n0 + chunk]
        gram = torch.bmm(tc.transpose(1, 2).contiguous(), tc) * scale           # (n, nC, nC)
        outs.append(gram.reshape(gram.shape[0], -1) @ Wm.T)
        A = (G[n0:n0 + chunk] @ Ws).reshape(-1, nC, nC)                            # A_n[i][j]
        grads.append(torch.bmm(tc, A.transpose(1, 2).contiguous()) * scale)       # dt[n][m][i]
    return torch.cat(outs), torch.cat(grads)


# Node counts large enough for the split-fp16 forward (more than 128 workgroups of 256-node tiles);
# node magnitudes spread over 8 decades, weight columns over 3, one all-zero node row and one
# all-zero gradient row: the per-node power-of-two scales must keep every node's own relative error.
WIDE = [(1100, 7, 384, 64), (1100, 3, 384, 64), (3400, 9, 192, 64), (2100, 1, 384, 32)]


@pytest.mark.parametrize("N,D,nC,S", WIDE)
def test_gram_bilinear_wide_dynamic_range(N, D, nC, S):
    from fsctep_amd import readout_ops  # noqa: F401
    g = torch.Generator().manual_seed(N + D)
    f64 = dict(generator=g, dtype=torch.float64)
    t = torch.randn(N, D, nC, **f64) * 10.0 ** (8 * torch.rand(N, 1, 1, **f64) - 4)
    t[5] = 0.0
    W = torch.randn(S, nC, nC, **f64) * 0.02 * 10.0 ** (-3 * torch.rand(S, 1, nC, **f64))
    G = torch.randn(N, S, **f64) * 10.0 ** (8 * torch.rand(N, 1, **f64) - 4)
    G[7] = 0.0
    scale = 1.0 / D ** 0.5
    tf, Wd, Gf = t.float(), W.float(), G.float()
    ref, gref = _ref_chunked(tf.double().to(DEV), Wd.double().to(DEV), Gf.double().to(DEV), scale)

    Wf, Wb = torch.ops.fsctep.gram_prepare_weights(Wd.to(DEV))
    td = tf.to(DEV).requires_grad_(True)
    out = torch.ops.fsctep.gram_bilinear(td, Wf, Wb, scale)
    (gt,) = torch.autograd.grad(out, td, Gf.to(DEV))
    torch.cuda.synchronize()
    assert _per_node_rel(out, ref) < TOL
    assert _per_node_rel(gt, gref) < TOL
