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
