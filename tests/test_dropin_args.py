"""Constructor arguments of the drop-in trunks (CPU: nothing here launches a kernel).

* Radial bases: the five names the reference offers (cli/train.py:589-590) are accepted, any other name
  is refused at construction, not at the first forward.
* O3 active irreps: the presets resolve as the reference resolves them
  (models/pure_cartesian_ictd_layers_o3.py:88-180); the expected lists below are worked out by hand from
  those rules (balanced: the products of the seed irreps with the geometric ones, l3 up to lmax,
  parity p1 p2).  Layouts the kernels cannot run (a missing geometric irrep, more than 16 components per
  channel) are refused at construction.
* Species tables of any size are accepted (more than 16 rows are served by a device-side mapping).
"""

import pytest

from fsctep_amd.ictd import (PureCartesianICTDO3TransformerLayer, PureCartesianICTDTransformerLayer,
                             resolve_o3_keys)
from fsctep_amd.sparse import PureCartesianSparseTransformerLayer

BASE = dict(max_embed_radius=5.0, main_max_radius=5.0, main_number_of_basis=8, hidden_dim_conv=32,
            num_interaction=2)

E0, O0, E1, O1, E2, O2, E3, O3 = (0, 1), (0, -1), (1, 1), (1, -1), (2, 1), (2, -1), (3, 1), (3, -1)


@pytest.mark.parametrize("basis", ["bessel", "gaussian", "fourier", "cosine", "smooth_finite"])
def test_reference_bases_accepted(basis):
    PureCartesianSparseTransformerLayer(**BASE, function_type_main=basis)
    PureCartesianICTDTransformerLayer(**BASE, function_type_main=basis, lmax=2)


def test_unknown_basis_refused_at_construction():
    with pytest.raises(ValueError, match="radial basis"):
        PureCartesianSparseTransformerLayer(**BASE, function_type_main="chebyshev")
    with pytest.raises(ValueError, match="radial basis"):
        PureCartesianICTDTransformerLayer(**BASE, function_type_main="chebyshev", lmax=2)
    with pytest.raises(NotImplementedError, match="number_of_basis"):
        PureCartesianSparseTransformerLayer(**{**BASE, "main_number_of_basis": 17})


def test_large_species_tables_accepted():
    m = PureCartesianSparseTransformerLayer(**BASE, max_atomvalue=50)
    assert m.e3_conv_layers[0].atom_embedding.weight.shape[0] == 50
    mi = PureCartesianICTDTransformerLayer(**BASE, max_atomvalue=50, lmax=2)
    assert mi.e3_conv_emb.atom_embedding.weight.shape[0] == 50


@pytest.mark.parametrize("lmax,preset,ext,phys,want", [
    (2, "auto", None, None, [E0, O1, E2]),
    (3, "auto", None, None, [E0, O1, E2, O3]),
    (2, "auto", "1e", None, [E0, E1, O1, E2]),
    (2, "minimal", None, None, [E0]),
    (2, "minimal", "1o", {"dipole": {"irreps": ["1o"]}}, [E0, O1]),
    (1, "balanced", None, None, [E0, E1, O1]),
    (2, "balanced", None, None, [E0, E1, O1, E2, O2]),
    (2, "full", None, None, [E0, O0, E1, O1, E2, O2]),
    (2, "auto", None, {"q": {"ls": [2]}}, [E0, O1, E2]),
])
def test_o3_presets_resolve_like_the_reference(lmax, preset, ext, phys, want):
    assert resolve_o3_keys(lmax, preset, None, ext, phys) == want


def test_o3_explicit_irreps_join_the_required_ones():
    assert resolve_o3_keys(2, "full", "2e, 1o + 0e", "1o", None) == [E0, O1, E2]
    assert resolve_o3_keys(2, "auto", ["0e", "1e", "1o", "2e"], None, None) == [E0, E1, O1, E2]
    assert resolve_o3_keys(2, "auto", "", None, None) == [E0, O1, E2]       # empty: the preset decides
    with pytest.raises(ValueError):
        resolve_o3_keys(2, "auto", "3o", None, None)
    with pytest.raises(ValueError):
        resolve_o3_keys(2, "fancy", None, None, None)


def test_o3_presets_the_kernels_cannot_run_are_refused():
    kw = dict(**BASE, lmax=2)
    m = PureCartesianICTDO3TransformerLayer(**kw, o3_irrep_preset="auto", external_tensor_rank=1,
                                            external_tensor_irrep="1o")
    assert m.keys == [E0, O1, E2]
    assert PureCartesianICTDO3TransformerLayer(**kw, o3_irrep_preset="full").layout.M == 18
    assert PureCartesianICTDO3TransformerLayer(**kw, o3_irrep_preset="balanced").layout.M == 17
    with pytest.raises(NotImplementedError, match="geometric"):
        PureCartesianICTDO3TransformerLayer(**kw, o3_irrep_preset="minimal")       # no 1o, 2e
    kw3 = dict(**BASE, lmax=3)
    with pytest.raises(NotImplementedError, match="kk rows 198"):
        PureCartesianICTDO3TransformerLayer(**kw3, o3_irrep_preset="full")         # 28 components, 198 kk rows
    with pytest.raises(NotImplementedError, match="kk tiles"):
        PureCartesianICTDO3TransformerLayer(**kw3, o3_irrep_preset="balanced")


def test_lmax_range_is_checked_at_construction():
    """lmax 0 to 3 construct (the kernels' 16 harmonic components); lmax 4 is refused before any forward."""
    for lmax in (0, 1, 3):
        m = PureCartesianICTDTransformerLayer(**BASE, lmax=lmax)
        assert m.layout.NY == (lmax + 1) ** 2
    m = PureCartesianICTDO3TransformerLayer(**BASE, lmax=1, o3_active_irreps="0e,1o")
    assert m.keys == [E0, O1]
    with pytest.raises(NotImplementedError, match="lmax 0 to 3"):
        PureCartesianICTDTransformerLayer(**BASE, lmax=4)
    with pytest.raises(NotImplementedError, match="lmax 0 to 3"):
        PureCartesianICTDO3TransformerLayer(**BASE, lmax=4, o3_active_irreps="0e,1o,2e,3o,4e")
