"""Host-side checks of the ICTD path (no GPU): model state_dict keys equal the reference's, the
layout tables are consistent, and the product's constants equal the oracle's."""

import json
import os

import numpy as np
import pytest
import torch

from conftest import GOLDEN, load_golden
from fsctep_amd import ictd_basis as B
from fsctep_amd import ictd_ops
from oracle import ictd_ref as I

CASES = ["ictd_open32_c32_l2", "ictd_pbc64_c128_l3", "ictdo3_pbc64_c64_l2_field"]


def _model_cpu(g):
    from fsctep_amd.ictd import PureCartesianICTDO3TransformerLayer, PureCartesianICTDTransformerLayer
    kw = dict(max_embed_radius=5.0, main_max_radius=5.0, main_number_of_basis=8,
              hidden_dim_conv=int(g["channels"]), hidden_dim_sh=int(g["channels"]), hidden_dim=64, channel_in2=32,
              embedding_dim=16, max_atomvalue=10, output_size=8, embed_size=[128, 128, 128],
              num_interaction=int(g["layers"]), function_type_main="bessel", lmax=int(g["lmax"]),
              ictd_tp_path_policy="full", invariant_channels=32)
    if bool(g["o3"]):
        return PureCartesianICTDO3TransformerLayer(
            **kw, o3_active_irreps="0e,1e,1o,2e", external_tensor_rank=1, external_tensor_irrep="1o",
            physical_tensor_outputs={"dipole": {"irreps": ["1o"], "channels_out": 1, "reduce": "sum"}})
    return PureCartesianICTDTransformerLayer(**kw)


@pytest.mark.parametrize("name", CASES)
def test_state_dict_keys_match_reference(name):
    g = load_golden(name)
    m = _model_cpu(g)
    ref = json.load(open(os.path.join(GOLDEN, name + "_state_dict.json")))
    assert sorted((k, tuple(v.shape)) for k, v in m.state_dict().items()) == sorted((k, tuple(s)) for k, s in ref)


def test_constants_equal_oracle():
    for l1 in range(4):
        for l2 in range(4):
            for l3 in range(4):
                np.testing.assert_allclose(B.coupling(l1, l2, l3), I.cg(l1, l2, l3).numpy(), atol=1e-13)
    n = torch.randn(20, 3, dtype=torch.float64)
    n = n / n.norm(dim=1, keepdim=True)
    for l in range(4):
        exps, coef, P = B.harmonic_projection(l)
        t = np.stack([coef[i] * np.prod(n.numpy() ** exps[i], axis=1) for i in range(len(coef))], axis=1)
        np.testing.assert_allclose(t @ P, I.direction_harmonics(n, l).numpy(), atol=1e-12)


@pytest.mark.parametrize("lay", B.COMPILED_LAYOUTS, ids=lambda l: l.name)
def test_layout_tables_consistent(lay):
    s = ictd_ops.layout_struct(ictd_ops.register_layout(lay))
    paths = lay.conv2_paths()
    assert s.NP == len(paths) and s.KT == sum(p["d3"] for p in paths)
    # groups tile the input components and the padded kk ranges in order
    assert sum(s.g_d1[g] for g in range(s.NG)) == s.M
    assert s.NBGP == sum(s.g_d1[g] * s.g_kpad[g] for g in range(s.NG))
    for kk in range(s.KT):
        p = s.kk_path[kk]
        assert s.p_koff[p] <= kk < s.p_koff[p] + s.p_d3[p]
        g = s.p_group[p]
        assert s.g_kstart[g] <= kk < s.g_kstart[g] + s.g_kcount[g]
    # conv1: the canonical harmonics map onto the canonical output components
    for y in range(s.NY):
        assert s.y_path1[y] >= 0
    assert len(lay.cg_table()) == sum(p["d1"] * p["d2"] * p["d3"] for p in paths)
