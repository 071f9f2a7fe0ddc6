"""The op boundary for TorchScript / LibTorch: every ``torch.ops.fsctep.*`` op is registered in C++
by ``libfsctep_torch.so`` with device, Meta and autograd kernels; scripted graphs call the ops by
name; and a C++ process with no Python loads the library (as the LAMMPS engine loads
MFF_CUSTOM_OPS_LIB, lammps_user_mfftorch/src/USER-MFFTORCH/mff_torch_engine.cpp:226-249) and runs a
scripted module that calls them.  No GPU is needed: these run on Meta tensors."""

import os
import subprocess

import pytest
import torch

from conftest import ROOT
from fsctep_amd import _lib

OPS = ["sparse_prepare_weights", "sparse_conv", "sparse_conv_backward", "sparse_conv1_pair_table", "sparse_conv1",
       "sparse_conv1_backward", "ictd_prepare_weights", "ictd_conv", "ictd_conv_backward", "ictd_conv1",
       "ictd_conv1_backward", "gram_prepare_weights", "gram_bilinear", "gram_bilinear_backward", "edge_geometry",
       "edge_geometry_backward", "radial_mlp", "radial_mlp_backward", "edge_harmonics", "edge_harmonics_backward",
       "readout_gather", "readout_scatter", "readout_features", "graph_prepare", "edge_vec_geometry",
       "edge_vec_geometry_backward", "spatial_order", "ictd_project", "sparse_conv_direction",
       "sparse_conv_direction_backward", "readout_mlp_prepare", "readout_mlp", "readout_mlp_backward",
       "gram_bilinear_blocked", "gram_bilinear_backward_blocked", "readout_gather_blocked",
       # the per-edge (bucketed) ICTD ops under the reference extension's names (csrc/ictd_tp.cpp:498-521)
       "project_bucket_forward", "project_bucket_transpose_a", "project_bucket_transpose_b",
       "project_bucket_transpose_u", "mix_bucket_forward", "mix_bucket_transpose_y", "mix_bucket_transpose_w",
       "mix_bucket_transpose_g", "bucketed_tp_forward", "project_dbl_bwd_grad_h", "project_dbl_bwd_grad_a",
       "project_dbl_bwd_grad_b", "project_dbl_bwd_grad_u", "mix_dbl_bwd_grad_g_out", "mix_dbl_bwd_grad_y",
       "mix_dbl_bwd_grad_w", "mix_dbl_bwd_grad_g"]


class GramProbe(torch.nn.Module):
    def forward(self, t: torch.Tensor, Wf: torch.Tensor, Wb: torch.Tensor) -> torch.Tensor:
        return torch.ops.fsctep.gram_bilinear(t, Wf, Wb, 0.5)


def test_schemas_registered_in_cpp():
    _lib.load_torch_ops()
    for name in OPS:
        op = getattr(torch.ops.fsctep, name)
        schema = op.default._schema
        assert schema.name == f"fsctep::{name}"
        # registered by the C++ library, not by Python
        assert torch._C._dispatch_has_kernel_for_dispatch_key(f"fsctep::{name}", "CUDA")
        assert torch._C._dispatch_has_kernel_for_dispatch_key(f"fsctep::{name}", "Meta")
    for name in ("sparse_conv", "sparse_conv1", "ictd_conv", "ictd_conv1", "gram_bilinear", "readout_features",
                 "edge_geometry", "edge_vec_geometry", "radial_mlp", "edge_harmonics", "readout_mlp"):
        assert torch._C._dispatch_has_computed_kernel_for_dispatch_key(f"fsctep::{name}", "AutogradCUDA")


def test_scripted_graph_calls_ops_by_name():
    _lib.load_torch_ops()
    m = torch.jit.script(GramProbe())
    assert "fsctep::gram_bilinear" in str(m.graph)


def test_ictd_layout_words_round_trip():
    from fsctep_amd import ictd_basis as B, ictd_ops
    lid = ictd_ops.register_layout(B.layout_full(3))
    t = ictd_ops.layout_words(lid)
    s = ictd_ops.layout_struct(lid)
    assert isinstance(t, list) and len(t) * 4 == ctypes_sizeof(s)
    assert t[0] == s.M and t[2] == s.KT
    with torch._subclasses.fake_tensor.FakeTensorMode():
        x = torch.empty(10, s.M, 128)
        out = torch.ops.fsctep.ictd_conv1(torch.empty(40, s.NY), torch.empty(40, s.NREF), torch.empty(64, s.NP1, 128),
                                          torch.empty(11, dtype=torch.int32), torch.empty(40, dtype=torch.int32),
                                          torch.empty(10, dtype=torch.int32), 8, s.M, t)
        assert out.shape == x.shape


def ctypes_sizeof(s):
    import ctypes
    return ctypes.sizeof(s)


def test_python_free_process_loads_ops_and_runs_scripted_module(tmp_path):
    _lib.load_torch_ops()
    pt = tmp_path / "gram_probe.pt"
    torch.jit.script(GramProbe()).save(str(pt))
    base = os.path.dirname(torch.__file__)
    inc, lib = os.path.join(base, "include"), os.path.join(base, "lib")
    exe = tmp_path / "load_ops"
    cmd = ["g++", "-std=c++17", "-O1", "-D_GLIBCXX_USE_CXX11_ABI=1", "-I", inc,
           "-I", os.path.join(inc, "torch", "csrc", "api", "include"), os.path.join(ROOT, "tests", "cpp", "load_ops.cpp"),
           "-o", str(exe), "-L", lib, "-ltorch", "-ltorch_cpu", "-lc10", f"-Wl,-rpath,{lib}", "-ldl"]
    res = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert res.returncode == 0, res.stderr[-3000:]
    env = {k: v for k, v in os.environ.items() if not k.startswith("PYTHON")}
    run = subprocess.run([str(exe), _lib.TORCH_LIB_PATH, str(pt)], capture_output=True, text=True, timeout=300, env=env)
    assert run.returncode == 0, run.stdout + run.stderr
    assert f"fsctep ops registered: {len(OPS)}; scripted module -> [7, 64]" in run.stdout
