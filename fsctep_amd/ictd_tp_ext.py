"""Drop-in for the reference's native ICTD extension module ``molecular_force_field._C_ictd_tp``
(csrc/ictd_tp.cpp:498-522): the same seventeen functions, argument order, output shapes and argument
errors, plus ``has_cuda()``, backed by the gfx950 kernels (``torch.ops.fsctep.*``, registered in C++ by
libfsctep_torch.so, launched on the current stream).

A reference trunk that keeps its own code selects this backend through its ``ictd_tp_backend="cuda_ext"``
switch (models/ictd_irreps_cuda.py:9-52, used by HarmonicFullyConnectedTensorProduct at
models/ictd_irreps.py:1035-1063) once the module is installed under the reference's name, before the
reference imports it::

    from fsctep_amd import ictd_tp_ext
    ictd_tp_ext.install()   # sys.modules["molecular_force_field._C_ictd_tp"] = ictd_tp_ext

The kernels take what the reference's CUDA kernels take (csrc/ictd_tp_cuda.cu:1230-1236): GPU float32 or
float64 tensors, all of one dtype, with mul_in2 == 1 (the trunks' conv2..n).  Other arguments raise
RuntimeError; there is no CPU path.
"""

from __future__ import annotations

import sys

import torch

from . import _lib

_lib.load_torch_ops()
_ops = torch.ops.fsctep

project_bucket_forward = _ops.project_bucket_forward
project_bucket_transpose_a = _ops.project_bucket_transpose_a
project_bucket_transpose_b = _ops.project_bucket_transpose_b
project_bucket_transpose_u = _ops.project_bucket_transpose_u
mix_bucket_forward = _ops.mix_bucket_forward
mix_bucket_transpose_y = _ops.mix_bucket_transpose_y
mix_bucket_transpose_w = _ops.mix_bucket_transpose_w
mix_bucket_transpose_g = _ops.mix_bucket_transpose_g
bucketed_tp_forward = _ops.bucketed_tp_forward
project_dbl_bwd_grad_h = _ops.project_dbl_bwd_grad_h
project_dbl_bwd_grad_a = _ops.project_dbl_bwd_grad_a
project_dbl_bwd_grad_b = _ops.project_dbl_bwd_grad_b
project_dbl_bwd_grad_u = _ops.project_dbl_bwd_grad_u
mix_dbl_bwd_grad_g_out = _ops.mix_dbl_bwd_grad_g_out
mix_dbl_bwd_grad_y = _ops.mix_dbl_bwd_grad_y
mix_dbl_bwd_grad_w = _ops.mix_dbl_bwd_grad_w
mix_dbl_bwd_grad_g = _ops.mix_dbl_bwd_grad_g

FUNCTIONS = ("project_bucket_forward", "project_bucket_transpose_a", "project_bucket_transpose_b",
             "project_bucket_transpose_u", "mix_bucket_forward", "mix_bucket_transpose_y", "mix_bucket_transpose_w",
             "mix_bucket_transpose_g", "bucketed_tp_forward", "project_dbl_bwd_grad_h", "project_dbl_bwd_grad_a",
             "project_dbl_bwd_grad_b", "project_dbl_bwd_grad_u", "mix_dbl_bwd_grad_g_out", "mix_dbl_bwd_grad_y",
             "mix_dbl_bwd_grad_w", "mix_dbl_bwd_grad_g")


def has_cuda() -> bool:
    """The reference reports whether its GPU kernels were compiled in; these always are."""
    return True


def install(name: str = "molecular_force_field._C_ictd_tp") -> None:
    """Make ``import molecular_force_field._C_ictd_tp`` (and ``from molecular_force_field import _C_ictd_tp``)
    resolve to this module."""
    mod = sys.modules[__name__]
    sys.modules[name] = mod
    parent, _, child = name.rpartition(".")
    if parent in sys.modules:
        setattr(sys.modules[parent], child, mod)
