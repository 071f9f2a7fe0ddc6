"""ctypes binding of ``libfsctep_hip.so`` (the C ABI declared in ``include/fsctep.h``) and the
loader of ``libfsctep_torch.so``, which registers ``torch.ops.fsctep.*``.

Both libraries are required: importing an op module without them raises, there is no CPU path.
"""

from __future__ import annotations

import ctypes
import os

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "libfsctep_hip.so")
TORCH_LIB_PATH = os.path.join(_PKG, "libfsctep_torch.so")

_i32, _i64, _f32, _p = ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p
_pi64 = ctypes.POINTER(ctypes.c_int64)

# name -> argtypes (all return int status)
SIGNATURES = {
    "fsc_timing_begin": [ctypes.c_char_p],
    "fsc_timing_end": [ctypes.POINTER(ctypes.c_double), _pi64],
    "fsc_sparse_conv_workspace": [_i64, _i64, _i32, _pi64, _pi64],
    "fsc_sparse_conv_prepare_weights": [_p, _p, _i32, _p, _p, _p],
    "fsc_sparse_conv_forward": [_i64, _i64, _i32, _p, _p, _p, _p, _p, _p, _p, _f32, _p, _p, _p, _i32, _p, _p],
    "fsc_sparse_conv_backward": [_i64, _i64, _i32, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _f32,
                                 _p, _p, _p, _p, _i32, _p, _p],
    "fsc_sparse_conv_direction": [_i64, _i64, _i32, _p, _p, _p, _p, _f32, _p, _p],
    "fsc_sparse_conv_direction_backward": [_i64, _i64, _i32] + [_p] * 11 + [_f32, _p, _p, _p, _p, _i32, _p, _p],
    "fsc_sparse_conv1_pair_table": [_p, _p, _p, _i32, _i32, _p, _p, _p],
    "fsc_sparse_conv1_forward": [_i64, _i64, _i32, _p, _i64, _p, _p, _p, _p, _p, _p, _p, _p],
    "fsc_sparse_conv1_backward": [_i64, _i64, _i32, _p, _i64, _p, _p, _p, _p, _p, _p, _p, _p, _p],
    "fsc_ictd_forward_workspace": [_p, _i64, _i32, _pi64],
    "fsc_ictd_conv_forward": [_p, _i64, _i64, _i32] + [_p] * 11,
    "fsc_ictd_prepare_weights": [_p, _i32, _i32, _p, _p],
    "fsc_ictd_project": [_p, _i64, _i64, _i32] + [_p] * 9,
    "fsc_ictd_backward_workspace": [_p, _i64, _i32, _pi64, _pi64],
    "fsc_ictd_conv_backward": [_p, _i64, _i64, _i32] + [_p] * 18,
    "fsc_ictd_conv1_forward": [_p, _i64, _i64, _i32, _i32] + [_p] * 8,
    "fsc_ictd_conv1_backward": [_p, _i64, _i64, _i32, _i32] + [_p] * 10,
    "fsc_gram_sizes": [_i64, _i32, _i32, _pi64, _pi64, _pi64],
    "fsc_gram_prepare_weights": [_p, _i32, _i32, _p, _p, _p],
    "fsc_gram_forward": [_i64, _i32, _i32, _i32, _f32, _p, _p, _p, _p, _p],
    "fsc_gram_backward": [_i64, _i32, _i32, _i32, _f32, _p, _p, _p, _p, _p],
    "fsc_gram_forward_blocked": [_i64, _i32, _i32, _i32, _f32, _p, _p, _p, _p, _p],
    "fsc_gram_backward_blocked": [_i64, _i32, _i32, _i32, _f32, _p, _p, _p, _p, _p],
    "fsc_edge_geometry_forward": [_i64, _p, _p, _p, _p, _p, _p, _p],
    "fsc_edge_geometry_backward": [_i64, _i64, _p, _p, _p, _p, _p, _p, _p, _p, _p],
    "fsc_edge_harmonics_forward": [_p, _i64, _p, _p, _p],
    "fsc_edge_harmonics_backward": [_p, _i64, _p, _p, _p, _p],
    "fsc_readout_gather": [_p, _i64, _p, _p, _p, _p, _p],
    "fsc_readout_gather_blocked": [_p, _i64, _p, _p, _p, _p, _p],
    "fsc_readout_scatter": [_p, _i64, _p, _p, _p, _p, _p, _p],
    "fsc_readout_mlp_weights_floats": [_p, _pi64],
    "fsc_readout_mlp_prepare": [_p, _p, _p, _p],
    "fsc_readout_mlp_forward": [_p, _i64, _p, _p, _p, _p],
    "fsc_readout_mlp_backward": [_p, _i64, _p, _p, _p, _p, _p],
    "fsc_radial_mlp_forward": [_i64, _p, _p, _p, _p, _p, _p, _p, _i32, _i32, _f32, _i32, _p, _p],
    "fsc_radial_mlp_backward": [_i64, _p, _p, _p, _p, _p, _p, _i32, _i32, _f32, _i32, _p, _p, _p],
    "fsc_graph_sizes": [_i64, _i64, _i32, _pi64, _pi64],
    "fsc_graph_prepare": [_i64, _i64, _i32] + [_p] * 15,
    "fsc_graph_prepare_noalloc": [_i64, _i64, _i32] + [_p] * 14,
    "fsc_spatial_order_workspace": [_i64, _pi64],
    "fsc_spatial_order": [_i64, _p, _p, _p, _p],
    "fsc_neighbor_workspace": [_i64, _pi64],
    "fsc_neighbor_count": [_i64, _p, _p, _p, ctypes.c_double, _p, _p, _p],
    "fsc_neighbor_fill": [_i64, _i64, _p, _p, _p, ctypes.c_double, _p, _p, _p, _p, _p, _p, _p],
    "fsc_edge_vec_geometry_forward": [_i64, _p, _p, _p, _p, _p],
    "fsc_edge_vec_geometry_backward": [_i64, _p, _p, _p, _p, _p, _p, _p],
    "fsc_bucket_project": [_i64] + [_i32] * 5 + [_p] * 4 + [_i32, _p],
    "fsc_bucket_project_transpose_a": [_i64] + [_i32] * 5 + [_p] * 4 + [_i32, _p],
    "fsc_bucket_project_workspace": [_i64] + [_i32] * 5 + [_pi64],
    "fsc_bucket_project_transpose_vu": [_i64] + [_i32] * 5 + [_p] * 6 + [_i32, _p, _p],
    "fsc_bucket_mix": [_i64] + [_i32] * 4 + [_p] * 4 + [_i32, _p],
    "fsc_bucket_mix_workspace": [_i64] + [_i32] * 4 + [_pi64],
    "fsc_bucket_mix_transpose_y": [_i64] + [_i32] * 4 + [_p] * 4 + [_i32, _p, _p],
    "fsc_bucket_mix_transpose_w": [_i64] + [_i32] * 4 + [_p] * 4 + [_i32, _p, _p],
    "fsc_bucket_mix_transpose_g": [_i64] + [_i32] * 4 + [_p] * 4 + [_i32, _p],
}
# the fp64 twins of the bucket functions take the same arguments (double arrays)
SIGNATURES.update({n + "_f64": SIGNATURES[n] for n in (
    "fsc_bucket_project", "fsc_bucket_project_transpose_a", "fsc_bucket_project_transpose_vu", "fsc_bucket_mix",
    "fsc_bucket_mix_transpose_y", "fsc_bucket_mix_transpose_w", "fsc_bucket_mix_transpose_g")})

_lib = None


def load(path: str = LIB_PATH):
    """Load the library once; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(f"{path} not found: build it with `python -m fsctep_amd.build` "
                           "(the HIP kernels are the only implementation)")
    lib = ctypes.CDLL(path, mode=ctypes.RTLD_GLOBAL)
    lib.fsc_last_error.restype = ctypes.c_char_p
    lib.fsc_last_error.argtypes = []
    lib.fsc_abi_version.restype = ctypes.c_int
    for name, args in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = ctypes.c_int
    _lib = lib
    return lib


_torch_ops_loaded = False


def load_torch_ops(path: str = TORCH_LIB_PATH) -> None:
    """Register ``torch.ops.fsctep.*`` from ``libfsctep_torch.so`` (once); raises if it is not built."""
    global _torch_ops_loaded
    if _torch_ops_loaded:
        return
    if not os.path.exists(path):
        raise RuntimeError(f"{path} not found: build it with `python -m fsctep_amd.build` "
                           "(the HIP kernels are the only implementation)")
    load()                          # the C ABI library first (same instance the op library links)
    import torch
    torch.ops.load_library(path)
    _torch_ops_loaded = True


def call(name: str, *args) -> None:
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.fsc_last_error().decode(errors="replace")
        raise RuntimeError(f"{name} failed ({rc}): {msg}")


def ptr(t) -> int:
    """Device pointer of a tensor (None -> NULL)."""
    return 0 if t is None else int(t.data_ptr())


def stream_handle(device) -> int:
    import torch
    return int(torch.cuda.current_stream(device).cuda_stream)


class KernelTimer:
    """Context manager: summed HIP-event duration of every launch of one named kernel."""

    def __init__(self, kernel: str):
        self.kernel = kernel
        self.total_ms = 0.0
        self.launches = 0

    def __enter__(self):
        call("fsc_timing_begin", self.kernel.encode())
        return self

    def __exit__(self, *exc):
        ms = ctypes.c_double()
        n = ctypes.c_int64()
        call("fsc_timing_end", ctypes.byref(ms), ctypes.byref(n))
        self.total_ms, self.launches = ms.value, n.value
        return False
